// Writes Philox4x32-10 vectors computed by rocRAND's engine (an independent
// implementation shipped with ROCm) so tests can pin oracle/walk_oracle.c's
// Philox against it.  Host-only; build and run with:
//   hipcc -O1 -I/opt/rocm/include tests/golden/philox_rocrand_vectors.cpp \
//         -o /tmp/philox_vectors && /tmp/philox_vectors > tests/golden/philox_rocrand.txt
#include <rocrand/rocrand_philox4x32_10.h>

#include <cstdint>
#include <cstdio>

// ten_rounds() is a protected member; a derived class makes it callable.
struct PhiloxRounds : rocrand_device::philox4x32_10_engine {
    using rocrand_device::philox4x32_10_engine::ten_rounds;
};

int main() {
    PhiloxRounds eng;
    uint64_t s = 0x0123456789abcdefull;  // SplitMix64 walk for the inputs
    auto next = [&s]() {
        uint64_t z = (s += 0x9e3779b97f4a7c15ull);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    };
    std::printf("# ctr0 ctr1 ctr2 ctr3 key0 key1 -> out0 out1 out2 out3 (hex)\n");
    for (int i = 0; i < 64; ++i) {
        uint64_t a = next(), b = next(), c = next();
        uint4 ctr = {static_cast<unsigned>(a), static_cast<unsigned>(a >> 32),
                     static_cast<unsigned>(b), static_cast<unsigned>(b >> 32)};
        if (i < 8) { ctr.z = 0; ctr.w = static_cast<unsigned>(i); }  // small counters too
        uint2 key = {static_cast<unsigned>(c), static_cast<unsigned>(c >> 32)};
        uint4 r = eng.ten_rounds(ctr, key);
        std::printf("%08x %08x %08x %08x %08x %08x %08x %08x %08x %08x\n", ctr.x, ctr.y, ctr.z,
                    ctr.w, key.x, key.y, r.x, r.y, r.z, r.w);
    }
    return 0;
}
