// Uniform random walk kernels (RandomWalk.cpp:41-60) and their launcher.
//
// The walk is a chain of dependent random reads, so throughput comes from
// the number of chains in flight and the number of reads per step, not from
// arithmetic.  Every lane runs a small state machine over W walk slots; a
// slot whose walk ends (or is absorbed by a node of out-degree 0) takes the
// next walk from a per-wavefront queue refilled by one global atomic per
// kQueueChunk (64) walks, so lanes never idle while walks remain and the
// kernel's tail is about one walk long.  Grids are the device's resident
// capacity.
#include <type_traits>

#include "walk_host.h"

namespace mlxc {

// Uniform walk without stream windows: W walk slots per lane, walks from the
// wave queue, 8-byte loads and stores.  Serves the cases the windowed
// kernels do not: buffers that are not 16-byte aligned, a rand tensor whose
// size is not a multiple of 4, graphs beyond int32 ids, and a workspace too
// small for the start records.
template <int W, bool kEdges, bool kGen, typename OutT>
__global__ __launch_bounds__(kBlock) void uniform_walk_kernel(WalkArgs a) {
    const int64_t L = a.walk_length;
    const int64_t N = a.num_walks;
    const int64_t goff = kGen ? a.walk_base * L : 0;  // stream position of uniform 0
    OutT* const nout = static_cast<OutT*>(a.n_out);
    OutT* const eout = static_cast<OutT*>(a.e_out);
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.work + 1);
    WaveQueue q{0, 0};
    int64_t n[W], v[W], l[W];
    uint32_t status = 0;

#pragma unroll
    for (int s = 0; s < W; ++s) { n[s] = -1; l[s] = L; v[s] = 0; }

    while (true) {
        // Acquire walks for empty slots; write their first column.
        bool unretired = false;
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool need = (n[s] < N) && (l[s] >= L);  // slot idle (or never used)
            const int64_t id = queue_take(q, need, counter);
            if (need) {
                n[s] = id;  // id >= N ends the slot for good
                if (id < N) {
                    const int64_t s0 = a.start[id];
                    nout[id * (L + 1)] = static_cast<OutT>(s0);
                    v[s] = s0;
                    l[s] = 0;
                    if (!node_ok(s0, a.num_nodes)) {
                        status |= MLXC_STATUS_BAD_NODE;
                        for (int64_t j = 1; j <= L; ++j) nout[id * (L + 1) + j] = static_cast<OutT>(s0);
                        if (kEdges)
                            for (int64_t j = 0; j < L; ++j) eout[id * L + j] = -1;
                        l[s] = L;
                    }
                }
            }
            unretired |= (n[s] < N);
        }
        // The whole wave leaves together, once every slot of every lane has
        // drawn an id past the end; until then idle lanes keep voting.
        if (!__any(unretired)) break;

        // Phase 1: rowptr pair and the step's uniform, for every live slot.
        RowBounds rb[W];
        float r[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            rb[s] = {0, 0};
            r[s] = 0.0f;
            if (live) {
                rb[s] = load_row(a.rowptr, v[s]);
                r[s] = kGen ? philox_uniform_at(goff + n[s] * L + l[s], a.key0, a.key1)
                            : __builtin_nontemporal_load(a.rand + n[s] * L + l[s]);
            }
        }
        // Phase 2: candidate edge and its target, for every moving slot.
        int64_t e[W], x[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            e[s] = -1;
            x[s] = v[s];
            if (live) {
                const int64_t deg = rb[s].end - rb[s].begin;
                if (!row_ok(rb[s], a.num_edges)) {
                    status |= MLXC_STATUS_BAD_ROW;
                } else if (deg > 0) {
                    e[s] = rb[s].begin + pick_index(r[s], deg);
                    x[s] = a.col[e[s]];
                }
            }
        }
        // Phase 3: store, advance, and finish sunk / broken walks.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool live = (n[s] < N) && (l[s] < L);
            if (!live) continue;
            OutT* out = nout + n[s] * (L + 1);
            const bool moved = e[s] >= 0;
            bool stop = !moved;  // deg == 0 (absorbing) or malformed row
            out[l[s] + 1] = static_cast<OutT>(x[s]);
            if (kEdges) eout[n[s] * L + l[s]] = static_cast<OutT>(e[s]);
            l[s] += 1;
            if (moved && !node_ok(x[s], a.num_nodes)) {
                status |= MLXC_STATUS_BAD_NODE;
                stop = true;
            }
            v[s] = x[s];
            if (stop) {
                for (int64_t j = l[s] + 1; j <= L; ++j) out[j] = static_cast<OutT>(x[s]);
                if (kEdges)
                    for (int64_t j = l[s]; j < L; ++j) eout[n[s] * L + j] = -1;
                l[s] = L;
            }
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.work), static_cast<unsigned long long>(status));
}

// Slot phases of the windowed walks.
enum : int {
    kSlotIdle = 0,   // wants a walk id
    kSlotStart = 1,  // reads the start record of walk n (and its first rand block)
    kSlotWalk = 2,   // record walk: reads the record of the chosen edge
    kSlotCol = 3,    // CSR walk: reads col[e] of the chosen edge
    kSlotRow = 4,    // CSR walk: reads rowptr[v], rowptr[v+1] of the new node; packed
                     // record walk: reads rowptr[v+1] of a row too long for its record
    kSlotDone = 5,   // the queue is exhausted
};

// Uniform walk over edge records (requires 16-byte aligned rand, n_out and
// e_out, num_nodes and num_edges below 2^31, num_walks * walk_length a
// multiple of 4 and at least RW).
//
// Loop invariant: every live slot issues exactly one dependent read per
// iteration (a start record or an edge record; with packed records also the
// end of a row too long for the degree field), plus at most one independent
// rand block, and the wave waits once.  The rand value for a step
// is taken from the window in the iteration before the read it addresses, so
// a new rand block always travels together with a record read and never costs
// a round trip of its own.  The whole blocks of output completed in one
// iteration are stored by the wavefront (ow_drain) right after the next
// iteration's reads are issued, so they overlap those reads.
template <int W, int RW, bool kGen, bool kEdges, typename OutT, bool kPacked>
__global__ __launch_bounds__(kBlock) void uniform_walk_rec_kernel(WalkArgs a,
                                                                  const void* __restrict__ recs,
                                                                  const void* __restrict__ init,
                                                                  PackedFormat fmt) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    typedef typename std::conditional<kPacked, uint64_t, i32x4>::type Rec;
    OutT* const nout = static_cast<OutT*>(a.n_out);
    OutT* const eout = static_cast<OutT*>(a.e_out);
    const int64_t L = a.walk_length;
    const int64_t L1 = L + 1;
    const int64_t N = a.num_walks;
    const int64_t rtotal = N * L;
    const int64_t goff = kGen ? a.walk_base * L : 0;  // stream position of uniform 0
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.work + 1);
    WaveQueue q{0, 0};
    int phase[W];
    int64_t n[W];
    int32_t l[W];
    const Rec* rp[W];          // what the slot reads next: a start or edge record, or
                               // (kSlotRow) the end of a long row; idle slots reread
                               // their last address
    int32_t row_begin[W];      // kSlotRow: the begin of that row
    int64_t fr[W];             // rand index whose block the next read brings along
    bool need_block[W];        // ... if set
    LdsWindow<RW> rw[W];
    __shared__ float rand_area[W][RW][kBlock];
    OutWin<int32_t> ow[W];
    OutWin<int32_t> ew[W];     // edge ids (kEdges): e_out[n*L + l] is step l's edge
    __shared__ WaveStage stage[kBlock / kWave];
    WaveStage& st = stage[threadIdx.x / kWave];
    uint32_t status = 0;

#pragma unroll
    for (int s = 0; s < W; ++s) {
        phase[s] = kSlotIdle;
        n[s] = 0;
        l[s] = 0;
        rp[s] = static_cast<const Rec*>(init);
        fr[s] = 0;
        need_block[s] = false;
        rw[s].pos = 0;
        rw[s].valid = 0;
        ow_init(ow[s]);
        ow_init(ew[s]);
    }

    while (true) {
        // 1. One read per slot (idle slots reread an earlier address, so the
        // load is unconditional and nothing merges with it before the wait in
        // step 3), and the rand blocks due.
        int ph[W];  // phase at issue: only these slots consume in step 3
        Rec rec[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            ph[s] = phase[s];
            rec[s] = *rp[s];
        }
        RandWindow<RW> blk[W];  // due rand blocks, stored to LDS in step 3
#pragma unroll
        for (int s = 0; s < W; ++s)
            if (need_block[s]) rw_fetch<RW, kGen>(blk[s], a, fr[s], rtotal, goff);
        // ... and the output blocks the last iteration completed are stored.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            ow_drain<OutT>(ow[s], st);
            if (kEdges) ow_drain<OutT>(ew[s], st);
        }

        // 2. While the reads are in flight, idle slots draw walk ids from the
        // wave queue; they issue their start reads next iteration.
        bool alive = false;
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool need = phase[s] == kSlotIdle;
            const int64_t id = queue_take(q, need, counter);
            if (need) {
                n[s] = id;
                l[s] = 0;
                phase[s] = id < N ? kSlotStart : kSlotDone;
                if (id < N) rp[s] = static_cast<const Rec*>(init) + id;
                fr[s] = id * L;  // the first step's uniform
            }
            alive |= phase[s] != kSlotDone;
        }
        if (!__any(alive)) break;  // every slot done: nothing was read above
        wait_vmem();
        if constexpr (!kPacked) {
#pragma unroll
            for (int s = 0; s < W; ++s) keep_vgpr(rec[s].w);
        }

        // 3. Consume: buffer the node, finish or pick the next edge.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const int64_t e0 = n[s] * L;  // edge output index of the walk's step 0
            bool pick = false;            // leave the node of row [begin, begin + deg)
            int32_t begin = 0, deg = 0;
            if (kPacked && ph[s] == kSlotRow) {  // the end of a long row
                pick = true;
                begin = row_begin[s];
                if constexpr (kPacked) deg = static_cast<int32_t>(static_cast<int64_t>(rec[s]) - begin);
            } else if (ph[s] != kSlotStart && ph[s] != kSlotWalk) {
                // a slot that just drew a walk reads its start record and
                // first rand block next iteration
                need_block[s] = phase[s] == kSlotStart && L > 0;
            } else {
                const int64_t g0 = n[s] * L1;  // output index of the walk's start node
                const int64_t g = g0 + l[s] + (ph[s] == kSlotWalk ? 1 : 0);
                if (need_block[s]) {
                    // the block holding rand[fr]; fr is its entry k
                    const int k = static_cast<int>(fr[s] - rw_base<RW, kGen>(fr[s], rtotal, goff));
                    lw_store(rand_area[s], rw[s], blk[s], k);
                    need_block[s] = false;
                }
                int32_t node;
                if constexpr (kPacked) {
                    fmt.unpack(rec[s], node, begin, deg);
                } else {
                    node = rec[s].x;
                    begin = rec[s].y;
                    deg = rec[s].z;
                }
                if (ph[s] == kSlotStart) {
                    ow[s].count = 0;
                    ew[s].count = 0;
                }
                // A malformed start or col entry, or the malformed row of a
                // node the walk is to leave, stops the walk (outputs
                // unspecified).  The row of the node a walk ends at is not
                // read by the reference, nor checked.
                const int32_t la = l[s] + (ph[s] == kSlotWalk ? 1 : 0);  // steps taken
                status |= (deg == kRecBadNode ? MLXC_STATUS_BAD_NODE : 0u) |
                          (deg == kRecBadRow && la < L ? MLXC_STATUS_BAD_ROW : 0u);
                // an absorbing node (the walk stays) or a malformed record
                // fills the rest of the row, this node included
                const bool stop = la < L && deg <= 0 && deg != kRecLongRow;
                if (stop) ow_fill(ow[s], nout, g, g0 + L, node);
                else ow_push(ow[s], nout, g, node);
                l[s] = la;
                if (la == L) {
                    if (ow[s].count) ow_flush(ow[s], nout, g);
                    if (kEdges && ew[s].count) ow_flush(ew[s], eout, e0 + L - 1);
                    phase[s] = kSlotIdle;
                } else if (stop) {
                    if (kEdges) ow_fill(ew[s], eout, e0 + la, e0 + L - 1, -1);
                    phase[s] = kSlotIdle;
                } else if (kPacked && deg == kRecLongRow) {  // read the row's end first
                    rp[s] = reinterpret_cast<const Rec*>(a.rowptr + node + 1);
                    row_begin[s] = begin;
                    phase[s] = kSlotRow;
                } else {
                    pick = true;
                }
            }
            if (pick) {  // step l (0-based) leaves the node with uniform rand[n*L + l]
                const float r = lw_take(rand_area[s], rw[s]);
                int64_t idx;
                if (kPacked && ph[s] != kSlotRow) {
                    // a degree held in a packed record: the float32 rule's exact
                    // branch only (the compiler drops the other)
                    __builtin_assume(deg <= PackedFormat::kMaxInlineDegree);
                    idx = pick_index(r, deg);
                } else {
                    idx = pick_index(r, deg);
                }
                const int32_t e = static_cast<int32_t>(begin + idx);
                if (kEdges) ow_push(ew[s], eout, e0 + l[s], e);
                rp[s] = static_cast<const Rec*>(recs) + e;
                need_block[s] = rw[s].valid == 0 && l[s] + 1 < L;
                fr[s] = n[s] * L + l[s] + 1;
                phase[s] = kSlotWalk;
            }
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.work), static_cast<unsigned long long>(status));
}

// Start record of the wide CSR walk, for graphs of 2^31 or more CSR entries
// (node ids below 2^31): {node, degree, row begin as int64}.  The degree
// field holds kRecBadNode or kRecBadRow for a malformed start or row, and
// kRecLongRow for a row of 2^31 or more entries, whose end the walk reads
// from rowptr first.
struct __attribute__((aligned(16))) WideStart {
    int32_t node, deg;
    int64_t begin;
};
static_assert(sizeof(WideStart) == sizeof(EdgeRecord), "both start layouts take 16 bytes a walk");

// Zeroes the status words and writes one WideStart per walk (one coalesced
// pass over start, one row read per walk).
__global__ __launch_bounds__(kBlock) void wide_init_kernel(const int64_t* __restrict__ rowptr,
                                                           const int64_t* __restrict__ start,
                                                           int64_t num_nodes, int64_t num_edges,
                                                           int64_t num_walks,
                                                           WideStart* __restrict__ init,
                                                           int64_t* __restrict__ work) {
    if (blockIdx.x == 0 && threadIdx.x < MLXC_WORK_WORDS) work[threadIdx.x] = 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t n = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; n < num_walks;
         n += stride) {
        const int64_t v = start[n];
        WideStart r{static_cast<int32_t>(v), kRecBadNode, 0};
        if (node_ok(v, num_nodes)) {
            const RowBounds rb = load_row(rowptr, v);
            if (!row_ok(rb, num_edges)) {
                r.deg = kRecBadRow;
            } else {
                const int64_t deg = rb.end - rb.begin;
                r.begin = rb.begin;
                r.deg = deg > INT32_MAX ? kRecLongRow : static_cast<int32_t>(deg);
            }
        }
        init[n] = r;
    }
}

// Uniform walk over the CSR arrays, for calls whose edge records would not
// pay for themselves (few steps per edge) or do not fit int32.  Same loop
// shape as the record walk — one dependent read per slot per iteration, one
// wait — but a step costs two reads: col[e] of the chosen edge, then the row
// of the new node.  Start records (walk_init_kernel) give the first row.
// Requirements as for the record walk except num_edges may be any size the
// int32 start records hold (num_nodes, num_edges below 2^31).  kWide: graphs
// of 2^31 or more entries (node ids still below 2^31), with WideStart records
// and int64 edge ids, which are stored directly instead of through a window.
template <int W, int RW, bool kGen, bool kEdges, typename OutT, bool kWide>
__global__ __launch_bounds__(kBlock) void uniform_walk_csr_kernel(WalkArgs a,
                                                                  const void* __restrict__ init_v) {
    typedef int32_t i32x4 __attribute__((ext_vector_type(4), aligned(8)));
    typedef typename std::conditional<kWide, int64_t, int32_t>::type EIdx;
    const EdgeRecord* const init = static_cast<const EdgeRecord*>(init_v);  // 16 bytes either way
    OutT* const nout = static_cast<OutT*>(a.n_out);
    OutT* const eout = static_cast<OutT*>(a.e_out);
    const int64_t L = a.walk_length;
    const int64_t L1 = L + 1;
    const int64_t N = a.num_walks;
    const int64_t rtotal = N * L;
    const int64_t goff = kGen ? a.walk_base * L : 0;  // stream position of uniform 0
    unsigned long long* counter = reinterpret_cast<unsigned long long*>(a.work + 1);
    WaveQueue q{0, 0};
    int phase[W];
    int64_t n[W], fr[W];
    int32_t l[W], v[W];        // steps and node ids fit in int32 here
    EIdx e[W];                 // edge ids: int32 unless kWide
    bool need_block[W];
    LdsWindow<RW> rw[W];
    __shared__ float rand_area[W][RW][kBlock];
    OutWin<int32_t> ow[W];
    OutWin<int32_t> ew[W];     // edge ids (kEdges): e_out[n*L + l] is step l's edge
    __shared__ WaveStage stage[kBlock / kWave];
    WaveStage& st = stage[threadIdx.x / kWave];
    uint32_t status = 0;

#pragma unroll
    for (int s = 0; s < W; ++s) {
        phase[s] = kSlotIdle;
        n[s] = 0;
        l[s] = 0;
        e[s] = 0;
        v[s] = 0;
        fr[s] = 0;
        need_block[s] = false;
        rw[s].pos = 0;
        rw[s].valid = 0;
        ow_init(ow[s]);
        ow_init(ew[s]);
    }

    while (true) {
        // 1. Reads: a 16-byte start record or rowptr pair (one instruction;
        // idle slots read init[0]), an 8-byte col entry (other slots reread
        // init[0]: both loads are unconditional), and due rand blocks.
        int ph[W];
        i32x4 row[W];
        int64_t cv[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
            ph[s] = phase[s];
            const i32x4* p = ph[s] == kSlotRow ? reinterpret_cast<const i32x4*>(a.rowptr + v[s])
                             : ph[s] == kSlotStart ? reinterpret_cast<const i32x4*>(init + n[s])
                                                   : reinterpret_cast<const i32x4*>(init);
            row[s] = *p;
            cv[s] = *(ph[s] == kSlotCol ? a.col + e[s] : reinterpret_cast<const int64_t*>(init));
        }
        RandWindow<RW> blk[W];  // due rand blocks, stored to LDS in step 3
#pragma unroll
        for (int s = 0; s < W; ++s)  // a block due after a pick travels with the col read
            if (need_block[s] && ph[s] != kSlotRow)
                rw_fetch<RW, kGen>(blk[s], a, fr[s], rtotal, goff);
        // ... and the output blocks the last iteration completed are stored.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            ow_drain<OutT>(ow[s], st);
            if (kEdges) ow_drain<OutT>(ew[s], st);
        }

        // 2. Idle slots draw walk ids while the reads are in flight.
        bool alive = false;
#pragma unroll
        for (int s = 0; s < W; ++s) {
            const bool need = phase[s] == kSlotIdle;
            const int64_t id = queue_take(q, need, counter);
            if (need) {
                n[s] = id;
                l[s] = 0;
                phase[s] = id < N ? kSlotStart : kSlotDone;
                fr[s] = id * L;
            }
            alive |= phase[s] != kSlotDone;
        }
        if (!__any(alive)) break;
        wait_vmem();

        // 3. Consume.  Each slot ends the iteration with at most one
        // buffered entry, then at most one tail fill or flush.
#pragma unroll
        for (int s = 0; s < W; ++s) {
            if (ph[s] == kSlotIdle || ph[s] == kSlotDone) {
                need_block[s] = phase[s] == kSlotStart && L > 0;
                continue;
            }
            if (need_block[s] && ph[s] != kSlotRow) {  // the block fetched above
                const int k = static_cast<int>(fr[s] - rw_base<RW, kGen>(fr[s], rtotal, goff));
                lw_store(rand_area[s], rw[s], blk[s], k);
                need_block[s] = false;
            }
            const int64_t g0 = n[s] * L1;
            const int64_t e0 = n[s] * L;  // edge output index of the walk's step 0
            int64_t g = g0 + l[s];  // output index of the last buffered entry
            int64_t eg = e0 + l[s];  // first edge output index not yet buffered
            int64_t begin = 0, deg = -1;  // row to pick from (deg >= 0: pick)
            bool push = false, fill = false, flush = false;
            uint32_t bad = 0;
            if (ph[s] == kSlotStart) {
                ow[s].count = 0;
                ew[s].count = 0;
                v[s] = row[s].x;
                push = true;
                // {node, begin, degree, pad}, or WideStart {node, degree, begin}
                const int32_t code = kWide ? row[s].y : row[s].z;
                if (code == kRecBadNode) {
                    bad = MLXC_STATUS_BAD_NODE;
                } else if (L == 0) {
                    flush = true;  // (the start's row is not read)
                } else if (kWide && code == kRecLongRow) {
                    phase[s] = kSlotRow;  // the row's bounds come from rowptr
                } else if (code < 0) {
                    bad = MLXC_STATUS_BAD_ROW;
                } else {
                    begin = kWide ? static_cast<int64_t>(
                                        (static_cast<uint64_t>(static_cast<uint32_t>(row[s].w)) << 32) |
                                        static_cast<uint32_t>(row[s].z))
                                  : row[s].y;
                    deg = code;
                }
            } else if (ph[s] == kSlotCol) {
                eg += 1;  // step l's edge was buffered at its pick
                if (!node_ok(cv[s], a.num_nodes)) {
                    bad = MLXC_STATUS_BAD_NODE;
                } else {
                    v[s] = static_cast<int32_t>(cv[s]);
                    l[s] += 1;
                    g += 1;
                    push = true;
                    if (l[s] == L) flush = true;
                    else phase[s] = kSlotRow;
                }
            } else {  // kSlotRow
                const RowBounds rb = {
                    static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(row[s].y)) << 32) |
                                         static_cast<uint32_t>(row[s].x)),
                    static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(row[s].w)) << 32) |
                                         static_cast<uint32_t>(row[s].z))};
                if (!row_ok(rb, a.num_edges)) {
                    bad = MLXC_STATUS_BAD_ROW;
                } else {
                    begin = rb.begin;
                    deg = rb.end - rb.begin;
                }
            }
            if (bad) {
                status |= bad;
                fill = true;  // stop the walk (outputs of a flagged call are unspecified)
            } else if (deg == 0) {
                fill = true;  // absorbing node: the walk stays
            } else if (deg > 0) {
                e[s] = static_cast<EIdx>(begin + pick_index(lw_take(rand_area[s], rw[s]), deg));
                if (kEdges) {
                    if constexpr (kWide) eout[eg] = static_cast<OutT>(e[s]);
                    else ow_push(ew[s], eout, eg, e[s]);
                }
                need_block[s] = rw[s].valid == 0 && l[s] + 1 < L;
                fr[s] = n[s] * L + l[s] + 1;
                phase[s] = kSlotCol;
            }
            if (fill) {
                ow_fill(ow[s], nout, push ? g : g + 1, g0 + L, v[s]);  // v[s] from g on
                if (kEdges) {
                    if constexpr (kWide) {
                        for (int64_t j = eg; j < e0 + L; ++j) eout[j] = static_cast<OutT>(-1);
                    } else {
                        ow_fill(ew[s], eout, eg, e0 + L - 1, -1);
                    }
                }
            } else {
                if (push) ow_push(ow[s], nout, g, v[s]);
                if (flush) {
                    if (ow[s].count) ow_flush(ow[s], nout, g);
                    if (kEdges && !kWide && ew[s].count) ow_flush(ew[s], eout, e0 + L - 1);
                }
            }
            if (fill || flush) phase[s] = kSlotIdle;
        }
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.work), static_cast<unsigned long long>(status));
}

// Uniform walk on a graph small enough for LDS, for calls bound by launch
// latency (the reference tests' Cora-sized workload): every block copies
// rowptr and col, as int32, into its LDS, then runs one walk per thread with
// no global random read at all.  Uniforms are read 8 at a time (one round
// trip per 8 steps); outputs are stored entry by entry, which only small
// calls can afford.  Out-of-range entries are marked -1 on the copy and flag
// the call when a walk meets them, as in the other kernels.


template <bool kGen, bool kEdges, typename OutT>
__global__ __launch_bounds__(kLdsBlock) void uniform_walk_lds_kernel(WalkArgs a) {
    __shared__ int32_t graph[kLdsGraphEntries];
    const int64_t V = a.num_nodes, E = a.num_edges, N = a.num_walks, L = a.walk_length;
    const int64_t goff = kGen ? a.walk_base * L : 0;  // stream position of uniform 0
    int32_t* const rp = graph;          // rowptr, -1 for an entry outside [0, E]
    int32_t* const cl = graph + V + 1;  // col, -1 for a value outside [0, V)
    for (int64_t i = threadIdx.x; i <= V; i += kLdsBlock) {
        const int64_t r = a.rowptr[i];
        rp[i] = r >= 0 && r <= E ? static_cast<int32_t>(r) : -1;
    }
    for (int64_t i = threadIdx.x; i < E; i += kLdsBlock) {
        const int64_t c = a.col[i];
        cl[i] = node_ok(c, V) ? static_cast<int32_t>(c) : -1;
    }
    __syncthreads();
    OutT* const nout = static_cast<OutT*>(a.n_out);
    OutT* const eout = static_cast<OutT*>(a.e_out);
    uint32_t status = 0;
    for (int64_t n = static_cast<int64_t>(blockIdx.x) * kLdsBlock + threadIdx.x; n < N;
         n += static_cast<int64_t>(gridDim.x) * kLdsBlock) {
        const int64_t s = a.start[n];
        OutT* const row = nout + n * (L + 1);
        OutT* const erow = kEdges ? eout + n * L : nullptr;
        row[0] = static_cast<OutT>(s);
        int64_t l = 0;                    // steps taken
        int32_t v = static_cast<int32_t>(s);
        bool stop = !node_ok(s, V);       // a sink or an error ends the walk
        if (stop) status |= MLXC_STATUS_BAD_NODE;
        while (l < L && !stop) {
            float r[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (l + j < L)
                    r[j] = kGen ? philox_uniform_at(goff + n * L + l + j, a.key0, a.key1) : a.rand[n * L + l + j];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (stop || l >= L) break;
                const int32_t b = rp[v], end = rp[v + 1];
                if (b < 0 || end < b) {
                    status |= MLXC_STATUS_BAD_ROW;
                    stop = true;
                } else if (end == b) {
                    stop = true;  // absorbing node: the walk stays
                } else {
                    const int32_t e = b + static_cast<int32_t>(pick_index(r[j], end - b));
                    const int32_t x = cl[e];
                    if (x < 0) {
                        status |= MLXC_STATUS_BAD_NODE;
                        stop = true;
                    } else {
                        row[l + 1] = static_cast<OutT>(x);
                        if (kEdges) erow[l] = static_cast<OutT>(e);
                        v = x;
                        l += 1;
                    }
                }
            }
        }
        for (int64_t j = l + 1; j <= L; ++j) row[j] = static_cast<OutT>(v);  // the walk stays
        if (kEdges)
            for (int64_t j = l; j < L; ++j) erow[j] = static_cast<OutT>(-1);
    }
    if (status) atomicOr(reinterpret_cast<unsigned long long*>(a.work), static_cast<unsigned long long>(status));
}

// ------------------------------------------------------------- launcher

// Walks in flight per lane.  Both walks run best with one slot at the
// higher occupancy it allows (measured on MI355X: configuration 4, CSR walk,
// 6.8 ms with one slot against 8.0 ms with two).
#ifndef MLXC_REC_SLOTS
#define MLXC_REC_SLOTS 1
#endif
#ifndef MLXC_CSR_SLOTS
#define MLXC_CSR_SLOTS 1
#endif
#ifndef MLXC_RAND_WINDOW
#define MLXC_RAND_WINDOW 16    // uniforms per rand block (4-byte floats)
#endif
// Uniforms per generated block (seed=): one Philox call.  Generating costs no
// memory traffic but VALU work, and a wavefront runs the generation whenever
// any of its lanes needs a block, which with 16-uniform blocks (four calls)
// was nearly every iteration.
#ifndef MLXC_GEN_WINDOW
#define MLXC_GEN_WINDOW 4
#endif
// Uniforms per rand block of the packed record walk on walks of at least
// kLongWalk steps: a whole 128-byte line per read, where a 64-byte block
// leaves the line's other half to a later miss.  Configuration 2 (L = 80):
// 7.43 -> 7.39 ms; on short walks most of a long block goes unused
// (configuration 4's CSR walk, L = 20: 6.33 -> 6.85 ms).
#ifndef MLXC_LONG_RAND_WINDOW
#define MLXC_LONG_RAND_WINDOW 32
#endif
constexpr int32_t kLongWalk = 64;

namespace {

enum class UniformMode { kRecords, kCsr, kCsrWide, kLds, kPlain };

// Edge records cost one random read per edge to build; they pay off when the
// call takes several steps per edge, or when the graph is small enough that
// the build is cheaper than a read per step of one walk's chain.  Measured
// on MI355X with the Cora-like graph (10,556 entries): 2,000 walks of 5
// steps 52 us with the CSR walk; 1,280 walks of 20 steps 171 us.
bool records_pay_off(int64_t num_edges, int64_t num_walks, int32_t walk_length) {
    return num_walks * static_cast<int64_t>(walk_length) >= 4 * num_edges ||
           num_edges <= kSmallGraphEdgesPerStep * walk_length;
}

// Edge and start records: 8 bytes each when the graph's ids pack
// (packed_format), else 16.
size_t record_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks) {
    PackedFormat f;
    const size_t each = packed_format(num_nodes, num_edges, f) ? sizeof(uint64_t) : sizeof(EdgeRecord);
    return kRecordOffset + static_cast<size_t>(num_edges + num_walks) * each;
}

size_t init_bytes(int64_t num_walks) {
    return kRecordOffset + static_cast<size_t>(num_walks) * sizeof(EdgeRecord);
}

UniformMode uniform_mode(const WalkArgs& a, size_t workspace_bytes, bool gen) {
    const int64_t rtotal = a.num_walks * a.walk_length;
    const bool rand_ok = gen || (reinterpret_cast<uintptr_t>(a.rand) % 16 == 0 && rtotal % 4 == 0 &&
                                 rtotal >= MLXC_RAND_WINDOW);
    const bool streams_ok = rand_ok && reinterpret_cast<uintptr_t>(a.n_out) % 16 == 0 &&
                            reinterpret_cast<uintptr_t>(a.e_out) % 16 == 0;  // e_out may be null
    if (streams_ok && records_fit(a.num_nodes, a.num_edges)) {
        if (records_pay_off(a.num_edges, a.num_walks, a.walk_length) &&
            workspace_bytes >= record_bytes(a.num_nodes, a.num_edges, a.num_walks))
            return UniformMode::kRecords;
        if (workspace_bytes >= init_bytes(a.num_walks)) return UniformMode::kCsr;
    } else if (streams_ok && a.num_nodes <= INT32_MAX &&
               workspace_bytes >= init_bytes(a.num_walks)) {
        return UniformMode::kCsrWide;  // 2^31 or more entries
    }
    // the LDS walk reads rand and stores its outputs one element at a time:
    // any alignment and length will do
    if (workspace_bytes >= kRecordOffset &&
        lds_walk_fits(a.num_nodes, a.num_edges, a.num_walks, a.walk_length))
        return UniformMode::kLds;
    return UniformMode::kPlain;
}

// Resident blocks per compute unit of the persistent walks (0: as many as
// the kernel's registers allow).  The record walk runs best well below its
// register limit: measured on MI355X at configuration 2, 7.55 ms with 3
// blocks per CU, 7.61 with 2 or 4, 7.68 with 5 and 7.73 with 6 (the same
// order for the seeded and the int32-output variants).  The CSR walk runs
// best with 4 (configuration 4 on one MI355X: 6.07, 5.97, 6.02 and 6.01 ms
// with 3, 4, 5 and 6 blocks per CU).
#ifndef MLXC_REC_BLOCKS_PER_CU
#define MLXC_REC_BLOCKS_PER_CU 3
#endif
#ifndef MLXC_CSR_BLOCKS_PER_CU
#define MLXC_CSR_BLOCKS_PER_CU 4
#endif

template <typename Kernel, typename... Extra>
int launch_walk_kernel(Kernel kernel, int slots, int max_per_cu, const WalkArgs& a,
                       hipStream_t stream, Extra... extra) {
    int grid = 0;
    if (int rc = persistent_grid(kernel, a.num_walks, slots, grid, max_per_cu)) return rc;
    if (int rc = record_walk_event(0, stream)) return rc;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kBlock), 0, stream, a, extra...);
    MLXC_HIP_TRY(hipGetLastError());
    return record_walk_event(1, stream);
}

}  // namespace

size_t uniform_workspace_bytes(int64_t num_nodes, int64_t num_edges, int64_t num_walks,
                               int32_t walk_length) {
    const size_t minimum = MLXC_WORK_WORDS * sizeof(int64_t);
    if (num_nodes < 0 || num_edges < 0 || num_walks < 0 || walk_length < 0) return minimum;
    if (!records_fit(num_nodes, num_edges))  // the wide CSR walk, while node ids fit int32
        return num_nodes <= INT32_MAX ? init_bytes(num_walks) : minimum;
    if (lds_walk_fits(num_nodes, num_edges, num_walks, walk_length))
        return kRecordOffset;  // the LDS walk: its size selects it
    return records_pay_off(num_edges, num_walks, walk_length)
               ? record_bytes(num_nodes, num_edges, num_walks)
               : init_bytes(num_walks);
}

namespace {

template <bool kGen, bool kEdges, typename OutT>
int launch_uniform_impl(const WalkArgs& a, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
    constexpr int RW = kGen ? MLXC_GEN_WINDOW : MLXC_RAND_WINDOW;
    EdgeRecord* recs = reinterpret_cast<EdgeRecord*>(static_cast<char*>(workspace) + kRecordOffset);
    switch (uniform_mode(a, workspace_bytes, kGen)) {
    case UniformMode::kRecords: {
        PackedFormat f;
        const bool packed = packed_format(a.num_nodes, a.num_edges, f);
        if (int rc = launch_record_prep(a.rowptr, a.col, a.start, a.num_nodes, a.num_edges,
                                        a.num_walks, recs, packed ? &f : nullptr, a.work, stream))
            return rc;
        if (packed) {
            const void* recs8 = recs;
            const void* init8 = reinterpret_cast<const uint64_t*>(recs) + a.num_edges;
            if (!kGen && a.walk_length >= kLongWalk)
                return launch_walk_kernel(
                    uniform_walk_rec_kernel<MLXC_REC_SLOTS, kGen ? RW : MLXC_LONG_RAND_WINDOW,
                                            kGen, kEdges, OutT, true>,
                    MLXC_REC_SLOTS, MLXC_REC_BLOCKS_PER_CU, a, stream, recs8, init8, f);
            return launch_walk_kernel(
                uniform_walk_rec_kernel<MLXC_REC_SLOTS, RW, kGen, kEdges, OutT, true>,
                MLXC_REC_SLOTS, MLXC_REC_BLOCKS_PER_CU, a, stream, recs8, init8, f);
        }
        return launch_walk_kernel(
            uniform_walk_rec_kernel<MLXC_REC_SLOTS, RW, kGen, kEdges, OutT, false>,
            MLXC_REC_SLOTS, MLXC_REC_BLOCKS_PER_CU, a, stream, static_cast<const void*>(recs),
            static_cast<const void*>(recs + a.num_edges), f);
    }
    case UniformMode::kCsr: {
        EdgeRecord* init = recs;
        if (int rc = launch_walk_init(a.rowptr, a.start, a.num_nodes, a.num_edges, a.num_walks,
                                      init, a.work, stream))
            return rc;
        return launch_walk_kernel(uniform_walk_csr_kernel<MLXC_CSR_SLOTS, RW, kGen, kEdges, OutT, false>,
                                  MLXC_CSR_SLOTS, MLXC_CSR_BLOCKS_PER_CU, a,
                                  stream,
                                  static_cast<const void*>(init));
    }
    case UniformMode::kCsrWide: {
        WideStart* init = reinterpret_cast<WideStart*>(recs);  // 16 bytes per walk, as EdgeRecord
        int grid = 0;
        if (int rc = stream_grid(a.num_walks, 16, grid)) return rc;
        hipLaunchKernelGGL(wide_init_kernel, dim3(grid), dim3(kBlock), 0, stream, a.rowptr, a.start,
                           a.num_nodes, a.num_edges, a.num_walks, init, a.work);
        MLXC_HIP_TRY(hipGetLastError());
        return launch_walk_kernel(uniform_walk_csr_kernel<MLXC_CSR_SLOTS, RW, kGen, kEdges, OutT, true>,
                                  MLXC_CSR_SLOTS, MLXC_CSR_BLOCKS_PER_CU, a, stream,
                                  static_cast<const void*>(init));
    }
    case UniformMode::kLds: {
        if (int rc = launch_zero_work(a.work, stream)) return rc;
        const int64_t blocks = (a.num_walks + kLdsBlock - 1) / kLdsBlock;  // at most 1024
        if (int rc = record_walk_event(0, stream)) return rc;
        hipLaunchKernelGGL((uniform_walk_lds_kernel<kGen, kEdges, OutT>), dim3(static_cast<int>(blocks)),
                           dim3(kLdsBlock), 0, stream, a);
        MLXC_HIP_TRY(hipGetLastError());
        return record_walk_event(1, stream);
    }
    case UniformMode::kPlain:
        break;
    }
    if (int rc = launch_zero_work(a.work, stream)) return rc;
    return launch_walk_kernel(uniform_walk_kernel<2, kEdges, kGen, OutT>, 2, 0, a, stream);
}

}  // namespace

namespace {

template <typename OutT>
int launch_uniform_typed(const WalkArgs& a, void* workspace, size_t workspace_bytes,
                         bool generate, hipStream_t stream) {
    const bool edges = a.e_out != nullptr;
    if (generate)
        return edges ? launch_uniform_impl<true, true, OutT>(a, workspace, workspace_bytes, stream)
                     : launch_uniform_impl<true, false, OutT>(a, workspace, workspace_bytes, stream);
    return edges ? launch_uniform_impl<false, true, OutT>(a, workspace, workspace_bytes, stream)
                 : launch_uniform_impl<false, false, OutT>(a, workspace, workspace_bytes, stream);
}

}  // namespace

int launch_uniform(const WalkArgs& a, void* workspace, size_t workspace_bytes, bool generate,
                   int32_t out_type, hipStream_t stream) {
    return out_type == MLXC_OUT_INT32
               ? launch_uniform_typed<int32_t>(a, workspace, workspace_bytes, generate, stream)
               : launch_uniform_typed<int64_t>(a, workspace, workspace_bytes, generate, stream);
}

}  // namespace mlxc
