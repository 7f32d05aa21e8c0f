/*
 * CPU oracle for the random-walk hot path of vinayhpandya/mlx_cluster.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU path is
 * compared with; it is never part of the product.  Only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 *
 * Every function restates the reference's CPU evaluation in plain C:
 *   uniform walk  <- /root/reference/random_walks/RandomWalk.cpp:41-60
 *   node2vec walk <- /root/reference/random_walks/BiasedRandomWalk.cpp:20-28,52-100
 * with the randomness replaced by a position-addressed Philox4x32-10 stream
 * where the reference used libc rand() (the libc-driven restatement is kept
 * too, for distribution tests and timing).
 */
#ifndef MLXC_WALK_ORACLE_H
#define MLXC_WALK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Rule selector for the node2vec acceptance test. */
#define ORACLE_RULE_REF_CHAIN 0      /* BiasedRandomWalk.cpp:86-91, verbatim chain */
#define ORACLE_RULE_NODE2VEC_EXACT 1 /* analytic node2vec: accept iff r < p_d      */

/* Trial cap per biased step.  The reference loops without bound
 * (BiasedRandomWalk.cpp:80); both this oracle and the HIP kernel stop after
 * this many rejected candidates and keep the last one. */
#define ORACLE_MAX_TRIALS 65536

/* Work counts that feed the roofline (one 64-B line per dependent read). */
typedef struct {
    int64_t moving_steps;     /* steps taken from a node with deg > 0           */
    int64_t sink_walks;       /* walks that met a deg-0 node before their end    */
    int64_t trials;           /* candidate draws (node2vec; deg==1 counts one)   */
    int64_t member_tests;     /* neighbour tests that were actually evaluated    */
    int64_t member_lines;     /* distinct 64-B col lines probed by those tests   */
} oracle_counts;

/* One Philox4x32-10 block (Salmon et al., SC'11): 10 rounds, multipliers
 * 0xD2511F53 / 0xCD9E8D57, Weyl key bumps 0x9E3779B9 / 0xBB67AE85. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* u = (x >> 8) * 2^-24, a float in [0, 1 - 2^-24]. */
float oracle_u32_to_unit_float(uint32_t x);

/* out[i] = unit float of word (i % 4) of Philox(ctr = (i/4 lo, i/4 hi, 0, 0),
 * key = (seed lo, seed hi)). */
void oracle_philox_uniform_fill(float* out, int64_t n, uint64_t seed);

/* Elements [first, first + n) of the same stream: out[i] is element
 * first + i (the uniforms of walks [w0, w1) of an L-step seeded uniform walk
 * are elements [w0 * L, w1 * L)). */
void oracle_philox_uniform_fill_at(float* out, int64_t first, int64_t n, uint64_t seed);

/* Trial-0 candidate uniform of the node2vec stream, materialised as a
 * [N, L] rand tensor: out[n*L + l] = u0(seed; n, l, 0). */
void oracle_node2vec_trial0_u0(float* out, int64_t N, int32_t L, uint64_t seed);

/* Candidate index inside a row of length deg > 0 from a uniform r:
 * (int64)(r * (float)deg) in float32 (RandomWalk.cpp:52), clamped to
 * [0, deg-1] (only reachable for r outside [0,1) or deg > 2^24). */
int64_t oracle_pick_index(float r, int64_t deg);

/* Uniform random walk, RandomWalk.cpp:41-60.  e_out may be NULL.  counts may
 * be NULL.  Returns 0, or -1 when an index leaves the graph (the reference
 * would read out of bounds there). */
int oracle_uniform_walk(const int64_t* rowptr, int64_t num_nodes,
                        const int64_t* col, int64_t num_edges,
                        const int64_t* start, int64_t num_walks,
                        const float* rand, int32_t walk_length,
                        int64_t* n_out, int64_t* e_out, oracle_counts* counts);

/* Acceptance constants, BiasedRandomWalk.cpp:52-55. */
void oracle_node2vec_probs(double p, double q, double probs[3]);

/* node2vec walk by rejection sampling, BiasedRandomWalk.cpp:57-100, driven
 * by the Philox stream u0/u1(seed; walk, step, trial) where walk n of this
 * call has stream index first_walk + n (so any block of a larger call can be
 * recomputed).  Rows are searched with a linear scan when rows_sorted == 0
 * (BiasedRandomWalk.cpp:20-28) and with lower_bound otherwise (same answer on
 * sorted rows). */
int oracle_node2vec_walk(const int64_t* rowptr, int64_t num_nodes,
                         const int64_t* col, int64_t num_edges,
                         const int64_t* start, int64_t num_walks, int64_t first_walk,
                         int32_t walk_length, double p, double q,
                         uint64_t seed, int32_t rule, int32_t rows_sorted,
                         int64_t* n_out, int64_t* e_out, oracle_counts* counts);

/* The same walk driven by libc rand() exactly as the reference draws it
 * (rand() % deg for the candidate, rand()/RAND_MAX for the test), for
 * distribution tests and the CPU timing baseline.  srand(libc_seed) first.
 * The reference chain is evaluated as written, with its linear is_neighbor
 * scan on every trial whose first clause fails, so the timing is the
 * reference's. */
int oracle_node2vec_walk_libc(const int64_t* rowptr, int64_t num_nodes,
                              const int64_t* col, int64_t num_edges,
                              const int64_t* start, int64_t num_walks,
                              int32_t walk_length, double p, double q,
                              uint32_t libc_seed, int32_t rule,
                              int64_t* n_out, int64_t* e_out);

/* CSR checks used by the tests: bit0 rowptr malformed, bit1 col out of range,
 * bit2 some row not sorted ascending, bit3 (only when bits 0-2 are clear)
 * some entry (u, v) without an entry (v, u). */
int32_t oracle_csr_flags(const int64_t* rowptr, int64_t num_nodes,
                         const int64_t* col, int64_t num_edges);

#ifdef __cplusplus
}
#endif
#endif
