/*
 * mlxc — C ABI of the MI355X random-walk library (libmlxc.so).
 *
 * The drop-in boundary for the random-walk hot path of vinayhpandya/mlx_cluster.
 * Plain pointers and sizes only.  Every pointer argument named d_* is a
 * device pointer (HIP/torch allocation on the current device); `stream` is a
 * hipStream_t (NULL = the legacy default stream).  All walk entry points are
 * asynchronous on `stream`: they enqueue work and return.
 *
 * Return codes: 0 on success, a negative MLXC_ERR_* code otherwise; the
 * message of the calling thread's last failure is in mlxc_last_error().
 * Every walk_length is in [0, 2^31 - 2]: a walk's row holds walk_length + 1
 * entries.
 *
 * Ownership: the caller allocates every buffer (inputs, outputs and the small
 * status/work buffers).  The library never allocates or frees device memory.
 */
#ifndef MLXC_H
#define MLXC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLXC_OK 0
#define MLXC_ERR_INVALID_ARGUMENT (-1)
#define MLXC_ERR_HIP (-2)

/* Device workspace.  Every walk entry point takes `d_workspace` (16-byte
 * aligned, at least MLXC_WORK_WORDS int64 words) and its size in bytes.  The
 * call zeroes the first MLXC_WORK_WORDS words on `stream` before its kernels
 * run; after the call has completed, word 0 holds the MLXC_STATUS_* bits of
 * that call (the other words are internal: the walk-queue counter).  A
 * workspace of the size the *_workspace_bytes queries return also holds
 * per-call layouts of the graph and the starts (8- or 16-byte records: node,
 * row begin, row degree) that cut the dependent reads per step; with a smaller
 * workspace the kernels read the CSR arrays directly.  For graphs small
 * enough (see the queries), a workspace of exactly the 256-byte header runs
 * the walk with the whole CSR in on-chip memory.  Same results every way. */
#define MLXC_WORK_WORDS 4

/* Bits a walk kernel ORs into workspace word 0 when the graph or the starts
 * are malformed (the reference reads out of bounds in these cases; these
 * kernels never do — the affected walk stops and its remaining output
 * entries are unspecified).  Which entries are checked does not depend on
 * the kernel path the workspace selects, nor on the uniforms drawn:
 *   mlxc_random_walk (and _seeded) reports the entries its walks read, which
 *     are those the reference's loop reads (RandomWalk.cpp:45-54): a start
 *     outside [0, num_nodes), the rowptr pair of a node a walk leaves, and
 *     a chosen col entry.  The row of the node a walk ends at is not read.
 *   mlxc_rejection_sampling validates the whole CSR on every call
 *     (rowptr[0] == 0, rowptr[num_nodes] == num_edges, non-decreasing; every
 *     col entry in [0, num_nodes)) and every start.
 * The host twins report the same bits. */
#define MLXC_STATUS_BAD_NODE 1 /* a start or col value outside [0, num_nodes) */
#define MLXC_STATUS_BAD_ROW 2  /* rowptr[v] / rowptr[v+1] outside [0, num_edges] or decreasing */

/* Acceptance rules of mlxc_rejection_sampling. */
#define MLXC_RULE_REF_CHAIN 0      /* BiasedRandomWalk.cpp:86-91, reproduced term for term */
#define MLXC_RULE_NODE2VEC_EXACT 1 /* analytic node2vec: accept iff r < prob_d(t, x)      */

/* Row order of the graph passed to mlxc_rejection_sampling. */
#define MLXC_ROWS_UNSORTED 0  /* scan rows linearly, as the reference's is_neighbor does */
#define MLXC_ROWS_SORTED 1    /* the caller promises every row is sorted ascending */
#define MLXC_ROWS_DETECT 2    /* the call checks the rows on the device (and validates the CSR) */
/* OR-ed into one of the three above: the caller promises the graph is
 * symmetric (every (u, v) entry has a (v, u) entry), so that "t in row(x)"
 * equals "x in row(t)" and the neighbour test may search the shorter row.
 * Results are those of the reference when the promise holds, unspecified
 * otherwise.  Record kernels only; the other paths ignore it. */
#define MLXC_ROWS_SYMMETRIC 4

/* Bits written by mlxc_csr_check. */
#define MLXC_CSR_BAD_ROWPTR 1   /* rowptr[0] != 0, rowptr[V] != E, or decreasing */
#define MLXC_CSR_BAD_COL 2      /* a col value outside [0, V) */
#define MLXC_CSR_UNSORTED 4     /* some row is not sorted ascending */
/* some entry (u, v) has no entry (v, u): the graph breaks the promise of
 * MLXC_ROWS_SYMMETRIC.  Checked (one search per entry) only on a graph with
 * none of the three bits above set; otherwise left clear. */
#define MLXC_CSR_ASYMMETRIC 8

/* Element type of the walk outputs (out_type argument).  The reference
 * writes int64 (RandomWalk.cpp:43,57-58); int32 halves the output bytes and
 * needs num_nodes (and, with edge output, num_edges) below 2^31. */
#define MLXC_OUT_INT64 0
#define MLXC_OUT_INT32 1

/* flags of mlxc_csr_build. */
#define MLXC_CSR_SYMMETRIZE 1 /* also add every reversed pair (col, row) */
#define MLXC_CSR_DEDUP 2      /* keep one entry of each repeated (row, col) pair */

/* Trial cap of one biased step (the reference loops without bound,
 * BiasedRandomWalk.cpp:80): after this many rejections the last candidate is
 * kept. */
#define MLXC_MAX_TRIALS 65536

/* Library version, major*10000 + minor*100 + patch. */
int mlxc_version(void);

/* Message of the calling thread's most recent failed call ("" if none). */
const char* mlxc_last_error(void);

/* Workspace bytes that let mlxc_random_walk use its fastest layout for this
 * call:
 *   256 when num_nodes + 1 + num_edges <= 14336 and the call takes 1 to 2^20
 *     steps (num_walks <= 2^20): the walk runs with rowptr and col in LDS;
 *   256 + R * (num_edges + num_walks) when the call takes at least
 *     4 * num_edges steps, or num_edges <= 32768 * walk_length (per-call edge
 *     records): R = 8 when the bits of num_nodes - 1 and of num_edges add up
 *     to at most 48 (node, row begin and degree packed in 64 bits), else 16;
 *   else 256 + 16 * num_walks (start records only);
 *   256 + 16 * num_walks also when num_edges is 2^31 or more (and num_nodes
 *     below 2^31): start records with 64-bit row begins for the CSR walk;
 *   MLXC_WORK_WORDS * 8 when num_nodes is 2^31 or more.
 * No reference counterpart (the reference allocates inside eval,
 * RandomWalk.cpp:28-29). */
size_t mlxc_random_walk_workspace_bytes(int64_t num_nodes, int64_t num_edges,
                                        int64_t num_walks, int32_t walk_length);

/* Workspace bytes for mlxc_rejection_sampling's fastest layout for these
 * arguments (same conventions).  Either edge records (16 bytes per edge), or
 * the CSR mode's layout, which reads each candidate's node id and then, only
 * when the decision needs it, its rowptr pair.  CSR mode is chosen when
 * num_walks * walk_length * (1 + 4 w) < 4 * num_edges, w being the share of
 * acceptance draws r that can need a row search (|prob1 - prob2| for
 * MLXC_RULE_NODE2VEC_EXACT, max(0, prob1 - prob2) for the chain).  Both
 * layouts add 16 bytes per walk, about 4.3 bytes per edge of search index and
 * 4 bytes per node of int32 row starts (the rows the preparation pass and the
 * CSR mode read).
 * Records are also chosen when num_edges <= 32768 * walk_length, and 256
 * bytes (the LDS walk) under the same conditions as for mlxc_random_walk.
 * When the call makes row searches (w > 0), the record layout ends with two
 * more parts: per-row hash tables (64 * (num_edges / 8 + num_nodes + 2)
 * bytes), which answer a membership test on a row of 2 to 1023 entries in
 * one read, then dense neighbour bitmaps of the rows of highest degree
 * (ceil(num_nodes / 32) words each, at most 1 GiB and one per 256 entries,
 * plus 4 * num_nodes bytes of slot map), which do the same for those rows.
 * A workspace that ends before the bitmaps runs without them, one that ends
 * before the tables without both; mlxc_rejection_sampling_layout_bytes gives
 * each size.  No reference counterpart. */
size_t mlxc_rejection_sampling_workspace_bytes(int64_t num_nodes, int64_t num_edges,
                                               int64_t num_walks, int32_t walk_length,
                                               double p, double q, int32_t rule);

/* Layouts of mlxc_rejection_sampling, smallest first.  The call runs the
 * largest one its workspace holds, with the same results every way. */
#define MLXC_N2V_LAYOUT_DIRECT 0        /* MLXC_WORK_WORDS words: the direct CSR kernel */
#define MLXC_N2V_LAYOUT_LDS 1           /* the 256-byte header: the LDS walk (small graphs) */
#define MLXC_N2V_LAYOUT_CSR 2           /* CSR mode: start records, search index, row starts */
#define MLXC_N2V_LAYOUT_RECORDS 3       /* edge records instead of CSR mode */
#define MLXC_N2V_LAYOUT_RECORDS_HASH 4  /* ... and the row hash tables */
#define MLXC_N2V_LAYOUT_RECORDS_FULL 5  /* ... and the hub bitmaps */

/* Workspace bytes of one MLXC_N2V_LAYOUT_* layout for these sizes (0 when it
 * does not apply: the LDS walk beyond its size limits, the CSR-mode and
 * record layouts for ids of 2^31 or more), for callers that trade speed for
 * memory and for tests that run every kernel path.  No reference
 * counterpart. */
size_t mlxc_rejection_sampling_layout_bytes(int64_t num_nodes, int64_t num_edges,
                                            int64_t num_walks, int32_t walk_length,
                                            int32_t layout);

/*
 * Uniform random walk.
 * Replaces: RandomWalk::eval_cpu / eval_gpu and the op random_walk(rowptr,
 *   col, start, rand, walk_length) —
 *   /root/reference/random_walks/RandomWalk.cpp:18-62 (CPU), :73-108 (GPU
 *   dispatch), :138-148 (op); /root/reference/random_walks/RandomWalk.h:56-61;
 *   binding /root/reference/bindings.cpp:12-33.
 *
 * d_rowptr  int64 [num_nodes + 1]     d_col  int64 [num_edges]
 * d_start   int64 [num_walks]         d_rand float32 [num_walks * walk_length]
 * d_n_out   [num_walks * (walk_length + 1)]  (row-major [N, L+1])
 * d_e_out   [num_walks * walk_length] or NULL (edge ids, -1 = stayed)
 * out_type  MLXC_OUT_INT64 or MLXC_OUT_INT32: element type of both outputs
 * d_workspace, workspace_bytes: device workspace (see above).
 *
 * Step l of walk n at node v: deg = rowptr[v+1] - rowptr[v]; deg == 0 keeps
 * v; otherwise e = rowptr[v] + (int64)(rand[n*L + l] * (float)deg) in IEEE
 * float32 (truncated; clamped to [0, deg-1]) and v = col[e].
 */
int mlxc_random_walk(const int64_t* d_rowptr, int64_t num_nodes,
                     const int64_t* d_col, int64_t num_edges,
                     const int64_t* d_start, int64_t num_walks,
                     const float* d_rand, int32_t walk_length,
                     void* d_n_out, void* d_e_out, int32_t out_type,
                     void* d_workspace, size_t workspace_bytes, void* stream);

/* Bytes of the device scratch array that mlxc_random_walk_noalloc uses in
 * place of a workspace (one array per GPU, held until the process ends). */
#define MLXC_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024)

/*
 * mlxc_random_walk without a workspace argument: allocates nothing.
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory around the call (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  The kernels, layouts and results are
 * those of mlxc_random_walk with a workspace of
 * min(mlxc_random_walk_workspace_bytes(num_nodes, num_edges, num_walks,
 * walk_length), MLXC_NOALLOC_SCRATCH_BYTES) bytes; that workspace lives in a
 * file-scope device array of MLXC_NOALLOC_SCRATCH_BYTES per GPU instead.  A
 * call whose fastest layout needs more runs the largest one the array holds
 * (start records only, or the direct kernel): the same walks, more slowly.
 * d_status (device pointer to one int64, or NULL) receives the call's
 * MLXC_STATUS_* bits on `stream`.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (different streams, or host threads
 * without ordering) race and must not be issued.  The first call on each GPU
 * looks up the array's device address (hipGetSymbolAddress) once.
 */
int mlxc_random_walk_noalloc(const int64_t* d_rowptr, int64_t num_nodes,
                             const int64_t* d_col, int64_t num_edges,
                             const int64_t* d_start, int64_t num_walks,
                             const float* d_rand, int32_t walk_length,
                             void* d_n_out, void* d_e_out, int32_t out_type,
                             int64_t* d_status, void* stream);

/*
 * Uniform random walk that generates its uniforms instead of reading a rand
 * tensor: the same walk as mlxc_random_walk with
 *   rand[n*L + l] = (w >> 8) * 2^-24, w = word (i % 4) of
 *   Philox4x32-10(key = seed; counter = (i/4 lo, i/4 hi, 0, 0)),
 *   i = (first_walk + n)*L + l,
 * i.e. bit-identical to mlxc_random_walk on elements [first_walk * L,
 * (first_walk + num_walks) * L) of the output of mlxc_philox_uniform(rand,
 * (first_walk + num_walks) * walk_length, seed).  Saves the 4-byte-per-step
 * rand stream and the pass that writes it.
 * first_walk (>= 0) is the index of this call's walk 0 in a larger batch:
 * walks [i0, i1) of a batch are rows i0 .. i1-1 of the whole batch's call
 * when called on start[i0:i1] with first_walk = i0, so a batch can be run in
 * slices (on one GPU, or one slice per GPU) with bit-identical results.
 * Extends: the reference's rand input, made by mx.random.uniform before the
 *   call (/root/reference/tests/test_random_walk.py:31-36).
 */
int mlxc_random_walk_seeded(const int64_t* d_rowptr, int64_t num_nodes,
                            const int64_t* d_col, int64_t num_edges,
                            const int64_t* d_start, int64_t num_walks,
                            int32_t walk_length, uint64_t seed, int64_t first_walk,
                            void* d_n_out, void* d_e_out, int32_t out_type,
                            void* d_workspace, size_t workspace_bytes, void* stream);

/*
 * node2vec walk by rejection sampling.
 * Replaces: BiasedRandomWalk::eval_cpu and the op rejection_sampling(rowptr,
 *   col, start, walk_length, p, q) —
 *   /root/reference/random_walks/BiasedRandomWalk.cpp:30-102 (CPU; its GPU
 *   path :150-155 only throws), :183-193 (op);
 *   /root/reference/random_walks/BiasedRandomWalk.h:58-64;
 *   binding /root/reference/bindings.cpp:35-63.
 *
 * The reference draws from libc rand(); this entry point draws from the
 * counter-based stream Philox4x32-10(key = seed; counter = (walk lo, walk hi,
 * step, trial)) with walk = first_walk + n for walk n of the call (>= 0; a
 * call on start[i0:i1] with first_walk = i0 gives rows i0 .. i1-1 of the
 * whole batch's call): word 0 picks the candidate as in mlxc_random_walk,
 * word 1 gives r = (x1 >> 8) * 2^-24 for the acceptance test against the FP64
 * constants of BiasedRandomWalk.cpp:52-55.  `rows` is one of MLXC_ROWS_*:
 * sorted rows are searched through a 16-ary index, unsorted rows scanned
 * linearly as the reference does; MLXC_ROWS_DETECT decides on the device in
 * the call's preparation pass, the pass that also validates the whole CSR
 * (status bits as above, for every MLXC_ROWS_* value).  No host
 * synchronisation on any path.
 */
int mlxc_rejection_sampling(const int64_t* d_rowptr, int64_t num_nodes,
                            const int64_t* d_col, int64_t num_edges,
                            const int64_t* d_start, int64_t num_walks,
                            int32_t walk_length, double p, double q,
                            uint64_t seed, int64_t first_walk, int32_t rule, int32_t rows,
                            void* d_n_out, void* d_e_out, int32_t out_type,
                            void* d_workspace, size_t workspace_bytes, void* stream);

/*
 * Validates a CSR graph on the device and reports MLXC_CSR_* bits in
 * *h_flags (host pointer).  Synchronises `stream`.  d_workspace: at least
 * MLXC_WORK_WORDS int64 words of device memory supplied by the caller.
 * No reference counterpart: the reference validates nothing (its
 * is_neighbor, BiasedRandomWalk.cpp:20-28, works on unsorted rows); this
 * picks the neighbour-test strategy for mlxc_rejection_sampling.
 */
int mlxc_csr_check(const int64_t* d_rowptr, int64_t num_nodes,
                   const int64_t* d_col, int64_t num_edges,
                   void* d_workspace, size_t workspace_bytes, int32_t* h_flags,
                   void* stream);

/*
 * Uniform float32 fill from Philox4x32-10: out[i] = (w >> 8) * 2^-24 with w
 * word (i % 4) of Philox(key = seed; counter = (i/4 lo, i/4 hi, 0, 0)).
 * Stands in for mx.random.uniform, which makes the reference tests' rand
 * tensor (/root/reference/tests/test_random_walk.py:31).
 */
int mlxc_philox_uniform(float* d_out, int64_t n, uint64_t seed, void* stream);

/* Workspace bytes mlxc_csr_build needs (at least 16-byte aligned): two key
 * arrays of 4 bytes per entry (5 when num_nodes > 65536, 6 when num_nodes >
 * 2^20, 8 when num_nodes > 2^24), entries = num_edges, or 2 * num_edges with
 * MLXC_CSR_SYMMETRIZE, plus 1 byte per entry of digits, 8 bytes per 16
 * entries of digit counts and a few KB of totals and block sums.  No
 * reference counterpart. */
size_t mlxc_csr_build_workspace_bytes(int64_t num_nodes, int64_t num_edges, int32_t flags);

/*
 * CSR of an edge list, built on the device: rows sorted by (row, col),
 * rowptr over all num_nodes rows (rows without entries included).
 * Replaces: the CSR pipeline of the reference tests,
 *   /root/reference/tests/test_random_walk.py:23-28 (and
 *   test_rejection_sampling.py:22-27): mlx_graphs 0.0.7 sort_edge_index
 *   (lexicographic (row, col) order, duplicates kept), then rowptr =
 *   [0, cumsum(np.unique(row, return_counts=True))], which drops rows
 *   without entries; here rowptr always has num_nodes + 1 entries.
 *
 * d_row, d_col  int64 [num_edges]: entry i is the pair (row[i], col[i])
 * num_nodes     V, at most 2^32; every id must lie in [0, V)
 * flags         MLXC_CSR_SYMMETRIZE | MLXC_CSR_DEDUP (or 0)
 * d_rowptr      int64 [V + 1]
 * d_col_out     int64 [num_edges] (2 * num_edges with MLXC_CSR_SYMMETRIZE)
 * d_workspace   mlxc_csr_build_workspace_bytes() bytes, 16-byte aligned.
 *
 * Asynchronous on `stream`.  After completion, workspace word 0 holds
 * MLXC_STATUS_BAD_NODE if some id lay outside [0, V) (the output is then
 * unspecified but every write stays inside the buffers), and word 1 the
 * number of entries written to d_col_out (= d_rowptr[V]).
 */
int mlxc_csr_build(const int64_t* d_row, const int64_t* d_col, int64_t num_edges,
                   int64_t num_nodes, int32_t flags, int64_t* d_rowptr, int64_t* d_col_out,
                   void* d_workspace, size_t workspace_bytes, void* stream);

/*
 * Host twin of mlxc_csr_build: the same CSR from host arrays, on the calling
 * thread.  *count receives the entries written to col_out, *status (may be
 * NULL) the MLXC_STATUS_* bits.  No workspace.
 */
int mlxc_csr_build_cpu(const int64_t* row, const int64_t* col, int64_t num_edges,
                       int64_t num_nodes, int32_t flags, int64_t* rowptr, int64_t* col_out,
                       int64_t* count, int64_t* status);

/*
 * Skip-gram context windows of walks, the step after the walk in node2vec
 * training.  No reference counterpart (the reference stops at the walks,
 * /root/reference/random_walks/BiasedRandomWalk.cpp:96); the layout is that
 * of torch_geometric's Node2Vec.pos_sample: with W = walk_nodes -
 * context_size + 1 windows per walk, window-major,
 *   d_out[(j * N + n) * C + k] = d_walks[n * walk_nodes + j + k]
 * for j < W, k < C = context_size, n < N = num_walks.
 *
 * d_walks    [N, walk_nodes] row-major, element type elem_type (MLXC_OUT_*)
 * d_out      [W * N, C], the same element type
 * walk_nodes in [1, 65536 / element size]; context_size in [1, min(32,
 * walk_nodes)].  One launch takes at most 16,777,215 tiles of walks (a tile
 * is min(64, 65536 / (walk_nodes * element size)) walks): larger calls fail
 * with MLXC_ERR_INVALID_ARGUMENT and are split by the caller.
 * Asynchronous on `stream`; no workspace.
 */
int mlxc_context_windows(const void* d_walks, int64_t num_walks, int32_t walk_nodes,
                         int32_t context_size, int32_t elem_type, void* d_out, void* stream);

/*
 * Negative context windows (torch_geometric Node2Vec.neg_sample layout): the
 * windows of mlxc_context_windows over the walks
 *   [start[n], u(n, 1), ..., u(n, walk_length)],
 * u(n, l) = (x * num_nodes) >> 32 with x = word 0 of Philox4x32-10(key =
 * seed; counter = (n lo, n hi, l, 0)): nodes drawn uniformly from
 * [0, num_nodes), num_nodes in [1, 2^32].  start values are copied as given.
 * out_type MLXC_OUT_INT64 or MLXC_OUT_INT32 (num_nodes and start values
 * below 2^31).  walk_length + 1 >= context_size, and (walk_length + 1) times
 * the element size at most 64 KiB.  No reference counterpart.
 */
int mlxc_negative_windows(const int64_t* d_start, int64_t num_walks, int32_t walk_length,
                          int32_t context_size, int64_t num_nodes, uint64_t seed,
                          int32_t out_type, void* d_out, void* stream);

/* Host twins of the two window entry points (host pointers, same output). */
int mlxc_context_windows_cpu(const void* walks, int64_t num_walks, int32_t walk_nodes,
                             int32_t context_size, int32_t elem_type, void* out);
int mlxc_negative_windows_cpu(const int64_t* start, int64_t num_walks, int32_t walk_length,
                              int32_t context_size, int64_t num_nodes, uint64_t seed,
                              int32_t out_type, void* out);

/*
 * Host twins of the three walk entry points: the same walks, the same
 * arguments with host pointers, evaluated on up to `threads` CPU threads
 * (<= 0: one per hardware thread; small calls use fewer, since starting a
 * thread costs more than thousands of steps) and returning when done.  Outputs are
 * bit-identical to the device entry points for the same inputs and seed.
 * *status (may be NULL) receives the MLXC_STATUS_* bits that the device
 * entry points leave in workspace word 0; no workspace is needed.
 * Replace: the eval_cpu paths the reference takes for stream=mx.cpu —
 *   /root/reference/random_walks/RandomWalk.cpp:18-62 and
 *   /root/reference/random_walks/BiasedRandomWalk.cpp:30-102 (serial loops
 *   there; the biased one draws from libc rand(), these from the Philox
 *   stream of mlxc_rejection_sampling).
 */
int mlxc_random_walk_cpu(const int64_t* rowptr, int64_t num_nodes,
                         const int64_t* col, int64_t num_edges,
                         const int64_t* start, int64_t num_walks,
                         const float* rand, int32_t walk_length,
                         void* n_out, void* e_out, int32_t out_type,
                         int32_t threads, int64_t* status);

int mlxc_random_walk_seeded_cpu(const int64_t* rowptr, int64_t num_nodes,
                                const int64_t* col, int64_t num_edges,
                                const int64_t* start, int64_t num_walks,
                                int32_t walk_length, uint64_t seed, int64_t first_walk,
                                void* n_out, void* e_out, int32_t out_type,
                                int32_t threads, int64_t* status);

int mlxc_rejection_sampling_cpu(const int64_t* rowptr, int64_t num_nodes,
                                const int64_t* col, int64_t num_edges,
                                const int64_t* start, int64_t num_walks,
                                int32_t walk_length, double p, double q,
                                uint64_t seed, int64_t first_walk, int32_t rule, int32_t rows,
                                void* n_out, void* e_out, int32_t out_type,
                                int32_t threads, int64_t* status);

/*
 * Publishes a call's status word to host memory without a device-to-host
 * copy: enqueues on `stream` a one-thread kernel that stores workspace word 0
 * (the MLXC_STATUS_* bits of the walk call enqueued before it on the same
 * stream and workspace) into h_status[1], then 1 into h_status[0], both as
 * system-scope stores.  Once h_status[0] reads 1 on the host (an acquire
 * load), h_status[1] holds the bits and the walk call has completed.  The
 * caller sets h_status[0] to 0 before the call and owns h_status: host
 * memory of at least 16 bytes, 8-byte aligned, that the device can write
 * (hipHostMalloc with hipHostMallocCoherent).  For callers that wait for each
 * call's status (a validated call of a few microseconds, where a copy of the
 * word back to the host costs more than the walk).  No reference
 * counterpart.
 */
int mlxc_publish_status(const void* d_workspace, int64_t* h_status, void* stream);

/*
 * Measurement hook: times the walk kernel alone, without the preparation
 * launches before it (a call's last launch is its walk kernel).  After
 * mlxc_set_walk_events(start_event, stop_event), with two hipEvent_t handles
 * created by the caller, every walk call the calling thread makes
 * (mlxc_random_walk*, mlxc_rejection_sampling) records start_event on its
 * stream right before its walk kernel and stop_event right after it;
 * hipEventElapsedTime between them is that kernel's duration.
 * mlxc_set_walk_events(NULL, NULL) stops the recording.  A call without
 * walks launches no walk kernel and records neither event.  Returns
 * MLXC_ERR_INVALID_ARGUMENT if exactly one handle is NULL.  No reference
 * counterpart.
 */
int mlxc_set_walk_events(void* start_event, void* stop_event);

/*
 * Diagnostic: random reads from a device table, the measurement behind the
 * walks' random-read ceiling (a walk step is one or two dependent reads at
 * random addresses, so the walk kernels are bound by how many such reads the
 * device completes per second).  Launches blocks_per_cu blocks of 256
 * threads per compute unit; each thread runs `iterations` rounds of
 * loads_per_lane (1, 2, 4 or 8) reads of load_bytes (4 or 16) bytes at
 * addresses uniform over the table (aligned to load_bytes).  dependent = 1
 * makes each read's address depend on the value the same chain read in the
 * round before, as a walk's next read depends on the record it just read.
 * *loads_issued (host) receives the number of reads the launch makes; time
 * the launch on `stream` to get reads per second.  d_table is 16-byte
 * aligned, table_bytes in [load_bytes, load_bytes * (2^32 - 1)]; iterations
 * in [1, 2^24]; blocks_per_cu in [1, 32].  d_sink (one uint32 of device
 * memory) is written only in the unlikely event that the XOR of the values
 * read equals a fixed constant, which keeps the reads from being removed.
 * No reference counterpart.
 */
int mlxc_gather_probe(const void* d_table, int64_t table_bytes, int32_t load_bytes,
                      int32_t loads_per_lane, int32_t dependent, int32_t blocks_per_cu,
                      int64_t iterations, uint64_t seed, uint32_t* d_sink,
                      int64_t* loads_issued, void* stream);

#ifdef __cplusplus
}
#endif
#endif
