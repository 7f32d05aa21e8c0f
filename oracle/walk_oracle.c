/*
 * CPU oracle for the random-walk hot path (TEST INFRASTRUCTURE ONLY: never
 * linked into or called by the product; tests, smoke() and the cpu_baseline
 * leg of bench.py are its only users).
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math), so float
 * arithmetic is IEEE single precision with round-to-nearest, as the reference
 * computes it.
 */
#include "walk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- Philox */

#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u

void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
        uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += PHILOX_W0;
        k1 += PHILOX_W1;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float oracle_u32_to_unit_float(uint32_t x) {
    return (float)(x >> 8) * (1.0f / 16777216.0f);
}

void oracle_philox_uniform_fill(float* out, int64_t n, uint64_t seed) {
    oracle_philox_uniform_fill_at(out, 0, n, seed);
}

void oracle_philox_uniform_fill_at(float* out, int64_t first, int64_t n, uint64_t seed) {
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    uint64_t have = UINT64_MAX;  /* block whose words are in w */
    for (int64_t i = 0; i < n; ++i) {
        uint64_t pos = (uint64_t)(first + i);
        uint64_t blk = pos >> 2;
        if (blk != have) {
            uint32_t ctr[4] = {(uint32_t)blk, (uint32_t)(blk >> 32), 0u, 0u};
            oracle_philox4x32_10(ctr, key, w);
            have = blk;
        }
        out[i] = oracle_u32_to_unit_float(w[pos & 3]);
    }
}

/* Two uniforms of the node2vec stream at (walk, step, trial). */
static void n2v_uniforms(uint64_t seed, int64_t walk, int32_t step, uint32_t trial,
                         float* u0, float* u1) {
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t ctr[4] = {(uint32_t)(uint64_t)walk, (uint32_t)((uint64_t)walk >> 32),
                       (uint32_t)step, trial};
    uint32_t w[4];
    oracle_philox4x32_10(ctr, key, w);
    *u0 = oracle_u32_to_unit_float(w[0]);
    *u1 = oracle_u32_to_unit_float(w[1]);
}

void oracle_node2vec_trial0_u0(float* out, int64_t N, int32_t L, uint64_t seed) {
    for (int64_t n = 0; n < N; ++n)
        for (int32_t l = 0; l < L; ++l) {
            float u0, u1;
            n2v_uniforms(seed, n, l, 0u, &u0, &u1);
            out[n * (int64_t)L + l] = u0;
        }
}

/* ------------------------------------------------------- index selection */

int64_t oracle_pick_index(float r, int64_t deg) {
    /* RandomWalk.cpp:51-53: static_cast<int64_t>(r * (row_end - row_start))
     * with r float, so the degree is converted to float and the product is a
     * float.  volatile keeps the product in single precision. */
    volatile float fdeg = (float)deg;
    volatile float prod = r * fdeg;
    float p = prod;
    if (!(p >= 0.0f)) return 0;                  /* negative or NaN */
    if (p >= 9.0e18f) return deg - 1;            /* beyond int64 */
    int64_t idx = (int64_t)p;                    /* truncation toward zero */
    return idx < deg ? idx : deg - 1;
}

/* ----------------------------------------------------------- uniform walk */

static int node_ok(int64_t v, int64_t num_nodes) { return v >= 0 && v < num_nodes; }

static int row_ok(int64_t rs, int64_t re, int64_t num_edges) {
    return rs >= 0 && re >= rs && re <= num_edges;
}

int oracle_uniform_walk(const int64_t* rowptr, int64_t num_nodes,
                        const int64_t* col, int64_t num_edges,
                        const int64_t* start, int64_t num_walks,
                        const float* rand, int32_t walk_length,
                        int64_t* n_out, int64_t* e_out, oracle_counts* counts) {
    const int64_t L = walk_length;
    oracle_counts c = {0, 0, 0, 0, 0};
    int status = 0;
    /* RandomWalk.cpp:41 */
    for (int64_t n = 0; n < num_walks; ++n) {
        int64_t v = start[n];
        int sunk = 0;
        n_out[n * (L + 1)] = v;                                      /* :43 */
        for (int64_t l = 0; l < L; ++l) {                            /* :44 */
            int64_t e = -1;
            if (!node_ok(v, num_nodes)) { status = -1; goto store; }
            {
                int64_t rs = rowptr[v], re = rowptr[v + 1];          /* :45-46 */
                if (!row_ok(rs, re, num_edges)) { status = -1; goto store; }
                if (re - rs == 0) {                                  /* :48-49 */
                    if (!sunk) { sunk = 1; c.sink_walks++; }
                } else {                                             /* :51-54 */
                    float r = rand[n * L + l];
                    e = rs + oracle_pick_index(r, re - rs);
                    v = col[e];
                    c.moving_steps++;
                    if (!node_ok(v, num_nodes)) status = -1;
                }
            }
        store:
            n_out[n * (L + 1) + l + 1] = v;                          /* :57 */
            if (e_out) e_out[n * L + l] = e;                         /* :58 */
        }
    }
    if (counts) *counts = c;
    return status;
}

/* ---------------------------------------------------------- node2vec walk */

void oracle_node2vec_probs(double p, double q, double probs[3]) {
    /* BiasedRandomWalk.cpp:52-55 */
    double max_prob = fmax(fmax(1. / p, 1.), 1. / q);
    probs[0] = 1. / p / max_prob;
    probs[1] = 1. / max_prob;
    probs[2] = 1. / q / max_prob;
}

/* is_neighbor(x, t): is t in row(x)?  BiasedRandomWalk.cpp:20-28 scans the
 * row; on a sorted row lower_bound gives the same answer. */
static int is_neighbor(const int64_t* rowptr, const int64_t* col, int64_t num_edges,
                       int64_t x, int64_t t, int sorted, oracle_counts* c, int* bad) {
    int64_t rs = rowptr[x], re = rowptr[x + 1];
    c->member_tests++;
    if (!row_ok(rs, re, num_edges)) { *bad = 1; return 0; }
    if (!sorted) {
        for (int64_t i = rs; i < re; ++i) {
            if (((i - rs) & 7) == 0 || i == rs) c->member_lines++;
            if (col[i] == t) return 1;
        }
        return 0;
    }
    int64_t lo = rs, count = re - rs;
    int64_t last_line = -1;
    while (count > 0) {
        int64_t half = count >> 1;
        int64_t mid = lo + half;
        int64_t line = mid >> 3;
        if (line != last_line) { c->member_lines++; last_line = line; }
        if (col[mid] < t) { lo = mid + 1; count -= half + 1; }
        else count = half;
    }
    if (lo < re) {
        int64_t line = lo >> 3;
        if (line != last_line) c->member_lines++;
        return col[lo] == t;
    }
    return 0;
}

/* Acceptance of candidate x (previous node t) for the uniform r. */
static int accept_candidate(int32_t rule, const double probs[3], double r,
                            const int64_t* rowptr, const int64_t* col, int64_t num_edges,
                            int64_t x, int64_t t, int sorted, oracle_counts* c, int* bad) {
    if (rule == ORACLE_RULE_REF_CHAIN) {
        /* BiasedRandomWalk.cpp:86-91: (x==t && r<p0) || (nb(x,t) && r<p1) || r<p2.
         * The terms have no side effects, so the cheap ones go first and the
         * row search runs only when its answer decides the outcome. */
        if (r < probs[2]) return 1;
        if (x == t && r < probs[0]) return 1;
        if (r < probs[1]) return is_neighbor(rowptr, col, num_edges, x, t, sorted, c, bad);
        return 0;
    }
    /* Analytic node2vec: d = 0 if x == t, 1 if t in row(x), else 2. */
    if (x == t) return r < probs[0];
    if (r < probs[1] && r < probs[2]) return 1;
    if (!(r < probs[1]) && !(r < probs[2])) return 0;
    return is_neighbor(rowptr, col, num_edges, x, t, sorted, c, bad) ? (r < probs[1])
                                                                     : (r < probs[2]);
}

int oracle_node2vec_walk(const int64_t* rowptr, int64_t num_nodes,
                         const int64_t* col, int64_t num_edges,
                         const int64_t* start, int64_t num_walks, int64_t first_walk,
                         int32_t walk_length, double p, double q,
                         uint64_t seed, int32_t rule, int32_t rows_sorted,
                         int64_t* n_out, int64_t* e_out, oracle_counts* counts) {
    const int64_t L = walk_length;
    double probs[3];
    oracle_node2vec_probs(p, q, probs);
    oracle_counts c = {0, 0, 0, 0, 0};
    int status = 0;
    for (int64_t n = 0; n < num_walks; ++n) {                        /* :57 */
        int64_t t = start[n], v = t, e = -1;                         /* :58 */
        int sunk = 0, bad = 0;
        n_out[n * (L + 1)] = t;                                      /* :59 */
        if (L == 0) {
            if (!node_ok(t, num_nodes)) status = -1;
            continue;
        }
        if (!node_ok(t, num_nodes)) { bad = 1; }
        else {
            int64_t rs = rowptr[t], re = rowptr[t + 1];              /* :60 */
            if (!row_ok(rs, re, num_edges)) bad = 1;
            else if (re - rs == 0) { sunk = 1; c.sink_walks++; }     /* :61-63 */
            else {                                                   /* :64-66 */
                float u0, u1;
                n2v_uniforms(seed, first_walk + n, 0, 0u, &u0, &u1);
                e = rs + oracle_pick_index(u0, re - rs);
                v = col[e];
                c.moving_steps++;
                c.trials++;
            }
        }
        n_out[n * (L + 1) + 1] = v;                                  /* :68 */
        if (e_out) e_out[n * L] = e;                                 /* :69 */
        for (int64_t l = 1; l < L; ++l) {                            /* :70 */
            int64_t x = v;
            e = -1;
            if (!bad && !node_ok(v, num_nodes)) bad = 1;
            if (!bad) {
                int64_t rs = rowptr[v], re = rowptr[v + 1];          /* :71 */
                if (!row_ok(rs, re, num_edges)) bad = 1;
                else if (re - rs == 0) {                             /* :73-75 */
                    if (!sunk) { sunk = 1; c.sink_walks++; }
                } else if (re - rs == 1) {                           /* :76-78 */
                    e = rs;
                    x = col[e];
                    c.moving_steps++;
                    c.trials++;
                } else {                                             /* :80-92 */
                    c.moving_steps++;
                    for (uint32_t trial = 0;; ++trial) {
                        float u0, u1;
                        n2v_uniforms(seed, first_walk + n, (int32_t)l, trial, &u0, &u1);
                        e = rs + oracle_pick_index(u0, re - rs);     /* :81 */
                        x = col[e];                                  /* :82 */
                        c.trials++;
                        double r = (double)u1;                       /* :84 */
                        if (!node_ok(x, num_nodes)) { bad = 1; break; }
                        if (accept_candidate(rule, probs, r, rowptr, col, num_edges, x, t,
                                             rows_sorted, &c, &bad))
                            break;
                        if (bad || trial + 1 >= ORACLE_MAX_TRIALS) break;
                    }
                }
            }
            n_out[n * (L + 1) + l + 1] = x;                          /* :95 */
            if (e_out) e_out[n * L + l] = e;                         /* :96 */
            t = v;                                                   /* :97 */
            v = x;                                                   /* :98 */
        }
        if (bad) status = -1;
    }
    if (counts) *counts = c;
    return status;
}

/* is_neighbor exactly as BiasedRandomWalk.cpp:20-28: a linear scan of
 * row(v) for w. */
static int is_neighbor_scan(const int64_t* rowptr, const int64_t* col, int64_t v, int64_t w) {
    for (int64_t i = rowptr[v]; i < rowptr[v + 1]; ++i)
        if (col[i] == w) return 1;
    return 0;
}

int oracle_node2vec_walk_libc(const int64_t* rowptr, int64_t num_nodes,
                              const int64_t* col, int64_t num_edges,
                              const int64_t* start, int64_t num_walks,
                              int32_t walk_length, double p, double q,
                              uint32_t libc_seed, int32_t rule,
                              int64_t* n_out, int64_t* e_out) {
    const int64_t L = walk_length;
    double probs[3];
    oracle_node2vec_probs(p, q, probs);
    oracle_counts c = {0, 0, 0, 0, 0};
    int status = 0;
    srand(libc_seed);
    for (int64_t n = 0; n < num_walks; ++n) {
        int64_t t = start[n], v = t, e = -1;
        int bad = 0;
        n_out[n * (L + 1)] = t;
        if (L == 0) continue;
        if (!node_ok(t, num_nodes)) bad = 1;
        else {
            int64_t rs = rowptr[t], re = rowptr[t + 1];
            if (!row_ok(rs, re, num_edges)) bad = 1;
            else if (re - rs != 0) {
                e = rs + (rand() % (re - rs));                       /* :65 */
                v = col[e];
            }
        }
        n_out[n * (L + 1) + 1] = v;
        if (e_out) e_out[n * L] = e;
        for (int64_t l = 1; l < L; ++l) {
            int64_t x = v;
            e = -1;
            if (!bad && !node_ok(v, num_nodes)) bad = 1;
            if (!bad) {
                int64_t rs = rowptr[v], re = rowptr[v + 1];
                if (!row_ok(rs, re, num_edges)) bad = 1;
                else if (re - rs == 1) { e = rs; x = col[e]; }
                else if (re - rs > 1) {
                    for (uint32_t trial = 0;; ++trial) {
                        e = rs + (rand() % (re - rs));               /* :81 */
                        x = col[e];
                        double r = ((double)rand() / (RAND_MAX));   /* :84 */
                        if (!node_ok(x, num_nodes)) { bad = 1; break; }
                        if (rule == ORACLE_RULE_REF_CHAIN) {
                            /* :86-91 evaluated as written: is_neighbor runs
                             * whenever the first clause fails */
                            if (x == t && r < probs[0]) break;
                            else if (is_neighbor_scan(rowptr, col, x, t) && r < probs[1]) break;
                            else if (r < probs[2]) break;
                        } else if (accept_candidate(rule, probs, r, rowptr, col, num_edges, x, t,
                                                    0, &c, &bad)) {
                            break;
                        }
                        if (bad || trial + 1 >= ORACLE_MAX_TRIALS) break;
                    }
                }
            }
            n_out[n * (L + 1) + l + 1] = x;
            if (e_out) e_out[n * L + l] = e;
            t = v;
            v = x;
        }
        if (bad) status = -1;
    }
    return status;
}

int32_t oracle_csr_flags(const int64_t* rowptr, int64_t num_nodes,
                         const int64_t* col, int64_t num_edges) {
    int32_t f = 0;
    if (rowptr[0] != 0 || rowptr[num_nodes] != num_edges) f |= 1;
    for (int64_t v = 0; v < num_nodes; ++v)
        if (rowptr[v + 1] < rowptr[v]) f |= 1;
    for (int64_t i = 0; i < num_edges; ++i)
        if (col[i] < 0 || col[i] >= num_nodes) f |= 2;
    if (!(f & 1)) {
        for (int64_t v = 0; v < num_nodes; ++v)
            for (int64_t i = rowptr[v] + 1; i < rowptr[v + 1]; ++i)
                if (col[i] < col[i - 1]) f |= 4;
    }
    if (f == 0) {  /* symmetry, by a linear scan of row(v) for each entry (u, v) */
        for (int64_t u = 0; u < num_nodes && !(f & 8); ++u)
            for (int64_t i = rowptr[u]; i < rowptr[u + 1] && !(f & 8); ++i) {
                const int64_t v = col[i];
                int found = 0;
                for (int64_t j = rowptr[v]; j < rowptr[v + 1] && !found; ++j) found = col[j] == u;
                if (!found) f |= 8;
            }
    }
    return f;
}
