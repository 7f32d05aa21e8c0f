/* The C ABI used from plain C99 (no C++, no Python): builds a CSR from an
 * edge list and walks it with the host twins, then checks argument errors.
 * Compiled and run by tests/test_c_abi_example.py. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "mlxc.h"

#define CHECK(cond)                                                      \
    do {                                                                 \
        if (!(cond)) {                                                   \
            fprintf(stderr, "check failed line %d: %s (%s)\n", __LINE__, \
                    #cond, mlxc_last_error());                          \
            return 1;                                                    \
        }                                                                \
    } while (0)

int main(void) {
    /* directed 4-cycle 0->1->2->3->0 plus 0->2, listed out of order, one duplicate */
    const int64_t row[] = {2, 0, 3, 1, 0, 0};
    const int64_t col[] = {3, 2, 0, 2, 1, 2};
    int64_t rowptr[5], cols[6], count = 0, status = -1;
    CHECK(mlxc_version() >= 300);
    CHECK(mlxc_csr_build_cpu(row, col, 6, 4, MLXC_CSR_DEDUP, rowptr, cols, &count, &status) ==
          MLXC_OK);
    CHECK(status == 0 && count == 5);
    const int64_t want_rowptr[] = {0, 2, 3, 4, 5}, want_cols[] = {1, 2, 2, 3, 0};
    CHECK(memcmp(rowptr, want_rowptr, sizeof rowptr) == 0);
    CHECK(memcmp(cols, want_cols, 5 * sizeof(int64_t)) == 0);

    /* uniform walk: r = 0.75 picks the second neighbour of node 0, else the only one */
    const int64_t start[] = {0, 3};
    const float rand[] = {0.75f, 0.75f, 0.75f, 0.75f, 0.75f, 0.75f};
    int64_t walks[2 * 4], edges[2 * 3];
    CHECK(mlxc_random_walk_cpu(rowptr, 4, cols, 5, start, 2, rand, 3, walks, edges,
                               MLXC_OUT_INT64, 1, &status) == MLXC_OK);
    const int64_t want_walks[] = {0, 2, 3, 0, 3, 0, 2, 3};
    CHECK(status == 0 && memcmp(walks, want_walks, sizeof walks) == 0);
    CHECK(edges[0] == 1 && edges[1] == 3);

    /* node2vec with p = q = 1 accepts the first candidate of every step */
    int64_t n2v[2 * 4];
    CHECK(mlxc_rejection_sampling_cpu(rowptr, 4, cols, 5, start, 2, 3, 1.0, 1.0, 42, 0,
                                      MLXC_RULE_REF_CHAIN, MLXC_ROWS_DETECT, n2v, NULL,
                                      MLXC_OUT_INT64, 2, &status) == MLXC_OK);
    CHECK(status == 0 && n2v[0] == 0 && n2v[4] == 3);

    /* skip-gram windows of the walks: W = 4 - 2 + 1 = 3 windows per walk */
    int64_t win[3 * 2 * 2];
    CHECK(mlxc_context_windows_cpu(walks, 2, 4, 2, MLXC_OUT_INT64, win) == MLXC_OK);
    CHECK(win[0] == 0 && win[1] == 2 && win[2] == 3 && win[3] == 0 && win[4] == 2 && win[5] == 3);

    /* errors come back as codes with a message, before any work */
    CHECK(mlxc_random_walk_cpu(rowptr, 4, cols, 5, start, 2, rand, -1, walks, NULL,
                               MLXC_OUT_INT64, 1, &status) == MLXC_ERR_INVALID_ARGUMENT);
    CHECK(strstr(mlxc_last_error(), "walk_length") != NULL);
    CHECK(mlxc_csr_build_cpu(row, col, 6, 4, 99, rowptr, cols, &count, &status) ==
          MLXC_ERR_INVALID_ARGUMENT);
    printf("c abi example ok\n");
    return 0;
}
