/*
 * matrix.c -- TEST INFRASTRUCTURE (parity oracle and timed CPU baseline, see
 * iq_oracle.h).
 *
 * QuantizedMatrix::fused_forward (src/gguf.rs:608-690): quantise each input
 * row with from_float, repack block-major, run the per-row kernel for every
 * output row (spread over threads like RowSpread::Pool, src/gguf.rs:672-676),
 * and transpose the column-major result to [m x n_rows].
 */
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "iq_oracle.h"

typedef struct {
    int dtype, impl;
    const void *w;
    size_t nb, rows; /* blocks per weight row, input rows */
    const void *packed;
    float *colmajor; /* [n_rows x rows] */
    size_t row_begin, row_end;
} row_job;

static void run_rows(const row_job *j) {
    size_t bb = or_block_bytes(j->dtype);
    for (size_t n = j->row_begin; n < j->row_end; n++) {
        const void *wrow = (const uint8_t *)j->w + n * j->nb * bb;
        float *o = j->colmajor + n * j->rows;
        if (j->dtype == OR_Q4_K) {
            if (j->impl == 1) or_q4k_q8k_row_avx2(wrow, j->nb, j->packed, j->rows, o);
            else or_q4k_q8k_row_lanes(wrow, j->nb, j->packed, j->rows, o);
        } else if (j->dtype == OR_Q6_K) {
            if (j->impl == 1) or_q6k_q8k_row_avx2(wrow, j->nb, j->packed, j->rows, o);
            else or_q6k_q8k_row_lanes(wrow, j->nb, j->packed, j->rows, o);
        } else {
            if (j->impl == 1) or_q80_q80_row_avx2(wrow, j->nb, j->packed, j->rows, o);
            else or_q80_q80_row_lanes(wrow, j->nb, j->packed, j->rows, o);
        }
    }
}

static void *row_thread(void *arg) {
    run_rows((const row_job *)arg);
    return NULL;
}

int or_matmul(int dtype, const void *w, size_t n_rows, size_t cols, const float *x, size_t m, float *y, int impl,
              int nthreads) {
    size_t be = or_block_elems(dtype);
    if (!be || cols % be || m == 0) return -1;
    if (impl == 1 && !or_have_avx2()) return -2;
    size_t nb = cols / be;
    size_t ib = dtype == OR_Q8_0 ? sizeof(or_q80_block) : sizeof(or_q8k_block);
    uint8_t *q = malloc(m * nb * ib), *packed = malloc(m * nb * ib);
    float *cm = malloc(n_rows * m * sizeof(float));
    if (!q || !packed || !cm) {
        free(q); free(packed); free(cm);
        return -3;
    }
    for (size_t r = 0; r < m; r++) {
        if (dtype == OR_Q8_0) or_quantize_q80(x + r * cols, cols, (or_q80_block *)(q + r * nb * ib));
        else or_quantize_q8k(x + r * cols, cols, (or_q8k_block *)(q + r * nb * ib));
    }
    /* block-major: packed[block * m + row] */
    for (size_t b = 0; b < nb; b++)
        for (size_t r = 0; r < m; r++) memcpy(packed + (b * m + r) * ib, q + (r * nb + b) * ib, ib);

    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > n_rows) nthreads = (int)n_rows;
    row_job jobs[256];
    pthread_t tids[256];
    if (nthreads > 256) nthreads = 256;
    size_t chunk = (n_rows + (size_t)nthreads - 1) / (size_t)nthreads;
    int launched = 0;
    for (int t = 0; t < nthreads; t++) {
        size_t b0 = (size_t)t * chunk, b1 = b0 + chunk < n_rows ? b0 + chunk : n_rows;
        if (b0 >= b1) break;
        jobs[t] = (row_job){dtype, impl, w, nb, m, packed, cm, b0, b1};
        if (t == 0) continue;
        pthread_create(&tids[t], NULL, row_thread, &jobs[t]);
        launched = t;
    }
    run_rows(&jobs[0]);
    for (int t = 1; t <= launched; t++) pthread_join(tids[t], NULL);

    for (size_t r = 0; r < m; r++)
        for (size_t n = 0; n < n_rows; n++) y[r * n_rows + n] = cm[n * m + r];
    free(q);
    free(packed);
    free(cm);
    return 0;
}

int or_matmul_tiled(int dtype, const void *w, size_t n_rows, size_t cols, const float *x, size_t m, float *y,
                    int impl, int nthreads) {
    const size_t tile = 16;
    size_t start = 0;
    float *buf = malloc(tile * n_rows * sizeof(float));
    if (!buf) return -3;
    while (start < m) {
        size_t remaining = m - start;
        size_t rows = remaining <= tile ? remaining : (remaining - tile == 1 ? tile - 1 : tile);
        int rc = or_matmul(dtype, w, n_rows, cols, x + start * cols, rows, buf, impl, nthreads);
        if (rc) {
            free(buf);
            return rc;
        }
        memcpy(y + start * n_rows, buf, rows * n_rows * sizeof(float));
        start += rows;
    }
    free(buf);
    return 0;
}
