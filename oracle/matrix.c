#define _GNU_SOURCE
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
        } else if (j->dtype == OR_Q5_K) {
            or_q5k_q8k_row_lanes(wrow, j->nb, j->packed, j->rows, o);  /* one order: no AVX2 twin */
        } else if (j->dtype == OR_Q6_K) {
            if (j->impl == 1) or_q6k_q8k_row_avx2(wrow, j->nb, j->packed, j->rows, o);
            else or_q6k_q8k_row_lanes(wrow, j->nb, j->packed, j->rows, o);
        } else {
            if (j->impl == 1) or_q80_q80_row_avx2(wrow, j->nb, j->packed, j->rows, o);
            else or_q80_q80_row_lanes(wrow, j->nb, j->packed, j->rows, o);
        }
    }
}

/* A persistent pool of spinning workers, like the reference's matvec pool
 * (candle's BarrierPool, src/threading.rs:4-9): a call publishes a job
 * generation, every thread (the caller included) takes static row chunks,
 * and the caller spins until all chunks are done. */
#include <stdatomic.h>

#define OR_MAX_THREADS 256
static struct {
    int n; /* threads including the caller */
    pthread_t tids[OR_MAX_THREADS];
    atomic_int gen, next, done;
    int nchunks;
    row_job jobs[OR_MAX_THREADS];
} pool;
static pthread_mutex_t pool_mu = PTHREAD_MUTEX_INITIALIZER;

static void pool_work(void) {
    for (;;) {
        int c = atomic_fetch_add(&pool.next, 1);
        if (c >= pool.nchunks) break;
        run_rows(&pool.jobs[c]);
        atomic_fetch_add(&pool.done, 1);
    }
}

/* Idle workers spin briefly (a matvec call is tens of microseconds), then
 * park on a condition variable so an idle pool costs no CPU. */
static pthread_mutex_t sleep_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t sleep_cv = PTHREAD_COND_INITIALIZER;
static atomic_int sleepers;

/* Optional pinning of pool threads (the CPU baseline pins one thread per
 * physical core, as the reference's pool does by default): worker t runs on
 * pin_cpus[t % pin_n]; worker 0 is the caller, which pins itself. */
static int pin_cpus[OR_MAX_THREADS];
static int pin_n;

static void pin_thread(pthread_t th, int t) {
    if (pin_n <= 0) return;
    cpu_set_t set;
    CPU_ZERO(&set);
    CPU_SET(pin_cpus[t % pin_n], &set);
    pthread_setaffinity_np(th, sizeof set, &set);
}

void or_pool_pin(const int *cpus, int n) {
    pthread_mutex_lock(&pool_mu);
    pin_n = n < 0 ? 0 : (n > OR_MAX_THREADS ? OR_MAX_THREADS : n);
    for (int i = 0; i < pin_n; i++) pin_cpus[i] = cpus[i];
    for (int t = 1; t < pool.n; t++) pin_thread(pool.tids[t], t);
    pthread_mutex_unlock(&pool_mu);
}

static void *pool_thread(void *arg) {
    (void)arg;
    int seen = 0;
    for (;;) {
        int g, spins = 0;
        while ((g = atomic_load(&pool.gen)) == seen) {
            if (++spins < 200000) continue;
            pthread_mutex_lock(&sleep_mu);
            atomic_fetch_add(&sleepers, 1);
            while (atomic_load(&pool.gen) == seen) pthread_cond_wait(&sleep_cv, &sleep_mu);
            atomic_fetch_sub(&sleepers, 1);
            pthread_mutex_unlock(&sleep_mu);
            spins = 0;
        }
        seen = g;
        pool_work();
    }
    return NULL;
}

static void pool_run(row_job *jobs, int nchunks, int nthreads) {
    if (nthreads > OR_MAX_THREADS) nthreads = OR_MAX_THREADS;
    if (pool.n < nthreads) {
        for (int t = pool.n > 0 ? pool.n : 1; t < nthreads; t++) {
            pthread_create(&pool.tids[t], NULL, pool_thread, NULL);
            pin_thread(pool.tids[t], t);
        }
        pool.n = nthreads;
    }
    memcpy(pool.jobs, jobs, (size_t)nchunks * sizeof(row_job));
    pool.nchunks = nchunks;
    atomic_store(&pool.done, 0);
    atomic_store(&pool.next, 0);
    atomic_fetch_add(&pool.gen, 1);
    if (atomic_load(&sleepers)) {
        pthread_mutex_lock(&sleep_mu);
        pthread_cond_broadcast(&sleep_cv);
        pthread_mutex_unlock(&sleep_mu);
    }
    pool_work();
    while (atomic_load(&pool.done) < nchunks) {
    }
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
    if (nthreads > OR_MAX_THREADS) nthreads = OR_MAX_THREADS;
    if (nthreads == 1) {
        row_job j = {dtype, impl, w, nb, m, packed, cm, 0, n_rows};
        run_rows(&j);
    } else {
        row_job jobs[OR_MAX_THREADS];
        size_t chunk = (n_rows + (size_t)nthreads - 1) / (size_t)nthreads;
        int nchunks = 0;
        for (int t = 0; t < nthreads; t++) {
            size_t b0 = (size_t)t * chunk, b1 = b0 + chunk < n_rows ? b0 + chunk : n_rows;
            if (b0 >= b1) break;
            jobs[nchunks++] = (row_job){dtype, impl, w, nb, m, packed, cm, b0, b1};
        }
        pthread_mutex_lock(&pool_mu);
        pool_run(jobs, nchunks, nthreads);
        pthread_mutex_unlock(&pool_mu);
    }

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
