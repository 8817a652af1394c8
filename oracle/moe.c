/*
 * moe.c -- TEST INFRASTRUCTURE (parity oracle and timed CPU baseline, see
 * iq_oracle.h).
 *
 * top_k_routes (src/qwen/moe.rs:21-54) and QuantizedMoeLayer::forward
 * (src/qwen/quantized_moe.rs:227-460): routed experts token-major or grouped
 * by expert, SwiGLU, ordered weighted combine, shared expert with sigmoid gate.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "iq_oracle.h"

float or_silu_mul(float gate, float up) {
    /* candle's Silu, elementwise: v / (1 + exp(-v)), then times up
     * (src/qwen/quantized_moe.rs:446) */
    return (gate / (1.f + expf(-gate))) * up;
}

void or_router_logits(const float *x, size_t m, size_t h, const float *router, size_t e, float *logits, int order) {
    for (size_t t = 0; t < m; t++) {
        for (size_t j = 0; j < e; j++) {
            const float *xr = x + t * h, *r = router + j * h;
            if (order == 0) {
                double s = 0.0;
                for (size_t i = 0; i < h; i++) s += (double)xr[i] * (double)r[i];
                logits[t * e + j] = (float)s;
            } else {
                float s = 0.f;
                for (size_t i = 0; i < h; i++) s = s + xr[i] * r[i];
                logits[t * e + j] = s;
            }
        }
    }
}

float or_sigmoid(float v) {
    /* candle-nn sigmoid: recip(exp(-v) + 1) */
    return 1.f / (expf(-v) + 1.f);
}

int or_top_k_routes(const float *logits, size_t m, size_t e, size_t k, int normalize, int32_t *experts,
                    float *weights) {
    if (k == 0 || k > e) return -1;
    float *p = malloc(e * sizeof(float));
    char *taken = malloc(e);
    if (!p || !taken) {
        free(p); free(taken);
        return -3;
    }
    for (size_t r = 0; r < m; r++) {
        const float *row = logits + r * e;
        float max = -INFINITY;
        for (size_t i = 0; i < e; i++) max = fmaxf(max, row[i]);
        float denom = 0.f;
        for (size_t i = 0; i < e; i++) denom += expf(row[i] - max);
        for (size_t i = 0; i < e; i++) p[i] = expf(row[i] - max) / denom;
        memset(taken, 0, e);
        for (size_t s = 0; s < k; s++) {
            size_t best = e;
            /* descending probability; the reference's unstable sort leaves
             * exactly equal probabilities unordered -- they are ordered here
             * by larger logit, then lower index (probability never decreases
             * with the logit, so this is one of the reference's orders) */
            for (size_t i = 0; i < e; i++) {
                if (taken[i]) continue;
                if (best == e || p[i] > p[best] || (p[i] == p[best] && row[i] > row[best])) best = i;
            }
            taken[best] = 1;
            experts[r * k + s] = (int32_t)best;
            weights[r * k + s] = p[best];
        }
        if (normalize) {
            float sum = 0.f;
            for (size_t s = 0; s < k; s++) sum += weights[r * k + s];
            for (size_t s = 0; s < k; s++) weights[r * k + s] /= sum;
        }
    }
    free(p);
    free(taken);
    return 0;
}

static const void *expert_ptr(const void *base, int dtype, size_t e, size_t rows, size_t cols) {
    size_t per = rows * (cols / or_block_elems(dtype)) * or_block_bytes(dtype);
    return (const uint8_t *)base + e * per;
}

/* gate_up -> SwiGLU -> down for `rows` contiguous input rows of one expert
 * (run_one_expert, src/qwen/quantized_moe.rs:414-460).  values: [rows x H]. */
static int run_expert(const or_moe_layer *L, const void *gate, const void *up, int gdt, const void *down, int ddt,
                      const float *inputs, size_t rows, float *values, int impl, int nthreads) {
    size_t H = L->hidden, I = L->inter;
    float *g = malloc(rows * I * sizeof(float)), *u = malloc(rows * I * sizeof(float));
    float *a = malloc(rows * I * sizeof(float));
    int rc = -3;
    if (!g || !u || !a) goto out;
    /* gate and up are the two halves of the row-concatenated gate_up matrix;
     * each output row depends only on its own weight row, so running the
     * halves separately is the concatenated product. */
    if ((rc = or_matmul(gdt, gate, I, H, inputs, rows, g, impl, nthreads))) goto out;
    if ((rc = or_matmul(gdt, up, I, H, inputs, rows, u, impl, nthreads))) goto out;
    for (size_t i = 0; i < rows * I; i++) a[i] = or_silu_mul(g[i], u[i]);
    rc = or_matmul(ddt, down, H, I, a, rows, values, impl, nthreads);
out:
    free(g);
    free(u);
    free(a);
    return rc;
}

typedef struct {
    const or_moe_layer *L;
    const float *x;
    size_t m;
    const int32_t *experts;
    size_t *group_expert, *group_start, *group_rows; /* groups sorted by expert */
    size_t *assign;                                  /* (row, route) pairs flattened: row*k+route */
    float **values;
    size_t n_groups, next;
    pthread_mutex_t lock;
    int impl, rc;
} group_ctx;

static void *group_worker(void *arg) {
    group_ctx *c = arg;
    const or_moe_layer *L = c->L;
    size_t H = L->hidden, I = L->inter, k = L->top_k;
    for (;;) {
        pthread_mutex_lock(&c->lock);
        size_t gi = c->next++;
        pthread_mutex_unlock(&c->lock);
        if (gi >= c->n_groups) break;
        size_t e = c->group_expert[gi], rows = c->group_rows[gi];
        float *in = malloc(rows * H * sizeof(float));
        c->values[gi] = malloc(rows * H * sizeof(float));
        if (!in || !c->values[gi]) {
            free(in);
            c->rc = -3;
            continue;
        }
        for (size_t r = 0; r < rows; r++) {
            size_t row = c->assign[c->group_start[gi] + r] / k;
            memcpy(in + r * H, c->x + row * H, H * sizeof(float));
        }
        int rc = run_expert(L, expert_ptr(L->gate, L->gate_dtype, e, I, H), expert_ptr(L->up, L->gate_dtype, e, I, H),
                            L->gate_dtype, expert_ptr(L->down, L->down_dtype, e, H, I), L->down_dtype, in, rows,
                            c->values[gi], c->impl, 1);
        if (rc) c->rc = rc;
        free(in);
    }
    return NULL;
}

int or_moe_forward(const or_moe_layer *L, const float *x, const float *logits, size_t m, float *out,
                   int32_t *experts, float *weights, int mode, int impl, int nthreads) {
    size_t H = L->hidden, I = L->inter, E = L->n_experts, k = L->top_k;
    int rc = or_top_k_routes(logits, m, E, k, L->normalize, experts, weights);
    if (rc) return rc;
    float *routed = calloc(m * H, sizeof(float));
    float *value = malloc(H * sizeof(float));
    if (!routed || !value) {
        free(routed); free(value);
        return -3;
    }
    if (nthreads < 1) nthreads = 1;

    if (mode == 0) {
        /* routed_token_major (src/qwen/quantized_moe.rs:283-318) */
        for (size_t t = 0; t < m && !rc; t++) {
            float *combined = routed + t * H;
            for (size_t s = 0; s < k && !rc; s++) {
                size_t e = (size_t)experts[t * k + s];
                float w = weights[t * k + s];
                rc = run_expert(L, expert_ptr(L->gate, L->gate_dtype, e, I, H),
                                expert_ptr(L->up, L->gate_dtype, e, I, H), L->gate_dtype,
                                expert_ptr(L->down, L->down_dtype, e, H, I), L->down_dtype, x + t * H, 1, value, impl,
                                nthreads);
                for (size_t j = 0; j < H; j++) combined[j] = combined[j] + value[j] * w;
            }
        }
    } else {
        /* routed_grouped_by_expert (src/qwen/quantized_moe.rs:336-406):
         * (row, route) pairs grouped by expert ascending, rows in order. */
        size_t na = m * k;
        size_t *assign = malloc(na * sizeof(size_t)), *slot_group = malloc(na * sizeof(size_t));
        size_t *slot_row = malloc(na * sizeof(size_t));
        size_t *count = calloc(E, sizeof(size_t));
        group_ctx c;
        memset(&c, 0, sizeof c);
        c.group_expert = malloc(E * sizeof(size_t));
        c.group_start = malloc(E * sizeof(size_t));
        c.group_rows = malloc(E * sizeof(size_t));
        c.values = calloc(E, sizeof(float *));
        for (size_t a = 0; a < na; a++) count[experts[a]]++;
        size_t pos = 0, ng = 0;
        for (size_t e = 0; e < E; e++) {
            if (!count[e]) continue;
            c.group_expert[ng] = e;
            c.group_start[ng] = pos;
            c.group_rows[ng] = 0;
            for (size_t a = 0; a < na; a++) {
                if ((size_t)experts[a] != e) continue;
                slot_group[a] = ng;
                slot_row[a] = c.group_rows[ng]++;
                assign[pos++] = a;
            }
            ng++;
        }
        c.L = L;
        c.x = x;
        c.m = m;
        c.experts = experts;
        c.assign = assign;
        c.n_groups = ng;
        c.impl = impl;
        pthread_mutex_init(&c.lock, NULL);
        int nt = nthreads > 64 ? 64 : nthreads;
        pthread_t tids[64];
        for (int t = 1; t < nt; t++) pthread_create(&tids[t], NULL, group_worker, &c);
        group_worker(&c);
        for (int t = 1; t < nt; t++) pthread_join(tids[t], NULL);
        pthread_mutex_destroy(&c.lock);
        rc = c.rc;
        /* ordered combine: token, then route order; multiply then add */
        for (size_t t = 0; t < m && !rc; t++) {
            float *o = routed + t * H;
            for (size_t s = 0; s < k; s++) {
                size_t a = t * k + s;
                const float *v = c.values[slot_group[a]] + slot_row[a] * H;
                float w = weights[a];
                for (size_t j = 0; j < H; j++) o[j] += v[j] * w;
            }
        }
        for (size_t g = 0; g < ng; g++) free(c.values[g]);
        free(c.values);
        free(c.group_expert);
        free(c.group_start);
        free(c.group_rows);
        free(assign);
        free(slot_group);
        free(slot_row);
        free(count);
    }

    if (!rc && L->selector) {
        /* shared expert (src/qwen/quantized_moe.rs:266-273) */
        float *sv = malloc(m * H * sizeof(float));
        if (!sv) rc = -3;
        else {
            /* per row: each output row of a matmul depends only on its own
             * input row, so this equals the reference's one M-row call */
            for (size_t t = 0; t < m && !rc; t++)
                rc = run_expert(L, L->shared_gate, L->shared_up, L->shared_gate_dtype, L->shared_down,
                                L->shared_down_dtype, x + t * H, 1, sv + t * H, impl, nthreads);
            for (size_t t = 0; t < m && !rc; t++) {
                /* flat.matmul(selector^T): accumulation order of candle's f32
                 * gemm is not visible here; a double-precision sum is used. */
                double s = 0.0;
                for (size_t j = 0; j < H; j++) s += (double)x[t * H + j] * (double)L->selector[j];
                float gate = or_sigmoid((float)s);
                for (size_t j = 0; j < H; j++) out[t * H + j] = routed[t * H + j] + sv[t * H + j] * gate;
            }
            free(sv);
        }
    } else if (!rc) {
        memcpy(out, routed, m * H * sizeof(float));
    }
    free(routed);
    free(value);
    return rc;
}
