/*
 * iq_oracle.h -- CPU restatement of inferq's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle for the HIP
 * kernels in inferq_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker (or as the
 * timed CPU baseline).  The product library never links or calls it.
 *
 * Every function restates reference behaviour read from the reference source
 * as text (paths relative to the reference root):
 *   block layouts            src/qgemm.rs:46-65
 *   unpack_k_scales          src/qgemm.rs:153-167
 *   q4k_tile / q6k_tile      src/qgemm.rs:175-346
 *   q80_tile                 src/qgemm.rs:369-397
 *   hsum_f32_8 / hsum_f32_4  src/qgemm.rs:132-148
 *   tiled_entry / row_entry  src/qgemm.rs:399-468
 *   fused_forward            src/gguf.rs:608-690
 *   tiled_multi_row          src/gguf.rs:493-520
 *   concatenate_rows         src/gguf.rs:379-404
 *   leading_rows             src/gguf.rs:352-377
 *   top_k_routes             src/qwen/moe.rs:21-54
 *   MoE forward              src/qwen/quantized_moe.rs:227-460
 * and the third-party arithmetic the path calls (candle-core 0.11.0, not
 * vendored in the reference): BlockQ8K::from_float / BlockQ8_0::from_float,
 * called at src/gguf.rs:648-654.  Those two are restated from candle/ggml's
 * published algorithm; their tie behaviour cannot be checked against candle
 * here ("parity unpinned" for exact .5 ties and equal-|x| maxima).
 */
#ifndef IQ_ORACLE_H
#define IQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, the values GGUF files carry. */
enum { OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14 };

/* GGUF block layouts (src/qgemm.rs:46-65). */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } or_q4k_block; /* 144 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } or_q5k_block; /* 176 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } or_q6k_block; /* 210 B */
typedef struct { uint16_t d; int8_t qs[32]; } or_q80_block;                                 /* 34 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } or_q8k_block;              /* 292 B */

/* IEEE binary16 <-> binary32 (the `half` crate's conversions: exact widening,
 * round-to-nearest-even narrowing). */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);

/* Bytes of one GGUF block and weights per block for a dtype; 0 if unknown. */
size_t or_block_bytes(int dtype);
size_t or_block_elems(int dtype);

/* candle BlockQ8K::from_float: k % 256 == 0, writes k/256 blocks. */
int or_quantize_q8k(const float *x, size_t k, or_q8k_block *out);
/* candle BlockQ8_0::from_float: k % 32 == 0, writes k/32 blocks. */
int or_quantize_q80(const float *x, size_t k, or_q80_block *out);

/* unpack_k_scales: 12 packed bytes -> 8 six-bit scales and 8 six-bit mins. */
void or_unpack_k_scales(const uint8_t packed[12], uint8_t sc[8], uint8_t mn[8]);

/* Per-block lane integers of the reference kernels: isum[k] is the i32 lane k
 * of `sumi` after one block; msum[k] (Q4_K only) is lane k of the mins
 * `prod` vector.  These are the "per-block integer dot products". */
void or_q4k_block_lanes(const or_q4k_block *w, const or_q8k_block *x, int32_t isum[8], int32_t msum[4]);
/* Q5_K (src/qgemm.rs:50-53; executed by candle's BlockQ5K::vec_dot at
 * src/gguf.rs:593, a port of ggml's AVX2 vec_dot_q5_K_q8_K -- candle-core
 * 0.11.0, not vendored here): the Q4_K lane structure with the fifth bit of
 * weight 64j + l (+32) from bit 2j (2j+1) of qh[l]; msum[k] are the four
 * lanes of madd(mins, pairwise bsums). */
void or_q5k_block_lanes(const or_q5k_block *w, const or_q8k_block *x, int32_t isum[8], int32_t msum[4]);
void or_q6k_block_lanes(const or_q6k_block *w, const or_q8k_block *x, int32_t isum[8]);
void or_q80_block_lanes(const or_q80_block *w, const or_q80_block *x, int32_t isum[8]);

/* Textbook per-block integers: the whole block's integer dot written from
 * the dequantisation formula (no lanes).  sum_k isum[k] must equal `isum`
 * here, and sum_k msum[k] must equal `msum`. */
void or_q4k_block_textbook(const or_q4k_block *w, const or_q8k_block *x, int64_t *isum, int64_t *msum);
void or_q5k_block_textbook(const or_q5k_block *w, const or_q8k_block *x, int64_t *isum, int64_t *msum);
void or_q6k_block_textbook(const or_q6k_block *w, const or_q8k_block *x, int64_t *isum);
void or_q80_block_textbook(const or_q80_block *w, const or_q80_block *x, int64_t *isum);

/* One weight row against `rows` pre-quantized inputs stored block-major
 * (inputs[block * rows + r]), writing out[r] -- the q4k_q8k_row /
 * q6k_q8k_row / q80_q80_row entry (src/qgemm.rs:447-468).
 * `_lanes` is a scalar emulation of the AVX2 lane arithmetic; `_avx2` is the
 * intrinsic form (only when built with AVX2+FMA; returns -1 otherwise). */
void or_q4k_q8k_row_lanes(const or_q4k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out);
/* Q5_K per (row, input): eight f32 lanes advanced by fma(d, isum_k) per
 * block, the mins as one f32 scalar summs = summs + dmin * (m . q8s) per
 * block (multiply, then add), result hsum_f32_8(acc) + summs -- ggml's
 * published vec_dot_q5_K_q8_K order.  PARITY UNPINNED against candle's
 * AVX2 code itself, which is absent here. */
void or_q5k_q8k_row_lanes(const or_q5k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out);
void or_q6k_q8k_row_lanes(const or_q6k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out);
void or_q80_q80_row_lanes(const or_q80_block *w, size_t nb, const or_q80_block *in, size_t rows, float *out);
int or_q4k_q8k_row_avx2(const or_q4k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out);
int or_q6k_q8k_row_avx2(const or_q6k_block *w, size_t nb, const or_q8k_block *in, size_t rows, float *out);
int or_q80_q80_row_avx2(const or_q80_block *w, size_t nb, const or_q80_block *in, size_t rows, float *out);
int or_have_avx2(void);

/* Dequantise n_rows rows of GGUF blocks to f32 (ggml's to_float formulas). */
int or_dequantize(int dtype, const void *blocks, size_t n_rows, size_t cols, float *out);

/* fused_forward: y[m x n_rows] = x[m x cols] . W^T, quantising each input row
 * with from_float, packing block-major, and running the per-row kernel over
 * all output rows.  impl: 0 = scalar lanes, 1 = AVX2.  nthreads >= 1 splits
 * the output rows over threads (RowSpread::Pool); the result does not depend
 * on it.  Returns 0 or a negative error. */
int or_matmul(int dtype, const void *w, size_t n_rows, size_t cols,
              const float *x, size_t m, float *y, int impl, int nthreads);

/* Pin the row-spread pool: worker t (t >= 1) runs on cpus[t % n]; the
 * calling thread is worker 0 and pins itself.  n = 0 unpins new workers. */
void or_pool_pin(const int *cpus, int n);

/* tiled_multi_row: the same product, in 16-row tiles never leaving one row
 * alone (src/gguf.rs:493-520). */
int or_matmul_tiled(int dtype, const void *w, size_t n_rows, size_t cols,
                    const float *x, size_t m, float *y, int impl, int nthreads);

/* top_k_routes (src/qwen/moe.rs:21-54): softmax over each row of logits
 * [m x e], rank descending by probability (exactly equal probabilities,
 * which the reference's unstable sort leaves unordered: larger logit, then
 * lower index), keep k,
 * renormalise when `normalize`.  experts/weights are [m x k]. */
int or_top_k_routes(const float *logits, size_t m, size_t e, size_t k, int normalize,
                    int32_t *experts, float *weights);

/* One quantised MoE sublayer (src/qwen/quantized_moe.rs).
 * Expert tensors are GGUF [experts, rows, cols] byte arrays:
 *   gate, up : [E, inter, hidden]   (gate rows then up rows form gate_up)
 *   down     : [E, hidden, inter]
 * Shared expert: shared_gate/shared_up [inter, hidden], shared_down
 * [hidden, inter]; selector f32 [hidden] (may be NULL: no shared expert).
 * Router logits [m x E] are given (the router matmul is not on this path).
 * mode: 0 = token-major (routed_token_major), 1 = grouped by expert
 * (routed_grouped_by_expert).  Both must agree bitwise. */
typedef struct {
    size_t hidden, inter, n_experts, top_k;
    int normalize;
    int gate_dtype, down_dtype, shared_gate_dtype, shared_down_dtype;
    const void *gate, *up, *down;
    const void *shared_gate, *shared_up, *shared_down;
    const float *selector;
} or_moe_layer;

int or_moe_forward(const or_moe_layer *layer, const float *x, const float *logits, size_t m,
                   float *out, int32_t *experts, float *weights, int mode, int impl, int nthreads);

/* The router matmul, logits[t][e] = x[t] . router[e] for f32 x [m x h]
 * and router [e x h] (src/qwen/quantized_moe.rs:253, a candle f32 Linear
 * whose summation order is not visible here).  order 0: summed in double
 * and rounded once (the exact product to within one rounding); order 1:
 * summed sequentially in f32 over h. */
void or_router_logits(const float *x, size_t m, size_t h, const float *router, size_t e, float *logits, int order);

/* Pieces of the MoE exposed for tests. */
float or_silu_mul(float gate, float up);  /* (g / (1 + exp(-g))) * u */
float or_sigmoid(float v);                /* 1 / (exp(-v) + 1) */

#ifdef __cplusplus
}
#endif
#endif
