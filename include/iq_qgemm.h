/*
 * iq_qgemm.h -- C ABI of the MI355X (gfx950) quantised-matmul library.
 *
 * This is the drop-in boundary for inferq's quantised-matmul hot path.  A
 * thin FFI crate binds these symbols so that the reference's matrix-level
 * entry points run on the GPU instead of the AVX2 kernels.  Each entry point
 * cites the reference interface it replaces (paths relative to the
 * reference root).
 *
 * Conventions
 *   - Plain pointers and sizes only.  Matrices are GGUF blocks in their
 *     native on-disk layout, row-major, rows * (cols / block_elems) blocks.
 *   - "device" pointers are HBM addresses on the current device; "host"
 *     pointers are ordinary process memory.
 *   - Every function returns IQ_OK (0) or a negative IQ_ERR_* code;
 *     iq_last_error() returns this thread's message for the last failure.
 *   - Results are deterministic and do not depend on the row count.  For
 *     Q4_K, Q6_K and Q8_0 matrices they are bit-identical to the
 *     reference's CPU kernels for the same inputs, on every entry except
 *     iq_matmul_via(..., IQ_PATH_PREFILL_TILES, ...) and MoE handles set to
 *     IQ_PATH_PREFILL_TILES (iq_moe_set_path), which a caller must request
 *     explicitly (their f32 order differs; within 1e-4).  Four f32
 *     orders follow a published or fixed order that the reference's own
 *     code (candle's, absent here) could not be checked against, so they
 *     are bit-identical to this library's CPU restatement and within 1e-4
 *     of the reference: Q5_K products (ggml's vec_dot_q5_K_q8_K order),
 *     F32 / BF16 matrix products, the router logits of iq_moe_forward_x,
 *     and the shared-expert selector dot.
 *   - Workspaces: library-owned device memory grows on the first call that
 *     needs more and is never freed under a graph that may still use it.
 *     Growth is refused during graph capture; the *_reserve entries size a
 *     workspace ahead of a capture.
 *   - stream is a hipStream_t (NULL = the default stream).
 */
#ifndef IQ_QGEMM_H
#define IQ_QGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids as carried by GGUF (the reference's GgmlDType).  The
 * executable matrix dtypes are the reference's (QuantizedMatrix::new,
 * src/gguf.rs:305-317).  Q5_K products follow ggml's published
 * vec_dot_q5_K_q8_K order on every kernel that takes them (the split-K
 * GEMV, the exact MFMA tiles, the lane kernel; the reference hands Q5_K to
 * candle's per-row vec_dot, src/gguf.rs:593).  F32 and BF16 matrices, which the reference
 * multiplies through candle's f32 matmul (no multi-row kernel,
 * src/gguf.rs:533-535, :599), take an f32 product in a fixed order of this
 * library's (the MoE router's: per lane over k = lane + 64 j, then a
 * butterfly), within 1e-4 of the reference and bitwise the same at every
 * row count; they have no fixed kernel paths and no per-block sums. */
enum iq_dtype { IQ_F32 = 0, IQ_Q8_0 = 8, IQ_Q4_K = 12, IQ_Q5_K = 13, IQ_Q6_K = 14, IQ_BF16 = 30 };

enum iq_status {
    IQ_OK = 0,
    IQ_ERR_INVALID = -1, /* null handle / pointer, bad argument */
    IQ_ERR_SHAPE = -2,   /* width not a whole number of blocks, wrong input width, size mismatch */
    IQ_ERR_DTYPE = -3,   /* dtype outside {F32, BF16, Q8_0, Q4_K, Q5_K, Q6_K}, mismatched dtypes, or no kernel */
    IQ_ERR_OOM = -4,     /* device allocation failed */
    IQ_ERR_HIP = -5,     /* HIP runtime error (launch, copy, no device) */
    IQ_ERR_RANGE = -6    /* index out of range (expert, rows) */
};

/* Kernel choice of iq_matmul_via (the reference's MultiRowPath,
 * src/gguf.rs:43-62): IQ_PATH_AUTO is iq_matmul's dispatch.  The fixed paths
 * run one kernel at any row count it covers, so a benchmark or a parity
 * test can hold everything but the kernel constant.  All give the
 * reference's bits except IQ_PATH_PREFILL_TILES: int8-MFMA prefill tiles
 * (Q4_K, 64 or more input rows) whose block integers are exact but whose
 * f32 combination runs in tile order, within 1e-4 normwise of the
 * reference -- faster at prefill widths, and not output-preserving across
 * row counts, so never chosen by the dispatch. */
enum iq_path {
    IQ_PATH_AUTO = 0,
    IQ_PATH_LANES = 1,        /* generic lane kernel (any dtype, any m) */
    IQ_PATH_GEMV = 2,         /* LDS-staged GEMV (1..63 rows, K-quant and Q8_0) */
    IQ_PATH_LANE_MFMA = 3,    /* exact lane order on int8 MFMA (Q4_K / Q6_K) */
    IQ_PATH_PREFILL_TILES = 4 /* tile-order int8 MFMA (Q4_K, m >= 64): NOT bitwise */
};

typedef struct iq_weight *iq_weight_t;
typedef struct iq_moe *iq_moe_t;
typedef struct iq_gguf *iq_gguf_t;
typedef struct iq_experts *iq_experts_t;
typedef void *iq_stream_t;

/* Library version string. */
const char *iq_version(void);

/* Thread-local message of the last failing call on this thread. */
const char *iq_last_error(void);

/* Select `device` for this thread and check it is a gfx950 GPU.
 * Replaces: threading::init / require_exact_kernels, the reference's
 * start-up capability gate (src/gguf.rs:1043-1053, src/threading.rs:35-55). */
int iq_init(int device);

/* ---- Weights resident in HBM, native GGUF block layout ---------------- */

/* Copy `nbytes` of host GGUF block bytes for a [rows x cols] matrix to HBM.
 * Replaces: GgufCheckpoint::load_matrix / QuantizedMatrix::new
 * (src/gguf.rs:1234, :297-320) -- the storage an executable matrix owns. */
int iq_weights_upload(const void *host_bytes, size_t nbytes, int dtype, int64_t rows, int64_t cols,
                      iq_weight_t *out);

/* Wrap block bytes already in HBM (not copied, not freed by the library);
 * `device_bytes` must be 16-byte aligned.  Used for slices of resident
 * expert tensors [experts, rows, cols].
 * Replaces: GgufExpertTensor::load (src/gguf.rs:1276-1319, :1404-1458). */
int iq_weights_view(const void *device_bytes, size_t nbytes, int dtype, int64_t rows, int64_t cols,
                    iq_weight_t *out);

/* Release a handle (and the HBM it owns, for uploads and derived matrices). */
int iq_weights_free(iq_weight_t w);

/* dtype, shape, storage bytes and HBM address of a matrix.
 * Replaces: QuantizedMatrix::{dtype, shape, storage_bytes} (src/gguf.rs:322-332). */
int iq_weights_info(iq_weight_t w, int *dtype, int64_t *rows, int64_t *cols, size_t *nbytes,
                    const void **device_bytes);

/* Row concatenation: a's rows then b's rows, byte-identical.
 * Replaces: QuantizedMatrix::concatenate_rows (src/gguf.rs:379-404). */
int iq_weights_concat_rows(iq_weight_t a, iq_weight_t b, iq_weight_t *out);

/* The first `rows` output rows as a new matrix (a contiguous byte prefix).
 * Replaces: QuantizedMatrix::leading_rows (src/gguf.rs:352-377). */
int iq_weights_leading_rows(iq_weight_t a, int64_t rows, iq_weight_t *out);

/* ---- Products ---------------------------------------------------------- */

/* y[m x rows] = x[m x cols] . W^T for device f32 x and y (row-major).  The
 * input rows are quantised on the GPU exactly as the reference's
 * from_float does (Q8K for K-quants, Q8_0 for Q8_0) and the product follows
 * the reference's per-lane f32 order, for any m >= 1: each output row is
 * bitwise what a one-row call gives.  Uses a library workspace per (device,
 * stream): calls on different streams or threads never share memory, and
 * the library lock is held while a call enqueues its launches.  A workspace
 * grows on the first call that needs more; such a call fails during graph
 * capture, so call iq_matmul_reserve for the widest call first (or make one
 * eager call of that size, or use iq_matmul_ws).  A grown workspace's old
 * buffer stays allocated until iq_workspace_release, so a graph captured
 * before a wider eager call on the same stream stays valid.
 * Replaces: QuantizedMatrix::forward / forward_spread / forward_rows /
 * multi_row_forward / fused_forward (src/gguf.rs:406-456, :558-690) and the
 * per-row kernels q4k_q8k_row / q6k_q8k_row / q80_q80_row they call
 * (src/qgemm.rs:447-468). */
int iq_matmul(iq_weight_t w, const float *x, int64_t m, float *y, iq_stream_t stream);

/* iq_matmul on one chosen kernel (enum iq_path); IQ_ERR_DTYPE when that
 * kernel does not cover the dtype, shape or row count.
 * Replaces: QuantizedMatrix::forward_via (src/gguf.rs:522-556). */
int iq_matmul_via(iq_weight_t w, const float *x, int64_t m, float *y, int path, iq_stream_t stream);

/* Size the library workspace of `stream` (current device) for calls of up
 * to m input rows of W through iq_matmul, iq_matmul_via and
 * iq_matmul_argmax, so that such calls can be captured into a graph
 * without an eager call first.  Not during capture.
 * Replaces: the reference's load-time allocation of the per-call buffers
 * fused_forward otherwise allocates per call (src/gguf.rs:608-690). */
int iq_matmul_reserve(iq_weight_t w, int64_t m, iq_stream_t stream);

/* Free the library workspace of `stream` on the current device (its live
 * buffer and every buffer it outgrew), after synchronising the stream.  A
 * graph captured with entries on that stream must not be replayed after
 * this call.  For callers that create and destroy many streams; the next
 * call on the stream allocates again.
 * No counterpart in the reference (its per-call buffers are Rust Vecs). */
int iq_workspace_release(iq_stream_t stream);

/* Device workspace bytes iq_matmul_ws needs for m input rows of W (any
 * path). */
size_t iq_matmul_workspace_size(iq_weight_t w, int64_t m);

/* iq_matmul with a caller-provided device workspace (>= the size above). */
int iq_matmul_ws(iq_weight_t w, const float *x, int64_t m, float *y, void *workspace, size_t workspace_bytes,
                 iq_stream_t stream);

/* iq_matmul that allocates nothing: its workspace is a fixed 16 MiB device
 * array per GPU (iq_matmul_noalloc_max_bytes()), resolved once per device
 * at iq_init (or at the first call on a device) and held until the process
 * ends.  Calls whose workspace would exceed it fail with IQ_ERR_RANGE
 * before any launch (iq_matmul_workspace_size tells the need).  Results
 * are bitwise iq_matmul's.  Every call on one GPU shares that array, so
 * calls that overlap in time on one device (other streams or threads)
 * race; serialise them.  Safe under graph capture: no allocation, no
 * memset, no synchronisation.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (HIP graph capture, allocation-free serving loops). */
int iq_matmul_noalloc(iq_weight_t w, const float *x, int64_t m, float *y, iq_stream_t stream);
size_t iq_matmul_noalloc_max_bytes(void);

/* iq_matmul for host x and y (copies in, computes, copies out, synchronises).
 * Replaces: the same entries, for a caller holding host slices
 * (QuantizedMatrix::forward_rows, src/gguf.rs:433-456). */
int iq_matmul_host(iq_weight_t w, const float *x_host, int64_t m, float *y_host);

/* ---- Per-row kernel entries (the reference's argument order) ------------- */

/* out[r] = weight-row . input row r for one weight row of GGUF blocks
 * (weight, weight_blocks of them) and `rows` input rows already quantised
 * by from_float (Q8K blocks of 292 B for the K-quants, Q8_0 blocks of 34 B),
 * stored block-major: inputs[block * rows + r], input_blocks of them.  Host
 * slices; synchronous.  The reference's preconditions are checked and
 * reported with IQ_ERR_SHAPE (out_len == rows, input_blocks == rows *
 * weight_blocks).  Results are the reference kernel's bit for bit.
 * Replaces: q4k_q8k_row / q6k_q8k_row / q80_q80_row (src/qgemm.rs:447-468)
 * for callers that keep the per-row structure; iq_matmul is the fast path. */
int iq_q4k_q8k_row(const void *weight, size_t weight_blocks, const void *inputs, size_t input_blocks, size_t rows,
                   float *out, size_t out_len);
int iq_q6k_q8k_row(const void *weight, size_t weight_blocks, const void *inputs, size_t input_blocks, size_t rows,
                   float *out, size_t out_len);
int iq_q80_q80_row(const void *weight, size_t weight_blocks, const void *inputs, size_t input_blocks, size_t rows,
                   float *out, size_t out_len);

/* ---- Greedy selection ----------------------------------------------------- */

/* idx[r] = the index of the largest finite value of logit row r of device
 * y [m x n] (row-major): among equal values the LAST index (Rust's max_by),
 * -0 equal to +0, NaN and +-inf skipped; -1 when row r has no finite value
 * (the reference's "all logits are non-finite" error).  val[r] (device, may
 * be NULL) receives that logit (NaN when idx is -1).  m <= 65535.
 * Replaces: sampling::argmax (src/sampling.rs:104-110), the greedy sampler
 * over the LM head's logits. */
int iq_argmax_rows(const float *y, int64_t m, int64_t n, int32_t *idx, float *val, iq_stream_t stream);

/* The LM head with greedy selection: idx/val as iq_argmax_rows over
 * x . W^T, whose logits (bitwise iq_matmul's) stay in the library workspace
 * and are never handed back -- a greedy decode step reads m indices
 * instead of m x rows floats.  Where the product runs on the one-row GEMV
 * or the 2..8-row MFMA tile (the LM head), its kernel reduces the logits as
 * it writes them and one small launch joins the partial maxima; the result
 * is the same either way.  With a leading_rows matrix it is the
 * vocab-prefix draft head's selection.
 * Replaces: lm_head.forward followed by sampling::argmax
 * (src/qwen/quantized_model.rs:737-743, src/sampling.rs:104-110;
 * draft head src/qwen/quantized_mtp.rs:142-143). */
int iq_matmul_argmax(iq_weight_t w, const float *x, int64_t m, int32_t *idx, float *val, iq_stream_t stream);

/* ---- Parity hooks ------------------------------------------------------- */

/* Quantise device x[m x k] into the reference block layouts on the device:
 * Q8K blocks (292 B: f32 d, 256 i8, 16 i16 bsums) or Q8_0 blocks (34 B).
 * Replaces: candle BlockQ8K::from_float / BlockQ8_0::from_float as called
 * at src/gguf.rs:648-654. */
int iq_quantize_q8k(const float *x, int64_t m, int64_t k, void *blocks_out, iq_stream_t stream);
int iq_quantize_q80(const float *x, int64_t m, int64_t k, void *blocks_out, iq_stream_t stream);

/* Per-block lane integers of y = x . W^T (device buffers): isum is
 * [m][rows][blocks][8] (the eight i32 lanes of the reference's `sumi` per
 * block; for Q8_0 the `dot` lanes), msum is [m][rows][blocks][4] (the Q4_K
 * mins `prod` lanes; ignored otherwise, may be NULL).  y receives the
 * product as iq_matmul.
 * Replaces: the intermediate integers of q4k_tile / q6k_tile / q80_tile
 * (src/qgemm.rs:204-237, :266-330, :384-390). */
int iq_block_sums(iq_weight_t w, const float *x, int64_t m, float *y, int32_t *isum, int32_t *msum,
                  iq_stream_t stream);

/* Per-block integer totals of the prefill-tile path (IQ_PATH_PREFILL_TILES,
 * Q4_K matrices at 64 or more input rows), whose f32 combination order
 * differs from the reference's (results agree within the path's 1e-4
 * normwise tolerance) while each block's integers are exact.
 * isum and msum are [m][rows][cols / 256]: isum the block's total integer
 * dot (the sum of the reference's eight `sumi` lanes), msum its mins term
 * (the sum of the four `prod` lanes).  y receives the product.
 * Replaces: the per-block integers of q4k_tile (src/qgemm.rs:204-237) on the
 * wide-M prefill path (tiled_multi_row, src/gguf.rs:493-520). */
int iq_prefill_block_sums(iq_weight_t w, const float *x, int64_t m, float *y, int32_t *isum, int32_t *msum,
                          iq_stream_t stream);

/* ---- MoE sublayer ---------------------------------------------------------- */

/* One quantised MoE sublayer: routed experts resident in HBM as the GGUF
 * expert tensors (not copied), plus an optional shared expert.  Shapes:
 *   gate, up     [n_experts, inter, hidden]   (blk.N.ffn_{gate,up}_exps)
 *   down         [n_experts, hidden, inter]   (blk.N.ffn_down_exps)
 *   shared_gate, shared_up [inter, hidden]; shared_down [hidden, inter]
 *   selector     f32 [hidden]                 (blk.N.ffn_gate_inp_shexp)
 * Expert formats: Q4_K, Q5_K, Q6_K or Q8_0, each matrix pair in its own
 * (gate and up share one); the shared expert's formats may differ from the
 * routed experts', as a GGUF file may mix them per tensor.
 * Replaces: QuantizedMoeLayer::load (src/qwen/quantized_moe.rs:141-225) over
 * a fully resident expert cache (src/residency.rs:39-131). */
typedef struct {
    int64_t hidden, inter, n_experts, top_k;
    int normalize; /* renormalise the top-k weights to sum to one */
    int gate_dtype, down_dtype;
    const void *gate, *up, *down; /* device, 16-byte aligned */
    size_t gate_bytes, up_bytes, down_bytes;
    int shared_gate_dtype, shared_down_dtype;
    const void *shared_gate, *shared_up, *shared_down; /* device or all NULL */
    const float *selector;                              /* device; required with a shared expert */
    const float *router; /* device f32 [n_experts x hidden] (blk.N.ffn_gate_inp.weight), or NULL:
                            required by iq_moe_forward_x */
} iq_moe_desc;

int iq_moe_create(const iq_moe_desc *desc, iq_moe_t *out);
int iq_moe_destroy(iq_moe_t moe);

/* Size the handle's workspace for calls of up to max_tokens tokens (one
 * slice at most), so that they can be captured into a graph without an
 * eager call first.  Not during capture.
 * Replaces: the buffers QuantizedMoeLayer::load prepares for the layer
 * (src/qwen/quantized_moe.rs:141-225); the reference allocates the rest per
 * call. */
int iq_moe_reserve(iq_moe_t moe, int64_t max_tokens, iq_stream_t stream);

/* Tokens one set of the layer's launches serves (wider calls are sliced):
 * 4096 / top_k, and at most 32 * (8192 / n_experts). */
int64_t iq_moe_slice_tokens(iq_moe_t moe);

/* Choose how the handle's grouped (many-token) calls form the down
 * products: IQ_PATH_AUTO (the default) keeps the reference's per-lane f32
 * order, so every token's output is bit-identical to a one-token call and
 * to the reference; IQ_PATH_PREFILL_TILES forms them in tile order on
 * chunks of up to 32 rows of one expert (exact per-block integers, one f32
 * step per output and block), within 1e-4 of the reference and NOT
 * bitwise.  Gate/up stay in the exact order on both (their SwiGLU rows are
 * quantised again), and so do calls on the token-major path (up to 32
 * tokens at the reference's shapes).  Any other path is IQ_ERR_INVALID.
 * The choice applies to calls made after it; a graph captured earlier
 * keeps the path it was captured with.
 * Replaces: the path choice the reference offers for matrix products
 * (MultiRowPath, src/gguf.rs:43-62), applied to the expert products of
 * QuantizedMoeLayer::forward (src/qwen/quantized_moe.rs:336-406). */
int iq_moe_set_path(iq_moe_t moe, int path);

/* out[m x hidden] = MoE(x[m x hidden]) for device x, router logits
 * [m x n_experts] and out.  Routing is softmax, top-k by probability,
 * renormalised (src/qwen/moe.rs:21-54); routed experts run grouped by
 * expert (src/qwen/quantized_moe.rs:336-406), SwiGLU between gate/up and
 * down, ordered combine, then routed + shared * sigmoid(x . selector)
 * (:266-273).  experts_out [m x top_k] i32 and weights_out [m x top_k] f32
 * (device, may be NULL) receive the routes.  Any m: a call wider than
 * iq_moe_slice_tokens runs as consecutive slices of that many tokens on
 * `stream`, which gives every token the same bits as one call would.
 * The handle owns a workspace, sized for one token at create and grown by
 * iq_moe_reserve or by the widest call so far (up to one slice); growth is
 * refused during graph capture, so reserve before capturing wider calls.
 * A grown workspace's old buffer stays allocated until iq_moe_destroy, so
 * graphs captured earlier stay valid.  Calls on one handle must not
 * overlap in time (they share the workspace); use one handle per stream.
 * Replaces: QuantizedMoeLayer::forward (src/qwen/quantized_moe.rs:227-281)
 * minus the router matmul, whose logits are the input here. */
int iq_moe_forward(iq_moe_t moe, const float *x, const float *router_logits, int64_t m, float *out,
                   int32_t *experts_out, float *weights_out, iq_stream_t stream);

/* The whole sublayer from x: router logits = x . router^T on the GPU (f32,
 * a fixed order per (token, expert): per lane over h = lane + 64 j, then a
 * butterfly -- the reference's candle gemm order is not visible), then as
 * iq_moe_forward; when `residual` (device [m x hidden], 16-byte aligned) is
 * not NULL, out = residual + MoE(x), the residual add of the decoder layer.
 * Needs a layer created with a router.
 * Replaces: QuantizedMoeLayer::forward (src/qwen/quantized_moe.rs:227-281,
 * router matmul at :253) and the residual add that follows it
 * (src/qwen/quantized_layer.rs:212). */
int iq_moe_forward_x(iq_moe_t moe, const float *x, int64_t m, const float *residual, float *out,
                     int32_t *experts_out, float *weights_out, iq_stream_t stream);

/* iq_moe_forward, also recording events[0..3] (hipEvent_t handles created by
 * the caller) on `stream`: before the routing launch, then after the
 * routing, gate/up and down launches.  Consecutive event pairs time the
 * three kernels.  At most iq_moe_slice_tokens tokens.
 * Replaces: the per-stage QuantizedMoeTimings the reference collects
 * (src/qwen/quantized_moe.rs:67-96, :252-275). */
int iq_moe_forward_timed(iq_moe_t moe, const float *x, const float *router_logits, int64_t m, float *out,
                         int32_t *experts_out, float *weights_out, void *const events[4], iq_stream_t stream);

/* Launch one stage of the last iq_moe_forward call on this handle again,
 * with the same inputs: stage 1 = the gate/up launch, stage 2 = the down
 * launch (the M = 1 path; stage 0 = the routing launch of the grouped
 * path).  The outputs are identical to that call's.  For timing a single
 * kernel in isolation.
 * Replaces: the per-stage timers of QuantizedMoeTimings
 * (src/qwen/quantized_moe.rs:67-96). */
int iq_moe_forward_stage(iq_moe_t moe, int stage, iq_stream_t stream);

/* ---- GGUF checkpoints and expert residency ------------------------------- */

/* Open a GGUF (v2/v3, little endian) checkpoint and parse its header,
 * metadata and tensor infos on the host (no device work).  Malformed or
 * truncated files are refused with IQ_ERR_SHAPE.
 * Replaces: GgufCheckpoint::open (src/gguf.rs:1200-1232, candle gguf_file). */
int iq_gguf_open(const char *path, iq_gguf_t *out);
int iq_gguf_close(iq_gguf_t g);

/* Tensor listing: count, the name of tensor `index` (file's info order). */
int64_t iq_gguf_tensor_count(iq_gguf_t g);
const char *iq_gguf_tensor_name(iq_gguf_t g, int64_t index);

/* dtype (GGML type id), dimension count, dims outermost first as the
 * reference's shapes read ([experts, rows, columns] for expert tensors;
 * unused trailing entries 0), absolute file offset and byte size (0 for a
 * dtype this library cannot size) of tensor `name`.
 * Replaces: GgufCheckpoint::tensor_info (src/gguf.rs:1236-1262). */
int iq_gguf_tensor_info(iq_gguf_t g, const char *name, int *dtype, int *n_dims, int64_t dims[4],
                        uint64_t *file_offset, uint64_t *nbytes);

/* Integer (or bool / float truncated) and string metadata values; the
 * string is owned by the handle, NULL when absent or not a string. */
int iq_gguf_meta_int(iq_gguf_t g, const char *key, int64_t *value);
const char *iq_gguf_meta_str(iq_gguf_t g, const char *key);

/* A 2-D quantised tensor streamed from the file into HBM as a matrix.
 * Replaces: GgufCheckpoint::load_matrix (src/gguf.rs:1234). */
int iq_gguf_load_matrix(iq_gguf_t g, const char *name, iq_weight_t *out);

/* Raw bytes of tensor `name` into device memory (capacity >= its size),
 * e.g. the F32 router and shared-expert selector; synchronises `stream`.
 * Replaces: TensorInfo::read as GgufCheckpoint uses it for F32 tensors
 * (src/gguf.rs:1263-1274). */
int iq_gguf_upload_tensor(iq_gguf_t g, const char *name, void *device_dst, size_t capacity, iq_stream_t stream);

/* Make every routed expert of layers [0, n_layers) resident in HBM: the
 * blk.N.ffn_{gate,up,down}_exps.weight tensors are read in file order
 * (sequential I/O through pinned staging, overlapped with the copies),
 * each layer's gate and up placed side by side as the pair one product
 * reads, and checked for pairing (same dtype and shape) and for down's
 * transposed shape.  Owned by the handle until iq_experts_free.
 * Replaces: warm_all_experts with a pinned expert cache
 * (src/residency.rs:39-131) and GgufCheckpoint::expert_tensor /
 * expert_pair (src/gguf.rs:1283-1360). */
int iq_gguf_load_experts(iq_gguf_t g, int64_t n_layers, iq_experts_t *out);
int iq_experts_free(iq_experts_t r);
size_t iq_experts_bytes(iq_experts_t r); /* file bytes made resident */

/* Fill the routed-expert fields of an iq_moe_desc (hidden, inter,
 * n_experts, dtypes, gate/up/down pointers and sizes) for one resident
 * layer; the caller adds top_k, normalize, the shared expert, selector
 * and router, then calls iq_moe_create.  The pointers stay valid until
 * iq_experts_free. */
int iq_experts_layer(iq_experts_t r, int64_t layer, iq_moe_desc *desc);

#ifdef __cplusplus
}
#endif
#endif
