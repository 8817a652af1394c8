// iq_moe_api.cpp -- C ABI of the MoE sublayer (include/iq_qgemm.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <mutex>
#include <vector>

#include "../../include/iq_qgemm.h"
#include "iq_api_internal.h"
#include "iq_moe.h"

#define IQ_API extern "C" __attribute__((visibility("default")))

struct iq_moe {
    iq::MoeParams layer;
    iq::MoeParams last;  // parameters of the last forward call
    bool has_last = false;
    int gfmt = 0, dfmt = 0;
    // A shared expert whose formats differ from the routed experts' runs
    // apart: the routed launches go without it, then its three products
    // (views of the caller's matrices) and a combine.
    bool shared_apart = false;
    iq_weight sgate, sup, sdown;
    const float* selector = nullptr;
    std::mutex mu;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    int ws_m = 0;
    // Workspaces replaced by a larger one.  A graph captured earlier still
    // holds their addresses, so they stay allocated until the handle is
    // destroyed.
    std::vector<void*> retired;
};

namespace {

using namespace iq;

constexpr size_t a256(size_t n) { return (n + 255) & ~(size_t)255; }

int64_t row_bytes_of(int dtype, int64_t cols) { return cols / block_elems(dtype) * block_bytes(dtype); }

// Carve the per-call workspace for m tokens; returns its size when base is null.
size_t carve(iq_moe* L, int m, uint8_t* base, MoeParams* p) {
    const int64_t K = L->layer.K, H = L->layer.H, I = L->layer.I;
    const int64_t na = m * K, gmax = na + 1, P = na + m;
    const int64_t ngI = (I + 255) / 256;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        uint8_t* ptr = base ? base + off : nullptr;
        off += a256(bytes);
        return ptr;
    };
    uint8_t* experts = take(na * 4);
    uint8_t* weights = take(na * 4);
    uint8_t* sgate = take(m * 4);
    uint8_t* meta = take(16);
    uint8_t* gexp = take(gmax * 4);
    uint8_t* gstart = take(gmax * 4);
    uint8_t* gcount = take(gmax * 4);
    uint8_t* arow = take(P * 4);
    uint8_t* spos = take(na * 4);
    uint8_t* ctr = take(gmax * ngI * 4);
    uint8_t* xq = take(act_bytes(m, H));
    uint8_t* act = take(P * I * 4);
    uint8_t* aq = take(act_bytes(P, I));
    uint8_t* vals = take(P * H * 4);
    const int64_t ngH = (H + 255) / 256;
    const int maxch = moep_max_chunks(m, K, L->layer.E, kMpRows);
    const int maxtch = moep_max_chunks(m, K, L->layer.E, kMpTileRows);
    uint8_t* xhs = take(m * ngH * 32);
    uint8_t* ahs = take(P * ngI * 32);
    uint8_t* chg = take((size_t)maxch * 4);
    uint8_t* chr = take((size_t)maxch * 4);
    uint8_t* tchg = take((size_t)maxtch * 4);
    uint8_t* tchr = take((size_t)maxtch * 4);
    uint8_t* lgw = L->layer.router ? take((size_t)m * L->layer.E * 4) : nullptr;
    // the shared expert run apart: gate, up and SwiGLU rows [m x I], its
    // output [m x H] and the products' workspace
    uint8_t *sg = nullptr, *su = nullptr, *sa = nullptr, *so = nullptr, *smw = nullptr;
    size_t smw_bytes = 0;
    if (L->shared_apart) {
        sg = take((size_t)m * I * 4);
        su = take((size_t)m * I * 4);
        sa = take((size_t)m * I * 4);
        so = take((size_t)m * H * 4);
        smw_bytes = std::max({matmul_ws_bytes(&L->sgate, m), matmul_ws_bytes(&L->sup, m), matmul_ws_bytes(&L->sdown, m)});
        smw = take(smw_bytes);
    }
    if (p) {
        p->shared_g = (float*)sg;
        p->shared_u = (float*)su;
        p->shared_act = (float*)sa;
        p->shared_out = (float*)so;
        p->shared_ws = smw;
        p->shared_ws_bytes = smw_bytes;
        p->logits_ws = (float*)lgw;
        p->experts = (int32_t*)experts;
        p->weights = (float*)weights;
        p->sgate = (float*)sgate;
        p->meta = (int32_t*)meta;
        p->group_expert = (int32_t*)gexp;
        p->group_start = (int32_t*)gstart;
        p->group_count = (int32_t*)gcount;
        p->assign_row = (int32_t*)arow;
        p->slot_pos = (int32_t*)spos;
        p->counters = (int32_t*)ctr;
        p->xq = act_carve(xq, m, H);
        p->act = (float*)act;
        p->aq = act_carve(aq, P, I);
        p->vals = (float*)vals;
        p->xhs = (_Float16*)xhs;
        p->ahs = (_Float16*)ahs;
        p->chunk_group = (int32_t*)chg;
        p->chunk_r0 = (int32_t*)chr;
        p->max_chunks = maxch;
        p->tchunk_group = (int32_t*)tchg;
        p->tchunk_r0 = (int32_t*)tchr;
        p->max_tchunks = maxtch;
    }
    (void)ctr;
    return off;
}

// Tokens one set of launches serves: the grouping kernels keep every
// (token, route) pair of a call on chip (kMoeMaxAssign of them), and the
// many-token path keeps a bitmask of tokens per expert in 32 KiB of LDS.
// A wider call runs as consecutive slices of this many tokens; every
// token's output is independent of the others in its call, so the slices
// give the same bits as one call would.
int slice_tokens(const iq_moe* L) {
    const int64_t by_assign = kMoeMaxAssign / L->layer.K;
    const int64_t by_mask = 32 * (8192 / std::max<int64_t>(L->layer.E, 1));
    return (int)std::max<int64_t>(1, std::min(by_assign, by_mask));
}

// Make the handle's workspace serve calls of m tokens (m <= slice_tokens).
// Refused during graph capture.  The buffer it replaces is kept until the
// handle is destroyed, so graphs captured on it stay valid.
int grow_workspace(iq_moe* L, int m, hipStream_t s, bool at_create = false) {
    if (L->ws_m >= m) return IQ_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = at_create ? hipSuccess : hipStreamIsCapturing(s, &cs);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
        return fail(IQ_ERR_INVALID,
                    "the MoE workspace must grow to %d tokens, which cannot happen during graph capture: call "
                    "iq_moe_reserve (or make one eager call of at least this many tokens) on the handle first",
                    m);
    const size_t bytes = carve(L, m, nullptr, nullptr);
    void* ws = nullptr;
    e = hipMalloc(&ws, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(IQ_ERR_OOM, "MoE workspace of %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    e = hipMemset(ws, 0, bytes);  // the completion counters start at zero
    if (e != hipSuccess) {
        (void)hipFree(ws);
        return hip_fail(e, "hipMemset");
    }
    if (L->ws) L->retired.push_back(L->ws);
    L->ws = ws;
    L->ws_bytes = bytes;
    L->ws_m = m;
    return IQ_OK;
}

}  // namespace

IQ_API int iq_moe_create(const iq_moe_desc* d, iq_moe_t* out) {
    if (!d || !out) return fail(IQ_ERR_INVALID, "null pointer");
    const int64_t E = d->n_experts, K = d->top_k, H = d->hidden, I = d->inter;
    if (!(K > 0 && K <= E)) return fail(IQ_ERR_SHAPE, "invalid top-k %lld for %lld experts", (long long)K, (long long)E);
    if (E > kMoeMaxExperts || K > kMoeMaxTopK)
        return fail(IQ_ERR_RANGE, "this build supports at most %d experts and top-%d (got %lld, %lld)", kMoeMaxExperts,
                    kMoeMaxTopK, (long long)E, (long long)K);
    if (!moe_dtype_ok(d->gate_dtype) || !moe_dtype_ok(d->down_dtype))
        return fail(IQ_ERR_DTYPE, "unsupported expert dtypes %d / %d; expected Q4_K, Q5_K, Q6_K or Q8_0",
                    d->gate_dtype, d->down_dtype);
    if (H <= 0 || I <= 0 || H % block_elems(d->gate_dtype) || I % block_elems(d->down_dtype) || I % 32)
        return fail(IQ_ERR_SHAPE, "hidden %lld / intermediate %lld do not fit %s gate and %s down blocks",
                    (long long)H, (long long)I, dtype_name(d->gate_dtype), dtype_name(d->down_dtype));
    const int64_t grb = row_bytes_of(d->gate_dtype, H), drb = row_bytes_of(d->down_dtype, I);
    if (!d->gate || !d->up || !d->down) return fail(IQ_ERR_INVALID, "null expert tensor");
    if (d->gate_bytes != (size_t)(E * I * grb))
        return fail(IQ_ERR_SHAPE, "invalid gate expert shape: %zu bytes for [%lld, %lld, %lld] %s", d->gate_bytes,
                    (long long)E, (long long)I, (long long)H, dtype_name(d->gate_dtype));
    if (d->up_bytes != d->gate_bytes)
        return fail(IQ_ERR_SHAPE, "up expert shape (%zu bytes) does not match gate shape (%zu bytes)", d->up_bytes,
                    d->gate_bytes);
    if (d->down_bytes != (size_t)(E * H * drb))
        return fail(IQ_ERR_SHAPE, "invalid down expert shape: %zu bytes for [%lld, %lld, %lld] %s", d->down_bytes,
                    (long long)E, (long long)H, (long long)I, dtype_name(d->down_dtype));
    for (const void* ptr : {d->gate, d->up, d->down, (const void*)d->shared_gate, (const void*)d->shared_up,
                            (const void*)d->shared_down, (const void*)d->selector, (const void*)d->router})
        if ((uintptr_t)ptr & 15u) return fail(IQ_ERR_INVALID, "device tensors must be 16-byte aligned");
    const int nshared = (d->shared_gate != nullptr) + (d->shared_up != nullptr) + (d->shared_down != nullptr);
    if (nshared != 0 && nshared != 3) return fail(IQ_ERR_INVALID, "shared expert needs gate, up and down matrices");
    const bool apart = nshared == 3 && (d->shared_gate_dtype != d->gate_dtype || d->shared_down_dtype != d->down_dtype);
    if (nshared == 3) {
        if (!d->selector) return fail(IQ_ERR_INVALID, "shared expert needs its f32 selector vector");
        if (!moe_dtype_ok(d->shared_gate_dtype) || !moe_dtype_ok(d->shared_down_dtype))
            return fail(IQ_ERR_DTYPE, "unsupported shared expert dtypes %d / %d; expected Q4_K, Q5_K, Q6_K or Q8_0",
                        d->shared_gate_dtype, d->shared_down_dtype);
        // the shared matrices are [inter, hidden] and [hidden, inter] in their own formats
        if (H % block_elems(d->shared_gate_dtype) || I % block_elems(d->shared_down_dtype))
            return fail(IQ_ERR_SHAPE, "hidden %lld / intermediate %lld do not fit %s shared gate and %s down blocks",
                        (long long)H, (long long)I, dtype_name(d->shared_gate_dtype),
                        dtype_name(d->shared_down_dtype));
    }
    iq_moe* L = new iq_moe;
    if (apart) {
        L->shared_apart = true;
        auto view = [&](iq_weight& w, const void* ptr, int dt, int64_t rows, int64_t cols) {
            w.dtype = dt;
            w.rows = rows;
            w.cols = cols;
            w.row_bytes = row_bytes_of(dt, cols);
            w.nbytes = (size_t)(rows * w.row_bytes);
            w.dev = (uint8_t*)ptr;
            w.owned = false;
            (void)hipGetDevice(&w.device);
        };
        view(L->sgate, d->shared_gate, d->shared_gate_dtype, I, H);
        view(L->sup, d->shared_up, d->shared_gate_dtype, I, H);
        view(L->sdown, d->shared_down, d->shared_down_dtype, H, I);
        L->selector = d->selector;
    }
    MoeParams& p = L->layer;
    p.H = H;
    p.I = I;
    p.E = E;
    p.K = K;
    p.normalize = d->normalize ? 1 : 0;
    p.gate = (const uint8_t*)d->gate;
    p.up = (const uint8_t*)d->up;
    p.down = (const uint8_t*)d->down;
    if (nshared == 3 && !apart) {
        p.sgate_w = (const uint8_t*)d->shared_gate;
        p.sup_w = (const uint8_t*)d->shared_up;
        p.sdown_w = (const uint8_t*)d->shared_down;
        p.selector = d->selector;
    }
    p.router = d->router;
    p.g_row_bytes = grb;
    p.d_row_bytes = drb;
    p.g_exp_bytes = I * grb;
    p.d_exp_bytes = H * drb;
    p.g_nbw = (int)(H / block_elems(d->gate_dtype));
    p.d_nbw = (int)(I / block_elems(d->down_dtype));
    L->gfmt = d->gate_dtype;
    L->dfmt = d->down_dtype;
    // a one-token (decode) call can be captured without an eager call first
    if (int rc = grow_workspace(L, 1, nullptr, true)) {
        delete L;
        return rc;
    }
    *out = L;
    return IQ_OK;
}

IQ_API int iq_moe_destroy(iq_moe_t L) {
    if (!L) return IQ_OK;
    if (L->ws || !L->retired.empty()) (void)hipDeviceSynchronize();  // launches may still read them
    if (L->ws) (void)hipFree(L->ws);
    for (void* p : L->retired) (void)hipFree(p);
    delete L;
    return IQ_OK;
}

IQ_API int iq_moe_reserve(iq_moe_t L, int64_t max_tokens, iq_stream_t stream) {
    if (!L) return fail(IQ_ERR_INVALID, "null MoE handle");
    if (max_tokens < 0) return fail(IQ_ERR_SHAPE, "negative token count");
    std::lock_guard<std::mutex> lock(L->mu);
    return grow_workspace(L, (int)std::min<int64_t>(max_tokens, slice_tokens(L)), (hipStream_t)stream);
}

IQ_API int64_t iq_moe_slice_tokens(iq_moe_t L) { return L ? slice_tokens(L) : 0; }

IQ_API int iq_moe_set_path(iq_moe_t L, int path) {
    if (!L) return fail(IQ_ERR_INVALID, "null MoE handle");
    if (path != IQ_PATH_AUTO && path != IQ_PATH_PREFILL_TILES)
        return fail(IQ_ERR_INVALID, "MoE path %d: expected IQ_PATH_AUTO or IQ_PATH_PREFILL_TILES", path);
    std::lock_guard<std::mutex> lock(L->mu);
    L->layer.down_tiles = path == IQ_PATH_PREFILL_TILES ? 1 : 0;
    return IQ_OK;
}

// One set of launches for m <= slice_tokens(L) tokens (the caller holds
// L->mu).  logits == nullptr: the layer's router computes them from x.
static int moe_slice(iq_moe_t L, const float* x, const float* logits, const float* residual, int64_t m, float* out,
                     int32_t* experts_out, float* weights_out, void* const* events, hipStream_t s) {
    if (int rc = grow_workspace(L, (int)m, s)) return rc;
    MoeParams p = L->layer;
    carve(L, L->ws_m, (uint8_t*)L->ws, &p);
    // carve() sized the views for ws_m tokens; the call uses m
    p.xq.m = (int)m;
    p.x = x;
    p.M = (int)m;
    p.out = out;
    // a shared expert run apart adds its term and the residual at the end
    p.residual = L->shared_apart ? nullptr : residual;
    L->has_last = false;
    hipError_t e = hipSuccess;
    if (logits) {
        p.logits = logits;
    } else {
        p.logits = p.logits_ws;
        e = launch_moe_router(p, s);
        if (e != hipSuccess) return hip_fail(e, "MoE router launch");
    }
    e = launch_moe(p, L->gfmt, L->dfmt, s, (hipEvent_t const*)events);
    if (e != hipSuccess) return hip_fail(e, "MoE launch");
    if (L->shared_apart) {
        // the reference's shared path: down(SwiGLU(gate . x, up . x)), then
        // out = residual + (routed + shared * sigmoid(x . selector))
        const int64_t I = L->layer.I, H = L->layer.H;
        if (int rc = matmul_impl(&L->sgate, x, m, p.shared_g, p.shared_ws, p.shared_ws_bytes, IQ_PATH_AUTO, nullptr,
                                 nullptr, s))
            return rc;
        if (int rc = matmul_impl(&L->sup, x, m, p.shared_u, p.shared_ws, p.shared_ws_bytes, IQ_PATH_AUTO, nullptr,
                                 nullptr, s))
            return rc;
        e = launch_moe_swiglu(p.shared_g, p.shared_u, m * I, p.shared_act, s);
        if (e != hipSuccess) return hip_fail(e, "MoE shared SwiGLU launch");
        if (int rc = matmul_impl(&L->sdown, p.shared_act, m, p.shared_out, p.shared_ws, p.shared_ws_bytes,
                                 IQ_PATH_AUTO, nullptr, nullptr, s))
            return rc;
        e = launch_moe_shared_combine(x, L->selector, p.shared_out, residual, m, H, out, s);
        if (e != hipSuccess) return hip_fail(e, "MoE shared combine launch");
    }
    L->last = p;
    L->has_last = true;
    const size_t rb = (size_t)(m * L->layer.K) * 4;
    if (experts_out && (e = hipMemcpyAsync(experts_out, p.experts, rb, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_fail(e, "hipMemcpyAsync (experts)");
    if (weights_out && (e = hipMemcpyAsync(weights_out, p.weights, rb, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_fail(e, "hipMemcpyAsync (weights)");
    return IQ_OK;
}

// A call of any width: consecutive slices of at most slice_tokens(L)
// tokens, each a complete set of launches on `stream`.
static int moe_forward(iq_moe_t L, const float* x, const float* logits, const float* residual, int64_t m,
                       float* out, int32_t* experts_out, float* weights_out, void* const* events,
                       iq_stream_t stream) {
    if (!L) return fail(IQ_ERR_INVALID, "null MoE handle");
    if (m < 0) return fail(IQ_ERR_SHAPE, "negative token count");
    if (m == 0) return IQ_OK;
    if (!logits && !L->layer.router)
        return fail(IQ_ERR_INVALID, "this MoE layer has no router: pass router logits (iq_moe_forward)");
    if (!x || !out) return fail(IQ_ERR_INVALID, "null input or output pointer");
    if (residual && ((uintptr_t)residual & 15u))
        return fail(IQ_ERR_INVALID, "the residual must be 16-byte aligned");
    if (m > INT32_MAX / std::max<int64_t>(L->layer.K, 1))
        return fail(IQ_ERR_RANGE, "%lld tokens is more than a call can route", (long long)m);
    const int64_t slice = slice_tokens(L);
    if (events && m > slice)
        return fail(IQ_ERR_RANGE, "timed MoE calls cover at most %lld tokens (got %lld)", (long long)slice,
                    (long long)m);
    hipStream_t s = (hipStream_t)stream;
    std::lock_guard<std::mutex> lock(L->mu);
    const int64_t H = L->layer.H, E = L->layer.E, K = L->layer.K;
    for (int64_t t0 = 0; t0 < m; t0 += slice) {
        const int64_t n = std::min(slice, m - t0);
        if (int rc = moe_slice(L, x + t0 * H, logits ? logits + t0 * E : nullptr, residual ? residual + t0 * H : nullptr,
                               n, out + t0 * H, experts_out ? experts_out + t0 * K : nullptr,
                               weights_out ? weights_out + t0 * K : nullptr, events, s))
            return rc;
    }
    return IQ_OK;
}

IQ_API int iq_moe_forward(iq_moe_t L, const float* x, const float* logits, int64_t m, float* out,
                          int32_t* experts_out, float* weights_out, iq_stream_t stream) {
    if (m > 0 && !logits) return fail(IQ_ERR_INVALID, "null router logits");
    return moe_forward(L, x, logits, nullptr, m, out, experts_out, weights_out, nullptr, stream);
}

IQ_API int iq_moe_forward_x(iq_moe_t L, const float* x, int64_t m, const float* residual, float* out,
                            int32_t* experts_out, float* weights_out, iq_stream_t stream) {
    return moe_forward(L, x, nullptr, residual, m, out, experts_out, weights_out, nullptr, stream);
}

IQ_API int iq_moe_forward_timed(iq_moe_t L, const float* x, const float* logits, int64_t m, float* out,
                                int32_t* experts_out, float* weights_out, void* const events[4],
                                iq_stream_t stream) {
    if (!events || !events[0] || !events[1] || !events[2] || !events[3])
        return fail(IQ_ERR_INVALID, "iq_moe_forward_timed needs four events");
    if (m > 0 && !logits) return fail(IQ_ERR_INVALID, "null router logits");
    return moe_forward(L, x, logits, nullptr, m, out, experts_out, weights_out, events, stream);
}

IQ_API int iq_moe_forward_stage(iq_moe_t L, int stage, iq_stream_t stream) {
    if (!L) return fail(IQ_ERR_INVALID, "null MoE handle");
    std::lock_guard<std::mutex> lock(L->mu);
    if (!L->has_last) return fail(IQ_ERR_INVALID, "iq_moe_forward_stage needs a previous iq_moe_forward call");
    if (L->shared_apart)
        return fail(IQ_ERR_RANGE, "stage launches cover layers whose shared expert runs in the fused kernels");
    hipError_t e = launch_moe_stage(L->last, L->gfmt, L->dfmt, stage, (hipStream_t)stream);
    if (e == hipErrorNotSupported)
        return fail(IQ_ERR_RANGE, "stage launches cover the single-token path of this layer shape only");
    if (e != hipSuccess) return hip_fail(e, "MoE stage launch");
    return IQ_OK;
}
