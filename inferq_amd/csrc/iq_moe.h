// iq_moe.h -- parameters of the MoE launches (host and device).
#pragma once

#include "iq_internal.h"

namespace iq {

constexpr int kMoeMaxExperts = 512;   // routed experts per layer
constexpr int kMoeMaxTopK = 16;       // experts per token
constexpr int kMoeMaxAssign = 4096;   // tokens * top_k per call
constexpr int kMoePrefillMinTokens = 17;  // the MFMA path serves calls of this many tokens or more

struct MoeParams {
    // The fields the one-token kernels read first share the first three
    // 64-byte lines of the kernel arguments, so that one scalar-cache fill
    // brings them in (a kernel argument on a line of its own costs its
    // kernel a dependent memory round trip before the loads that need it).
    int64_t H = 0, I = 0, E = 0, K = 0;
    int32_t* experts = nullptr;     // [M][K] (workspace)
    float* act = nullptr;           // [P][I] SwiGLU output (workspace)
    const float* x = nullptr;       // [M][H]
    const float* logits = nullptr;  // [M][E] (given, or computed from router into logits_ws)
    // layer (device pointers, GGUF native layout)
    const uint8_t* gate = nullptr;  // [E][I][H]
    const uint8_t* up = nullptr;    // [E][I][H]
    const uint8_t* down = nullptr;  // [E][H][I]
    const uint8_t* sgate_w = nullptr;  // shared expert [I][H], or null
    const uint8_t* sup_w = nullptr;    // [I][H]
    const uint8_t* sdown_w = nullptr;  // [H][I]
    int64_t g_row_bytes = 0, d_row_bytes = 0, g_exp_bytes = 0, d_exp_bytes = 0;
    int g_nbw = 0, d_nbw = 0;  // weight blocks per row of gate/up and of down
    float* weights = nullptr;  // [M][K] (workspace)
    float* sgate = nullptr;    // [M] sigmoid(x . selector) (workspace)
    const float* residual = nullptr;  // [M][H] added to the output, or null
    float* out = nullptr;             // [M][H]
    int M = 0;
    int normalize = 1;
    const float* selector = nullptr;  // [H]
    const float* router = nullptr;  // f32 [E][H] (blk.N.ffn_gate_inp.weight), or null
    float* logits_ws = nullptr;     // [M][E] workspace for the router's logits
    // workspace
    int32_t* meta = nullptr;     // [0] number of groups
    int32_t* group_expert = nullptr;
    int32_t* group_start = nullptr;
    int32_t* group_count = nullptr;
    int32_t* assign_row = nullptr;  // [P] token of each grouped position
    int32_t* slot_pos = nullptr;    // [M][K] grouped position of (token, route)
    int32_t* counters = nullptr;    // [M*K+1][ceil(I/256)], zero between calls
    ActView xq;                     // x quantised, M rows of width H
    ActView aq;                     // act quantised, P rows of width I
    float* vals = nullptr;          // [P][H] expert outputs before the combine
    // MFMA (prefill) path
    _Float16* xhs = nullptr;        // [M][H/256][16] 16-value sums of quantised x
    _Float16* ahs = nullptr;        // [P][I/256][16] the same of quantised act
    int32_t* chunk_group = nullptr;  // [max_chunks] group of each chunk of rows
    int32_t* chunk_r0 = nullptr;     // [max_chunks] first row of the chunk in its group
    int max_chunks = 0;
    // a shared expert run apart (formats other than the routed experts'):
    // gate, up, SwiGLU rows [M][I], output [M][H] and the products' workspace
    float* shared_g = nullptr;
    float* shared_u = nullptr;
    float* shared_act = nullptr;
    float* shared_out = nullptr;
    void* shared_ws = nullptr;
    size_t shared_ws_bytes = 0;
    // the grouped path's down products in tile order (on request): chunks
    // of up to kMpTileRows grouped rows, meta[2] of them
    int down_tiles = 0;
    int32_t* tchunk_group = nullptr;  // [max_tchunks]
    int32_t* tchunk_r0 = nullptr;     // [max_tchunks]
    int max_tchunks = 0;
};

constexpr int kMpRows = 16;  // grouped rows per chunk of the exact expert products
#ifndef IQ_MP_TILE_ROWS
#define IQ_MP_TILE_ROWS 32
#endif
constexpr int kMpTileRows = IQ_MP_TILE_ROWS;  // grouped rows per chunk of the tile-order down products
static_assert(kMpTileRows % 16 == 0 && kMpTileRows <= 64, "tile-order chunk rows");

// logits_ws[t][e] = x[t] . router[e] (the router matmul of
// src/qwen/quantized_moe.rs:253) in a fixed order: lane l of a wave sums
// x[h] * r[h] for h = l, l + 64, ... in order, then the lanes meet in a
// butterfly; every (token, expert) pair is formed the same way at any M.
hipError_t launch_moe_router(const MoeParams& p, hipStream_t s);

// A shared expert run apart from the routed experts (formats that differ
// from theirs): act = SwiGLU(g, u) over n values, then out = residual +
// (out + shared * sigmoid(x . selector)) for m tokens of width H.
hipError_t launch_moe_swiglu(const float* g, const float* u, int64_t n, float* act, hipStream_t s);
hipError_t launch_moe_shared_combine(const float* x, const float* selector, const float* shared, const float* residual,
                                     int64_t m, int64_t H, float* out, hipStream_t s);

// Launch prep, gate_up and down for one layer call.
// events (may be null): 4 hipEvent_t recorded before and between the launches.
hipError_t launch_moe(const MoeParams& p, int gate_dtype, int down_dtype, hipStream_t s,
                      hipEvent_t const* events = nullptr);
// The many-token path on int8 MFMA (iq_moe_prefill.hip).
bool moep_supported(const MoeParams& p, int gate_dtype, int down_dtype);
hipError_t launch_moe_prefill(const MoeParams& p, int gate_dtype, int down_dtype, hipStream_t s,
                              hipEvent_t const* events);
// Upper bound of the chunks of `rows` grouped rows a call of M tokens makes.
int moep_max_chunks(int64_t M, int64_t K, int64_t E, int rows);
// One launch of a call already made with these parameters (stage 0 routing
// of the grouped path, 1 gate/up, 2 down).
hipError_t launch_moe_stage(const MoeParams& p, int gate_dtype, int down_dtype, int stage, hipStream_t s);
}  // namespace iq
