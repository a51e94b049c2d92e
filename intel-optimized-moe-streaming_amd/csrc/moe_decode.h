// moe_decode.h -- parameter block shared by the decode kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace mqh {

// workspace flag words (int32) at the start of every workspace, sticky until
// read by mqh_status
enum : int { FLAG_NONFINITE = 0, FLAG_BAD_ID = 1, N_FLAGS = 64 };
constexpr int64_t WS_HEAD_BYTES = (int64_t)N_FLAGS * 4;

constexpr int ROUTE_PROLOGUE_MAX_EXPERTS = 256;   // 4 router scores per lane

constexpr int ROWS_A = 8;    // intermediate rows per workgroup, kernel A
constexpr int ROWS_W = 4;    // hidden rows per wavefront, kernel B
constexpr int ROWS_B = 4 * ROWS_W;

struct DecodeParams {
    // The first 64 bytes are what the fast kernels need before their first
    // loads (the token, the expert ids, the activations and the geometry of
    // the work split); the kernels take this struct as their only argument and
    // are built to preload the first 16 argument dwords into scalar registers,
    // so these are in registers when the first instruction runs.
    const float* x;         // [n_tokens x hidden]
    const int32_t* ids;     // [n_tokens x top_k]
    float* act;             // [n_tokens x S x Imax]
    const float* weights;   // [n_tokens x top_k]
    const float* sh_gate_inp;  // optional sigmoid gate vector [hidden] of the shared expert
    int top_k;
    int S, has_shared;      // slots per token (top_k + has_shared); has_shared: 0 or 1
    int n_experts;
    int a_inter;            // fast kernels: the activation row length (routed, else shared intermediate)
    int a_waves;            // fast kernels: waves per gate/up workgroup (blockDim.x / 64)
    // routed experts: stacked GGUF tensors, n_experts consecutive slices each
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    int gate_type, up_type, down_type;
    int64_t gate_eb, up_eb, down_eb;  // bytes per expert slice
    int hidden, inter;
    // shared expert (has_shared == 0: absent)
    const uint8_t* sh_gate;
    const uint8_t* sh_up;
    const uint8_t* sh_down;
    int sh_gate_type, sh_up_type, sh_down_type;
    int sh_inter;
    int n_tokens;
    // routing in the gate/up prologue (route_scores != nullptr, fast path,
    // n_experts <= ROUTE_PROLOGUE_MAX_EXPERTS): router scores [n_tokens x
    // n_experts] in; the top-k ids and weights are written to route_ids /
    // route_weights (the same memory as ids / weights, read by the down kernel)
    const float* route_scores;
    int32_t* route_ids;
    float* route_weights;
    float* y;               // [n_tokens x hidden]
    int fp16;
    // workspace views
    int* flags;             // [N_FLAGS]
    float* sh_scale;        // [n_tokens]
    int Imax;
};

struct WorkspaceLayout {
    int64_t flags_off, scale_off, act_off, total;
};

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

inline WorkspaceLayout decode_workspace_layout(int n_tokens, int top_k, int inter, int sh_inter) {
    WorkspaceLayout w;
    const int S = top_k + 1;  // room for the shared slot
    const int Imax = std::max(inter, sh_inter);
    w.flags_off = 0;
    w.scale_off = align256(WS_HEAD_BYTES);
    w.act_off = align256(w.scale_off + (int64_t)n_tokens * 4);
    w.total = align256(w.act_off + (int64_t)n_tokens * S * Imax * 4);
    return w;
}

// Grouped prefill (moe_prefill.hip).  Token/slot pairs are bucketed by expert
// on the device; a tile is up to PREFILL_TILE tokens of one expert (or of the
// shared expert, expert id -1): 8 or 16 (the MFMA's 16 token columns; with 8,
// columns 8..15 repeat 0..7 and their results are dropped).
#ifndef MQH_PREFILL_TILE
#define MQH_PREFILL_TILE 16
#endif
constexpr int PREFILL_TILE = MQH_PREFILL_TILE;
static_assert(PREFILL_TILE == 8 || PREFILL_TILE == 16, "prefill tiles of 8 or 16 tokens");
constexpr int PREFILL_MAX_EXPERTS = 1024;

struct PrefillParams {
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
    int gate_type, up_type, down_type;
    int64_t gate_eb, up_eb, down_eb;
    int n_experts, hidden, inter;
    const uint8_t* sh_gate;
    const uint8_t* sh_up;
    const uint8_t* sh_down;
    int sh_gate_type, sh_up_type, sh_down_type;   // the routed types, or Q6_K
    const float* sh_gate_inp;
    int has_shared;
    const void* x;          // [n_tokens x hidden], FP32 or BF16
    int x_bf16;
    int n_tokens;
    const int32_t* ids;     // [n_tokens x top_k]
    const float* weights;
    int top_k;
    int S;                  // slots per token: top_k + has_shared
    float* y;               // [n_tokens x hidden]
    // workspace views
    int* flags;             // [N_FLAGS]
    float* sh_scale;        // [n_tokens]
    int* tiles;             // [max_tiles x 4]: expert, first pair, token count, 0
    int* n_tiles;           // [1]
    int* tile_tok;          // [max_tiles x PREFILL_TILE]: token of column c of tile i (stale past the tile's count)
    int* tile_dst;          // [max_tiles x PREFILL_TILE]: its output row t S + s (token t, slot s)
    float* act;             // [P x inter] SwiGLU activations, in sorted pair order
    float* ypair;           // [P x hidden] expert outputs, row t S + s
    // the tokens as the gate/up kernel's B operand, made once per token by the
    // route pass: FP16 high and low planes [n_tokens x hidden] at scale 2^-k,
    // the 32-column sub-block sums [n_tokens x hidden / 32] as (high, low)
    // FP16 pairs, and k [n_tokens]
    uint16_t* xhi;
    uint16_t* xlo;
    uint32_t* xsum;
    int* xexp;
    int max_tiles;
};

struct PrefillLayout {
    int64_t flags_off, scale_off, tiles_off, ntiles_off, tok_off, dst_off, act_off, ypair_off;
    int64_t xhi_off, xlo_off, xsum_off, xexp_off, total;
    int max_tiles;
};

PrefillLayout prefill_layout(int n_tokens, int top_k, int n_experts, int hidden, int inter, int has_shared);
bool prefill_supported(const PrefillParams& p);

// Optional HIP events recorded at the start and end of the two GEMM kernels of
// a layer (A: gate/up + SwiGLU, B: down projection, with the combine in
// decode), for profiling; null members are ignored.
struct KernelEvents {
    hipEvent_t a_start = nullptr, a_stop = nullptr, b_start = nullptr, b_stop = nullptr;
    bool armed_a() const { return a_start || a_stop; }
    bool armed_b() const { return b_start || b_stop; }
};

hipError_t launch_decode_generic(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev);
hipError_t launch_delta_heads(float* state, const float* q, const float* k, const float* v, const float* beta,
                              const float* gate, float* out, int heads, int key_dim, int value_dim, int* flags,
                              hipStream_t stream, const KernelEvents& ev);
bool fast_supported(const DecodeParams& p);
hipError_t launch_decode_fast(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev);
hipError_t launch_prefill(const PrefillParams& p, hipStream_t stream, const KernelEvents& ev);
hipError_t launch_dequant(int type, const uint8_t* src, void* dst, int64_t n, int want_f16, hipStream_t stream);
hipError_t launch_route(const float* x, int n_tokens, int hidden, const float* w, int n_experts, int top_k,
                        float* scores, int32_t* ids, float* weights, hipStream_t stream);
hipError_t launch_route_scores(const float* x, int n_tokens, int hidden, const float* w, int n_experts, float* scores,
                               hipStream_t stream);
hipError_t launch_route_select(const float* scores, int n_tokens, int n_experts, int top_k, int32_t* ids,
                               float* weights, hipStream_t stream);
hipError_t launch_read_floor(const void* src, int64_t bytes, uint32_t* sink, hipStream_t stream, hipEvent_t start,
                             hipEvent_t stop);

}  // namespace mqh
