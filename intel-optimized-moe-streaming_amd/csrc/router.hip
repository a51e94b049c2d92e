// router.hip -- top-k expert routing on the GPU (ExpertRouter.route).
//
// Replaces src/flash_moe/router.py:140-170 for tokens already in HBM, so a
// decode step needs no host round trip between the router and the experts:
//   scores = x . W       FP32; W is the layer's ffn_gate_inp as the GGUF file
//                        stores it, n_experts rows of hidden floats (the
//                        reference keeps its transpose, router.py:39-59,101-135)
//   ids    = top-k of scores in descending order (argsort, last k, reversed)
//   w      = float64 softmax over the selected scores, then FP32 (the combine
//            multiplies by fl32(w), moe_layer.py:70,85-86); a non-finite or
//            non-positive exponential sum gives 1/k each (router.py:161-166).
//
// Two launches.  k_route_scores: each workgroup owns 4/SPLIT experts and a
// group of tokens; SPLIT waves share one expert row, each summing a contiguous
// share of the hidden dimension with 16-byte loads (a lane's chain, then a
// fixed DPP tree over the wave), and the shares are added in wave order, so
// the summation order of a score is fixed for a given SPLIT.
// k_route_select: one wavefront per token takes the top k by k rounds of a
// wave maximum over (score, expert) keys (route_topk.h): NaN ranks above every
// number, as np.argsort places NaN last (a NaN among the selected then makes
// the softmax sum NaN and the weights uniform, as in the reference); equal
// scores, and NaNs among themselves, are taken in ascending expert order
// (NumPy's order for ties is unspecified); -0.0 and +0.0 count as equal.
// The routed decode runs the select step inside its gate/up kernel instead
// (moe_fast.hip) when the experts number at most 256.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "moe_decode.h"
#include "route_topk.h"

namespace mqh {

constexpr int RS_WAVES = 4;    // waves per scores workgroup
constexpr int SEL_WAVES = 4;   // tokens per select workgroup, one wave each

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the wavefront in a fixed order (quads, half rows, rows, then
// (row3 + row2) + (row1 + row0)); the total lands in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v += dpp_f32<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v += dpp_f32<0x141, 0xF>(v);   // row_half_mirror
    v += dpp_f32<0x140, 0xF>(v);   // row_mirror
    const float a = dpp_f32<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v = (threadIdx.x & 16) ? v + a : v;
    const float b = dpp_f32<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
    return (threadIdx.x & 32) ? v + b : v;
}

template <int SPLIT, int TT>
__global__ __launch_bounds__(64 * RS_WAVES) void k_route_scores(const float* __restrict__ x, int n_tokens, int hidden,
                                                                const float* __restrict__ w, int n_experts,
                                                                float* __restrict__ scores) {
    constexpr int EPG = RS_WAVES / SPLIT;   // experts per workgroup
    __shared__ float part[RS_WAVES][TT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = blockIdx.x * EPG + wave / SPLIT, piece = wave % SPLIT;
    const int t0 = blockIdx.y * TT, nt = min(TT, n_tokens - t0);
    const int n4 = hidden >> 2;
    const int per = (n4 + SPLIT - 1) / SPLIT;
    const int j0 = piece * per, j1 = min(n4, j0 + per);

    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = 0.0f;
    if (e < n_experts) {
        const float4* wr = reinterpret_cast<const float4*>(w + (int64_t)e * hidden);
        const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)t0 * hidden);
        // two 16-byte columns per lane per pass, both loads issued before
        // either is used; a second column past j1 re-reads the first's and is
        // not accumulated
        for (int j = j0 + lane; j < j1; j += 128) {
            const int j2 = j + 64 < j1 ? j + 64 : j;
            const float4 wv = wr[j], wv2 = wr[j2];
            float4 xv[TT], xv2[TT];
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const int64_t row = (int64_t)min(t, nt - 1) * n4;   // rows past nt repeat the last
                xv[t] = xr[row + j];
                xv2[t] = xr[row + j2];
            }
#pragma unroll
            for (int t = 0; t < TT; ++t)
                acc[t] = fmaf(xv[t].w, wv.w, fmaf(xv[t].z, wv.z, fmaf(xv[t].y, wv.y, fmaf(xv[t].x, wv.x, acc[t]))));
            if (j + 64 < j1) {
#pragma unroll
                for (int t = 0; t < TT; ++t)
                    acc[t] = fmaf(xv2[t].w, wv2.w,
                                  fmaf(xv2[t].z, wv2.z, fmaf(xv2[t].y, wv2.y, fmaf(xv2[t].x, wv2.x, acc[t]))));
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const float v = wave_sum_to_lane63(acc[t]);
        if (lane == 63) part[wave][t] = v;
    }
    __syncthreads();
    const int le = threadIdx.x / TT, t = threadIdx.x % TT;
    const int oe = blockIdx.x * EPG + le;
    if (le < EPG && t < nt && oe < n_experts) {
        float s = part[le * SPLIT][t];
#pragma unroll
        for (int p = 1; p < SPLIT; ++p) s += part[le * SPLIT + p][t];
        scores[(int64_t)(t0 + t) * n_experts + oe] = s;
    }
}

template <int NM>
__global__ __launch_bounds__(64 * SEL_WAVES) void k_route_select(const float* __restrict__ scores, int n_tokens,
                                                                 int n_experts, int top_k, int32_t* __restrict__ ids,
                                                                 float* __restrict__ weights) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * SEL_WAVES + (threadIdx.x >> 6);
    if (t >= n_tokens) return;   // the whole wave leaves: no workgroup barrier below
    uint32_t ord[NM];
    route_ords<NM>(scores + (int64_t)t * n_experts, n_experts, lane, ord);
    float mine = 0.0f;   // lane r keeps the r-th selected score
    for (int r = 0; r < top_k; ++r) {
        uint32_t best;
        const int win = route_next<NM>(ord, lane, best);
        if (lane == r) mine = ord_score(best);
        if (lane == 0) ids[(int64_t)t * top_k + r] = win;
    }
    const float w = route_weight(mine, top_k, lane);
    if (lane < top_k) weights[(int64_t)t * top_k + lane] = w;
}

template <int SPLIT, int TT>
static void launch_scores(const float* x, int n_tokens, int hidden, const float* w, int n_experts, float* scores,
                          hipStream_t stream) {
    constexpr int EPG = RS_WAVES / SPLIT;
    const dim3 grid((n_experts + EPG - 1) / EPG, (n_tokens + TT - 1) / TT);
    hipLaunchKernelGGL((k_route_scores<SPLIT, TT>), grid, dim3(64 * RS_WAVES), 0, stream, x, n_tokens, hidden, w,
                       n_experts, scores);
}

template <int NM>
static void launch_select(const float* scores, int n_tokens, int n_experts, int top_k, int32_t* ids, float* weights,
                          hipStream_t stream) {
    hipLaunchKernelGGL((k_route_select<NM>), dim3((n_tokens + SEL_WAVES - 1) / SEL_WAVES), dim3(64 * SEL_WAVES), 0,
                       stream, scores, n_tokens, n_experts, top_k, ids, weights);
}

// Few tokens: four waves per expert row, so the n_experts x 4 waves spread
// over the chip, and as many token accumulators as there are tokens (up to 8);
// many tokens: one wave per expert over 16 tokens, so each row is read once
// per 16 tokens.
hipError_t launch_route_scores(const float* x, int n_tokens, int hidden, const float* w, int n_experts, float* scores,
                               hipStream_t stream) {
    if (n_tokens == 1) launch_scores<4, 1>(x, n_tokens, hidden, w, n_experts, scores, stream);
    else if (n_tokens == 2) launch_scores<4, 2>(x, n_tokens, hidden, w, n_experts, scores, stream);
    else if (n_tokens <= 4) launch_scores<4, 4>(x, n_tokens, hidden, w, n_experts, scores, stream);
    else if (n_tokens <= 32) launch_scores<4, 8>(x, n_tokens, hidden, w, n_experts, scores, stream);
    else launch_scores<1, 16>(x, n_tokens, hidden, w, n_experts, scores, stream);
    return hipGetLastError();
}

hipError_t launch_route_select(const float* scores, int n_tokens, int n_experts, int top_k, int32_t* ids,
                               float* weights, hipStream_t stream) {
    const int nm = (n_experts + 63) / 64;
    if (nm <= 1) launch_select<1>(scores, n_tokens, n_experts, top_k, ids, weights, stream);
    else if (nm <= 2) launch_select<2>(scores, n_tokens, n_experts, top_k, ids, weights, stream);
    else if (nm <= 4) launch_select<4>(scores, n_tokens, n_experts, top_k, ids, weights, stream);
    else if (nm <= 8) launch_select<8>(scores, n_tokens, n_experts, top_k, ids, weights, stream);
    else launch_select<16>(scores, n_tokens, n_experts, top_k, ids, weights, stream);
    return hipGetLastError();
}

hipError_t launch_route(const float* x, int n_tokens, int hidden, const float* w, int n_experts, int top_k,
                        float* scores, int32_t* ids, float* weights, hipStream_t stream) {
    const hipError_t e = launch_route_scores(x, n_tokens, hidden, w, n_experts, scores, stream);
    if (e != hipSuccess) return e;
    return launch_route_select(scores, n_tokens, n_experts, top_k, ids, weights, stream);
}

}  // namespace mqh
