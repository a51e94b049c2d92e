// route_topk.h -- one wavefront's top-k of a token's router scores and the
// softmax of the selected scores (ExpertRouter.route, src/flash_moe/router.py:
// 140-170), shared by the router's select kernel and the routed decode
// prologue.
//
// Each lane holds NM scores (experts lane, lane+64, ...) as orderable 32-bit
// values.  A round takes their wavefront maximum over DPP row operations and
// then the lowest expert holding it (ballots), so at equal scores the lower
// expert wins.  Every NaN ranks above every number (np.argsort places NaN
// last, so the reference selects NaN scores first); -0.0 and +0.0 are equal.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mqh {

// Orderable form of a score: a larger value ranks first, every NaN above
// +inf, -0.0 equal to +0.0.  Never 0, which marks an expert already selected
// or past n_experts.
__device__ __forceinline__ uint32_t route_ord(float s) {
    uint32_t u = __float_as_uint(s);
    if (s != s) return 0xFFFFFFFFu;
    if (u == 0x80000000u) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float ord_score(uint32_t ord) {
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
}

// One step of the wavefront maximum inside each row of 16 lanes: the DPP move
// and the maximum stay two instructions (the empty asm keeps the compiler from
// folding them into one DPP maximum).  The patterns used write every lane (row
// and bank masks full, every source lane inside the row), so the move carries
// no old value and needs no copy ahead of it.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max_full(uint32_t v) {
    int o = __builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
    __asm__ volatile("" : "+v"(o));
    return (uint32_t)o > v ? (uint32_t)o : v;
}

// Maximum over the wavefront, returned uniform: each row's maximum by four DPP
// steps, then the four rows' (lanes 15, 31, 47, 63) in scalar registers (two
// more DPP steps across rows and one read of lane 63 took longer: the routed
// decode 13.99 -> 13.77 us per layer).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = dpp_max_full<0xB1>(v);    // quad_perm [1,0,3,2]
    v = dpp_max_full<0x4E>(v);    // quad_perm [2,3,0,1]
    v = dpp_max_full<0x141>(v);   // row_half_mirror
    v = dpp_max_full<0x140>(v);   // row_mirror: every lane holds its row's maximum
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
    const uint32_t a = r0 > r1 ? r0 : r1, b = r2 > r3 ? r2 : r3;
    return a > b ? a : b;
}

// The ords of one token's n_experts scores (st), NM per lane (expert
// lane + 64 m); every load is issued before any is used (indexes past
// n_experts re-read the last score and get 0).
template <int NM>
__device__ __forceinline__ void route_ords(const float* st, int n_experts, int lane, uint32_t (&ord)[NM]) {
    float sv[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) sv[m] = st[min(lane + 64 * m, n_experts - 1)];
#pragma unroll
    for (int m = 0; m < NM; ++m) ord[m] = lane + 64 * m < n_experts ? route_ord(sv[m]) : 0u;
}

// One round: the best remaining score (its ord, uniform, in `best`) and its
// expert, the lowest index among equal scores (a ballot per m, smallest m
// first, lowest lane first), removed from the lanes' ords.
template <int NM>
__device__ __forceinline__ int route_next(uint32_t (&ord)[NM], int lane, uint32_t& best) {
    uint32_t b = ord[0];
#pragma unroll
    for (int m = 1; m < NM; ++m) b = ord[m] > b ? ord[m] : b;
    best = wave_max_u32(b);
    int win = 0;
#pragma unroll
    for (int m = NM - 1; m >= 0; --m) {
        const uint64_t hit = __ballot(ord[m] == best);
        if (hit != 0) win = 64 * m + (int)__builtin_ctzll(hit);
    }
#pragma unroll
    for (int m = 0; m < NM; ++m)
        if (lane + 64 * m == win) ord[m] = 0u;
    return win;
}

// The FP32 routing weight of this lane's rank, lanes 0..top_k-1 holding the
// selected scores in rank order (`mine`): exp(s_r - max) / sum in float64,
// summed in rank order; 1/top_k each when the sum is not finite and positive
// (router.py:157-168).  Called by the whole wavefront.
__device__ __forceinline__ float route_weight(float mine, int top_k, int lane) {
    double mx = -__builtin_huge_val();
    for (int r = 0; r < top_k; ++r)
        mx = fmax(mx, (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), r)));
    const double ex = lane < top_k ? exp((double)mine - mx) : 0.0;
    const uint64_t exb = (uint64_t)__double_as_longlong(ex);
    double total = 0.0;
    for (int r = 0; r < top_k; ++r) {
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)exb, r);
        const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(exb >> 32), r);
        total += __longlong_as_double((int64_t)(((uint64_t)hi << 32) | lo));
    }
    const bool uniform = !(total > 0.0) || !isfinite(total);
    return uniform ? (float)(1.0 / top_k) : (float)(ex / total);
}

}  // namespace mqh
