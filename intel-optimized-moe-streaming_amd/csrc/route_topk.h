// route_topk.h -- one wavefront's top-k of a token's router scores and the
// softmax of the selected scores (ExpertRouter.route, src/flash_moe/router.py:
// 140-170), shared by the router's select kernel and the routed decode
// prologue.
//
// Each lane holds NM scores (experts lane, lane+64, ...) as 64-bit keys: the
// score's orderable bits above, the complemented expert index below, so a
// larger key ranks first and, at equal scores, the lower expert wins.  Every
// NaN ranks above every number (np.argsort places NaN last, so the reference
// selects NaN scores first); -0.0 and +0.0 are equal.  A round takes the
// wavefront maximum over DPP row operations and removes it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mqh {

// Orderable key of (score, expert): a larger key ranks first.  Never 0.
__device__ __forceinline__ uint64_t route_key(float s, int e) {
    uint32_t u = __float_as_uint(s);
    uint32_t ord;
    if (s != s) {
        ord = 0xFFFFFFFFu;                            // every NaN above +inf
    } else {
        if (u == 0x80000000u) u = 0;                  // -0.0 == +0.0
        ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    return ((uint64_t)ord << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}

__device__ __forceinline__ float key_score(uint64_t k) {
    const uint32_t ord = (uint32_t)(k >> 32);
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
}

__device__ __forceinline__ int key_expert(uint64_t k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_step(uint64_t v) {
    const int vlo = (int)(uint32_t)v, vhi = (int)(uint32_t)(v >> 32);
    const int lo = __builtin_amdgcn_update_dpp(vlo, vlo, CTRL, ROW_MASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(vhi, vhi, CTRL, ROW_MASK, 0xF, false);
    const uint64_t o = ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
    return o > v ? o : v;
}

// Maximum over the wavefront, returned uniform.  Lanes outside a step's row
// mask keep their own value.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = dpp_max_step<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v = dpp_max_step<0x141, 0xF>(v);   // row_half_mirror
    v = dpp_max_step<0x140, 0xF>(v);   // row_mirror: every lane holds its row's maximum
    v = dpp_max_step<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v = dpp_max_step<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3: lane 63 holds the maximum
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

// The keys of one token's n_experts scores (st), NM per lane; every load is
// issued before any is used (indexes past n_experts re-read the last score
// and get key 0).
template <int NM>
__device__ __forceinline__ void route_keys(const float* st, int n_experts, int lane, uint64_t (&key)[NM]) {
    float sv[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) sv[m] = st[min(lane + 64 * m, n_experts - 1)];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const int e = lane + 64 * m;
        key[m] = e < n_experts ? route_key(sv[m], e) : 0;
    }
}

// One round: the best remaining key (uniform), removed from the lanes' keys.
template <int NM>
__device__ __forceinline__ uint64_t route_next(uint64_t (&key)[NM]) {
    uint64_t b = key[0];
#pragma unroll
    for (int m = 1; m < NM; ++m) b = key[m] > b ? key[m] : b;
    const uint64_t win = wave_max_u64(b);
#pragma unroll
    for (int m = 0; m < NM; ++m)
        if (key[m] == win) key[m] = 0;
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
