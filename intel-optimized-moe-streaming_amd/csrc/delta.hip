// delta.hip -- the DeltaNet decode recurrence (moe_delta_heads) on the GPU.
//
// One gated delta-rule step for every value row of every head, the state
// [heads x value_dim x key_dim] FP32 updated in place (cpp/moe_delta.cpp:18-69,
// gated_deltanet.py:264-298):
//   decay = exp(gate[h]) in double;  s_j = (float)((double)s_j * decay)
//   kv = sum_j s_j k_j;  delta = beta[h] (v[h][r] - kv);  s_j = s_j + delta k_j
//   out[h][r] = sum_j s_j q_j
// The reference sums each dot product with eight accumulators (accumulator l
// takes columns j = l mod 8 of the leading multiple of 8, in column order),
// adds the eight into a zero in order, then the remaining key_dim % 8 columns
// one by one, every product and sum rounded on its own.  Here eight lanes own
// one row, lane l holding accumulator l, so each lane's chain is the
// reference's; the eight are gathered with ds_swizzle and summed in the same
// order by every lane of the row, and the remaining columns follow serially.
// Products and sums are separately rounded (contraction off), the decay
// product is taken in double, so the state and outputs are the reference's
// bit for bit whenever exp(gate) in double agrees with the host's libm.
//
// Traffic per step: the state read once and written once (8 * heads *
// value_dim * key_dim bytes); q and k are per head and come from cache.  A
// wavefront covers 8 rows; with key_dim <= 128 a lane keeps its 16 decayed
// values in registers between the two passes, above that it re-reads them.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "moe_decode.h"

namespace mqh {

// value of lane (group * 8 + l) of this lane's group of 8 (ds_swizzle, bit mask
// mode: lane' = (lane & 0x18) | l within each 32-lane half)
template <int L>
__device__ __forceinline__ float group_lane(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (L << 5)));
}

// ((((0 + a0) + a1) + ...) + a7) over the eight accumulators of this lane's
// row, the same value in all eight lanes
__device__ __forceinline__ float sum8_group(float a) {
#pragma clang fp contract(off)
    const float a0 = group_lane<0>(a), a1 = group_lane<1>(a), a2 = group_lane<2>(a), a3 = group_lane<3>(a);
    const float a4 = group_lane<4>(a), a5 = group_lane<5>(a), a6 = group_lane<6>(a), a7 = group_lane<7>(a);
    float s = 0.0f;
    s = s + a0; s = s + a1; s = s + a2; s = s + a3;
    s = s + a4; s = s + a5; s = s + a6; s = s + a7;
    return s;
}

// NB: 8-column groups per row kept in registers (key_dim / 8 <= NB); 0: any
// key_dim, the decayed values written to the state and read back.
template <int NB>
__global__ __launch_bounds__(64) void k_delta_heads(float* __restrict__ state, const float* __restrict__ q,
                                                    const float* __restrict__ k, const float* __restrict__ v,
                                                    const float* __restrict__ beta, const float* __restrict__ gate,
                                                    float* __restrict__ out, int heads, int key_dim, int value_dim,
                                                    unsigned vd_magic, int* __restrict__ flags) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, l = lane & 7;
    const int n_rows = heads * value_dim;
    const int R0 = blockIdx.x * 8 + (lane >> 3);
    const bool live = R0 < n_rows;
    const int R = live ? R0 : n_rows - 1;   // a row past the end computes the last row and stores nothing
    // R / value_dim as one multiply-high (vd_magic = ceil(2^32 / value_dim), 0 for
    // value_dim 1): exact while R * (vd_magic * value_dim - 2^32) < 2^32, which
    // R < 2^18 and value_dim <= 1024 guarantee
    const int h = vd_magic ? (int)__umulhi((unsigned)R, vd_magic) : R;
    float* row = state + (int64_t)R * key_dim;
    const float* kh = k + (int64_t)h * key_dim;
    const float* qh = q + (int64_t)h * key_dim;
    const double decay = exp((double)gate[h]);
    const int nblk = key_dim >> 3, full = nblk << 3, ntail = key_dim - full;
    const int last = key_dim - 1;

    // pass 1: decay, kv
    float s[NB > 0 ? NB : 1];
    float acc = 0.0f;
    if constexpr (NB > 0) {
        float x[NB], kk[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int j = min(8 * i + l, last);   // groups past nblk re-read a valid column and are not used
            x[i] = row[j];
            kk[i] = kh[j];
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            s[i] = (float)((double)x[i] * decay);
            if (i < nblk) acc = acc + s[i] * kk[i];
        }
    } else {
        for (int i = 0; i < nblk; ++i) {
            const int j = 8 * i + l;
            const float d = (float)((double)row[j] * decay);
            if (live) row[j] = d;
            acc = acc + d * kh[j];
        }
    }
    float kv = sum8_group(acc);
    float tv[7];
#pragma unroll
    for (int m = 0; m < 7; ++m) {
        const int j = min(full + m, last);
        tv[m] = (float)((double)row[j] * decay);
        if (m < ntail) kv = kv + tv[m] * kh[j];
    }

    // pass 2: rank-1 write, output
    const float delta = beta[h] * (v[R] - kv);
    float acc2 = 0.0f;
    if constexpr (NB > 0) {
        float kk[NB], qq[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int j = min(8 * i + l, last);
            kk[i] = kh[j];
            qq[i] = qh[j];
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (i < nblk) {
                const float u = s[i] + delta * kk[i];
                if (live) row[8 * i + l] = u;
                acc2 = acc2 + u * qq[i];
            }
        }
    } else {
        for (int i = 0; i < nblk; ++i) {
            const int j = 8 * i + l;
            const float u = row[j] + delta * kh[j];
            if (live) row[j] = u;
            acc2 = acc2 + u * qh[j];
        }
    }
    float result = sum8_group(acc2);
#pragma unroll
    for (int m = 0; m < 7; ++m) {
        if (m < ntail) {
            const int j = full + m;
            const float u = tv[m] + delta * kh[j];
            if (live && l == 0) row[j] = u;
            result = result + u * qh[j];
        }
    }
    if (live && l == 0) {
        out[R] = result;
        if (flags && !isfinite(result)) atomicOr(&flags[FLAG_NONFINITE], 1);
    }
}

template <int NB>
static void launch_delta_nb(float* state, const float* q, const float* k, const float* v, const float* beta,
                            const float* gate, float* out, int heads, int key_dim, int value_dim, int* flags,
                            hipStream_t stream, const KernelEvents& ev) {
    const int64_t n_rows = (int64_t)heads * value_dim;
    const dim3 grid((unsigned)((n_rows + 7) / 8));
    // heads <= 256 and value_dim <= 1024 (the entry points' limits) keep the
    // kernel's multiply-high division exact
    const unsigned vd_magic = value_dim > 1 ? (unsigned)((0x100000000ull + value_dim - 1) / value_dim) : 0u;
    if (ev.armed_a())
        hipExtLaunchKernelGGL((k_delta_heads<NB>), grid, dim3(64), 0, stream, ev.a_start, ev.a_stop, 0, state, q, k,
                              v, beta, gate, out, heads, key_dim, value_dim, vd_magic, flags);
    else
        hipLaunchKernelGGL((k_delta_heads<NB>), grid, dim3(64), 0, stream, state, q, k, v, beta, gate, out, heads,
                           key_dim, value_dim, vd_magic, flags);
}

hipError_t launch_delta_heads(float* state, const float* q, const float* k, const float* v, const float* beta,
                              const float* gate, float* out, int heads, int key_dim, int value_dim, int* flags,
                              hipStream_t stream, const KernelEvents& ev) {
    const int nblk = key_dim / 8;
#define MQH_DELTA(NB) launch_delta_nb<NB>(state, q, k, v, beta, gate, out, heads, key_dim, value_dim, flags, stream, ev)
    if (nblk <= 1) MQH_DELTA(1);
    else if (nblk <= 2) MQH_DELTA(2);
    else if (nblk <= 4) MQH_DELTA(4);
    else if (nblk <= 8) MQH_DELTA(8);
    else if (nblk <= 16) MQH_DELTA(16);
    else MQH_DELTA(0);
#undef MQH_DELTA
    return hipGetLastError();
}

}  // namespace mqh
