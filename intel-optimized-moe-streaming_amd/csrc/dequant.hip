// dequant.hip -- standalone GGUF block dequantization to FP32 or FP16.
//
// Replaces the CPU routine dequant_k (cpp/dequant_k.cpp:350-394) for weights
// that live in HBM.  The work is HBM-bound: every 8 output values cost
// bytes_per_block/32 (Q4_K: 4.5 B) of input plus 16 B (FP16) or 32 B (FP32)
// of output.
//
// Mapping: one thread produces 8 consecutive outputs, so a wavefront writes
// 64 x 16 B = 1 KiB of FP16 contiguously (one global_store_dwordx4 per lane).
// The 8 outputs are values 8t..8t+7 of one block; their quant bytes are one
// 8-byte load, the block header a few bytes that the wavefront shares in L1.
// FP16 outputs are RN_f16 of the FP32 decode, as the reference's F16C
// conversion produces them (dequant_k.cpp:124-136).
#include "kquant_device.h"

namespace mqh {

// threads per workgroup, a compile-time constant: blockDim.x would cost every
// workgroup a memory round trip before its first address is known
constexpr int DQ_THREADS = 256;

template <int T, bool F16>
__global__ __launch_bounds__(DQ_THREADS) void k_dequant(const uint8_t* __restrict__ src, void* __restrict__ dst,
                                                 int64_t n_groups) {
    constexpr int G = block_size(T) / 8;
    constexpr int PB = block_bytes(T);
    const int64_t stride = (int64_t)gridDim.x * DQ_THREADS;
    // two groups per pass, stride apart, both decoded before either is stored,
    // so each thread has two groups' loads in flight
    for (int64_t g0 = (int64_t)blockIdx.x * DQ_THREADS + threadIdx.x; g0 < n_groups; g0 += 2 * stride) {
        float v[2][8];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            // a second group past the end decodes the last group again (in
            // bounds, not stored), so both loads issue without a branch
            const int64_t gi = min(g0 + u * stride, n_groups - 1);
            const int64_t b = gi / G;
            decode8<T>(src + b * PB, (int)(gi - b * G), v[u]);
        }
        // pin both groups' values here: otherwise the second decode (and its
        // loads) sinks into the conditional store below, behind the first store
#pragma unroll
        for (int k = 0; k < 8; ++k) v[1][k] = opaque(v[1][k]);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t gi = g0 + u * stride;
            if (gi >= n_groups) break;
            if constexpr (F16) {
                uint4 o;
                o.x = f2h_rn(v[u][0]) | (f2h_rn(v[u][1]) << 16);
                o.y = f2h_rn(v[u][2]) | (f2h_rn(v[u][3]) << 16);
                o.z = f2h_rn(v[u][4]) | (f2h_rn(v[u][5]) << 16);
                o.w = f2h_rn(v[u][6]) | (f2h_rn(v[u][7]) << 16);
                ((uint4*)dst)[gi] = o;
            } else {
                float4* o = (float4*)dst + 2 * gi;
                o[0] = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
                o[1] = make_float4(v[u][4], v[u][5], v[u][6], v[u][7]);
            }
        }
    }
}

template <int T>
static hipError_t launch_t(const uint8_t* src, void* dst, int64_t n, int want_f16, hipStream_t stream) {
    const int64_t n_groups = n / 8;
    const int threads = DQ_THREADS;
    int64_t blocks = (n_groups + threads - 1) / threads;
    if (blocks > 65536) blocks = 65536;
    if (want_f16)
        hipLaunchKernelGGL((k_dequant<T, true>), dim3((unsigned)blocks), dim3(threads), 0, stream, src, dst, n_groups);
    else
        hipLaunchKernelGGL((k_dequant<T, false>), dim3((unsigned)blocks), dim3(threads), 0, stream, src, dst, n_groups);
    return hipGetLastError();
}

// Launch the dequantizer.  n must be a positive multiple of the block size;
// src, dst are device pointers, dst 16-byte aligned.
hipError_t launch_dequant(int type, const uint8_t* src, void* dst, int64_t n, int want_f16, hipStream_t stream) {
    switch (type) {
        case T_Q8_0: return launch_t<T_Q8_0>(src, dst, n, want_f16, stream);
        case T_IQ4_NL: return launch_t<T_IQ4_NL>(src, dst, n, want_f16, stream);
        case T_Q3_K: return launch_t<T_Q3_K>(src, dst, n, want_f16, stream);
        case T_Q4_K: return launch_t<T_Q4_K>(src, dst, n, want_f16, stream);
        case T_Q5_K: return launch_t<T_Q5_K>(src, dst, n, want_f16, stream);
        case T_Q6_K: return launch_t<T_Q6_K>(src, dst, n, want_f16, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mqh
