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

template <int T, bool F16>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ src, void* __restrict__ dst,
                                                 int64_t n_groups) {
    constexpr int G = block_size(T) / 8;
    constexpr int PB = block_bytes(T);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gi < n_groups; gi += stride) {
        const int64_t b = gi / G;
        const int t = (int)(gi - b * G);
        float v[8];
        decode8<T>(src + b * PB, t, v);
        if constexpr (F16) {
            uint4 o;
            o.x = f2h_rn(v[0]) | (f2h_rn(v[1]) << 16);
            o.y = f2h_rn(v[2]) | (f2h_rn(v[3]) << 16);
            o.z = f2h_rn(v[4]) | (f2h_rn(v[5]) << 16);
            o.w = f2h_rn(v[6]) | (f2h_rn(v[7]) << 16);
            ((uint4*)dst)[gi] = o;
        } else {
            float4* o = (float4*)dst + 2 * gi;
            o[0] = make_float4(v[0], v[1], v[2], v[3]);
            o[1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
}

template <int T>
static hipError_t launch_t(const uint8_t* src, void* dst, int64_t n, int want_f16, hipStream_t stream) {
    const int64_t n_groups = n / 8;
    const int threads = 256;
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
        case T_Q3_K: return launch_t<T_Q3_K>(src, dst, n, want_f16, stream);
        case T_Q4_K: return launch_t<T_Q4_K>(src, dst, n, want_f16, stream);
        case T_Q5_K: return launch_t<T_Q5_K>(src, dst, n, want_f16, stream);
        case T_Q6_K: return launch_t<T_Q6_K>(src, dst, n, want_f16, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mqh
