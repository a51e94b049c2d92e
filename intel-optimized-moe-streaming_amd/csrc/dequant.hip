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

// LDS-staged form.  A workgroup owns one chunk of DQ_CHUNK_VALUES consecutive
// values (16 K-quant blocks, or 128 blocks of the 32-value types), staged in
// LDS one block per slot (slot_bytes/slot_offset: the 16-byte fields land on
// 16-byte boundaries).  Every thread then decodes two adjacent 8-value groups
// of one block -- the two share the block header and, for the K-quants, the
// sub-block scale -- and the wave stores its 1,024 values with coalesced
// 16-byte pieces.  (Two or more chunks per workgroup, all their loads in
// flight together, measured no faster.)
constexpr int DQ_CHUNK_VALUES = DQ_THREADS * 16;

// Copy NBK consecutive blocks into their LDS slots with aligned, coalesced
// 16-byte loads (all issued before the first write).  Where slot and block
// coincide (Q4_K, Q5_K: 144 and 176 bytes) the words go to LDS as they are;
// otherwise each 16-byte word (which spans at most two blocks: every block is
// longer than 16 bytes) is written as 2-byte pieces, each at its block's slot
// -- naturally aligned LDS writes, where 16-byte writes at 2 mod 4 addresses
// would stall.
template <int T, int NBK>
__device__ __forceinline__ void stage_blocks(const uint8_t* __restrict__ src, uint8_t* lds) {
    constexpr int PB = block_bytes(T), SL = slot_bytes(T), OFF = slot_offset(T);
    constexpr int NW = NBK * PB / 16, IT = (NW + DQ_THREADS - 1) / DQ_THREADS;
    static_assert(PB > 16, "a 16-byte word meets at most two blocks");
    uint4 w[IT];
#pragma unroll
    for (int k = 0; k < IT; ++k) {
        const int i = threadIdx.x + k * DQ_THREADS;
        if (NW % DQ_THREADS == 0 || i < NW) w[k] = ((const uint4*)src)[i];
    }
#pragma unroll
    for (int k = 0; k < IT; ++k) {
        const int i = threadIdx.x + k * DQ_THREADS;
        if (NW % DQ_THREADS != 0 && i >= NW) break;
        if constexpr (SL == PB && OFF == 0) {
            ((uint4*)lds)[i] = w[k];
        } else {
            // pieces m < mb belong to block b0, the rest to block b0 + 1
            const int x = 16 * i, b0 = x / PB, mb = ((b0 + 1) * PB - x) / 2;
            uint16_t* at0 = (uint16_t*)(lds + x + b0 * (SL - PB) + OFF);
            uint16_t* at1 = at0 + (SL - PB) / 2;
            const uint32_t q[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
            for (int m = 0; m < 8; ++m) (m < mb ? at0 : at1)[m] = (uint16_t)(q[m >> 1] >> (16 * (m & 1)));
        }
    }
}

// A wave's 64 x 16 decoded values (lane l: values 16l .. 16l+15 of the wave's
// run) to dst, through the wave's LDS exchange area xw, so that every store
// instruction writes 64 consecutive 16-byte pieces (lane l piece l): stores of
// 32 contiguous bytes per lane, half-filled lines per instruction, ran 3-13 %
// slower on the full-size workload.  LDS operations of one wave complete in
// order; the wave fences only keep the compiler from moving them.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <bool F16>
__device__ __forceinline__ void store16_wave(const float v[16], uint4* xw, uint4* dst_wave, int lane) {
    constexpr int P = F16 ? 2 : 4;   // 16-byte pieces per lane
    uint4 o[P];
    if constexpr (F16) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            o[h].x = pack_f2h_rn(v[8 * h + 0], v[8 * h + 1]);
            o[h].y = pack_f2h_rn(v[8 * h + 2], v[8 * h + 3]);
            o[h].z = pack_f2h_rn(v[8 * h + 4], v[8 * h + 5]);
            o[h].w = pack_f2h_rn(v[8 * h + 6], v[8 * h + 7]);
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = make_uint4(__float_as_uint(v[4 * q]), __float_as_uint(v[4 * q + 1]), __float_as_uint(v[4 * q + 2]),
                              __float_as_uint(v[4 * q + 3]));
    }
#pragma unroll
    for (int k = 0; k < P; ++k) xw[P * lane + k] = o[k];
    wave_lds_sync();
#pragma unroll
    for (int k = 0; k < P; ++k) o[k] = xw[64 * k + lane];
#pragma unroll
    for (int k = 0; k < P; ++k) dst_wave[64 * k + lane] = o[k];
    wave_lds_sync();   // the next call's writes follow this call's reads
}

template <int T, bool F16>
__global__ __launch_bounds__(DQ_THREADS) void k_dequant_lds(const uint8_t* __restrict__ src, void* __restrict__ dst) {
    constexpr int PB = block_bytes(T), G = block_size(T) / 8, SL = slot_bytes(T);
    constexpr int NB = DQ_CHUNK_VALUES / block_size(T);
    static_assert(SL % 16 == 0 && G % 2 == 0 && PB % 2 == 0, "16-byte slots, group pairs in one block");
    __shared__ __attribute__((aligned(16))) uint8_t buf[NB * SL];
    const int64_t chunk = blockIdx.x;
    stage_blocks<T, NB>(src + chunk * (NB * PB), buf);
    __syncthreads();
    __shared__ uint4 xch[DQ_THREADS / 64][F16 ? 128 : 256];
    const int b = 2 * threadIdx.x / G, t = 2 * threadIdx.x - b * G;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    float v[16];
    decode16<T>(buf + b * SL + slot_offset(T), t, v);
    // the wave's 1,024 values start at value chunk * 4096 + 1024 wv
    store16_wave<F16>(v, xch[wv], (uint4*)dst + (chunk * DQ_CHUNK_VALUES + 1024 * wv) / (F16 ? 8 : 4), lane);
}

template <int T>
static hipError_t launch_t(const uint8_t* src, void* dst, int64_t n, int want_f16, hipStream_t stream) {
    // whole chunks from a 16-byte aligned source go through LDS; the rest (a
    // tail of fewer than DQ_CHUNK_VALUES values, or an unaligned source)
    // through the per-thread kernel
    const int64_t n_chunks = ((uintptr_t)src & 15) ? 0 : n / DQ_CHUNK_VALUES;
    if (n_chunks > 0) {
        if (want_f16)
            hipLaunchKernelGGL((k_dequant_lds<T, true>), dim3((unsigned)n_chunks), dim3(DQ_THREADS), 0, stream, src, dst);
        else
            hipLaunchKernelGGL((k_dequant_lds<T, false>), dim3((unsigned)n_chunks), dim3(DQ_THREADS), 0, stream, src,
                               dst);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t done = n_chunks * DQ_CHUNK_VALUES;
        if (done == n) return hipSuccess;
        src += done / block_size(T) * block_bytes(T);
        dst = (uint8_t*)dst + done * (want_f16 ? 2 : 4);
        n -= done;
    }
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
