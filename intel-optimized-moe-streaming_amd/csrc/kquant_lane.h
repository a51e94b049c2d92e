// kquant_lane.h -- exact integer dot products of GGUF K-quant weights with activations,
// in the per-lane layout of the decode kernels.
//
// Work unit.  A lane owns 32 weights of one 256-weight super-block: lane k (0..7)
// of the block.  Its 32 columns are NR "runs" of RL consecutive columns:
//
//   Q4_K, Q5_K  qs bytes [16k, 16k+16): run 0 = low nibbles,  columns 64g + l0 + [0,16)
//                                       run 1 = high nibbles, columns 64g + 32 + l0 + [0,16)
//               with g = k/2, l0 = 16 (k%2); the runs are sub-blocks 2g and 2g+1.
//   Q6_K        ql bytes [64h + 16j, +16) with h = k/4, j = k%4, s0 = j/2, l0 = 16 (k%2):
//               run r = low (r=0) / high (r=1) nibbles, columns 128h + 32 (s0 + 2r) + l0 + [0,16);
//               the two high bits come from qh bytes [32h + l0, +16), bits 2 (s0 + 2r).
//   Q3_K        qs bytes [32h + l0, +8) with h = k/4, l0 = 8 (k%4): run s (0..3) = bit pair s,
//               columns 128h + 32s + l0 + [0,8); hmask bytes [l0, +8), bit 4h + s.
//
// These are the bit positions of the reference decoders (cpp/dequant_k.cpp: Q4_K :182-206,
// Q5_K :221-240, Q6_K :254-268, Q3_K :278-298), regrouped so that 8 lanes cover one block
// with one 16-byte (Q3_K: 8-byte) quant load each, contiguous across the 8 lanes.
//
// Arithmetic.  Activations are split into three int8 "digits" per value with a
// power-of-two scale per aligned 16-column run (max |x| in [2^(E-1), 2^E), s = 2^(E-6)):
//   X = x/s in (-64, 64), x0 = rint(X), x1 = rint((X-x0)*128), x2 = rint(((X-x0)*128-x1)*128)
//   x = s (x0 + x1/128 + x2/16384) + r,   |r| <= s/32768 = 2^-21 * 2^E
// Every step is exact in FP32, so r is the only error (at most 2^-20 of the run's max |x|).
// A run's dot product with the raw (unsigned) quants is then the exact integer
//   I = 16384 I0 + 128 I1 + I2,  Id = sum_k q_k xd_k   (v_dot4_i32_i8, 4 MACs per instruction)
// scaled by s/16384.  Quant offsets (Q6_K's -32, Q3_K's -4, the -dmin*m of Q4_K/Q5_K) use the
// FP32 column sums of the activation run instead of more dot products.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kquant_device.h"

namespace mqh {

constexpr int NDIG = 3;   // activation digits

__host__ __device__ inline int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
#else
    for (int i = 0; i < 4; ++i) c += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
    return c;
#endif
}

// Scale exponent e of a run whose max |x| is amax: s = 2^e, |x / s| < 64.
__host__ __device__ inline int digit_exp(float amax) {
    if (!(amax > 0.0f)) return 0;
    int E;
    (void)frexpf(amax, &E);   // amax = m * 2^E, m in [0.5, 1)
    return E - 6;
}

__host__ __device__ inline void split_digits(float x, int e, int8_t& d0, int8_t& d1, int8_t& d2) {
    const float X = ldexpf(x, -e);
    const float x0 = rintf(X);
    const float r1 = (X - x0) * 128.0f;
    const float x1 = rintf(r1);
    const float r2 = (r1 - x1) * 128.0f;
    const float x2 = rintf(r2);
    d0 = (int8_t)x0;
    d1 = (int8_t)x1;
    d2 = (int8_t)x2;
}

// Three digits packed in the low 24 bits (d0 | d1 << 8 | d2 << 16).
__host__ __device__ inline uint32_t split_digits_packed(float x, int e) {
    int8_t d0, d1, d2;
    split_digits(x, e, d0, d1, d2);
    return (uint32_t)(uint8_t)d0 | ((uint32_t)(uint8_t)d1 << 8) | ((uint32_t)(uint8_t)d2 << 16);
}

__host__ __device__ inline float f16_bits_to_f32(uint32_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __half2float(__ushort_as_half((unsigned short)h));
#else
    uint32_t sign = (h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = 0;
            while (!(man & 0x400u)) { man <<= 1; ++e; }
            bits = sign | ((uint32_t)(113 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    __builtin_memcpy(&f, &bits, 4);
    return f;
#endif
}

// ------------------------------------------------------------------ geometry

template <int T> struct LaneGeo;
template <> struct LaneGeo<T_Q4_K> { static constexpr int NR = 2, RL = 16, NRAW = 8; };
template <> struct LaneGeo<T_Q5_K> { static constexpr int NR = 2, RL = 16, NRAW = 12; };
template <> struct LaneGeo<T_Q6_K> { static constexpr int NR = 2, RL = 16, NRAW = 11; };
template <> struct LaneGeo<T_Q3_K> { static constexpr int NR = 4, RL = 8, NRAW = 8; };

// First column (within the super-block) of run r of lane k.
template <int T>
__host__ __device__ inline int lane_col(int k, int r) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) return 64 * (k >> 1) + 32 * r + 16 * (k & 1);
    else if constexpr (T == T_Q6_K) return 128 * (k >> 2) + 32 * (((k & 3) >> 1) + 2 * r) + 16 * (k & 1);
    else return 128 * (k >> 2) + 32 * r + 8 * (k & 3);
}

// Activation operand of one lane: digits of its 32 columns in run order
// (run r at dwords [r*RL/4, (r+1)*RL/4)), per-run scale s/16384 and FP32 sum.
struct LaneX {
    uint32_t d[NDIG][8];
    float xs[4];
    float sum[4];
};

// Digit view of an activation vector of n values: planes int8 [3][n] (column
// order), xs16 [n/16] = 2^e/16384 per 16-column run, sum8 [n/8] = FP32 sums of
// 8 consecutive values.
struct DigitsRef {
    const int8_t* planes;
    const float* xs16;
    const float* sum8;
    int n;
};

template <int T>
__host__ __device__ inline void lane_x(const DigitsRef& v, int blk, int k, LaneX& x) {
    constexpr int NR = LaneGeo<T>::NR, RL = LaneGeo<T>::RL;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int c = 256 * blk + lane_col<T>(k, r);
#pragma unroll
        for (int d = 0; d < NDIG; ++d) {
            const int8_t* src = v.planes + (int64_t)d * v.n + c;
            if constexpr (RL == 16) {
                const uint4 q = *(const uint4*)src;
                x.d[d][4 * r + 0] = q.x; x.d[d][4 * r + 1] = q.y;
                x.d[d][4 * r + 2] = q.z; x.d[d][4 * r + 3] = q.w;
            } else {
                const uint2 q = *(const uint2*)src;
                x.d[d][2 * r + 0] = q.x; x.d[d][2 * r + 1] = q.y;
            }
        }
        x.xs[r] = v.xs16[c >> 4];
        x.sum[r] = RL == 16 ? v.sum8[c >> 3] + v.sum8[(c >> 3) + 1] : v.sum8[c >> 3];
    }
}

// Exact integer dot of run r (RL/4 quant dwords q) with the three digit planes.
template <int RL>
__host__ __device__ inline float run_dot(const uint32_t* q, const LaneX& x, int r) {
    int32_t i0 = 0, i1 = 0, i2 = 0;
#pragma unroll
    for (int i = 0; i < RL / 4; ++i) {
        i0 = sdot4(q[i], x.d[0][r * (RL / 4) + i], i0);
        i1 = sdot4(q[i], x.d[1][r * (RL / 4) + i], i1);
        i2 = sdot4(q[i], x.d[2][r * (RL / 4) + i], i2);
    }
    // |i0| <= 16 * 63 * 64, so 16384 * i0 + 128 * i1 + i2 fits in int32
    return x.xs[r] * (float)((i0 << 14) + (i1 << 7) + i2);
}

// ------------------------------------------------------------------- loads

__host__ __device__ inline void put4(uint32_t* w, const uint8_t* p) { __builtin_memcpy(w, p, 16); }
__host__ __device__ inline void put2(uint32_t* w, const uint8_t* p) { __builtin_memcpy(w, p, 8); }

// Raw bytes lane k needs from the block at blk, into raw[0 .. NRAW).
template <int T>
__host__ __device__ inline void lane_load(const uint8_t* blk, int k, uint32_t* raw) {
    if constexpr (T == T_Q4_K) {
        put4(raw, blk);                         // d, dmin, scales
        put4(raw + 4, blk + 16 + 16 * k);       // qs
    } else if constexpr (T == T_Q5_K) {
        put4(raw, blk);
        put4(raw + 4, blk + 16 + 16 * (k & 1)); // qh
        put4(raw + 8, blk + 48 + 16 * k);       // qs
    } else if constexpr (T == T_Q6_K) {
        const int h = k >> 2;
        put4(raw, blk + 64 * h + 16 * (k & 3));         // ql
        put4(raw + 4, blk + 128 + 32 * h + 16 * (k & 1)); // qh
        put2(raw + 8, blk + 192 + 8 * h);                // int8 scales 8h .. 8h+7
        uint16_t d;
        __builtin_memcpy(&d, blk + 208, 2);
        raw[10] = d;
    } else {  // Q3_K
        const int h = k >> 2, l0 = 8 * (k & 3);
        put2(raw, blk + l0);                    // hmask
        put2(raw + 2, blk + 32 + 32 * h + l0);  // qs
        __builtin_memcpy(raw + 4, blk + 96, 12);  // scales
        uint16_t d;
        __builtin_memcpy(&d, blk + 108, 2);
        raw[7] = d;
    }
}

// ------------------------------------------------------------------ scales

// Q4_K/Q5_K 6-bit scale and min j (0..7) from header dwords 1..3.  j is
// lane-dependent, so bytes are selected with shifts (indexing a register
// array with it would move the array to scratch memory).
__host__ __device__ inline void k4_scale_min(const uint32_t* hdr, int j, int& sc, int& mn) {
    const uint64_t lo = (uint64_t)hdr[1] | ((uint64_t)hdr[2] << 32);   // bytes 0..7
    const uint32_t hi = hdr[3];                                        // bytes 8..11
    if (j < 4) {
        sc = (int)((lo >> (8 * j)) & 63);
        mn = (int)((lo >> (8 * j + 32)) & 63);
    } else {
        const int k = j - 4;
        const uint32_t b8 = (hi >> (8 * k)) & 0xFFu;
        sc = (int)((b8 & 15) | ((((lo >> (8 * k)) >> 6) & 3) << 4));
        mn = (int)((b8 >> 4) | ((((lo >> (8 * j)) >> 6) & 3) << 4));
    }
}

// Q3_K signed 6-bit scale j (0..15) from the 12 scale bytes.
__host__ __device__ inline int k3_scale(const uint32_t* sc, int j) {
    const uint64_t lo64 = (uint64_t)sc[0] | ((uint64_t)sc[1] << 32);
    const int lo = (int)((lo64 >> (8 * (j & 7) + 4 * (j >> 3))) & 15);
    const int hi = (int)((sc[2] >> (8 * (j & 3) + 2 * (j >> 2))) & 3);
    return (lo | (hi << 4)) - 32;
}

// ---------------------------------------------------------------- lane dots

// Dot product of lane k's 32 weights (raw bytes from lane_load) with x.
template <int T>
__host__ __device__ inline float lane_dot(const uint32_t* raw, int k, const LaneX& x) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        constexpr int QS = T == T_Q4_K ? 4 : 8;
        const float d = f16_bits_to_f32(raw[0] & 0xFFFFu), dmin = f16_bits_to_f32(raw[0] >> 16);
        const int g = k >> 1;
        float acc = 0.0f, off = 0.0f;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int j = 2 * g + r;
            int sc, mn;
            k4_scale_min(raw, j, sc, mn);
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                q[i] = (raw[QS + i] >> (4 * r)) & 0x0F0F0F0Fu;
                if constexpr (T == T_Q5_K) q[i] |= ((raw[4 + i] >> j) & 0x01010101u) << 4;
            }
            acc = fmaf((float)sc, run_dot<16>(q, x, r), acc);
            off = fmaf((float)mn, x.sum[r], off);
        }
        return fmaf(d, acc, -dmin * off);
    } else if constexpr (T == T_Q6_K) {
        const float d = f16_bits_to_f32(raw[10] & 0xFFFFu);
        const int s0 = (k & 3) >> 1, odd = k & 1;
        const uint64_t sc64 = (uint64_t)raw[8] | ((uint64_t)raw[9] << 32);
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int s = s0 + 2 * r;
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q[i] = ((raw[i] >> (4 * r)) & 0x0F0F0F0Fu) | (((raw[4 + i] >> (2 * s)) & 0x03030303u) << 4);
            const int sc = (int)(int8_t)(uint8_t)(sc64 >> (8 * (2 * s + odd)));
            acc = fmaf((float)sc, fmaf(-32.0f, x.sum[r], run_dot<16>(q, x, r)), acc);
        }
        return d * acc;
    } else {  // Q3_K
        const float d = f16_bits_to_f32(raw[7] & 0xFFFFu);
        const int h = k >> 2, half16 = (k & 3) >> 1;
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint32_t q[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                q[i] = ((raw[2 + i] >> (2 * s)) & 0x03030303u) | (((raw[i] >> (4 * h + s)) & 0x01010101u) << 2);
            const int sc = k3_scale(raw + 4, 8 * h + 2 * s + half16);
            acc = fmaf((float)sc, fmaf(-4.0f, x.sum[s], run_dot<8>(q, x, s)), acc);
        }
        return d * acc;
    }
}

}  // namespace mqh
