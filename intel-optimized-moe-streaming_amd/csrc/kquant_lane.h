// kquant_lane.h -- exact-integer dot products of GGUF K-quant weights with activations,
// in the per-lane layout of the decode kernels.
//
// Work unit.  A lane owns 64 weights of one 256-weight super-block: lane k (0..3)
// of the block.  Its 64 columns are runs of consecutive columns:
//
//   Q4_K, Q5_K  qs bytes [32k, 32k+32): run 0 = low nibbles  = columns 64k + [0,32)  (sub-block 2k)
//                                       run 1 = high nibbles = columns 64k + 32 + [0,32) (sub-block 2k+1)
//               Q5_K adds bit 2k+r of qh bytes [0, 32) as bit 4.
//   Q6_K        ql bytes [64h + 32j, +32) with h = k/2, j = k%2: run r = low (r=0) / high (r=1) nibbles,
//               columns 128h + 32 (j + 2r) + [0,32); the two high bits come from qh bytes [32h, +32),
//               bits 2 (j + 2r); int8 scales per 16 columns.
//   Q3_K        qs bytes [32h + l0, +16) with h = k/2, l0 = 16 (k%2): run s (0..3) = bit pair s,
//               columns 128h + 32s + l0 + [0,16); hmask bytes [l0, +16), bit 4h + s.
//   Q8_0        a 256-column unit is 8 consecutive 34-byte blocks (272 bytes); lane k owns blocks
//               2k and 2k+1 (bytes [68k, 68k+68)): run r = block 2k + r, columns 64k + 32r + [0,32),
//               its FP16 scale then 32 int8 quants.
//
// These are the bit positions of the reference decoders (cpp/dequant_k.cpp: Q8_0 :146-154,
// Q4_K :182-206, Q5_K :221-240, Q6_K :254-268, Q3_K :278-298), regrouped so that 4 lanes cover
// one block with contiguous 32-byte (Q3_K: 16-byte) quant loads.
//
// Arithmetic.  Activations are split into two int8 "digits" per value with one scale per
// aligned 16-column run:  s = max|x| / 127 over the run, X = x/s in [-127, 127],
//   x0 = rint(X),  x1 = rint((X - x0) * 254)  (both in [-127, 127]),
//   x = (s/254) * (254 x0 + x1) + r,   |r| <= s/508 (+ FP32 rounding) < 1.6e-5 * max|x|.
// A run's dot product with the raw quants (unsigned; Q8_0's are signed) is then the exact integer
//   I = 254 I0 + I1,  Id = sum_k q_k xd_k   (v_dot4_i32_i8, 4 MACs per instruction; |I| < 2^31)
// times the run scale s/254.  Quant offsets (Q6_K's -32, Q3_K's -4, the -dmin*m of Q4_K/Q5_K)
// use the FP32 column sums of 16-column pieces instead of more dot products.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kquant_device.h"

namespace mqh {

__host__ __device__ inline int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
#else
    for (int i = 0; i < 4; ++i) c += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
    return c;
#endif
}

// sdot4(a, b, 0).  On the device the three-operand form with an inline zero
// accumulator: the compiler selects the two-operand v_dot4c for the builtin,
// whose accumulator must first be zeroed by a v_mov of its own.
__host__ __device__ inline int32_t sdot4_0(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
    int32_t r;
    __asm__("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
#else
    return sdot4(a, b, 0);
#endif
}

// Reciprocal scale 127 / amax of a run (0 for an all-zero run); the run scale
// stored beside the digits is amax / (127 * 254).  The device uses the hardware
// reciprocal (1 ulp): a scale off by 1e-7 changes the reconstruction by 1e-7 of
// the value, far inside the digit error.
__host__ __device__ inline float digit_inv(float amax) {
#if defined(__HIP_DEVICE_COMPILE__)
    return amax > 0.0f ? 127.0f * __builtin_amdgcn_rcpf(amax) : 0.0f;
#else
    return amax > 0.0f ? 127.0f / amax : 0.0f;
#endif
}
__host__ __device__ inline float digit_scale(float amax) { return amax * (1.0f / (127.0f * 254.0f)); }

// Two digits of x (d0 | d1 << 8) for the run's reciprocal scale inv.
__host__ __device__ inline uint32_t split2(float x, float inv) {
    const float X = x * inv;
    const float x0 = rintf(X);
    const float x1 = rintf((X - x0) * 254.0f);
    return (uint32_t)(uint8_t)(int8_t)(int)x0 | ((uint32_t)(uint8_t)(int8_t)(int)x1 << 8);
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

constexpr int LANES_PER_BLOCK = 4;

// A block's scale word, read where a dot product needs it: on the device the
// word passes through an empty asm statement, so the compiler cannot move its
// conversion up to the load (with a wait for the load at that point).  Used
// for Q3_K, where that happened; for the other types the plain read measured
// the same or faster.
__host__ __device__ inline uint32_t scale_word(const uint32_t* raw, int i) {
    uint32_t w = raw[i];
#if defined(__HIP_DEVICE_COMPILE__)
    __asm__ volatile("" : "+v"(w));
#endif
    return w;
}

// NR runs of RL columns per lane; NRAW dwords of raw block bytes per lane.
template <int T> struct LaneGeo;
template <> struct LaneGeo<T_Q4_K> { static constexpr int NR = 2, RL = 32, NRAW = 12; };
template <> struct LaneGeo<T_Q5_K> { static constexpr int NR = 2, RL = 32, NRAW = 20; };
template <> struct LaneGeo<T_Q6_K> { static constexpr int NR = 2, RL = 32, NRAW = 19; };
template <> struct LaneGeo<T_Q3_K> { static constexpr int NR = 4, RL = 16, NRAW = 12; };
// Q3_K in 112-byte slots: the same lane code (the final branches of the type
// switches below), a block every 112 bytes
template <> struct LaneGeo<T_Q3_K_A112> : LaneGeo<T_Q3_K> {};
template <> struct LaneGeo<T_Q8_0> { static constexpr int NR = 2, RL = 32, NRAW = 17; };

// Bytes of one 256-column unit of a row: a K-quant super-block, or 8 Q8_0 blocks.
__host__ __device__ constexpr int unit_bytes(int t) { return t == T_Q8_0 ? 8 * 34 : block_bytes(t); }

// First column (within the super-block) of run r of lane k.
template <int T>
__host__ __device__ inline int lane_col(int k, int r) {
    if constexpr (T == T_Q4_K || T == T_Q5_K || T == T_Q8_0) return 64 * k + 32 * r;
    else if constexpr (T == T_Q6_K) return 128 * (k >> 1) + 32 * ((k & 1) + 2 * r);
    else return 128 * (k >> 1) + 32 * r + 16 * (k & 1);
}

// Activation operand of one lane: the two digit planes of its 64 columns in run
// order (16-column piece p at dwords [4p, 4p+4)), and per 16-column piece the
// run scale (s/254) and the FP32 sum of the activations.
struct LaneX {
    uint32_t d0[16], d1[16];
    float xs[4], sum[4];
};

// Digit view of an activation vector of n values: planes int8 [2][n] (column
// order), xs16 [n/16] run scales, sum16 [n/16] run sums.
struct DigitsRef {
    const int8_t* planes;
    const float* xs16;
    const float* sum16;
    int n;
};

template <int T>
__host__ __device__ inline void lane_x(const DigitsRef& v, int blk, int k, LaneX& x) {
    constexpr int NR = LaneGeo<T>::NR, RL = LaneGeo<T>::RL;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int c = 256 * blk + lane_col<T>(k, r);
#pragma unroll
        for (int p = 0; p < RL / 16; ++p) {
            const int piece = r * (RL / 16) + p, cc = c + 16 * p;
            const uint4 a = *(const uint4*)(v.planes + cc);
            const uint4 b = *(const uint4*)(v.planes + v.n + cc);
            x.d0[4 * piece + 0] = a.x; x.d0[4 * piece + 1] = a.y; x.d0[4 * piece + 2] = a.z; x.d0[4 * piece + 3] = a.w;
            x.d1[4 * piece + 0] = b.x; x.d1[4 * piece + 1] = b.y; x.d1[4 * piece + 2] = b.z; x.d1[4 * piece + 3] = b.w;
            x.xs[piece] = v.xs16[cc >> 4];
            x.sum[piece] = v.sum16[cc >> 4];
        }
    }
}

// Exact integer dot of 16-column piece p (quant dwords q[0..3]) with both planes: 254*I0 + I1.
// Z: the chains start with sdot4_0 (no zeroing v_mov); without it the builtin
// form throughout, which the register allocator handles with less pressure.
template <bool Z = true>
__host__ __device__ inline int32_t piece_dot(const uint32_t* q, const LaneX& x, int p) {
    int32_t i0, i1;
    if constexpr (Z) {
        i0 = sdot4_0(q[0], x.d0[4 * p]);
        i1 = sdot4_0(q[0], x.d1[4 * p]);
    } else {
        i0 = sdot4(q[0], x.d0[4 * p], 0);
        i1 = sdot4(q[0], x.d1[4 * p], 0);
    }
#pragma unroll
    for (int i = 1; i < 4; ++i) {
        i0 = sdot4(q[i], x.d0[4 * p + i], i0);
        i1 = sdot4(q[i], x.d1[4 * p + i], i1);
    }
    return i0 * 254 + i1;
}

// ------------------------------------------------------------------- loads

__host__ __device__ inline void put4(uint32_t* w, const uint8_t* p) { __builtin_memcpy(w, p, 16); }
__host__ __device__ inline void put2(uint32_t* w, const uint8_t* p) { __builtin_memcpy(w, p, 8); }

// Raw bytes lane k needs from the block (Q8_0: the 256-column unit) at blk,
// into raw[0 .. NRAW).
// DW: Q6_K's d as the high half of the block's last dword (bytes 206..209,
// read through scale_word), else as a 16-bit load.  The gate/up kernel takes
// the dword form: with the 16-bit load, the shared expert's Q6_K instance held
// its first barrier for its weight loads (FP16-graph layers with a Q6_K shared
// expert 12.4-12.6 -> 11.7-11.9 us).  The down kernel keeps the 16-bit load
// (9.52 against 9.57 us for the benchmark layer).
template <int T, bool DW = false>
__host__ __device__ inline void lane_load(const uint8_t* blk, int k, uint32_t* raw) {
    if constexpr (T == T_Q8_0) {
        const uint8_t* b = blk + 68 * k;         // blocks 2k, 2k+1: d0 qs0[32] d1 qs1[32]
        put4(raw, b);
        put4(raw + 4, b + 16);
        put4(raw + 8, b + 32);
        put4(raw + 12, b + 48);
        __builtin_memcpy(raw + 16, b + 64, 4);
    } else if constexpr (T == T_Q4_K) {
        put4(raw, blk);                          // d, dmin, scales
        put4(raw + 4, blk + 16 + 32 * k);        // qs
        put4(raw + 8, blk + 32 + 32 * k);
    } else if constexpr (T == T_Q5_K) {
        put4(raw, blk);
        put4(raw + 4, blk + 16);                 // qh[32]
        put4(raw + 8, blk + 32);
        put4(raw + 12, blk + 48 + 32 * k);       // qs
        put4(raw + 16, blk + 64 + 32 * k);
    } else if constexpr (T == T_Q6_K) {
        const int h = k >> 1;
        put4(raw, blk + 64 * h + 32 * (k & 1));         // ql
        put4(raw + 4, blk + 64 * h + 32 * (k & 1) + 16);
        put4(raw + 8, blk + 128 + 32 * h);               // qh
        put4(raw + 12, blk + 128 + 32 * h + 16);
        put2(raw + 16, blk + 192 + 8 * h);               // int8 scales 8h .. 8h+7
        if constexpr (DW) {
            __builtin_memcpy(raw + 18, blk + 206, 4);
        } else {
            uint16_t d;
            __builtin_memcpy(&d, blk + 208, 2);
            raw[18] = d;
        }
    } else {  // Q3_K
        const int h = k >> 1, l0 = 16 * (k & 1);
        put4(raw, blk + l0);                     // hmask
        put4(raw + 4, blk + 32 + 32 * h + l0);   // qs
        __builtin_memcpy(raw + 8, blk + 96, 12); // scales
        // d in the high half of the block's last dword (bytes 106..109): a
        // 16-bit load's zero extension was placed, with a wait for the load,
        // ahead of the kernel's first barrier, so that barrier waited for every
        // weight load of the wave
        __builtin_memcpy(raw + 11, blk + 106, 4);
    }
}

// ------------------------------------------------------------------ scales

// Q4_K/Q5_K 6-bit scales and mins of sub-blocks 2k and 2k+1 from header dwords
// 1..3 (scale bytes 0..11), branch-free: both are in byte positions 2(k%2) and
// 2(k%2)+1 of their dwords; sub-blocks 0..3 take 6 bits of bytes 0..7,
// sub-blocks 4..7 combine the low/high nibble of bytes 8..11 with the top two
// bits of bytes 0..7.  Returns (sc0 | sc1 << 8) and (m0 | m1 << 8).
__host__ __device__ inline void k4_scale_min_pair(const uint32_t* hdr, int k, uint32_t& sc, uint32_t& mn) {
    const int p = 16 * (k & 1);
    const uint32_t A = hdr[1] >> p, B = hdr[2] >> p, C = hdr[3] >> p;
    const uint32_t sc_lo = A & 0x3F3Fu, mn_lo = B & 0x3F3Fu;
    const uint32_t sc_hi = (C & 0x0F0Fu) | ((A >> 2) & 0x3030u);
    const uint32_t mn_hi = ((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u);
    sc = k < 2 ? sc_lo : sc_hi;
    mn = k < 2 ? mn_lo : mn_hi;
}

// Bit field of `width` bits of x at `off` (v_bfe_u32 on the device).
__host__ __device__ inline uint32_t bfe(uint32_t x, int off, int width) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_ubfe(x, (uint32_t)off, (uint32_t)width);
#else
    return (x >> off) & ((1u << width) - 1u);
#endif
}

// x rotated right by r (0..31) (v_alignbit_b32 on the device).
__host__ __device__ inline uint32_t rotr(uint32_t x, int r) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_alignbit(x, x, (uint32_t)r);
#else
    return r ? (x >> r) | (x << (32 - r)) : x;
#endif
}

// The 32 bits of the 64-bit value hi:lo starting at bit r (0..31)
// (v_alignbit_b32 on the device).
__host__ __device__ inline uint32_t rotr_pair(uint32_t hi, uint32_t lo, int r) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_alignbit(hi, lo, (uint32_t)r);
#else
    return r ? (lo >> r) | (hi << (32 - r)) : lo;
#endif
}

// Q3_K signed 6-bit scale 8h + 2s + odd (the scale of run s of lane k = 2h +
// odd) from the 12 scale bytes sc[0..2]: its low nibble is nibble h of byte
// 2s + odd, its high two bits are bits 2(s/2) of byte 8 + 2(s%2) + odd, so both
// sit at the lane constant sh = 8 odd + 4h plus a per-run constant.
__host__ __device__ inline int k3_scale_run(const uint32_t* sc, int sh, int s) {
    const uint32_t lo = bfe(sc[s >> 1], sh + 16 * (s & 1), 4);
    const uint32_t hi = bfe(sc[2], sh + 16 * (s & 1) + 2 * (s >> 1), 2);
    return (int)(lo | (hi << 4)) - 32;
}

// ---------------------------------------------------------------- lane dots

// Dot product of lane k's 64 weights (raw bytes from lane_load) with x.
// Q6_K's d from raw as lane_load<T_Q6_K, DW> left it
template <bool DW>
__host__ __device__ inline float q6_d(const uint32_t* raw) {
    if constexpr (DW) return f16_bits_to_f32(scale_word(raw, 18) >> 16);
    else return f16_bits_to_f32(raw[18] & 0xFFFFu);
}

// Z: piece_dot's form (see there).
template <int T, bool DW = false, bool Z = true>
__host__ __device__ inline float lane_dot(const uint32_t* raw, int k, const LaneX& x) {
    if constexpr (T == T_Q8_0) {
        // block 0: d at bytes 0-1, quants at bytes 2..33 (dwords shifted by two
        // bytes); block 1: d at bytes 34-35, quants at bytes 36..67 (dwords 9..16)
        const float d0 = f16_bits_to_f32(raw[0] & 0xFFFFu), d1 = f16_bits_to_f32(raw[8] >> 16);
        float run0 = 0.0f, run1 = 0.0f;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = rotr_pair(raw[4 * p + i + 1], raw[4 * p + i], 16);
            run0 = fmaf(x.xs[p], (float)piece_dot<Z>(q, x, p), run0);
            run1 = fmaf(x.xs[2 + p], (float)piece_dot<Z>(raw + 9 + 4 * p, x, 2 + p), run1);
        }
        return fmaf(d0, run0, d1 * run1);
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        constexpr int QS = T == T_Q4_K ? 4 : 12;
        const uint32_t dw = raw[0];
        const float d = f16_bits_to_f32(dw & 0xFFFFu), dmin = f16_bits_to_f32(dw >> 16);
        uint32_t sc2, mn2;
        k4_scale_min_pair(raw, k, sc2, mn2);
        float acc = 0.0f, off = 0.0f;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            float run = 0.0f;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                uint32_t q[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    q[i] = (raw[QS + 4 * p + i] >> (4 * r)) & 0x0F0F0F0Fu;
                    if constexpr (T == T_Q5_K) q[i] |= ((raw[4 + 4 * p + i] >> (2 * k + r)) & 0x01010101u) << 4;
                }
                run = fmaf(x.xs[2 * r + p], (float)piece_dot<Z>(q, x, 2 * r + p), run);
            }
            acc = fmaf((float)((sc2 >> (8 * r)) & 0xFFu), run, acc);
            off = fmaf((float)((mn2 >> (8 * r)) & 0xFFu), x.sum[2 * r] + x.sum[2 * r + 1], off);
        }
        return fmaf(d, acc, -dmin * off);
    } else if constexpr (T == T_Q6_K) {
        const float d = q6_d<DW>(raw);
        const int j = k & 1;
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int s = j + 2 * r;
            // qh bits 2s, 2s + 1 of every byte moved to bits 4, 5 by one rotation
            const int rq = (2 * s - 4) & 31;
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                uint32_t q[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    q[i] = ((raw[4 * p + i] >> (4 * r)) & 0x0F0F0F0Fu) |
                           (rotr(raw[8 + 4 * p + i], rq) & 0x30303030u);   // 0..63; -32 below
                // int8 scale of the 16-column sub-block 8h + 2s + p (byte 2s + p of the 8 loaded)
                const int sb = 2 * s + p;
                const int sc = (int)(int8_t)(uint8_t)((sb < 4 ? raw[16] >> (8 * sb) : raw[17] >> (8 * (sb - 4))) & 0xFFu);
                const int pc = 2 * r + p;
                acc = fmaf((float)sc, fmaf(x.xs[pc], (float)piece_dot<Z>(q, x, pc), -32.0f * x.sum[pc]), acc);
            }
        }
        return d * acc;
    } else {  // Q3_K
        const float d = f16_bits_to_f32(scale_word(raw, 11) >> 16);
        const int h = k >> 1, odd = k & 1, sh = 8 * odd + 4 * h;
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // Runs 1 and 2 keep their two quant bits in place (bits 2s, 2s + 1 of
            // every byte: the byte is 4^s q <= 112, still an int8, and the piece's
            // integer dot 4^s times the run's, taken back exactly by the run
            // scale); runs 0 and 3 shift them to bits 0, 1.  The mask bit 4h + s
            // goes to the bit above them, sp + 2, by one rotation (right by
            // 4h + s - 2 - sp mod 32, which takes byte k's bit 4h + s to bit
            // 8k + sp + 2 without crossing the word's top).
            const int sp = (s == 1 || s == 2) ? 2 * s : 0;
            const int r = (4 * h + s - 2 - sp) & 31;
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = sp ? raw[4 + i] & (0x03030303u << sp) : (raw[4 + i] >> (2 * s)) & 0x03030303u;
                q[i] = lo | (rotr(raw[i], r) & (0x04040404u << sp));
            }
            const float xs = sp ? x.xs[s] * (sp == 2 ? 0.25f : 0.0625f) : x.xs[s];
            const int sc = k3_scale_run(raw + 8, sh, s);
            acc = fmaf((float)sc, fmaf(xs, (float)piece_dot<Z>(q, x, s), -4.0f * x.sum[s]), acc);
        }
        return d * acc;
    }
}


// ------------------------------------------------------------ FP16 graph
//
// The reference's FP16 graph (moe_quant_dot.cpp:154-157, 189-211) multiplies
// FP16-rounded weights with FP16-rounded activations and accumulates in FP32.
// A lane's 64 weights are decoded to FP32 with the reference decoders'
// arithmetic (the formulas of decode8 in kquant_device.h: Q4_K/Q5_K
// RN(RN(d1 q) - m1), Q6_K RN(ds (q - 32)), Q3_K RN(ds (q - 4)), Q8_0 RN(q d)),
// rounded to FP16 (RNE) and paired in column order, as the FP16 activations of
// the same columns are.

// f rounded to FP16 (RNE), as bits.  On the device the operand is made opaque
// first: the instruction selector would otherwise fold the FP32 arithmetic
// that produced it into a mixed-precision instruction with one rounding.
__host__ __device__ inline uint32_t rn16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
    __asm__ volatile("" : "+v"(f));
#endif
    const _Float16 h = (_Float16)f;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__host__ __device__ inline uint32_t pack_rn16(float lo, float hi) { return rn16_bits(lo) | (rn16_bits(hi) << 16); }

// The FP16 activations of one lane's 64 columns, column pairs in run order
// (pair i = the lane's columns 2i and 2i + 1).
struct LaneH {
    uint32_t h[32];
};

// x16: an activation vector of FP16 bit patterns (the FP16 graph's rounded x).
template <int T>
__host__ __device__ inline void lane_xh(const uint16_t* x16, int blk, int k, LaneH& x) {
    constexpr int NR = LaneGeo<T>::NR, RL = LaneGeo<T>::RL;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int c = 256 * blk + lane_col<T>(k, r);
#pragma unroll
        for (int p = 0; p < RL / 8; ++p) {
            const uint4 a = *(const uint4*)(x16 + c + 8 * p);
            const int b = (r * RL + 8 * p) / 2;
            x.h[b] = a.x; x.h[b + 1] = a.y; x.h[b + 2] = a.z; x.h[b + 3] = a.w;
        }
    }
}

namespace detail {
// separately rounded FP32 products and differences, as the reference decoders
// compute them (never contracted into one fused multiply-add)
__host__ __device__ inline float mul_rn(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __fmul_rn(a, b);
#else
#pragma clang fp contract(off)
    return a * b;
#endif
}
__host__ __device__ inline float sub_rn(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __fsub_rn(a, b);
#else
#pragma clang fp contract(off)
    return a - b;
#endif
}

// the FP16 value of the low / high half of v, in FP32 (exact, subnormals included)
__host__ __device__ inline float half_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)v); }
__host__ __device__ inline float half_hi(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

// w[j] = f(byte j of the 4 dwords at q) for 16 bytes, packed as FP16 pairs into out[0..7]
template <class F>
__host__ __device__ inline void pack16_bytes(const uint32_t* q, uint32_t* out, F&& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float b0 = (float)(q[i] & 0xFFu), b1 = (float)((q[i] >> 8) & 0xFFu);
        const float b2 = (float)((q[i] >> 16) & 0xFFu), b3 = (float)(q[i] >> 24);
        out[2 * i] = pack_rn16(f(b0), f(b1));
        out[2 * i + 1] = pack_rn16(f(b2), f(b3));
    }
}
// w[j] = s * (signed byte j of the 4 dwords at w) for 16 bytes, packed as FP16
// pairs into out[0..7] (one sign-extending byte conversion and one product a
// weight)
__host__ __device__ inline void pack16_sbytes(const uint32_t* w, float s, uint32_t* out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float b0 = (float)(int8_t)(w[i] & 0xFFu), b1 = (float)(int8_t)((w[i] >> 8) & 0xFFu);
        const float b2 = (float)(int8_t)((w[i] >> 16) & 0xFFu), b3 = (float)(int8_t)(w[i] >> 24);
        out[2 * i] = pack_rn16(mul_rn(s, b0), mul_rn(s, b1));
        out[2 * i + 1] = pack_rn16(mul_rn(s, b2), mul_rn(s, b3));
    }
}
}  // namespace detail

// Piece P (0..3, 16 weights) of lane k's 64 weights as FP16 pairs, in run
// order: out[0..7] are the pairs 8P .. 8P+7 of lane_w16 (raw bytes from
// lane_load).
template <int T, int P, bool DW = false>
__host__ __device__ inline void lane_w16_piece(const uint32_t* raw, int k, uint32_t* out) {
    if constexpr (T == T_Q8_0) {
        // pieces 0, 1: block 2k (d at bytes 0-1, quants at bytes 2..33); 2, 3: block 2k+1
        if constexpr (P < 2) {
            const float d0 = f16_bits_to_f32(raw[0] & 0xFFFFu);
            uint32_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = rotr_pair(raw[4 * P + i + 1], raw[4 * P + i], 16);
            detail::pack16_bytes(q, out, [&](float b) { return detail::mul_rn((float)(int8_t)(int)b, d0); });
        } else {
            const float d1 = f16_bits_to_f32(raw[8] >> 16);
            detail::pack16_bytes(raw + 9 + 4 * (P - 2), out,
                                 [&](float b) { return detail::mul_rn((float)(int8_t)(int)b, d1); });
        }
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        constexpr int QS = T == T_Q4_K ? 4 : 12, r = P / 2, p = P % 2;
        const uint32_t dw = raw[0];
        const float d = f16_bits_to_f32(dw & 0xFFFFu), dmin = f16_bits_to_f32(dw >> 16);
        uint32_t sc2, mn2;
        k4_scale_min_pair(raw, k, sc2, mn2);
        const float d1 = detail::mul_rn(d, (float)((sc2 >> (8 * r)) & 0xFFu));
        const float m1 = detail::mul_rn(dmin, (float)((mn2 >> (8 * r)) & 0xFFu));
        // RN(RN(d1 q) - m1) as one fused multiply-add: d1 = d sc has at most 17
        // significant bits (FP16 d, 6-bit sc), so d1 q (q < 32) has at most 22 and
        // RN(d1 q) = d1 q; the fused form rounds d1 q - m1 once, as the
        // reference's subtraction does.  The quants enter the multiply-add as
        // FP16 subnormals: a 16-bit half holding the integer v is v 2^-24
        // exactly, so the masked halves of a quant dword (bytes 0 and 2, then 1
        // and 3) times d1 2^24 (exact: a power of two) give d1 q.  gfx950 reads
        // an FP16 operand from either half of a register in v_fma_mix_f32, so a
        // weight is one instruction, with no byte extraction or conversion.  A
        // Q4_K high nibble stays in place (16 q in the half) with d1 2^20.
        uint32_t e[4], o[4];
        float ds;
        if constexpr (T == T_Q4_K) {
            constexpr uint32_t M = r == 0 ? 0x000F000Fu : 0x00F000F0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t w = raw[QS + 4 * p + i];
                e[i] = w & M;
                o[i] = (w >> 8) & M;
            }
            ds = d1 * (r == 0 ? 16777216.0f : 1048576.0f);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t q = ((raw[QS + 4 * p + i] >> (4 * r)) & 0x0F0F0F0Fu) |
                                   (((raw[4 + 4 * p + i] >> (2 * k + r)) & 0x01010101u) << 4);
                e[i] = q & 0x00FF00FFu;
                o[i] = (q >> 8) & 0x00FF00FFu;
            }
            ds = d1 * 16777216.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float w0 = fmaf(ds, detail::half_lo(e[i]), -m1), w1 = fmaf(ds, detail::half_lo(o[i]), -m1);
            const float w2 = fmaf(ds, detail::half_hi(e[i]), -m1), w3 = fmaf(ds, detail::half_hi(o[i]), -m1);
            out[2 * i] = pack_rn16(w0, w1);
            out[2 * i + 1] = pack_rn16(w2, w3);
        }
    } else if constexpr (T == T_Q6_K) {
        // q - 32 for the 6-bit u: its two's complement is u ^ 32 in bits 2..7 of a
        // byte (low nibble rotated to bits 2..5, the two high bits to 6..7, the
        // top bit flipped), i.e. the int8 4 (u - 32); times RN(d sc) / 4 (exact)
        // that is RN(d sc (u - 32)), the reference decoder's product
        constexpr int r = P / 2, p = P % 2;
        const float d = q6_d<DW>(raw);
        const int s = (k & 1) + 2 * r, ra = (4 * r + 30) & 31, rb = (2 * s + 26) & 31;
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = ((rotr(raw[4 * p + i], ra) & 0x3C3C3C3Cu) | (rotr(raw[8 + 4 * p + i], rb) & 0xC0C0C0C0u)) ^ 0x80808080u;
        const int sb = 2 * s + p;
        const int sc = (int)(int8_t)(uint8_t)((sb < 4 ? raw[16] >> (8 * sb) : raw[17] >> (8 * (sb - 4))) & 0xFFu);
        detail::pack16_sbytes(w, detail::mul_rn(d, (float)sc) * 0.25f, out);
    } else {  // Q3_K: piece P is run s = P
        // q - 4 = low2 - 4 (1 - hbit): the two low bits rotated to bits 5..6 and
        // the inverted mask bit to bit 7 make the int8 32 (q - 4); times
        // RN(d sc) / 32 (exact) that is RN(d sc (q - 4))
        const float d = f16_bits_to_f32(scale_word(raw, 11) >> 16);
        const int h = k >> 1, odd = k & 1, sh = 8 * odd + 4 * h;
        const int ra = (2 * P + 27) & 31, rb = (4 * h + P + 25) & 31;
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (rotr(raw[4 + i], ra) & 0x60606060u) | (~rotr(raw[i], rb) & 0x80808080u);
        detail::pack16_sbytes(w, detail::mul_rn(d, (float)k3_scale_run(raw + 8, sh, P)) * 0.03125f, out);
    }
}

// Lane k's 64 weights as FP16 pairs in run order.
template <int T, bool DW = false>
__host__ __device__ inline void lane_w16(const uint32_t* raw, int k, uint32_t (&w)[32]) {
    lane_w16_piece<T, 0, DW>(raw, k, w);
    lane_w16_piece<T, 1, DW>(raw, k, w + 8);
    lane_w16_piece<T, 2, DW>(raw, k, w + 16);
    lane_w16_piece<T, 3, DW>(raw, k, w + 24);
}

namespace detail {
template <int T, int P, bool DW>
__host__ __device__ inline float dot16_piece(const uint32_t* raw, int k, const LaneH& x, float acc) {
    uint32_t w[8];
    lane_w16_piece<T, P, DW>(raw, k, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#if defined(__HIP_DEVICE_COMPILE__)
        typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w[i]), __builtin_bit_cast(half2_t, x.h[8 * P + i]),
                                     acc, false);
#else
        acc += f16_bits_to_f32(w[i] & 0xFFFFu) * f16_bits_to_f32(x.h[8 * P + i] & 0xFFFFu) +
               f16_bits_to_f32(w[i] >> 16) * f16_bits_to_f32(x.h[8 * P + i] >> 16);
#endif
    }
    return acc;
}
}  // namespace detail

// FP16-graph dot product of lane k's 64 weights with x: FP16 products summed
// in FP32, two columns per v_dot2_f32_f16 (the host build sums the exact
// products in FP32 in the same order), decoded one 16-weight piece at a time.
template <int T, bool DW = false>
__host__ __device__ inline float lane_dot_f16(const uint32_t* raw, int k, const LaneH& x) {
    float acc = detail::dot16_piece<T, 0, DW>(raw, k, x, 0.0f);
    acc = detail::dot16_piece<T, 1, DW>(raw, k, x, acc);
    acc = detail::dot16_piece<T, 2, DW>(raw, k, x, acc);
    return detail::dot16_piece<T, 3, DW>(raw, k, x, acc);
}

}  // namespace mqh
