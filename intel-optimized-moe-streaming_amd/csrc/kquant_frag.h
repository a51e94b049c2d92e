// kquant_frag.h -- K-quant super-blocks as exact FP16 MFMA operands.
//
// The prefill GEMMs multiply quantized weight rows by FP16 token tiles on
// v_mfma_f32_16x16x32_f16.  Rounding the dequantized weight d*sc*q - dmin*m to
// FP16 costs ~2^-12 relative per weight, and with Q4_K's large min offsets the
// cancellation in a 2048-term dot product turns that into ~1e-3 of the output.
// So the A operand carries only the exact small integers sc_m * q (|value| <=
// 1953, or a split pair for Q6_K), the MFMA sums one 32-column sub-block per
// step, and the FP32 factors d and dmin are applied once per super-block:
//
//   sum_c w_c x_c = d * sum_m sum_{c in m} (sc_m q_c) x_c  -  dmin * sum_m mn_m X_m
//
// with X_m = sum_{c in m} x_c (the min term is a second, tiny MFMA).  Every
// product inside the MFMA is exact, so the only rounding is the FP32
// accumulation, as in the reference's FP32 kernels (cpp/moe_quant_dot.cpp:30-150,
// block formats of cpp/dequant_k.cpp:1-200).
//
// Lane l of a wave feeds weight row l % 16 and, in 32-column step m of a block,
// columns 32m + 8q .. 32m + 8q + 7 with q = l / 16 (the A layout of
// v_mfma_f32_16x16x32_f16).  frag_load fetches every byte of a block that the
// lane needs (NW words); frag_step builds step m's operands.  Host and device
// share this code; the host build is a test helper.
#pragma once

#include <stdint.h>
#include <string.h>

#include "kquant_device.h"

namespace mqh {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));

template <int T> struct FragGeo;
// NW: raw words per lane and block; NA: A operands per step (Q6_K splits its
// scale); MIN: has a min term; HDR: word holding the FP16 d (low half) and dmin
template <> struct FragGeo<T_Q4_K> { static constexpr int NW = 12, NA = 1, HDR = 0; static constexpr bool MIN = true; };
template <> struct FragGeo<T_Q5_K> { static constexpr int NW = 14, NA = 1, HDR = 0; static constexpr bool MIN = true; };
template <> struct FragGeo<T_Q6_K> { static constexpr int NW = 17, NA = 2, HDR = 16; static constexpr bool MIN = false; };
template <> struct FragGeo<T_Q3_K> { static constexpr int NW = 10, NA = 1, HDR = 9; static constexpr bool MIN = false; };

// 32 bits at any byte offset of a block (Q6_K and Q3_K blocks are only 2-byte
// aligned; gfx950 global loads accept unaligned addresses).  On the device the
// load is explicitly global: a generic (flat) load would also count against the
// LDS wait counter and serialise with the LDS traffic of the GEMM.
__host__ __device__ inline uint32_t frag_ld32(const uint8_t* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef uint32_t __attribute__((aligned(1))) u32_unaligned;
    return *(const __attribute__((address_space(1))) u32_unaligned*)p;
#else
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
#endif
}

template <int T>
__host__ __device__ inline void frag_load(const uint8_t* blk, int q, uint32_t* r) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        constexpr int QS = T == T_Q4_K ? 16 : 48;
        for (int i = 0; i < 4; ++i) r[i] = frag_ld32(blk + 4 * i);                 // d, dmin, scales[12]
        for (int g = 0; g < 4; ++g) {                                               // qs pieces
            r[4 + 2 * g] = frag_ld32(blk + QS + 32 * g + 8 * q);
            r[5 + 2 * g] = frag_ld32(blk + QS + 32 * g + 8 * q + 4);
        }
        if constexpr (T == T_Q5_K) {                                                // qh piece
            r[12] = frag_ld32(blk + 16 + 8 * q);
            r[13] = frag_ld32(blk + 20 + 8 * q);
        }
    } else if constexpr (T == T_Q6_K) {
        for (int c = 0; c < 4; ++c) {                                               // ql: 64h + 32(s&1)
            r[2 * c] = frag_ld32(blk + 32 * c + 8 * q);
            r[2 * c + 1] = frag_ld32(blk + 32 * c + 8 * q + 4);
        }
        for (int h = 0; h < 2; ++h) {                                               // qh: 128 + 32h
            r[8 + 2 * h] = frag_ld32(blk + 128 + 32 * h + 8 * q);
            r[9 + 2 * h] = frag_ld32(blk + 132 + 32 * h + 8 * q);
        }
        for (int i = 0; i < 4; ++i) r[12 + i] = frag_ld32(blk + 192 + 4 * i);       // int8 scales
        uint16_t d;
        memcpy(&d, blk + 208, 2);
        r[16] = d;
    } else {  // Q3_K
        for (int h = 0; h < 2; ++h) {                                               // qs: 32 + 32h
            r[2 * h] = frag_ld32(blk + 32 + 32 * h + 8 * q);
            r[2 * h + 1] = frag_ld32(blk + 36 + 32 * h + 8 * q);
        }
        r[4] = frag_ld32(blk + 8 * q);                                              // hmask
        r[5] = frag_ld32(blk + 8 * q + 4);
        for (int i = 0; i < 3; ++i) r[6 + i] = frag_ld32(blk + 96 + 4 * i);         // scales[12]
        uint16_t d;
        memcpy(&d, blk + 108, 2);
        r[9] = d;
    }
}

__host__ __device__ inline h2_t frag_bits_h2(uint32_t v) {
    h2_t h;
    memcpy(&h, &v, 4);
    return h;
}

// The 4 bytes of w (each < 64) as halves 1024 + byte: FP16 1024 has ulp 1, so
// 0x6400 | byte is exact.
__host__ __device__ inline void frag_biased(uint32_t w, h2_t& lo, h2_t& hi) {
    lo = frag_bits_h2((w & 0xFFu) | ((w & 0xFF00u) << 8) | 0x64006400u);
    hi = frag_bits_h2(((w >> 16) & 0xFFu) | ((w >> 8) & 0xFF0000u) | 0x64006400u);
}

__host__ __device__ inline h2_t frag_splat(float v) {
    h2_t h;
    h[0] = (_Float16)v;
    h[1] = (_Float16)v;
    return h;
}

// sc * (biased - bias) for the 8 bytes of (w0, w1), as one fused multiply-add
// per pair: the exact result is a small integer, so the single rounding of the
// fma is exact.
__host__ __device__ inline h8_t frag_scaled(uint32_t w0, uint32_t w1, float sc, float bias) {
    const h2_t s = frag_splat(sc), c = frag_splat(-bias * sc);
    h2_t p[4];
    frag_biased(w0, p[0], p[1]);
    frag_biased(w1, p[2], p[3]);
    h8_t a;
    for (int i = 0; i < 4; ++i) {
        const h2_t v = __builtin_elementwise_fma(p[i], s, c);
        a[2 * i] = v[0];
        a[2 * i + 1] = v[1];
    }
    return a;
}

// Q4_K / Q5_K 6-bit scale and min of sub-block m (get_scale_min_k4,
// cpp/dequant_k.cpp:60-75); s = the 12 scale bytes in words r[1..3]
template <int M>
__host__ __device__ inline void frag_scale_min(const uint32_t* r, int& sc, int& mn) {
    auto sb = [&](int i) { return (int)((r[1 + i / 4] >> (8 * (i % 4))) & 0xFFu); };
    if constexpr (M < 4) {
        sc = sb(M) & 63;
        mn = sb(M + 4) & 63;
    } else {
        sc = (sb(M + 4) & 15) | ((sb(M - 4) >> 6) << 4);
        mn = (sb(M + 4) >> 4) | ((sb(M) >> 6) << 4);
    }
}

// Step M's A operands.  a[0] (and a[1] for Q6_K) are exact; the operand for a
// low-order B plane is a[0] (Q6_K: a[0] + a[1], one rounding of an exact sum).
template <int T, int M>
__host__ __device__ inline void frag_step(const uint32_t* r, int q, h8_t* a) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        // columns 32M + 8q + e: nibble M&1 of qs byte 32(M>>1) + 8q + e; Q5_K bit 5 = qh bit M
        constexpr int g = M >> 1, h = M & 1;
        uint32_t b0 = (r[4 + 2 * g] >> (4 * h)) & 0x0F0F0F0Fu, b1 = (r[5 + 2 * g] >> (4 * h)) & 0x0F0F0F0Fu;
        if constexpr (T == T_Q5_K) {
            b0 |= ((r[12] >> M) & 0x01010101u) << 4;
            b1 |= ((r[13] >> M) & 0x01010101u) << 4;
        }
        int sc, mn;
        frag_scale_min<M>(r, sc, mn);
        a[0] = frag_scaled(b0, b1, (float)sc, 1024.0f);
    } else if constexpr (T == T_Q6_K) {
        // columns 128H + 32S + 8q + e: ql byte 64H + 32(S&1) + 8q + e (nibble S>>1),
        // qh byte 32H + 8q + e (bits 2S), int8 scale 8H + 2S + q/2
        constexpr int H = M >> 2, S = M & 3, c = 2 * H + (S & 1);
        const uint32_t q0 = ((r[2 * c] >> (4 * (S >> 1))) & 0x0F0F0F0Fu) | (((r[8 + 2 * H] >> (2 * S)) & 0x03030303u) << 4);
        const uint32_t q1 = ((r[2 * c + 1] >> (4 * (S >> 1))) & 0x0F0F0F0Fu) | (((r[9 + 2 * H] >> (2 * S)) & 0x03030303u) << 4);
        const int sc = (int)(int8_t)((r[12 + 2 * H + (S >> 1)] >> (16 * (S & 1))) >> (8 * (q >> 1)));
        // sc * (q - 32) reaches 4096, past FP16's exact integers: split sc = 16*hi + lo
        const h2_t s_hi = frag_splat((float)(16 * (sc >> 4))), s_lo = frag_splat((float)(sc & 15));
        const h2_t bias = frag_splat(-1056.0f);
        h2_t p[4];
        frag_biased(q0, p[0], p[1]);
        frag_biased(q1, p[2], p[3]);
        for (int i = 0; i < 4; ++i) {
            const h2_t v = p[i] + bias;          // q - 32, exact
            const h2_t x = v * s_hi, y = v * s_lo;
            a[0][2 * i] = x[0];
            a[0][2 * i + 1] = x[1];
            a[1][2 * i] = y[0];
            a[1][2 * i + 1] = y[1];
        }
    } else {  // Q3_K: columns 128H + 32S + 8q + e; 2 bits of qs, hmask bit 4H + S; scale 8H + 2S + q/2
        constexpr int H = M >> 2, S = M & 3;
        const uint32_t q0 = ((r[2 * H] >> (2 * S)) & 0x03030303u) | (((r[4] >> (4 * H + S)) & 0x01010101u) << 2);
        const uint32_t q1 = ((r[2 * H + 1] >> (2 * S)) & 0x03030303u) | (((r[5] >> (4 * H + S)) & 0x01010101u) << 2);
        // scale j = 8H + 2S + q/2: low nibble of byte j&7 (high nibble for H = 1), top two
        // bits at 2(j>>2) of byte 8 + (j&3); j&7 and j&3 are byte 2(S&1) + q/2 of a word
        const int bsh = 16 * (S & 1) + 8 * (q >> 1);
        const int lo = (int)((r[6 + (S >> 1)] >> (bsh + 4 * H)) & 15u);
        const int hi = (int)((r[8] >> (bsh + 2 * (2 * H + (S >> 1)))) & 3u);
        // (q - 4) * sc with both steps exact (the fused form's addend 1028*sc is not an FP16 value)
        const h2_t s = frag_splat((float)((lo | (hi << 4)) - 32)), bias = frag_splat(-1028.0f);
        h2_t p[4];
        frag_biased(q0, p[0], p[1]);
        frag_biased(q1, p[2], p[3]);
        for (int i = 0; i < 4; ++i) {
            const h2_t v = (p[i] + bias) * s;
            a[0][2 * i] = v[0];
            a[0][2 * i + 1] = v[1];
        }
    }
}

template <int T>
__host__ __device__ inline h8_t frag_lo_operand(const h8_t* a) {
    if constexpr (FragGeo<T>::NA == 2) return a[0] + a[1];
    else return a[0];
}

// A operand of the min-term MFMA (v_mfma_f32_16x16x16_f16, K = 16): lane q holds
// k = 4q .. 4q+3, i.e. the mins of sub-blocks 4(q&1) .. 4(q&1)+3 (the second
// half of K repeats them against the low-order sums).  The operand is 32 * min
// (exact, <= 2016) because the B side holds the sub-block sums divided by 32,
// which keeps a sum of 32 values below 2^14 inside FP16.
template <int T>
__host__ __device__ inline h4_t frag_mins(const uint32_t* r, int q) {
    const uint32_t lo4 = r[2] & 0x3F3F3F3Fu;                                      // mins 0..3: scales[4..7] & 63
    const uint32_t hi4 = ((r[3] >> 4) & 0x0F0F0F0Fu) | ((r[2] >> 2) & 0x30303030u); // mins 4..7
    h2_t p0, p1;
    frag_biased((q & 1) ? hi4 : lo4, p0, p1);
    const h2_t bias = frag_splat(-1024.0f), x32 = frag_splat(32.0f);
    p0 = (p0 + bias) * x32;
    p1 = (p1 + bias) * x32;
    h4_t m;
    m[0] = p0[0];
    m[1] = p0[1];
    m[2] = p1[0];
    m[3] = p1[1];
    return m;
}

// FP16 bits of the block's d (low half) and dmin (high half) from the header word
__host__ __device__ inline float frag_h2f(uint32_t bits) {
    _Float16 h;
    const uint16_t b = (uint16_t)bits;
    memcpy(&h, &b, 2);
    return (float)h;
}

// ------------------------------------------------------------ B operand
//
// A token row enters the MFMA as FP16 after an exact power-of-two scale 2^-k
// that puts its max |value| in [2^13, 2^14) (activations reach ~5e4, next to
// FP16's limit, and small rows would otherwise lose bits to subnormals), split
// into a high plane and the FP16 rounding of the remainder: hi + lo carries
// ~22 significant bits.  BF16 inputs are exact in the high plane alone.

__host__ __device__ inline int frag_exp(float amax) {
    if (!(amax > 0.0f) || !(amax <= 3.4028235e38f)) return 0;
    int e;
    (void)frexpf(amax, &e);
    return e - 14;
}

__host__ __device__ inline void frag_split(float v, int k, _Float16& hi, _Float16& lo) {
    // (a sub-block sum of 32 scaled values enters as frag_split(sum, 5, ...))
    const float s = ldexpf(v, -k);
    hi = (_Float16)s;
    lo = (_Float16)(s - (float)hi);
}

}  // namespace mqh
