// kquant_frag.h -- K-quant super-blocks as exact FP16 MFMA operands.
//
// The prefill GEMMs multiply quantized weight rows by FP16 token tiles on
// v_mfma_f32_16x16x32_f16.  Rounding the dequantized weight d*sc*q - dmin*m to
// FP16 costs ~2^-12 relative per weight, and with Q4_K's large min offsets the
// cancellation in a 2048-term dot product turns that into ~1e-3 of the output.
// So the A operand carries only the exact small integers sc_s * q (|value| <=
// 1953, or a split pair for Q6_K), eight MFMA steps cover one 256-column
// super-block, and the FP32 factors d and dmin are applied once per super-block:
//
//   sum_c w_c x_c = d * sum_c (sc_s(c) q_c) x_c  -  dmin * sum_s mn_s X_s
//
// with X_s the sum of x over 32-column sub-block s (the min term is a second,
// tiny MFMA).  Every product inside the MFMA is exact, so the only rounding is
// the FP32 accumulation, as in the reference's FP32 kernels
// (cpp/moe_quant_dot.cpp:30-150; block formats cpp/dequant_k.cpp:146-298).
//
// Lane layout.  v_mfma_f32_16x16x32_f16 takes A row l % 16 from lane l and
// eight consecutive k-slots 8q .. 8q+7 with q = l / 16.  Inside one
// super-block the columns may be dealt to (step, lane, slot) in any order as
// long as the token operand follows the same order, so each lane owns the
// columns whose quants sit in contiguous 16-byte runs of the block: the four
// lanes of a row then read 64 contiguous bytes per load (the natural order reads
// 32-byte pieces, at half the achieved bandwidth).  With qq = (q + 3) & 3 the
// lane's step-m columns are the 8 consecutive columns
// frag_col<T, m>() + frag_lane_col<T>(qq).  frag_load fetches a lane's bytes of
// a block (NW words), frag_prep its scales, frag_step the operands of step m.
// Host and device share this code; the host build is a test helper.
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
// products); MIN: has a min term; HDR: word holding the FP16 d at bit D_SHIFT,
// with dmin in the high half for Q4_K/Q5_K
template <> struct FragGeo<T_Q4_K> { static constexpr int NW = 12, NA = 1, HDR = 0, D_SHIFT = 0; static constexpr bool MIN = true; };
template <> struct FragGeo<T_Q5_K> { static constexpr int NW = 16, NA = 1, HDR = 0, D_SHIFT = 0; static constexpr bool MIN = true; };
template <> struct FragGeo<T_Q6_K> { static constexpr int NW = 21, NA = 2, HDR = 20, D_SHIFT = 0; static constexpr bool MIN = false; };
template <> struct FragGeo<T_Q3_K> { static constexpr int NW = 12, NA = 1, HDR = 11, D_SHIFT = 16; static constexpr bool MIN = false; };
// Q8_0 (a unit of 256 columns is 8 blocks of 34 bytes, each with its own FP16
// d): step M is block M, its operand the 32 int8 quants as exact halves, and
// d is applied per step (PfRows::block); words 16 and 17 hold the FP16 d of
// blocks 2qq and 2qq + 1 of the lane's row
template <> struct FragGeo<T_Q8_0> { static constexpr int NW = 18, NA = 1, HDR = 16, D_SHIFT = 0; static constexpr bool MIN = false; };

// Bytes of one 256-column unit of a row: a K-quant super-block, or eight
// Q8_0 blocks.
template <int T>
__host__ __device__ constexpr int frag_unit_bytes() { return T == T_Q8_0 ? 8 * 34 : block_bytes(T); }

// First column of step M's 8 columns, before the lane's offset.
template <int T, int M>
__host__ __device__ constexpr int frag_col() {
    if constexpr (T == T_Q8_0) return 32 * M;
    else if constexpr (T == T_Q6_K) return 128 * (M >> 2) + 64 * ((M >> 1) & 1) + 8 * (M & 1);
    else if constexpr (T == T_Q3_K) return 32 * (M >> 1) + 8 * (M & 1);
    else return 128 * (M >> 2) + 32 * ((M >> 1) & 1) + 8 * (M & 1);
}

// The lane's column offset (qq = (q + 3) & 3).
template <int T>
__host__ __device__ inline int frag_lane_col(int qq) {
    if constexpr (T == T_Q8_0) return 8 * qq;
    else if constexpr (T == T_Q6_K) return 32 * (qq >> 1) + 16 * (qq & 1);
    else if constexpr (T == T_Q3_K) return 128 * (qq >> 1) + 16 * (qq & 1);
    else return 64 * (qq >> 1) + 16 * (qq & 1);
}

// Loads.  On the device they are explicitly global (a generic load would also
// count against the LDS wait counter) and may be unaligned (Q6_K and Q3_K
// blocks are only 2-byte aligned; gfx950 global loads accept that).
__host__ __device__ inline void frag_ld128(const uint8_t* p, uint32_t* w) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef uint4 __attribute__((aligned(1))) u128_unaligned;
    const uint4 v = *(const __attribute__((address_space(1))) u128_unaligned*)p;
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
#else
    memcpy(w, p, 16);
#endif
}

__host__ __device__ inline void frag_ld64(const uint8_t* p, uint32_t* w) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef uint2 __attribute__((aligned(1))) u64_unaligned;
    const uint2 v = *(const __attribute__((address_space(1))) u64_unaligned*)p;
    w[0] = v.x;
    w[1] = v.y;
#else
    memcpy(w, p, 8);
#endif
}

__host__ __device__ inline uint32_t frag_ld16(const uint8_t* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef uint16_t __attribute__((aligned(1))) u16_unaligned;
    return *(const __attribute__((address_space(1))) u16_unaligned*)p;
#else
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
#endif
}

// 16 bytes from a 2-byte aligned p with dword-aligned loads: the 16 bytes at
// the dword at or below p and the dword after them, shifted by 0 or 16 bits.
// Reads up to 2 bytes before p and 4 bytes past p + 16 (a 16-byte load that is
// not dword aligned is slow on this GPU; every other Q6_K block starts 2 bytes
// off a dword).
__host__ __device__ inline void frag_ld128_a2(const uint8_t* p, uint32_t* w) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uintptr_t a = (uintptr_t)p;
    const __attribute__((address_space(1))) uint32_t* q =
        (const __attribute__((address_space(1))) uint32_t*)(a & ~(uintptr_t)3);
    const uint4 v = *(const __attribute__((address_space(1))) uint4*)q;
    const uint32_t e = q[4];
    const uint32_t sh = (uint32_t)(a & 3) * 8;
    w[0] = __builtin_amdgcn_alignbit(v.y, v.x, sh);
    w[1] = __builtin_amdgcn_alignbit(v.z, v.y, sh);
    w[2] = __builtin_amdgcn_alignbit(v.w, v.z, sh);
    w[3] = __builtin_amdgcn_alignbit(e, v.w, sh);
#else
    memcpy(w, p, 16);
#endif
}

template <int T>
__host__ __device__ inline void frag_load(const uint8_t* blk, int q, uint32_t* r) {
    const int qq = (q + 3) & 3;
    if constexpr (T == T_Q4_K) {
        frag_ld128(blk, r);                             // d, dmin, scales[12]
        frag_ld128(blk + 16 + 16 * qq, r + 4);          // qs bytes 16qq .. +16
        frag_ld128(blk + 80 + 16 * qq, r + 8);          // qs bytes 64 + 16qq .. +16
    } else if constexpr (T == T_Q5_K) {
        frag_ld128(blk, r);                             // d, dmin, scales[12]
        frag_ld128(blk + 16 + 16 * (qq & 1), r + 4);    // qh bytes 16(qq&1) .. +16
        frag_ld128(blk + 48 + 16 * qq, r + 8);          // qs bytes 16qq .. +16
        frag_ld128(blk + 112 + 16 * qq, r + 12);        // qs bytes 64 + 16qq .. +16
    } else if constexpr (T == T_Q6_K) {
        frag_ld128_a2(blk + 16 * qq, r);                   // ql bytes 16qq .. +16
        frag_ld128_a2(blk + 64 + 16 * qq, r + 4);          // ql bytes 64 + 16qq .. +16
        frag_ld128_a2(blk + 128 + 16 * (qq & 1), r + 8);   // qh bytes 16(qq&1) .. +16
        frag_ld128_a2(blk + 160 + 16 * (qq & 1), r + 12);  // qh bytes 32 + 16(qq&1) .. +16
        // (the four reads above end by byte 196, inside the block)
        frag_ld128(blk + 192, r + 16);                  // int8 scales[16]
        r[20] = frag_ld16(blk + 208);                   // d
    } else if constexpr (T == T_Q8_0) {
        // quants 8qq .. 8qq+7 of each of the unit's eight blocks (block m at
        // byte 34m, its quants from byte 34m + 2), then the d of blocks 2qq, 2qq+1
#pragma unroll
        for (int m = 0; m < 8; ++m) frag_ld64(blk + 34 * m + 2 + 8 * qq, r + 2 * m);
        r[16] = frag_ld16(blk + 68 * qq);
        r[17] = frag_ld16(blk + 68 * qq + 34);
    } else {  // Q3_K
        frag_ld128(blk + 32 + 16 * qq, r);              // qs bytes 16qq .. +16
        frag_ld128(blk + 16 * (qq & 1), r + 4);         // hmask bytes 16(qq&1) .. +16
        frag_ld128(blk + 94, r + 8);                    // qs[62..63], scales[12], d: the block's last 16 bytes
    }
}

__host__ __device__ inline h2_t frag_bits_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

// v_perm_b32: byte i of the result is byte sel.byte[i] of the 8-byte value
// {hi = s0, lo = s1} (only selectors 0..7 are used here)
__host__ __device__ inline uint32_t frag_perm(uint32_t s0, uint32_t s1, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_perm(s0, s1, sel);
#else
    const uint64_t v = ((uint64_t)s0 << 32) | s1;
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) r |= (uint32_t)((v >> (8 * ((sel >> (8 * i)) & 7))) & 0xFF) << (8 * i);
    return r;
#endif
}

// The 4 bytes of w as halves 1024 + byte (FP16 1024 has ulp 1, so 0x64 in the
// high byte over the byte value is exact): lo = bytes 0, 1; hi = bytes 2, 3.
__host__ __device__ inline void frag_biased(uint32_t w, h2_t& lo, h2_t& hi) {
    lo = frag_bits_h2(frag_perm(0x64646464u, w, 0x04010400u));
    hi = frag_bits_h2(frag_perm(0x64646464u, w, 0x04030402u));
}

// x rotated right by r (0..31) (v_alignbit_b32 on the device)
__host__ __device__ inline uint32_t frag_rotr(uint32_t x, int r) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_alignbit(x, x, (uint32_t)r);
#else
    return r ? (x >> r) | (x << (32 - r)) : x;
#endif
}

__host__ __device__ inline h2_t frag_splat(_Float16 v) {
    h2_t h;
    h[0] = v;
    h[1] = v;
    return h;
}

// The 4 byte values of w minus `bias` as exact halves (bytes 0, 1 in lo; 2, 3 in hi).
__host__ __device__ inline void frag_bytes_f16(uint32_t w, _Float16 bias, h2_t& lo, h2_t& hi) {
    frag_biased(w, lo, hi);
    const h2_t b = frag_splat((_Float16)(-1024.0f) - bias);
    lo = lo + b;
    hi = hi + b;
}

// Per lane and super-block: the four scales its steps use (and for Q4_K/Q5_K
// the -1024 * scale fma addends) as FP16 pairs; step m takes
// s[m >> 2][(m >> 1) & 1].
template <int T> struct FragPrep { h2_t s[2], c[2]; };

// IP: the Q3_K operand with its quant bits in place (frag_step); the other
// types ignore it.
template <int T, bool IP = true>
__host__ __device__ inline void frag_prep(const uint32_t* r, int q, FragPrep<T>& P) {
    const int qq = (q + 3) & 3;
    if constexpr (T == T_Q8_0) {
        (void)r;   // no sub-block scales: each step's d is applied to its product
        (void)qq;
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        // get_scale_min_k4 (cpp/dequant_k.cpp:166-175): sc0..3 = s[0..3] & 63,
        // sc4..7 = (s[8..11] & 15) | (s[0..3] >> 6) << 4, s = words r[1..3].  Step m
        // is sub-block 4(m >> 2) + 2(qq >> 1) + ((m >> 1) & 1).
        const uint32_t lo4 = r[1] & 0x3F3F3F3Fu;
        const uint32_t hi4 = (r[3] & 0x0F0F0F0Fu) | ((r[1] >> 2) & 0x30303030u);
        const uint32_t sel = (qq >> 1) ? 0x07060302u : 0x05040100u;   // sc 2j, 2j+1, 4+2j, 5+2j
        frag_bytes_f16(frag_perm(hi4, lo4, sel), (_Float16)0.0f, P.s[0], P.s[1]);
        const h2_t k = frag_splat((_Float16)(-1024.0f));
        P.c[0] = P.s[0] * k;   // exact: multiples of 1024 up to 64512
        P.c[1] = P.s[1] * k;
    } else if constexpr (T == T_Q6_K) {
        // int8 scale of step m: 8H + 2S + (qq & 1) with H = m >> 2 and
        // S = 2((m >> 1) & 1) + (qq >> 1), i.e. byte qq + 4((m >> 1) & 1) + 8H of
        // scales[16] (words r[16..19])
        const uint32_t sel = (uint32_t)qq | ((uint32_t)(4 + qq) << 8);
        const uint32_t e0 = frag_perm(r[17], r[16], sel);          // bytes 0, 1: H = 0
        const uint32_t e1 = frag_perm(r[19], r[18], sel << 16);    // bytes 2, 3: H = 1
        const uint32_t e = ((e0 & 0xFFFFu) | (e1 & 0xFFFF0000u)) ^ 0x80808080u;   // int8 + 128
        frag_bytes_f16(e, (_Float16)128.0f, P.s[0], P.s[1]);
    } else {  // Q3_K
        // scale j = 8H + 2S + lo with H = qq >> 1, lo = qq & 1, S = m >> 1
        // (cpp/dequant_k.cpp:285-289): nibble H of scales[2S + lo], | bits
        // 4H + 2(S >> 1) of scales[8 + 2(S & 1) + lo] << 4, minus 32.  The window
        // r[8..11] is block bytes 94..109, so scales[k] is its byte 2 + k.
        const int H = qq >> 1, lo = qq & 1;
        // window bytes 2 + lo, 4 + lo, 6 + lo (r[8..9]), then 8 + lo (r[10])
        const uint32_t t = frag_perm(r[9], r[8], lo ? 0x07070503u : 0x07060402u);
        const uint32_t bytes = frag_perm(r[10], t, lo ? 0x05020100u : 0x04020100u);
        const uint32_t nib = (bytes >> (4 * H)) & 0x0F0F0F0Fu;
        // window bytes 10 + lo, 12 + lo, 10 + lo, 12 + lo (for S = 0..3)
        const uint32_t hb = frag_perm(r[11], r[10], lo ? 0x05030503u : 0x04020402u);
        const uint32_t top = ((hb >> (4 * H)) & 0x00000303u) | ((hb >> (4 * H + 2)) & 0x03030000u);
        frag_bytes_f16(nib | (top << 4), (_Float16)32.0f, P.s[0], P.s[1]);
        if constexpr (!IP) return;
        // run S's operand bytes are F q with F = 1, 4, 16, 16 (frag_step): its
        // scale is taken as sc / F (exact)
        h2_t f0, f1;
        f0[0] = (_Float16)1.0f;
        f0[1] = (_Float16)0.25f;
        f1[0] = (_Float16)0.0625f;
        f1[1] = (_Float16)0.0625f;
        P.s[0] = P.s[0] * f0;
        P.s[1] = P.s[1] * f1;
    }
}

template <int M>
__host__ __device__ inline _Float16 frag_pick(const h2_t* v) { return v[M >> 2][(M >> 1) & 1]; }

// Step M's A operands: a[0] (and a[1] for Q6_K) are exact integers, their sum
// the scaled quants.  The operand against a low-order B plane is a[0] (for
// Q6_K a[0] is sc*q rounded to FP16: its error on a term that is itself 2^-12
// of the result is below FP32 rounding).
template <int T, int M, bool IP = true>
__host__ __device__ inline void frag_step(const uint32_t* r, const FragPrep<T>& P, int q, h8_t* a) {
    const int qq = (q + 3) & 3;
    h2_t p[4];
    if constexpr (T == T_Q8_0) {
        // block M's int8 quants 8qq .. 8qq+7: byte ^ 0x80 = q + 128, a biased
        // half less 1152 is q, exact
        (void)P;
        (void)qq;
        frag_bytes_f16(r[2 * M] ^ 0x80808080u, (_Float16)128.0f, p[0], p[1]);
        frag_bytes_f16(r[2 * M + 1] ^ 0x80808080u, (_Float16)128.0f, p[2], p[3]);
        for (int i = 0; i < 4; ++i) {
            a[0][2 * i] = p[i][0];
            a[0][2 * i + 1] = p[i][1];
        }
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        // qs run M >> 2, bytes 8(M & 1) .. +8, nibble (M >> 1) & 1; the Q5_K fifth
        // bit is qh (same byte index) bit column / 32 = 4(M >> 2) + 2(qq >> 1) + nibble
        constexpr int QW = (T == T_Q4_K ? 4 : 8) + 4 * (M >> 2) + 2 * (M & 1), NIB = (M >> 1) & 1;
        uint32_t b0 = (r[QW] >> (4 * NIB)) & 0x0F0F0F0Fu, b1 = (r[QW + 1] >> (4 * NIB)) & 0x0F0F0F0Fu;
        if constexpr (T == T_Q5_K) {
            const int sh = 4 * (M >> 2) + 2 * (qq >> 1) + NIB;
            b0 |= ((r[4 + 2 * (M & 1)] >> sh) & 0x01010101u) << 4;
            b1 |= ((r[5 + 2 * (M & 1)] >> sh) & 0x01010101u) << 4;
        }
        frag_biased(b0, p[0], p[1]);
        frag_biased(b1, p[2], p[3]);
        // sc * (1024 + q) - 1024 sc = sc * q: exact result, one rounding
        const h2_t s = frag_splat(frag_pick<M>(P.s)), c = frag_splat(frag_pick<M>(P.c));
        for (int i = 0; i < 4; ++i) {
            const h2_t v = __builtin_elementwise_fma(p[i], s, c);
            a[0][2 * i] = v[0];
            a[0][2 * i + 1] = v[1];
        }
    } else if constexpr (T == T_Q6_K) {
        // ql run H = M >> 2, bytes 8(M & 1) .. +8, nibble (M >> 1) & 1; qh run H,
        // same bytes, bits 2S with S = 2((M >> 1) & 1) + (qq >> 1)
        constexpr int LW = 4 * (M >> 2) + 2 * (M & 1), HW = 8 + LW, NIB = (M >> 1) & 1;
        const int sh = 4 * NIB + 2 * (qq >> 1);
        const uint32_t q0 = ((r[LW] >> (4 * NIB)) & 0x0F0F0F0Fu) | (((r[HW] >> sh) & 0x03030303u) << 4);
        const uint32_t q1 = ((r[LW + 1] >> (4 * NIB)) & 0x0F0F0F0Fu) | (((r[HW + 1] >> sh) & 0x03030303u) << 4);
        frag_bytes_f16(q0, (_Float16)32.0f, p[0], p[1]);   // q - 32, exact
        frag_bytes_f16(q1, (_Float16)32.0f, p[2], p[3]);
        // sc * (q - 32) reaches 4096, past FP16's exact integers: hi = its rounding,
        // lo = the exact remainder (|lo| <= 1) from one fused multiply-add
        const h2_t s = frag_splat(frag_pick<M>(P.s));
        for (int i = 0; i < 4; ++i) {
            const h2_t hi = p[i] * s;
            const h2_t lo = __builtin_elementwise_fma(p[i], s, -hi);
            a[0][2 * i] = hi[0];
            a[0][2 * i + 1] = hi[1];
            a[1][2 * i] = lo[0];
            a[1][2 * i + 1] = lo[1];
        }
    } else {  // Q3_K: qs bytes 8(M & 1) .. +8, bits 2(M >> 1); hmask same bytes, bit 4(qq >> 1) + (M >> 1)
        // IP: run S's two quant bits stay at bits 2S, 2S + 1 of every byte (run
        // 3's move down to bits 4, 5) and the mask bit goes to the bit above them
        // by one rotation (right by sh - QS - 2 mod 32 takes byte k's bit sh to
        // bit 8k + QS + 2): the byte is F q with F = 2^QS (<= 112), and frag_prep
        // holds the run's scale as sc / F.  Otherwise q itself, at bits 0..2.
        constexpr int W = 2 * (M & 1), S = M >> 1, QS = IP ? (S == 3 ? 4 : 2 * S) : 0;
        constexpr float F = (float)(1 << QS);
        const int sh = 4 * (qq >> 1) + S, rr = (sh - QS - 2) & 31;
        uint32_t q0, q1;
        if constexpr (IP) {
            const uint32_t l0 = S == 3 ? (r[W] >> 2) & 0x30303030u : r[W] & (0x03030303u << QS);
            const uint32_t l1 = S == 3 ? (r[W + 1] >> 2) & 0x30303030u : r[W + 1] & (0x03030303u << QS);
            q0 = l0 | (frag_rotr(r[4 + W], rr) & (0x04040404u << QS));
            q1 = l1 | (frag_rotr(r[5 + W], rr) & (0x04040404u << QS));
        } else {
            q0 = ((r[W] >> (2 * S)) & 0x03030303u) | (((r[4 + W] >> sh) & 0x01010101u) << 2);
            q1 = ((r[W + 1] >> (2 * S)) & 0x03030303u) | (((r[5 + W] >> sh) & 0x01010101u) << 2);
        }
        frag_bytes_f16(q0, (_Float16)(4.0f * F), p[0], p[1]);     // F (q - 4), exact
        frag_bytes_f16(q1, (_Float16)(4.0f * F), p[2], p[3]);
        const h2_t s = frag_splat(frag_pick<M>(P.s));
        for (int i = 0; i < 4; ++i) {
            const h2_t v = p[i] * s;
            a[0][2 * i] = v[0];
            a[0][2 * i + 1] = v[1];
        }
    }
}

template <int T>
__host__ __device__ inline h8_t frag_lo_operand(const h8_t* a) {
    return a[0];
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
    frag_bytes_f16((q & 1) ? hi4 : lo4, (_Float16)0.0f, p0, p1);
    const h2_t x32 = frag_splat((_Float16)32.0f);
    p0 = p0 * x32;
    p1 = p1 * x32;
    h4_t m;
    m[0] = p0[0];
    m[1] = p0[1];
    m[2] = p1[0];
    m[3] = p1[1];
    return m;
}

// FP16 bits to float
__host__ __device__ inline float frag_h2f(uint32_t bits) {
    _Float16 h;
    const uint16_t b = (uint16_t)bits;
    memcpy(&h, &b, 2);
    return (float)h;
}

// The block's d (and for Q4_K/Q5_K dmin) from its header word
template <int T>
__host__ __device__ inline float frag_d(uint32_t hdr) { return frag_h2f(hdr >> FragGeo<T>::D_SHIFT); }
__host__ __device__ inline float frag_dmin(uint32_t hdr) { return frag_h2f(hdr >> 16); }

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
