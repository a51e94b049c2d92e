// kquant_device.h -- GGUF K-quant block decoding on gfx950.
//
// Every kernel in this library decodes weights through these functions, so a
// weight value is the same bit pattern in the standalone dequantizer, the
// decode GEMV and the prefill GEMM.  The arithmetic follows the reference
// decoders in cpp/dequant_k.cpp (Q8_0 :146-154, scale/min unpack :166-175,
// Q4_K :182-206, Q5_K :221-240, Q6_K :254-268, Q3_K :278-298):
//
//   Q8_0  y = q * d                          (exact)
//   Q3_K  y = (d * sc) * q                   (exact)
//   Q4_K  y = (d * sc) * q - (dmin * m)      (one rounding, in the subtraction)
//   Q5_K  y = (d * sc) * q - (dmin * m)      (one rounding)
//   Q6_K  y = (d * sc) * q                   (exact: |m_d * sc * q| < 2^23)
//
// Products are written with __fmul_rn/__fsub_rn so the compiler cannot fuse
// them; by the exactness above a fused form would round identically, but the
// explicit form keeps the claim independent of -ffp-contract.
//
// Block bit positions (values i = 0..255 of a 256-value super-block):
//   Q4_K  qs[32*(i/64) + i%32] >> 4*((i/32)&1), sub-block i/32
//   Q5_K  as Q4_K at qs@48, plus bit (i/32) of qh[i%32] as bit 4
//   Q6_K  ql[64h + 32*(s&1) + l] >> 4*(s>>1) | (qh[32h + l] >> 2s & 3) << 4, minus 32,
//         with h = i/128, s = (i/32)%4, l = i%32; scale i/16
//   Q3_K  (qs[32h + l] >> 2s & 3) - 4*(1 - (hmask[l] >> (i/32) & 1)); scale i/16
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mqh {

enum : int { T_Q8_0 = 8, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ4_NL = 20 };
// A resident form of this library, not a GGUF type: Q3_K blocks, byte for byte,
// each in a 112-byte slot (two zero bytes after the 110), so that every block and
// its 16-byte fields start on a 16-byte boundary.  Only the decode kernels take it.
enum : int { T_Q3_K_A112 = 111 };

__host__ __device__ constexpr int block_size(int t) {
    return (t == T_Q8_0 || t == T_IQ4_NL) ? 32 : (t == T_Q3_K || t == T_Q3_K_A112 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K) ? 256 : 0;
}

__host__ __device__ constexpr int block_bytes(int t) {
    return t == T_Q8_0 ? 34 : t == T_Q3_K ? 110 : t == T_Q3_K_A112 ? 112 : t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 210
         : t == T_IQ4_NL ? 18 : 0;
}

// The five types of the reference's dequant_k and moe_quant_expert
// (cpp/dequant_k.cpp:342-348); IQ4_NL is decoded by the device entry points
// only, as the reference decodes it in a library of its own.
__host__ __device__ constexpr bool reference_type(int t) {
    return t == T_Q8_0 || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K;
}

// ------------------------------------------------------------------ loads

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }

// 8 bytes from any byte address (gfx950 global loads tolerate misalignment:
// Q6_K and Q3_K blocks are 210 and 110 bytes, so fields land on 2-byte offsets).
__device__ __forceinline__ uint64_t ld_u64(const uint8_t* p) {
    uint64_t v;
    __builtin_memcpy(&v, p, 8);
    return v;
}

// 16 bytes from any byte address, as four dwords
__device__ __forceinline__ uint4 ld_u128(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

__device__ __forceinline__ float h2f(uint32_t bits) {
    return __half2float(__ushort_as_half((unsigned short)bits));
}

// Opaque copy of f.  Without it the instruction selector folds a product that
// feeds an FP16 conversion into v_fma_mix*_f16 with a +0 addend, and
// (-0) + (+0) = +0 drops the sign of negative-zero results.
__device__ __forceinline__ float opaque(float f) {
    __asm__ volatile("" : "+v"(f));
    return f;
}

__device__ __forceinline__ uint32_t f2h_rn(float f) {
    return (uint32_t)__half_as_ushort(__float2half_rn(opaque(f)));
}

// two values rounded to FP16 (RNE), packed low then high: one v_cvt_pk_f16_f32
__device__ __forceinline__ uint32_t pack_f2h_rn(float lo, float hi) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {opaque(lo), opaque(hi)};
    const f16x2 h = __builtin_convertvector(v, f16x2);
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ float round16(float f) { return __half2float(__float2half_rn(opaque(f))); }

// byte k of a 64-bit word
__device__ __forceinline__ uint32_t byte_of(uint64_t w, int k) { return (uint32_t)(w >> (8 * k)) & 0xFFu; }

// byte k (a compile-time 0..3) of w as a float: one v_cvt_f32_ubyte<k>
template <int k>
__device__ __forceinline__ float ubyte_f(uint32_t w) { return (float)((w >> (8 * k)) & 0xFFu); }

// out[4 * half + k] = f(byte k of w[half]) for the 8 bytes of two dwords
template <class F>
__device__ __forceinline__ void per_byte8(uint32_t w0, uint32_t w1, float out[8], F&& f) {
    out[0] = f(ubyte_f<0>(w0)); out[1] = f(ubyte_f<1>(w0)); out[2] = f(ubyte_f<2>(w0)); out[3] = f(ubyte_f<3>(w0));
    out[4] = f(ubyte_f<0>(w1)); out[5] = f(ubyte_f<1>(w1)); out[6] = f(ubyte_f<2>(w1)); out[7] = f(ubyte_f<3>(w1));
}

// ---------------------------------------------------- 8 consecutive values
//
// decode8<T>(blk, t, out): values 8t .. 8t+7 of the block at blk, as FP32,
// bit-identical to the reference decoders.  t ranges over block_size(T)/8.

template <int T>
__device__ __forceinline__ void decode8(const uint8_t* blk, int t, float out[8]);

template <>
__device__ __forceinline__ void decode8<T_Q8_0>(const uint8_t* blk, int t, float out[8]) {
    const float d = h2f(ld_u16(blk));
    const uint64_t w = ld_u64(blk + 2 + 8 * t);
#pragma unroll
    for (int k = 0; k < 8; ++k) out[k] = __fmul_rn((float)(int8_t)byte_of(w, k), d);
}

// IQ4_NL: an FP16 scale, then 16 bytes of 4-bit indices into a 16-entry table;
// values 0..15 are the low nibbles of bytes 0..15, values 16..31 the high
// nibbles, each scale * table[index] rounded once (cpp/fast_dequant.cpp:40-65,
// fast_dequant_avx2.cpp:80-97).  The table is the reference's own constants
// (fast_dequant.cpp:4-9), which are not gguf's kvalues_iq4nl / 127: the output
// follows the reference library this replaces.
__host__ __device__ constexpr float IQ4NL_TABLE[16] = {
    -1.0f, -0.6961914f, -0.515625f, -0.375f, -0.25390625f, -0.1484375f, -0.0546875f, 0.02734375f,
    0.1015625f, 0.1796875f, 0.265625f, 0.359375f, 0.46875f, 0.59765625f, 0.7578125f, 1.0f};

// Table lookups in registers.  Every entry's low 16 bits are zero except
// entry 1's (0x3999), so an entry is its two high bytes, each found for four
// indices at once with v_perm_b32 over the 8 bytes of entries 0..7 and of
// entries 8..15 (index bit 3 picks between the two), plus that one fix-up.
// IQ4NL_BYTES(first, shift): byte `shift` of entries first .. first+3.
__host__ __device__ constexpr uint32_t iq4nl_bytes(int first, int shift) {
    uint32_t w = 0;
    for (int i = 0; i < 4; ++i)
        w |= ((__builtin_bit_cast(uint32_t, IQ4NL_TABLE[first + i]) >> (8 * shift)) & 0xFFu) << (8 * i);
    return w;
}

// (byte `shift` of table[n_i]) for the four nibbles n_i held one per byte of u
template <int SHIFT>
__device__ __forceinline__ uint32_t iq4nl_byte4(uint32_t u, uint32_t sel, uint32_t hi_mask) {
    const uint32_t lo = __builtin_amdgcn_perm(iq4nl_bytes(4, SHIFT), iq4nl_bytes(0, SHIFT), sel);
    const uint32_t hi = __builtin_amdgcn_perm(iq4nl_bytes(12, SHIFT), iq4nl_bytes(8, SHIFT), sel);
    return (hi & hi_mask) | (lo & ~hi_mask);
}

// table[n] for the four nibbles of u (one per byte), scaled by d
__device__ __forceinline__ void iq4nl_decode4(uint32_t u, float d, float out[4]) {
    const uint32_t sel = u & 0x07070707u;
    const uint32_t hi_mask = ((u >> 3) & 0x01010101u) * 0xFFu;
    const uint32_t b3 = iq4nl_byte4<3>(u, sel, hi_mask), b2 = iq4nl_byte4<2>(u, sel, hi_mask);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // bytes 3, 2 of the entry from b3, b2 (byte k of each), bytes 1, 0 zero
        const uint32_t bits = __builtin_amdgcn_perm(b3, b2, 0x0C0Cu | ((uint32_t)k << 16) | ((uint32_t)(4 + k) << 24));
        const uint32_t lo16 = ((u >> (8 * k)) & 0xFFu) == 1u ? (__builtin_bit_cast(uint32_t, IQ4NL_TABLE[1]) & 0xFFFFu) : 0u;
        out[k] = __fmul_rn(d, __uint_as_float(bits | lo16));
    }
}

template <>
__device__ __forceinline__ void decode8<T_IQ4_NL>(const uint8_t* blk, int t, float out[8]) {
    const float d = h2f(ld_u16(blk));
    const uint64_t w = ld_u64(blk + 2 + 8 * (t & 1));
    const int sh = 4 * (t >> 1);
    iq4nl_decode4(((uint32_t)w >> sh) & 0x0F0F0F0Fu, d, out);
    iq4nl_decode4(((uint32_t)(w >> 32) >> sh) & 0x0F0F0F0Fu, d, out + 4);
}

// Scale and min j (0..7) of Q4_K/Q5_K from header dwords h1..h3 (scale bytes
// 0..11), the same bits as scale_min_k4, without per-byte loads.
__device__ __forceinline__ void scale_min_k4_regs(uint32_t h1, uint32_t h2, uint32_t h3, int j, int& sc, int& mn) {
    const int sh = 8 * (j & 3);
    const uint32_t a = (h1 >> sh) & 0xFFu, b = (h2 >> sh) & 0xFFu, c = (h3 >> sh) & 0xFFu;
    sc = j < 4 ? (int)(a & 63u) : (int)((c & 0x0Fu) | ((a >> 6) << 4));
    mn = j < 4 ? (int)(b & 63u) : (int)((c >> 4) | ((b >> 6) << 4));
}

template <>
__device__ __forceinline__ void decode8<T_Q4_K>(const uint8_t* blk, int t, float out[8]) {
    const int j = t >> 2;                       // sub-block 0..7
    const int g = t >> 3, hi = (t >> 2) & 1, lq = 8 * (t & 3);
    const uint4 h = ld_u128(blk);               // d, dmin, 12 scale bytes: one load
    const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
    int sc, mn;
    scale_min_k4_regs(h.y, h.z, h.w, j, sc, mn);
    const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
    const uint64_t w = ld_u64(blk + 16 + 32 * g + lq);
    const uint32_t u0 = ((uint32_t)w >> (4 * hi)) & 0x0F0F0F0Fu, u1 = ((uint32_t)(w >> 32) >> (4 * hi)) & 0x0F0F0F0Fu;
    per_byte8(u0, u1, out, [&](float q) { return __fsub_rn(__fmul_rn(d1, q), m1); });
}

template <>
__device__ __forceinline__ void decode8<T_Q5_K>(const uint8_t* blk, int t, float out[8]) {
    const int j = t >> 2;
    const int g = t >> 3, hi = (t >> 2) & 1, lq = 8 * (t & 3);
    const uint4 h = ld_u128(blk);
    const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
    int sc, mn;
    scale_min_k4_regs(h.y, h.z, h.w, j, sc, mn);
    const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
    const uint64_t lo = ld_u64(blk + 48 + 32 * g + lq);
    const uint64_t hb = ld_u64(blk + 16 + lq);
    const uint32_t u0 = (((uint32_t)lo >> (4 * hi)) & 0x0F0F0F0Fu) | ((((uint32_t)hb >> j) & 0x01010101u) << 4);
    const uint32_t u1 =
        (((uint32_t)(lo >> 32) >> (4 * hi)) & 0x0F0F0F0Fu) | ((((uint32_t)(hb >> 32) >> j) & 0x01010101u) << 4);
    per_byte8(u0, u1, out, [&](float q) { return __fsub_rn(__fmul_rn(d1, q), m1); });
}

template <>
__device__ __forceinline__ void decode8<T_Q6_K>(const uint8_t* blk, int t, float out[8]) {
    const int h = t >> 4, s = (t >> 2) & 3, lq = 8 * (t & 3);
    const float d = h2f(ld_u16(blk + 208));
    const float ds = __fmul_rn(d, (float)(int8_t)blk[192 + (t >> 1)]);
    const uint64_t lo = ld_u64(blk + 64 * h + 32 * (s & 1) + lq);
    const uint64_t hq = ld_u64(blk + 128 + 32 * h + lq);
    const int sl = 4 * (s >> 1), sh = 2 * s;
    // q + 32 in each byte (0..63); q = that - 32, exact in FP32
    const uint32_t u0 = (((uint32_t)lo >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)hq >> sh) & 0x03030303u) << 4);
    const uint32_t u1 = (((uint32_t)(lo >> 32) >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)(hq >> 32) >> sh) & 0x03030303u) << 4);
    per_byte8(u0, u1, out, [&](float u) { return __fmul_rn(ds, u - 32.0f); });
}

template <>
__device__ __forceinline__ void decode8<T_Q3_K>(const uint8_t* blk, int t, float out[8]) {
    const int h = t >> 4, s = (t >> 2) & 3, lq = 8 * (t & 3);
    // bytes 94..109: two quant bytes, the 12 scale bytes, d.  A 16-byte load
    // that is not dword aligned is slow, and every other block starts 2 bytes
    // off a dword: read the 16 bytes at the dword at or below byte 94 (from
    // byte 92 at the latest, inside the block) and bytes 108..109 on their own,
    // then shift down by 0 or 16 bits.
    const uintptr_t a = (uintptr_t)(blk + 94);
    // (pointer arithmetic, not an integer cast, so an LDS source stays an LDS read)
    const uint4 w = *(const uint4*)(blk + 94 - (a & 3));
    const uint32_t d16 = ld_u16(blk + 108);
    const bool mis = (a & 3) != 0;
    uint4 v;
    v.x = mis ? __builtin_amdgcn_alignbit(w.y, w.x, 16) : w.x;
    v.y = mis ? __builtin_amdgcn_alignbit(w.z, w.y, 16) : w.y;
    v.z = mis ? __builtin_amdgcn_alignbit(w.w, w.z, 16) : w.z;
    v.w = mis ? ((w.w >> 16) | (d16 << 16)) : w.w;
    const uint32_t s0 = __builtin_amdgcn_alignbit(v.y, v.x, 16);   // scale bytes 0..3
    const uint32_t s1 = __builtin_amdgcn_alignbit(v.z, v.y, 16);   // 4..7
    const uint32_t s2 = __builtin_amdgcn_alignbit(v.w, v.z, 16);   // 8..11
    const float d = h2f(v.w >> 16);
    const int j = t >> 1;
    const uint64_t lo64 = (uint64_t)s0 | ((uint64_t)s1 << 32);
    const int sc = (int)(((lo64 >> (8 * (j & 7) + 4 * (j >> 3))) & 15u) |
                         (((s2 >> (8 * (j & 3) + 2 * (j >> 2))) & 3u) << 4)) - 32;
    const float ds = __fmul_rn(d, (float)sc);
    const uint64_t lo = ld_u64(blk + 32 + 32 * h + lq);
    const uint64_t hm = ld_u64(blk + lq);
    const int hb = t >> 2;
    // q + 4 in each byte: the two low bits, plus 4 when the hmask bit is set
    // (q = low - 4 when it is clear, dequant_k.cpp:292-294); q = that - 4, exact
    const uint32_t u0 = (((uint32_t)lo >> (2 * s)) & 0x03030303u) | ((((uint32_t)hm >> hb) & 0x01010101u) << 2);
    const uint32_t u1 =
        (((uint32_t)(lo >> 32) >> (2 * s)) & 0x03030303u) | ((((uint32_t)(hm >> 32) >> hb) & 0x01010101u) << 2);
    per_byte8(u0, u1, out, [&](float u) { return __fmul_rn(ds, u - 4.0f); });
}

// ---------------------------------------------------- 16 consecutive values
//
// decode16<T>(blk, t, out): values 8t .. 8t+15 of the block at blk (t even),
// bit-identical to decode8<T>(blk, t, out) then decode8<T>(blk, t + 1, out + 8).
// The two groups share one sub-block, so the header and scale work is done
// once.  blk is an LDS block in its slot (slot_bytes/slot_offset below): every
// 16-byte read is 16-byte aligned, which LDS serves without the stall of an
// unaligned wide read, and the slot's padding after the block is readable.
//
// The signed-quant types (Q3_K, Q6_K, Q8_0) put each quant q, times a power of
// two 2^e, in the top bits of a byte, as an int8: one sign-extending byte
// conversion (v_cvt_f32_i32 with an SDWA byte operand) yields 2^e q as a float
// and the scale s is divided by 2^e once.  Both steps are exact -- these scales
// are an FP16 value times a small integer, so when not zero they are at least
// 2^-24 in magnitude, far from FP32's subnormal range -- hence
// RN((s / 2^e) (2^e q)) = RN(s q) bit for bit, signed zeros, infinities and
// NaNs included.

// LDS slot of one block: slot_bytes(T), a multiple of 16, with the block at
// byte slot_offset(T), placed so that the 16-byte fields decode16 reads (the
// quants, the Q3_K scales) start on 16-byte boundaries.
__host__ __device__ constexpr int slot_bytes(int t) {
    return t == T_Q8_0 ? 48 : t == T_IQ4_NL ? 32 : t == T_Q3_K ? 112 : t == T_Q6_K ? 224 : block_bytes(t);
}
__host__ __device__ constexpr int slot_offset(int t) { return (t == T_Q8_0 || t == T_IQ4_NL) ? 14 : 0; }

// w rotated right by n (mod 32) bits: one v_alignbit_b32
__device__ __forceinline__ uint32_t rotr32(uint32_t w, uint32_t n) { return __builtin_amdgcn_alignbit(w, w, n); }

// byte k (a compile-time 0..3) of w as a signed integer, as a float
template <int k>
__device__ __forceinline__ float sbyte_f(uint32_t w) { return (float)(int32_t)(int8_t)(w >> (8 * k)); }

// out[4 i + k] = RN(s * (int8) byte k of w[i]) for the 16 bytes of w
__device__ __forceinline__ void scale_sbytes16(const uint32_t w[4], float s, float out[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[4 * i + 0] = __fmul_rn(s, sbyte_f<0>(w[i]));
        out[4 * i + 1] = __fmul_rn(s, sbyte_f<1>(w[i]));
        out[4 * i + 2] = __fmul_rn(s, sbyte_f<2>(w[i]));
        out[4 * i + 3] = __fmul_rn(s, sbyte_f<3>(w[i]));
    }
}

template <int T>
__device__ __forceinline__ void decode16(const uint8_t* blk, int t, float out[16]) {
    if constexpr (T == T_Q8_0) {
        const float d = h2f(ld_u16(blk));
        const uint4 q = *(const uint4*)(blk + 2 + 8 * t);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        scale_sbytes16(w, d, out);
    } else if constexpr (T == T_Q6_K) {
        const int h = t >> 4, s = (t >> 2) & 3, lq = 8 * (t & 3);
        const float d = h2f(ld_u16(blk + 208));
        // q = u - 32 for the 6-bit u; its 6-bit two's complement is u ^ 32, which
        // sits in bits 2..7 of the byte, so the byte is 4q as an int8
        const float ds4 = __fmul_rn(d, (float)(int8_t)blk[192 + (t >> 1)]) * 0.25f;
        const uint4 lo = *(const uint4*)(blk + 64 * h + 32 * (s & 1) + lq);
        const uint4 hq = *(const uint4*)(blk + 128 + 32 * h + lq);
        const uint32_t ra = (30 + 4 * (s >> 1)) & 31;   // low nibble field -> bits 2..5
        const uint32_t rb = (26 + 2 * s) & 31;          // 2-bit high field -> bits 6..7
        const uint32_t l[4] = {lo.x, lo.y, lo.z, lo.w}, hh[4] = {hq.x, hq.y, hq.z, hq.w};
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = ((rotr32(l[i], ra) & 0x3C3C3C3Cu) | (rotr32(hh[i], rb) & 0xC0C0C0C0u)) ^ 0x80808080u;
        scale_sbytes16(w, ds4, out);
    } else if constexpr (T == T_Q3_K) {
        const int h = t >> 4, s = (t >> 2) & 3, lq = 8 * (t & 3), j = t >> 1, hb = t >> 2;
        // bytes 96..111: the 12 scale bytes, d, two bytes of slot padding
        const uint4 v = *(const uint4*)(blk + 96);
        const float d = h2f(v.w & 0xFFFFu);
        // 6-bit scale j: low nibble j & 7 of bytes 0..7 (high nibble for j >= 8),
        // high two bits from bytes 8..11 (dequant_k.cpp scale layout)
        const uint32_t lw = (j & 4) ? v.y : v.x;
        const int sc = (int)(__builtin_amdgcn_ubfe(lw, 8 * (j & 3) + 4 * (j >> 3), 4) |
                             (__builtin_amdgcn_ubfe(v.z, 8 * (j & 3) + 2 * (j >> 2), 2) << 4)) - 32;
        const float ds32 = __fmul_rn(d, (float)sc) * 0.03125f;
        // q = low - 4 when the hmask bit is clear, low when set: the 3-bit two's
        // complement (~hbit, low1, low0), placed in bits 7..5, so the byte is 32q
        const uint4 lo = *(const uint4*)(blk + 32 + 32 * h + lq);
        const uint4 hm = *(const uint4*)(blk + lq);
        const uint32_t ra = (27 + 2 * s) & 31;   // 2-bit field -> bits 5..6
        const uint32_t rb = (25 + hb) & 31;      // hmask bit -> bit 7
        const uint32_t l[4] = {lo.x, lo.y, lo.z, lo.w}, m[4] = {hm.x, hm.y, hm.z, hm.w};
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (rotr32(l[i], ra) & 0x60606060u) | (~rotr32(m[i], rb) & 0x80808080u);
        scale_sbytes16(w, ds32, out);
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const int j = t >> 2, g = t >> 3, hi = (t >> 2) & 1, lq = 8 * (t & 3);
        const uint4 h = *(const uint4*)blk;
        const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
        int sc, mn;
        scale_min_k4_regs(h.y, h.z, h.w, j, sc, mn);
        const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
        const uint32_t sh = 4 * hi;
        auto f = [&](float q) { return __fsub_rn(__fmul_rn(d1, q), m1); };
        if constexpr (T == T_Q4_K) {
            const uint4 q = *(const uint4*)(blk + 16 + 32 * g + lq);
            per_byte8((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu, out, f);
            per_byte8((q.z >> sh) & 0x0F0F0F0Fu, (q.w >> sh) & 0x0F0F0F0Fu, out + 8, f);
        } else {
            const uint4 lo = *(const uint4*)(blk + 48 + 32 * g + lq);
            const uint4 hb = *(const uint4*)(blk + 16 + lq);
            const uint32_t rb = (28 + j) & 31;   // high bit j -> bit 4
            auto u = [&](uint32_t l, uint32_t m) { return ((l >> sh) & 0x0F0F0F0Fu) | (rotr32(m, rb) & 0x10101010u); };
            per_byte8(u(lo.x, hb.x), u(lo.y, hb.y), out, f);
            per_byte8(u(lo.z, hb.z), u(lo.w, hb.w), out + 8, f);
        }
    } else {
        decode8<T>(blk, t, out);
        decode8<T>(blk, t + 1, out + 8);
    }
}

// Runtime-type dispatch; `type` is uniform across the wavefront, so the
// branch does not diverge.
__device__ __forceinline__ void decode8_any(int type, const uint8_t* blk, int t, float out[8]) {
    switch (type) {
        case T_Q8_0: decode8<T_Q8_0>(blk, t, out); break;
        case T_IQ4_NL: decode8<T_IQ4_NL>(blk, t, out); break;
        case T_Q3_K: decode8<T_Q3_K>(blk, t, out); break;
        case T_Q4_K: decode8<T_Q4_K>(blk, t, out); break;
        case T_Q5_K: decode8<T_Q5_K>(blk, t, out); break;
        default:     decode8<T_Q6_K>(blk, t, out); break;
    }
}

// ------------------------------------------------------------ reductions

// Sum over aligned groups of `width` lanes (width a power of two <= 64);
// every lane of the group receives the group total.  Fixed butterfly order,
// so the result is deterministic.
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace mqh
