// kquant_dot.h -- exact integer dot products of GGUF K-quant chunks with activations.
//
// The decode GEMV reads each weight once, so its cost per weight must be a few
// VALU operations.  Instead of decoding every weight to FP32 and issuing an
// FMA, a lane keeps the activation as three int8 "digits" and multiplies the
// raw quants with v_dot4_i32_i8 (4 MACs per instruction, exact int32 sums):
//
//   activation group of 32 columns, power-of-two scale s = 2^(E-6) with
//   max|x| in [2^(E-1), 2^E):  X = x/s in (-64, 64),
//   x0 = rint(X), x1 = rint((X-x0)*128), x2 = rint(((X-x0)*128-x1)*128),
//   x = s*(x0 + x1/128 + x2/16384) + r,  |r| <= s/32768 <= 2^-20 * max|x|
//
// Every step of the split is exact in FP32, so the only error is r.  The
// sub-block scales of the quant format are applied once per 16-column run:
//   sum_k q_k x_k  ~  (s/16384) * (16384*I0 + 128*I1 + I2),  Ij = sum_k q_k xj_k.
// Quant offsets (Q6_K's -32, Q3_K's -4, Q4_K/Q5_K's -dmin*m) use the exact
// FP32 column sums of the activation instead of more dot products.
//
// A lane works on a 64-weight "chunk" of one 256-weight super-block: four runs
// of 16 consecutive columns, each run four int8 dwords.
//   Q4_K/Q5_K chunk c: runs at columns 64c + {0,16} (low nibbles of qs[32c..])
//                      and 64c + {32,48} (high nibbles); sub-block 2c + (run>=2)
//   Q6_K/Q3_K chunk c: h = c/2, l0 = 16*(c%2); run s at 128h + 32s + l0;
//                      16-value sub-block 8h + 2s + (c%2)
// Column sums and digit scales are per 16 and 32 columns respectively.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kquant_device.h"

namespace mqh {

constexpr int NDIG = 3;             // activation digits
constexpr int CHUNK = 64;           // weights per lane chunk
constexpr int RUNS = 4;             // 16-column runs per chunk

__host__ __device__ inline int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
#else
    for (int i = 0; i < 4; ++i) c += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
    return c;
#endif
}

// Power-of-two digit scale exponent for a group whose max |x| is `amax`:
// returns e with s = 2^e, so that |x / s| < 64.
__host__ __device__ inline int digit_exp(float amax) {
    if (!(amax > 0.0f)) return 0;
    int E;
    (void)frexpf(amax, &E);           // amax = m * 2^E, m in [0.5, 1)
    return E - 6;
}

// Three int8 digits of x for scale exponent e (see the header comment).
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

// Per-lane activation operand for one chunk: digits (12 dwords per digit plane,
// i.e. 4 runs x 4 dwords), the run's digit scale s/16384 and the run's column sum.
struct ChunkX {
    uint32_t d[NDIG][16];
    float xs[RUNS];     // 2^e / 16384 for the run's 32-column group
    float sum[RUNS];    // exact FP32 sum of the run's 16 activation values
};

// Integer part: I = 16384*I0 + 128*I1 + I2 as float, for one run of 4 quant dwords.
__host__ __device__ inline float run_dot(const uint32_t q[4], const ChunkX& x, int run) {
    int32_t i0 = 0, i1 = 0, i2 = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        i0 = sdot4(q[k], x.d[0][4 * run + k], i0);
        i1 = sdot4(q[k], x.d[1][4 * run + k], i1);
        i2 = sdot4(q[k], x.d[2][4 * run + k], i2);
    }
    // |i0| <= 16*127*64 < 2^17, so the combination fits comfortably in int32
    return (float)((i0 << 14) + (i1 << 7) + i2);
}

__host__ __device__ inline uint32_t lo_nib(uint32_t w) { return w & 0x0F0F0F0Fu; }
__host__ __device__ inline uint32_t hi_nib(uint32_t w) { return (w >> 4) & 0x0F0F0F0Fu; }

__host__ __device__ inline float f16_bits_to_f32(uint32_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __half2float(__ushort_as_half((unsigned short)h));
#else
    uint32_t sign = (h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) bits = sign;
        else { int e = 0; while (!(man & 0x400u)) { man <<= 1; ++e; } bits = sign | ((uint32_t)(113 - e) << 23) | ((man & 0x3FFu) << 13); }
    } else if (exp == 31) bits = sign | 0x7F800000u | (man << 13);
    else bits = sign | ((exp + 112u) << 23) | (man << 13);
    float f; __builtin_memcpy(&f, &bits, 4); return f;
#endif
}

__host__ __device__ inline uint32_t byte_at(const uint32_t* w, int i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xFFu; }

// ---------------------------------------------------------------- raw chunks
//
// Raw bytes a lane loads for its chunk; the loads themselves live in the
// kernels (they decide when to issue them).

struct RawQ4K { uint32_t hdr[4]; uint32_t qs[8]; };              // block[0..15], qs[32c..32c+31]
struct RawQ5K { uint32_t hdr[4]; uint32_t qs[8]; uint32_t qh[8]; };
struct RawQ6K { uint32_t ql0[4], ql1[4], qh[4]; uint32_t sc[2]; uint32_t d; };
struct RawQ3K { uint32_t qs[4], hm[4]; uint32_t sc[3]; uint32_t d; };

// Q4_K/Q5_K 6-bit scale and min j from the 12 packed bytes (header dwords
// 1..3).  j is lane-dependent, so bytes are picked with shifts of 64-bit words
// (indexing a register array with it would push the array to scratch memory).
__host__ __device__ inline void k4_scale_min(const uint32_t hdr[4], int j, int& sc, int& mn) {
    const uint64_t lo = (uint64_t)hdr[1] | ((uint64_t)hdr[2] << 32);   // bytes 0..7
    const uint32_t hi = hdr[3];                                        // bytes 8..11
    if (j < 4) {
        sc = (int)((lo >> (8 * j)) & 63);
        mn = (int)((lo >> (8 * j + 32)) & 63);
    } else {
        const int k = j - 4;
        const uint32_t b8 = (hi >> (8 * k)) & 0xFFu;
        sc = (int)((b8 & 15) | (((lo >> (8 * k)) >> 6 & 3) << 4));
        mn = (int)((b8 >> 4) | (((lo >> (8 * j)) >> 6 & 3) << 4));
    }
}

__host__ __device__ inline float chunk_dot_q4k(const RawQ4K& r, int c, const ChunkX& x) {
    const float d = f16_bits_to_f32(r.hdr[0] & 0xFFFFu), dmin = f16_bits_to_f32(r.hdr[0] >> 16);
    float acc = 0.0f, off = 0.0f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {          // half 0: low nibbles, 1: high nibbles
        int sc, mn;
        k4_scale_min(r.hdr, 2 * c + half, sc, mn);
        float s = 0.0f, m = 0.0f;
#pragma unroll
        for (int run = 2 * half; run < 2 * half + 2; ++run) {
            uint32_t q[4];
            const int base = 4 * (run - 2 * half);
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = half ? hi_nib(r.qs[base + k]) : lo_nib(r.qs[base + k]);
            s = fmaf(x.xs[run], run_dot(q, x, run), s);
            m += x.sum[run];
        }
        acc = fmaf((float)sc, s, acc);
        off = fmaf((float)mn, m, off);
    }
    return fmaf(d, acc, -dmin * off);
}

__host__ __device__ inline float chunk_dot_q5k(const RawQ5K& r, int c, const ChunkX& x) {
    const float d = f16_bits_to_f32(r.hdr[0] & 0xFFFFu), dmin = f16_bits_to_f32(r.hdr[0] >> 16);
    float acc = 0.0f, off = 0.0f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int j = 2 * c + half;
        int sc, mn;
        k4_scale_min(r.hdr, j, sc, mn);
        float s = 0.0f, m = 0.0f;
#pragma unroll
        for (int run = 2 * half; run < 2 * half + 2; ++run) {
            uint32_t q[4];
            const int base = 4 * (run - 2 * half);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = half ? hi_nib(r.qs[base + k]) : lo_nib(r.qs[base + k]);
                const uint32_t hb = (r.qh[base + k] >> j) & 0x01010101u;   // qh[l] bit j for the run's columns
                q[k] = lo | (hb << 4);
            }
            s = fmaf(x.xs[run], run_dot(q, x, run), s);
            m += x.sum[run];
        }
        acc = fmaf((float)sc, s, acc);
        off = fmaf((float)mn, m, off);
    }
    return fmaf(d, acc, -dmin * off);
}

__host__ __device__ inline float chunk_dot_q6k(const RawQ6K& r, int c, const ChunkX& x) {
    const float d = f16_bits_to_f32(r.d & 0xFFFFu);
    const int h = c >> 1, odd = c & 1;
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {                  // run s: columns 128h + 32s + l0 + 0..15
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t l = (s & 1) ? r.ql1[k] : r.ql0[k];
            const uint32_t lo = (s >> 1) ? hi_nib(l) : lo_nib(l);
            const uint32_t hi = (r.qh[k] >> (2 * s)) & 0x03030303u;
            q[k] = lo | (hi << 4);                 // 0..63; the -32 is folded below
        }
        // int8 scale of 16-value sub-block 8h + 2s + odd; sc[] holds bytes 8h..8h+7
        const uint64_t sc64 = (uint64_t)r.sc[0] | ((uint64_t)r.sc[1] << 32);
        const int sc = (int)(int8_t)(uint8_t)(sc64 >> (8 * (2 * s + odd)));
        const float dot = fmaf(x.xs[s], run_dot(q, x, s), -32.0f * x.sum[s]);
        acc = fmaf((float)sc, dot, acc);
    }
    (void)h;
    return d * acc;
}

// Q3_K signed 6-bit scale j (0..15): low nibble from byte j%8 (high nibble
// when j >= 8), two high bits from byte 8 + j%4 at shift 2*(j/4).
__host__ __device__ inline int k3_scale(const uint32_t sc[3], int j) {
    const uint64_t lo64 = (uint64_t)sc[0] | ((uint64_t)sc[1] << 32);
    const int lo = (int)((lo64 >> (8 * (j & 7) + 4 * (j >> 3))) & 15);
    const int hi = (int)((sc[2] >> (8 * (j & 3) + 2 * (j >> 2))) & 3);
    return (lo | (hi << 4)) - 32;
}

__host__ __device__ inline float chunk_dot_q3k(const RawQ3K& r, int c, const ChunkX& x) {
    const float d = f16_bits_to_f32(r.d & 0xFFFFu);
    const int h = c >> 1, odd = c & 1;
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = (r.qs[k] >> (2 * s)) & 0x03030303u;
            const uint32_t hb = (r.hm[k] >> (4 * h + s)) & 0x01010101u;
            q[k] = lo | (hb << 2);                 // 0..7 = q + 4
        }
        const int sc = k3_scale(r.sc, 8 * h + 2 * s + odd);
        const float dot = fmaf(x.xs[s], run_dot(q, x, s), -4.0f * x.sum[s]);
        acc = fmaf((float)sc, dot, acc);
    }
    return d * acc;
}

// ------------------------------------------------------ chunk loads and dots

__host__ __device__ inline uint4 ld16(const uint8_t* p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

__host__ __device__ inline uint2 ld8(const uint8_t* p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}

// Raw bytes of one lane chunk.  Sized per type so a phase-A lane can keep
// eight rows of quants in registers; phase B keeps one chunk per slot in the
// widest form (20 dwords) because its slots may differ in type.
template <int T> struct RawOf;
template <> struct RawOf<T_Q4_K> { static constexpr int N = 12; };   // header 16 B + qs 32 B
template <> struct RawOf<T_Q5_K> { static constexpr int N = 20; };   // + qh 32 B
template <> struct RawOf<T_Q6_K> { static constexpr int N = 15; };   // ql 2x16 B, qh 16 B, scales 8 B, d
template <> struct RawOf<T_Q3_K> { static constexpr int N = 12; };   // qs 16 B, hmask 16 B, scales 12 B, d

template <int N>
struct Raw {
    uint32_t w[N];
};

__host__ __device__ inline void put4(uint32_t* w, uint4 v) { w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w; }

// Issue the loads of chunk c of the block at blk into w[0 .. RawOf<T>::N).
template <int T>
__host__ __device__ inline void load_chunk(const uint8_t* blk, int c, uint32_t* w) {
    if constexpr (T == T_Q4_K) {
        put4(w, *(const uint4*)blk);
        put4(w + 4, *(const uint4*)(blk + 16 + 32 * c));
        put4(w + 8, *(const uint4*)(blk + 32 + 32 * c));
    } else if constexpr (T == T_Q5_K) {
        put4(w, *(const uint4*)blk);
        put4(w + 4, *(const uint4*)(blk + 48 + 32 * c));
        put4(w + 8, *(const uint4*)(blk + 64 + 32 * c));
        put4(w + 12, *(const uint4*)(blk + 16));
        put4(w + 16, *(const uint4*)(blk + 32));
    } else if constexpr (T == T_Q6_K) {
        const int h = c >> 1, l0 = 16 * (c & 1);
        put4(w, ld16(blk + 64 * h + l0));
        put4(w + 4, ld16(blk + 64 * h + 32 + l0));
        put4(w + 8, ld16(blk + 128 + 32 * h + l0));
        const uint2 sc = ld8(blk + 192 + 8 * h);
        w[12] = sc.x; w[13] = sc.y;
        w[14] = *(const uint16_t*)(blk + 208);
    } else {  // Q3_K
        const int h = c >> 1, l0 = 16 * (c & 1);
        put4(w, ld16(blk + 32 + 32 * h + l0));
        put4(w + 4, ld16(blk + l0));
        const uint2 sc = ld8(blk + 96);
        w[8] = sc.x; w[9] = sc.y;
        uint32_t sc2;
        __builtin_memcpy(&sc2, blk + 104, 4);
        w[10] = sc2;
        w[11] = *(const uint16_t*)(blk + 108);
    }
}

template <int T>
__host__ __device__ inline float chunk_dot(const uint32_t* w, int c, const ChunkX& x) {
    if constexpr (T == T_Q4_K) {
        RawQ4K q;
        for (int i = 0; i < 4; ++i) q.hdr[i] = w[i];
        for (int i = 0; i < 8; ++i) q.qs[i] = w[4 + i];
        return chunk_dot_q4k(q, c, x);
    } else if constexpr (T == T_Q5_K) {
        RawQ5K q;
        for (int i = 0; i < 4; ++i) q.hdr[i] = w[i];
        for (int i = 0; i < 8; ++i) q.qs[i] = w[4 + i];
        for (int i = 0; i < 8; ++i) q.qh[i] = w[12 + i];
        return chunk_dot_q5k(q, c, x);
    } else if constexpr (T == T_Q6_K) {
        RawQ6K q;
        for (int i = 0; i < 4; ++i) { q.ql0[i] = w[i]; q.ql1[i] = w[4 + i]; q.qh[i] = w[8 + i]; }
        q.sc[0] = w[12]; q.sc[1] = w[13]; q.d = w[14];
        return chunk_dot_q6k(q, c, x);
    } else {
        RawQ3K q;
        for (int i = 0; i < 4; ++i) { q.qs[i] = w[i]; q.hm[i] = w[4 + i]; }
        q.sc[0] = w[8]; q.sc[1] = w[9]; q.sc[2] = w[10]; q.d = w[11];
        return chunk_dot_q3k(q, c, x);
    }
}

__host__ __device__ inline void load_chunk_any(int type, const uint8_t* blk, int c, uint32_t* w) {
    switch (type) {
        case T_Q4_K: load_chunk<T_Q4_K>(blk, c, w); break;
        case T_Q5_K: load_chunk<T_Q5_K>(blk, c, w); break;
        case T_Q6_K: load_chunk<T_Q6_K>(blk, c, w); break;
        default: load_chunk<T_Q3_K>(blk, c, w); break;
    }
}

__host__ __device__ inline float chunk_dot_any(int type, const uint32_t* w, int c, const ChunkX& x) {
    switch (type) {
        case T_Q4_K: return chunk_dot<T_Q4_K>(w, c, x);
        case T_Q5_K: return chunk_dot<T_Q5_K>(w, c, x);
        case T_Q6_K: return chunk_dot<T_Q6_K>(w, c, x);
        default: return chunk_dot<T_Q3_K>(w, c, x);
    }
}

// Column of the first value of run `run` of chunk c, within its super-block.
__host__ __device__ inline int run_col(int type, int c, int run) {
    if (type == T_Q4_K || type == T_Q5_K) return 64 * c + 16 * run;
    return 128 * (c >> 1) + 32 * run + 16 * (c & 1);
}

}  // namespace mqh
