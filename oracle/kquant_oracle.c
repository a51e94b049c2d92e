/*
 * kquant_oracle.c -- CPU oracle for the quantized-expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in intel-optimized-moe-streaming_amd/.  Only tests/, the smoke entry
 * point and bench.py's CPU-baseline leg may load it; the product path never
 * does, and the HIP library never falls back to it.
 *
 * It is a plain-C restatement of the reference's CPU kernels:
 *   - cpp/dequant_k.cpp          (f16<->f32 conversion, the five block
 *                                 decoders, the dequant_k export contract)
 *   - cpp/moe_quant_dot.cpp      (quant_dot's 8-lane FMA order, the fused
 *                                 SwiGLU expert with its FP16-graph rounding
 *                                 points, validation and status codes)
 * Bit positions are written in closed form (derived from the GGUF block
 * layouts), not copied from cpp/dequant_k_tables.h; tests/test_oracle_pin.py
 * checks them against those tables by one-bit probes when the reference tree
 * is present, and against an independent NumPy restatement of gguf.quants.
 *
 * Arithmetic notes (why the results are bit-exact and order-insensitive):
 *   every decoded weight is an f16 scale (11-bit significand) times integers
 *   whose product stays below 2^24, so it is exact in FP32; Q4_K and Q5_K then
 *   subtract an exact dmin*m term, which rounds once.  The FP16 output is
 *   RN_f16 of that FP32 value, exactly as dequant_k.cpp:324-340 produces it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK_K 256
enum { T_Q8_0 = 8, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

/* ---------------------------------------------- f16 <-> f32 (dequant_k.cpp:49-111) */

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal half: normalise the significand into an FP32 normal */
            int e = 0;
            while ((man & 0x400u) == 0) { man <<= 1; ++e; }
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(113 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Round-to-nearest-even FP32 -> FP16 with subnormals and overflow to inf. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t e32 = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (e32 == 0xFFu)
        return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0u));
    int32_t e = (int32_t)e32 - 112;           /* biased half exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t full = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t q = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);        /* q may carry into the exponent: correct */
    }
    uint32_t q = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) {
        ++q;
        if (q == 0x400u) { q = 0; ++e; if (e >= 31) return (uint16_t)(sign | 0x7C00u); }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | q);
}

void oracle_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_f16(src[i]);
}

void oracle_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f16_to_f32(src[i]);
}

static inline float round16(float x) { return oracle_f16_to_f32(oracle_f32_to_f16(x)); }

static inline float ld_f16(const uint8_t* p) { return oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ---------------------------------------------------------- block decoders */

/* Q8_0, 34 B: f16 d, int8 qs[32]; y = qs*d.  (dequant_k.cpp:146-154) */
static void dec_q8_0(const uint8_t* blk, float* out) {
    const float d = ld_f16(blk);
    for (int j = 0; j < 32; ++j) out[j] = (float)(int8_t)blk[2 + j] * d;
}

/* 6-bit scale/min pairs shared by Q4_K and Q5_K.  (dequant_k.cpp:166-175) */
static void scale_min_k4(const uint8_t* s, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K, 144 B: d@0 dmin@2 scales@4 qs[128]@16.  Group g of 64 outputs reads
 * qs[32g..32g+31]: low nibbles -> outputs 64g..64g+31 (sub-block 2g), high
 * nibbles -> 64g+32.. (sub-block 2g+1).  y = (d*sc)*q - dmin*m.
 * (dequant_k.cpp:182-206) */
static void dec_q4_k(const uint8_t* blk, float* out) {
    const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
    const uint8_t* qs = blk + 16;
    for (int g = 0; g < 4; ++g) {
        int sc0, m0, sc1, m1;
        scale_min_k4(blk + 4, 2 * g, &sc0, &m0);
        scale_min_k4(blk + 4, 2 * g + 1, &sc1, &m1);
        const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
        const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) {
            out[64 * g + l] = d0 * (float)(qs[32 * g + l] & 15) - mm0;
            out[64 * g + 32 + l] = d1 * (float)(qs[32 * g + l] >> 4) - mm1;
        }
    }
}

/* Q5_K, 176 B: d@0 dmin@2 scales@4 qh[32]@16 qs[128]@48.  Output i takes its
 * low 4 bits from qs[32*(i/64) + i%32] >> (4*((i/32)&1)) and its 5th bit from
 * qh[i%32] >> (i/32).  y = (d*sc[i/32])*q - dmin*m[i/32].
 * (dequant_k.cpp:221-240 with the Q5_K maps of dequant_k_tables.h:29-36) */
static void dec_q5_k(const uint8_t* blk, float* out) {
    const float d = ld_f16(blk), dmin = ld_f16(blk + 2);
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    for (int i = 0; i < QK_K; ++i) {
        int sc, mn;
        scale_min_k4(blk + 4, i >> 5, &sc, &mn);
        const int lo = (qs[32 * (i >> 6) + (i & 31)] >> (4 * ((i >> 5) & 1))) & 15;
        const int hi = (qh[i & 31] >> (i >> 5)) & 1;
        const int q = lo | (hi << 4);
        out[i] = d * (float)sc * (float)q - dmin * (float)mn;
    }
}

/* Q6_K, 210 B: ql[128]@0 qh[64]@128 int8 sc[16]@192 d@208.  For output i with
 * h=i/128, s=(i%128)/32, l=i%32: low nibble of ql[64h + 32*(s&1) + l] >> 4*(s>>1),
 * two high bits qh[32h + l] >> 2s.  q = (lo | hi<<4) - 32, y = (d*sc[i/16])*q.
 * (dequant_k.cpp:254-268 with dequant_k_tables.h:24-27) */
static void dec_q6_k(const uint8_t* blk, float* out) {
    const float d = ld_f16(blk + 208);
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int i = 0; i < QK_K; ++i) {
        const int h = i >> 7, s = (i >> 5) & 3, l = i & 31;
        const int lo = (blk[64 * h + 32 * (s & 1) + l] >> (4 * (s >> 1))) & 15;
        const int hi = (blk[128 + 32 * h + l] >> (2 * s)) & 3;
        const int q = (lo | (hi << 4)) - 32;
        out[i] = d * (float)sc[i >> 4] * (float)q;
    }
}

/* Q3_K, 110 B: hmask[32]@0 qs[64]@32 scales[12]@96 d@108.  For output i with
 * h=i/128, s=(i%128)/32, l=i%32: two low bits qs[32h + l] >> 2s, mask bit
 * hmask[l] >> (i/32); q = lo - 4*(1-bit).  Scale j (16 of them, 6-bit signed):
 * low nibble from s[j] (j<8) or s[j-8]>>4, two high bits s[8 + j%4] >> 2*(j/4).
 * y = (d*scale[i/16])*q.  (dequant_k.cpp:278-298 with dequant_k_tables.h:19-22) */
static void dec_q3_k(const uint8_t* blk, float* out) {
    const uint8_t* s = blk + 96;
    const float d = ld_f16(blk + 108);
    int scale[16];
    for (int j = 0; j < 16; ++j) {
        const int lo = (j < 8) ? (s[j] & 15) : ((s[j - 8] >> 4) & 15);
        const int hi = (s[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
        scale[j] = (lo | (hi << 4)) - 32;
    }
    for (int i = 0; i < QK_K; ++i) {
        const int h = i >> 7, sh = (i >> 5) & 3, l = i & 31;
        const int lo = (blk[32 + 32 * h + l] >> (2 * sh)) & 3;
        const int bit = (blk[l] >> (i >> 5)) & 1;
        out[i] = d * (float)scale[i >> 4] * (float)(lo - ((bit ^ 1) << 2));
    }
}

/* ------------------------------------------------------------------ dispatch */

int oracle_block_size(int type) {
    switch (type) {
        case T_Q8_0: return 32;
        case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: return QK_K;
        default: return 0;
    }
}

int oracle_bytes_per_block(int type) {
    switch (type) {
        case T_Q8_0: return 34;
        case T_Q3_K: return 110;
        case T_Q4_K: return 144;
        case T_Q5_K: return 176;
        case T_Q6_K: return 210;
        default: return 0;
    }
}

static int decode_block(int type, const uint8_t* blk, float* out) {
    switch (type) {
        case T_Q8_0: dec_q8_0(blk, out); return 1;
        case T_Q3_K: dec_q3_k(blk, out); return 1;
        case T_Q4_K: dec_q4_k(blk, out); return 1;
        case T_Q5_K: dec_q5_k(blk, out); return 1;
        case T_Q6_K: dec_q6_k(blk, out); return 1;
        default: return 0;
    }
}

int oracle_decode_block(int type, const uint8_t* blk, float* out) { return decode_block(type, blk, out); }

int oracle_dequant_k_supported(int type) { return oracle_block_size(type) != 0; }
int oracle_dequant_k_block_size(int type) { return oracle_block_size(type); }

/* dequant_k contract (dequant_k.cpp:350-394): 0 on success; -1 for an unknown
 * type, a null pointer, n <= 0 or n not a multiple of the block size.  The
 * FP16 output is the RNE conversion of the FP32 decode, block by block. */
int oracle_dequant_k(int type, const uint8_t* src, void* dst, int64_t n, int want_f16) {
    const int bs = oracle_block_size(type), pb = oracle_bytes_per_block(type);
    if (bs == 0 || src == NULL || dst == NULL) return -1;
    if (n <= 0 || n % bs != 0) return -1;
    const int64_t nb = n / bs;
    float tmp[QK_K];
    for (int64_t b = 0; b < nb; ++b) {
        if (want_f16) {
            decode_block(type, src + b * pb, tmp);
            uint16_t* o = (uint16_t*)dst + b * bs;
            for (int j = 0; j < bs; ++j) o[j] = oracle_f32_to_f16(tmp[j]);
        } else {
            decode_block(type, src + b * pb, (float*)dst + b * bs);
        }
    }
    return 0;
}

/* ----------------------------------------------- fused expert (moe_quant_dot) */

/* One row . x with the reference accumulation order (moe_quant_dot.cpp:143-169):
 * lane k of 8 accumulates the values whose column is == k (mod 8) with fused
 * multiply-adds in column order; the 8 lanes are then summed serially.  With
 * round_w the decoded weight is rounded to FP16 before its FMA. */
static float quant_dot(int type, const uint8_t* row, const float* x, int cols, int round_w) {
    const int bs = oracle_block_size(type), pb = oracle_bytes_per_block(type);
    float tmp[QK_K];
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int off = 0; off < cols; off += bs, row += pb) {
        decode_block(type, row, tmp);
        for (int j = 0; j < bs; j += 8) {
            for (int k = 0; k < 8; ++k) {
                const float w = round_w ? round16(tmp[j + k]) : tmp[j + k];
                lanes[k] = fmaf(w, x[off + j + k], lanes[k]);
            }
        }
    }
    float r = 0.0f;
    for (int k = 0; k < 8; ++k) r += lanes[k];
    return r;
}

/* The fused SwiGLU expert of moe_quant_expert (moe_quant_dot.cpp:171-214) over
 * a given row dot: its validation, its FP16-graph rounding points and its
 * status codes (listed at oracle_moe_quant_expert below). */
typedef float (*row_dot_fn)(int type, const uint8_t* row, const float* x, int cols, int round_w);

static int expert_with(row_dot_fn quant_dot, int gate_type, const uint8_t* gate, int64_t gate_bytes,
                       int up_type, const uint8_t* up, int64_t up_bytes,
                       int down_type, const uint8_t* down, int64_t down_bytes,
                       const float* input, int hidden, int intermediate, float* output, int fp16_graph) {
    const int types[3] = {gate_type, up_type, down_type};
    const int cols[3] = {hidden, hidden, intermediate};
    const int rows[3] = {intermediate, intermediate, hidden};
    const int64_t sizes[3] = {gate_bytes, up_bytes, down_bytes};
    if (!gate || !up || !down || !input || !output || hidden <= 0 || intermediate <= 0 ||
        hidden > 65536 || intermediate > 65536 || (fp16_graph != 0 && fp16_graph != 1))
        return -1;
    for (int i = 0; i < 3; ++i) {
        const int bs = oracle_block_size(types[i]);
        if (!bs || cols[i] % bs) return -2;
        const int64_t want = (int64_t)rows[i] * (cols[i] / bs) * oracle_bytes_per_block(types[i]);
        if (sizes[i] != want) return -3;
    }
    float* x = (float*)malloc(sizeof(float) * (size_t)hidden);
    float* act = (float*)malloc(sizeof(float) * (size_t)intermediate);
    if (!x || !act) { free(x); free(act); return -5; }
    for (int i = 0; i < hidden; ++i) x[i] = fp16_graph ? round16(input[i]) : input[i];
    const int64_t gr = (int64_t)(hidden / oracle_block_size(gate_type)) * oracle_bytes_per_block(gate_type);
    const int64_t ur = (int64_t)(hidden / oracle_block_size(up_type)) * oracle_bytes_per_block(up_type);
    const int64_t dr = (int64_t)(intermediate / oracle_block_size(down_type)) * oracle_bytes_per_block(down_type);
    for (int r = 0; r < intermediate; ++r) {
        float g = quant_dot(gate_type, gate + r * gr, x, hidden, fp16_graph);
        float u = quant_dot(up_type, up + r * ur, x, hidden, fp16_graph);
        if (fp16_graph) { g = round16(g); u = round16(u); }
        float sig = 1.0f / (1.0f + expf(-g));
        if (fp16_graph) sig = round16(sig);
        float silu = g * sig;
        if (fp16_graph) silu = round16(silu);
        const float a = silu * u;
        act[r] = fp16_graph ? round16(a) : a;
    }
    int status = 0;
    for (int r = 0; r < hidden; ++r) {
        const float y = quant_dot(down_type, down + r * dr, act, intermediate, fp16_graph);
        output[r] = fp16_graph ? round16(y) : y;
        if (!isfinite(output[r])) { status = -4; break; }
    }
    free(x);
    free(act);
    return status;
}

/* Same signature, argument meaning and status codes as the reference export
 * moe_quant_expert (moe_quant_dot.cpp:171-214):
 *   0 ok; -1 null pointer, hidden/intermediate <= 0 or > 65536, fp16_graph not
 *   0/1; -2 unsupported type or cols % block; -3 byte size mismatch; -4 a
 *   non-finite output (outputs up to and including that row are written);
 *   -5 allocation failure. */
int oracle_moe_quant_expert(int gate_type, const uint8_t* gate, int64_t gate_bytes,
                            int up_type, const uint8_t* up, int64_t up_bytes,
                            int down_type, const uint8_t* down, int64_t down_bytes,
                            const float* input, int hidden, int intermediate,
                            float* output, int fp16_graph) {
    return expert_with(quant_dot, gate_type, gate, gate_bytes, up_type, up, up_bytes, down_type, down, down_bytes,
                       input, hidden, intermediate, output, fp16_graph);
}

/* The same expert with the AVX2 row dot of kquant_avx2.c (bit-identical
 * results; the CPU baseline of the bench). */
float oracle_quant_dot_avx2(int type, const uint8_t* row, const float* x, int cols, int round_w);

int oracle_moe_quant_expert_avx2(int gate_type, const uint8_t* gate, int64_t gate_bytes,
                                 int up_type, const uint8_t* up, int64_t up_bytes,
                                 int down_type, const uint8_t* down, int64_t down_bytes,
                                 const float* input, int hidden, int intermediate,
                                 float* output, int fp16_graph) {
    return expert_with(oracle_quant_dot_avx2, gate_type, gate, gate_bytes, up_type, up, up_bytes, down_type, down,
                       down_bytes, input, hidden, intermediate, output, fp16_graph);
}

/* ------------------------------------------ IQ4_NL (cpp/fast_dequant.cpp:40-65) */

/* The reference library's 16-entry table, its own constants
 * (fast_dequant.cpp:4-9, fast_dequant_avx2.cpp:34-39); not gguf's
 * kvalues_iq4nl / 127. */
static const float IQ4NL_TABLE[16] = {-1.0f,     -0.6961914f, -0.515625f, -0.375f,     -0.25390625f, -0.1484375f,
                                      -0.0546875f, 0.02734375f, 0.1015625f, 0.1796875f, 0.265625f,    0.359375f,
                                      0.46875f,    0.59765625f, 0.7578125f, 1.0f};

/* rows x (cols / 32) 18-byte blocks: FP16 scale d, then qs[16]; value i
 * (0..15) = d * table[qs[i] & 15], value 16 + i = d * table[qs[i] >> 4];
 * output row r at dst + r * cols. */
void oracle_dequantize_iq4_nl(const uint8_t* src, float* dst, int rows, int cols) {
    const int bpr = cols / 32;
    for (int r = 0; r < rows; ++r) {
        for (int b = 0; b < bpr; ++b) {
            const uint8_t* blk = src + ((int64_t)r * bpr + b) * 18;
            const float d = ld_f16(blk);
            float* out = dst + (int64_t)r * cols + 32 * b;
            for (int i = 0; i < 16; ++i) {
                out[i] = d * IQ4NL_TABLE[blk[2 + i] & 15];
                out[i + 16] = d * IQ4NL_TABLE[blk[2 + i] >> 4];
            }
        }
    }
}
