/*
 * kquant_avx2.c -- AVX2 form of the oracle's fused-expert row dot, the CPU
 * baseline of the bench.
 *
 * TEST INFRASTRUCTURE ONLY (like kquant_oracle.c): bench.py's CPU-baseline leg
 * times it and tests/test_oracle_avx2.py checks it bit-for-bit against the
 * scalar oracle; nothing on the product path loads it.
 *
 * The reference's quant_dot (cpp/moe_quant_dot.cpp:143-169) runs on AVX2: one
 * __m256 accumulator whose lane k takes the columns == k (mod 8) by FMA in
 * column order, the lanes summed serially at the end.  Q3_K and Q6_K rows are
 * decoded straight from their bit fields into that accumulator
 * (moe_quant_dot.cpp:23-139); every other type decodes a block into a
 * 256-float buffer first and then streams it through the same FMAs.  This
 * file does the same work with its own decoding: a whole 32-value group of
 * quants is assembled as 32 signed bytes in one 256-bit register (low bits,
 * high bits and offset in three byte-wise operations) and then widened eight
 * at a time.  The weight of each value is float(q) * (d * float(scale)), the
 * same two roundings as the scalar oracle's decoders, so the accumulator sees
 * the same operands in the same order: the result equals the scalar oracle's
 * bit for bit (and the FP16-graph rounding uses the F16C round-to-nearest-even
 * conversion, which is the oracle's round16).
 */
#include <immintrin.h>
#include <stdint.h>

#define QK_K 256
enum { A_Q3_K = 11, A_Q6_K = 14 };

float oracle_f16_to_f32(uint16_t h);
int oracle_block_size(int type);
int oracle_bytes_per_block(int type);
int oracle_decode_block(int type, const uint8_t* blk, float* out);

static inline float f16_at(const uint8_t* p) { return oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

static inline __m256 round16_ps(__m256 w) { return _mm256_cvtph_ps(_mm256_cvtps_ph(w, _MM_FROUND_TO_NEAREST_INT)); }

/* The 32 signed quants q of one group (columns 32g..32g+31 of the block) times
 * the two 16-column scales sc[0], sc[1], FMA'd into acc against x[0..31]. */
static inline __m256 group_fma(__m256i q, const float* sc, const float* x, int round_w, __m256 acc) {
    const __m128i lo = _mm256_castsi256_si128(q), hi = _mm256_extracti128_si256(q, 1);
    const __m128i part[4] = {lo, _mm_srli_si128(lo, 8), hi, _mm_srli_si128(hi, 8)};
    for (int p = 0; p < 4; ++p) {
        __m256 w = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(part[p])), _mm256_set1_ps(sc[p >> 1]));
        if (round_w) w = round16_ps(w);
        acc = _mm256_fmadd_ps(w, _mm256_loadu_ps(x + 8 * p), acc);
    }
    return acc;
}

/* Q3_K (110 B: hmask[32]@0 qs[64]@32 scales[12]@96 d@108).  Group g: two low
 * bits from qs[32(g/4) + l] >> 2(g%4), the mask bit hmask[l] >> g; the quant
 * is (low | bit << 2) - 4, i.e. low - 4 when the bit is clear. */
static inline __m256 q3k_block(const uint8_t* blk, const float* x, int round_w, __m256 acc) {
    const uint8_t* s = blk + 96;
    const float d = f16_at(blk + 108);
    float sc[16];
    for (int j = 0; j < 16; ++j) {
        const int low = (j < 8 ? s[j] : s[j - 8] >> 4) & 15, high = (s[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
        sc[j] = d * (float)((low | (high << 4)) - 32);
    }
    const __m256i mask = _mm256_loadu_si256((const __m256i*)blk);
    const __m256i qs[2] = {_mm256_loadu_si256((const __m256i*)(blk + 32)),
                           _mm256_loadu_si256((const __m256i*)(blk + 64))};
    const __m256i three = _mm256_set1_epi8(3), four = _mm256_set1_epi8(4);
    for (int g = 0; g < 8; ++g) {
        const __m128i sh_lo = _mm_cvtsi32_si128(2 * (g & 3)), sh_bit = _mm_cvtsi32_si128(g);
        const __m256i low = _mm256_and_si256(_mm256_srl_epi16(qs[g >> 2], sh_lo), three);
        const __m256i bit4 = _mm256_and_si256(_mm256_sll_epi16(_mm256_srl_epi16(mask, sh_bit), _mm_cvtsi32_si128(2)), four);
        const __m256i q = _mm256_sub_epi8(_mm256_or_si256(low, bit4), four);
        acc = group_fma(q, sc + 2 * g, x + 32 * g, round_w, acc);
    }
    return acc;
}

/* Q6_K (210 B: ql[128]@0 qh[64]@128 int8 scales[16]@192 d@208).  Group g,
 * h = g/4, s = g%4: low nibble of ql[64h + 32(s&1) + l] >> 4(s/2), two high
 * bits qh[32h + l] >> 2s; the quant is (low | high << 4) - 32. */
static inline __m256 q6k_block(const uint8_t* blk, const float* x, int round_w, __m256 acc) {
    const float d = f16_at(blk + 208);
    const int8_t* s8 = (const int8_t*)(blk + 192);
    float sc[16];
    for (int j = 0; j < 16; ++j) sc[j] = d * (float)s8[j];
    const __m256i nib = _mm256_set1_epi8(15), two = _mm256_set1_epi8(0x30), off = _mm256_set1_epi8(32);
    for (int g = 0; g < 8; ++g) {
        const int h = g >> 2, s = g & 3;
        const __m256i ql = _mm256_loadu_si256((const __m256i*)(blk + 64 * h + 32 * (s & 1)));
        const __m256i qh = _mm256_loadu_si256((const __m256i*)(blk + 128 + 32 * h));
        const __m256i low = _mm256_and_si256(_mm256_srl_epi16(ql, _mm_cvtsi32_si128(4 * (s >> 1))), nib);
        /* the two bits at 2s moved to bits 4..5: shift right by 2s, left by 4 */
        const __m256i high = _mm256_and_si256(
            _mm256_sll_epi16(_mm256_srl_epi16(qh, _mm_cvtsi32_si128(2 * s)), _mm_cvtsi32_si128(4)), two);
        const __m256i q = _mm256_sub_epi8(_mm256_or_si256(low, high), off);
        acc = group_fma(q, sc + 2 * g, x + 32 * g, round_w, acc);
    }
    return acc;
}

/* One row . x, the reference's lane order (moe_quant_dot.cpp:143-169). */
float oracle_quant_dot_avx2(int type, const uint8_t* row, const float* x, int cols, int round_w) {
    const int bs = oracle_block_size(type), pb = oracle_bytes_per_block(type);
    float tmp[QK_K] __attribute__((aligned(32)));
    __m256 acc = _mm256_setzero_ps();
    for (int off = 0; off < cols; off += bs, row += pb) {
        if (type == A_Q3_K) {
            acc = q3k_block(row, x + off, round_w, acc);
        } else if (type == A_Q6_K) {
            acc = q6k_block(row, x + off, round_w, acc);
        } else {
            oracle_decode_block(type, row, tmp);
            for (int j = 0; j < bs; j += 8) {
                __m256 w = _mm256_load_ps(tmp + j);
                if (round_w) w = round16_ps(w);
                acc = _mm256_fmadd_ps(w, _mm256_loadu_ps(x + off + j), acc);
            }
        }
    }
    float lanes[8] __attribute__((aligned(32)));
    _mm256_store_ps(lanes, acc);
    float r = 0.0f;
    for (int k = 0; k < 8; ++k) r += lanes[k];
    return r;
}
