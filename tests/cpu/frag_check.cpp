// Host build of the prefill GEMM's operand math (kquant_frag.h): a 64-lane wave
// emulated lane by lane, with the MFMA layouts of v_mfma_f32_16x16x32_f16
// (A: row l%16, k = 8(l/16) + i; B: column l%16, same k, the lane's k-slots
// holding the 8 consecutive columns frag_col + frag_lane_col) and
// v_mfma_f32_16x16x16_f16 (k = 4(l/16) + i), for checking the integer-operand
// decomposition against the oracle without a GPU.  Test helper only.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "kquant_frag.h"

using namespace mqh;

namespace {

struct Tile {
    int ntok, K;
    std::vector<float> xh, xl;   // [ntok][K], the FP16 planes as floats
    std::vector<float> sh, sl;   // [ntok][K/32] sub-block sums / 32, FP16 planes
    std::vector<int> k;          // power-of-two exponent per token
};

Tile stage(const float* x, int ntok, int K, int split) {
    Tile t;
    t.ntok = ntok;
    t.K = K;
    t.xh.assign((size_t)ntok * K, 0.0f);
    t.xl.assign((size_t)ntok * K, 0.0f);
    t.sh.assign((size_t)ntok * K / 32, 0.0f);
    t.sl.assign((size_t)ntok * K / 32, 0.0f);
    t.k.assign(ntok, 0);
    for (int j = 0; j < ntok; ++j) {
        const float* row = x + (size_t)j * K;
        float amax = 0.0f;
        for (int c = 0; c < K; ++c) amax = fmaxf(amax, fabsf(row[c]));
        const int k = frag_exp(amax);
        t.k[j] = k;
        for (int g = 0; g < K / 32; ++g) {
            float s = 0.0f;
            for (int c = 32 * g; c < 32 * g + 32; ++c) {
                _Float16 hi, lo;
                frag_split(row[c], k, hi, lo);
                t.xh[(size_t)j * K + c] = (float)hi;
                t.xl[(size_t)j * K + c] = split ? (float)lo : 0.0f;
                s += ldexpf(row[c], -k);
            }
            _Float16 hi, lo;
            frag_split(s, 5, hi, lo);
            t.sh[(size_t)j * K / 32 + g] = (float)hi;
            t.sl[(size_t)j * K / 32 + g] = (float)lo;
        }
    }
    return t;
}

template <int T, int M, bool IP = true>
void step(const uint32_t* r, int row, int q, int b, const Tile& t, int split, std::vector<double>& P) {
    h8_t a[2];
    FragPrep<T> sp;
    frag_prep<T, IP>(r, q, sp);
    frag_step<T, M, IP>(r, sp, q, a);
    const h8_t alo = frag_lo_operand<T>(a);
    const int col = frag_col<T, M>() + frag_lane_col<T>((q + 3) & 3);
    for (int j = 0; j < t.ntok; ++j) {
        const size_t base = (size_t)j * t.K + 256 * b + col;
        double s = 0.0;
        for (int e = 0; e < 8; ++e) {
            for (int n = 0; n < FragGeo<T>::NA; ++n) s += (double)(float)a[n][e] * t.xh[base + e];
            if (split) s += (double)(float)alo[e] * t.xl[base + e];
        }
        P[row * 16 + j] += s;
    }
}

// Q8_0: each step is one 32-column block with its own d, applied to that
// step's product (the lane of k-group qq holds the d of blocks 2qq and 2qq+1)
template <int M>
void step_q8(const uint32_t* r, int row, int q, int b, const Tile& t, int split, std::vector<double>& P) {
    std::vector<double> Pm(16 * 16, 0.0);
    step<T_Q8_0, M>(r, row, q, b, t, split, Pm);
    for (int j = 0; j < t.ntok; ++j) P[(M * 16 + row) * 16 + j] += Pm[row * 16 + j];
}

void gemm_q8(const uint8_t* w, int K, const Tile& t, int split, float* out) {
    constexpr int BB = frag_unit_bytes<T_Q8_0>();
    const int nb = K / 256;
    std::vector<double> acc(16 * 16, 0.0);
    for (int b = 0; b < nb; ++b) {
        std::vector<double> P(8 * 16 * 16, 0.0);   // [step][row][token]
        float d[16][8];
        for (int l = 0; l < 64; ++l) {
            const int row = l % 16, q = l / 16, qq = (q + 3) & 3;
            uint32_t r[FragGeo<T_Q8_0>::NW];
            frag_load<T_Q8_0>(w + (size_t)row * nb * BB + (size_t)b * BB, q, r);
            step_q8<0>(r, row, q, b, t, split, P);
            step_q8<1>(r, row, q, b, t, split, P);
            step_q8<2>(r, row, q, b, t, split, P);
            step_q8<3>(r, row, q, b, t, split, P);
            step_q8<4>(r, row, q, b, t, split, P);
            step_q8<5>(r, row, q, b, t, split, P);
            step_q8<6>(r, row, q, b, t, split, P);
            step_q8<7>(r, row, q, b, t, split, P);
            d[row][2 * qq] = frag_h2f(r[16]);
            d[row][2 * qq + 1] = frag_h2f(r[17]);
        }
        for (int m = 0; m < 8; ++m)
            for (int row = 0; row < 16; ++row)
                for (int j = 0; j < t.ntok; ++j) acc[row * 16 + j] += (double)d[row][m] * P[(m * 16 + row) * 16 + j];
    }
    for (int j = 0; j < t.ntok; ++j)
        for (int row = 0; row < 16; ++row) out[(size_t)j * 16 + row] = (float)ldexp(acc[row * 16 + j], t.k[j]);
}

template <int T, bool IP = true>
void gemm(const uint8_t* w, int K, const Tile& t, int split, float* out) {
    constexpr int BB = block_bytes(T);
    const int nb = K / 256;
    std::vector<double> acc(16 * 16, 0.0);
    for (int b = 0; b < nb; ++b) {
        std::vector<double> P(16 * 16, 0.0), Mn(16 * 16, 0.0);
        float d[16], dmin[16];
        for (int l = 0; l < 64; ++l) {
            const int row = l % 16, q = l / 16;
            uint32_t r[FragGeo<T>::NW];
            frag_load<T>(w + (size_t)row * nb * BB + (size_t)b * BB, q, r);
            step<T, 0, IP>(r, row, q, b, t, split, P);
            step<T, 1, IP>(r, row, q, b, t, split, P);
            step<T, 2, IP>(r, row, q, b, t, split, P);
            step<T, 3, IP>(r, row, q, b, t, split, P);
            step<T, 4, IP>(r, row, q, b, t, split, P);
            step<T, 5, IP>(r, row, q, b, t, split, P);
            step<T, 6, IP>(r, row, q, b, t, split, P);
            step<T, 7, IP>(r, row, q, b, t, split, P);
            const uint32_t hdr = r[FragGeo<T>::HDR];
            d[row] = frag_d<T>(hdr);
            dmin[row] = frag_dmin(hdr);
            if constexpr (FragGeo<T>::MIN) {
                const h4_t mm = frag_mins<T>(r, q);
                for (int j = 0; j < t.ntok; ++j)
                    for (int i = 0; i < 4; ++i) {
                        const int kk = 4 * q + i;   // k < 8: high sums, k >= 8: low sums
                        const float bx = kk < 8 ? t.sh[(size_t)j * K / 32 + 8 * b + kk] : t.sl[(size_t)j * K / 32 + 8 * b + kk - 8];
                        Mn[row * 16 + j] += (double)(float)mm[i] * bx;
                    }
            }
        }
        for (int row = 0; row < 16; ++row)
            for (int j = 0; j < t.ntok; ++j) {
                acc[row * 16 + j] += (double)d[row] * P[row * 16 + j];
                if constexpr (FragGeo<T>::MIN) acc[row * 16 + j] -= (double)dmin[row] * Mn[row * 16 + j];
            }
    }
    for (int j = 0; j < t.ntok; ++j)
        for (int row = 0; row < 16; ++row) out[(size_t)j * 16 + row] = (float)ldexp(acc[row * 16 + j], t.k[j]);
}

}  // namespace

// out[tok][row] = sum_c W[row][c] x[tok][c] for 16 quantized rows (K columns)
// and ntok <= 16 FP32 token rows, computed from the kernel's operands.  split:
// 1 = high and low FP16 planes of x, 0 = high plane only (BF16 inputs).  Type
// 11 takes the in-place Q3_K operand (the down kernel's), -11 the other (the
// gate/up kernel's).
extern "C" void mqh_cpu_frag_gemm(int type, const uint8_t* w, int K, const float* x, int ntok, int split, float* out) {
    const Tile t = stage(x, ntok, K, split);
    switch (type) {
        case T_Q4_K: gemm<T_Q4_K>(w, K, t, split, out); break;
        case T_Q5_K: gemm<T_Q5_K>(w, K, t, split, out); break;
        case T_Q6_K: gemm<T_Q6_K>(w, K, t, split, out); break;
        case T_Q8_0: gemm_q8(w, K, t, split, out); break;
        case -T_Q3_K: gemm<T_Q3_K, false>(w, K, t, split, out); break;
        default: gemm<T_Q3_K>(w, K, t, split, out); break;
    }
}

// How often each of a super-block's 256 columns is dealt to a (lane, step,
// slot): every column must be owned exactly once.
template <int T>
static void cover(int* count) {
    for (int q = 0; q < 4; ++q) {
        const int lc = frag_lane_col<T>((q + 3) & 3);
        const int c[8] = {frag_col<T, 0>(), frag_col<T, 1>(), frag_col<T, 2>(), frag_col<T, 3>(),
                          frag_col<T, 4>(), frag_col<T, 5>(), frag_col<T, 6>(), frag_col<T, 7>()};
        for (int m = 0; m < 8; ++m)
            for (int e = 0; e < 8; ++e) count[c[m] + lc + e]++;
    }
}

extern "C" void mqh_cpu_frag_cover(int type, int* count) {
    for (int c = 0; c < 256; ++c) count[c] = 0;
    switch (type) {
        case T_Q4_K: cover<T_Q4_K>(count); break;
        case T_Q5_K: cover<T_Q5_K>(count); break;
        case T_Q6_K: cover<T_Q6_K>(count); break;
        case T_Q8_0: cover<T_Q8_0>(count); break;
        default: cover<T_Q3_K>(count); break;
    }
}
