// Host build of the decode fast path's per-lane arithmetic (kquant_lane.h), for
// checking it against the CPU oracle without a GPU.  Test helper only.
#include <stdint.h>
#include <string.h>

#include <vector>

#include "kquant_lane.h"

using namespace mqh;

// Activation digits as the kernels build them: aligned 16-column runs with
// scale max|x|/127, two int8 digit planes, FP32 sums of each run.
struct HostDigits {
    std::vector<int8_t> planes;
    std::vector<float> xs16, sum16;
    int n;
    HostDigits(const float* x, int n_) : planes(2 * (size_t)n_), xs16(n_ / 16), sum16(n_ / 16), n(n_) {
        for (int g = 0; g < n / 16; ++g) {
            float amax = 0.0f, s = 0.0f;
            for (int k = 0; k < 16; ++k) {
                amax = fmaxf(amax, fabsf(x[16 * g + k]));
                s += x[16 * g + k];
            }
            const float inv = digit_inv(amax);
            for (int k = 0; k < 16; ++k) {
                const uint32_t dg = split2(x[16 * g + k], inv);
                planes[16 * g + k] = (int8_t)(dg & 0xFF);
                planes[n + 16 * g + k] = (int8_t)(dg >> 8);
            }
            xs16[g] = digit_scale(amax);
            sum16[g] = s;
        }
    }
    DigitsRef ref() const {
        DigitsRef v;
        v.planes = planes.data();
        v.xs16 = xs16.data();
        v.sum16 = sum16.data();
        v.n = n;
        return v;
    }
};

// (both forms of the loaded scale words, lane_load<T, DW>, must give the same
// bits; a difference returns NaN)
template <int T>
static float row_dot(const uint8_t* row, int ncols, const HostDigits& hd) {
    float acc = 0.0f, acc_dw = 0.0f;
    for (int b = 0; b < ncols / 256; ++b) {
        for (int k = 0; k < LANES_PER_BLOCK; ++k) {
            uint32_t raw[LaneGeo<T>::NRAW], raw_dw[LaneGeo<T>::NRAW];
            LaneX x;
            lane_x<T>(hd.ref(), b, k, x);
            lane_load<T>(row + (int64_t)b * unit_bytes(T), k, raw);
            lane_load<T, true>(row + (int64_t)b * unit_bytes(T), k, raw_dw);
            acc += lane_dot<T>(raw, k, x);
            acc_dw += lane_dot<T, true>(raw_dw, k, x);
        }
    }
    return __builtin_memcmp(&acc, &acc_dw, 4) == 0 ? acc : __builtin_nanf("");
}

extern "C" float mqh_cpu_row_dot(int type, const uint8_t* row, int ncols, const float* x) {
    HostDigits hd(x, ncols);
    switch (type) {
        case T_Q4_K: return row_dot<T_Q4_K>(row, ncols, hd);
        case T_Q5_K: return row_dot<T_Q5_K>(row, ncols, hd);
        case T_Q6_K: return row_dot<T_Q6_K>(row, ncols, hd);
        case T_Q8_0: return row_dot<T_Q8_0>(row, ncols, hd);
        default: return row_dot<T_Q3_K>(row, ncols, hd);
    }
}

// digits of x and the reconstruction (s/254) * (254 x0 + x1)
extern "C" void mqh_cpu_digit_roundtrip(const float* x, int n, float* out) {
    HostDigits hd(x, n);
    for (int i = 0; i < n; ++i)
        out[i] = (float)((double)hd.xs16[i / 16] * (254.0 * hd.planes[i] + hd.planes[n + i]));
}

// Columns each (lane k, run r) covers, as 256 counts per type: every column of
// a super-block must be owned by exactly one lane.
template <int T>
static void cover(int* count) {
    for (int k = 0; k < LANES_PER_BLOCK; ++k)
        for (int r = 0; r < LaneGeo<T>::NR; ++r)
            for (int i = 0; i < LaneGeo<T>::RL; ++i) count[lane_col<T>(k, r) + i]++;
}

extern "C" void mqh_cpu_lane_cover(int type, int* count) {
    for (int c = 0; c < 256; ++c) count[c] = 0;
    switch (type) {
        case T_Q3_K: cover<T_Q3_K>(count); break;
        case T_Q6_K: cover<T_Q6_K>(count); break;
        case T_Q5_K: cover<T_Q5_K>(count); break;
        case T_Q8_0: cover<T_Q8_0>(count); break;
        default: cover<T_Q4_K>(count); break;
    }
}

// The FP16-graph operands of one 256-column unit: for every lane k and every
// weight of its 64, the FP16 bits lane_w16 produces and the column it belongs
// to (lane_col order), 256 of each.
template <int T>
static void w16_unit(const uint8_t* unit, uint16_t* bits, int* cols) {
    for (int k = 0; k < LANES_PER_BLOCK; ++k) {
        uint32_t raw[LaneGeo<T>::NRAW], raw_dw[LaneGeo<T>::NRAW];
        uint32_t w[32], w_dw[32];
        lane_load<T>(unit, k, raw);
        lane_w16<T>(raw, k, w);
        lane_load<T, true>(unit, k, raw_dw);
        lane_w16<T, true>(raw_dw, k, w_dw);
        if (__builtin_memcmp(w, w_dw, sizeof(w)) != 0) w[0] = 0xFFFFFFFFu;   // (flagged by the caller's check)
        for (int i = 0; i < 64; ++i) {
            const int r = i / LaneGeo<T>::RL;
            bits[64 * k + i] = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
            cols[64 * k + i] = lane_col<T>(k, r) + i % LaneGeo<T>::RL;
        }
    }
}

extern "C" void mqh_cpu_lane_w16(int type, const uint8_t* unit, uint16_t* bits, int* cols) {
    switch (type) {
        case T_Q4_K: w16_unit<T_Q4_K>(unit, bits, cols); break;
        case T_Q5_K: w16_unit<T_Q5_K>(unit, bits, cols); break;
        case T_Q6_K: w16_unit<T_Q6_K>(unit, bits, cols); break;
        case T_Q8_0: w16_unit<T_Q8_0>(unit, bits, cols); break;
        default: w16_unit<T_Q3_K>(unit, bits, cols); break;
    }
}
