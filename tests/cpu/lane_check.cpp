// Host build of the decode fast path's per-lane arithmetic (kquant_lane.h), for
// checking it against the CPU oracle without a GPU.  Test helper only.
#include <stdint.h>
#include <string.h>

#include <vector>

#include "kquant_lane.h"

using namespace mqh;

// Activation digits as the kernels build them: aligned 16-column runs with a
// power-of-two scale, three int8 digit planes, FP32 sums of 8 values.
struct HostDigits {
    std::vector<int8_t> planes;
    std::vector<float> xs16, sum8;
    int n;
    HostDigits(const float* x, int n_) : planes(3 * (size_t)n_), xs16(n_ / 16), sum8(n_ / 8), n(n_) {
        for (int g = 0; g < n / 16; ++g) {
            float amax = 0.0f;
            for (int k = 0; k < 16; ++k) amax = fmaxf(amax, fabsf(x[16 * g + k]));
            const int e = digit_exp(amax);
            for (int k = 0; k < 16; ++k) {
                int8_t d0, d1, d2;
                split_digits(x[16 * g + k], e, d0, d1, d2);
                planes[16 * g + k] = d0;
                planes[n + 16 * g + k] = d1;
                planes[2 * n + 16 * g + k] = d2;
            }
            xs16[g] = ldexpf(1.0f, e - 14);
        }
        for (int g = 0; g < n / 8; ++g) {
            float s = 0.0f;
            for (int k = 0; k < 8; ++k) s += x[8 * g + k];
            sum8[g] = s;
        }
    }
    DigitsRef ref() const {
        DigitsRef v;
        v.planes = planes.data();
        v.xs16 = xs16.data();
        v.sum8 = sum8.data();
        v.n = n;
        return v;
    }
};

template <int T>
static float row_dot(const uint8_t* row, int ncols, const HostDigits& hd) {
    float acc = 0.0f;
    for (int b = 0; b < ncols / 256; ++b) {
        for (int k = 0; k < 8; ++k) {
            uint32_t raw[LaneGeo<T>::NRAW];
            LaneX x;
            lane_x<T>(hd.ref(), b, k, x);
            lane_load<T>(row + (int64_t)b * block_bytes(T), k, raw);
            acc += lane_dot<T>(raw, k, x);
        }
    }
    return acc;
}

extern "C" float mqh_cpu_row_dot(int type, const uint8_t* row, int ncols, const float* x) {
    HostDigits hd(x, ncols);
    switch (type) {
        case T_Q4_K: return row_dot<T_Q4_K>(row, ncols, hd);
        case T_Q5_K: return row_dot<T_Q5_K>(row, ncols, hd);
        case T_Q6_K: return row_dot<T_Q6_K>(row, ncols, hd);
        default: return row_dot<T_Q3_K>(row, ncols, hd);
    }
}

// digits of x and the reconstruction s*(x0 + x1/128 + x2/16384)
extern "C" void mqh_cpu_digit_roundtrip(const float* x, int n, float* out) {
    HostDigits hd(x, n);
    for (int i = 0; i < n; ++i) {
        const float s = hd.xs16[i / 16];   // 2^e / 16384
        out[i] = s * (16384.0f * hd.planes[i] + 128.0f * hd.planes[n + i] + hd.planes[2 * n + i]);
    }
}

// Columns each (lane k, run r) covers, as 256 flags per type: every column of
// a super-block must be owned by exactly one lane.
extern "C" void mqh_cpu_lane_cover(int type, int* count) {
    for (int c = 0; c < 256; ++c) count[c] = 0;
    for (int k = 0; k < 8; ++k) {
        switch (type) {
            case T_Q3_K:
                for (int r = 0; r < 4; ++r)
                    for (int i = 0; i < 8; ++i) count[lane_col<T_Q3_K>(k, r) + i]++;
                break;
            case T_Q6_K:
                for (int r = 0; r < 2; ++r)
                    for (int i = 0; i < 16; ++i) count[lane_col<T_Q6_K>(k, r) + i]++;
                break;
            default:
                for (int r = 0; r < 2; ++r)
                    for (int i = 0; i < 16; ++i) count[lane_col<T_Q4_K>(k, r) + i]++;
                break;
        }
    }
}
