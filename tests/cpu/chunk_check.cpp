// Host build of the fused decode's per-chunk arithmetic (kquant_dot.h), for
// checking it against the CPU oracle without a GPU.  Test helper only.
#include <stdint.h>
#include <string.h>

#include <vector>

#include "kquant_dot.h"

using namespace mqh;

// Activation digits exactly as the kernels build them: 32-column groups with a
// power-of-two scale, three int8 digits, FP32 sums of 16-column runs.
struct HostDigits {
    std::vector<int8_t> dig;
    std::vector<float> xs, sum;
    int n;
    HostDigits(const float* x, int n_) : dig(3 * (size_t)n_), xs(n_ / 32), sum(n_ / 16), n(n_) {
        for (int g = 0; g < n / 32; ++g) {
            float amax = 0.0f;
            for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(x[32 * g + k]));
            const int e = digit_exp(amax);
            for (int k = 0; k < 32; ++k) {
                int8_t d0, d1, d2;
                split_digits(x[32 * g + k], e, d0, d1, d2);
                dig[32 * g + k] = d0;
                dig[n + 32 * g + k] = d1;
                dig[2 * n + 32 * g + k] = d2;
            }
            xs[g] = ldexpf(1.0f, e - 14);
        }
        for (int g = 0; g < n / 16; ++g) {
            float s = 0.0f;
            for (int k = 0; k < 16; ++k) s += x[16 * g + k];
            sum[g] = s;
        }
    }
    void chunk(int type, int blk, int c, ChunkX& cx) const {
        for (int run = 0; run < RUNS; ++run) {
            const int col = blk * 256 + run_col(type, c, run);
            for (int d = 0; d < NDIG; ++d) memcpy(&cx.d[d][4 * run], &dig[(size_t)d * n + col], 16);
            cx.xs[run] = xs[col >> 5];
            cx.sum[run] = sum[col >> 4];
        }
    }
};

extern "C" float mqh_cpu_row_dot(int type, const uint8_t* row, int ncols, const float* x) {
    HostDigits hd(x, ncols);
    float acc = 0.0f;
    for (int b = 0; b < ncols / 256; ++b) {
        for (int c = 0; c < 4; ++c) {
            uint32_t w[20];
            ChunkX cx;
            hd.chunk(type, b, c, cx);
            load_chunk_any(type, row + (int64_t)b * block_bytes(type), c, w);
            acc += chunk_dot_any(type, w, c, cx);
        }
    }
    return acc;
}

// digits of x (3 planes of n int8) and the reconstruction s*(x0 + x1/128 + x2/16384)
extern "C" void mqh_cpu_digit_roundtrip(const float* x, int n, float* out) {
    HostDigits hd(x, n);
    for (int i = 0; i < n; ++i) {
        const float s = hd.xs[i / 32];   // 2^e / 16384
        out[i] = s * (16384.0f * hd.dig[i] + 128.0f * hd.dig[n + i] + hd.dig[2 * n + i]);
    }
}
