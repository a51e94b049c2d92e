/*
 * delta_oracle.c -- CPU oracle for the DeltaNet decode recurrence.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker of the HIP library's
 * mqh_delta_heads / moe_delta_heads; never on the product path).
 *
 * A plain-C restatement of cpp/moe_delta.cpp:18-69 (moe_delta_heads), one
 * gated delta-rule step for every value row of every head, state updated in
 * place (arXiv 2412.06464 eq. 10):
 *   decay = exp(gate[h])                      in double           (:25)
 *   s_j   = (float)((double)s_j * decay)      per state element   (:33-38, :46-47)
 *   kv    = sum_j s_j * k_j                                       (:39, :44, :48)
 *   delta = beta[h] * (v[h][r] - kv)                              (:50)
 *   s_j   = s_j + delta * k_j                                     (:54-57, :62)
 *   out   = sum_j s_j * q_j                                       (:58, :61, :63)
 * The reference sums with eight accumulators, accumulator l taking the columns
 * j = l (mod 8) of the leading multiple of 8 in column order, then adds the
 * eight into a zero in accumulator order (sum8, :10-16) and then the remaining
 * key_dim % 8 columns one by one; every product and sum is rounded on its own
 * (separate _mm256_mul_ps / _mm256_add_ps, no contraction).  This file keeps
 * exactly that order, so its results are the reference's bit for bit (the
 * Makefile builds with -ffp-contract=off).
 *
 * Status: -1 for a null pointer or heads outside 1..256, key_dim or value_dim
 * outside 1..1024 (:22-24); -2 at the first non-finite output, after updating
 * that row's state and writing the outputs of the rows before it (:65).
 */
#include <math.h>
#include <stdint.h>

static float sum8(const float* lanes) {
    float s = 0.0f;
    for (int l = 0; l < 8; ++l) s += lanes[l];
    return s;
}

int oracle_delta_heads(float* state, const float* q, const float* k, const float* v, const float* beta,
                       const float* gate, float* output, int heads, int key_dim, int value_dim) {
    if (!state || !q || !k || !v || !beta || !gate || !output || heads < 1 || heads > 256 || key_dim < 1 ||
        key_dim > 1024 || value_dim < 1 || value_dim > 1024)
        return -1;
    const int full = key_dim / 8 * 8;
    for (int h = 0; h < heads; ++h) {
        const double decay = exp((double)gate[h]);
        const float* kh = k + (int64_t)h * key_dim;
        const float* qh = q + (int64_t)h * key_dim;
        for (int r = 0; r < value_dim; ++r) {
            float* row = state + ((int64_t)h * value_dim + r) * key_dim;
            float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int j = 0; j < full; ++j) {
                row[j] = (float)((double)row[j] * decay);
                const float p = row[j] * kh[j];
                acc[j & 7] = acc[j & 7] + p;
            }
            float kv = sum8(acc);
            for (int j = full; j < key_dim; ++j) {
                row[j] = (float)((double)row[j] * decay);
                const float p = row[j] * kh[j];
                kv = kv + p;
            }
            const float delta = beta[h] * (v[(int64_t)h * value_dim + r] - kv);
            for (int l = 0; l < 8; ++l) acc[l] = 0.0f;
            for (int j = 0; j < full; ++j) {
                const float dk = delta * kh[j];
                row[j] = row[j] + dk;
                const float p = row[j] * qh[j];
                acc[j & 7] = acc[j & 7] + p;
            }
            float result = sum8(acc);
            for (int j = full; j < key_dim; ++j) {
                const float dk = delta * kh[j];
                row[j] = row[j] + dk;
                const float p = row[j] * qh[j];
                result = result + p;
            }
            if (!isfinite(result)) return -2;
            output[(int64_t)h * value_dim + r] = result;
        }
    }
    return 0;
}
