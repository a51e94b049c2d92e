// moe_decode.hip -- fused quantized-expert decode for a few tokens (GEMV regime).
//
// Computes, for each token t and each of its routed slots s (expert ids[t,s],
// routing weight w[t,s]) plus an optional shared expert:
//   y_s  = W_down (silu(W_gate x) * (W_up x))            (moe_quant_dot.cpp:189-211)
//   y[t] = sum_s fl32(w_s) * y_s  (+ sigmoid(x . g_inp) * y_shared)
//                                                    (moe_layer.py:70-106,
//                                                     shared_expert.py:221-251)
// straight from the GGUF-quantized expert slices resident in HBM; experts are
// addressed through an index gather into the stacked [n_experts x slice]
// tensors, so one launch pair covers every expert of every token.
//
// Generic path (this file): kernel A (gate/up/act) then kernel B (down and
// weighted combine).  A 32-value "part" of a row is the unit a lane decodes:
// a row of `cols` columns has cols/32 parts; L lanes share one row (L = the
// power of two >= parts, at most 64) and a lane owning part p holds
// x[32p .. 32p+31] in registers for all the rows it visits.
//
// Graph modes: fp16_graph=1 reproduces the reference's FP16 graph on the
// routed experts (x, weights, g, u, sigmoid, silu, act and y rounded to FP16
// at the points of moe_quant_dot.cpp:192-209); the shared expert always runs
// the FP32 graph, as the reference's NumPy shared expert does.
#include <hip/hip_ext.h>

#include "kquant_device.h"
#include "moe_decode.h"

namespace mqh {

__device__ __forceinline__ float sigmoid_ref(float g) { return 1.0f / (1.0f + expf(-g)); }

// Stable sigmoid of shared_expert.py:55-62.
__device__ __forceinline__ float sigmoid_stable(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

struct RowMap {
    int P;      // parts per row
    int L;      // lanes per row (power of two)
    int rpi;    // rows per wavefront iteration
    int nk;     // parts per lane
};

__device__ __forceinline__ RowMap row_map(int cols) {
    RowMap m;
    m.P = cols >> 5;
    int L = 1;
    while (L < m.P && L < 64) L <<= 1;
    m.L = L;
    m.rpi = 64 / L;
    m.nk = (m.P + L - 1) / L;
    return m;
}

__device__ __forceinline__ int ppb_of(int type) { return block_size(type) / 32; }

// Partial dot product of the parts a lane owns, against values in registers
// (NK > 0) or read from `xmem` (NK == 0).
template <int NK>
__device__ __forceinline__ float lane_dot(int type, const uint8_t* row, const RowMap& m, int lp,
                                          const float (&xr)[NK > 0 ? NK : 1][32], const float* xmem,
                                          bool round_w) {
    const int ppb = ppb_of(type), pb = block_bytes(type);
    float acc = 0.0f;
    // part p's 32 weights against its 32 values x, in column order
    auto part = [&](int p, const float* x) {
        const uint8_t* blk = row + (int64_t)(p / ppb) * pb;
        const int sub = p % ppb;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float w[8];
            decode8_any(type, blk, 4 * sub + q, w);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = fmaf(round_w ? round16(w[j]) : w[j], x[8 * q + j], acc);
        }
    };
    if constexpr (NK > 0) {
        // unrolled, so xr is indexed by constants and stays in registers (a
        // runtime index puts the array in scratch memory); p grows with k, so
        // the guard skips exactly the parts past the row's end
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int p = lp + k * m.L;
            if (p < m.P) part(p, xr[k]);
        }
    } else {
        for (int k = 0; k < m.nk; ++k) {
            const int p = lp + k * m.L;
            if (p >= m.P) break;
            part(p, xmem + 32 * p);
        }
    }
    return acc;
}

template <int NK>
__device__ __forceinline__ void load_parts(float (&xr)[NK > 0 ? NK : 1][32], const float* src, const RowMap& m,
                                           int lp, bool round_x) {
    if constexpr (NK > 0) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int p = lp + k * m.L;
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                const float v = p < m.P ? src[32 * p + j] : 0.0f;
                xr[k][j] = round_x ? round16(v) : v;
            }
        }
    }
}

// ------------------------------------------------------------ kernel A

template <int NK>
__global__ __launch_bounds__(256) void k_gate_up(DecodeParams p) {
    const int t = blockIdx.z, s = blockIdx.y;
    const bool shared = (s == p.top_k);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint8_t *G, *U;
    int gt, ut, I;
    if (shared) {
        G = p.sh_gate; U = p.sh_up; gt = p.sh_gate_type; ut = p.sh_up_type; I = p.sh_inter;
    } else {
        const int e = p.ids[t * p.top_k + s];
        I = p.inter;
        if (e < 0 || e >= p.n_experts) {
            // Out-of-range expert id: flag it and contribute nothing.
            if (threadIdx.x == 0 && blockIdx.x == 0) atomicOr(&p.flags[FLAG_BAD_ID], 1);
            for (int r = blockIdx.x * ROWS_A + threadIdx.x; r < min(I, (int)(blockIdx.x + 1) * ROWS_A); r += 256)
                p.act[((int64_t)t * p.S + s) * p.Imax + r] = 0.0f;
            return;
        }
        G = p.gate + (int64_t)e * p.gate_eb; U = p.up + (int64_t)e * p.up_eb;
        gt = p.gate_type; ut = p.up_type;
    }
    const bool f16 = p.fp16 && !shared;
    const float* xt = p.x + (int64_t)t * p.hidden;

    if (shared && blockIdx.x == 0 && wave == 0) {
        float sc = 1.0f;
        if (p.sh_gate_inp) {
            float acc = 0.0f;
            for (int c = lane; c < p.hidden; c += 64) acc = fmaf(xt[c], p.sh_gate_inp[c], acc);
            sc = sigmoid_stable(group_sum(acc, 64));
        }
        if (lane == 0) p.sh_scale[t] = sc;
    }

    const int r_begin = blockIdx.x * ROWS_A;
    if (r_begin >= I) return;
    const int r_end = min(I, r_begin + ROWS_A);
    const RowMap m = row_map(p.hidden);
    const int lr = lane / m.L, lp = lane % m.L;
    float xr[NK > 0 ? NK : 1][32];
    load_parts<NK>(xr, xt, m, lp, f16);
    const int64_t g_row = (int64_t)(p.hidden / block_size(gt)) * block_bytes(gt);
    const int64_t u_row = (int64_t)(p.hidden / block_size(ut)) * block_bytes(ut);

    for (int rb = r_begin + wave * m.rpi; rb < r_end; rb += 4 * m.rpi) {
        const int r = rb + lr;
        const bool valid = (lane < m.rpi * m.L) && r < r_end;
        float pg = 0.0f, pu = 0.0f;
        if (valid) {
            pg = lane_dot<NK>(gt, G + r * g_row, m, lp, xr, xt, f16);
            pu = lane_dot<NK>(ut, U + r * u_row, m, lp, xr, xt, f16);
        }
        float g = group_sum(pg, m.L), u = group_sum(pu, m.L);
        if (valid && lp == 0) {
            float a;
            if (f16) {
                g = round16(g); u = round16(u);
                const float sig = round16(sigmoid_ref(g));
                const float silu = round16(g * sig);
                a = round16(silu * u);
            } else {
                a = (g * sigmoid_ref(g)) * u;
            }
            p.act[((int64_t)t * p.S + s) * p.Imax + r] = a;
        }
    }
}

// ------------------------------------------------------------ kernel B

template <int NK>
__global__ __launch_bounds__(256) void k_down_combine(DecodeParams p) {
    const int t = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int w_begin = blockIdx.x * ROWS_B + wave * ROWS_W;   // this wavefront's rows
    float acc[ROWS_W];
#pragma unroll
    for (int i = 0; i < ROWS_W; ++i) acc[i] = 0.0f;

    for (int s = 0; s < p.S; ++s) {
        const bool shared = (s == p.top_k);
        const uint8_t* D;
        int dt, I;
        float w;
        if (shared) {
            D = p.sh_down; dt = p.sh_down_type; I = p.sh_inter; w = p.sh_scale[t];
        } else {
            const int e = p.ids[t * p.top_k + s];
            if (e < 0 || e >= p.n_experts) continue;
            D = p.down + (int64_t)e * p.down_eb; dt = p.down_type; I = p.inter;
            w = p.weights[t * p.top_k + s];
        }
        const bool f16 = p.fp16 && !shared;
        const RowMap m = row_map(I);
        const int lr = lane / m.L, lp = lane % m.L;
        const float* at = p.act + ((int64_t)t * p.S + s) * p.Imax;
        float xr[NK > 0 ? NK : 1][32];
        load_parts<NK>(xr, at, m, lp, false);
        const int64_t d_row = (int64_t)(I / block_size(dt)) * block_bytes(dt);
        for (int c = 0; c < ROWS_W; c += m.rpi) {
            const int r = w_begin + c + lr;
            const bool valid = (lane < m.rpi * m.L) && (c + lr) < ROWS_W && r < p.hidden;
            const float part = valid ? lane_dot<NK>(dt, D + r * d_row, m, lp, xr, at, f16) : 0.0f;
            float ys = group_sum(part, m.L);
            if (f16) ys = round16(ys);
            if (valid && lp == 0 && !isfinite(ys)) atomicOr(&p.flags[FLAG_NONFINITE], 1);
#pragma unroll
            for (int i = 0; i < ROWS_W; ++i) {
                const int rel = i - c;
                if (rel >= 0 && rel < m.rpi) {
                    const float v = __shfl(ys, rel * m.L, 64);
                    acc[i] = __fadd_rn(acc[i], __fmul_rn(w, v));
                }
            }
        }
    }
    if (lane < ROWS_W) {
        float v = acc[0];
#pragma unroll
        for (int i = 1; i < ROWS_W; ++i)
            if (lane == i) v = acc[i];
        const int r = w_begin + lane;
        if (r < p.hidden) {
            p.y[(int64_t)t * p.hidden + r] = v;
            if (!isfinite(v)) atomicOr(&p.flags[FLAG_NONFINITE], 1);
        }
    }
}

static int nk_for(int cols) {
    const int P = cols / 32;
    int L = 1;
    while (L < P && L < 64) L <<= 1;
    return (P + L - 1) / L;
}

hipError_t launch_decode_generic(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    const int nk_a = nk_for(p.hidden);
    const int nk_b = std::max(nk_for(p.inter), p.has_shared ? nk_for(p.sh_inter) : 1);
    dim3 ga((p.Imax + ROWS_A - 1) / ROWS_A, p.S, p.n_tokens);
    dim3 gb((p.hidden + ROWS_B - 1) / ROWS_B, p.n_tokens);
#define MQH_LAUNCH_A(NK)                                                                                     \
    do {                                                                                                     \
        if (ev.armed_a())                                                                                    \
            hipExtLaunchKernelGGL((k_gate_up<NK>), ga, dim3(256), 0, stream, ev.a_start, ev.a_stop, 0, p);   \
        else                                                                                                 \
            hipLaunchKernelGGL((k_gate_up<NK>), ga, dim3(256), 0, stream, p);                                \
    } while (0)
#define MQH_LAUNCH_B(NK)                                                                                     \
    do {                                                                                                     \
        if (ev.armed_b())                                                                                    \
            hipExtLaunchKernelGGL((k_down_combine<NK>), gb, dim3(256), 0, stream, ev.b_start, ev.b_stop, 0, p); \
        else                                                                                                 \
            hipLaunchKernelGGL((k_down_combine<NK>), gb, dim3(256), 0, stream, p);                           \
    } while (0)
    if (nk_a == 1) MQH_LAUNCH_A(1);
    else if (nk_a == 2) MQH_LAUNCH_A(2);
    else if (nk_a <= 4) MQH_LAUNCH_A(4);
    else MQH_LAUNCH_A(0);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (nk_b == 1) MQH_LAUNCH_B(1);
    else if (nk_b == 2) MQH_LAUNCH_B(2);
    else if (nk_b <= 4) MQH_LAUNCH_B(4);
    else MQH_LAUNCH_B(0);
#undef MQH_LAUNCH_A
#undef MQH_LAUNCH_B
    return hipGetLastError();
}

}  // namespace mqh
