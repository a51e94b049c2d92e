// moe_fused.hip -- single-launch fused MoE decode for gfx950.
//
// One launch computes, for T tokens, all routed experts plus the shared expert
// and the weighted combine (same result as kernels A+B of moe_decode.hip, see
// that file for the formula and reference lines).  Workgroups take a ticket
// from a global counter when they start:
//
//   tickets [0, n_a)        phase A: 32 intermediate rows of one (token, slot):
//                           gate/up dot products, silu(g)*u, then the 32
//                           activations are split into int8 digits and
//                           published to the workspace.
//   tickets [n_a, n_a+n_b)  phase B: RB output rows of one token: the down rows
//                           of every slot are loaded into registers first,
//                           then the workgroup waits until all phase-A
//                           workgroups have published, then computes the down
//                           dot products and the combine sum_s w_s * y_s in
//                           top-k order (+ the sigmoid-gated shared expert).
//
// A phase-B workgroup only exists after every phase-A ticket was taken, i.e.
// after every phase-A workgroup is running, and phase A never waits, so the
// wait always ends; it is also bounded (FLAG_TIMEOUT) so a kernel can never
// hang.  The last workgroup to leave resets the counters, so the next launch
// on the stream (or the next replay of a captured graph) starts from zero.
//
// The down-projection weights are in flight while phase A runs, so the whole
// layer's quantized bytes stream from HBM concurrently in one launch.
//
// Dot products use kquant_dot.h (exact int8 digit dot products).  Fast-path
// conditions (checked on the host): FP32 graph, K-quant types Q3_K/Q4_K/Q5_K/
// Q6_K, hidden and intermediate in {256, 512, 1024, 2048}, shared expert (if
// any) with the routed intermediate size.
#include "kquant_dot.h"
#include "moe_decode.h"

namespace mqh {

constexpr int FA_ROWS = 32;         // intermediate rows per phase-A workgroup
constexpr int MAX_SLOTS_PER_WAVE = 3;
constexpr int MAX_H = 2048;
constexpr int SPIN_LIMIT = 1 << 17;

__device__ __forceinline__ float sigmoid_f(float g) { return 1.0f / (1.0f + expf(-g)); }

__device__ __forceinline__ float sigmoid_stable_f(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

// Digit view of an activation vector: planes int8 [3][n], xs float [n/32]
// (2^e / 16384), colsum float [n/16].
struct DigitView {
    const int8_t* dig;
    const float* xs;
    const float* sum;
    int n;
};

__device__ __forceinline__ void load_chunkx(const DigitView& v, int type, int blk, int c, ChunkX& x) {
#pragma unroll
    for (int run = 0; run < RUNS; ++run) {
        const int col = blk * 256 + run_col(type, c, run);
#pragma unroll
        for (int d = 0; d < NDIG; ++d) {
            const uint4 q = *(const uint4*)(v.dig + (int64_t)d * v.n + col);
            x.d[d][4 * run + 0] = q.x; x.d[d][4 * run + 1] = q.y;
            x.d[d][4 * run + 2] = q.z; x.d[d][4 * run + 3] = q.w;
        }
        x.xs[run] = v.xs[col >> 5];
        x.sum[run] = v.sum[col >> 4];
    }
}

struct FusedParams {
    DecodeParams p;
    int* counters;          // [0] ticket, [1] phase-A done, [2] exit
    uint8_t* act_base;      // per (t, s): digits [3][I] | xs [I/32] | sum [I/16], stride act_stride
    int64_t act_stride;
    int n_a, n_b;
    int rb;                 // output rows per phase-B workgroup
};

__device__ __forceinline__ DigitView act_view(const FusedParams& f, int t, int s) {
    const int I = f.p.inter;
    const uint8_t* base = f.act_base + ((int64_t)t * f.p.S + s) * f.act_stride;
    DigitView v;
    v.dig = (const int8_t*)base;
    v.xs = (const float*)(base + 3 * I);
    v.sum = (const float*)(base + 3 * I + I / 8);
    v.n = I;
    return v;
}

// Split n = 32*k values (one per thread i < n, value v) into digits stored at
// dig/xs/sum.  Called by whole wavefronts; lanes with i >= n pass v = 0.
__device__ __forceinline__ void publish_digits(float v, int i, int n, int8_t* dig, float* xs, float* sum) {
    float amax = fabsf(v);
    for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    float s16 = v;
    for (int off = 1; off < 16; off <<= 1) s16 += __shfl_xor(s16, off, 64);
    if (i < n) {
        const int e = digit_exp(amax);
        int8_t d0, d1, d2;
        split_digits(v, e, d0, d1, d2);
        dig[i] = d0;
        dig[n + i] = d1;
        dig[2 * n + i] = d2;
        if ((i & 31) == 0) xs[i >> 5] = ldexpf(1.0f, e - 14);
        if ((i & 15) == 0) sum[i >> 4] = s16;
    }
}

// ------------------------------------------------------------------ phase A

// Digits of token x (H values, fp32) into LDS: planes [3][H], xs [H/32],
// 16-column sums [H/16].  Whole workgroup; H in {256..2048} so a thread
// holds H/256 <= 8 consecutive values.
__device__ __forceinline__ void x_digits_to_lds(const float* xt, int H, int8_t* dig, float* xs, float* sum) {
    const int per = H / 256;
    const int i0 = threadIdx.x * per;
    float v[8], amax = 0.0f, ssum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        v[k] = k < per ? xt[i0 + k] : 0.0f;
        amax = fmaxf(amax, fabsf(v[k]));
        ssum += v[k];
    }
    const int tpg = 32 / per;                    // threads per 32-column group
    for (int off = 1; off < tpg; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const int tps = 16 / per;                    // threads per 16-column run
    for (int off = 1; off < tps; off <<= 1) ssum += __shfl_xor(ssum, off, 64);
    const int e = digit_exp(amax);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if (k < per) {
            int8_t d0, d1, d2;
            split_digits(v[k], e, d0, d1, d2);
            dig[i0 + k] = d0;
            dig[H + i0 + k] = d1;
            dig[2 * H + i0 + k] = d2;
        }
    }
    if ((i0 & 31) == 0) xs[i0 >> 5] = ldexpf(1.0f, e - 14);
    if ((i0 & 15) == 0) sum[i0 >> 4] = ssum;
}

// Phase A for gate/up type T: 32 intermediate rows of one (token, slot).
template <int T>
__device__ void phase_a(const FusedParams& f, int t, int s, int rc, const uint8_t* G, const uint8_t* U, bool bad,
                        int8_t* lds_dig, float* lds_xs, float* lds_sum, float* lds_act) {
    const DecodeParams& p = f.p;
    constexpr int N = RawOf<T>::N;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = p.hidden;
    const float* xt = p.x + (int64_t)t * H;

    // lane -> (gate/up half, row within iteration, chunk)
    const int CPR = H / CHUNK;                  // chunks per row: 4..32
    const int RPH = 32 / CPR;                   // rows per half-wave iteration
    const int half = lane >> 5, li = lane & 31;
    const int rr = li / CPR, ci = li % CPR;
    const int blk = ci >> 2, c = ci & 3;
    const uint8_t* M = half ? U : G;
    const int64_t row_bytes = (int64_t)(H / 256) * block_bytes(T);
    const int iters = FA_ROWS / (4 * RPH);      // 1..8
    const int row0 = rc * FA_ROWS + wave * RPH * iters;

    // 1. issue every weight load of this lane (up to 8 rows)
    uint32_t raw[8][N];
#pragma unroll
    for (int it = 0; it < 8; ++it)
        if (it < iters)
            load_chunk<T>(M + (int64_t)(row0 + it * RPH + rr) * row_bytes + blk * block_bytes(T), c, raw[it]);

    // 2. activation digits of token t (overlaps the loads in flight)
    x_digits_to_lds(xt, H, lds_dig, lds_xs, lds_sum);
    __syncthreads();

    // 3. this lane's activation operand, the same for all its rows
    ChunkX x;
    DigitView xv;
    xv.dig = lds_dig; xv.xs = lds_xs; xv.sum = lds_sum; xv.n = H;
    load_chunkx(xv, T, blk, c, x);

    // 4. dot products and SwiGLU; the up row's sum comes from lane + 32
#pragma unroll
    for (int it = 0; it < 8; ++it) {
        if (it < iters) {
            float part = bad ? 0.0f : chunk_dot<T>(raw[it], c, x);
            part = group_sum(part, CPR);
            const float other = __shfl_down(part, 32, 64);
            if (half == 0 && ci == 0) {
                const float g = part, u = other;
                lds_act[wave * RPH * iters + it * RPH + rr] = (g * sigmoid_f(g)) * u;
            }
        }
    }
}

__device__ __forceinline__ void phase_a_item(const FusedParams& f, int item, int8_t* lds_dig, float* lds_xs, float* lds_sum,
                             float* lds_act, int at) {
    const DecodeParams& p = f.p;
    const int chunks_i = p.inter / FA_ROWS;
    const int t = item / (p.S * chunks_i);
    const int s = (item / chunks_i) % p.S;
    const int rc = item % chunks_i;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool shared = (s == p.top_k);

    const uint8_t *G, *U;
    bool bad = false;
    if (shared) {
        G = p.sh_gate; U = p.sh_up;
    } else {
        int e = p.ids[t * p.top_k + s];
        if (e < 0 || e >= p.n_experts) { bad = true; e = 0; }
        G = p.gate + (int64_t)e * p.gate_eb; U = p.up + (int64_t)e * p.up_eb;
        if (bad && threadIdx.x == 0) atomicOr(&p.flags[FLAG_BAD_ID], 1);
    }
    switch (at) {
        case T_Q4_K: phase_a<T_Q4_K>(f, t, s, rc, G, U, bad, lds_dig, lds_xs, lds_sum, lds_act); break;
        case T_Q5_K: phase_a<T_Q5_K>(f, t, s, rc, G, U, bad, lds_dig, lds_xs, lds_sum, lds_act); break;
        case T_Q6_K: phase_a<T_Q6_K>(f, t, s, rc, G, U, bad, lds_dig, lds_xs, lds_sum, lds_act); break;
        default: phase_a<T_Q3_K>(f, t, s, rc, G, U, bad, lds_dig, lds_xs, lds_sum, lds_act); break;
    }

    // shared slot, first row chunk: the sigmoid gate of the shared expert
    if (shared && rc == 0 && wave == 0) {
        const float* xt = p.x + (int64_t)t * p.hidden;
        float sc = 1.0f;
        if (p.sh_gate_inp) {
            float acc = 0.0f;
            for (int k = lane; k < p.hidden; k += 64) acc = fmaf(xt[k], p.sh_gate_inp[k], acc);
            sc = sigmoid_stable_f(group_sum(acc, 64));
        }
        if (lane == 0) p.sh_scale[t] = sc;
    }
    __syncthreads();

    // publish the 32 activations as digits (wave 0, lanes 0..31)
    if (wave == 0) {
        const DigitView av = act_view(f, t, s);
        const float a = lane < FA_ROWS ? lds_act[lane] : 0.0f;
        publish_digits(a, rc * FA_ROWS + lane, lane < FA_ROWS ? p.inter : 0, (int8_t*)av.dig, (float*)av.xs,
                       (float*)av.sum);
    }
}

// ------------------------------------------------------------------ phase B

template <int DT>
__device__ void phase_b(const FusedParams& f, int item, float* lds_y, int* lds_flag) {
    const DecodeParams& p = f.p;
    const int rows_per_token = p.hidden / f.rb;
    const int t = item / rows_per_token;
    const int r0 = (item % rows_per_token) * f.rb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int I = p.inter;
    const int CPR = I / CHUNK;                  // 4..32
    const int rr = lane / CPR, ci = lane % CPR; // rr < rb
    const int blk = ci >> 2, c = ci & 3;

    // 1. down rows of this wave's slots (s = wave, wave + 4, wave + 8) into registers
    constexpr int N = RawOf<DT>::N;
    constexpr int64_t BB = block_bytes(DT);
    const int64_t row_bytes = (int64_t)(I / 256) * BB;
    uint32_t raw[MAX_SLOTS_PER_WAVE][N];
#pragma unroll
    for (int k = 0; k < MAX_SLOTS_PER_WAVE; ++k) {
        const int s = wave + 4 * k;
        if (s < p.S) {
            const uint8_t* D;
            if (s == p.top_k) {
                D = p.sh_down;
            } else {
                int e = p.ids[t * p.top_k + s];
                if (e < 0 || e >= p.n_experts) e = 0;   // flagged in phase A; weight zeroed below
                D = p.down + (int64_t)e * p.down_eb;
            }
            load_chunk<DT>(D + (int64_t)(r0 + rr) * row_bytes + blk * BB, c, raw[k]);
        }
    }

    // 2. wait for every phase-A workgroup (bounded)
    if (threadIdx.x == 0) {
        int ok = 1, spins = 0;
        while (__hip_atomic_load(&f.counters[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < f.n_a) {
            __builtin_amdgcn_s_sleep(2);
            if (++spins > SPIN_LIMIT) {
                ok = 0;
                atomicOr(&p.flags[FLAG_TIMEOUT], 1);
                break;
            }
        }
        *lds_flag = ok;
    }
    __syncthreads();
    __threadfence();
    if (!*lds_flag) return;

    // 3. down dot products per slot
#pragma unroll
    for (int k = 0; k < MAX_SLOTS_PER_WAVE; ++k) {
        const int s = wave + 4 * k;
        if (s < p.S) {
            ChunkX x;
            load_chunkx(act_view(f, t, s), DT, blk, c, x);
            float part = chunk_dot<DT>(raw[k], c, x);
            part = group_sum(part, CPR);
            if (ci == 0) lds_y[rr * 16 + s] = part;
        }
    }
    __syncthreads();

    // 4. combine in top-k order, then the shared expert
    if (threadIdx.x < f.rb) {
        const int r = threadIdx.x;
        float acc = 0.0f;
        for (int s = 0; s < p.top_k; ++s) {
            const int e = p.ids[t * p.top_k + s];
            const float w = (e >= 0 && e < p.n_experts) ? p.weights[t * p.top_k + s] : 0.0f;
            acc = __fadd_rn(acc, __fmul_rn(w, lds_y[r * 16 + s]));
        }
        if (p.has_shared) acc = __fadd_rn(acc, __fmul_rn(p.sh_scale[t], lds_y[r * 16 + p.top_k]));
        p.y[(int64_t)t * p.hidden + r0 + r] = acc;
        if (!isfinite(acc)) atomicOr(&p.flags[FLAG_NONFINITE], 1);
    }
}

// AT: gate/up type, DT: down type, of every slot (routed and shared).
template <int AT, int DT>
__global__ __launch_bounds__(256) void k_moe_fused(FusedParams f) {
    __shared__ int s_ticket, s_flag;
    __shared__ __attribute__((aligned(16))) int8_t lds_dig[3 * MAX_H];
    __shared__ float lds_xs[MAX_H / 32];
    __shared__ float lds_sum[MAX_H / 16];
    __shared__ float lds_act[FA_ROWS];
    __shared__ float lds_y[16 * 16];

    if (threadIdx.x == 0) s_ticket = atomicAdd(&f.counters[0], 1);
    __syncthreads();
    const int ticket = s_ticket;
    if (ticket < f.n_a) {
        phase_a_item(f, ticket, lds_dig, lds_xs, lds_sum, lds_act, AT);
        // publish: every thread's stores reach agent scope before the count
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(&f.counters[1], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    } else if (ticket < f.n_a + f.n_b) {
        phase_b<DT>(f, ticket - f.n_a, lds_y, &s_flag);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int left = __hip_atomic_fetch_add(&f.counters[2], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (left == f.n_a + f.n_b - 1) {
            __hip_atomic_store(&f.counters[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&f.counters[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&f.counters[2], 0, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

static bool kq_fast_type(int t) { return t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }
static bool fast_dim(int n) { return n == 256 || n == 512 || n == 1024 || n == 2048; }

bool fused_supported(const DecodeParams& p) {
    if (p.fp16) return false;
    if (!fast_dim(p.hidden) || !fast_dim(p.inter)) return false;
    if (p.S > 4 * MAX_SLOTS_PER_WAVE) return false;
    int at = -1, dt = -1;
    if (p.top_k > 0) {
        if (!(kq_fast_type(p.gate_type) && p.up_type == p.gate_type && kq_fast_type(p.down_type))) return false;
        at = p.gate_type;
        dt = p.down_type;
    }
    if (p.has_shared) {
        if (p.sh_inter != p.inter) return false;
        if (!(kq_fast_type(p.sh_gate_type) && p.sh_up_type == p.sh_gate_type && kq_fast_type(p.sh_down_type)))
            return false;
        if ((at >= 0 && p.sh_gate_type != at) || (dt >= 0 && p.sh_down_type != dt)) return false;
    }
    return true;
}

template <int AT>
static void launch_at(int dt, const dim3& grid, hipStream_t stream, const FusedParams& f) {
    switch (dt) {
        case T_Q4_K: hipLaunchKernelGGL((k_moe_fused<AT, T_Q4_K>), grid, dim3(256), 0, stream, f); break;
        case T_Q5_K: hipLaunchKernelGGL((k_moe_fused<AT, T_Q5_K>), grid, dim3(256), 0, stream, f); break;
        case T_Q6_K: hipLaunchKernelGGL((k_moe_fused<AT, T_Q6_K>), grid, dim3(256), 0, stream, f); break;
        default: hipLaunchKernelGGL((k_moe_fused<AT, T_Q3_K>), grid, dim3(256), 0, stream, f); break;
    }
}

hipError_t launch_decode_fused(const DecodeParams& p, int* counters, hipStream_t stream) {
    FusedParams f;
    f.p = p;
    f.counters = counters;
    f.act_base = (uint8_t*)p.act;
    f.act_stride = (int64_t)p.Imax * 4;
    f.n_a = p.n_tokens * p.S * (p.inter / FA_ROWS);
    f.rb = 64 / (p.inter / CHUNK);
    f.n_b = p.n_tokens * (p.hidden / f.rb);
    const int at = p.top_k > 0 ? p.gate_type : p.sh_gate_type;
    const int dt = p.top_k > 0 ? p.down_type : p.sh_down_type;
    const dim3 grid(f.n_a + f.n_b);
    switch (at) {
        case T_Q4_K: launch_at<T_Q4_K>(dt, grid, stream, f); break;
        case T_Q5_K: launch_at<T_Q5_K>(dt, grid, stream, f); break;
        case T_Q6_K: launch_at<T_Q6_K>(dt, grid, stream, f); break;
        default: launch_at<T_Q3_K>(dt, grid, stream, f); break;
    }
    return hipGetLastError();
}

}  // namespace mqh
