// moe_fast.hip -- the decode fast path: fused quantized SwiGLU experts for a few
// tokens, as two kernels with no inter-workgroup synchronisation.
//
// Same result as the generic kernels of moe_decode.hip (formula and reference
// lines there): for every token t and slot s (the top-k routed experts in order,
// then the optional shared expert)
//   act[t,s] = silu(W_gate x_t) * (W_up x_t)
//   y[t]     = sum_s w[t,s] * W_down act[t,s]   (+ sigmoid(x_t . g_inp) * shared)
//
// Kernel A  grid (ceil(items / W), T), W waves per workgroup.  An item is the
//           64/(H/64) rows of the gate and up matrices that one wave covers, of
//           one slot; a token's S * I / (64/(H/64)) items are dealt to the
//           workgroups in order, W chosen per launch so the workgroups spread
//           evenly over the CUs (top-8 + shared at H 2048, I 512: 2,304 items,
//           256 workgroups of 9 waves).  The token's activation digits go to
//           LDS, each lane keeps the digits of its 64 columns in registers, and
//           the gate and up rows' quantized bytes are all requested before any
//           arithmetic.  Each item writes its SwiGLU activations in FP32.
// Kernel B  grid (H / RB, T), 64*S threads: wave s splits slot s's activations
//           into digits in LDS (while its weights are in flight), computes the
//           down rows of slot s for RB output rows, then the workgroup combines
//           the slots in top-k order (+ shared) from LDS.
//
// Lanes follow kquant_lane.h: lane k of a super-block owns 64 of its weights,
// so a row of C columns is C/64 consecutive lanes and an instruction covers
// 64/(C/64) rows.  Every weight byte is read once per (token, slot).
//
// Supported (checked by fast_supported): the FP32 graph, and the FP16 graph
// (fp16_graph = 1: FP16 operands and rounding points for the routed experts);
// types Q3_K/Q4_K/Q5_K/Q6_K/Q8_0
// with gate type == up type; hidden and intermediate in {256, 512, 1024, 2048};
// at most 16 slots (12 at intermediate 2048: kernel B's digit LDS); a shared
// expert with the routed intermediate size and the routed types or Q6_K.
#include <hip/hip_ext.h>

#include <algorithm>
#include <atomic>
#include <climits>

#include "kquant_lane.h"
#include "moe_decode.h"
#include "route_topk.h"

namespace mqh {

constexpr int FAST_MAX_SLOTS = 16;
constexpr int RUN = 16;          // activation digit run (columns sharing one scale)

// What a fast kernel needs before its first loads: the token, the expert ids,
// the activations and the work split.  The kernels take these as their
// leading scalar arguments (the rest of DecodeParams follows), so that the
// build's kernel-argument preloading puts them in scalar registers before the
// first instruction: the expert-id load goes out at once instead of after a
// round trip to the argument block.
struct DecodeHot {
    const float* x;
    const int32_t* ids;
    float* act;
    const float* weights;
    const float* sh_gate_inp;
    int top_k, S, has_shared, n_experts, a_inter, a_waves;
    // kernel B: the shared expert's gate (from kernel A) and down weights
    const float* sh_scale;
    const uint8_t* sh_down;
    // kernel A (given ids): the shared expert's gate and up weights
    const uint8_t* sh_gate;
    const uint8_t* sh_up;
};

// silu(g) * u with the hardware exp2 and reciprocal (a few ulp; the FP32 graph
// of moe_quant_dot.cpp:200-206 with std::exp and a division)
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);   // exp(-g)
    return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

__device__ __forceinline__ float sigmoid_stable(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

// Sum over aligned groups of W lanes (W = 4 .. 64); every lane of a group
// receives the group's sum, in a fixed butterfly order (deterministic).
// Partners within 32 lanes come from ds_swizzle (bit mode: lane ^ m), across
// the halves from ds_bpermute.  DPP row operations would keep this in the VALU,
// but hipcc's DPP-combined form of this reduction gave intermittently wrong
// sums on gfx950, so the LDS crossbar forms are used.
template <int M>
__device__ __forceinline__ float swz_xor(float v) {
    static_assert(M > 0 && M < 32, "swizzle xor mask");
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (M << 10)));
}

template <int W>
__device__ __forceinline__ float lane_group_sum(float v) {
    static_assert(W >= 4 && W <= 64 && (W & (W - 1)) == 0, "group width");
    v += swz_xor<1>(v);
    v += swz_xor<2>(v);
    if constexpr (W > 4) v += swz_xor<4>(v);
    if constexpr (W > 8) v += swz_xor<8>(v);
    if constexpr (W > 16) v += swz_xor<16>(v);
    if constexpr (W > 32) v += __shfl_xor(v, 32, 64);
    return v;
}

// Wave-uniform value held in a VGPR, as a scalar.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Max |v| and sum of a 16-value run, in the order every digit producer uses
// (four-value groups, left to right).
__device__ __forceinline__ void run_stats(const float4* q, float& amax, float& sum) {
    amax = 0.0f;
    sum = 0.0f;
#pragma unroll
    for (int i = 0; i < RUN / 4; ++i) {
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(q[i].x), fabsf(q[i].y)), fmaxf(fabsf(q[i].z), fabsf(q[i].w))));
        sum += (q[i].x + q[i].y) + (q[i].z + q[i].w);
    }
}

// Two digit planes of four values, one byte each per word.
__device__ __forceinline__ uint2 split4(float4 v, float inv) {
    const uint32_t a = split2(v.x, inv), b = split2(v.y, inv), c = split2(v.z, inv), d = split2(v.w, inv);
    return make_uint2((a & 0xFFu) | ((b & 0xFFu) << 8) | ((c & 0xFFu) << 16) | ((d & 0xFFu) << 24),
                      (a >> 8) | ((b >> 8) << 8) | ((c >> 8) << 16) | ((d >> 8) << 24));
}

// Kernel B's digits of one slot's I FP32 activations, in two steps so the
// loads go out before the weight loads and the arithmetic runs while those are
// in flight.  Lane l owns columns [l*V, (l+1)*V), V = I/64, and reads the
// whole 16-column run(s) it lies in: every lane of a run takes the same max and
// sum (run_stats), and for V < 16 picks its own four-value groups out of the
// run by lane-constant selects.
template <int I>
struct ActRegs {
    static constexpr int V = I / 64;
    static constexpr int NQ = V >= RUN ? V / 4 : RUN / 4;   // float4 per lane
    float4 q[NQ];
};

template <int I>
__device__ __forceinline__ void act_load(const float* a, int lane, ActRegs<I>& r) {
    constexpr int V = ActRegs<I>::V;
    const float* src = a + (V >= RUN ? lane * V : (lane * V) & ~(RUN - 1));
#pragma unroll
    for (int i = 0; i < ActRegs<I>::NQ; ++i) r.q[i] = *(const float4*)(src + 4 * i);
}

// r.q[g] for a lane-dependent g < RUN / 4, by selects (an indexed read of the
// register array makes the compiler put it in scratch memory)
template <int NQ>
__device__ __forceinline__ float4 pick_group(const float4 (&q)[NQ], int g) {
    static_assert(NQ == RUN / 4, "one run of float4 groups");
    const float4 lo = (g & 1) ? q[1] : q[0], hi = (g & 1) ? q[3] : q[2];
    return (g & 2) ? hi : lo;
}

template <int I>
__device__ __forceinline__ void act_digits_lds(const ActRegs<I>& r, int lane, int8_t* planes, float* xs16,
                                               float* sum16) {
    constexpr int V = ActRegs<I>::V;
    if constexpr (V >= RUN) {
#pragma unroll
        for (int run = 0; run < V / RUN; ++run) {
            const int c0 = lane * V + run * RUN;
            float amax, sum;
            run_stats(r.q + 4 * run, amax, sum);
            const float inv = digit_inv(amax);
            uint4 lo, hi;
            uint2 w = split4(r.q[4 * run + 0], inv); lo.x = w.x; hi.x = w.y;
            w = split4(r.q[4 * run + 1], inv); lo.y = w.x; hi.y = w.y;
            w = split4(r.q[4 * run + 2], inv); lo.z = w.x; hi.z = w.y;
            w = split4(r.q[4 * run + 3], inv); lo.w = w.x; hi.w = w.y;
            *(uint4*)(planes + c0) = lo;
            *(uint4*)(planes + I + c0) = hi;
            xs16[c0 / RUN] = digit_scale(amax);
            sum16[c0 / RUN] = sum;
        }
    } else {
        const int c0 = lane * V, g0 = (c0 & (RUN - 1)) / 4;   // first own four-value group of the run
        float amax, sum;
        run_stats(r.q, amax, sum);
        const float inv = digit_inv(amax);
        uint32_t lo[V / 4], hi[V / 4];
#pragma unroll
        for (int j = 0; j < V / 4; ++j) {
            const float4 v = pick_group(r.q, g0 + j);
            const uint2 w = split4(v, inv);
            lo[j] = w.x;
            hi[j] = w.y;
        }
        if constexpr (V == 8) {
            *(uint2*)(planes + c0) = make_uint2(lo[0], lo[1]);
            *(uint2*)(planes + I + c0) = make_uint2(hi[0], hi[1]);
        } else {
            static_assert(V == 4, "intermediate 256 or 512 below a run per lane");
            *(uint32_t*)(planes + c0) = lo[0];
            *(uint32_t*)(planes + I + c0) = hi[0];
        }
        if (g0 == 0) {
            xs16[c0 / RUN] = digit_scale(amax);
            sum16[c0 / RUN] = sum;
        }
    }
}

// The FP16 graph's activations of one slot into LDS as FP16 bits: kernel A
// rounded them to FP16 already, so the conversion is exact.  Lane l writes its
// own V = I/64 columns (picked out of its run as in act_digits_lds).
template <int I>
__device__ __forceinline__ void act_halves_lds(const ActRegs<I>& r, int lane, uint16_t* dst) {
    constexpr int V = ActRegs<I>::V;
    const int c0 = lane * V;
    if constexpr (V >= RUN) {
#pragma unroll
        for (int i = 0; i < V / 8; ++i) {
            const float4 a = r.q[2 * i], b = r.q[2 * i + 1];
            *(uint4*)(dst + c0 + 8 * i) = make_uint4(pack_rn16(a.x, a.y), pack_rn16(a.z, a.w), pack_rn16(b.x, b.y),
                                                     pack_rn16(b.z, b.w));
        }
    } else {
        const int g0 = (c0 & (RUN - 1)) / 4;   // first own four-value group of the run
        uint32_t w[V / 2];
#pragma unroll
        for (int j = 0; j < V / 4; ++j) {
            const float4 v = pick_group(r.q, g0 + j);
            w[2 * j] = pack_rn16(v.x, v.y);
            w[2 * j + 1] = pack_rn16(v.z, v.w);
        }
        if constexpr (V == 8) *(uint4*)(dst + c0) = make_uint4(w[0], w[1], w[2], w[3]);
        else *(uint2*)(dst + c0) = make_uint2(w[0], w[1]);
    }
}

// LDS bytes of one slot's digits in kernel B: planes [2][I], run scales and sums.
__host__ __device__ constexpr int act_lds_bytes(int inter) { return 2 * inter + 2 * (inter / RUN) * 4; }

// Digits of the H values of token x into LDS: thread i (i < NT = H/4) holds
// values 4i .. 4i+3, loaded early by the caller; x_digits splits them and
// writes the two planes, run scales and run sums.
template <int H, int NT>
__device__ __forceinline__ void x_digits(float4 v, int8_t* planes, float* xs16, float* sum16) {
    static_assert(H / NT == 4, "four values per thread");
    const int i0 = threadIdx.x * 4;
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    float s = (v.x + v.y) + (v.z + v.w);
    // 4 threads per 16-column run (lane-xor swizzles: no address arithmetic)
    amax = fmaxf(amax, swz_xor<1>(amax));
    s += swz_xor<1>(s);
    amax = fmaxf(amax, swz_xor<2>(amax));
    s += swz_xor<2>(s);
    static_assert(RUN / 4 == 4, "two swizzle steps cover a run");
    const float inv = digit_inv(amax);
    const uint32_t a = split2(v.x, inv), b = split2(v.y, inv), c = split2(v.z, inv), d = split2(v.w, inv);
    *(uint32_t*)(planes + i0) = (a & 0xFFu) | ((b & 0xFFu) << 8) | ((c & 0xFFu) << 16) | ((d & 0xFFu) << 24);
    *(uint32_t*)(planes + H + i0) = (a >> 8) | ((b >> 8) << 8) | ((c >> 8) << 16) | ((d >> 8) << 24);
    if ((i0 & (RUN - 1)) == 0) {
        xs16[i0 / RUN] = digit_scale(amax);
        sum16[i0 / RUN] = s;
    }
}

// ---------------------------------------------------------------- kernel A

// Kernel A of the two-kernel path.  An item is RPI = 64 / LPR rows (LPR =
// hidden / 64 lanes per row) of the gate and of the up matrix of one slot, one
// wave's work.  Token t's S * inter / RPI items go to workgroups of
// blockDim.x / 64 waves in order (grid (ceil(items / waves), T)); the waves of
// a workgroup share the token's digits in LDS.  The token's last workgroup
// also computes the shared expert's sigmoid gate.

template <int H, bool F16G>
struct SharedX {
    __attribute__((aligned(16))) int8_t planes[2 * H];
    float xs16[H / RUN];
    float sum16[H / RUN];
    float s_gate[16];
    __attribute__((aligned(16))) uint16_t x16[F16G ? H : 8];   // the FP16 graph's token (FP16 bits)
    float half_dot[2][64 / (H / 64)];   // a split shared item: its gate and up row dots
    int half_done;                      // and how many of its two waves have written theirs
};

// The shared expert's scale: sigmoid(x . g_inp) (shared_expert.py:221-251)
// or 1, once per token, by every wave of the token's last workgroup
// (scale_wg); the first NX threads hold 4 products each.
template <int NX, int H, bool F16G>
__device__ __forceinline__ void shared_scale(const DecodeParams& p, SharedX<H, F16G>& sh, bool scale_wg, bool gate_wg,
                                             float4 xv, float4 gi) {
    if (!scale_wg) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (gate_wg && wave < NX / 64) {
        float acc = fmaf(xv.x, gi.x, xv.y * gi.y) + fmaf(xv.z, gi.z, xv.w * gi.w);
        acc = lane_group_sum<64>(acc);
        if (lane == 0) sh.s_gate[wave] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float scale = 1.0f;
        if (gate_wg) {
            float dsum = 0.0f;
#pragma unroll
            for (int w = 0; w < NX / 64; ++w) dsum += sh.s_gate[w];
            scale = sigmoid_stable(dsum);
        }
        p.sh_scale[blockIdx.z] = scale;
    }
}

// every weight load of one item's lane (type T)
template <int T, int H>
__device__ __forceinline__ void item_loads(const uint8_t* Gm, const uint8_t* Um, int row, int blk, int k,
                                           uint32_t* rg, uint32_t* ru) {
    constexpr int64_t ROW_BYTES = (int64_t)(H / 256) * unit_bytes(T);
    const int64_t off = (int64_t)row * ROW_BYTES + blk * unit_bytes(T);
    lane_load<T, true>(Gm + off, k, rg);
    lane_load<T, true>(Um + off, k, ru);
}

// SGT: the shared expert's gate/up type (its waves take that code path).
// ROUTED: the router's select step first (p.route_scores set, at most
// ROUTE_PROLOGUE_MAX_EXPERTS experts).  IPW: consecutive items per wave (the
// same slot: items per slot are a multiple of it), loaded together and
// sharing the wave's token operand.  SPLIT: the routed waves of a workgroup of
// top_k + 2 waves whose last two split the shared expert's item
// (gate_up_shared_half); the routed waves are dealt by slot.
template <int GT, int SGT, int LPR, bool ROUTED, bool F16G, int IPW = 1, bool SPLIT = false>
__device__ __forceinline__ void gate_up_items(const DecodeHot& h, const DecodeParams& p, SharedX<64 * LPR, F16G>& sh) {
    constexpr int H = 64 * LPR, RPI = 64 / LPR, NX = H / 4;   // NX threads hold the token, four values each
    constexpr int NA = LaneGeo<GT>::NRAW > LaneGeo<SGT>::NRAW ? LaneGeo<GT>::NRAW : LaneGeo<SGT>::NRAW;
    // workgroup x of token t: x = blockIdx.x + 8 blockIdx.y, t = blockIdx.z (a
    // single token is launched as (8, ceil(n / 8), 1): 10.06 -> 9.85 us per
    // layer against (n, 1); several tokens as (n, 1, T)).  The padding test
    // multiplies: an integer division here, ahead of the first loads, cost the
    // 16-token layer ~1.3 us
    const int t = blockIdx.z, xg = (int)blockIdx.y * 8 + (int)blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // this wave's item, slot and expert-id address, from preloaded arguments
    // (h.a_waves = blockDim.x / 64: blockDim.x is a 16-bit field that takes a
    // vector load and a full wait); items per slot are a power of two
    const int per_slot = h.a_inter / RPI;
    const int n_items = h.S * per_slot, wg_items = h.a_waves * IPW;
    // padding of the last group of eight (no division on this path)
    if (SPLIT ? xg >= per_slot : xg * wg_items >= n_items) return;
    // Items are dealt in order (a workgroup's waves take consecutive items,
    // mostly of one slot), or, with one wave per slot and one item a wave
    // (then per_slot workgroups), by slot: wave s takes slot s's row group xg.
    // A CU's nine waves are then eight routed items and the shared expert's,
    // and the SIMD that holds three of them holds the shared one, which in
    // the FP16 graph runs the cheaper integer-digit path.  (The routed
    // prologue needs consecutive slots per workgroup: it ranks only as many
    // experts as its workgroup uses.)
    const bool by_slot = SPLIT || (!ROUTED && IPW == 1 && h.a_waves == h.S);
    const int item = uniform(by_slot ? wave * per_slot + xg : (xg * h.a_waves + wave) * IPW);
    const bool live = item < h.S * per_slot;
    const int s = live ? item >> __builtin_ctz(per_slot) : 0;
    const int row0 = live ? (item & (per_slot - 1)) * RPI : 0;
    // (bitwise: a short-circuit would branch on its first kernel argument)
    const bool shared = live & (h.has_shared != 0) & (s == h.top_k);
    // the token's last workgroup
    const bool scale_wg = (h.has_shared != 0) & (SPLIT ? xg + 1 >= per_slot : (xg + 1) * wg_items >= n_items);
    const bool gate_wg = scale_wg & (h.sh_gate_inp != nullptr);

    // 1. the token's values and the expert id, together and before any branch
    // (each branch would wait for its own kernel-argument loads): threads past
    // NX re-read the last four values, outside the gate workgroup the gate
    // vector's load re-reads the token, and a wave with no id to read (shared
    // slot, past the end, routed in the prologue) reads the token's first word;
    // none of these is used.
    const float* xt = h.x + (int64_t)t * H;
    const int xi = min((int)threadIdx.x, NX - 1) * 4;
    const bool id_item = !ROUTED & live & !shared;
    const int id_raw = *(id_item ? h.ids + (t * h.top_k + s) : (const int32_t*)xt);
    const float4 xv = *(const float4*)(xt + xi);
    const float4 gi = *(const float4*)((gate_wg ? h.sh_gate_inp : xt) + xi);   // the shared expert's gate vector
    // the argument-block fields the weight addresses need, awaited together
    // with the expert id (left to itself the compiler loads the id inside the
    // branch below, after a round trip of its own for these fields)
    const uint8_t *p_gate = p.gate, *p_up = p.up;
    const uint8_t *p_sh_gate = ROUTED ? p.sh_gate : h.sh_gate, *p_sh_up = ROUTED ? p.sh_up : h.sh_up;
    const int64_t gate_eb = p.gate_eb, up_eb = p.up_eb;
    const int n_exp = ROUTED ? h.n_experts : p.n_experts;
    __asm__ volatile("" ::"s"(p_gate), "s"(p_up), "s"(p_sh_gate), "s"(p_sh_up), "s"(gate_eb), "s"(up_eb), "s"(id_raw),
                     "s"(n_exp));
    __builtin_amdgcn_sched_barrier(0);

    // The expert slices: routed expert e, the shared expert, or -- for a wave
    // past the end -- the first slice, whose first row is read and discarded.
    // Every wave issues the same loads with no branch around them: a
    // conditional load makes the compiler's wait counts conservative at the
    // join, and the token digits below would then wait for the weights.
    const uint8_t *Gm = h.top_k > 0 ? p_gate : p_sh_gate, *Um = h.top_k > 0 ? p_up : p_sh_up;
    if (shared) { Gm = p_sh_gate; Um = p_sh_up; }
    bool bad = false;
    bool route_publish = false;   // (ROUTED: the token's first workgroup writes the ids and weights)
    float route_mine = 0.0f;      // (its wave 0: lane r keeps the r-th selected score)
    if constexpr (ROUTED) {
        // routing in the prologue (router.py:140-170).  A workgroup's items are
        // consecutive, so its routed waves need the experts of ranks s_first ..
        // s_last: its first wave takes the top s_last + 1 of token t's router
        // scores (all top_k in the token's first workgroup, which also writes
        // the ids and softmax weights for the down kernel and the caller) while
        // the token's load is in flight, and hands the experts to the other
        // waves through LDS.
        __shared__ int s_rank[FAST_MAX_SLOTS];
        const int sh_ps = __builtin_ctz(per_slot);
        const int it_first = xg * h.a_waves * IPW;
        const int it_last = min(it_first + h.a_waves * IPW - 1, h.S * per_slot - 1);
        if ((it_first >> sh_ps) < h.top_k) {   // the workgroup has a routed item (uniform)
            const bool publish = xg == 0;
            route_publish = publish;
            if (wave == 0) {
                const int rounds = publish ? h.top_k : min(it_last >> sh_ps, h.top_k - 1) + 1;
                uint32_t ord[ROUTE_PROLOGUE_MAX_EXPERTS / 64];
                route_ords(p.route_scores + (int64_t)t * h.n_experts, h.n_experts, lane, ord);
                for (int r = 0; r < rounds; ++r) {
                    uint32_t best;
                    const int win = route_next(ord, lane, best);
                    if (lane == r) route_mine = ord_score(best);
                    if (lane == 0) {
                        s_rank[r] = win;
                        if (publish) p.route_ids[t * h.top_k + r] = win;
                    }
                }
            }
            // (LDS only: the token's and id loads stay in flight)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            if (live && !shared) {
                const int e = s_rank[s];
                Gm = p_gate + (int64_t)e * gate_eb; Um = p_up + (int64_t)e * up_eb;
            }
        }
    } else if (live && !shared) {
        int e = id_raw;
        if (e < 0 || e >= n_exp) { bad = true; e = 0; }
        Gm = p_gate + (int64_t)e * gate_eb; Um = p_up + (int64_t)e * up_eb;
    }

    const int rr = lane / LPR, li = lane % LPR, blk = li / LANES_PER_BLOCK, k = li % LANES_PER_BLOCK;
    const int row = row0 + rr;
    const bool sw = SGT != GT && shared;   // wave-uniform

    // then every weight load of this lane (waiting for x does not wait for them)
    uint32_t rg[IPW][NA], ru[IPW][NA];
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
        if constexpr (SGT == GT) {
            item_loads<GT, H>(Gm, Um, row + i * RPI, blk, k, rg[i], ru[i]);
        } else {
            if (sw) item_loads<SGT, H>(Gm, Um, row + i * RPI, blk, k, rg[i], ru[i]);
            else item_loads<GT, H>(Gm, Um, row + i * RPI, blk, k, rg[i], ru[i]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the routing weights are read by the down kernel only: the token's first
    // workgroup computes them here, with its weight loads in flight
    if constexpr (ROUTED) {
        if (route_publish && wave == 0) {
            const float w = route_weight(route_mine, h.top_k, lane);
            if (lane < h.top_k) p.route_weights[t * h.top_k + lane] = w;
        }
    }
    // 2. token digits (in the FP16 graph also the token rounded to FP16), and
    // this lane's operands out of LDS, while the weight loads are in flight
    if (threadIdx.x < NX) {
        x_digits<H, NX>(xv, sh.planes, sh.xs16, sh.sum16);
        if constexpr (F16G)
            *(uint2*)(sh.x16 + 4 * threadIdx.x) = make_uint2(pack_rn16(xv.x, xv.y), pack_rn16(xv.z, xv.w));
    }
    __syncthreads();
    // the routed experts of the FP16 graph take FP16 operands (moe_quant_dot.cpp:
    // 189-206); the shared expert always runs the FP32 graph, as the
    // reference's shared expert does
    // (each path reads its operands and runs its dot products in one branch, so
    // only one operand set is live; the weight loads are all issued already,
    // so the waits inside stay exact)
    const bool f16w = F16G && !shared;   // wave-uniform
    float g[IPW], u[IPW];
    if (f16w) {
        if constexpr (F16G) {
            static_assert(IPW == 1, "one item per wave in the FP16 graph");
            LaneH XH;
            lane_xh<GT>(sh.x16, blk, k, XH);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            // 3. gate and up dot products, a scheduling barrier between them:
            // every gate dot product then issues ahead of the wait for the up
            // loads (without it the last one waited behind it: 10.53 -> 10.50 us
            // per FP16-graph layer; the same barrier in the digit path changed
            // nothing)
            g[0] = lane_dot_f16<GT, true>(rg[0], k, XH);
            __builtin_amdgcn_sched_barrier(0);
            u[0] = lane_dot_f16<GT, true>(ru[0], k, XH);
        }
    } else {
        DigitsRef xd;
        xd.planes = sh.planes; xd.xs16 = sh.xs16; xd.sum16 = sh.sum16; xd.n = H;
        LaneX X;
        if (sw) lane_x<SGT>(xd, blk, k, X);
        else lane_x<GT>(xd, blk, k, X);
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // 3. gate and up dot products (the zero-accumulator dot form except in
        // the two-item Q3_K and Q8_0 instances, where it spilled: the 16-token
        // Q3_K layer 53.4 -> 63.6 us)
        constexpr bool Z = IPW == 1 || (GT != T_Q3_K && GT != T_Q3_K_A112 && GT != T_Q8_0);
#pragma unroll
        for (int i = 0; i < IPW; ++i) {
            if (sw) {
                g[i] = lane_dot<SGT, true, Z>(rg[i], k, X);
                u[i] = lane_dot<SGT, true, Z>(ru[i], k, X);
            } else {
                g[i] = lane_dot<GT, true, Z>(rg[i], k, X);
                u[i] = lane_dot<GT, true, Z>(ru[i], k, X);
            }
        }
    }

    // SwiGLU: one FP32 activation per row
    if (live) {
#pragma unroll
        for (int i = 0; i < IPW; ++i) {
            float gs = lane_group_sum<LPR>(g[i]), us = lane_group_sum<LPR>(u[i]);
            if (li == 0) {
                float a;
                if (f16w) {
                    // the FP16 graph's rounding points (moe_quant_dot.cpp:197-206)
                    gs = round16(gs);
                    us = round16(us);
                    const float sig = round16(1.0f / (1.0f + expf(-gs)));
                    a = round16(round16(gs * sig) * us);
                } else {
                    a = silu_mul(gs, us);
                }
                (ROUTED ? h.act : p.act)[((int64_t)t * h.S + s) * h.a_inter + row + i * RPI] = bad ? 0.0f : a;
            }
        }
        if (bad && lane == 0 && row0 == 0) atomicOr(&p.flags[FLAG_BAD_ID], 1);
    }

    shared_scale<NX>(p, sh, scale_wg, gate_wg, xv, gi);
}

// The shared expert's item split over two waves, one token, one row group xg
// a workgroup beside the top_k routed waves of that row group (SPLIT): wave
// top_k takes the gate rows, wave top_k + 1 the same up rows, each loading and
// dotting one matrix, so neither is the workgroup's longest wave.  Each hands
// its row dots to the other through LDS; the second to finish (an LDS counter
// decides, no barrier) applies SwiGLU.  The shared expert runs the FP32 graph
// in either graph, as in the whole-item path.
template <int T, int LPR, bool F16G>
__device__ __forceinline__ void gate_up_shared_half(const DecodeHot& h, const DecodeParams& p,
                                                    SharedX<64 * LPR, F16G>& sh) {
    constexpr int H = 64 * LPR, RPI = 64 / LPR, NX = H / 4;
    const int t = blockIdx.z, xg = (int)blockIdx.y * 8 + (int)blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int per_slot = h.a_inter / RPI;
    if (xg >= per_slot) return;
    const bool upw = uniform(wave) != h.top_k;
    const bool scale_wg = xg + 1 >= per_slot;
    const bool gate_wg = scale_wg & (h.sh_gate_inp != nullptr);
    const float* xt = h.x + (int64_t)t * H;
    const int xi = min((int)threadIdx.x, NX - 1) * 4;
    const float4 xv = *(const float4*)(xt + xi);
    const float4 gi = *(const float4*)((gate_wg ? h.sh_gate_inp : xt) + xi);
    const uint8_t* M = upw ? h.sh_up : h.sh_gate;   // (preloaded arguments)
    __builtin_amdgcn_sched_barrier(0);
    const int rr = lane / LPR, li = lane % LPR, blk = li / LANES_PER_BLOCK, k = li % LANES_PER_BLOCK;
    const int row = xg * RPI + rr;
    constexpr int64_t ROW_BYTES = (int64_t)(H / 256) * unit_bytes(T);
    uint32_t rw[LaneGeo<T>::NRAW];
    lane_load<T, true>(M + (int64_t)row * ROW_BYTES + blk * unit_bytes(T), k, rw);
    __builtin_amdgcn_sched_barrier(0);
    if (threadIdx.x < NX) {
        x_digits<H, NX>(xv, sh.planes, sh.xs16, sh.sum16);
        if constexpr (F16G)
            *(uint2*)(sh.x16 + 4 * threadIdx.x) = make_uint2(pack_rn16(xv.x, xv.y), pack_rn16(xv.z, xv.w));
    }
    if (!upw && lane == 0) sh.half_done = 0;   // (read only after the barrier)
    __syncthreads();
    DigitsRef xd;
    xd.planes = sh.planes; xd.xs16 = sh.xs16; xd.sum16 = sh.sum16; xd.n = H;
    LaneX X;
    lane_x<T>(xd, blk, k, X);
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const float v = lane_group_sum<LPR>(lane_dot<T, true>(rw, k, X));
    if (li == 0) sh.half_dot[upw][rr] = v;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    int before = 0;
    if (lane == 0) before = __hip_atomic_fetch_add(&sh.half_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (uniform(before) == 1) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        if (li == 0) {
            const float o = sh.half_dot[!upw][rr];
            p.act[((int64_t)t * h.S + h.top_k) * h.a_inter + row] = upw ? silu_mul(o, v) : silu_mul(v, o);
        }
    }
    shared_scale<NX>(p, sh, scale_wg, gate_wg, xv, gi);
}

// Whether the calling wave's item is the shared expert's: the item and slot
// as gate_up_items computes them (wave-uniform).
template <int LPR, bool ROUTED, int IPW>
__device__ __forceinline__ bool wave_is_shared(const DecodeHot& h) {
    constexpr int RPI = 64 / LPR;
    const int xg = (int)blockIdx.y * 8 + (int)blockIdx.x, wave = threadIdx.x >> 6;
    const int per_slot = h.a_inter / RPI;
    const bool by_slot = !ROUTED && IPW == 1 && h.a_waves == h.S;
    const int item = uniform(by_slot ? wave * per_slot + xg : (xg * h.a_waves + wave) * IPW);
    return (h.has_shared != 0) & (item < h.S * per_slot) & ((item >> __builtin_ctz(per_slot)) == h.top_k);
}

// A shared expert of another type than the routed ones: the shared expert's
// waves run their own instance of the item code, chosen once at the start by a
// scalar branch.  With both types in one body, the weight loads of the two
// types sat in two branches whose join made the wait-count pass hold the
// shared expert's header loads for the token's load, and the compiler
// converted the Q6_K scale right after its load (a round trip ahead of the
// main weight loads): Q3_K beside a Q6_K shared expert took 11.0 us for this
// kernel against 6.2 us with a Q3_K shared expert.  Each wave executes the
// same barriers whichever instance it runs.
template <int GT, int SGT, int LPR, bool ROUTED, bool F16G, int IPW, bool SPLIT = false>
__device__ __forceinline__ void gate_up_waves(const DecodeHot& h, const DecodeParams& p, SharedX<64 * LPR, F16G>& sh) {
    if constexpr (SPLIT) {
        static_assert(!ROUTED && IPW == 1, "the split shared item is dealt by slot");
        if (uniform(threadIdx.x >> 6) >= h.top_k) gate_up_shared_half<SGT, LPR, F16G>(h, p, sh);
        else gate_up_items<GT, GT, LPR, false, F16G, 1, true>(h, p, sh);
        return;
    }
    if constexpr (SGT != GT) {
        if (wave_is_shared<LPR, ROUTED, IPW>(h)) {
            gate_up_items<SGT, SGT, LPR, ROUTED, F16G, IPW>(h, p, sh);
            return;
        }
    }
    gate_up_items<GT, GT, LPR, ROUTED, F16G, IPW>(h, p, sh);
}

// The leading arguments are the ones preloaded into scalar registers: with the
// shared expert's gate and up pointers among them (has_shared is S - top_k; the
// expert count is read from the argument block with the expert id and the
// output pointer at the end), the shared expert's waves issue their weight
// loads with no argument load first.
template <int GT, int SGT, int LPR, bool F16G, int IPW = 1, bool SPLIT = false>
__global__ __launch_bounds__(1024) void k_fast_gate_up(const float* x, const int32_t* ids, const float* sh_gate_inp,
                                                  const uint8_t* sh_gate, const uint8_t* sh_up, int top_k, int S,
                                                  int a_inter, int a_waves, DecodeParams p) {
    __shared__ SharedX<64 * LPR, F16G> sh;
    const DecodeHot h{x, ids, nullptr, nullptr, sh_gate_inp, top_k, S, S - top_k, -1, a_inter, a_waves, nullptr, nullptr, sh_gate, sh_up};
    gate_up_waves<GT, SGT, LPR, false, F16G, IPW, SPLIT>(h, p, sh);
}

// Kernel A with the router's select step in its prologue: the same work as
// k_fast_gate_up once each wave knows its expert.
template <int GT, int SGT, int LPR, bool F16G>
__global__ __launch_bounds__(1024) void k_fast_gate_up_routed(const float* x, const int32_t* ids, float* act, const float* sh_gate_inp, int top_k,
                                                  int S, int has_shared, int n_experts, int a_inter, int a_waves,
                                                  DecodeParams p) {
    __shared__ SharedX<64 * LPR, F16G> sh;
    const DecodeHot h{x, ids, act, nullptr, sh_gate_inp, top_k, S, has_shared, n_experts, a_inter, a_waves};
    gate_up_waves<GT, SGT, LPR, true, F16G, 1>(h, p, sh);
}

// ---------------------------------------------------------------- kernel B

// LPR = intermediate / 64 lanes per down row; RPI = 64 / LPR rows per
// instruction; NPB row groups per wave, so RB = NPB * RPI output rows per
// workgroup.  Wave s of the workgroup computes slot s.
template <int LPR, int NPB_ = 1>
struct GeoB {
    static constexpr int RPI = 64 / LPR;
    static constexpr int NPB = NPB_;
    static constexpr int RB = NPB * RPI;
};

template <int RB>
struct SharedB {
    float s_y[FAST_MAX_SLOTS][RB];
    float s_w[FAST_MAX_SLOTS];
};

// Workgroup (bx, t) of kernel B: RB down rows of token t for every slot (wave
// s = slot s; waves at or past S only join the barriers), combined in top-k
// order.  down_slot is the calling wave's part (its slot's rows into LDS, with
// the slot's weight type DT), down_combine the workgroup's.
// BAL (balanced, FP32 graph, NPB row groups a wave, a shared expert): the
// workgroup has one wave per routed slot, and the shared slot's NPB row groups
// go to waves 0 .. NPB-1, one each, after their own slot.  With eight routed
// slots and four row groups, waves w and w + 4 (one SIMD) then hold nine row
// groups between them on every SIMD, where nine waves (one per slot) put three
// on one SIMD.  SDT is the shared expert's down type.  ARGD: the shared
// expert's down weights from the kernel's preloaded argument (h.sh_down), else
// from the argument block.
template <int DT, int LPR, int NPB_, bool F16G, int SDT = DT, bool BAL = false, bool ARGD = true>
__device__ __forceinline__ void down_slot(const DecodeHot& h, const DecodeParams& p, int bx, int t,
                                          SharedB<GeoB<LPR, NPB_>::RB>& sh) {
    constexpr int N = LaneGeo<DT>::NRAW, NS = LaneGeo<SDT>::NRAW;
    constexpr int BB = unit_bytes(DT), BBS = unit_bytes(SDT);
    constexpr int I = 64 * LPR;
    constexpr int RPI = GeoB<LPR, NPB_>::RPI, NPB = GeoB<LPR, NPB_>::NPB, RB = GeoB<LPR, NPB_>::RB;
    constexpr int64_t ROW_BYTES = (int64_t)(I / 256) * BB, ROW_BYTES_S = (int64_t)(I / 256) * BBS;
    static_assert(!BAL || !F16G, "the balanced form is the FP32 graph's");

    const int lane = threadIdx.x & 63, s = uniform(threadIdx.x >> 6);   // wave = slot (64 * S threads)
    const int rr = lane / LPR, li = lane % LPR, blk = li / LANES_PER_BLOCK, k = li % LANES_PER_BLOCK;
    const int r0 = bx * RB;
    const bool shared = !BAL && h.has_shared && s == h.top_k;

    // the slot's activations first: their address needs no expert id, so the
    // loads go out while the id is still being read
    ActRegs<I> A;
    act_load<I>(h.act + ((int64_t)t * h.S + s) * I, lane, A);
    __builtin_amdgcn_sched_barrier(0);

    const uint8_t* D = BAL || !ARGD ? p.sh_down : h.sh_down;
    bool bad = false;
    float w = 0.0f, w_sh = 0.0f;
    if (!shared) {
        int e = h.ids[t * h.top_k + s];
        if constexpr (BAL) {
            // (the balanced form keeps the compiler's order: the form below
            // measured 17.4 -> 17.8 us for its 16-token launch)
            if (e < 0 || e >= h.n_experts) { bad = true; e = 0; }
            D = p.down + (int64_t)e * p.down_eb;
            w = bad ? 0.0f : h.weights[t * h.top_k + s];
            // (wave 0 also reads the shared expert's gate here, ahead of the
            // weights, not where it stores it after its shared rows: eight
            // tokens 37.2 -> 36.9 us per layer)
            if (s == 0) w_sh = h.sh_scale[t];
        } else {
            // the id, the routing weight and the argument-block fields the
            // weight address needs in one round trip (the compiler would
            // otherwise load the routing weight after the id, ahead of the
            // weight loads: one token 9.78 -> 9.67 us per layer)
            const float w_raw = h.weights[t * h.top_k + s];
            const uint8_t* down = p.down;
            const int64_t down_eb = p.down_eb;
            // (k_fast_down leaves the expert count out of its preloaded
            // arguments, -1 here, to make room for the shared expert's pointers)
            const int n_exp = h.n_experts >= 0 ? h.n_experts : p.n_experts;
            __asm__ volatile("" ::"s"(e), "s"(w_raw), "s"(down), "s"(down_eb), "s"(n_exp));
            if (e < 0 || e >= n_exp) { bad = true; e = 0; }
            D = down + (int64_t)e * down_eb;
            w = bad ? 0.0f : w_raw;
        }
    } else if constexpr (!BAL) {
        // the shared expert's gate (kernel A's sigmoid), issued here, ahead of
        // the weights, from a preloaded argument: loaded where lane 0 stores
        // it, after the dot products, it was two round trips (the argument
        // block, then the value) in the shared wave's tail ahead of the combine
        // (config 3 9.33 -> 9.22 us per layer, FP16 graph 10.47 -> 10.33, four
        // tokens 24.57 -> 24.29)
        w = h.sh_scale[t];
    }

    // then every weight load, with no branch around them (a conditional load
    // makes the compiler's wait counts conservative at the join, and the digit
    // split below would then wait for the weights)
    uint32_t raw[NPB][N];
#pragma unroll
    for (int q = 0; q < NPB; ++q) lane_load<DT>(D + (int64_t)(r0 + q * RPI + rr) * ROW_BYTES + blk * BB, k, raw[q]);
    __builtin_amdgcn_sched_barrier(0);
    // the slot's digits (the FP16 graph's routed slots: its FP16 activations)
    // into this wave's LDS region, and this lane's operands back out of it,
    // while the weights are in flight
    extern __shared__ __attribute__((aligned(16))) uint8_t b_digits[];
    int8_t* planes = (int8_t*)(b_digits + s * act_lds_bytes(I));
    float* xs16 = (float*)(planes + 2 * I);
    float* sum16 = xs16 + I / RUN;
    // (each path in one branch, so only one operand set is live)
    const bool f16w = F16G && !shared;   // wave-uniform
    float v[NPB];
    if (f16w) {
        if constexpr (F16G) {
            act_halves_lds<I>(A, lane, (uint16_t*)planes);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            LaneH XH;
            lane_xh<DT>((const uint16_t*)planes, blk, k, XH);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < NPB; ++q)   // the expert's output in the FP16 graph (moe_quant_dot.cpp:208-209)
                v[q] = round16(lane_group_sum<LPR>(lane_dot_f16<DT>(raw[q], k, XH)));
        }
    } else {
        act_digits_lds<I>(A, lane, planes, xs16, sum16);
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        DigitsRef xd;
        xd.planes = planes; xd.xs16 = xs16; xd.sum16 = sum16; xd.n = I;
        LaneX X;
        lane_x<DT>(xd, blk, k, X);
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < NPB; ++q) v[q] = lane_group_sum<LPR>(lane_dot<DT>(raw[q], k, X));
    }
#pragma unroll
    for (int q = 0; q < NPB; ++q)
        if (li == 0) sh.s_y[s][q * RPI + rr] = bad ? 0.0f : v[q];
    if (lane == 0) sh.s_w[s] = w;
    if constexpr (BAL) {
        if (s < NPB) {   // wave-uniform: the shared slot's row group s, from its own copy of the shared digits
            // (loaded only now: held from the start, these registers keep the
            // workgroup to one per CU)
            ActRegs<I> A2;
            act_load<I>(h.act + ((int64_t)t * h.S + h.top_k) * I, lane, A2);
            uint32_t raw2[NS];
            lane_load<SDT>(p.sh_down + (int64_t)(r0 + s * RPI + rr) * ROW_BYTES_S + blk * BBS, k, raw2);
            int8_t* planes2 = (int8_t*)(b_digits + (h.top_k + s) * act_lds_bytes(I));
            float* xs2 = (float*)(planes2 + 2 * I);
            float* sum2 = xs2 + I / RUN;
            act_digits_lds<I>(A2, lane, planes2, xs2, sum2);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            DigitsRef xd;
            xd.planes = planes2; xd.xs16 = xs2; xd.sum16 = sum2; xd.n = I;
            LaneX X;
            lane_x<SDT>(xd, blk, k, X);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            const float v2 = lane_group_sum<LPR>(lane_dot<SDT>(raw2, k, X));
            if (li == 0) sh.s_y[h.top_k][s * RPI + rr] = v2;
            if (lane == 0 && s == 0) sh.s_w[h.top_k] = w_sh;
        }
    }
}

template <int LPR, int NPB_>
__device__ __forceinline__ void down_combine(const DecodeHot& h, const DecodeParams& p, int bx, int t,
                                             SharedB<GeoB<LPR, NPB_>::RB>& sh) {
    constexpr int RB = GeoB<LPR, NPB_>::RB;
    __syncthreads();
    // combine in top-k order, then the shared expert (moe_layer.py:70-106)
    if (threadIdx.x < RB) {
        const int r = threadIdx.x;
        float acc = 0.0f;
        for (int j = 0; j < h.top_k; ++j) acc = __fadd_rn(acc, __fmul_rn(sh.s_w[j], sh.s_y[j][r]));
        if (h.has_shared) acc = __fadd_rn(acc, __fmul_rn(sh.s_w[h.top_k], sh.s_y[h.top_k][r]));
        p.y[(int64_t)t * p.hidden + bx * RB + r] = acc;
        if (!isfinite(acc)) atomicOr(&p.flags[FLAG_NONFINITE], 1);
    }
}

// SDT: the shared expert's down type (its wave takes that code path).  The
// leading arguments are the ones preloaded into scalar registers: the shared
// expert's gate and down pointers among them, so the shared wave issues its
// weight loads with no argument load first (config 3 9.24 -> 9.10 us per layer
// against the down pointer read from the argument block); the expert count
// comes from the argument block with the expert id.
// Row group bx = blockIdx.x + 8 blockIdx.y of token blockIdx.z (fast_grid).
// 64 threads a slot: at intermediate 2048 (LPR 32) at most 12 slots fit the
// digit LDS (fast_supported), so 768 threads, which leaves the FP16 graph's
// two-type instances the registers they need (a 1024-thread bound caps them at
// 128 VGPRs and they spill)
template <int DT, int SDT, int LPR, int NPB, bool F16G>
__global__ __launch_bounds__(LPR == 32 ? 768 : 1024) void k_fast_down(const int32_t* ids, float* act, const float* weights,
                                                   const float* sh_scale, const uint8_t* sh_down, int top_k,
                                                   int S, int has_shared, int nbx, DecodeParams p) {
    __shared__ SharedB<GeoB<LPR, NPB>::RB> sh;
    const int bx = (int)blockIdx.y * 8 + (int)blockIdx.x;
    if (bx >= nbx) return;   // padding of the last group of eight
    const DecodeHot h{nullptr, ids, act, weights, nullptr, top_k, S, has_shared, -1, 0, 0, sh_scale, sh_down};
    if constexpr (SDT != DT) {
        // (the shared expert's down weights from the argument block: with the
        // preloaded argument this two-type kernel measured no faster, the Q3_K
        // layer with a Q6_K shared expert 9.68 against 9.70 us, where one-type
        // kernels gained 0.14 us)
        const int s = uniform(threadIdx.x >> 6);
        if (has_shared && s == top_k) down_slot<SDT, LPR, NPB, F16G, SDT, false, false>(h, p, bx, blockIdx.z, sh);
        else down_slot<DT, LPR, NPB, F16G, DT, false, false>(h, p, bx, blockIdx.z, sh);
    } else {
        down_slot<DT, LPR, NPB, F16G>(h, p, bx, blockIdx.z, sh);
    }
    down_combine<LPR, NPB>(h, p, bx, blockIdx.z, sh);
}

// The balanced form (down_slot BAL): one wave per routed slot, at most 8,
// with the register budget of two such workgroups per CU (four waves a SIMD).
template <int DT, int SDT, int LPR, int NPB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_fast_down_bal(const int32_t* ids, float* act, const float* weights, int top_k,
                                                      int S, int has_shared, int n_experts, int nbx,
                                                      const float* sh_scale, DecodeParams p) {
    __shared__ SharedB<GeoB<LPR, NPB>::RB> sh;
    const int bx = (int)blockIdx.y * 8 + (int)blockIdx.x;
    if (bx >= nbx) return;
    const DecodeHot h{nullptr, ids, act, weights, nullptr, top_k, S, has_shared, n_experts, 0, 0, sh_scale, nullptr};
    down_slot<DT, LPR, NPB, false, SDT, true>(h, p, bx, blockIdx.z, sh);
    down_combine<LPR, NPB>(h, p, bx, blockIdx.z, sh);
}

// ------------------------------------------------------------------ launch

static bool fast_type(int t) {
    return t == T_Q3_K || t == T_Q3_K_A112 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_Q8_0;
}
static bool fast_dim(int n) { return n == 256 || n == 512 || n == 1024 || n == 2048; }

bool fast_supported(const DecodeParams& p) {
    if (!fast_dim(p.hidden) || p.S > FAST_MAX_SLOTS || p.S < 1) return false;
    int gt = -1, dt = -1, I = -1;
    if (p.top_k > 0) {
        if (!(fast_type(p.gate_type) && p.up_type == p.gate_type && fast_type(p.down_type))) return false;
        gt = p.gate_type; dt = p.down_type; I = p.inter;
    }
    if (p.has_shared) {
        if (!(fast_type(p.sh_gate_type) && p.sh_up_type == p.sh_gate_type && fast_type(p.sh_down_type))) return false;
        // the shared expert shares the routed geometry; its types are the routed
        // ones or Q6_K (the layout of the reference model's shared experts)
        if (gt >= 0 && (p.sh_inter != I || (p.sh_gate_type != gt && p.sh_gate_type != T_Q6_K) ||
                        (p.sh_down_type != dt && p.sh_down_type != T_Q6_K)))
            return false;
    }
    const int inter = p.top_k > 0 ? p.inter : p.sh_inter;
    // kernel B holds every slot's digits in LDS (64 KiB per workgroup, its
    // static part below 4 KiB)
    return fast_dim(inter) && (int64_t)p.S * act_lds_bytes(inter) <= 65536 - 4096;
}

// Compute units of the current device (cached per device).
static int device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Waves per kernel-A workgroup for `items` items per token: at least
// hidden / 256 (the threads that hold the token, four values each), at most
// 16; the fewest waves on the busiest CU when the launch's workgroups are
// dealt evenly over the CUs.  Ties go to the smaller workgroup: with many
// tokens the kernel is VALU-bound, and a workgroup of 9 waves (three on one
// SIMD) or 16 (no second workgroup on the CU) measured 14 % and 23 % slower
// than one of 8 at 16 tokens.
static int gate_up_waves(int items, int tokens, int hidden, int cus) {
    const int lo = std::max(1, hidden / 256);
    int best = lo;
    int64_t best_cost = INT64_MAX;
    for (int w = lo; w <= 16; ++w) {
        const int64_t wgs = (int64_t)((items + w - 1) / w) * tokens;
        const int64_t cost = ((wgs + cus - 1) / cus) * w;
        if (cost < best_cost) {
            best_cost = cost;
            best = w;
        }
    }
    return best;
}

// Grid of n workgroups a token (kernels index x = blockIdx.x + 8 blockIdx.y,
// token blockIdx.z, and return for x >= n): a single token as (8, ceil(n/8), 1),
// several as (n, 1, T).
static dim3 fast_grid(int n, int tokens) {
    return tokens == 1 ? dim3(8, (n + 7) / 8, 1) : dim3(n, 1, tokens);
}

#ifndef FAST_A_SPLIT_SHARED
#define FAST_A_SPLIT_SHARED 1   // one token, one wave a slot: two waves for the shared expert's item
#endif

#ifndef FAST_A_PAIR_TOKENS
#define FAST_A_PAIR_TOKENS 4   // tokens from which kernel A gives each wave two items
#endif

template <int GT, int SGT, int LPR, bool F16G, int IPW>
static void launch_a_ipw(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    const int items = p.S * (p.inter / (64 / LPR)) / IPW;   // wave-items
    const int w = gate_up_waves(items, p.n_tokens, 64 * LPR, device_cus());
    const dim3 grid = fast_grid((items + w - 1) / w, p.n_tokens), block(64 * w);
    if (ev.armed_a())
        hipExtLaunchKernelGGL((k_fast_gate_up<GT, SGT, LPR, F16G, IPW>), grid, block, 0, stream, ev.a_start, ev.a_stop, 0, p.x, p.ids, p.sh_gate_inp, p.sh_gate, p.sh_up, p.top_k, p.S, p.a_inter, w, p);
    else
        hipLaunchKernelGGL((k_fast_gate_up<GT, SGT, LPR, F16G, IPW>), grid, block, 0, stream, p.x, p.ids, p.sh_gate_inp, p.sh_gate, p.sh_up, p.top_k, p.S, p.a_inter, w, p);
}

template <int GT, int SGT, int LPR, bool F16G>
static void launch_a(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    if constexpr (!F16G && SGT == GT && GT != T_Q5_K && GT != T_Q6_K) {
        // many tokens: two items a wave, so each wave has twice the weights in
        // flight behind one prologue (the per-token launches are latency-bound).
        // Only where two items fit in the 128 VGPRs of the kernel's 1024-thread
        // bound: Q5_K and Q6_K items, and a shared expert of another type (both
        // types' operands live at once), spill 14-53 VGPRs to scratch, and one item a
        // wave is faster (16 tokens: Q5_K 85 -> 65, Q6_K 96 -> 78, Q4_K with a
        // Q6_K shared expert 97 -> 78 us per layer)
        if (p.route_scores == nullptr && p.n_tokens >= FAST_A_PAIR_TOKENS) {
            launch_a_ipw<GT, SGT, LPR, F16G, 2>(p, stream, ev);
            return;
        }
    }
    const int items = p.S * (p.inter / (64 / LPR));
    const int w = gate_up_waves(items, p.n_tokens, 64 * LPR, device_cus());
    if (FAST_A_SPLIT_SHARED && p.route_scores == nullptr && p.n_tokens == 1 && p.has_shared && p.top_k > 0 &&
        w == p.S && p.S + 1 <= 16) {
        // one wave a slot (dealt by slot): the shared expert's item goes to two
        // waves, gate and up
        const int per_slot = p.inter / (64 / LPR);
        const dim3 grid = fast_grid(per_slot, 1), block(64 * (p.S + 1));
        if (ev.armed_a())
            hipExtLaunchKernelGGL((k_fast_gate_up<GT, SGT, LPR, F16G, 1, true>), grid, block, 0, stream, ev.a_start, ev.a_stop, 0, p.x, p.ids, p.sh_gate_inp, p.sh_gate, p.sh_up, p.top_k, p.S, p.a_inter, p.S + 1, p);
        else
            hipLaunchKernelGGL((k_fast_gate_up<GT, SGT, LPR, F16G, 1, true>), grid, block, 0, stream, p.x, p.ids, p.sh_gate_inp, p.sh_gate, p.sh_up, p.top_k, p.S, p.a_inter, p.S + 1, p);
        return;
    }
    const dim3 grid = fast_grid((items + w - 1) / w, p.n_tokens), block(64 * w);
    if (p.route_scores != nullptr) {
        if (ev.armed_a())
            hipExtLaunchKernelGGL((k_fast_gate_up_routed<GT, SGT, LPR, F16G>), grid, block, 0, stream, ev.a_start,
                                  ev.a_stop, 0, p.x, p.ids, p.act, p.sh_gate_inp, p.top_k, p.S, p.has_shared, p.n_experts, p.a_inter, w, p);
        else
            hipLaunchKernelGGL((k_fast_gate_up_routed<GT, SGT, LPR, F16G>), grid, block, 0, stream, p.x, p.ids, p.act, p.sh_gate_inp, p.top_k, p.S, p.has_shared, p.n_experts, p.a_inter, w, p);
        return;
    }
    if (ev.armed_a())
        hipExtLaunchKernelGGL((k_fast_gate_up<GT, SGT, LPR, F16G>), grid, block, 0, stream, ev.a_start, ev.a_stop, 0, p.x, p.ids, p.sh_gate_inp, p.sh_gate, p.sh_up, p.top_k, p.S, p.a_inter, w, p);
    else
        hipLaunchKernelGGL((k_fast_gate_up<GT, SGT, LPR, F16G>), grid, block, 0, stream, p.x, p.ids, p.sh_gate_inp, p.sh_gate, p.sh_up, p.top_k, p.S, p.a_inter, w, p);
}

template <int GT, int SGT, bool F16G>
static void launch_a_h(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    switch (p.hidden) {
        case 256: launch_a<GT, SGT, 4, F16G>(p, stream, ev); break;
        case 512: launch_a<GT, SGT, 8, F16G>(p, stream, ev); break;
        case 1024: launch_a<GT, SGT, 16, F16G>(p, stream, ev); break;
        default: launch_a<GT, SGT, 32, F16G>(p, stream, ev); break;
    }
}

// a shared expert of another type is Q6_K (fast_supported admits no other)
template <int GT, bool F16G>
static void launch_a_t(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    if (p.has_shared && p.top_k > 0 && p.sh_gate_type != GT) launch_a_h<GT, T_Q6_K, F16G>(p, stream, ev);
    else launch_a_h<GT, GT, F16G>(p, stream, ev);
}

#ifndef FAST_DOWN_WG_TARGET
#define FAST_DOWN_WG_TARGET 1024   // kernel B workgroups above which rows per workgroup grow
#endif

template <int DT, int SDT, int LPR, int NPB, bool F16G>
static void launch_b_n(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    const int nbx = p.hidden / GeoB<LPR, NPB>::RB;
    const dim3 grid = fast_grid(nbx, p.n_tokens);
    if constexpr (!F16G && NPB >= 2) {
        if (p.has_shared && p.top_k >= NPB && p.top_k <= 8 &&
            (int64_t)(p.top_k + NPB) * act_lds_bytes(64 * LPR) <= 65536 - 4096) {   // one wave per routed slot,
                                                                                    // shared rows to waves 0 .. NPB-1
            const size_t lds = (size_t)(p.top_k + NPB) * act_lds_bytes(64 * LPR);
            if (ev.armed_b())
                hipExtLaunchKernelGGL((k_fast_down_bal<DT, SDT, LPR, NPB>), grid, dim3(64 * p.top_k), lds, stream,
                                      ev.b_start, ev.b_stop, 0, p.ids, p.act, p.weights, p.top_k, p.S, p.has_shared,
                                      p.n_experts, nbx, (const float*)p.sh_scale, p);
            else
                hipLaunchKernelGGL((k_fast_down_bal<DT, SDT, LPR, NPB>), grid, dim3(64 * p.top_k), lds, stream, p.ids,
                                   p.act, p.weights, p.top_k, p.S, p.has_shared, p.n_experts, nbx,
                                   (const float*)p.sh_scale, p);
            return;
        }
    }
    const size_t lds = (size_t)p.S * act_lds_bytes(64 * LPR);   // the slots' digits
    if (ev.armed_b())
        hipExtLaunchKernelGGL((k_fast_down<DT, SDT, LPR, NPB, F16G>), grid, dim3(64 * p.S), lds, stream, ev.b_start,
                              ev.b_stop, 0, p.ids, p.act, p.weights, (const float*)p.sh_scale, p.sh_down, p.top_k, p.S,
                              p.has_shared, nbx, p);
    else
        hipLaunchKernelGGL((k_fast_down<DT, SDT, LPR, NPB, F16G>), grid, dim3(64 * p.S), lds, stream, p.ids, p.act,
                           p.weights, (const float*)p.sh_scale, p.sh_down, p.top_k, p.S, p.has_shared, nbx, p);
}

// Row groups per wave: one while the grid is small (a single token: every
// workgroup on its own CU), more when many tokens would otherwise make many
// short workgroups.
template <int DT, int SDT, int LPR, bool F16G>
static void launch_b_s(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    const int64_t wg1 = (int64_t)(p.hidden / GeoB<LPR, 1>::RB) * p.n_tokens;
    constexpr bool wide = LaneGeo<DT>::NRAW > 12 || LaneGeo<SDT>::NRAW > 12;   // four row groups would spill
    if constexpr (F16G) {   // the FP16 graph's decode holds one row group per wave (more would spill)
        launch_b_n<DT, SDT, LPR, 1, F16G>(p, stream, ev);
    } else {
        if (!wide && wg1 >= 4 * FAST_DOWN_WG_TARGET && p.hidden / GeoB<LPR, 4>::RB >= 1)
            launch_b_n<DT, SDT, LPR, wide ? 2 : 4, F16G>(p, stream, ev);
        else if (wg1 >= 2 * FAST_DOWN_WG_TARGET && p.hidden / GeoB<LPR, 2>::RB >= 1)
            launch_b_n<DT, SDT, LPR, 2, F16G>(p, stream, ev);
        else
            launch_b_n<DT, SDT, LPR, 1, F16G>(p, stream, ev);
    }
}

// a shared expert of another type is Q6_K (fast_supported admits no other)
template <int DT, int LPR, bool F16G>
static void launch_b(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    if (p.has_shared && p.top_k > 0 && p.sh_down_type != DT) launch_b_s<DT, T_Q6_K, LPR, F16G>(p, stream, ev);
    else launch_b_s<DT, DT, LPR, F16G>(p, stream, ev);
}

template <int DT, bool F16G>
static void launch_b_t(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    switch (p.inter) {
        case 256: launch_b<DT, 4, F16G>(p, stream, ev); break;
        case 512: launch_b<DT, 8, F16G>(p, stream, ev); break;
        case 1024: launch_b<DT, 16, F16G>(p, stream, ev); break;
        default: launch_b<DT, 32, F16G>(p, stream, ev); break;
    }
}

template <bool F16G>
static hipError_t launch_fast(const DecodeParams& p0, hipStream_t stream, const KernelEvents& ev) {
    DecodeParams p = p0;
    if (p.top_k == 0) {   // shared expert only: present it as the routed types
        p.gate_type = p.sh_gate_type; p.up_type = p.sh_up_type; p.down_type = p.sh_down_type;
        p.inter = p.sh_inter;
    }
    p.a_inter = p.inter;
    switch (p.gate_type) {
        case T_Q4_K: launch_a_t<T_Q4_K, F16G>(p, stream, ev); break;
        case T_Q5_K: launch_a_t<T_Q5_K, F16G>(p, stream, ev); break;
        case T_Q6_K: launch_a_t<T_Q6_K, F16G>(p, stream, ev); break;
        case T_Q8_0: launch_a_t<T_Q8_0, F16G>(p, stream, ev); break;
        case T_Q3_K_A112: launch_a_t<T_Q3_K_A112, F16G>(p, stream, ev); break;
        default: launch_a_t<T_Q3_K, F16G>(p, stream, ev); break;
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    switch (p.down_type) {
        case T_Q4_K: launch_b_t<T_Q4_K, F16G>(p, stream, ev); break;
        case T_Q5_K: launch_b_t<T_Q5_K, F16G>(p, stream, ev); break;
        case T_Q6_K: launch_b_t<T_Q6_K, F16G>(p, stream, ev); break;
        case T_Q8_0: launch_b_t<T_Q8_0, F16G>(p, stream, ev); break;
        case T_Q3_K_A112: launch_b_t<T_Q3_K_A112, F16G>(p, stream, ev); break;
        default: launch_b_t<T_Q3_K, F16G>(p, stream, ev); break;
    }
    return hipGetLastError();
}


hipError_t launch_decode_fast(const DecodeParams& p, hipStream_t stream, const KernelEvents& ev) {
    return p.fp16 ? launch_fast<true>(p, stream, ev) : launch_fast<false>(p, stream, ev);
}

}  // namespace mqh
