// moe_prefill.hip -- grouped-GEMM MoE layer for a prompt (many tokens).
//
// Replaces run_moe_sequence (src/flash_moe/moe_layer.py:110-195), which runs the
// routed experts expert by expert on their token batches (backend_ov.py:210-237,
// 407-431) and then adds the batched shared expert (shared_expert.py:200-219):
//   for every expert e and the tokens routed to it:
//     act = silu(X_e W_gate^T) * (X_e W_up^T),  Y_e = act W_down^T
//   y[t] = sum_s w[t,s] * Y_{ids[t,s]}[t]  (top-k order)  + sigmoid(x_t . g_inp) * shared(x_t)
//
// Four launches, no inter-workgroup synchronisation:
//   P0 k_prefill_route     workgroup 0 buckets the (token, slot) pairs by expert and
//                          cuts each expert's tokens into tiles of 16; the others
//                          stage every token once as the B operand (token planes)
//                          and the shared expert's sigmoid gate.
//   P1 k_prefill_gate_up   (I/64) x max_tiles workgroups: 64 intermediate rows x one tile,
//                          SwiGLU fused.
//   P2 k_prefill_down      (H/128) x max_tiles workgroups: 128 output rows x one tile.
//   P3 k_prefill_combine   grid (H/256, T): the weighted sum in top-k order.
//
// P1/P2 are MFMA GEMMs (v_mfma_f32_16x16x32_f16, FP32 accumulate) whose weight
// operand is built in registers straight from the quantized blocks as exact
// integers (kquant_frag.h); the tile's tokens are the other operand, FP16
// planes with a power-of-two scale per token, in LDS (P1 copies the planes P0
// made; P2 stages its activation rows itself).
#include <hip/hip_ext.h>

#include <algorithm>
#include <utility>

#include "kquant_frag.h"
#include "moe_decode.h"

namespace mqh {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_WAVES = 8;      // waves per workgroup of the GEMM kernels
constexpr int PF_ROWS_GU = 64;   // gate/up rows per workgroup: 4 waves on gate, 4 on up
constexpr int PF_ROWS_DOWN = 128; // down rows per workgroup chunk: 8 waves x 16
// Gate/up workgroups take PF_BIG_GU 64-row chunks on one continuous load ring
// (one chunk each: 89.8, two: 86.4, four: 93.2 us at the 128-token prompt),
// except at least PF_SMALL_GU one-chunk workgroups per tile launched after all
// the others.
#ifndef PF_BIG_GU
#define PF_BIG_GU 2
#endif
#ifndef PF_SMALL_GU
#define PF_SMALL_GU 2
#endif
// Down row chunks per workgroup: one (two: 63 -> 88 us, four: 93 us for the
// 128-token prompt's Q6_K down projections -- fewer workgroups in flight).
#ifndef PF_CPW_DOWN
#define PF_CPW_DOWN 1
#endif
// Register ring of super-blocks per lane (R - 1 in flight).  Three: the
// mixed-type gate/up kernel (Q3_K routed, Q6_K shared) holds 126 VGPRs and
// two workgroups a CU (155 and one a CU with four: 107 -> 94 us at the
// 128-token prompt), Q4_K gate/up 77 -> 75 us; six measured slower.
#ifndef PF_RING
#define PF_RING 3
#endif
#ifndef PF_RING_DOWN
#define PF_RING_DOWN PF_RING
#endif
// A shared expert of another type than the routed experts runs in the same
// launch (its tiles take their own instance of the body), and the kernel's
// register allocation is the larger body's: its ring may be set shallower, so
// that a Q6_K shared expert does not cost the routed tiles their occupancy.
#ifndef PF_RING_SHARED
#define PF_RING_SHARED 3
#endif
// In the down kernel a Q6_K shared expert beside routed experts of another
// type takes a two-slot ring, and the kernel asks for six waves a SIMD (80
// VGPRs, three workgroups a CU instead of two) when the intermediate size is
// at most 512 and the routed type is a K-quant (a Q8_0 body would spill): the
// Q3_K-routed down projections 47.4 -> 44.7 us at the 128-token prompt.  (A
// two-slot ring for Q6_K throughout measured 65.3 -> 66.8 us.)
#ifndef PF_RING_SHARED_DOWN
#define PF_RING_SHARED_DOWN 2
#endif
#ifndef PF_MIXED_WAVES_DOWN
#define PF_MIXED_WAVES_DOWN 6
#endif
constexpr int PF_PAD = 8;        // LDS row padding (halves)

// Waves per SIMD that the LDS footprint of one workgroup (PF_WAVES waves)
// admits; the GEMM kernels ask the register allocator for that occupancy.
constexpr int pf_lds_bytes(int K, bool split) {
    return 2 * PREFILL_TILE * (K + PF_PAD) * (split ? 2 : 1) + PREFILL_TILE * (K / 256) * 32 + 2048;
}
constexpr int pf_occupancy(int lds_bytes) {
    return (160 * 1024 / lds_bytes) * PF_WAVES / 4 < 8 ? (160 * 1024 / lds_bytes) * PF_WAVES / 4 : 8;
}

#ifndef PF_OCC_GU
#define PF_OCC_GU
#endif
#ifndef PF_OCC_DOWN
#define PF_OCC_DOWN
#endif

template <int... Ms, class F>
__device__ __forceinline__ void pf_unroll(std::integer_sequence<int, Ms...>, F&& f) {
    (f(std::integral_constant<int, Ms>{}), ...);
}

__device__ __forceinline__ float pf_silu_mul(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
    return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

__device__ __forceinline__ float pf_sigmoid(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

__device__ __forceinline__ float pf_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float pf_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ------------------------------------------------------------ token staging
//
// One wave stages token row `row` of src (K values, FP32 or BF16) as LDS column
// j of the B operand: high plane xh[j][K + PF_PAD], low plane xl (SPLIT only),
// and the 32-column sub-block sums / 32 as [block][j][hi 0..7 | lo 0..7] in xs
// (block-major, so the 16 token columns of one block sit in distinct banks).
// A lane owns 8 consecutive values per 512-column pass.  The loads
// (pf_stage_load) and the rest (pf_stage_finish, or pf_stage_planes into
// device memory) are separate.
template <int K, bool BF16>
struct PfStageRaw {
    static constexpr int NIT = K >= 512 ? K / 512 : 1;
    uint4 r[NIT][BF16 ? 1 : 2];
};

// live = false (a token column past the tile's count): every lane reads the
// row's first values, one request per instruction instead of a row's worth
template <int K, bool BF16>
__device__ __forceinline__ void pf_stage_load(const void* src, int64_t row, bool live, PfStageRaw<K, BF16>& raw) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int it = 0; it < PfStageRaw<K, BF16>::NIT; ++it) {
        // lanes past K (K = 256) read the row's first values again (in bounds, unused)
        const int c = live ? (512 * it + 8 * lane) % K : 0;
        if constexpr (BF16) {
            raw.r[it][0] = *(const uint4*)((const uint16_t*)src + row * K + c);
        } else {
            raw.r[it][0] = *(const uint4*)((const float*)src + row * K + c);
            raw.r[it][1] = *(const uint4*)((const float*)src + row * K + c + 4);
        }
    }
}

// Hands the loaded words through an empty asm statement placed after the
// weight prefetch: everything computed from them is then ordered after the
// prefetch (the instruction selector is otherwise free to put the row's
// arithmetic, and its wait for the row, ahead of the prefetch loads).
template <int K, bool BF16>
__device__ __forceinline__ void pf_stage_pin(PfStageRaw<K, BF16>& raw) {
#pragma unroll
    for (int it = 0; it < PfStageRaw<K, BF16>::NIT; ++it)
#pragma unroll
        for (int j = 0; j < (BF16 ? 1 : 2); ++j)
            __asm__ volatile("" : "+v"(raw.r[it][j].x), "+v"(raw.r[it][j].y), "+v"(raw.r[it][j].z), "+v"(raw.r[it][j].w));
}

// The values of pass `it` (8 per lane) from the loaded words; zero past K
template <int K, bool BF16>
__device__ __forceinline__ void pf_raw_vals(const PfStageRaw<K, BF16>& raw, int it, int c, float v[8]) {
    if constexpr (BF16) {
        const uint32_t w[4] = {raw.r[it][0].x, raw.r[it][0].y, raw.r[it][0].z, raw.r[it][0].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(w[e] << 16);
            v[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
        }
    } else {
        const uint4 a = raw.r[it][0], b = raw.r[it][1];
        v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
        v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
    }
    if (c >= K) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    }
}

// The row's scale exponent k (its max |value| to [2^13, 2^14), frag_exp); with
// gvec set, also x_row . gvec (FP32, unscaled) in every lane, else 0.
template <int K, bool BF16>
__device__ __forceinline__ int pf_row_exp(const PfStageRaw<K, BF16>& raw, const float* gvec, float& gdot_out) {
    constexpr int NIT = PfStageRaw<K, BF16>::NIT;
    const int lane = threadIdx.x & 63;
    float amax = 0.0f, gdot = 0.0f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int c = 512 * it + 8 * lane;
        float v[8];
        pf_raw_vals(raw, it, c, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
        if (gvec != nullptr && c < K) {
            const float4 g0 = *(const float4*)(gvec + c), g1 = *(const float4*)(gvec + c + 4);
            gdot = fmaf(v[0], g0.x, gdot); gdot = fmaf(v[1], g0.y, gdot);
            gdot = fmaf(v[2], g0.z, gdot); gdot = fmaf(v[3], g0.w, gdot);
            gdot = fmaf(v[4], g1.x, gdot); gdot = fmaf(v[5], g1.y, gdot);
            gdot = fmaf(v[6], g1.z, gdot); gdot = fmaf(v[7], g1.w, gdot);
        }
    }
    gdot_out = pf_wave_sum(gdot);
    return frag_exp(pf_wave_max(amax));
}

// Pass `it` of the row at scale 2^-k: the lane's 8 values as FP16 high and low
// parts, and the sum of its 32-column sub-block (the same in lanes 4m .. 4m+3)
// as an FP16 (high, low) pair.
template <int K, bool BF16>
__device__ __forceinline__ void pf_split_pass(const PfStageRaw<K, BF16>& raw, int it, int k, h8_t& hi, h8_t& lo,
                                              _Float16& sh, _Float16& sl) {
    const int c = 512 * it + 8 * (threadIdx.x & 63);
    float v[8];
    pf_raw_vals(raw, it, c, v);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        _Float16 h, l;
        frag_split(v[e], k, h, l);
        hi[e] = h;
        lo[e] = l;
        s += ldexpf(v[e], -k);
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    frag_split(s, 5, sh, sl);
}

// Stages the row as LDS column j; the arithmetic runs for a dead column too
// (live = false), with its LDS writes skipped.
template <int K, bool BF16, bool SPLIT>
__device__ __forceinline__ void pf_stage_finish(const PfStageRaw<K, BF16>& raw, int j, bool live, _Float16* xh,
                                                _Float16* xl, _Float16* xs, int* s_exp) {
    constexpr int NIT = PfStageRaw<K, BF16>::NIT, KP = K + PF_PAD;
    const int lane = threadIdx.x & 63;
    float unused;
    const int k = pf_row_exp(raw, nullptr, unused);
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int c = 512 * it + 8 * lane;
        h8_t hi, lo;
        _Float16 sh, sl;
        pf_split_pass(raw, it, k, hi, lo, sh, sl);
        if (live && c < K) {
            *(h8_t*)(xh + j * KP + c) = hi;
            if constexpr (SPLIT) *(h8_t*)(xl + j * KP + c) = lo;
            if ((lane & 3) == 0) {
                const int sb = c >> 5;   // sub-block: block sb / 8, slot sb % 8
                xs[((sb >> 3) * PREFILL_TILE + j) * 16 + (sb & 7)] = sh;
                xs[((sb >> 3) * PREFILL_TILE + j) * 16 + 8 + (sb & 7)] = sl;
            }
        }
    }
    if (live && lane == 0) s_exp[j] = k;
}

// The same staging of token t into the token planes in device memory (the
// route pass makes them once per token; every gate/up workgroup of the token's
// tiles then copies them into LDS with no arithmetic).  Returns x_t . gvec.
template <int K, bool BF16, bool SPLIT>
__device__ __forceinline__ float pf_stage_planes(const PfStageRaw<K, BF16>& raw, int64_t t, const PrefillParams& p,
                                                 const float* gvec) {
    constexpr int NIT = PfStageRaw<K, BF16>::NIT;
    const int lane = threadIdx.x & 63;
    float gdot;
    const int k = pf_row_exp(raw, gvec, gdot);
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int c = 512 * it + 8 * lane;
        h8_t hi, lo;
        _Float16 sh, sl;
        pf_split_pass(raw, it, k, hi, lo, sh, sl);
        if (c < K) {
            *(h8_t*)((_Float16*)p.xhi + t * K + c) = hi;
            if constexpr (SPLIT) *(h8_t*)((_Float16*)p.xlo + t * K + c) = lo;
            if ((lane & 3) == 0)
                p.xsum[t * (K / 32) + (c >> 5)] =
                    (uint32_t)__builtin_bit_cast(uint16_t, sh) | (uint32_t)__builtin_bit_cast(uint16_t, sl) << 16;
        }
    }
    if (lane == 0) p.xexp[t] = k;
    return gdot;
}

// A token column of the gate/up kernel's B operand as the route pass left it:
// the lane's 8 columns per 512-column pass of the high (and low) plane, the
// lane's sub-block sum pair (lanes below K / 32) and the exponent.
template <int K, bool SPLIT>
struct PfPlanes {
    static constexpr int NIT = K >= 512 ? K / 512 : 1;
    uint4 h[NIT];
    uint4 l[SPLIT ? NIT : 1];
    uint32_t s;
    int e;
};

// live = false: every lane reads the row's first words (in bounds, unused)
template <int K, bool SPLIT>
__device__ __forceinline__ void pf_planes_load(const uint16_t* xhi, const uint16_t* xlo, const uint32_t* xsum,
                                               const int* xexp, int64_t t, bool live, PfPlanes<K, SPLIT>& r) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int it = 0; it < PfPlanes<K, SPLIT>::NIT; ++it) {
        // lanes past K (K = 256) read the row's first columns again
        const int c = live ? (512 * it + 8 * lane) % K : 0;
        r.h[it] = *(const uint4*)(xhi + t * K + c);
        if constexpr (SPLIT) r.l[it] = *(const uint4*)(xlo + t * K + c);
    }
    r.s = xsum[t * (K / 32) + (live ? min(lane, K / 32 - 1) : 0)];
    r.e = xexp[t];
}

template <int K, bool SPLIT>
__device__ __forceinline__ void pf_planes_pin(PfPlanes<K, SPLIT>& r) {
#pragma unroll
    for (int it = 0; it < PfPlanes<K, SPLIT>::NIT; ++it) {
        __asm__ volatile("" : "+v"(r.h[it].x), "+v"(r.h[it].y), "+v"(r.h[it].z), "+v"(r.h[it].w));
        if constexpr (SPLIT) __asm__ volatile("" : "+v"(r.l[it].x), "+v"(r.l[it].y), "+v"(r.l[it].z), "+v"(r.l[it].w));
    }
    __asm__ volatile("" : "+v"(r.s), "+v"(r.e));
}

// The column's LDS copy (the layout pf_stage_finish writes)
template <int K, bool SPLIT>
__device__ __forceinline__ void pf_planes_store(const PfPlanes<K, SPLIT>& r, int j, bool live, _Float16* xh,
                                                _Float16* xl, _Float16* xs, int* s_exp) {
    constexpr int KP = K + PF_PAD;
    const int lane = threadIdx.x & 63;
    if (!live) return;
#pragma unroll
    for (int it = 0; it < PfPlanes<K, SPLIT>::NIT; ++it) {
        const int c = 512 * it + 8 * lane;
        if (c < K) {
            *(uint4*)(xh + j * KP + c) = r.h[it];
            if constexpr (SPLIT) *(uint4*)(xl + j * KP + c) = r.l[it];
        }
    }
    if (lane < K / 32) {
        const int sb = lane;
        xs[((sb >> 3) * PREFILL_TILE + j) * 16 + (sb & 7)] = __builtin_bit_cast(_Float16, (uint16_t)(r.s & 0xFFFFu));
        xs[((sb >> 3) * PREFILL_TILE + j) * 16 + 8 + (sb & 7)] = __builtin_bit_cast(_Float16, (uint16_t)(r.s >> 16));
    }
    if (lane == 0) s_exp[j] = r.e;
}

// ------------------------------------------------------------ the GEMM core
//
// A wave accumulates W[16 rows] x B^T over K = NB * 256 columns for NMAT weight
// matrices sharing the B operand, for CPW row chunks in turn (the chunk stride
// is given in bytes); one register ring of super-blocks runs across the chunks,
// so the loads of the next chunk are in flight while one ends.  prefetch()
// loads the first blocks before the caller stages the tokens, so that the two
// overlap.  D layout: lane l holds rows 4(l/16) + i, token column l % 16.
// IP: the Q3_K operand form (frag_step): the down kernel takes the in-place
// one (the Q3_K-routed, Q6_K-shared down projections 44.3/44.7 -> 43.1/42.8 us
// at the 128-token prompt), the gate/up kernel the other (its mixed instance
// measured 94.2/94.8 -> 97.2/96.7 us with the in-place form, at 128 VGPRs).
template <int T, int NMAT, int NB, int CPW, int RING = PF_RING, bool IP = true>
struct PfRows {
    static constexpr int NW = FragGeo<T>::NW, BB = frag_unit_bytes<T>(), NBT = NB * CPW;
    // R ring slots: block b lives in slot b % R; while block b is computed,
    // blocks b+1 .. b+R-1 are in flight (all of them for short rows)
    static constexpr bool UNROLLED = NBT <= RING;
    static constexpr int R = UNROLLED && NBT + 1 < RING ? NBT + 1 : RING;
    static_assert(R >= 2, "a ring of at least two slots");
    uint32_t raw[R][NMAT][NW];
    const uint8_t* W[NMAT];
    int64_t chunk_stride;
    int q;
    int nbt = NBT;   // blocks this workgroup runs: NB x its chunks (at most CPW)

    __device__ __forceinline__ void load(int b, uint32_t (&dst)[NMAT][NW]) {
        const int64_t off = (int64_t)(b / NB) * chunk_stride + (b % NB) * BB;
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) frag_load<T>(W[mt] + off, q, dst[mt]);
    }

    // (a ring slot past nbt re-reads the last block: in bounds, unused)
    __device__ __forceinline__ void prefetch() {
#pragma unroll
        for (int b = 0; b < (NBT < R - 1 ? NBT : R - 1); ++b) load(min(b, nbt - 1), raw[b]);
    }

    // one 256-column unit of eight Q8_0 blocks (unit kb of its row): step m is
    // block m, P_m its exact integer product with the token planes, acc +=
    // d_m * P_m.  The D layout wants the d of rows 4q .. 4q+3, held by other
    // lanes (k-group qq of row r loaded blocks 2qq, 2qq+1), so each lane puts
    // its two into the wave's LDS table [block][row] and reads four back per
    // step (one wave's LDS accesses complete in order: no barrier)
    template <bool SPLIT>
    __device__ __forceinline__ void block_q8(const uint32_t (&cur)[NMAT][NW], int kb, const _Float16* xh,
                                             const _Float16* xl, f32x4 (&acc)[NMAT]) {
        static_assert(NMAT == 1, "one Q8_0 matrix a wave");
        constexpr int KP = NB * 256 + PF_PAD;
        __shared__ __attribute__((aligned(16))) float s_d8[PF_WAVES][8][16];
        const int lane = threadIdx.x & 63, tok = lane & (PREFILL_TILE - 1), qq = (q + 3) & 3;
        const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        s_d8[wave][2 * qq][lane & 15] = frag_h2f(cur[0][16]);
        s_d8[wave][2 * qq + 1][lane & 15] = frag_h2f(cur[0][17]);
        const int brow = tok * KP + kb * 256 + frag_lane_col<T>(qq);
        FragPrep<T> sp;
        pf_unroll(std::make_integer_sequence<int, 8>{}, [&](auto mc) {
            constexpr int m = decltype(mc)::value;
            const int off = brow + frag_col<T, m>();
            const h8_t bh = *(const h8_t*)(xh + off);
            h8_t a[2];
            frag_step<T, m, IP>(cur[0], sp, q, a);
            f32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], bh, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            if constexpr (SPLIT) {
                const h8_t bl = *(const h8_t*)(xl + off);
                P = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], bl, P, 0, 0, 0);
            }
            const float4 d = *(const float4*)&s_d8[wave][m][4 * q];
            acc[0][0] = fmaf(d.x, P[0], acc[0][0]);
            acc[0][1] = fmaf(d.y, P[1], acc[0][1]);
            acc[0][2] = fmaf(d.z, P[2], acc[0][2]);
            acc[0][3] = fmaf(d.w, P[3], acc[0][3]);
        });
    }

    // one super-block (block kb of its row): P = sum over its 8 steps of the exact
    // integer operands times the token planes, then acc += d * P (- dmin * min term)
    template <bool SPLIT>
    __device__ __forceinline__ void block_k(const uint32_t (&cur)[NMAT][NW], int kb, const _Float16* xh,
                                            const _Float16* xl, const _Float16* xs, f32x4 (&acc)[NMAT]) {
        constexpr int KP = NB * 256 + PF_PAD;
        // B column lane % 16 reads LDS token column lane % PREFILL_TILE
        const int lane = threadIdx.x & 63, tok = lane & (PREFILL_TILE - 1);
        const int brow = tok * KP + kb * 256 + frag_lane_col<T>((q + 3) & 3);
        f32x4 P[NMAT];
        FragPrep<T> sp[NMAT];
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) {
            P[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            frag_prep<T, IP>(cur[mt], q, sp[mt]);
        }
        pf_unroll(std::make_integer_sequence<int, 8>{}, [&](auto mc) {
            constexpr int m = decltype(mc)::value;
            const int off = brow + frag_col<T, m>();
            const h8_t bh = *(const h8_t*)(xh + off);
            h8_t bl;
            if constexpr (SPLIT) bl = *(const h8_t*)(xl + off);
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt) {
                h8_t a[2];
                frag_step<T, m, IP>(cur[mt], sp[mt], q, a);
                P[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], bh, P[mt], 0, 0, 0);
                if constexpr (FragGeo<T>::NA == 2) P[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1], bh, P[mt], 0, 0, 0);
                if constexpr (SPLIT)
                    P[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag_lo_operand<T>(a), bl, P[mt], 0, 0, 0);
            }
        });
        f32x4 Mn[NMAT];
        if constexpr (FragGeo<T>::MIN) {
            const h4_t bs = *(const h4_t*)(xs + (kb * PREFILL_TILE + tok) * 16 + 4 * q);
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt)
                Mn[mt] = __builtin_amdgcn_mfma_f32_16x16x16f16(frag_mins<T>(cur[mt], q), bs,
                                                               f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        }
        // d (and dmin) of D row 4q + i live in the header word of A lane 4q + i
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t hdr = (uint32_t)__shfl((int)cur[mt][FragGeo<T>::HDR], 4 * q + i, 64);
                acc[mt][i] = fmaf(frag_d<T>(hdr), P[mt][i], acc[mt][i]);
                if constexpr (FragGeo<T>::MIN) acc[mt][i] = fmaf(-frag_dmin(hdr), Mn[mt][i], acc[mt][i]);
            }
    }

    template <bool SPLIT>
    __device__ __forceinline__ void block(const uint32_t (&cur)[NMAT][NW], int kb, const _Float16* xh,
                                          const _Float16* xl, const _Float16* xs, f32x4 (&acc)[NMAT]) {
        if constexpr (T == T_Q8_0) block_q8<SPLIT>(cur, kb, xh, xl, acc);
        else block_k<SPLIT>(cur, kb, xh, xl, xs, acc);
    }

    // All NBT blocks; end(c, acc) runs after the last block of chunk c, with the
    // ring already loading chunk c + 1, and must leave acc zeroed.  The refill
    // of block b + R - 1 goes to the slot block b - 1 has just released, ahead
    // of block b's arithmetic (the sched barrier stops the scheduler from
    // sinking it to the end of the loop body, which would expose the memory
    // latency once per iteration).
    template <bool SPLIT, class End>
    __device__ __forceinline__ void run(const _Float16* xh, const _Float16* xl, const _Float16* xs,
                                        f32x4 (&acc)[NMAT], End&& end) {
        if constexpr (UNROLLED) {
#pragma unroll
            for (int b = 0; b < NBT; ++b) {
                if (b >= nbt) break;
                if (b + R - 1 < NBT) load(b + R - 1, raw[(b + R - 1) % R]);
                __builtin_amdgcn_sched_barrier(0);
                block<SPLIT>(raw[b % R], b % NB, xh, xl, xs, acc);
                if ((b + 1) % NB == 0) end(b / NB, acc);
            }
        } else {
#pragma unroll 1
            for (int b0 = 0; b0 < nbt; b0 += R)
#pragma unroll
            for (int bi = 0; bi < R; ++bi) {
                const int b = b0 + bi;
                if (NB % R != 0 && b >= nbt) break;   // (a whole number of rings otherwise)
                // the tail re-reads the last block (in bounds, unused)
                load(min(b + R - 1, nbt - 1), raw[(bi + R - 1) % R]);
                __builtin_amdgcn_sched_barrier(0);
                block<SPLIT>(raw[bi], b % NB, xh, xl, xs, acc);
                if ((b + 1) % NB == 0) end(b / NB, acc);
            }
        }
    }
};

// Workgroup -> (tile, row chunk).  Workgroup i runs on XCD i % 8 (the
// dispatcher deals workgroups to the eight XCDs in turn), so the nch row
// chunks of one tile are given indices that agree mod 8: the tile's token rows
// are then fetched into one XCD's L2 and read there by all of its chunks,
// instead of once per XCD (8 x the token bytes through the fabric).  Launches
// are 1-D, nch x round_up(max_tiles, 8) workgroups; nch is a power of two (its
// log2 comes in: a division would sit ahead of the first loads).
constexpr int PF_XCDS = 8;
__device__ __forceinline__ void pf_wg(int nch_log2, int& tile, int& chunk) {
    const int i = blockIdx.x, r = i / PF_XCDS;
    chunk = r & ((1 << nch_log2) - 1);
    tile = (r >> nch_log2) * PF_XCDS + i % PF_XCDS;
}
// The gate/up kernel's workgroups: the first nbig x mt (mt = max_tiles rounded
// up to 8) take CB 64-row chunks of a tile, the rest one, in that order, so
// the dispatcher's last workgroups are the short ones (a launch runs ~2
// workgroups a slot, and its end waits for the last started).  Per tile, nbig
// workgroups cover chunks 0 .. CB nbig - 1 and nsmall the remaining ones; the
// chunks of one tile again agree mod 8.  r / d is one multiply-high by
// m = ceil(2^32 / d) (0 for d = 1), exact for every r a launch reaches.
struct PfSplit {
    int nbig, nsmall;
    unsigned mbig, msmall;
};
template <int CB>
__device__ __forceinline__ void pf_wg_split(int max_tiles, const PfSplit& sp, int& tile, int& chunk0, int& nch) {
    const int mt = (max_tiles + PF_XCDS - 1) & ~(PF_XCDS - 1);
    const int i = blockIdx.x, na = sp.nbig * mt;
    const bool big = i < na;
    const int j = big ? i : i - na, r = j / PF_XCDS;
    const int d = big ? sp.nbig : sp.nsmall;
    const unsigned m = big ? sp.mbig : sp.msmall;
    const int g = m ? (int)__umulhi((unsigned)r, m) : r;
    const int k = r - g * d;
    tile = g * PF_XCDS + j % PF_XCDS;
    chunk0 = big ? CB * k : CB * sp.nbig + k;
    nch = big ? CB : 1;
}
static unsigned pf_magic(int d) { return d > 1 ? (unsigned)((0x100000000ull + d - 1) / d) : 0u; }

// The tile's descriptor, when tile is below the launch's tile count: the
// count and the descriptor are loaded together (every slot below max_tiles
// exists; past the count it holds stale words, never used).  The test reads
// the descriptor too (a live tile has at least one pair), so that the compiler
// cannot move its load behind the branch.
__device__ __forceinline__ bool pf_live_tile(const int* n_tiles, const int4* tiles, int max_tiles, int tile, int4& td) {
    const int n = *n_tiles;
    td = tiles[min(tile, max_tiles - 1)];
    return (tile < n) & (td.z > 0);
}

// The GEMM kernels take what their first loads need (the tile list, the token
// source) as leading scalar arguments, which the build preloads into scalar
// registers: the first loads need no round trip to the argument block.
struct PfHot {
    const int* n_tiles;
    const int4* tiles;
    const int* tile_tok;
    const void* src;   // P1: the tokens x; P2: the activations
    int max_tiles;
};
static int pf_grid(int nch, int max_tiles) { return nch * ((max_tiles + PF_XCDS - 1) / PF_XCDS * PF_XCDS); }

// ------------------------------------------------------------ P0

constexpr int PF_ROUTE_THREADS = 1024;   // one workgroup (a constant: blockDim.x costs a memory round trip)
constexpr int PF_ROUTE_IDS = 4;          // (token, slot) ids a routing thread keeps in registers

// Tokens a staging workgroup takes: one wave each on waves 0..3 (one a SIMD;
// sixteen a workgroup measured 1.2 us longer for the route pass at 128 tokens)
constexpr int PF_STAGE_TOKENS = 4;

// Workgroup 0 routes; workgroup b > 0 stages tokens 4 (b - 1) .. 4 b - 1 into
// the token planes, one wave a token, and sets the shared expert's gate per
// token (sigmoid(x . g_inp), shared_expert.py:221-251).
template <int NBH, bool XBF16>
__global__ __launch_bounds__(PF_ROUTE_THREADS) void k_prefill_route(PrefillParams p) {
    __shared__ int cnt[PREFILL_MAX_EXPERTS], off[PREFILL_MAX_EXPERTS], fill[PREFILL_MAX_EXPERTS];
    __shared__ int toff[PREFILL_MAX_EXPERTS];
    __shared__ int wsum[16][2];
    const int T = p.n_tokens, K = p.top_k, E = p.n_experts, TK = T * K;
    const int e = threadIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (blockIdx.x > 0) {
        constexpr int H = NBH * 256;
        const int t = (blockIdx.x - 1) * PF_STAGE_TOKENS + wave;
        if (wave >= PF_STAGE_TOKENS || t >= T) return;
        PfStageRaw<H, XBF16> r;
        pf_stage_load<H, XBF16>(p.x, t, true, r);
        const float* gv = p.has_shared ? p.sh_gate_inp : nullptr;
        const float gd = pf_stage_planes<H, XBF16, !XBF16>(r, t, p, gv);
        if (p.has_shared && lane == 0) p.sh_scale[t] = gv != nullptr ? pf_sigmoid(gd) : 1.0f;
        return;
    }
    if (e < E) { cnt[e] = 0; fill[e] = 0; }
    __syncthreads();
    // a thread's first PF_ROUTE_IDS ids stay in registers for the second pass
    // (one memory round trip fewer on the pass's path); the rest are re-read
    int idr[PF_ROUTE_IDS];
#pragma unroll
    for (int j = 0; j < PF_ROUTE_IDS; ++j) {
        const int i = threadIdx.x + j * PF_ROUTE_THREADS;
        idr[j] = i < TK ? p.ids[i] : 0;
    }
    for (int i = threadIdx.x; i < TK; i += PF_ROUTE_THREADS) {
        const int j = (i - threadIdx.x) / PF_ROUTE_THREADS;
        const int id = j < PF_ROUTE_IDS ? idr[j < PF_ROUTE_IDS ? j : 0] : p.ids[i];
        if (id < 0 || id >= E) atomicOr(&p.flags[FLAG_BAD_ID], 1);
        else atomicAdd(&cnt[id], 1);
    }
    __syncthreads();
    // exclusive scans of pair counts and tile counts over experts
    const int c = e < E ? cnt[e] : 0, tc = (c + PREFILL_TILE - 1) / PREFILL_TILE;
    int ic = c, it = tc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int yc = __shfl_up(ic, o, 64), yt = __shfl_up(it, o, 64);
        if (lane >= o) { ic += yc; it += yt; }
    }
    if (lane == 63) { wsum[wave][0] = ic; wsum[wave][1] = it; }
    __syncthreads();
    int bc = 0, bt = 0, tott = 0;
    for (int w = 0; w < 16; ++w) {
        if (w < wave) { bc += wsum[w][0]; bt += wsum[w][1]; }
        tott += wsum[w][1];
    }
    // the shared expert's tiles come first (tile j: tokens 16 j .. 16 j + 15):
    // they are the fullest tiles and, with a shared expert of another type, the
    // slowest, so they start in the launch's first round rather than its tail
    const int nsh = p.has_shared ? (T + PREFILL_TILE - 1) / PREFILL_TILE : 0;
    const int first = bc + ic - c, tfirst = nsh + bt + it - tc;
    if (e < E) {
        off[e] = first;
        toff[e] = tfirst;
        for (int j = 0; j < tc; ++j)
            ((int4*)p.tiles)[tfirst + j] =
                make_int4(e, first + PREFILL_TILE * j, min(PREFILL_TILE, c - PREFILL_TILE * j), 0);
    }
    for (int j = threadIdx.x; j < nsh; j += PF_ROUTE_THREADS)
        ((int4*)p.tiles)[j] = make_int4(-1, TK + PREFILL_TILE * j, min(PREFILL_TILE, T - PREFILL_TILE * j), 0);
    if (threadIdx.x == 0) *p.n_tiles = nsh + tott;
    __syncthreads();
    // pair order inside an expert follows the atomics; a pair's result does not
    // depend on its column in the tile, so outputs do not depend on it.  Each
    // column also gets the output row of its (token, slot), where the down
    // kernel writes it and the combine reads it.
    for (int i = threadIdx.x; i < TK; i += PF_ROUTE_THREADS) {
        const int j = (i - threadIdx.x) / PF_ROUTE_THREADS;
        const int id = j < PF_ROUTE_IDS ? idr[j < PF_ROUTE_IDS ? j : 0] : p.ids[i];
        if (id >= 0 && id < E) {
            const int k = atomicAdd(&fill[id], 1);
            const int c = (toff[id] + k / PREFILL_TILE) * PREFILL_TILE + k % PREFILL_TILE;
            p.tile_tok[c] = i / K;
            p.tile_dst[c] = (i / K) * p.S + i % K;
        }
    }
    if (p.has_shared) {
        // column c of shared tile j is token PREFILL_TILE j + c
        for (int t = threadIdx.x; t < T; t += PF_ROUTE_THREADS) {
            p.tile_tok[t] = t;
            p.tile_dst[t] = t * p.S + K;
        }
    }
}

// ------------------------------------------------------------ P1

// SGT: the shared expert's gate/up type.  A tile is one expert's, so a
// workgroup runs one type: with SGT != GT, the shared tiles (expert -1) take
// the SGT instance of the body and the routed tiles the GT one, in one launch.
template <int GT, int SGT, int NBH, bool XBF16, int CPW>
__global__ __launch_bounds__(64 * PF_WAVES) PF_OCC_GU void k_prefill_gate_up(const int* n_tiles, const int4* tiles,
                                                                             const int* tile_tok, const void* xsrc,
                                                                             int max_tiles, int nbig, int nsmall,
                                                                             unsigned mbig, unsigned msmall,
                                                                             PrefillParams p) {
    static_assert(CPW >= 1, "workgroups take one or CPW chunks");
    constexpr int H = NBH * 256, KP = H + PF_PAD;
    constexpr bool SPLIT = !XBF16;   // BF16 tokens are exact in the high plane
    __shared__ __attribute__((aligned(16))) _Float16 xh[PREFILL_TILE * KP];
    __shared__ __attribute__((aligned(16))) _Float16 xl[SPLIT ? PREFILL_TILE * KP : 8];
    __shared__ __attribute__((aligned(16))) _Float16 xs[PREFILL_TILE * NBH * 16];
    __shared__ __attribute__((aligned(16))) float s_up[PF_WAVES / 2][64][4];
    __shared__ int s_exp[PREFILL_TILE];
    int tile, chunk0, nch;
    pf_wg_split<CPW>(max_tiles, PfSplit{nbig, nsmall, mbig, msmall}, tile, chunk0, nch);
    // the tile's tokens, one a lane (lane j: column j), need the tile index only,
    // so their load goes out ahead of the descriptor's
    const int pt = tile_tok[min(tile, max_tiles - 1) * PREFILL_TILE + (threadIdx.x & (PREFILL_TILE - 1))];
    int4 td;
    const bool live = pf_live_tile(n_tiles, tiles, max_tiles, tile, td);
    // the argument-block fields the weight addresses need, awaited together
    // with the tile (each would otherwise be loaded after the branch below)
    const uint8_t *gate = p.gate, *up = p.up, *sh_gate = p.sh_gate, *sh_up = p.sh_up;
    const int64_t gate_eb = p.gate_eb, up_eb = p.up_eb;
    const uint16_t *xhi = (const uint16_t*)xsrc, *xlo = p.xlo;
    const uint32_t* xsum = p.xsum;
    const int* xexp = p.xexp;
    __asm__ volatile("" ::"s"(gate), "s"(up), "s"(sh_gate), "s"(sh_up), "s"(gate_eb), "s"(up_eb), "s"(xlo), "s"(xsum),
                     "s"(xexp), "s"(td.x), "s"(td.y), "s"(td.z), "s"((int)live));
    if (!live) return;
    const int e = td.x, first = td.y, cnt = td.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4;
    // waves 0..3: gate rows, waves 4..7: the same up rows; nch chunks of 64 rows
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int mat = wv / (PF_WAVES / 2), wsub = wv % (PF_WAVES / 2);
    const int rbase = chunk0 * PF_ROWS_GU + wsub * 16;

    // (selects of wave-uniform values, no branch: each branch would load its
    // own arguments after the tile's round trip)
    const uint8_t* Ws = mat ? sh_up : sh_gate;
    const uint8_t* Wr = (mat ? up : gate) + (int64_t)max(e, 0) * (mat ? up_eb : gate_eb);
    const uint8_t* W0 = e < 0 ? Ws : Wr;
    // the wave's token column wv (and wv + 8 in 16-token tiles; a column past
    // cnt reads token 0's first words and stages nothing): their loads go out
    // before the weight prefetch, so the staging below waits for them only
    constexpr bool TWO = PREFILL_TILE == 2 * PF_WAVES;
    static_assert(PREFILL_TILE == PF_WAVES || TWO, "one or two token columns per wave");
    const bool l0 = wv < cnt, l1 = TWO && wv + PF_WAVES < cnt;
    // (columns at or past cnt hold stale words: token 0 stands in)
    const int t0 = l0 ? __builtin_amdgcn_readlane(pt, wv) : 0;
    const int t1 = l1 ? __builtin_amdgcn_readlane(pt, (wv + PF_WAVES) & (PREFILL_TILE - 1)) : 0;
    PfPlanes<H, SPLIT> r0, r1;
    pf_planes_load<H, SPLIT>(xhi, xlo, xsum, xexp, t0, l0, r0);
    if constexpr (TWO) pf_planes_load<H, SPLIT>(xhi, xlo, xsum, xexp, t1, l1, r1);
    __builtin_amdgcn_sched_barrier(0);

    auto body = [&](auto tc) {
        constexpr int T = decltype(tc)::value;
        const int64_t row_bytes = (int64_t)NBH * frag_unit_bytes<T>();
        PfRows<T, 1, NBH, CPW, (SGT != GT && T == SGT) ? PF_RING_SHARED : PF_RING, false> g;
        g.W[0] = W0 + (int64_t)(rbase + (lane & 15)) * row_bytes;
        g.chunk_stride = PF_ROWS_GU * row_bytes;
        g.q = q;
        g.nbt = NBH * nch;
        g.prefetch();
        // (a compiler memory barrier: the prefetched values are first used after
        // the staging's branches, and hipcc would otherwise sink their loads there)
        __asm__ volatile("" ::: "memory");
        pf_planes_pin(r0);
        if constexpr (TWO) pf_planes_pin(r1);
        __builtin_amdgcn_sched_barrier(0);
        pf_planes_store(r0, wv, l0, xh, xl, xs, s_exp);
        if constexpr (TWO) pf_planes_store(r1, wv + PF_WAVES, l1, xh, xl, xs, s_exp);
        __syncthreads();

        const int col = lane & 15;
        const float sc = col < cnt ? ldexpf(1.0f, s_exp[col]) : 0.0f;
        f32x4 acc[1] = {{0, 0, 0, 0}};
        g.template run<SPLIT>(xh, xl, xs, acc, [&](int c, f32x4 (&a)[1]) {
            // the up waves hand their results to the gate waves of the same rows
            // (same D layout, so no transposition); columns at or past cnt hold
            // stale LDS and are never stored
            if (mat) *(float4*)s_up[wsub][lane] = make_float4(a[0][0], a[0][1], a[0][2], a[0][3]);
            __syncthreads();
            if (!mat && col < cnt) {
                const float4 u = *(const float4*)s_up[wsub][lane];
                float4 o;
                o.x = pf_silu_mul(a[0][0] * sc, u.x * sc);
                o.y = pf_silu_mul(a[0][1] * sc, u.y * sc);
                o.z = pf_silu_mul(a[0][2] * sc, u.z * sc);
                o.w = pf_silu_mul(a[0][3] * sc, u.w * sc);
                *(float4*)(p.act + (int64_t)(first + col) * p.inter + rbase + PF_ROWS_GU * c + 4 * q) = o;
            }
            __syncthreads();
            a[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        });
    };
    if constexpr (SGT == GT) body(std::integral_constant<int, GT>{});
    else if (e < 0) body(std::integral_constant<int, SGT>{});   // (uniform: the workgroup's tile)
    else body(std::integral_constant<int, GT>{});
}

// ------------------------------------------------------------ P2

// SDT: the shared expert's down type (its tiles take that instance of the
// body, as in the gate/up kernel).
template <int DT, int SDT, int NBI, int CPW>
__global__ __launch_bounds__(64 * PF_WAVES) PF_OCC_DOWN
__attribute__((amdgpu_waves_per_eu(SDT != DT && DT != T_Q8_0 && NBI <= 2 ? PF_MIXED_WAVES_DOWN : 1))) void k_prefill_down(const int* n_tiles, const int4* tiles,
                                                                           const int* tile_dst, const void* act,
                                                                           int max_tiles, int nch_log2, PrefillParams p) {
    constexpr int I = NBI * 256, KP = I + PF_PAD;
    __shared__ __attribute__((aligned(16))) _Float16 xh[PREFILL_TILE * KP];
    __shared__ __attribute__((aligned(16))) _Float16 xl[PREFILL_TILE * KP];
    __shared__ __attribute__((aligned(16))) _Float16 xs[PREFILL_TILE * NBI * 16];
    __shared__ int s_exp[PREFILL_TILE];
    int tile, chunk;
    pf_wg(nch_log2, tile, chunk);
    // the output row of the lane's token column (stale past the tile's count,
    // never used there), loaded with the tile's descriptor
    const int dst = tile_dst[min(tile, max_tiles - 1) * PREFILL_TILE + (threadIdx.x & (PREFILL_TILE - 1))];
    int4 td;
    const bool live = pf_live_tile(n_tiles, tiles, max_tiles, tile, td);
    const uint8_t *down = p.down, *sh_down = p.sh_down;
    const int64_t down_eb = p.down_eb;
    __asm__ volatile("" ::"s"(down), "s"(sh_down), "s"(down_eb), "s"(td.x), "s"(td.y), "s"(td.z), "s"((int)live));
    if (!live) return;
    const int e = td.x, first = td.y, cnt = td.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4;
    const int rbase = chunk * PF_ROWS_DOWN * CPW + wave * 16;
    const uint8_t* W0 = e < 0 ? sh_down : down + (int64_t)max(e, 0) * down_eb;

    auto body = [&](auto tc) {
        constexpr int T = decltype(tc)::value;
        const int64_t row_bytes = (int64_t)NBI * frag_unit_bytes<T>();
        PfRows<T, 1, NBI, CPW, (SDT != DT && T == SDT) ? PF_RING_SHARED_DOWN : PF_RING_DOWN> g;
        g.W[0] = W0 + (int64_t)(rbase + (lane & 15)) * row_bytes;
        g.chunk_stride = PF_ROWS_DOWN * row_bytes;
        g.q = q;
        // (here the live activation rows follow the prefetch: issuing the tile's
        // rows first, as the gate/up kernel does with its tokens, measured 66 ->
        // 72 us for this kernel at the 128-token prompt)
        g.prefetch();
        for (int j = wave; j < cnt; j += PF_WAVES) {
            PfStageRaw<I, false> r;
            pf_stage_load<I, false>(act, first + j, true, r);
            pf_stage_finish<I, false, true>(r, j, true, xh, xl, xs, s_exp);
        }
        __syncthreads();

        const int col = lane & 15;
        const float sc = col < cnt ? ldexpf(1.0f, s_exp[col]) : 0.0f;
        f32x4 acc[1] = {{0, 0, 0, 0}};
        g.template run<true>(xh, xl, xs, acc, [&](int c, f32x4 (&a)[1]) {
            if (col < cnt)
                *(float4*)(p.ypair + (int64_t)dst * p.hidden + rbase + PF_ROWS_DOWN * c + 4 * q) =
                    make_float4(a[0][0] * sc, a[0][1] * sc, a[0][2] * sc, a[0][3] * sc);
            a[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        });
    };
    if constexpr (SDT == DT) body(std::integral_constant<int, DT>{});
    else if (e < 0) body(std::integral_constant<int, SDT>{});   // (uniform: the workgroup's tile)
    else body(std::integral_constant<int, DT>{});
}

// ------------------------------------------------------------ P3

// Eight slots at a time: their expert ids and weights (scalar loads) and
// their eight expert outputs (rows t S + s, written there by the down
// kernel) together, then the sum in top-k order; the shared expert's output
// (row t S + top_k) is loaded with the first eight and added last.
constexpr int PF_COMBINE_SLOTS = 8;
__global__ __launch_bounds__(256) void k_prefill_combine(PrefillParams p) {
    const int t = blockIdx.y, h = blockIdx.x * 256 + threadIdx.x;
    if (h >= p.hidden) return;
    const float* yt = p.ypair + (int64_t)t * p.S * p.hidden + h;
    const int32_t* it = p.ids + t * p.top_k;
    const float* wt = p.weights + t * p.top_k;
    const float ssh = p.has_shared ? p.sh_scale[t] : 0.0f;
    const float ysh = p.has_shared ? yt[(int64_t)p.top_k * p.hidden] : 0.0f;
    float acc = 0.0f;
    for (int s0 = 0; s0 < p.top_k; s0 += PF_COMBINE_SLOTS) {
        int id[PF_COMBINE_SLOTS];
        float w[PF_COMBINE_SLOTS], y[PF_COMBINE_SLOTS];
#pragma unroll
        for (int j = 0; j < PF_COMBINE_SLOTS; ++j) {
            const int s = min(s0 + j, p.top_k - 1);
            id[j] = it[s];
            w[j] = wt[s];
            y[j] = yt[(int64_t)s * p.hidden];
        }
#pragma unroll
        for (int j = 0; j < PF_COMBINE_SLOTS; ++j)   // (an expert id out of range: no row, flagged by the route pass)
            if (s0 + j < p.top_k && id[j] >= 0 && id[j] < p.n_experts) acc = __fadd_rn(acc, __fmul_rn(w[j], y[j]));
    }
    if (p.has_shared) acc = __fadd_rn(acc, __fmul_rn(ssh, ysh));
    p.y[(int64_t)t * p.hidden + h] = acc;
    if (!isfinite(acc)) atomicOr(&p.flags[FLAG_NONFINITE], 1);
}

// ------------------------------------------------------------ host side

// gate/up: the K-quants; down: the K-quants and Q8_0 (the reference model's
// first-layer down projection)
static bool pf_type(int t) { return t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }
static bool pf_down_type(int t) { return pf_type(t) || t == T_Q8_0; }
static bool pf_dim(int n) { return n == 256 || n == 512 || n == 1024 || n == 2048; }

bool prefill_supported(const PrefillParams& p) {
    if (!pf_dim(p.hidden) || !pf_dim(p.inter) || p.n_experts < 1 || p.n_experts > PREFILL_MAX_EXPERTS) return false;
    if (!(pf_type(p.gate_type) && p.up_type == p.gate_type && pf_down_type(p.down_type))) return false;
    // a shared expert inside the grouped kernels: the routed types, or Q6_K
    // (the reference model's shared experts beside Q3_K or Q4_K routed ones)
    if (p.has_shared && ((p.sh_gate_type != p.gate_type && p.sh_gate_type != T_Q6_K) ||
                         p.sh_up_type != p.sh_gate_type ||
                         (p.sh_down_type != p.down_type && p.sh_down_type != T_Q6_K)))
        return false;
    return true;
}

PrefillLayout prefill_layout(int n_tokens, int top_k, int n_experts, int hidden, int inter, int has_shared) {
    PrefillLayout L;
    const int S = top_k + (has_shared ? 1 : 0);
    const int64_t P = (int64_t)n_tokens * S;
    const int64_t TK = (int64_t)n_tokens * top_k;
    L.max_tiles = (int)(std::min<int64_t>(n_experts, TK) + (TK + PREFILL_TILE - 1) / PREFILL_TILE +
                        (has_shared ? (n_tokens + PREFILL_TILE - 1) / PREFILL_TILE : 0));
    L.flags_off = 0;
    L.scale_off = align256(WS_HEAD_BYTES);
    L.tiles_off = align256(L.scale_off + (int64_t)n_tokens * 4);
    L.ntiles_off = align256(L.tiles_off + (int64_t)std::max(L.max_tiles, 1) * 16);
    L.tok_off = align256(L.ntiles_off + 4);
    L.dst_off = align256(L.tok_off + (int64_t)std::max(L.max_tiles, 1) * PREFILL_TILE * 4);
    L.act_off = align256(L.dst_off + (int64_t)std::max(L.max_tiles, 1) * PREFILL_TILE * 4);
    L.ypair_off = align256(L.act_off + P * inter * 4);
    L.xhi_off = align256(L.ypair_off + P * hidden * 4);
    L.xlo_off = align256(L.xhi_off + (int64_t)n_tokens * hidden * 2);
    L.xsum_off = align256(L.xlo_off + (int64_t)n_tokens * hidden * 2);
    L.xexp_off = align256(L.xsum_off + (int64_t)n_tokens * (hidden / 32) * 4);
    L.total = align256(L.xexp_off + (int64_t)n_tokens * 4);
    return L;
}

// a kernel launch, bracketed by the profiling events when they are armed
#define PF_LAUNCH(kernel, grid, armed, e0, e1, s, src, nch, p)                                                       \
    do {                                                                                                      \
        if (armed)                                                                                            \
            hipExtLaunchKernelGGL(kernel, grid, dim3(64 * PF_WAVES), 0, s, e0, e1, 0, (const int*)p.n_tiles,   \
                                  (const int4*)p.tiles, (const int*)p.tile_dst, (const void*)(src), p.max_tiles, __builtin_ctz(nch), p); \
        else                                                                                                  \
            hipLaunchKernelGGL(kernel, grid, dim3(64 * PF_WAVES), 0, s, (const int*)p.n_tiles,                 \
                               (const int4*)p.tiles, (const int*)p.tile_dst, (const void*)(src), p.max_tiles, __builtin_ctz(nch), p); \
    } while (0)

// down row chunks per workgroup (CPW x 128 rows)
constexpr int pf_cpw_down(int hidden) { return hidden / PF_ROWS_DOWN < PF_CPW_DOWN ? hidden / PF_ROWS_DOWN : PF_CPW_DOWN; }

template <int GT, int SGT, int NBH, bool XBF16>
static void launch_p1(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    // per tile, PF_BIG_GU-chunk workgroups over all but at least PF_SMALL_GU
    // chunks, one-chunk workgroups for the rest
    constexpr int CB = PF_BIG_GU;
    const int chunks = p.inter / PF_ROWS_GU;   // 4 .. 32
    const int nbig = std::max(chunks - PF_SMALL_GU, 0) / CB, nsmall = chunks - CB * nbig;
    const dim3 grid((nbig + nsmall) * ((p.max_tiles + PF_XCDS - 1) / PF_XCDS * PF_XCDS)), block(64 * PF_WAVES);
    const unsigned mbig = pf_magic(nbig), msmall = pf_magic(nsmall);
    if (ev.armed_a())
        hipExtLaunchKernelGGL((k_prefill_gate_up<GT, SGT, NBH, XBF16, CB>), grid, block, 0, s, ev.a_start, ev.a_stop, 0,
                              (const int*)p.n_tiles, (const int4*)p.tiles, (const int*)p.tile_tok, (const void*)p.xhi,
                              p.max_tiles, nbig, nsmall, mbig, msmall, p);
    else
        hipLaunchKernelGGL((k_prefill_gate_up<GT, SGT, NBH, XBF16, CB>), grid, block, 0, s, (const int*)p.n_tiles,
                           (const int4*)p.tiles, (const int*)p.tile_tok, (const void*)p.xhi, p.max_tiles, nbig, nsmall,
                           mbig, msmall, p);
}

template <int GT, int SGT, int NBH>
static void launch_p1_i(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    if (p.x_bf16) launch_p1<GT, SGT, NBH, true>(p, s, ev);
    else launch_p1<GT, SGT, NBH, false>(p, s, ev);
}

template <int GT, int SGT>
static void launch_p1_h(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    switch (p.hidden) {
        case 256: launch_p1_i<GT, SGT, 1>(p, s, ev); break;
        case 512: launch_p1_i<GT, SGT, 2>(p, s, ev); break;
        case 1024: launch_p1_i<GT, SGT, 4>(p, s, ev); break;
        default: launch_p1_i<GT, SGT, 8>(p, s, ev); break;
    }
}

// a shared expert of another type is Q6_K (prefill_supported admits no other)
template <int GT>
static void launch_p1_t(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    if constexpr (GT != T_Q6_K) {
        if (p.has_shared && p.sh_gate_type != GT) {
            launch_p1_h<GT, T_Q6_K>(p, s, ev);
            return;
        }
    }
    launch_p1_h<GT, GT>(p, s, ev);
}

template <int DT, int SDT, int NBI, int CPW>
static void launch_p2(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    const int nch = p.hidden / (PF_ROWS_DOWN * CPW);
    const dim3 grid(pf_grid(nch, p.max_tiles));
    PF_LAUNCH((k_prefill_down<DT, SDT, NBI, CPW>), grid, ev.armed_b(), ev.b_start, ev.b_stop, s, p.act, nch, p);
}

template <int DT, int SDT, int NBI>
static void launch_p2_h(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    if (p.hidden == 256) launch_p2<DT, SDT, NBI, pf_cpw_down(256)>(p, s, ev);
    else launch_p2<DT, SDT, NBI, PF_CPW_DOWN>(p, s, ev);
}

template <int DT, int SDT>
static void launch_p2_i(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    switch (p.inter) {
        case 256: launch_p2_h<DT, SDT, 1>(p, s, ev); break;
        case 512: launch_p2_h<DT, SDT, 2>(p, s, ev); break;
        case 1024: launch_p2_h<DT, SDT, 4>(p, s, ev); break;
        default: launch_p2_h<DT, SDT, 8>(p, s, ev); break;
    }
}

template <int DT>
static void launch_p2_t(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    if constexpr (DT != T_Q6_K) {
        if (p.has_shared && p.sh_down_type != DT) {
            launch_p2_i<DT, T_Q6_K>(p, s, ev);
            return;
        }
    }
    launch_p2_i<DT, DT>(p, s, ev);
}

hipError_t launch_prefill(const PrefillParams& p, hipStream_t s, const KernelEvents& ev) {
    if (p.n_tokens <= 0) return hipSuccess;
    const dim3 route_grid(1 + (p.n_tokens + PF_STAGE_TOKENS - 1) / PF_STAGE_TOKENS);
#define MQH_ROUTE(NBH)                                                                                               \
    if (p.x_bf16) hipLaunchKernelGGL((k_prefill_route<NBH, true>), route_grid, dim3(PF_ROUTE_THREADS), 0, s, p);     \
    else hipLaunchKernelGGL((k_prefill_route<NBH, false>), route_grid, dim3(PF_ROUTE_THREADS), 0, s, p)
    switch (p.hidden) {
        case 256: MQH_ROUTE(1); break;
        case 512: MQH_ROUTE(2); break;
        case 1024: MQH_ROUTE(4); break;
        default: MQH_ROUTE(8); break;
    }
#undef MQH_ROUTE
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    switch (p.gate_type) {
        case T_Q4_K: launch_p1_t<T_Q4_K>(p, s, ev); break;
        case T_Q5_K: launch_p1_t<T_Q5_K>(p, s, ev); break;
        case T_Q6_K: launch_p1_t<T_Q6_K>(p, s, ev); break;
        default: launch_p1_t<T_Q3_K>(p, s, ev); break;
    }
    if ((err = hipGetLastError()) != hipSuccess) return err;
    switch (p.down_type) {
        case T_Q4_K: launch_p2_t<T_Q4_K>(p, s, ev); break;
        case T_Q5_K: launch_p2_t<T_Q5_K>(p, s, ev); break;
        case T_Q6_K: launch_p2_t<T_Q6_K>(p, s, ev); break;
        case T_Q8_0: launch_p2_t<T_Q8_0>(p, s, ev); break;
        default: launch_p2_t<T_Q3_K>(p, s, ev); break;
    }
    if ((err = hipGetLastError()) != hipSuccess) return err;
    hipLaunchKernelGGL(k_prefill_combine, dim3((p.hidden + 255) / 256, p.n_tokens), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace mqh
