/*
 * moe_quant_hip.h -- C ABI of the MI355X (gfx950) quantized-expert library
 * (libmoe_quant_hip.so).
 *
 * Two groups of entry points:
 *
 *  1. Drop-ins for the reference's CPU exports, same names, signatures,
 *     argument meaning and status codes.  Pointers are HOST pointers; the
 *     library stages them through HBM.  They are reentrant and may be called
 *     from several threads at once (each call uses its own stream and staging
 *     buffers).
 *
 *  2. Device-resident entry points (prefix mqh_).  Every pointer is a DEVICE
 *     address in HBM; `stream` is a hipStream_t (NULL = the null stream).
 *     They only validate arguments and enqueue kernels; they do not
 *     synchronize.  Numerical faults found by the kernels (non-finite outputs,
 *     out-of-range expert ids) are latched in the caller's workspace and
 *     reported by mqh_status().
 *
 * GGML type ids: Q8_0 = 8, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14
 * (dequant_k, moe_quant_expert); the device entry points also IQ4_NL = 20.
 * Quantized matrices are GGUF row-major: rows = output features, each row a
 * run of (cols / block_size) blocks.  A stacked expert tensor holds
 * n_experts such matrices back to back, exactly as a GGUF *_exps tensor.
 * Device-resident quantized pointers must be even addresses (every block is
 * an even number of bytes and GGUF aligns tensor data to 32 bytes); an odd
 * one is rejected with -1.
 *
 * Status codes (shared by all entry points):
 *    0  ok
 *   -1  invalid argument (null pointer, non-positive or too large size,
 *       fp16_graph not 0/1, n not a multiple of the block size)
 *   -2  unsupported type, or a column count not a multiple of its block size
 *   -3  byte count does not match rows x blocks x bytes_per_block
 *   -4  non-finite output
 *   -5  HIP runtime failure (allocation, copy or launch)
 *   -6  workspace too small
 *   -9  an expert id outside [0, n_experts)
 */
#ifndef MOE_QUANT_HIP_H
#define MOE_QUANT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* 1. Reference drop-ins (host pointers)                                     */
/* ------------------------------------------------------------------------ */

/* Replaces dequant_k_supported (cpp/dequant_k.cpp:342-344): 1 if `type` is
 * one of the five decodable GGML types, else 0. */
int dequant_k_supported(int type);

/* Replaces dequant_k_block_size (cpp/dequant_k.cpp:346-348): values per block
 * (32 for Q8_0, 256 for the K-quants), 0 for an unsupported type. */
int dequant_k_block_size(int type);

/* Replaces dequant_k (cpp/dequant_k.cpp:350-394): decode n values of `type`
 * from `src` into FP32 (want_f16 = 0) or FP16 bit patterns (want_f16 = 1) at
 * `dst`.  Bit-identical to the reference.  Returns 0, -1 (unknown type, null
 * pointer, n <= 0 or n % block_size != 0) or -5. */
int dequant_k(int type, const uint8_t* src, void* dst, int64_t n, int want_f16);

/* Replaces moe_quant_expert (cpp/moe_quant_dot.cpp:171-214): one token
 * through one SwiGLU expert straight from quantized bytes,
 *   output = W_down (silu(W_gate input) * (W_up input)),
 * gate/up shaped [intermediate x hidden], down [hidden x intermediate].
 * fp16_graph = 1 rounds to FP16 at the reference's points.  Returns 0, -1,
 * -2, -3, -4 or -5.  On -4 (non-finite output) the output rows up to and
 * including the first non-finite one are written and every later row is left
 * as the caller had it, as the reference's row loop leaves them. */
int moe_quant_expert(int gate_type, const uint8_t* gate, int64_t gate_bytes,
                     int up_type, const uint8_t* up, int64_t up_bytes,
                     int down_type, const uint8_t* down, int64_t down_bytes,
                     const float* input, int hidden, int intermediate,
                     float* output, int fp16_graph);

/* IQ4_NL to FP32, replacing the reference's IQ4_NL library
 * (cpp/fast_dequant.cpp:40-65 dequantize_iq4_nl_cpp and
 * cpp/fast_dequant_avx2.cpp:100-116 dequantize_iq4_nl_avx2, bound by
 * run_native_int4_openvino.py:35,98): rows x (cols / 32) 18-byte blocks (FP16
 * scale, 16 bytes of 4-bit indices: low nibbles give values 0..15, high
 * nibbles 16..31), value = scale * table[index] with the reference's own
 * 16-entry table; output row r at dst + r * cols, columns past the last whole
 * block untouched.  Host pointers, staged through HBM; no status, as in the
 * reference (a call it cannot run leaves dst untouched). */
void dequantize_iq4_nl_cpp(const uint8_t* src_bytes, float* dst, int rows, int cols);
void dequantize_iq4_nl_avx2(const uint8_t* src_bytes, float* dst, int rows, int cols);

/* ------------------------------------------------------------------------ */
/* 2. Device-resident entry points                                           */
/* ------------------------------------------------------------------------ */

/* Device form of dequant_k for weights already in HBM (the conversion that
 * dequant_to_f16, src/run_q4k_f16_openvino.py:62-85, performs on the host),
 * for the five types and IQ4_NL (FP16 output: RN_f16 of the FP32 value).
 * `dst` must be 16-byte aligned and `src` even.  Returns 0, -1 or -5. */
int mqh_dequant(int type, const void* src, void* dst, int64_t n, int want_f16, void* stream);

/* A resident weight form with no counterpart in the reference (GGUF has no
 * such type): Q3_K blocks byte for byte, each in a 112-byte slot whose last
 * two bytes are zero, so every block starts on a 16-byte boundary (GGUF's
 * 110-byte blocks leave most decode loads unaligned).  For resident layers
 * that are decoded often.  Only mqh_moe_decode takes it, on its fast kernels
 * (routed and shared matrices in this form, or Q6_K shared matrices beside
 * it); every other call with it returns -2 (unsupported type). */
#define MQH_TYPE_Q3_K_A112 111

/* Bytes of workspace mqh_moe_decode needs for n_tokens tokens of top_k
 * routed experts (plus one shared slot). */
int64_t mqh_moe_workspace_bytes(int n_tokens, int top_k, int intermediate, int sh_intermediate);

/* Fused MoE layer for a batch of tokens, replacing the per-expert loop of
 * run_moe_layer (src/flash_moe/moe_layer.py:39-107) over NativeExpert.forward
 * (src/flash_moe/native_expert.py:23-37) plus SharedExpert.forward
 * (src/flash_moe/shared_expert.py:221-251):
 *   y[t] = sum_s weights[t,s] * E_{ids[t,s]}(x[t]) + sigmoid(x[t].sh_gate_inp) * E_sh(x[t])
 * gate/up/down are stacked [n_experts x slice] tensors; ids and weights are
 * [n_tokens x top_k] (int32, FP32) in top-k order; x and y [n_tokens x
 * hidden] FP32.  The shared expert is optional (sh_gate == NULL: none;
 * sh_gate_inp == NULL: no sigmoid scale).  fp16_graph applies to the routed
 * experts.  Types: the five of moe_quant_expert and IQ4_NL (the latter, like
 * the FP16 graph, through the FP32 generic kernels), and MQH_TYPE_Q3_K_A112.
 * The workspace must hold mqh_moe_workspace_bytes(...) bytes and be
 * zeroed once (mqh_workspace_init) before first use.  Returns 0, -1, -2, -5
 * or -6; kernel-side faults are read with mqh_status. */
int mqh_moe_decode(int gate_type, const void* gate, int up_type, const void* up,
                   int down_type, const void* down, int n_experts, int hidden, int intermediate,
                   int sh_gate_type, const void* sh_gate, int sh_up_type, const void* sh_up,
                   int sh_down_type, const void* sh_down, int sh_intermediate,
                   const float* sh_gate_inp,
                   const float* x, int n_tokens, const int32_t* ids, const float* weights, int top_k,
                   float* y, int fp16_graph, void* workspace, int64_t workspace_bytes, void* stream);

/* Scratch bytes each GPU holds for mqh_moe_decode_noalloc (until the process
 * ends). */
#define MQH_NOALLOC_SCRATCH_BYTES (4 << 20)

/* mqh_moe_decode without a workspace: it allocates nothing (no hipMalloc,
 * hipFree or allocating library call), for callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * it.  No counterpart in the reference.  Same arguments, validation, kernels
 * and results as mqh_moe_decode; the kernels' scratch (the shared expert's
 * scale per token and the FP32 SwiGLU activations per (token, slot)) lives in
 * a library-owned device array of MQH_NOALLOC_SCRATCH_BYTES per GPU, and a
 * call that needs more (about 4 * n_tokens * (top_k + 1) * intermediate
 * bytes) returns -6.  Every call on one GPU shares that array: calls that
 * overlap on one GPU (other streams, other host threads) race, so order them
 * on one stream.  `flags`: device memory of at least 256 bytes (as a
 * workspace head: zero it once, e.g. with mqh_workspace_init(flags, 256,
 * stream)); non-finite outputs and bad expert ids latch there as in
 * mqh_moe_decode, read and cleared with mqh_status(flags, stream).
 * Returns 0, -1, -2, -5 or -6. */
int mqh_moe_decode_noalloc(int gate_type, const void* gate, int up_type, const void* up,
                           int down_type, const void* down, int n_experts, int hidden, int intermediate,
                           int sh_gate_type, const void* sh_gate, int sh_up_type, const void* sh_up,
                           int sh_down_type, const void* sh_down, int sh_intermediate,
                           const float* sh_gate_inp,
                           const float* x, int n_tokens, const int32_t* ids, const float* weights, int top_k,
                           float* y, int fp16_graph, int32_t* flags, void* stream);

/* mqh_moe_decode with the routing on the device, for tokens whose router
 * input is already in HBM (ExpertRouter.route, src/flash_moe/router.py:140-170,
 * fused into the decode prologue): router_weights [n_experts x hidden] FP32
 * (ffn_gate_inp as the GGUF file stores it, 16-byte aligned, hidden % 4 == 0);
 * scores [n_tokens x n_experts], ids and weights [n_tokens x top_k] are
 * written (the router's outputs, as mqh_route returns them), then the layer
 * runs as mqh_moe_decode on those ids and weights.  With at most 256 experts
 * and the two fast kernels (path 0), the top-k and softmax run inside the
 * gate/up kernel; otherwise (or on path 1) a select kernel of its own runs
 * first.  n_experts <=
 * 1024, 1 <= top_k <= min(64, n_experts).  Returns as mqh_moe_decode. */
int mqh_moe_decode_routed(int gate_type, const void* gate, int up_type, const void* up,
                          int down_type, const void* down, int n_experts, int hidden, int intermediate,
                          int sh_gate_type, const void* sh_gate, int sh_up_type, const void* sh_up,
                          int sh_down_type, const void* sh_down, int sh_intermediate,
                          const float* sh_gate_inp, const float* x, int n_tokens,
                          const float* router_weights, int top_k, float* scores, int32_t* ids,
                          float* weights, float* y, int fp16_graph, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* Router kernels of the calling thread's last mqh_moe_decode_routed: 1 (the
 * select step ran inside the gate/up kernel) or 2; 0 before the first.  No
 * counterpart in the reference (a profiling aid). */
int mqh_last_route_kernels(void);

/* One DeltaNet decode step for every head (replaces moe_delta_heads,
 * cpp/moe_delta.cpp:18-69, bound by NativeDelta, src/flash_moe/native_expert.py:
 * 76-97): state [heads x value_dim x key_dim] FP32 updated in place,
 * q, k [heads x key_dim], v [heads x value_dim], beta, gate [heads],
 * output [heads x value_dim].  Host pointers, same signature and codes: -1 for
 * a null pointer or heads outside 1..256, key_dim or value_dim outside
 * 1..1024; -2 when an output is not finite: as in the reference's row loop
 * (heads major, value rows minor), the state rows up to and including the
 * first such row are updated, the outputs before it written, and that row's
 * output and every later row's state and output left as the caller had them;
 * -5 on a HIP failure.  The buffers are staged through HBM: the
 * PCIe-inclusive compatibility path. */
int moe_delta_heads(float* state, const float* q, const float* k, const float* v, const float* beta,
                    const float* gate, float* output, int heads, int key_dim, int value_dim);

/* moe_delta_heads on device pointers, enqueued on `stream`: the state stays
 * resident in HBM across steps.  workspace (optional, zeroed once with
 * mqh_workspace_init): a non-finite output latches, and mqh_status then
 * returns -4.  Returns 0, -1 or -5. */
int mqh_delta_heads(float* state, const float* q, const float* k, const float* v, const float* beta,
                    const float* gate, float* output, int heads, int key_dim, int value_dim, void* workspace,
                    void* stream);

/* Bytes of workspace mqh_moe_prefill needs (has_shared: 0 or 1). */
int64_t mqh_moe_prefill_workspace_bytes(int n_tokens, int top_k, int n_experts, int hidden, int intermediate,
                                        int has_shared);

/* Grouped-GEMM MoE layer for a prompt, replacing run_moe_sequence
 * (src/flash_moe/moe_layer.py:110-195): the expert-by-expert batched forward of
 * the routed experts (backend_ov.py:210-237, 407-431, or NativeExpert.forward
 * per token) and the batched shared expert (src/flash_moe/shared_expert.py:200-219):
 *   y[t] = sum_s weights[t,s] * E_{ids[t,s]}(x[t]) + sigmoid(x[t].sh_gate_inp) * E_sh(x[t])
 * Same tensors and ids/weights as mqh_moe_decode; x is [n_tokens x hidden],
 * FP32 (x_bf16 = 0) or BF16 (x_bf16 = 1), 16-byte aligned; y FP32.  The shared
 * expert (optional, sh_gate == NULL: none) runs in the same grouped launches:
 * its intermediate size is the routed one (sh_intermediate == intermediate,
 * else -1), its gate/up type the routed gate/up type or Q6_K, its down type
 * the routed down type or Q6_K (the reference model's layers: Q6_K shared
 * experts beside Q3_K, Q4_K or Q8_0 routed matrices).  Tokens are bucketed per
 * expert on the device; weights are multiplied as exact integer MFMA operands
 * with FP32 accumulation.  Supported: gate == up type in Q3_K/Q4_K/Q5_K/Q6_K,
 * down type in Q3_K/Q4_K/Q5_K/Q6_K/Q8_0, hidden and intermediate in
 * {256, 512, 1024, 2048}, at most 1024 experts; else -2.  The workspace
 * (256-byte aligned, mqh_moe_prefill_workspace_bytes(...)) is zeroed once with
 * mqh_workspace_init.  Returns 0, -1, -2, -5 or -6; mqh_status reads -4 / -9. */
int mqh_moe_prefill(int gate_type, const void* gate, int up_type, const void* up,
                    int down_type, const void* down, int n_experts, int hidden, int intermediate,
                    int sh_gate_type, const void* sh_gate, int sh_up_type, const void* sh_up,
                    int sh_down_type, const void* sh_down, int sh_intermediate, const float* sh_gate_inp,
                    const void* x, int x_bf16, int n_tokens, const int32_t* ids, const float* weights,
                    int top_k, float* y, void* workspace, int64_t workspace_bytes, void* stream);

/* Select the kernels behind mqh_moe_decode and moe_quant_expert: 0 (default)
 * = the two integer-digit fast kernels (gate/up + SwiGLU, then down +
 * combine) whenever the shapes and types allow it (FP32 graph, K-quant or
 * Q8_0 types, hidden and intermediate in 256..2048), else the generic
 * kernels; 1 = always the generic kernels.  Process-wide; returns the
 * previous setting, or -1 for another value. */
int mqh_set_decode_path(int path);

/* Number of kernels (2) the calling thread's last mqh_moe_decode or
 * moe_quant_expert launched; 0 before the first.  No counterpart in the
 * reference (a profiling aid). */
int mqh_last_decode_kernels(void);

/* The kernels the calling thread's last mqh_moe_decode, mqh_moe_decode_routed,
 * mqh_moe_decode_noalloc or moe_quant_expert ran on: 0 the two integer-digit
 * fast kernels, 1 the generic kernels (forced by mqh_set_decode_path(1), or a
 * type, shape or slot count the fast kernels do not take); -1 before the
 * first.  No counterpart in the reference (a test and profiling aid). */
int mqh_last_decode_path(void);

/* Top-k routing of n_tokens tokens on `stream` (replaces ExpertRouter.route,
 * src/flash_moe/router.py:140-170).  All pointers are device memory:
 *   x            [n_tokens x hidden] FP32
 *   gate_weights [n_experts x hidden] FP32: ffn_gate_inp as the GGUF file
 *                stores it (the transpose of the reference's gate_weights)
 *   scores       [n_tokens x n_experts] FP32 out: x . W, summed in FP32
 *   ids          [n_tokens x top_k] int32 out, descending score order
 *   weights      [n_tokens x top_k] FP32 out: the float64 softmax over the
 *                selected scores (1/top_k each when its sum is not finite
 *                and positive), rounded to FP32.
 * NaN scores rank above every number (np.argsort puts NaN last); equal scores,
 * and NaNs, go in ascending expert order.  hidden % 4 == 0, x and
 * gate_weights 16-byte aligned, n_experts <= 1024,
 * 1 <= top_k <= min(64, n_experts).  Returns 0, -1 or -5. */
int mqh_route(const float* x, int n_tokens, int hidden, const float* gate_weights, int n_experts, int top_k,
              float* scores, int32_t* ids, float* weights, void* stream);

/* Read `bytes` (a multiple of 16) at `src` (device memory, 16-byte aligned)
 * once with a plain streaming kernel on `stream`, between the optional HIP
 * events start_event / stop_event (recorded at the kernel's own start and
 * end).  Timed on the same byte count as a decode or prefill kernel it gives
 * the read time this GPU achieves for a launch of that size.  `sink` (may be
 * NULL) is a device word the kernel practically never writes.  No
 * counterpart in the reference (a measurement aid).  Returns 0, -1 or -5. */
int mqh_read_floor(const void* src, int64_t bytes, void* sink, void* start_event, void* stop_event, void* stream);

/* Profiling: record HIP events (hipEvent_t, any may be NULL) at the start and
 * end of the two GEMM kernels of the calling thread's next mqh_moe_decode,
 * moe_quant_expert or mqh_moe_prefill -- A: gate/up and SwiGLU, B: down
 * projection (with the weighted combine in decode) -- or of the one kernel of
 * its next mqh_delta_heads (A; B is not recorded).
 * One-shot; the launch itself is unchanged.  No counterpart in the reference
 * (its timers are host wall clocks, bench_phases.py:45-56). */
int mqh_profile_next_decode(void* a_start, void* a_stop, void* b_start, void* b_stop);

/* Zero a workspace's flag words on `stream` (once, before first use). */
int mqh_workspace_init(void* workspace, int64_t workspace_bytes, void* stream);

/* Synchronize `stream`, then read and clear the fault flags latched in
 * `workspace`: 0, -4 (non-finite output), -9 (bad expert id) or -5. */
int mqh_status(void* workspace, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_QUANT_HIP_H */
