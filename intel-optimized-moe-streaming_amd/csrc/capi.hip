// capi.hip -- the library's C ABI (declared in include/moe_quant_hip.h).
//
// Host-pointer drop-ins stage their buffers through HBM with a pooled staging
// context per concurrent call; device-resident entry points validate and
// enqueue only.
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/moe_quant_hip.h"
#include "kquant_device.h"
#include "moe_decode.h"

using namespace mqh;

namespace {

constexpr int ST_OK = 0, ST_ARG = -1, ST_TYPE = -2, ST_BYTES = -3, ST_NONFINITE = -4, ST_HIP = -5,
              ST_WORKSPACE = -6, ST_BAD_ID = -9;

// dequant_k and moe_quant_expert accept the reference's five types; the
// device entry points also IQ4_NL
bool supported(int t) { return reference_type(t); }
bool device_supported(int t) { return reference_type(t) || t == T_IQ4_NL; }

// 0: the two integer-digit kernels when the shapes allow them, else the
// generic kernels; 1: always the generic kernels
int g_decode_path = 0;

// events armed by mqh_profile_next_decode for this thread's next decode, and
// the number of kernels this thread's last decode launched
thread_local KernelEvents t_events;
thread_local int t_last_kernels = 0;
// kernels this thread's last decode ran on: 0 the fast kernels, 1 the
// generic ones, -1 before the first
thread_local int t_last_path = -1;
// router kernels of this thread's last routed decode (1: the select step ran
// inside the gate/up kernel, 2: a select kernel of its own)
thread_local int t_last_route_kernels = 0;

hipError_t launch_decode(const DecodeParams& p, hipStream_t s) {
    const KernelEvents ev = t_events;
    t_events = KernelEvents();
    t_last_kernels = 2;
    if (g_decode_path != 1 && fast_supported(p)) {
        t_last_path = 0;
        return launch_decode_fast(p, s, ev);
    }
    t_last_path = 1;
    return launch_decode_generic(p, s, ev);
}

// words to zero in a fresh workspace: the flags
constexpr int64_t WS_INIT_WORDS = WS_HEAD_BYTES / 4;

// Expected bytes of a [rows x cols] matrix, or a negative status.
int64_t matrix_bytes(int type, int rows, int cols) {
    const int bs = block_size(type);
    if (!bs || cols % bs) return ST_TYPE;
    return (int64_t)rows * (cols / bs) * block_bytes(type);
}

__global__ void k_zero_words(int* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

hipError_t zero_words(void* p, int64_t n_words, hipStream_t s) {
    if (n_words <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n_words + 255) / 256, 1024);
    hipLaunchKernelGGL(k_zero_words, dim3((unsigned)blocks), dim3(256), 0, s, (int*)p, n_words);
    return hipGetLastError();
}

// Device buffer that grows on demand (never shrinks).
struct DevBuf {
    void* ptr = nullptr;
    size_t cap = 0;
    hipError_t reserve(size_t n) {
        if (n <= cap) return hipSuccess;
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        cap = 0;
        const size_t want = (n + 4095) & ~(size_t)4095;
        hipError_t e = hipMalloc(&ptr, want);
        if (e == hipSuccess) cap = want;
        return e;
    }
};

// Staging for one in-flight host-pointer call.  Pooled, so threads that come
// and go (the reference runs experts on a ThreadPoolExecutor) reuse them.
struct Ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    DevBuf w, io, ws;
};

std::mutex g_pool_mu;
std::vector<Ctx*> g_pool;

Ctx* acquire_ctx(int& status) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { status = ST_HIP; return nullptr; }
    {
        std::lock_guard<std::mutex> lk(g_pool_mu);
        for (size_t i = 0; i < g_pool.size(); ++i) {
            if (g_pool[i]->device == dev) {
                Ctx* c = g_pool[i];
                g_pool.erase(g_pool.begin() + (long)i);
                return c;
            }
        }
    }
    Ctx* c = new Ctx();
    c->device = dev;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        status = ST_HIP;
        return nullptr;
    }
    return c;
}

void release_ctx(Ctx* c) {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    g_pool.push_back(c);
}

int read_and_clear_flags(int* flags_dev, hipStream_t s) {
    int h[2] = {0, 0};   // FLAG_NONFINITE, FLAG_BAD_ID
    if (hipStreamSynchronize(s) != hipSuccess) return ST_HIP;
    if (hipMemcpyAsync(h, flags_dev, sizeof(h), hipMemcpyDeviceToHost, s) != hipSuccess) return ST_HIP;
    if (hipStreamSynchronize(s) != hipSuccess) return ST_HIP;
    if (h[0] | h[1]) {
        if (zero_words(flags_dev, 2, s) != hipSuccess) return ST_HIP;
        if (hipStreamSynchronize(s) != hipSuccess) return ST_HIP;
    }
    if (h[FLAG_BAD_ID]) return ST_BAD_ID;
    if (h[FLAG_NONFINITE]) return ST_NONFINITE;
    return ST_OK;
}

// Validate shapes and types of one expert triple.  Returns 0 or a status.
int check_expert_types(int gt, int ut, int dt, int hidden, int inter, bool device = false) {
    if (device ? !(device_supported(gt) && device_supported(ut) && device_supported(dt))
               : !(supported(gt) && supported(ut) && supported(dt)))
        return ST_TYPE;
    if (hidden % block_size(gt) || hidden % block_size(ut) || inter % block_size(dt)) return ST_TYPE;
    return ST_OK;
}

// Quantized weights must start at an even address: every block is an even
// number of bytes, so each block then starts 0 or 2 bytes past a dword, the
// two cases the Q3_K header load of the decoders handles.
bool odd(const void* p) { return ((uintptr_t)p & 1) != 0; }

}  // namespace

// ------------------------------------------------- decode without allocation
//
// The scratch memory of mqh_moe_decode_noalloc: a file-scope device array, one
// copy per GPU at that GPU's own address, held until the process ends.  Every
// call on a GPU shares it (overlapping calls on one GPU race).  In host code
// the name `scratch` is a host-side stand-in, not a device address: host code
// only ever uses the address hipGetSymbolAddress returns with the device
// current, looked up on the entry point's first call on each device.
static __device__ __align__(256) uint8_t scratch[MQH_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int64_t NOALLOC_SCRATCH_BYTES = MQH_NOALLOC_SCRATCH_BYTES;
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[MAX_DEVICES] = {};

// Device address of `scratch` on the current device, or nullptr.
void* scratch_address() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        g_scratch_addr[dev] = ptr;
    }
    return g_scratch_addr[dev];
}

}  // namespace

extern "C" {

int dequant_k_supported(int type) { return supported(type) ? 1 : 0; }

int dequant_k_block_size(int type) { return supported(type) ? block_size(type) : 0; }

int dequant_k(int type, const uint8_t* src, void* dst, int64_t n, int want_f16) {
    const int bs = supported(type) ? block_size(type) : 0;
    if (bs == 0 || src == nullptr || dst == nullptr) return ST_ARG;
    if (n <= 0 || n % bs != 0) return ST_ARG;
    int status = ST_OK;
    Ctx* c = acquire_ctx(status);
    if (!c) return status;
    const size_t in_bytes = (size_t)(n / bs) * block_bytes(type);
    const size_t out_bytes = (size_t)n * (want_f16 ? 2 : 4);
    status = ST_HIP;
    if (c->w.reserve(in_bytes) == hipSuccess && c->io.reserve(out_bytes) == hipSuccess &&
        hipMemcpyAsync(c->w.ptr, src, in_bytes, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
        launch_dequant(type, (const uint8_t*)c->w.ptr, c->io.ptr, n, want_f16, c->stream) == hipSuccess &&
        hipMemcpyAsync(dst, c->io.ptr, out_bytes, hipMemcpyDeviceToHost, c->stream) == hipSuccess &&
        hipStreamSynchronize(c->stream) == hipSuccess)
        status = ST_OK;
    release_ctx(c);
    return status;
}

int moe_quant_expert(int gate_type, const uint8_t* gate, int64_t gate_bytes, int up_type, const uint8_t* up,
                     int64_t up_bytes, int down_type, const uint8_t* down, int64_t down_bytes, const float* input,
                     int hidden, int intermediate, float* output, int fp16_graph) {
    // validation order and codes of moe_quant_dot.cpp:177-188
    if (!gate || !up || !down || !input || !output || hidden <= 0 || intermediate <= 0 || hidden > 65536 ||
        intermediate > 65536 || (fp16_graph != 0 && fp16_graph != 1))
        return ST_ARG;
    const int types[3] = {gate_type, up_type, down_type};
    const int cols[3] = {hidden, hidden, intermediate};
    const int rows[3] = {intermediate, intermediate, hidden};
    const int64_t sizes[3] = {gate_bytes, up_bytes, down_bytes};
    for (int i = 0; i < 3; ++i) {
        const int64_t want = matrix_bytes(types[i], rows[i], cols[i]);
        if (want < 0) return (int)want;
        if (sizes[i] != want) return ST_BYTES;
    }
    int status = ST_OK;
    Ctx* c = acquire_ctx(status);
    if (!c) return status;

    const int64_t off_up = align256(gate_bytes), off_down = off_up + align256(up_bytes);
    const int64_t w_total = off_down + align256(down_bytes);
    // io: x [hidden] | y [hidden] | id | weight
    const int64_t off_y = align256((int64_t)hidden * 4), off_id = off_y + align256((int64_t)hidden * 4);
    const int64_t io_total = off_id + 256;
    const WorkspaceLayout wl = decode_workspace_layout(1, 1, intermediate, 0);
    const bool fresh_ws = c->ws.cap < (size_t)wl.total;

    status = ST_HIP;
    if (c->w.reserve(w_total) != hipSuccess || c->io.reserve(io_total) != hipSuccess ||
        c->ws.reserve(wl.total) != hipSuccess) {
        release_ctx(c);
        return ST_HIP;
    }
    uint8_t* W = (uint8_t*)c->w.ptr;
    uint8_t* IO = (uint8_t*)c->io.ptr;
    uint8_t* WS = (uint8_t*)c->ws.ptr;
    struct { int32_t id; float w; } route = {0, 1.0f};

    DecodeParams p{};
    p.gate = W; p.up = W + off_up; p.down = W + off_down;
    p.gate_type = gate_type; p.up_type = up_type; p.down_type = down_type;
    p.gate_eb = gate_bytes; p.up_eb = up_bytes; p.down_eb = down_bytes;
    p.n_experts = 1; p.hidden = hidden; p.inter = intermediate;
    p.has_shared = 0;
    p.x = (const float*)IO; p.n_tokens = 1;
    p.ids = (const int32_t*)(IO + off_id); p.weights = (const float*)(IO + off_id + 4); p.top_k = 1;
    p.y = (float*)(IO + off_y); p.fp16 = fp16_graph;
    p.flags = (int*)(WS + wl.flags_off);
    p.sh_scale = (float*)(WS + wl.scale_off); p.act = (float*)(WS + wl.act_off);
    p.S = 1; p.Imax = intermediate;

    // The rows come back into a host copy first: the reference writes output
    // rows in order and returns -4 at the first non-finite one, leaving every
    // later row as the caller had it (moe_quant_dot.cpp:207-211).
    std::vector<float> y(hidden);
    if ((!fresh_ws || zero_words(WS, WS_INIT_WORDS, c->stream) == hipSuccess) &&
        hipMemcpyAsync(W, gate, gate_bytes, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
        hipMemcpyAsync(W + off_up, up, up_bytes, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
        hipMemcpyAsync(W + off_down, down, down_bytes, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
        hipMemcpyAsync(IO, input, (size_t)hidden * 4, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
        hipMemcpyAsync(IO + off_id, &route, sizeof(route), hipMemcpyHostToDevice, c->stream) == hipSuccess &&
        launch_decode(p, c->stream) == hipSuccess &&
        hipMemcpyAsync(y.data(), IO + off_y, (size_t)hidden * 4, hipMemcpyDeviceToHost, c->stream) == hipSuccess)
        status = read_and_clear_flags(p.flags, c->stream);
    release_ctx(c);
    if (status == ST_OK || status == ST_NONFINITE) {
        int bad = -1;   // the first non-finite row
        for (int r = 0; r < hidden && bad < 0; ++r)
            if (!std::isfinite(y[r])) bad = r;
        std::memcpy(output, y.data(), (size_t)(bad < 0 ? hidden : bad + 1) * 4);
        status = bad < 0 ? ST_OK : ST_NONFINITE;
    }
    return status;
}

int moe_delta_heads(float* state, const float* q, const float* k, const float* v, const float* beta,
                    const float* gate, float* output, int heads, int key_dim, int value_dim) {
    // validation of moe_delta.cpp:21-24
    if (!state || !q || !k || !v || !beta || !gate || !output || heads < 1 || heads > 256 || key_dim < 1 ||
        key_dim > 1024 || value_dim < 1 || value_dim > 1024)
        return ST_ARG;
    int status = ST_OK;
    Ctx* c = acquire_ctx(status);
    if (!c) return status;
    // io: state | q | k | v | beta | gate | output | flags
    const int64_t n_state = (int64_t)heads * value_dim * key_dim, n_qk = (int64_t)heads * key_dim;
    const int64_t n_v = (int64_t)heads * value_dim;
    const int64_t o_q = align256(n_state * 4), o_k = o_q + align256(n_qk * 4), o_v = o_k + align256(n_qk * 4);
    const int64_t o_b = o_v + align256(n_v * 4), o_g = o_b + align256((int64_t)heads * 4);
    const int64_t o_out = o_g + align256((int64_t)heads * 4), o_fl = o_out + align256(n_v * 4);
    const int64_t total = o_fl + 256;
    if (c->io.reserve(total) != hipSuccess) {
        release_ctx(c);
        return ST_HIP;
    }
    uint8_t* IO = (uint8_t*)c->io.ptr;
    float* S = (float*)IO;
    int* fl = (int*)(IO + o_fl);
    const hipStream_t s = c->stream;
    // The reference walks the rows (head-major, value row minor) and returns -2
    // at the first row whose output is not finite: that row's state is already
    // updated, its output is not written, and no later row's state or output
    // changes (moe_delta.cpp:30-66).  The outputs come back first so the host
    // knows how many rows to hand back.
    std::vector<float> out(n_v);
    status = ST_HIP;
    if (zero_words(fl, 3, s) == hipSuccess &&
        hipMemcpyAsync(S, state, n_state * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
        hipMemcpyAsync(IO + o_q, q, n_qk * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
        hipMemcpyAsync(IO + o_k, k, n_qk * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
        hipMemcpyAsync(IO + o_v, v, n_v * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
        hipMemcpyAsync(IO + o_b, beta, (size_t)heads * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
        hipMemcpyAsync(IO + o_g, gate, (size_t)heads * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
        launch_delta_heads(S, (const float*)(IO + o_q), (const float*)(IO + o_k), (const float*)(IO + o_v),
                           (const float*)(IO + o_b), (const float*)(IO + o_g), (float*)(IO + o_out), heads,
                           key_dim, value_dim, fl, s, KernelEvents()) == hipSuccess &&
        hipMemcpyAsync(out.data(), IO + o_out, n_v * 4, hipMemcpyDeviceToHost, s) == hipSuccess) {
        status = read_and_clear_flags(fl, s);
        if (status == ST_OK || status == ST_NONFINITE) {
            int64_t rows = n_v;   // the first non-finite row, or all of them
            for (int64_t r = 0; r < n_v; ++r)
                if (!std::isfinite(out[r])) { rows = r; break; }
            // state rows 0 .. rows (inclusive when a row failed), outputs 0 .. rows - 1
            const int64_t state_rows = rows < n_v ? rows + 1 : n_v;
            if (hipMemcpyAsync(state, S, state_rows * key_dim * 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess) {
                status = ST_HIP;
            } else {
                std::memcpy(output, out.data(), (size_t)rows * 4);
                status = rows < n_v ? -2 : ST_OK;   // moe_delta.cpp:65
            }
        }
    }
    release_ctx(c);
    return status;
}

int mqh_delta_heads(float* state, const float* q, const float* k, const float* v, const float* beta,
                    const float* gate, float* output, int heads, int key_dim, int value_dim, void* workspace,
                    void* stream) {
    if (!state || !q || !k || !v || !beta || !gate || !output || heads < 1 || heads > 256 || key_dim < 1 ||
        key_dim > 1024 || value_dim < 1 || value_dim > 1024)
        return ST_ARG;
    int* flags = workspace ? (int*)workspace : nullptr;   // the flag words lead every workspace
    const KernelEvents ev = t_events;
    t_events = KernelEvents();
    return launch_delta_heads(state, q, k, v, beta, gate, output, heads, key_dim, value_dim, flags,
                              (hipStream_t)stream, ev) == hipSuccess
               ? ST_OK
               : ST_HIP;
}

void dequantize_iq4_nl_cpp(const uint8_t* src_bytes, float* dst, int rows, int cols) {
    // fast_dequant.cpp:40-65: rows x (cols / 32) blocks, row r of the output at
    // dst + r * cols; no status (a call it cannot run leaves dst untouched)
    if (!src_bytes || !dst || rows <= 0 || cols < 32) return;
    const int bpr = cols / 32;
    const int64_t n = (int64_t)rows * bpr * 32;
    int status = ST_OK;
    Ctx* c = acquire_ctx(status);
    if (!c) return;
    const size_t in_bytes = (size_t)rows * bpr * 18;
    if (c->w.reserve(in_bytes) == hipSuccess && c->io.reserve((size_t)n * 4) == hipSuccess &&
        hipMemcpyAsync(c->w.ptr, src_bytes, in_bytes, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
        launch_dequant(T_IQ4_NL, (const uint8_t*)c->w.ptr, c->io.ptr, n, 0, c->stream) == hipSuccess) {
        // rows land cols floats apart; the columns past bpr * 32 stay as they were
        if (cols % 32 == 0)
            (void)hipMemcpyAsync(dst, c->io.ptr, (size_t)n * 4, hipMemcpyDeviceToHost, c->stream);
        else
            (void)hipMemcpy2DAsync(dst, (size_t)cols * 4, c->io.ptr, (size_t)bpr * 128, (size_t)bpr * 128,
                                   (size_t)rows, hipMemcpyDeviceToHost, c->stream);
        (void)hipStreamSynchronize(c->stream);
    }
    release_ctx(c);
}

void dequantize_iq4_nl_avx2(const uint8_t* src_bytes, float* dst, int rows, int cols) {
    // fast_dequant_avx2.cpp:100-116 computes the same values as the scalar export
    dequantize_iq4_nl_cpp(src_bytes, dst, rows, cols);
}

int mqh_dequant(int type, const void* src, void* dst, int64_t n, int want_f16, void* stream) {
    const int bs = device_supported(type) ? block_size(type) : 0;
    if (bs == 0 || src == nullptr || dst == nullptr) return ST_ARG;
    if (n <= 0 || n % bs != 0 || ((uintptr_t)dst & 15) || odd(src)) return ST_ARG;
    return launch_dequant(type, (const uint8_t*)src, dst, n, want_f16, (hipStream_t)stream) == hipSuccess ? ST_OK
                                                                                                      : ST_HIP;
}

int64_t mqh_moe_workspace_bytes(int n_tokens, int top_k, int intermediate, int sh_intermediate) {
    if (n_tokens <= 0 || top_k < 0 || intermediate < 0 || sh_intermediate < 0) return ST_ARG;
    if ((top_k > 0 && intermediate == 0) || (top_k == 0 && sh_intermediate == 0)) return ST_ARG;
    return decode_workspace_layout(n_tokens, top_k, intermediate, sh_intermediate).total;
}

int mqh_workspace_init(void* workspace, int64_t workspace_bytes, void* stream) {
    if (!workspace || workspace_bytes < WS_HEAD_BYTES) return ST_ARG;
    return zero_words(workspace, WS_INIT_WORDS, (hipStream_t)stream) == hipSuccess ? ST_OK : ST_HIP;
}

int mqh_status(void* workspace, void* stream) {
    if (!workspace) return ST_ARG;
    return read_and_clear_flags((int*)workspace, (hipStream_t)stream);
}

}  // extern "C" (reopened below)

namespace {

// Validate the arguments of a decode call and fill p (ids/weights may be
// outputs of the routed call).  Returns a status.
int decode_params(int gate_type, const void* gate, int up_type, const void* up, int down_type, const void* down,
                  int n_experts, int hidden, int intermediate, int sh_gate_type, const void* sh_gate, int sh_up_type,
                  const void* sh_up, int sh_down_type, const void* sh_down, int sh_intermediate,
                  const float* sh_gate_inp, const float* x, int n_tokens, const int32_t* ids, const float* weights,
                  int top_k, float* y, int fp16_graph, void* workspace, int64_t workspace_bytes, DecodeParams& p,
                  bool a112 = false) {
    const bool has_shared = sh_gate != nullptr;
    // the 112-byte Q3_K resident form: validated as Q3_K; only the fast decode
    // kernels read it (checked once the call's parameters are known)
    if (a112) {
        auto base = [](int t) { return t == T_Q3_K_A112 ? (int)T_Q3_K : t; };
        if (top_k > 0 && !(gate_type == T_Q3_K_A112) + !(up_type == T_Q3_K_A112) + !(down_type == T_Q3_K_A112) < 3) {
            const int st = check_expert_types(base(gate_type), base(up_type), base(down_type), hidden, intermediate, true);
            if (st) return st;
        }
        if (has_shared && !(sh_gate_type == T_Q3_K_A112) + !(sh_up_type == T_Q3_K_A112) + !(sh_down_type == T_Q3_K_A112) < 3) {
            const int st = check_expert_types(base(sh_gate_type), base(sh_up_type), base(sh_down_type), hidden,
                                              sh_intermediate > 0 ? sh_intermediate : 256, true);
            if (st) return st;
        }
    }
    auto dev_ok = [a112](int t) { return a112 && t == T_Q3_K_A112; };
    if (!x || !y || !workspace) return ST_ARG;
    if (hidden <= 0 || hidden > 65536 || n_tokens <= 0 || top_k < 0 || top_k > 64 ||
        (top_k == 0 && !has_shared) || (fp16_graph != 0 && fp16_graph != 1))
        return ST_ARG;
    int st = ST_OK;
    if (top_k > 0) {
        if (!gate || !up || !down || !ids || !weights) return ST_ARG;
        if (odd(gate) || odd(up) || odd(down)) return ST_ARG;
        if (n_experts <= 0 || intermediate <= 0 || intermediate > 65536) return ST_ARG;
        if (!(dev_ok(gate_type) || dev_ok(up_type) || dev_ok(down_type)))
            st = check_expert_types(gate_type, up_type, down_type, hidden, intermediate, true);
        if (st) return st;
    } else {
        intermediate = 0;
    }
    if (has_shared) {
        if (!sh_up || !sh_down || sh_intermediate <= 0 || sh_intermediate > 65536) return ST_ARG;
        if (odd(sh_gate) || odd(sh_up) || odd(sh_down)) return ST_ARG;
        if (!(dev_ok(sh_gate_type) || dev_ok(sh_up_type) || dev_ok(sh_down_type)))
            st = check_expert_types(sh_gate_type, sh_up_type, sh_down_type, hidden, sh_intermediate, true);
        if (st) return st;
    }
    const WorkspaceLayout wl = decode_workspace_layout(n_tokens, top_k, intermediate, has_shared ? sh_intermediate : 0);
    if (workspace_bytes < wl.total) return ST_WORKSPACE;

    uint8_t* WS = (uint8_t*)workspace;
    p = DecodeParams{};
    p.gate = (const uint8_t*)gate; p.up = (const uint8_t*)up; p.down = (const uint8_t*)down;
    p.gate_type = gate_type; p.up_type = up_type; p.down_type = down_type;
    if (top_k > 0) {
        p.gate_eb = matrix_bytes(gate_type, intermediate, hidden);
        p.up_eb = matrix_bytes(up_type, intermediate, hidden);
        p.down_eb = matrix_bytes(down_type, hidden, intermediate);
    }
    p.n_experts = n_experts; p.hidden = hidden; p.inter = intermediate;
    p.has_shared = has_shared ? 1 : 0;
    if (has_shared) {
        p.sh_gate = (const uint8_t*)sh_gate; p.sh_up = (const uint8_t*)sh_up; p.sh_down = (const uint8_t*)sh_down;
        p.sh_gate_type = sh_gate_type; p.sh_up_type = sh_up_type; p.sh_down_type = sh_down_type;
        p.sh_inter = sh_intermediate; p.sh_gate_inp = sh_gate_inp;
    }
    p.x = x; p.n_tokens = n_tokens; p.ids = ids; p.weights = weights; p.top_k = top_k;
    p.y = y; p.fp16 = fp16_graph;
    p.flags = (int*)(WS + wl.flags_off);
    p.sh_scale = (float*)(WS + wl.scale_off); p.act = (float*)(WS + wl.act_off);
    p.S = top_k + (has_shared ? 1 : 0);
    p.Imax = std::max(intermediate, has_shared ? sh_intermediate : 0);
    return ST_OK;
}

}  // namespace

extern "C" {

int mqh_moe_decode(int gate_type, const void* gate, int up_type, const void* up, int down_type, const void* down,
                   int n_experts, int hidden, int intermediate, int sh_gate_type, const void* sh_gate,
                   int sh_up_type, const void* sh_up, int sh_down_type, const void* sh_down, int sh_intermediate,
                   const float* sh_gate_inp, const float* x, int n_tokens, const int32_t* ids, const float* weights,
                   int top_k, float* y, int fp16_graph, void* workspace, int64_t workspace_bytes, void* stream) {
    DecodeParams p;
    const int st = decode_params(gate_type, gate, up_type, up, down_type, down, n_experts, hidden, intermediate,
                                 sh_gate_type, sh_gate, sh_up_type, sh_up, sh_down_type, sh_down, sh_intermediate,
                                 sh_gate_inp, x, n_tokens, ids, weights, top_k, y, fp16_graph, workspace,
                                 workspace_bytes, p, true);
    if (st) return st;
    // the 112-byte Q3_K form runs on the fast kernels only
    const auto a = [&](int t) { return t == T_Q3_K_A112; };
    const bool uses_a112 = (p.top_k > 0 && (a(p.gate_type) || a(p.up_type) || a(p.down_type))) ||
                           (p.has_shared && (a(p.sh_gate_type) || a(p.sh_up_type) || a(p.sh_down_type)));
    if (uses_a112 && (g_decode_path == 1 || !fast_supported(p))) return ST_TYPE;
    return launch_decode(p, (hipStream_t)stream) == hipSuccess ? ST_OK : ST_HIP;
}

int mqh_moe_decode_noalloc(int gate_type, const void* gate, int up_type, const void* up, int down_type,
                           const void* down, int n_experts, int hidden, int intermediate, int sh_gate_type,
                           const void* sh_gate, int sh_up_type, const void* sh_up, int sh_down_type,
                           const void* sh_down, int sh_intermediate, const float* sh_gate_inp, const float* x,
                           int n_tokens, const int32_t* ids, const float* weights, int top_k, float* y,
                           int fp16_graph, int32_t* flags, void* stream) {
    if (!flags) return ST_ARG;
    void* ws = scratch_address();
    if (!ws) return ST_HIP;
    // the same validation and kernels as mqh_moe_decode, on the scratch array
    // (-6 when the call needs more than MQH_NOALLOC_SCRATCH_BYTES); the fault
    // flags go to the caller's words instead of the scratch's own head
    DecodeParams p;
    const int st = decode_params(gate_type, gate, up_type, up, down_type, down, n_experts, hidden, intermediate,
                                 sh_gate_type, sh_gate, sh_up_type, sh_up, sh_down_type, sh_down, sh_intermediate,
                                 sh_gate_inp, x, n_tokens, ids, weights, top_k, y, fp16_graph, ws,
                                 NOALLOC_SCRATCH_BYTES, p);
    if (st) return st;
    p.flags = (int*)flags;
    return launch_decode(p, (hipStream_t)stream) == hipSuccess ? ST_OK : ST_HIP;
}

int mqh_moe_decode_routed(int gate_type, const void* gate, int up_type, const void* up, int down_type,
                          const void* down, int n_experts, int hidden, int intermediate, int sh_gate_type,
                          const void* sh_gate, int sh_up_type, const void* sh_up, int sh_down_type,
                          const void* sh_down, int sh_intermediate, const float* sh_gate_inp, const float* x,
                          int n_tokens, const float* router_weights, int top_k, float* scores, int32_t* ids,
                          float* weights, float* y, int fp16_graph, void* workspace, int64_t workspace_bytes,
                          void* stream) {
    if (!router_weights || !scores || !ids || !weights || top_k < 1 || n_experts > 1024 || top_k > n_experts ||
        hidden % 4 || ((uintptr_t)x | (uintptr_t)router_weights) % 16)
        return ST_ARG;
    DecodeParams p;
    const int st = decode_params(gate_type, gate, up_type, up, down_type, down, n_experts, hidden, intermediate,
                                 sh_gate_type, sh_gate, sh_up_type, sh_up, sh_down_type, sh_down, sh_intermediate,
                                 sh_gate_inp, x, n_tokens, ids, weights, top_k, y, fp16_graph, workspace,
                                 workspace_bytes, p);
    if (st) return st;
    const hipStream_t s = (hipStream_t)stream;
    if (launch_route_scores(x, n_tokens, hidden, router_weights, n_experts, scores, s) != hipSuccess) return ST_HIP;
    if (g_decode_path == 0 && n_experts <= ROUTE_PROLOGUE_MAX_EXPERTS && fast_supported(p)) {
        // the select step inside the gate/up kernel; the two-kernel fast path
        p.route_scores = scores; p.route_ids = ids; p.route_weights = weights;
        const KernelEvents ev = t_events;
        t_events = KernelEvents();
        t_last_kernels = 2;
        t_last_path = 0;
        t_last_route_kernels = 1;
        return launch_decode_fast(p, s, ev) == hipSuccess ? ST_OK : ST_HIP;
    }
    if (launch_route_select(scores, n_tokens, n_experts, top_k, ids, weights, s) != hipSuccess) return ST_HIP;
    t_last_route_kernels = 2;
    return launch_decode(p, s) == hipSuccess ? ST_OK : ST_HIP;
}

int mqh_last_route_kernels(void) { return t_last_route_kernels; }

int64_t mqh_moe_prefill_workspace_bytes(int n_tokens, int top_k, int n_experts, int hidden, int intermediate,
                                        int has_shared) {
    if (n_tokens <= 0 || top_k < 0 || top_k > 64 || n_experts <= 0 || hidden <= 0 || intermediate <= 0 ||
        (has_shared != 0 && has_shared != 1) || (top_k == 0 && !has_shared))
        return ST_ARG;
    return prefill_layout(n_tokens, top_k, n_experts, hidden, intermediate, has_shared).total;
}

int mqh_moe_prefill(int gate_type, const void* gate, int up_type, const void* up, int down_type, const void* down,
                    int n_experts, int hidden, int intermediate, int sh_gate_type, const void* sh_gate,
                    int sh_up_type, const void* sh_up, int sh_down_type, const void* sh_down, int sh_intermediate,
                    const float* sh_gate_inp, const void* x, int x_bf16, int n_tokens, const int32_t* ids,
                    const float* weights, int top_k, float* y, void* workspace, int64_t workspace_bytes,
                    void* stream) {
    const int has_shared = sh_gate != nullptr ? 1 : 0;
    if (!x || !y || !workspace || (x_bf16 != 0 && x_bf16 != 1)) return ST_ARG;
    if (n_tokens <= 0 || top_k < 0 || top_k > 64 || (top_k == 0 && !has_shared)) return ST_ARG;
    if (n_experts <= 0 || hidden <= 0 || intermediate <= 0) return ST_ARG;
    if (top_k > 0 && (!gate || !up || !down || !ids || !weights)) return ST_ARG;
    if (has_shared && (!sh_up || !sh_down || sh_intermediate != intermediate)) return ST_ARG;
    if (odd(gate) || odd(up) || odd(down) || odd(sh_gate) || odd(sh_up) || odd(sh_down)) return ST_ARG;
    int st = check_expert_types(gate_type, up_type, down_type, hidden, intermediate);
    if (st) return st;
    if (has_shared && (st = check_expert_types(sh_gate_type, sh_up_type, sh_down_type, hidden, intermediate)))
        return st;
    // 16-byte vector loads of x rows, of the gate vector and of the packed tile records
    if (((uintptr_t)x & 15) || ((uintptr_t)sh_gate_inp & 15) || ((uintptr_t)workspace & 255)) return ST_ARG;

    PrefillParams p{};
    p.gate = (const uint8_t*)gate; p.up = (const uint8_t*)up; p.down = (const uint8_t*)down;
    p.gate_type = gate_type; p.up_type = up_type; p.down_type = down_type;
    p.gate_eb = matrix_bytes(gate_type, intermediate, hidden);
    p.up_eb = matrix_bytes(up_type, intermediate, hidden);
    p.down_eb = matrix_bytes(down_type, hidden, intermediate);
    p.n_experts = n_experts; p.hidden = hidden; p.inter = intermediate;
    p.has_shared = has_shared;
    p.sh_gate_type = sh_gate_type; p.sh_up_type = sh_up_type; p.sh_down_type = sh_down_type;
    if (!prefill_supported(p)) return ST_TYPE;
    const PrefillLayout L = prefill_layout(n_tokens, top_k, n_experts, hidden, intermediate, has_shared);
    if (workspace_bytes < L.total) return ST_WORKSPACE;

    uint8_t* WS = (uint8_t*)workspace;
    p.sh_gate = (const uint8_t*)sh_gate; p.sh_up = (const uint8_t*)sh_up; p.sh_down = (const uint8_t*)sh_down;
    p.sh_gate_inp = sh_gate_inp; p.has_shared = has_shared;
    p.x = x; p.x_bf16 = x_bf16; p.n_tokens = n_tokens;
    p.ids = ids; p.weights = weights; p.top_k = top_k; p.S = top_k + has_shared;
    p.y = y;
    p.flags = (int*)(WS + L.flags_off); p.sh_scale = (float*)(WS + L.scale_off);
    p.tiles = (int*)(WS + L.tiles_off); p.n_tiles = (int*)(WS + L.ntiles_off);
    p.tile_tok = (int*)(WS + L.tok_off); p.tile_dst = (int*)(WS + L.dst_off);
    p.act = (float*)(WS + L.act_off); p.ypair = (float*)(WS + L.ypair_off);
    p.xhi = (uint16_t*)(WS + L.xhi_off); p.xlo = (uint16_t*)(WS + L.xlo_off);
    p.xsum = (uint32_t*)(WS + L.xsum_off); p.xexp = (int*)(WS + L.xexp_off);
    p.max_tiles = L.max_tiles;
    const KernelEvents ev = t_events;
    t_events = KernelEvents();
    return launch_prefill(p, (hipStream_t)stream, ev) == hipSuccess ? ST_OK : ST_HIP;
}

int mqh_profile_next_decode(void* a_start, void* a_stop, void* b_start, void* b_stop) {
    t_events.a_start = (hipEvent_t)a_start;
    t_events.a_stop = (hipEvent_t)a_stop;
    t_events.b_start = (hipEvent_t)b_start;
    t_events.b_stop = (hipEvent_t)b_stop;
    return ST_OK;
}

int mqh_last_decode_kernels(void) { return t_last_kernels; }

int mqh_last_decode_path(void) { return t_last_path; }

int mqh_route(const float* x, int n_tokens, int hidden, const float* gate_weights, int n_experts, int top_k,
              float* scores, int32_t* ids, float* weights, void* stream) {
    if (!x || !gate_weights || !scores || !ids || !weights || n_tokens <= 0 || hidden <= 0 || hidden % 4 ||
        n_experts <= 0 || n_experts > 1024 || top_k < 1 || top_k > 64 || top_k > n_experts ||
        ((uintptr_t)x | (uintptr_t)gate_weights) % 16)
        return ST_ARG;
    return launch_route(x, n_tokens, hidden, gate_weights, n_experts, top_k, scores, ids, weights,
                        (hipStream_t)stream) == hipSuccess
               ? ST_OK
               : ST_HIP;
}

int mqh_read_floor(const void* src, int64_t bytes, void* sink, void* start_event, void* stop_event, void* stream) {
    if (!src || bytes <= 0 || bytes % 16 || ((uintptr_t)src & 15)) return ST_ARG;
    return launch_read_floor(src, bytes, (uint32_t*)sink, (hipStream_t)stream, (hipEvent_t)start_event,
                             (hipEvent_t)stop_event) == hipSuccess
               ? ST_OK
               : ST_HIP;
}

int mqh_set_decode_path(int path) {
    if (path < 0 || path > 1) return ST_ARG;
    const int old = g_decode_path;
    g_decode_path = path;
    return old;
}

}  // extern "C"
