"""Benchmark of the quantized-expert hot path on one MI355X.

Headline workload (one "step" = one token through one MoE layer):
  hidden 2048; 256 experts x intermediate 512; top-8 routing plus one shared
  expert (intermediate 512, sigmoid-gated); gate/up Q4_K, down Q6_K; router
  FP32 [2048 x 256] ~ N(0, 0.02), top-8 of the scores, softmax renormalised.
  One GPU call (two kernels) covers the 9 experts and the weighted combine.  40
  independently seeded layers are resident in HBM (~21 GB) and the steps
  rotate through them, so the 256 MB Infinity Cache cannot hold the working set.

value = quantized weight bytes the step must read (9 x 2,039,808 B =
18,358,272 B) / time per step, in GB/s.  Inputs (weights, activations,
routing) are resident in HBM before timing starts; the 40-layer sweep is
captured once as a HIP graph and replayed, so the time per step includes the
gap between graph nodes.  roofline: the dominant kernel's algorithmic bytes /
its average duration, from HIP events the runtime records at each kernel's
start and end during a second, eager pass over the same layers.

cpu_baseline: the oracle's AVX2 form of the reference's fused expert (direct
Q3_K/Q6_K bit-field decoding into an 8-lane FMA accumulator, the reference's
quant_dot; bit-identical to the scalar oracle) running the same layer as 9
moe_quant_expert calls on 4 worker threads -- the reference's expert-worker
policy -- on the host cores, for a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "intel-optimized-moe-streaming_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "quant-weight GB/s & µs per MoE layer (decode top-8); prefill TFLOP/s"
H, E, I, K = 2048, 256, 512, 8
TYPES = {"gate": 12, "up": 12, "down": 14}
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_layers(n_layers: int, device):
    from flash_moe_hip.layer_store import ExpertLayer

    layers = []
    for l in range(n_layers):
        layers.append(ExpertLayer.synthetic(TYPES, E, H, I, seed=1000 * l + 1, shared_types=TYPES,
                                            shared_intermediate=I, gate_inp=True, device=device))
    return layers


def route_layers(n_layers: int, seed: int = 0, layers=None):
    """Per layer: x ~ N(0,1) [H]; router W ~ N(0, 0.02) [H x E]; top-8 ids and
    softmax weights with the reference router's semantics.  W becomes the
    router of layers[l] when layers are given."""
    from flash_moe_hip.router import ExpertRouter

    xs, ids, ws = [], [], []
    for l in range(n_layers):
        rng = np.random.default_rng(seed + 1000 * l)
        W = (rng.standard_normal((H, E)) * 0.02).astype(np.float32)
        x = rng.standard_normal(H).astype(np.float32)
        r = ExpertRouter(H, E, top_k=K, gate_weights=W, gate_dtype=np.float32)
        i, w = r.route(x)
        xs.append(x)
        ids.append(np.asarray(i, np.int32))
        ws.append(np.asarray(w, np.float32))
        if layers is not None:
            layers[l].router_weights = W
    return np.stack(xs), np.stack(ids), np.stack(ws)


def bench_routed_decode(runner, layers, X, ids_host, ws_host, reps: int, dev) -> dict:
    """The decode step with routing on the device (mqh_moe_decode_routed: the
    router's scores kernel, then the gate/up kernel taking the top-8 and the
    softmax in its prologue, then the down kernel), per layer, captured as one
    graph over the resident layers; and the two-call form (mqh_route, then
    mqh_moe_decode).  Also the router alone, for 1 and 16 tokens.  Parity: the
    device's ids equal the host router's, weights within 2e-6."""
    import torch

    n = len(layers)
    IDS = torch.empty((n, K), dtype=torch.int32, device=dev)
    WS = torch.empty((n, K), dtype=torch.float32, device=dev)
    SC = torch.empty((n, E), dtype=torch.float32, device=dev)
    Y = torch.empty((n, H), dtype=torch.float32, device=dev)
    for L in layers:
        L.router_device()

    def route_all():
        for l in range(n):
            runner.route(layers[l], X[l:l + 1], K, ids=IDS[l:l + 1], weights=WS[l:l + 1], scores=SC[l:l + 1])

    def two_call_all():
        for l in range(n):
            runner.route(layers[l], X[l:l + 1], K, ids=IDS[l:l + 1], weights=WS[l:l + 1], scores=SC[l:l + 1])
            runner.decode(layers[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1])

    def routed_all():
        for l in range(n):
            runner.decode_routed(layers[l], X[l:l + 1], K, ids=IDS[l:l + 1], weights=WS[l:l + 1],
                                 scores=SC[l:l + 1], y=Y[l:l + 1])

    from flash_moe_hip import _lib

    routed_all()
    torch.cuda.synchronize()
    assert runner.status() == 0
    prologue = _lib.load().mqh_last_route_kernels() == 1
    ids_dev, ws_dev = IDS.cpu().numpy(), WS.cpu().numpy()
    same_ids = int(np.sum(np.all(ids_dev == ids_host, axis=1)))
    ok = ids_dev == ids_host
    w_err = float(np.abs(ws_dev - ws_host)[np.all(ok, axis=1)].max()) if same_ids else None
    ms_route = _time(_graph(route_all, dev), reps) / n
    ms_layer = _time(_graph(routed_all, dev), reps) / n
    ms_two = _time(_graph(two_call_all, dev), reps) / n
    assert runner.status() == 0
    X16 = torch.randn((16, H), dtype=torch.float32, device=dev, generator=torch.Generator(dev).manual_seed(3))
    I16 = torch.empty((16, K), dtype=torch.int32, device=dev)
    W16 = torch.empty((16, K), dtype=torch.float32, device=dev)
    S16 = torch.empty((16, E), dtype=torch.float32, device=dev)
    ms16 = _time(_graph(lambda: [runner.route(layers[l], X16, K, ids=I16, weights=W16, scores=S16)
                                 for l in range(n)], dev), reps) / n
    log(f"device router: {ms_route * 1e3:.2f} us (1 token), {ms16 * 1e3:.2f} us (16 tokens); routed decode "
        f"{ms_layer * 1e3:.2f} us/layer (route then decode: {ms_two * 1e3:.2f}); ids equal to the host router's "
        f"on {same_ids}/{n} layers")
    return {
        "workload": f"the headline decode step with routing on the device: x . W (FP32 [{E} x {H}] router, "
                    f"row per expert), top-{K}, float64 softmax, then the fused experts; {n} layers rotated",
        "us_per_layer": round(ms_layer * 1e3, 3),
        "select_in_gate_up_prologue": bool(prologue),
        "gbs": round(step_bytes(layers[0]) / (ms_layer * 1e-3) / 1e9, 1),
        "us_per_layer_route_then_decode": round(ms_two * 1e3, 3),
        "router_us": {"1_token": round(ms_route * 1e3, 3), "16_tokens": round(ms16 * 1e3, 3)},
        "router_bytes_per_call": E * H * 4,
        "ids_equal_layers": f"{same_ids}/{n}",
        "weights_max_abs_err": w_err,
    }


def step_bytes(layer) -> int:
    return (K + 1) * layer.bytes_per_expert()


TRAFFIC_FILE = ROOT / "profiles" / "kernel_traffic.json"
COUNTERS_FILE = ROOT / "profiles" / "kernel_counters.json"
DURATIONS_FILE = ROOT / "profiles" / "kernel_durations.json"


def _profiled(path, instance: str):
    """The committed per-dispatch record of a kernel instance (keyed "name | grid
    N"), taking the largest launch when several workloads run the instance."""
    try:
        kernels = json.loads(path.read_text())["kernels"]
    except (OSError, KeyError, ValueError):
        return None
    rows = [v for k, v in kernels.items() if k.split(" | ")[0] == instance]
    size = lambda v: v.get("hbm_bytes", v.get("active_cycles", v.get("grid_threads", 0)))
    return max(rows, key=size) if rows else None


def measured_traffic(instance: str):
    """HBM bytes per dispatch of a kernel instance from the committed counter
    runs (FETCH_SIZE / WRITE_SIZE scaled by a copy of known size), or None."""
    row = _profiled(TRAFFIC_FILE, instance)
    return row["hbm_bytes"] if row else None


def measured_mfma(instance: str):
    """Matrix-core counters per dispatch of a kernel instance from the committed
    counter run: MFMA busy fraction of the SIMDs and FLOPs issued, or None."""
    row = _profiled(COUNTERS_FILE, instance)
    if not row:
        return None
    return {"mfma_busy_frac": row["mfma_busy_frac"], "mfma_flop_per_dispatch": round(row["mfma_flop"]),
            "mfma_instructions_per_dispatch": round(row["mfma_instructions"]),
            "source": "profiles/prefill_mfma_counters.md"}


def roofline(kern: dict, layer, floor=None) -> dict:
    """The dominant kernel (the larger average duration) against HBM peak.
    Algorithmic bytes per launch: the quantized weight bytes it must read --
    kernel A the gate and up slices, kernel B the down slices -- plus
    activations in and out (a few KB)."""
    a_bytes = (K + 1) * (layer.expert_bytes("gate") + layer.expert_bytes("up"))
    b_bytes = (K + 1) * layer.expert_bytes("down")
    if kern["a_us"] >= kern["b_us"]:
        name, nbytes, us = "mqh::k_fast_gate_up<12, 12, 32, false, 1, true>", a_bytes, kern["a_us"]
    else:
        name, nbytes, us = "mqh::k_fast_down<14, 14, 8, 1, false>", b_bytes, kern["b_us"]
    return _hbm_roofline(name, nbytes, us, floor(nbytes) if floor else None)


def parity_check(layer, x, ids, ws, y_gpu) -> float:
    import oracle

    outs = [oracle.expert_forward(layer.host_expert(int(e)), TYPES, x, H, I, 0) for e in ids]
    sh = layer.host_shared()
    gate = oracle._sigmoid(np.float32(x @ layer.shared.gate_inp.cpu().numpy()).reshape(()))
    sh_out = (gate * oracle.expert_forward(sh, TYPES, x, H, I, 0)).astype(np.float32)
    want = oracle.combine(outs, [float(v) for v in ws], sh_out)
    return oracle.max_relative_error(y_gpu, want)


def cpu_baseline(layers, xs, ids, ws, seconds: float, workers: int = 4):
    """Oracle expert calls on `workers` host threads, 9 per layer-step."""
    import oracle

    oracle.lib()
    n_src = min(len(layers), 8)
    jobs = []
    for l in range(n_src):
        L = layers[l]
        experts = [L.host_expert(int(e)) for e in ids[l]] + [L.host_shared()]
        jobs.append((experts, xs[l], ws[l]))

    def one_step_parallel(pool, job):
        experts, x, w = job
        futs = [pool.submit(oracle.expert_forward, t, TYPES, x, H, I, 0, True) for t in experts]
        outs = [f.result() for f in futs]
        return oracle.combine(outs[:K], [float(v) for v in w], outs[K])

    with ThreadPoolExecutor(workers) as pool:
        one_step_parallel(pool, jobs[0])  # warm
        steps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            one_step_parallel(pool, jobs[steps % n_src])
            steps += 1
        dt = time.perf_counter() - t0
    per_step = dt / steps
    # the same calls on every host thread of the GPU's share, several token-layers in flight
    with ThreadPoolExecutor(CPU_THREADS) as pool:
        calls, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds / 2:
            futs = [pool.submit(oracle.expert_forward, t, TYPES, jobs[j % n_src][1], H, I, 0, True)
                    for j in range(4) for t in jobs[j % n_src][0]]
            for f in futs:
                f.result()
            calls += len(futs)
        dt_all = time.perf_counter() - t0
    per_step_all = dt_all / calls * (K + 1)
    return {
        "value": round(step_bytes(layers[0]) / per_step / 1e9, 3),
        "unit": "GB/s",
        "cores": workers,
        "kind": "port",
        "sample": f"{steps} token-layers (9 AVX2 expert calls each, FP32 graph) over {n_src} layers, "
                  f"{dt:.1f} s on {workers} threads (the reference's expert-worker count); host has "
                  f"{os.cpu_count()} logical CPUs",
        "us_per_layer": round(per_step * 1e6, 1),
        "all_cores": {"value": round(step_bytes(layers[0]) / per_step_all / 1e9, 3), "cores": CPU_THREADS,
                      "us_per_layer": round(per_step_all * 1e6, 1),
                      "sample": f"{calls} expert calls, four token-layers in flight, {dt_all:.1f} s"},
    }


def _hip_runtime():
    """The process's HIP runtime (the one torch and the library already share)."""
    import ctypes as C

    rt = C.CDLL("libamdhip64.so.7")
    rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    rt.hipEventDestroy.argtypes = [C.c_void_p]
    return rt


def kernel_times(runner, layers, X, IDS, WS, Y, reps: int, fp16_graph: int = 0) -> dict:
    """Duration of each decode kernel: an eager pass of reps x layers steps,
    every kernel launched with start/stop HIP events; the median over the
    launches (the mean beside it)."""
    import ctypes as C

    import torch

    from flash_moe_hip import _lib

    lib, rt = _lib.load(), _hip_runtime()
    n = reps * len(layers)
    ev = []
    for _ in range(4 * n):
        h = C.c_void_p()
        if rt.hipEventCreate(C.byref(h)) != 0:
            raise RuntimeError("hipEventCreate failed")
        ev.append(h)
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    for i in range(n):
        l = i % len(layers)
        _lib.check(lib.mqh_profile_next_decode(ev[4 * i], ev[4 * i + 1], ev[4 * i + 2], ev[4 * i + 3]),
                   "mqh_profile_next_decode")
        runner.decode(layers[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1], stream=stream,
                      fp16_graph=fp16_graph)
    torch.cuda.synchronize()

    def ms(a, b):
        v = C.c_float()
        if rt.hipEventElapsedTime(C.byref(v), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return v.value

    a = [ms(ev[4 * i], ev[4 * i + 1]) * 1e3 for i in range(n)]
    b = [ms(ev[4 * i + 2], ev[4 * i + 3]) * 1e3 for i in range(n)]
    for h in ev:
        rt.hipEventDestroy(h)
    return {"a_us": float(np.median(a)), "b_us": float(np.median(b)), "launches": n,
            "a_mean_us": float(np.mean(a)), "b_mean_us": float(np.mean(b)),
            "kernels": int(lib.mqh_last_decode_kernels())}


# ---------------------------------------------------------------- other workloads

CPU_THREADS = 16   # host threads per GPU (the host-CPU share of one MI355X)
DEQ_TYPES = (11, 12, 14, 8)


class StepRunner:
    """Runs n steps of a sweep over `layers` layers (step i = layer i % layers)
    as replays of one captured graph of the whole sweep plus, for n % layers,
    a graph of the first n % layers steps (captured on first use).
    sweep(n, start=0) runs layers start .. start + n - 1."""

    def __init__(self, sweep, layers: int, dev, eager: bool = False):
        self.sweep, self.layers, self.dev, self.eager = sweep, layers, dev, eager
        self.parts = {}

    def _replay(self, n: int):
        if n not in self.parts:
            self.parts[n] = (lambda: self.sweep(n)) if self.eager else _graph(lambda: self.sweep(n), self.dev)
        return self.parts[n]

    def __call__(self, n: int) -> None:
        full, rem = divmod(n, self.layers)
        if full:
            g = self._replay(self.layers)
            for _ in range(full):
                g()
        if rem:
            self._replay(rem)()

    def timed(self, n: int) -> float:
        """ms of GPU time for exactly n steps.  Every graph is captured (and
        warm) first; a short spin kernel ahead of the start event keeps the GPU
        busy while the host queues the launches, so the timed region holds the
        n steps and their graph-node gaps only."""
        import torch

        full, rem = divmod(n, self.layers)
        if full:
            self._replay(self.layers)
        if rem:
            self._replay(rem)
        if not full:
            # capturing the partial graph ran layers 0 .. rem - 1 last: run the
            # other layers after them, so the timed layers are the least
            # recently touched (the resident layers are ~3x the Infinity Cache)
            self.sweep(self.layers - rem, rem)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        s.record()
        self(n)
        e.record()
        e.synchronize()
        return s.elapsed_time(e)


def _graph(fn, dev):
    """Capture fn() (already run once eagerly) as a graph; return its replay."""
    import torch

    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(cap):
        fn()
    torch.cuda.current_stream(dev).wait_stream(cap)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=cap):
        fn()
    return g.replay


def _time(fn, reps: int) -> float:
    """ms per call of fn over reps calls, after one warm call."""
    import torch

    fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


def _kernel_pair_times(calls, reps: int) -> dict:
    """Duration of the two GEMM kernels (A: gate/up, B: down) of each call in
    calls (run eagerly reps times each), from runtime HIP events: the median
    over the launches (a launch after an idle host gap runs at lower clocks
    now and then; the mean is returned beside it)."""
    import ctypes as C

    import torch

    from flash_moe_hip import _lib

    lib, rt = _lib.load(), _hip_runtime()
    n = reps * len(calls)
    ev = []
    for _ in range(4 * n):
        h = C.c_void_p()
        if rt.hipEventCreate(C.byref(h)) != 0:
            raise RuntimeError("hipEventCreate failed")
        ev.append(h)
    torch.cuda.synchronize()
    for i in range(n):
        _lib.check(lib.mqh_profile_next_decode(ev[4 * i], ev[4 * i + 1], ev[4 * i + 2], ev[4 * i + 3]),
                   "mqh_profile_next_decode")
        calls[i % len(calls)]()
    torch.cuda.synchronize()

    def us(a, b):
        v = C.c_float()
        if rt.hipEventElapsedTime(C.byref(v), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return v.value * 1e3

    a = [us(ev[4 * i], ev[4 * i + 1]) for i in range(n)]
    b = [us(ev[4 * i + 2], ev[4 * i + 3]) for i in range(n)]
    for h in ev:
        rt.hipEventDestroy(h)
    return {"a_us": float(np.median(a)), "b_us": float(np.median(b)), "a_mean_us": float(np.mean(a)),
            "b_mean_us": float(np.mean(b)), "launches": n, "kernels": int(lib.mqh_last_decode_kernels())}


def read_floor_us(nbytes: int, reps: int = 40) -> float:
    """Duration of a plain streaming read of nbytes (mqh_read_floor), rotated
    over regions of a scratch buffer larger than the 256 MB MALL, timed like
    the kernels: HIP events recorded at the kernel's own start and end, on the
    current stream, the median over the launches after the first quarter."""
    import ctypes as C

    import torch

    from flash_moe_hip import _lib

    lib, rt = _lib.load(), _hip_runtime()
    nbytes = nbytes // 256 * 256
    n_reg = max(2, -(-(512 << 20) // nbytes))
    buf = torch.empty(n_reg * nbytes, dtype=torch.uint8, device="cuda")
    ev = []
    for _ in range(2 * reps):
        h = C.c_void_p()
        if rt.hipEventCreate(C.byref(h)) != 0:
            raise RuntimeError("hipEventCreate failed")
        ev.append(h)
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    for i in range(reps):
        _lib.check(lib.mqh_read_floor(buf.data_ptr() + (i % n_reg) * nbytes, nbytes, None, ev[2 * i], ev[2 * i + 1],
                                      stream), "mqh_read_floor")
    torch.cuda.synchronize()
    del buf
    vals = []
    for i in range(reps):
        v = C.c_float()
        if rt.hipEventElapsedTime(C.byref(v), ev[2 * i], ev[2 * i + 1]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        vals.append(v.value * 1e3)
    for h in ev:
        rt.hipEventDestroy(h)
    return float(np.median(vals[reps // 4:]))   # (the first quarter warms the buffer's translations)


def _hbm_roofline(name: str, nbytes: float, us: float, floor_us: float | None = None) -> dict:
    """name: the kernel instance as the profiler names it; floor_us: the
    streaming-read time of the same byte count (read_floor_us).  Beside the
    live event time, the committed kernel trace's average duration of the same
    instance (its largest launch, graph-replayed in the full benchmark)."""
    gbs = nbytes / (us * 1e-6) / 1e9
    traced = _profiled(DURATIONS_FILE, name)
    out = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(name), "kernel": name,
           "algorithmic_bytes": int(nbytes), "kernel_us": round(us, 3),
           "kernel_us_profiled": traced["mean_us"] if traced else None}
    if floor_us is not None:
        out["read_floor_us"] = round(floor_us, 3)
        out["frac_of_read_floor"] = round(floor_us / us, 4)
    return out


def _topk_routing(rng, T: int, k: int):
    """top-k of N(0,1) logits per token, softmax over the selected k."""
    logits = rng.standard_normal((T, E))
    ids = np.argsort(-logits, axis=1)[:, :k]
    sel = np.take_along_axis(logits, ids, 1)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    return ids.astype(np.int32), (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def _oracle_tokens(layer, types, X, ids, ws, t_list):
    """Oracle layer outputs (run_moe_sequence arithmetic) for tokens t_list."""
    import oracle

    sh = layer.host_shared()
    gi = layer.shared.gate_inp.cpu().numpy()
    out = {}
    for t in t_list:
        x = X[t]
        outs = [oracle.expert_forward(layer.host_expert(int(e)), types, x, H, I, 0) for e in ids[t]]
        gate = oracle._sigmoid(np.float32(x @ gi).reshape(()))
        sh_out = (gate * oracle.expert_forward(sh, layer.shared.types, x, H, I, 0)).astype(np.float32)
        out[t] = oracle.combine(outs, [float(v) for v in ws[t]], sh_out)
    return out


def _cpu_pairs(jobs, seconds: float, workers: int):
    """Run AVX2 oracle expert calls (types, bytes, x) on `workers` threads for about
    `seconds`; returns (calls, elapsed)."""
    import oracle

    oracle.lib()
    calls, t0 = 0, time.perf_counter()
    with ThreadPoolExecutor(workers) as pool:
        while time.perf_counter() - t0 < seconds:
            batch = [jobs[(calls + i) % len(jobs)] for i in range(4 * workers)]
            list(pool.map(lambda j: oracle.expert_forward(j[1], j[0], j[2], H, I, 0, True), batch))
            calls += len(batch)
    return calls, time.perf_counter() - t0


def _one_thread_expert_us(job, seconds: float) -> float:
    """Microseconds per AVX2 expert call (types, bytes, x) on one thread."""
    import oracle

    types, tensors, x = job
    oracle.expert_forward(tensors, types, x, H, I, 0, True)
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.expert_forward(tensors, types, x, H, I, 0, True)
        calls += 1
    return round((time.perf_counter() - t0) / calls * 1e6, 1)


def bench_batched_decode(dev, n_layers: int, steps: int, cpu_seconds: float) -> dict:
    """16 tokens through one all-Q3_K layer, top-8 of N(0,1) logits + shared;
    n_layers independently seeded layers rotated.  Both kernel families are
    timed; the reported value is the faster one."""
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    T, types = 16, {"gate": 11, "up": 11, "down": 11}
    layers = [ExpertLayer.synthetic(types, E, H, I, seed=7000 + 1000 * l, shared_types=types,
                                    shared_intermediate=I, gate_inp=True, device=dev) for l in range(n_layers)]
    rng = np.random.default_rng(4)
    Xh, IDh, WSh = [], [], []
    for _ in range(n_layers):
        Xh.append(rng.standard_normal((T, H)).astype(np.float32))
        i, w = _topk_routing(rng, T, K)
        IDh.append(i)
        WSh.append(w)
    X = [torch.from_numpy(v).to(dev) for v in Xh]
    IDS = [torch.from_numpy(v).to(dev) for v in IDh]
    WS = [torch.from_numpy(v).to(dev) for v in WSh]
    Y = torch.empty((T, H), dtype=torch.float32, device=dev)
    U = [len(np.unique(v)) for v in IDh]
    nbytes = float(np.mean([(u + 1) * layers[0].bytes_per_expert() for u in U]))
    runner = MoeRunner(dev)
    # the same layers in the 112-byte-slot Q3_K resident form (decode only)
    aligned = [L.aligned_q3k() for L in layers]
    paths = {
        "prefill": lambda l: runner.prefill(layers[l], X[l], IDS[l], WS[l], y=Y),
        "decode": lambda l: runner.decode(layers[l], X[l], IDS[l], WS[l], y=Y),
        "decode_aligned_q3k": lambda l: runner.decode(aligned[l], X[l], IDS[l], WS[l], y=Y),
    }
    res = {}
    want = _oracle_tokens(layers[0], types, Xh[0], IDh[0], WSh[0], [0, 7, 15])
    import oracle

    for name, call in paths.items():
        call(0)
        torch.cuda.synchronize()
        assert runner.status() == 0
        got = Y.cpu().numpy()
        err = max(oracle.max_relative_error(got[t], want[t]) for t in want)
        replay = _graph(lambda: [call(l) for l in range(n_layers)], dev)
        ms = _time(replay, max(1, steps // n_layers)) / n_layers
        kern = _kernel_pair_times([lambda l=l: call(l) for l in range(n_layers)], 2)
        res[name] = {"us_per_layer": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "parity_max_rel_err": float(f"{err:.3e}"),
                     "kernels_us": {"A": round(kern["a_us"], 2), "B": round(kern["b_us"], 2)}}
        log(f"batched decode via {name}: {ms * 1e3:.2f} us/layer, parity {err:.2e}")
    best = min(res, key=lambda k: res[k]["us_per_layer"])
    kb = res[best]["kernels_us"]
    frac_a = (layers[0].expert_bytes("gate") + layers[0].expert_bytes("up")) / layers[0].bytes_per_expert()
    dom = "A" if kb["A"] >= kb["B"] else "B"
    frac = frac_a if dom == "A" else 1 - frac_a
    kname = {"prefill": {"A": "mqh::k_prefill_gate_up<11, 11, 8, false, 2>", "B": "mqh::k_prefill_down<11, 11, 2, 1>"},
             "decode": {"A": "mqh::k_fast_gate_up<11, 11, 32, false, 2, false>", "B": "mqh::k_fast_down_bal<11, 11, 8, 4>"},
             "decode_aligned_q3k": {"A": "mqh::k_fast_gate_up<111, 111, 32, false, 2, false>",
                                    "B": "mqh::k_fast_down_bal<111, 111, 8, 4>"}}[best][dom]
    out = {
        "workload": f"batched decode: {T} tokens, hidden {H}, {E} experts x intermediate {I}, top-8 of N(0,1) "
                    f"logits + shared, all Q3_K, {n_layers} resident layers rotated (path decode_aligned_q3k: the "
                    f"same blocks in 112-byte slots; GB/s counts the GGUF bytes)",
        "metric": "quant-weight GB/s per layer-step (weights of the U distinct routed experts + shared)",
        "value": res[best]["gbs"], "unit": "GB/s", "us_per_layer": res[best]["us_per_layer"],
        "path": best, "paths": res, "distinct_experts_mean": float(np.mean(U)),
        "weight_bytes_per_step": int(nbytes),
        "roofline": _hbm_roofline(kname, nbytes * frac, kb[dom], read_floor_us(int(nbytes * frac))),
    }
    if cpu_seconds > 0:
        L0 = layers[0]
        jobs = [(types, L0.host_expert(int(e)), Xh[0][t]) for t in range(T) for e in IDh[0][t]]
        jobs += [(types, L0.host_shared(), Xh[0][t]) for t in range(T)]
        calls, dt = _cpu_pairs(jobs, cpu_seconds, CPU_THREADS)
        per_step = dt / calls * T * (K + 1)
        out["cpu_baseline"] = {"value": round(nbytes / per_step / 1e9, 3), "unit": "GB/s", "cores": CPU_THREADS,
                               "kind": "port", "us_per_layer": round(per_step * 1e6, 1),
                               "sample": f"{calls} per-token AVX2 expert calls (16 tokens x 9 per step), {dt:.1f} s",
                               "per_expert_us_1_thread": _one_thread_expert_us(jobs[0], cpu_seconds / 4)}
    del layers
    torch.cuda.empty_cache()
    return out


def bench_prefill(dev, n_layers: int, reps: int, cpu_seconds: float, types=None, shared_types=None,
                  what: str = "gate/up Q4_K, down Q6_K, shared expert the same") -> dict:
    """128-token BF16 prompt through one layer (default: gate/up Q4_K, down Q6_K,
    top-8 of N(0,1) logits + a shared expert of the routed types), n_layers
    seeded layers rotated."""
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    types = dict(types or TYPES)
    shared_types = dict(shared_types or types)
    T = 128
    layers = [ExpertLayer.synthetic(types, E, H, I, seed=9000 + 1000 * l, shared_types=shared_types,
                                    shared_intermediate=I, gate_inp=True, device=dev) for l in range(n_layers)]
    assert MoeRunner.prefill_supported(layers[0]) and MoeRunner._shared_in_prefill(layers[0])
    rng = np.random.default_rng(5)
    gen = torch.Generator().manual_seed(5)
    Xh, IDh, WSh = [], [], []
    for _ in range(n_layers):
        x = torch.randn((T, H), generator=gen).to(torch.bfloat16)
        Xh.append(x)
        i, w = _topk_routing(rng, T, K)
        IDh.append(i)
        WSh.append(w)
    X = [v.to(dev) for v in Xh]
    IDS = [torch.from_numpy(v).to(dev) for v in IDh]
    WS = [torch.from_numpy(v).to(dev) for v in WSh]
    Y = torch.empty((T, H), dtype=torch.float32, device=dev)
    runner = MoeRunner(dev)
    call = lambda l: runner.prefill(layers[l], X[l], IDS[l], WS[l], y=Y)
    call(0)
    torch.cuda.synchronize()
    assert runner.status() == 0
    import oracle

    xf = Xh[0].float().numpy()
    want = _oracle_tokens(layers[0], types, xf, IDh[0], WSh[0], [0, 64, 127])
    got = Y.cpu().numpy()
    err = max(oracle.max_relative_error(got[t], want[t]) for t in want)
    replay = _graph(lambda: [call(l) for l in range(n_layers)], dev)
    ms = _time(replay, reps) / n_layers
    kern = _kernel_pair_times([lambda l=l: call(l) for l in range(n_layers)], 3)
    U = [len(np.unique(v)) for v in IDh]
    flop = 2.0 * T * (K + 1) * 3 * H * I
    L0 = layers[0]
    sh_gu = L0.shared.gate.numel() + L0.shared.up.numel()
    nbytes = float(np.mean([u * L0.bytes_per_expert() + L0.shared_bytes() for u in U]))
    gu = float(np.mean([u * (L0.expert_bytes("gate") + L0.expert_bytes("up")) + sh_gu for u in U]))
    tflops = flop / (ms * 1e-3) / 1e12
    dom = "A" if kern["a_us"] >= kern["b_us"] else "B"
    dom_bytes = gu if dom == "A" else nbytes - gu
    gt, dt, sgt, sdt = types["gate"], types["down"], shared_types["gate"], shared_types["down"]
    name_a, name_b = f"mqh::k_prefill_gate_up<{gt}, {sgt}, 8, true, 2>", f"mqh::k_prefill_down<{dt}, {sdt}, 2, 1>"
    roof = _hbm_roofline(name_a if dom == "A" else name_b, dom_bytes, kern["a_us"] if dom == "A" else kern["b_us"],
                         read_floor_us(int(dom_bytes)))
    log(f"prefill ({what}): {ms * 1e3:.1f} us/layer, {tflops:.1f} TFLOP/s, parity {err:.2e}; "
        f"gate/up {kern['a_us']:.1f} us, down {kern['b_us']:.1f} us")
    out = {
        "workload": f"prefill: {T}-token BF16 prompt, hidden {H}, {E} experts x intermediate {I}, top-8 of N(0,1) "
                    f"logits + shared, {what}, {n_layers} resident layers rotated",
        "metric": "prefill TFLOP/s (useful FLOPs: 1152 pairs x 6,291,456)", "value": round(tflops, 2),
        "unit": "TFLOP/s", "us_per_layer": round(ms * 1e3, 2), "flop_per_layer": int(flop),
        "weight_bytes_per_layer": int(nbytes), "weight_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "distinct_experts_mean": float(np.mean(U)), "parity_max_rel_err": float(f"{err:.3e}"),
        "kernels_us": {"k_prefill_gate_up": round(kern["a_us"], 2), "k_prefill_down": round(kern["b_us"], 2)},
        "roofline": roof,
        "mfma_ceiling": {"peak_tflops_fp16_dense": 2500.0, "frac": round(tflops / 2500.0, 5)},
        # matrix-core activity of the gate/up GEMM from the committed counter run
        # (useful FLOPs are about a quarter of those issued: ~4 of 16 token columns)
        "mfma_counters": measured_mfma(name_a),
    }
    if cpu_seconds > 0:
        jobs = [(types, L0.host_expert(int(e)), xf[t]) for t in range(0, T, 8) for e in IDh[0][t]]
        calls, dt = _cpu_pairs(jobs, cpu_seconds, CPU_THREADS)
        per_layer = dt / calls * T * (K + 1)
        out["cpu_baseline"] = {"value": round(flop / per_layer / 1e12, 5), "unit": "TFLOP/s",
                               "cores": CPU_THREADS, "kind": "port", "us_per_layer": round(per_layer * 1e6, 1),
                               "sample": f"{calls} (token, expert) AVX2 calls of the native-kernel port, {dt:.1f} s; "
                                         "the reference prefill (OpenVINO) is not available"}
    del layers
    torch.cuda.empty_cache()
    return out


def bench_dequant(dev, reps: int, cpu_seconds: float) -> dict:
    """256 experts x 3 matrices (gate/up [512x2048], down [2048x512]) to FP16,
    once per type; GB/s over quantized bytes read + FP16 bytes written."""
    import torch

    import oracle
    from flash_moe_hip.dequant import dequant_device
    from flash_moe_hip.quant_types import block_info
    from flash_moe_hip.synthetic import torch_random_stack

    n = 3 * E * H * I
    out = torch.empty(n, dtype=torch.float16, device=dev)
    res = {}
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    for t in DEQ_TYPES:
        src = torch_random_stack(t, 3 * E, I, H, generator=g, device=dev)
        dequant_device(src, t, n, out=out)
        torch.cuda.synchronize()
        # bit-exact check on a sample of blocks
        bs, pb = block_info(t)
        nb = 4096
        sample = src[: nb * pb].cpu().numpy()
        want = oracle.dequant(t, sample, nb * bs, want_f16=True)
        ok = bool(np.array_equal(out[: nb * bs].cpu().numpy().view(np.uint16), np.asarray(want).view(np.uint16)))
        ms = _time(lambda: dequant_device(src, t, n, out=out), reps)
        nbytes = src.numel() + 2 * n
        res[str(t)] = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "us": round(ms * 1e3, 1), "bytes": nbytes,
                       "bit_exact_sample": ok, "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"dequant type {t}: {ms * 1e3:.1f} us, {res[str(t)]['gbs']} GB/s, bit-exact sample {ok}")
        del src
    best = max(res, key=lambda k: res[k]["gbs"])
    worst = min(res, key=lambda k: res[k]["gbs"])
    out_d = {
        "workload": "dequantization to FP16: 256 experts x 3 matrices ([512x2048] gate, up, [2048x512] down), "
                    "types Q3_K (11), Q4_K (12), Q6_K (14), Q8_0 (8)",
        "metric": "GB/s (quantized bytes read + FP16 bytes written)", "per_type": res,
        "value": res[worst]["gbs"], "unit": "GB/s",
        "roofline": _hbm_roofline("mqh::k_dequant_lds<%s, true>" % worst, res[worst]["bytes"], res[worst]["us"]),
    }
    if cpu_seconds > 0:
        t = 12
        src = torch_random_stack(t, 64, I, H, generator=g, device=dev).cpu().numpy()
        mats = src.reshape(64, -1)
        oracle.lib()
        done, t0 = 0, time.perf_counter()
        with ThreadPoolExecutor(CPU_THREADS) as pool:
            while time.perf_counter() - t0 < cpu_seconds:
                list(pool.map(lambda m: oracle.dequant(t, m, H * I, want_f16=True), mats))
                done += len(mats)
        dt = time.perf_counter() - t0
        per = (mats.shape[1] + 2 * H * I) * done / dt
        out_d["cpu_baseline"] = {"value": round(per / 1e9, 3), "unit": "GB/s", "cores": CPU_THREADS, "kind": "port",
                                 "sample": f"{done} Q4_K matrices [512x2048] -> FP16 in {dt:.1f} s"}
    del out
    torch.cuda.empty_cache()
    return out_d


def _delta_kernel_us(states, ins, outs, reps: int) -> float:
    """Average duration of the DeltaNet kernel over reps eager passes of the
    layers, from HIP events the runtime records at its start and end."""
    import ctypes as C

    import torch

    from flash_moe_hip import _lib

    lib, rt = _lib.load(), _hip_runtime()
    n = reps * len(states)
    ev = []
    for _ in range(2 * n):
        h = C.c_void_p()
        if rt.hipEventCreate(C.byref(h)) != 0:
            raise RuntimeError("hipEventCreate failed")
        ev.append(h)
    torch.cuda.synchronize()
    for i in range(n):
        l = i % len(states)
        _lib.check(lib.mqh_profile_next_decode(ev[2 * i], ev[2 * i + 1], None, None), "mqh_profile_next_decode")
        states[l].step(*ins[l], out=outs[l])
    torch.cuda.synchronize()
    us = []
    for i in range(n):
        v = C.c_float()
        if rt.hipEventElapsedTime(C.byref(v), ev[2 * i], ev[2 * i + 1]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        us.append(v.value * 1e3)
    for h in ev:
        rt.hipEventDestroy(h)
    return float(np.mean(us))


def bench_fp16_graph_decode(dev, n_layers: int, reps: int, cpu_seconds: float) -> dict:
    """The headline decode step in the FP16 graph (fp16_graph=1), the
    reference's production mode (native_expert.py:33-34): x, every decoded
    weight, g, u, the sigmoid, silu, the activation and y rounded to FP16 at the
    points of moe_quant_dot.cpp:189-211.  At the headline's scales the FP16
    graph overflows (the reference returns -4 there too), so the layers use the
    reference's FP16-graph check scales: super-block scales |N(0,1)| * 0.002,
    x ~ N(0,1) * 0.05.  Same shape, types and routing as the headline."""
    import torch

    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    layers = [ExpertLayer.synthetic(TYPES, E, H, I, seed=1000 * l + 1, shared_types=TYPES, shared_intermediate=I,
                                    gate_inp=True, scale=0.002, device=dev) for l in range(n_layers)]
    xs, ids, ws = route_layers(n_layers, layers=layers)
    xs = (xs * 0.05).astype(np.float32)
    X, IDS, WS = (torch.from_numpy(a).to(dev) for a in (xs, ids, ws))
    Y = torch.empty((n_layers, H), dtype=torch.float32, device=dev)
    runner = MoeRunner(dev)

    def sweep(n=n_layers):
        for l in range(n):
            runner.decode(layers[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1], fp16_graph=1)

    sweep()
    torch.cuda.synchronize()
    assert runner.status() == 0
    import oracle

    L0 = layers[0]
    outs = [oracle.expert_forward(L0.host_expert(int(e)), TYPES, xs[0], H, I, 1) for e in ids[0]]
    gate = oracle._sigmoid(np.float32(xs[0] @ L0.shared.gate_inp.cpu().numpy()).reshape(()))
    sh = (gate * oracle.expert_forward(L0.host_shared(), TYPES, xs[0], H, I, 0)).astype(np.float32)
    err = oracle.max_relative_error(Y[0].cpu().numpy(), oracle.combine(outs, [float(v) for v in ws[0]], sh))
    ms = _time(_graph(sweep, dev), reps) / n_layers
    kern = kernel_times(runner, layers, X, IDS, WS, Y, reps=4, fp16_graph=1)
    log(f"FP16-graph decode: {ms * 1e3:.2f} us/layer, parity {err:.2e}; kernels {kern['a_us']:.2f} / "
        f"{kern['b_us']:.2f} us")
    a_bytes = (K + 1) * (L0.expert_bytes("gate") + L0.expert_bytes("up"))
    dom = "A" if kern["a_us"] >= kern["b_us"] else "B"
    out = {
        "workload": f"the headline decode step in the FP16 graph (fp16_graph=1): hidden {H}, {E} experts x "
                    f"intermediate {I}, top-8 + shared, gate/up Q4_K, down Q6_K, super-block scales |N|*0.002, "
                    f"x ~ N(0,1)*0.05; {n_layers} resident layers rotated",
        "metric": "quant-weight GB/s per layer-step", "value": round(step_bytes(L0) / (ms * 1e-3) / 1e9, 1),
        "unit": "GB/s", "us_per_layer": round(ms * 1e3, 3), "parity_max_rel_err": float(f"{err:.3e}"),
        "kernels_us": {"A": round(kern["a_us"], 3), "B": round(kern["b_us"], 3)},
        "roofline": _hbm_roofline("mqh::k_fast_gate_up<12, 12, 32, true, 1, true>" if dom == "A" else
                                  "mqh::k_fast_down<14, 14, 8, 1, true>",
                                  a_bytes if dom == "A" else step_bytes(L0) - a_bytes,
                                  kern["a_us"] if dom == "A" else kern["b_us"]),
    }
    if cpu_seconds > 0:
        oracle.lib()
        jobs = [L0.host_expert(int(e)) for e in ids[0]]
        done, t0 = 0, time.perf_counter()
        with ThreadPoolExecutor(4) as pool:
            while time.perf_counter() - t0 < cpu_seconds:
                list(pool.map(lambda t: oracle.expert_forward(t, TYPES, xs[0], H, I, 1, True), jobs))
                done += 1
        dt = time.perf_counter() - t0
        per = dt / done * (K + 1) / K
        out["cpu_baseline"] = {"value": round(step_bytes(L0) / per / 1e9, 3), "unit": "GB/s", "cores": 4,
                               "kind": "port", "us_per_layer": round(per * 1e6, 1),
                               "sample": f"{done} x 8 FP16-graph AVX2 expert calls on 4 threads, {dt:.1f} s"}
    del layers
    torch.cuda.empty_cache()
    return out


# The reference model's expert type mixes (every layer has a Q6_K shared
# expert): routed Q3_K throughout in layers 5-34, Q4_K gate/up with Q6_K down in
# layers 1-4 and 35-39, Q4_K gate/up with Q8_0 down in layer 0.
REF_MIXES = (("layers 5-34", {"gate": 11, "up": 11, "down": 11}),
             ("layers 1-4, 35-39", {"gate": 12, "up": 12, "down": 14}),
             ("layer 0", {"gate": 12, "up": 12, "down": 8}))
Q6_SHARED = {"gate": 14, "up": 14, "down": 14}


def bench_decode_mixes(dev, n_layers: int, reps: int) -> dict:
    """The decode step (one token, top-8 + the Q6_K shared expert, hidden 2048,
    256 experts x intermediate 512) in the reference model's type mixes, in both
    graphs: n_layers resident layers rotated in one graph, as the headline.
    The FP16 graph uses the reference's FP16-graph check scales (super-block
    scales |N| * 0.002, x ~ N(0,1) * 0.05).  Parity on layer 0 of each against
    the oracle's experts, combine and FP32-graph shared expert."""
    import torch

    import oracle
    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner

    runner = MoeRunner(dev)
    out = {"workload": f"decode MoE layer, 1 token, top-8 + Q6_K shared expert, hidden {H}, {E} experts x "
                       f"intermediate {I}, the reference model's type mixes; {n_layers} resident layers rotated",
           "metric": "us per layer step", "unit": "us", "higher_is_better": False, "mixes": {}}
    for name, types in REF_MIXES:
        row = {}
        for fp16 in (0, 1):
            kw = {"scale": 0.002} if fp16 else {}
            layers = [ExpertLayer.synthetic(types, E, H, I, seed=1000 * l + 7, shared_types=Q6_SHARED,
                                            shared_intermediate=I, gate_inp=True, device=dev, **kw)
                      for l in range(n_layers)]
            xs, ids, ws = route_layers(n_layers, seed=31, layers=layers)
            if fp16:
                xs = (xs * 0.05).astype(np.float32)
            X, IDS, WS = (torch.from_numpy(a).to(dev) for a in (xs, ids, ws))
            Y = torch.empty((n_layers, H), dtype=torch.float32, device=dev)

            def sweep(n=n_layers):
                for l in range(n):
                    runner.decode(layers[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1], fp16_graph=fp16)

            sweep()
            torch.cuda.synchronize()
            assert runner.status() == 0
            L0 = layers[0]
            outs = [oracle.expert_forward(L0.host_expert(int(e)), types, xs[0], H, I, fp16) for e in ids[0]]
            gate = oracle._sigmoid(np.float32(xs[0] @ L0.shared.gate_inp.cpu().numpy()).reshape(()))
            sh = (gate * oracle.expert_forward(L0.host_shared(), Q6_SHARED, xs[0], H, I, 0)).astype(np.float32)
            err = oracle.max_relative_error(Y[0].cpu().numpy(), oracle.combine(outs, [float(v) for v in ws[0]], sh))
            ms = _time(_graph(sweep, dev), reps) / n_layers
            kern = kernel_times(runner, layers, X, IDS, WS, Y, reps=4, fp16_graph=fp16)
            nbytes = K * L0.bytes_per_expert() + L0.shared_bytes()
            row["fp16_graph" if fp16 else "fp32_graph"] = {
                "us_per_layer": round(ms * 1e3, 3), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "kernels_us": {"A": round(kern["a_us"], 3), "B": round(kern["b_us"], 3)},
                "parity_max_rel_err": float(f"{err:.3e}")}
            if 11 in types.values():
                # the same layers with their Q3_K matrices in 112-byte slots
                y0 = Y.clone()
                layers_a = [L.aligned_q3k() for L in layers]

                def sweep_a(n=n_layers):
                    for l in range(n):
                        runner.decode(layers_a[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1],
                                      fp16_graph=fp16)

                sweep_a()
                torch.cuda.synchronize()
                assert runner.status() == 0 and torch.equal(Y.view(torch.int32), y0.view(torch.int32))
                ms_a = _time(_graph(sweep_a, dev), reps) / n_layers
                row["fp16_graph" if fp16 else "fp32_graph"]["aligned_q3k"] = {
                    "us_per_layer": round(ms_a * 1e3, 3), "outputs_bit_identical": True}
                log(f"decode, {name} ({'FP16' if fp16 else 'FP32'} graph), Q3_K in 112-byte slots: "
                    f"{ms_a * 1e3:.2f} us/layer")
                del layers_a
            log(f"decode, {name} ({'FP16' if fp16 else 'FP32'} graph): {ms * 1e3:.2f} us/layer, parity {err:.2e}; "
                f"kernels {kern['a_us']:.2f} / {kern['b_us']:.2f} us")
            del layers
            torch.cuda.empty_cache()
        out["mixes"][name] = {"types": types, "shared_types": Q6_SHARED, **row}
    return out


def bench_single_expert(dev, reps: int, cpu_seconds: float) -> dict:
    """One Q4_K expert (gate/up [512x2048], down [2048x512]), one token, x ~ N(0,1),
    seed 0 (the reference's single-expert decode): 40 such experts resident and
    rotated, each call through the fused decode with top-1 weight 1.0 and no
    shared expert.  The 70 MB of weights fit in the Infinity Cache, and the call
    is launch-bound: this line is the CPU comparison of the smallest unit."""
    import torch

    import oracle
    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_gpu import MoeRunner
    from flash_moe_hip.synthetic import config1_expert

    n = 40
    tensors, kinds, x = config1_expert(0)
    layers = [ExpertLayer.from_host(tensors, kinds, 1, H, I, device=dev)]
    layers += [ExpertLayer.synthetic(kinds, 1, H, I, seed=500 + l, device=dev) for l in range(n - 1)]
    X = torch.from_numpy(x[None]).to(dev)
    IDS = torch.zeros((1, 1), dtype=torch.int32, device=dev)
    WS = torch.ones((1, 1), dtype=torch.float32, device=dev)
    Y = torch.empty((n, H), dtype=torch.float32, device=dev)
    runner = MoeRunner(dev)

    def sweep():
        for l in range(n):
            runner.decode(layers[l], X, IDS, WS, y=Y[l:l + 1], use_shared=False)

    sweep()
    torch.cuda.synchronize()
    assert runner.status() == 0
    want = oracle.expert_forward(tensors, kinds, x, H, I, 0)
    err = oracle.max_relative_error(Y[0].cpu().numpy(), want)
    ms = _time(_graph(sweep, dev), reps) / n
    nbytes = layers[0].bytes_per_expert()
    log(f"single expert: {ms * 1e3:.2f} us per call, parity {err:.2e}")
    out = {
        "workload": "one Q4_K expert, 1 token (gate/up [512x2048], down [2048x512], x ~ N(0,1), seed 0); 40 resident "
                    "experts rotated (70 MB: Infinity-Cache resident), fused decode top-1, no shared expert",
        "metric": "us per expert call", "value": round(ms * 1e3, 3), "unit": "us", "higher_is_better": False,
        "weight_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "parity_max_rel_err": float(f"{err:.3e}"),
    }
    if cpu_seconds > 0:
        oracle.lib()
        calls, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds / 2:
            oracle.expert_forward(tensors, kinds, x, H, I, 0, True)
            calls += 1
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(dt / calls * 1e6, 1), "unit": "us", "cores": 1, "kind": "port",
                               "sample": f"{calls} calls of the AVX2 moe_quant_expert port (FP32 graph), one thread, "
                                         f"{dt:.1f} s"}
    del layers
    torch.cuda.empty_cache()
    return out


def bench_reference_callers(dev, reps: int) -> dict:
    """The paths a caller of the reference's Python API takes without edits,
    timed on the host clock (each call stages host buffers over PCIe and
    synchronises): NativeExpert.forward (native_expert.py:23-37; the config-1
    Q4_K expert's 1.77 MB of host bytes staged per call, FP32 graph since the
    FP16 graph overflows on those scales), and run_moe_layer
    (moe_layer.py:39-107) over HipExpertBackend with resident weights, through
    the backend's fused hook and through forward() fanned out on its 4-worker
    executor, on the headline layer shape in the reference decode's FP16 graph
    (scales of the reference's FP16-graph check, d ~ 0.002, x ~ 0.05).  These
    are PCIe- and host-inclusive latencies, not kernel throughput."""
    import torch

    import oracle
    from flash_moe_hip.backend import HipExpertBackend
    from flash_moe_hip.layer_store import ExpertLayer
    from flash_moe_hip.moe_layer import run_moe_layer
    from flash_moe_hip.native_expert import NativeExpert
    from flash_moe_hip.shared_expert import SharedExpert
    from flash_moe_hip.synthetic import config1_expert

    def per_call_us(fn, n):
        fn()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        return round((time.perf_counter() - t0) / n * 1e6, 1)

    tensors, kinds, x = config1_expert(0)
    native = NativeExpert()
    native.fp16_graph = 0
    err_native = oracle.max_relative_error(native.forward(tensors, kinds, x, H, I),
                                           oracle.expert_forward(tensors, kinds, x, H, I, 0))
    us_native = per_call_us(lambda: native.forward(tensors, kinds, x, H, I), reps)

    layer = ExpertLayer.synthetic(TYPES, E, H, I, seed=31, shared_types=TYPES, shared_intermediate=I,
                                  gate_inp=True, scale=0.002, device=dev)
    rng = np.random.default_rng(31)
    W = (rng.standard_normal((H, E)) * 0.02).astype(np.float32)
    xs = [(rng.standard_normal(H) * 0.05).astype(np.float32) for _ in range(8)]

    class Router:
        top_k = K

        def route(self, v):
            return oracle.route(v, W, K)

    class ProtocolOnly:   # the attributes a reference backend has (no fused hook)
        def __init__(self, b):
            self._b, self.store, self._moe_executor = b, b.store, b._moe_executor

        def forward(self, *a):
            return self._b.forward(*a)

    backend = HipExpertBackend({0: layer})
    try:
        sh = SharedExpert.from_backend(backend)
        router = Router()
        res = {}
        for name, b in (("fused_hook", backend), ("forward_fan_out", ProtocolOnly(backend))):
            i = [0]

            def one(b=b):
                i[0] += 1
                return run_moe_layer(0, xs[i[0] % len(xs)], router, b, H, I, shared_expert=sh)

            res[name] = per_call_us(one, max(4, reps // 4))
        torch.cuda.synchronize()
    finally:
        backend.close()
    log(f"reference callers: NativeExpert.forward {us_native} us, run_moe_layer fused {res['fused_hook']} us, "
        f"forward fan-out {res['forward_fan_out']} us")
    del layer
    torch.cuda.empty_cache()
    return {
        "workload": "the reference's Python entry points unchanged: NativeExpert.forward on one Q4_K expert "
                    "(host bytes, staged per call) and run_moe_layer over HipExpertBackend (resident weights, "
                    "host x, host routing) on the headline layer shape in the FP16 graph",
        "metric": "us per call, host clock (PCIe- and synchronisation-inclusive)",
        "higher_is_better": False,
        "native_expert_forward_us": us_native, "native_expert_parity_max_rel_err": float(f"{err_native:.3e}"),
        "run_moe_layer_fused_hook_us": res["fused_hook"],
        "run_moe_layer_forward_fan_out_us": res["forward_fan_out"],
    }


def bench_deltanet(dev, reps: int, cpu_seconds: float) -> dict:
    """The DeltaNet decode recurrence (moe_delta_heads) of the reference model's
    recurrent layers: 30 layers, each a [32 heads x 128 x 128] FP32 state
    (2 MiB) resident in HBM, one step per layer per token, all 30 captured as
    one graph and replayed.  Bytes per step: the state read and written
    (4 MiB); q, k, v, beta, gate are a few KiB."""
    import torch

    import oracle
    from flash_moe_hip.native_expert import DeltaState

    NL, NV, DV, DK = 30, 32, 128, 128
    rng = np.random.default_rng(5)
    host0 = (rng.standard_normal((NV, DV, DK)) * 0.01).astype(np.float32)
    states = [DeltaState(NV, DV, DK, device=dev, state=host0 if l == 0 else
                         (rng.standard_normal((NV, DV, DK)) * 0.01).astype(np.float32)) for l in range(NL)]
    hins = []
    for _ in range(NL):
        hins.append(((rng.standard_normal((NV, DK)) * 0.05).astype(np.float32),
                     (rng.standard_normal((NV, DK)) * 0.05).astype(np.float32),
                     (rng.standard_normal((NV, DV)) * 0.1).astype(np.float32),
                     rng.uniform(0.01, 0.99, NV).astype(np.float32),
                     (-rng.uniform(0.001, 5, NV)).astype(np.float32)))
    ins = [[torch.from_numpy(a).to(dev) for a in h] for h in hins]
    outs = torch.empty((NL, NV, DV), dtype=torch.float32, device=dev)
    # parity: one step of layer 0 against the oracle, bit for bit
    states[0].step(*ins[0], out=outs[0])
    torch.cuda.synchronize()
    ref_state = host0.copy()
    rc, want = oracle.delta_heads(ref_state, *hins[0])
    exact = bool(rc == 0 and np.array_equal(outs[0].cpu().numpy(), want)
                 and np.array_equal(states[0].state.cpu().numpy(), ref_state))

    def sweep():
        for l in range(NL):
            states[l].step(*ins[l], out=outs[l])

    ms = _time(_graph(sweep, dev), reps) / NL
    kus = _delta_kernel_us(states, ins, outs, 4)
    assert all(s.status() == 0 for s in states)
    nbytes = 2 * NV * DV * DK * 4
    log(f"deltanet: {ms * 1e3:.2f} us per layer step, kernel {kus:.2f} us, bit-exact {exact}")
    out = {
        "workload": f"DeltaNet decode step (moe_delta_heads): {NV} heads x {DV} x {DK} FP32 state per layer, "
                    f"{NL} recurrent layers resident and rotated, one step per layer",
        "metric": "state GB/s per layer step (state read + written)",
        "value": round(nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "us_per_layer": round(ms * 1e3, 3),
        "bit_exact_vs_oracle": exact,
        "roofline": _hbm_roofline("mqh::k_delta_heads<16>", nbytes, kus, read_floor_us(nbytes)),
    }
    if cpu_seconds > 0:
        L = oracle.reference_delta_lib()
        kind = "reference" if L is not None else "port"
        fn = oracle.reference_delta_heads if L is not None else oracle.delta_heads
        st = host0.copy()
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds:
            fn(st, *hins[done % NL])
            done += 1
        dt = time.perf_counter() - t0
        per = dt / done
        out["cpu_baseline"] = {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
                               "us_per_layer": round(per * 1e6, 1),
                               "sample": f"{done} steps of one [{NV}x{DV}x{DK}] state in {dt:.1f} s, one thread "
                                         f"({'the reference kernel built from cpp/moe_delta.cpp' if L else 'the oracle'})"}
    del states, ins, outs
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch every step from Python instead of a graph")
    ap.add_argument("--only-decode", action="store_true", help="skip the batched-decode, prefill and dequant lines")
    # single_expert (one Q4_K expert, one token) runs the headline's gate/up kernel
    # instance: a profile of the headline kernels leaves it out (--workloads)
    ap.add_argument("--workloads", default="single_expert,fp16_graph_decode,decode_reference_mixes,batched_decode,"
                                           "prefill,prefill_q3k_q6k_shared,dequant,deltanet,reference_callers",
                    help="comma-separated workloads run after the headline decode")
    ap.add_argument("--extra-cpu-seconds", type=float, default=4.0)
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="run one device-to-device copy of this many MiB first (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: there is no multi-GPU path (the experts would shard by "
              "expert, one reduce per layer); run with --gpus 1", file=sys.stderr)
        return 1

    import torch

    from flash_moe_hip.moe_gpu import MoeRunner

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}; building {args.layers} resident layers")
    layers = build_layers(args.layers, dev)
    xs, ids, ws = route_layers(args.layers, layers=layers)
    resident_gb = sum(L.resident_bytes() for L in layers) / 1e9
    log(f"resident expert bytes {resident_gb:.2f} GB")
    X = torch.from_numpy(xs).to(dev)
    IDS = torch.from_numpy(ids).to(dev)
    WS = torch.from_numpy(ws).to(dev)
    Y = torch.empty((args.layers, H), dtype=torch.float32, device=dev)
    runner = MoeRunner(dev)

    def sweep(n=args.layers, start=0):
        for l in range(start, start + n):
            l %= args.layers
            runner.decode(layers[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1])

    # eager warm-up (allocates the workspace), parity spot check on four layers
    sweep()
    torch.cuda.synchronize()
    assert runner.status() == 0, "kernel fault during warm-up"
    Yh = Y.cpu().numpy()
    check = sorted({0, args.layers // 3, 2 * args.layers // 3, args.layers - 1})
    err = max(parity_check(layers[l], xs[l], ids[l], ws[l], Yh[l]) for l in check)
    log(f"parity vs oracle (layers {check}): max rel err {err:.3e}")
    if not err <= 1e-3:
        log("PARITY FAILURE")
        return 3

    if args.calib_copy_mb:
        n = args.calib_copy_mb << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy of {n} bytes done")
        del src, dst

    # exactly `warmup` untimed and then exactly `steps` timed steps: a step is
    # one token through one layer; layer l of step i is i % layers, as the
    # graph of one whole sweep replayed plus a graph of the first
    # (steps % layers) layers
    run_steps = StepRunner(sweep, args.layers, dev, eager=args.eager)
    run_steps(args.warmup)
    torch.cuda.synchronize()
    ms_total = run_steps.timed(args.steps)
    assert runner.status() == 0, "kernel fault during timing"
    steps = args.steps
    ms_step = ms_total / steps
    nbytes = step_bytes(layers[0])
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    log(f"{steps} steps in {ms_total:.2f} ms: {ms_step * 1e3:.2f} us/layer, {gbs:.1f} GB/s")

    # graph result must equal the eager result
    y_graph = Y[0].cpu().numpy()
    err_graph = parity_check(layers[0], xs[0], ids[0], ws[0], y_graph)

    # per-kernel durations: every step of an eager pass over the same layers,
    # each kernel bracketed by HIP events recorded by the runtime at its
    # start and end (mqh_profile_next_decode), on the stream it runs on
    kern = kernel_times(runner, layers, X, IDS, WS, Y, reps=10)
    log(f"kernel A (gate/up) {kern['a_us']:.3f} us, kernel B (down+combine) {kern['b_us']:.3f} us per launch")
    kernels_us = {"k_fast_gate_up": round(kern["a_us"], 3), "k_fast_down": round(kern["b_us"], 3),
                  "launches_each": kern["launches"], "statistic": "median over launches",
                  "mean": {"k_fast_gate_up": round(kern["a_mean_us"], 3), "k_fast_down": round(kern["b_mean_us"], 3)}}
    # each kernel against a plain streaming read of its own byte count
    a_bytes = (K + 1) * (layers[0].expert_bytes("gate") + layers[0].expert_bytes("up"))
    b_bytes = (K + 1) * layers[0].expert_bytes("down")
    floors = {}
    for kname, nb, kus in (("k_fast_gate_up", a_bytes, kern["a_us"]), ("k_fast_down", b_bytes, kern["b_us"])):
        f_us = read_floor_us(nb)
        floors[kname] = {"algorithmic_bytes": nb, "kernel_us": round(kus, 3), "read_floor_us": round(f_us, 3),
                         "frac_of_read_floor": round(f_us / kus, 4)}
    log("read floors: " + ", ".join(f"{k} {v['read_floor_us']:.3f} us ({v['frac_of_read_floor']:.2f})"
                                    for k, v in floors.items()))

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 accumulate; activations as two int8 digits per 16 columns, exact int32 dot products "
                 "with the 4/6-bit weights",
        "data": "synthetic",
        "config": {
            "workload": "decode MoE layer, 1 token: hidden 2048, 256 experts x intermediate 512, top-8 + "
                        "1 shared expert (sigmoid-gated), gate/up Q4_K, down Q6_K, FP32 router; "
                        f"{args.layers} resident layers rotated",
            "weight_bytes_per_step": nbytes,
            "resident_gb": round(resident_gb, 2),
        },
        "us_per_layer": round(ms_step * 1e3, 3),
        "parity_max_rel_err": float(f"{max(err, err_graph):.3e}"),
        "kernels_us": kernels_us,
        "kernels_read_floor": floors,
        "roofline": roofline(kern, layers[0], floor=read_floor_us),
    }
    result["routed_decode"] = bench_routed_decode(runner, layers, X, ids, ws, 20, dev)
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle, 4 threads)")
        result["cpu_baseline"] = cpu_baseline(layers, xs, ids, ws, args.cpu_seconds)
    if not args.only_decode:
        del layers, run_steps
        torch.cuda.empty_cache()
        cpu_s = 0.0 if args.no_cpu_baseline else args.extra_cpu_seconds
        wanted = set(args.workloads.split(","))
        runs = {
            "single_expert": lambda: bench_single_expert(dev, 50, cpu_s),
            "fp16_graph_decode": lambda: bench_fp16_graph_decode(dev, args.layers, 20, cpu_s),
            "decode_reference_mixes": lambda: bench_decode_mixes(dev, args.layers, 20),
            "batched_decode": lambda: bench_batched_decode(dev, args.layers, 25 * args.layers, cpu_s),
            "prefill": lambda: bench_prefill(dev, 8, 20, cpu_s),
            # the reference model's layers 5-34 (docs/PHASE0_FINDINGS.md:60-69)
            "prefill_q3k_q6k_shared": lambda: bench_prefill(
                dev, 8, 20, cpu_s, types={"gate": 11, "up": 11, "down": 11},
                shared_types={"gate": 14, "up": 14, "down": 14},
                what="every routed matrix Q3_K, the shared expert Q6_K (the reference model's layers 5-34)"),
            "dequant": lambda: bench_dequant(dev, 10, cpu_s),
            "deltanet": lambda: bench_deltanet(dev, 50, cpu_s),
            "reference_callers": lambda: bench_reference_callers(dev, 40),
        }
        result["workloads"] = {name: run() for name, run in runs.items() if name in wanted}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
