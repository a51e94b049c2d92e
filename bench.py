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

cpu_baseline: the CPU oracle (a restatement of the reference's AVX2 kernel)
running the same layer as 9 moe_quant_expert calls on 4 worker threads -- the
reference's expert-worker policy -- on the host cores, for a bounded sample.

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


def route_layers(n_layers: int, seed: int = 0):
    """Per layer: x ~ N(0,1) [H]; router W ~ N(0, 0.02) [H x E]; top-8 ids and
    softmax weights with the reference router's semantics."""
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
    return np.stack(xs), np.stack(ids), np.stack(ws)


def step_bytes(layer) -> int:
    return (K + 1) * layer.bytes_per_expert()


def roofline(kern: dict, layer) -> dict:
    """The dominant kernel (the larger average duration) against HBM peak.
    Algorithmic bytes per launch: the quantized weight bytes it must read --
    kernel A the gate and up slices of the 9 experts, kernel B their down
    slices -- plus activations in and out (a few KB)."""
    a_bytes = (K + 1) * (layer.expert_bytes("gate") + layer.expert_bytes("up"))
    b_bytes = (K + 1) * layer.expert_bytes("down")
    if kern["a_us"] >= kern["b_us"]:
        name, nbytes, us = "k_fast_gate_up", a_bytes, kern["a_us"]
    else:
        name, nbytes, us = "k_fast_down", b_bytes, kern["b_us"]
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": name,
            "algorithmic_bytes": nbytes, "kernel_us": round(us, 3)}


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

    def one_step(job):
        experts, x, w = job
        outs = [oracle.expert_forward(t, TYPES, x, H, I, 0) for t in experts[:K]]
        return oracle.combine(outs, [float(v) for v in w], oracle.expert_forward(experts[K], TYPES, x, H, I, 0))

    def one_step_parallel(pool, job):
        experts, x, w = job
        futs = [pool.submit(oracle.expert_forward, t, TYPES, x, H, I, 0) for t in experts]
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
    return {
        "value": round(step_bytes(layers[0]) / per_step / 1e9, 3),
        "unit": "GB/s",
        "cores": workers,
        "kind": "port",
        "sample": f"{steps} token-layers (9 expert calls each, FP32 graph) over {n_src} layers, "
                  f"{dt:.1f} s on {workers} threads; host has {os.cpu_count()} logical CPUs",
        "us_per_layer": round(per_step * 1e6, 1),
    }


def _hip_runtime():
    """The process's HIP runtime (the one torch and the library already share)."""
    import ctypes as C

    rt = C.CDLL("libamdhip64.so.7")
    rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    rt.hipEventDestroy.argtypes = [C.c_void_p]
    return rt


def kernel_times(runner, layers, X, IDS, WS, Y, reps: int) -> dict:
    """Average duration of each decode kernel: an eager pass of reps x layers
    steps, every kernel launched with start/stop HIP events."""
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
        runner.decode(layers[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1], stream=stream)
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
    return {"a_us": float(np.mean(a)), "b_us": float(np.mean(b)), "launches": n,
            "a_us_median": float(np.median(a)), "b_us_median": float(np.median(b))}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch every step from Python instead of a graph")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="run one device-to-device copy of this many MiB first (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(see DESIGN.md for how the experts would shard); run with --gpus 1", file=sys.stderr)
        return 1

    import torch

    from flash_moe_hip.moe_gpu import MoeRunner

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}; building {args.layers} resident layers")
    layers = build_layers(args.layers, dev)
    xs, ids, ws = route_layers(args.layers)
    resident_gb = sum(L.resident_bytes() for L in layers) / 1e9
    log(f"resident expert bytes {resident_gb:.2f} GB")
    X = torch.from_numpy(xs).to(dev)
    IDS = torch.from_numpy(ids).to(dev)
    WS = torch.from_numpy(ws).to(dev)
    Y = torch.empty((args.layers, H), dtype=torch.float32, device=dev)
    runner = MoeRunner(dev)

    def sweep():
        for l in range(args.layers):
            runner.decode(layers[l], X[l:l + 1], IDS[l:l + 1], WS[l:l + 1], y=Y[l:l + 1])

    # eager warm-up (allocates the workspace), parity spot check on layer 0
    sweep()
    torch.cuda.synchronize()
    assert runner.status() == 0, "kernel fault during warm-up"
    err = parity_check(layers[0], xs[0], ids[0], ws[0], Y[0].cpu().numpy())
    log(f"parity vs oracle (layer 0): max rel err {err:.3e}")
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

    reps_w = max(1, args.warmup // args.layers)
    reps = max(1, args.steps // args.layers)
    if args.eager:
        run_sweep = sweep
    else:
        # capture one sweep over all layers as a graph
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream(dev)
        cap.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(cap):
            sweep()
        torch.cuda.current_stream(dev).wait_stream(cap)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            sweep()
        run_sweep = graph.replay
    for _ in range(reps_w):
        run_sweep()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        run_sweep()
    end.record()
    end.synchronize()
    assert runner.status() == 0, "kernel fault during timing"
    steps = reps * args.layers
    ms_total = start.elapsed_time(end)
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
    kern = kernel_times(runner, layers, X, IDS, WS, Y, reps=max(1, min(reps, 10)))
    log(f"kernel A (gate/up) {kern['a_us']:.3f} us, kernel B (down+combine) {kern['b_us']:.3f} us per launch")

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": reps_w * args.layers,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
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
        "kernels_us": {"k_fast_gate_up": round(kern["a_us"], 3), "k_fast_down": round(kern["b_us"], 3),
                       "launches_each": kern["launches"]},
        "roofline": roofline(kern, layers[0]),
    }
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle, 4 threads)")
        result["cpu_baseline"] = cpu_baseline(layers, xs, ids, ws, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
