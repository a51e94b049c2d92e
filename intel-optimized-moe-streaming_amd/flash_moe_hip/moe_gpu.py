"""Device-resident fused MoE calls (thin wrapper over the mqh_* C ABI).

``MoeRunner.decode(layer, x, ids, weights)`` enqueues the fused GEMV kernels
for every routed expert of every token plus the layer's shared expert;
``MoeRunner.prefill(...)`` the grouped-GEMM kernels for a prompt (tokens
bucketed per expert on the device).  Nothing is synchronized.
``MoeRunner.status()`` synchronizes and returns the fault status latched by
the kernels (0, -4 non-finite, -9 bad expert id).

Threads.  The reference fans one token's experts out over a thread pool
(``moe_layer.py:74-94``), so one runner is called from several threads at
once.  Every calling thread gets a workspace of its own (activations and
fault flags), so concurrent calls never share scratch memory, and ``status()``
reports the faults of the calling thread's calls only.
"""
from __future__ import annotations

import threading

import numpy as np

from . import _lib
from .layer_store import ExpertLayer

_NULL = None

# shapes and types the grouped prefill kernels are built for: gate/up in the
# K-quants, down also Q8_0 (the reference model's first-layer down projection)
PREFILL_TYPES = (11, 12, 13, 14)
PREFILL_DOWN_TYPES = PREFILL_TYPES + (8,)
PREFILL_DIMS = (256, 512, 1024, 2048)
PREFILL_MAX_EXPERTS = 1024
Q6_K = 14


class MoeRunner:
    """Owns the workspaces of the fused kernels on one device (one per calling thread)."""

    def __init__(self, device=None):
        import torch

        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.lib = _lib.load()
        self._local = threading.local()

    @property
    def _ws(self):
        return getattr(self._local, "ws", None)

    def pinned(self, slot: str, nbytes: int):
        """The calling thread's pinned host buffer `slot` (uint8, at least
        `nbytes`, grown on demand and kept): host-staged calls reuse it
        instead of allocating pinned memory per call, which costs hundreds of
        microseconds each time.  The caller must have finished with the
        previous contents (every host-staged call synchronizes before
        returning)."""
        import torch

        buf = getattr(self._local, "pin_" + slot, None)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(int(nbytes), 1 << 16), dtype=torch.uint8, pin_memory=True)
            setattr(self._local, "pin_" + slot, buf)
        return buf[:nbytes]

    def upload(self, arrays, slot: str = "stage", stream=None):
        """Copy host arrays to the device through the calling thread's pinned
        buffer `slot`: one host-to-device copy, enqueued on `stream`; returns
        the device views (uint8 flat, in order).  Waits first for this slot's
        previous copy, so a call that raised before synchronizing cannot have
        its buffer overwritten under a copy in flight."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        prev = getattr(self._local, "ev_" + slot, None)
        if prev is not None:
            prev.synchronize()
        raws = [np.ascontiguousarray(a).reshape(-1).view(np.uint8) for a in arrays]
        offs, n = [], 0
        for r in raws:
            offs.append(n)
            n += (r.size + 15) & ~15
        host = self.pinned(slot, n)
        h = host.numpy()
        for r, o in zip(raws, offs):
            h[o:o + r.size] = r
        with torch.cuda.stream(stream):
            dev = host.to(self.device, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(stream)
        setattr(self._local, "ev_" + slot, ev)
        return [dev[o:o + r.size] for r, o in zip(raws, offs)]

    def _workspace(self, n_tokens: int, top_k: int, inter: int, sh_inter: int, stream):
        need = int(self.lib.mqh_moe_workspace_bytes(n_tokens, top_k, inter, sh_inter))
        if need < 0:
            _lib.check(need, "mqh_moe_workspace_bytes")
        return self._reserve(need, stream)

    def _reserve(self, need: int, stream):
        """The calling thread's workspace, grown to at least `need` bytes.  A
        new buffer is zeroed (its flag words) before it replaces the old one;
        the old one's latched faults are raised first."""
        import torch

        ws = self._ws
        if ws is None or need > ws.numel():
            size = max(need, 2 * ws.numel()) if ws is not None else need
            if ws is not None:
                _lib.check(self.lib.mqh_status(ws.data_ptr(), stream.cuda_stream), "pending kernel")
            new = torch.empty(size, dtype=torch.uint8, device=self.device)
            _lib.check(self.lib.mqh_workspace_init(new.data_ptr(), new.numel(), stream.cuda_stream),
                       "mqh_workspace_init")
            self._local.ws = new
            ws = new
        return ws

    def decode(self, layer: ExpertLayer, x, ids=None, weights=None, *, y=None, fp16_graph: int = 0,
               use_shared: bool = True, stream=None):
        """y[t] = sum_s weights[t,s] * E_ids[t,s](x[t]) (+ shared).  x [T,H] FP32,
        ids [T,k] int32, weights [T,k] FP32, all CUDA tensors on the layer's device."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        x = x.reshape(-1, layer.hidden)
        T = x.shape[0]
        if x.dtype != torch.float32 or not x.is_contiguous():
            raise ValueError("x must be contiguous FP32")
        top_k = 0 if ids is None else int(ids.shape[-1])
        if top_k:
            ids = ids.reshape(T, top_k)
            weights = weights.reshape(T, top_k)
            if ids.dtype != torch.int32 or weights.dtype != torch.float32:
                raise ValueError("ids must be int32 and weights FP32")
            if not (ids.is_contiguous() and weights.is_contiguous()):
                raise ValueError("ids and weights must be contiguous")
        sh = layer.shared if use_shared else None
        if y is None:
            y = torch.empty((T, layer.hidden), dtype=torch.float32, device=x.device)
        if T == 0:
            return y
        ws = self._workspace(T, top_k, layer.intermediate if top_k else 0, sh.intermediate if sh else 0, stream)
        t = layer.tensors
        rc = self.lib.mqh_moe_decode(
            layer.types["gate"], t["gate"].data_ptr(), layer.types["up"], t["up"].data_ptr(),
            layer.types["down"], t["down"].data_ptr(), layer.n_experts, layer.hidden, layer.intermediate,
            sh.types["gate"] if sh else 0, sh.gate.data_ptr() if sh else _NULL,
            sh.types["up"] if sh else 0, sh.up.data_ptr() if sh else _NULL,
            sh.types["down"] if sh else 0, sh.down.data_ptr() if sh else _NULL,
            sh.intermediate if sh else 0,
            sh.gate_inp.data_ptr() if (sh is not None and sh.gate_inp is not None) else _NULL,
            x.data_ptr(), T, ids.data_ptr() if top_k else _NULL, weights.data_ptr() if top_k else _NULL, top_k,
            y.data_ptr(), int(fp16_graph), ws.data_ptr(), ws.numel(), stream.cuda_stream)
        _lib.check(rc, "mqh_moe_decode")
        return y

    def decode_shared(self, shared, hidden: int, x, *, y=None, stream=None):
        """y[t] = sigmoid(x[t] . gate_inp) * E_sh(x[t]) for a shared expert on
        its own (``SharedWeights``: no routed experts), x [T, hidden] FP32."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        x = x.reshape(-1, hidden)
        T = x.shape[0]
        if x.dtype != torch.float32 or not x.is_contiguous():
            raise ValueError("x must be contiguous FP32")
        if y is None:
            y = torch.empty((T, hidden), dtype=torch.float32, device=x.device)
        if T == 0:
            return y
        ws = self._workspace(T, 0, 0, shared.intermediate, stream)
        sh = shared
        rc = self.lib.mqh_moe_decode(
            0, _NULL, 0, _NULL, 0, _NULL, 0, hidden, 0,
            sh.types["gate"], sh.gate.data_ptr(), sh.types["up"], sh.up.data_ptr(),
            sh.types["down"], sh.down.data_ptr(), sh.intermediate,
            sh.gate_inp.data_ptr() if sh.gate_inp is not None else _NULL,
            x.data_ptr(), T, _NULL, _NULL, 0, y.data_ptr(), 0, ws.data_ptr(), ws.numel(), stream.cuda_stream)
        _lib.check(rc, "mqh_moe_decode")
        return y

    def route(self, layer: ExpertLayer, x, top_k: int, *, router_w=None, ids=None, weights=None, scores=None,
              stream=None):
        """Top-k routing on the device (``ExpertRouter.route``, router.py:140-170):
        x [T,H] FP32; router_w [E,H] FP32, one row per expert as the GGUF file
        stores ffn_gate_inp (default: the layer's router weights).  Returns
        (ids [T,k] int32, weights [T,k] FP32) in descending score order; the
        FP32 scores [T,E] land in ``scores`` when given."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        w = layer.router_device() if router_w is None else router_w
        x = x.reshape(-1, layer.hidden)
        T = x.shape[0]
        if x.dtype != torch.float32 or not x.is_contiguous():
            raise ValueError("x must be contiguous FP32")
        if w.dtype != torch.float32 or not w.is_contiguous() or tuple(w.shape) != (layer.n_experts, layer.hidden):
            raise ValueError(f"router weights must be contiguous FP32 [{layer.n_experts}, {layer.hidden}]")
        if ids is None:
            ids = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
        if weights is None:
            weights = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
        if scores is None:
            scores = torch.empty((T, layer.n_experts), dtype=torch.float32, device=x.device)
        if T == 0:
            return ids, weights
        rc = self.lib.mqh_route(x.data_ptr(), T, layer.hidden, w.data_ptr(), layer.n_experts, int(top_k),
                                scores.data_ptr(), ids.data_ptr(), weights.data_ptr(), stream.cuda_stream)
        _lib.check(rc, "mqh_route")
        return ids, weights

    def decode_routed(self, layer: ExpertLayer, x, top_k: int, *, router_w=None, y=None, ids=None, weights=None,
                      scores=None, use_shared: bool = True, stream=None):
        """The layer with its routing on the device (mqh_moe_decode_routed): the
        router scores, top-k and softmax of ``route`` followed by ``decode``, in
        one call; with at most 256 experts and the fast kernels the top-k runs
        inside the gate/up kernel.  Returns (y, ids, weights)."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        w = layer.router_device() if router_w is None else router_w
        x = x.reshape(-1, layer.hidden)
        T = x.shape[0]
        if x.dtype != torch.float32 or not x.is_contiguous():
            raise ValueError("x must be contiguous FP32")
        if w.dtype != torch.float32 or not w.is_contiguous() or tuple(w.shape) != (layer.n_experts, layer.hidden):
            raise ValueError(f"router weights must be contiguous FP32 [{layer.n_experts}, {layer.hidden}]")
        dev = x.device
        if ids is None:
            ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
        if weights is None:
            weights = torch.empty((T, top_k), dtype=torch.float32, device=dev)
        if scores is None:
            scores = torch.empty((T, layer.n_experts), dtype=torch.float32, device=dev)
        if y is None:
            y = torch.empty((T, layer.hidden), dtype=torch.float32, device=dev)
        if T == 0:
            return y, ids, weights
        sh = layer.shared if use_shared else None
        ws = self._workspace(T, top_k, layer.intermediate, sh.intermediate if sh else 0, stream)
        t = layer.tensors
        rc = self.lib.mqh_moe_decode_routed(
            layer.types["gate"], t["gate"].data_ptr(), layer.types["up"], t["up"].data_ptr(),
            layer.types["down"], t["down"].data_ptr(), layer.n_experts, layer.hidden, layer.intermediate,
            sh.types["gate"] if sh else 0, sh.gate.data_ptr() if sh else _NULL,
            sh.types["up"] if sh else 0, sh.up.data_ptr() if sh else _NULL,
            sh.types["down"] if sh else 0, sh.down.data_ptr() if sh else _NULL,
            sh.intermediate if sh else 0,
            sh.gate_inp.data_ptr() if (sh is not None and sh.gate_inp is not None) else _NULL,
            x.data_ptr(), T, w.data_ptr(), int(top_k), scores.data_ptr(), ids.data_ptr(), weights.data_ptr(),
            y.data_ptr(), 0, ws.data_ptr(), ws.numel(), stream.cuda_stream)
        _lib.check(rc, "mqh_moe_decode_routed")
        return y, ids, weights

    @staticmethod
    def prefill_supported(layer: ExpertLayer) -> bool:
        """Whether the grouped prefill kernels cover this layer's routed experts."""
        t = layer.types
        return (t["gate"] == t["up"] and t["gate"] in PREFILL_TYPES and t["down"] in PREFILL_DOWN_TYPES
                and layer.hidden in PREFILL_DIMS and layer.intermediate in PREFILL_DIMS
                and layer.n_experts <= PREFILL_MAX_EXPERTS)

    @staticmethod
    def _shared_in_prefill(layer: ExpertLayer) -> bool:
        """Whether the layer's shared expert runs inside the grouped kernels:
        the routed intermediate size, gate type == up type, each role the
        routed type or Q6_K (the reference model's Q6_K shared experts)."""
        sh = layer.shared
        if sh is None or sh.intermediate != layer.intermediate:
            return False
        st, t = sh.types, layer.types
        return (st["gate"] == st["up"] and st["gate"] in (t["gate"], Q6_K) and st["down"] in (t["down"], Q6_K))

    def prefill(self, layer: ExpertLayer, x, ids, weights, *, y=None, use_shared: bool = True, stream=None):
        """The layer for a prompt: x [T,H] FP32 or BF16, ids [T,k] int32, weights
        [T,k] FP32 (CUDA tensors).  Same result as ``decode`` up to FP32
        summation order inside each dot product.  The shared expert runs inside
        the grouped kernels when it has the routed size and, per role, the
        routed type or Q6_K; any other shared expert runs through the decode
        kernels and is added after the routed sum, as in run_moe_sequence."""
        import torch

        if not self.prefill_supported(layer):
            raise ValueError("the grouped prefill kernels do not cover this layer's types or shape")
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        x = x.reshape(-1, layer.hidden)
        T = x.shape[0]
        if x.dtype not in (torch.float32, torch.bfloat16) or not x.is_contiguous():
            raise ValueError("x must be contiguous FP32 or BF16")
        top_k = int(ids.shape[-1])
        ids = ids.reshape(T, top_k)
        weights = weights.reshape(T, top_k)
        if ids.dtype != torch.int32 or weights.dtype != torch.float32:
            raise ValueError("ids must be int32 and weights FP32")
        if not (ids.is_contiguous() and weights.is_contiguous()):
            raise ValueError("ids and weights must be contiguous")
        sh = layer.shared if use_shared else None
        inside = sh is not None and self._shared_in_prefill(layer)
        if y is None:
            y = torch.empty((T, layer.hidden), dtype=torch.float32, device=x.device)
        if T == 0:
            return y
        need = int(self.lib.mqh_moe_prefill_workspace_bytes(T, top_k, layer.n_experts, layer.hidden,
                                                           layer.intermediate, int(inside)))
        if need < 0:
            _lib.check(need, "mqh_moe_prefill_workspace_bytes")
        ws = self._reserve(need, stream)
        t = layer.tensors
        rc = self.lib.mqh_moe_prefill(
            layer.types["gate"], t["gate"].data_ptr(), layer.types["up"], t["up"].data_ptr(),
            layer.types["down"], t["down"].data_ptr(), layer.n_experts, layer.hidden, layer.intermediate,
            sh.types["gate"] if inside else 0, sh.gate.data_ptr() if inside else _NULL,
            sh.types["up"] if inside else 0, sh.up.data_ptr() if inside else _NULL,
            sh.types["down"] if inside else 0, sh.down.data_ptr() if inside else _NULL,
            sh.intermediate if inside else 0,
            sh.gate_inp.data_ptr() if (inside and sh.gate_inp is not None) else _NULL,
            x.data_ptr(), int(x.dtype == torch.bfloat16), T, ids.data_ptr(), weights.data_ptr(), top_k,
            y.data_ptr(), ws.data_ptr(), ws.numel(), stream.cuda_stream)
        _lib.check(rc, "mqh_moe_prefill")
        if sh is not None and not inside:
            y += self.decode(layer, x.float(), None, None, use_shared=True, stream=stream)
        return y

    def status(self, stream=None) -> int:
        """Synchronize `stream` and return (and clear) the faults latched by
        the calling thread's calls."""
        import torch

        ws = self._ws
        if ws is None:
            return 0
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        return int(self.lib.mqh_status(ws.data_ptr(), stream.cuda_stream))

    def fetch(self, y, stream=None):
        """(y as a NumPy array, status) with one synchronisation: y and the
        calling thread's fault flags are copied to the host together; the flags
        are cleared (a second synchronisation) only when a fault was latched."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        ws = self._ws
        nbytes = y.numel() * y.element_size()
        host = self.pinned("fetch", nbytes + 8)
        with torch.cuda.stream(stream):
            out = host[:nbytes].view(y.dtype).view(y.shape)
            out.copy_(y, non_blocking=True)
            flags = None
            if ws is not None:
                flags = host[nbytes:nbytes + 8].view(torch.int32)
                flags.copy_(ws[:8].view(torch.int32), non_blocking=True)
        stream.synchronize()
        rc = 0
        if flags is not None and bool(flags.any()):
            rc = int(self.lib.mqh_status(ws.data_ptr(), stream.cuda_stream))
        return out.numpy().copy(), rc
