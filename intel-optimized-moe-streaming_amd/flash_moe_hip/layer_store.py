"""HBM-resident expert layers.

A layer keeps each expert role (gate, up, down) as ONE stacked uint8 tensor of
``n_experts`` consecutive GGUF slices, exactly as the GGUF ``*_exps`` tensor
lays them out (expert e's slice starts at ``e * (n_bytes // n_experts)``,
``src/run_q4k_f16_openvino.py:112-122``).  The kernels index experts through
this layout, so no per-expert copies or pointer tables exist.  The optional
shared expert (``ffn_{gate,up,down}_shexp`` + ``ffn_gate_inp_shexp``) sits
beside it.  On a 288 GB MI355X a whole 40-layer, 256-expert model of this
shape (~21 GB) stays resident, so the reference's disk streaming (its L2 store
and prefetch windows) has no counterpart here.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .quant_types import DECODE_TYPES, Q3_K_A112, name_of, pad_blocks, tensor_bytes

ROLES = ("gate", "up", "down")


def _shape(role: str, hidden: int, intermediate: int) -> tuple[int, int]:
    return (intermediate, hidden) if role in ("gate", "up") else (hidden, intermediate)


def _to_device_bytes(raw, device):
    import torch

    if isinstance(raw, torch.Tensor):
        t = raw.to(device=device, dtype=torch.uint8).contiguous().view(-1)
        return t
    arr = np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) else \
        np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    return torch.from_numpy(arr.copy()).to(device)


@dataclass
class SharedWeights:
    gate: object
    up: object
    down: object
    types: dict
    intermediate: int
    gate_inp: object | None = None   # FP32 [hidden] sigmoid gate vector, or None


class ExpertLayer:
    """One MoE layer's expert tensors in HBM."""

    def __init__(self, gate, up, down, types: dict, n_experts: int, hidden: int, intermediate: int,
                 shared: SharedWeights | None = None, router_weights=None):
        import torch

        self.types = {r: int(types[r]) for r in ROLES}
        for r in ROLES:
            if self.types[r] not in DECODE_TYPES:
                raise ValueError(f"{r}: unsupported ggml type {self.types[r]}")
        self.n_experts, self.hidden, self.intermediate = int(n_experts), int(hidden), int(intermediate)
        self.tensors = {"gate": gate, "up": up, "down": down}
        for r in ROLES:
            t = self.tensors[r]
            if t.dtype != torch.uint8 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{r} must be a contiguous uint8 CUDA tensor")
            want = self.n_experts * self.expert_bytes(r)
            if t.numel() != want:
                raise ValueError(f"{r}: {t.numel()} bytes, expected {want} "
                                 f"({self.n_experts} x {name_of(self.types[r])} {_shape(r, hidden, intermediate)})")
        self.shared = shared
        if shared is not None:
            for r in ROLES:
                rows, cols = _shape(r, hidden, shared.intermediate)
                want = tensor_bytes(shared.types[r], rows, cols)
                t = getattr(shared, r)
                if t.dtype != torch.uint8 or not t.is_cuda or t.numel() != want:
                    raise ValueError(f"shared {r}: expected {want} uint8 bytes on the GPU")
            if shared.gate_inp is not None and (shared.gate_inp.dtype != torch.float32
                                                 or shared.gate_inp.numel() != hidden):
                raise ValueError("shared gate_inp must be FP32 [hidden]")
        # FP32 router weights [hidden x n_experts] (host, NumPy) when known
        self.router_weights = router_weights
        self._router_dev = None

    def router_device(self):
        """The router weights on the layer's device as the GGUF file stores
        ffn_gate_inp: a contiguous FP32 [n_experts x hidden] tensor, one row per
        expert (uploaded once)."""
        import torch

        if self.router_weights is None:
            raise ValueError("this layer has no router weights")
        if self._router_dev is None:
            w = np.asarray(self.router_weights, dtype=np.float32).reshape(self.hidden, self.n_experts)
            self._router_dev = torch.from_numpy(np.ascontiguousarray(w.T)).to(self.device)
        return self._router_dev

    # ------------------------------------------------------------- geometry
    def aligned_q3k(self) -> "ExpertLayer":
        """This layer with every Q3_K matrix (routed and shared) in the 112-byte
        resident form: the same blocks, each starting on a 16-byte boundary
        (GGUF's 110-byte blocks leave most decode loads unaligned).  Decode
        only: prefill and dequantization reject the form."""
        def conv(t, ty):
            return (pad_blocks(t, 110, 112), Q3_K_A112) if ty == 11 else (t, ty)
        tens, types = {}, {}
        for r in ROLES:
            tens[r], types[r] = conv(self.tensors[r], self.types[r])
        sh = None
        if self.shared is not None:
            s = self.shared
            parts, st = {}, {}
            for r in ROLES:
                parts[r], st[r] = conv(getattr(s, r), s.types[r])
            sh = SharedWeights(parts["gate"], parts["up"], parts["down"], types=st, intermediate=s.intermediate,
                               gate_inp=s.gate_inp)
        return ExpertLayer(tens["gate"], tens["up"], tens["down"], types, self.n_experts, self.hidden,
                           self.intermediate, sh, router_weights=getattr(self, "router_weights", None))

    def expert_bytes(self, role: str) -> int:
        rows, cols = _shape(role, self.hidden, self.intermediate)
        return tensor_bytes(self.types[role], rows, cols)

    def expert_slice(self, role: str, e: int):
        n = self.expert_bytes(role)
        return self.tensors[role][e * n:(e + 1) * n]

    @property
    def device(self):
        return self.tensors["gate"].device

    def bytes_per_expert(self) -> int:
        return sum(self.expert_bytes(r) for r in ROLES)

    def shared_bytes(self) -> int:
        if self.shared is None:
            return 0
        return sum(getattr(self.shared, r).numel() for r in ROLES)

    def resident_bytes(self) -> int:
        return self.n_experts * self.bytes_per_expert() + self.shared_bytes()

    # ------------------------------------------------------------ builders
    @classmethod
    def from_host(cls, tensors: dict, types: dict, n_experts: int, hidden: int, intermediate: int,
                  shared: dict | None = None, router_weights=None, device="cuda"):
        """Upload stacked host tensors (bytes or uint8 arrays).  ``shared`` is
        ``{"gate","up","down": bytes, "types": {...}, "intermediate": int,
        "gate_inp": FP32 array or None}``."""
        import torch

        dev = {r: _to_device_bytes(tensors[r], device) for r in ROLES}
        sh = None
        if shared is not None:
            gi = shared.get("gate_inp")
            sh = SharedWeights(
                *(_to_device_bytes(shared[r], device) for r in ROLES),
                types={r: int(shared["types"][r]) for r in ROLES},
                intermediate=int(shared["intermediate"]),
                gate_inp=None if gi is None else torch.from_numpy(
                    np.array(gi, dtype=np.float32).reshape(-1)).to(device))   # a copy: sources may be read-only maps
        return cls(dev["gate"], dev["up"], dev["down"], types, n_experts, hidden, intermediate, sh,
                   router_weights)

    @classmethod
    def synthetic(cls, types: dict, n_experts: int, hidden: int, intermediate: int, *, seed: int,
                  shared_types: dict | None = None, shared_intermediate: int | None = None,
                  gate_inp: bool = True, scale: float = 0.01, device="cuda"):
        """Random layer generated on the GPU with the benchmark distributions
        (super-block scales |N(0,1)| * scale in FP16)."""
        import torch

        from .synthetic import torch_random_stack

        g = torch.Generator(device=device)
        g.manual_seed(int(seed))
        dev = {r: torch_random_stack(types[r], n_experts, *_shape(r, hidden, intermediate),
                                     generator=g, device=device, scale=scale) for r in ROLES}
        sh = None
        if shared_types is not None:
            si = int(shared_intermediate or intermediate)
            parts = [torch_random_stack(shared_types[r], 1, *_shape(r, hidden, si), generator=g, device=device,
                                        scale=scale) for r in ROLES]
            gi = (torch.randn(hidden, generator=g, device=device) * 0.02).float() if gate_inp else None
            sh = SharedWeights(*parts, types={r: int(shared_types[r]) for r in ROLES}, intermediate=si,
                               gate_inp=gi)
        return cls(dev["gate"], dev["up"], dev["down"], types, n_experts, hidden, intermediate, sh)

    def host_expert(self, e: int) -> dict:
        """Expert e's raw bytes copied to the host (for checking against the oracle)."""
        return {r: self.expert_slice(r, e).cpu().numpy() for r in ROLES}

    def host_shared(self) -> dict | None:
        if self.shared is None:
            return None
        return {r: getattr(self.shared, r).cpu().numpy() for r in ROLES}
