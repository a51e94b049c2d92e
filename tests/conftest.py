"""Shared pytest setup.

Markers: ``gpu`` -- needs a HIP GPU (MI355X); everything else runs on the CPU.
Every parity test checks the HIP results against the CPU oracle (``oracle/``).
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "intel-optimized-moe-streaming_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)

REFERENCE = Path(os.environ.get("MQH_REFERENCE_TREE", "/root/reference"))


def build_check_library(src: Path, out: Path, deps: list) -> Path:
    """Compile a host-side check library (`hipcc -x hip`, host code only runs) when it
    is missing or older than any of `deps`.  The compiler writes a name of this
    process's own and the result is renamed into place, so parallel test workers
    never load a half-written file."""
    import subprocess

    if not out.exists() or out.stat().st_mtime < max(Path(d).stat().st_mtime for d in deps):
        out.parent.mkdir(exist_ok=True)
        tmp = out.with_name(f"{out.stem}.{os.getpid()}{out.suffix}")
        subprocess.run(["hipcc", "-O2", "-std=c++17", "-fPIC", "-shared", "-x", "hip", "--offload-arch=gfx950",
                        f"-I{PKG_DIR / 'csrc'}", str(src), "-o", str(tmp)], check=True, capture_output=True)
        os.replace(tmp, out)
    return out


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (gfx950)")


def gpu_available() -> bool:
    try:
        import torch
    except ImportError:
        return False
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The HIP library (ctypes); GPU tests only."""
    if not gpu_available():
        pytest.skip("no HIP GPU")
    from flash_moe_hip import _lib

    return _lib.load()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
