"""Shared test setup.

* ``gpu`` marks tests that need an MI355X; everything else runs on the CPU.
* The repo root (for ``oracle``) and ``nano-vllm-int4_amd`` (for ``nv4``) go
  on sys.path.  Tests load the libraries that are already built and build
  them only when missing (``__graft_entry__.build()`` rebuilds both).
"""
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "nano-vllm-int4_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


def _ensure_built():
    if not (ROOT / "oracle" / "liboracle.so").exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, stdout=subprocess.DEVNULL)
    if not (PKG / "nv4" / "libnv4.so").exists():
        subprocess.run(["make", "-C", str(PKG), "-j8"], check=True, stdout=subprocess.DEVNULL)


_ensure_built()


def pytest_collection_modifyitems(config, items):
    """Skip GPU tests cleanly on a host without a GPU (they are selected
    explicitly with -m gpu on a host with one)."""
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


# ------------------------------------------------------------------ helpers
def bf16_bits(t) -> np.ndarray:
    """bf16 torch tensor (any device) -> numpy uint16 bit patterns."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f16_bits(t) -> np.ndarray:
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_to_bf16(a: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def nv4_mod():
    import nv4
    return nv4
