"""Test configuration: import paths, the ``gpu`` marker, shared helpers.

``-m "not gpu"`` runs on any host (oracle pins, host logic, library symbol export);
``-m gpu`` needs an MI355X and calls libcfhip.so through its C ABI.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "chain-flow_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libcfhip.so")


def pytest_collection_modifyitems(config, items):
    # A GPU test on a host without a GPU fails loudly rather than silently skipping: the GPU
    # tier is only selected (-m gpu) on machines that have a GPU.
    return None


def rel_err(a, b) -> float:
    """Norm-relative error ||a - b|| / ||b|| in float64."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def to64(t):
    """torch tensor (any device / dtype) -> float64 numpy."""
    return t.detach().to("cpu").double().numpy()


def weights64(W: dict) -> dict:
    return {k: to64(v) for k, v in W.items()}


def oracle_numerics(cfg, batch: int = 1) -> str:
    """The oracle mode matching the numerics the reference runs this flow shape in: its fused
    kernel's ("fp16") or torch's fp16 modules' ("fp16_modules")."""
    from oracle import flow as oflow
    rows = [(c + 1) * cfg.chunk_size for c in range(cfg.draft_length // cfg.chunk_size)]
    fused = oflow.fused_kernel_shape(cfg.flow_dim, cfg.ffn_multiplier, cfg.num_heads, rows, cfg.context_size, batch)
    return "fp16" if fused else "fp16_modules"


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but torch.cuda is not available")
    return torch.device("cuda:0")
