"""Shared pytest setup: import paths, the ``gpu`` marker, common helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "flashprefillv2-mlx_amd"
for path in (str(ROOT), str(PKG_DIR)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; skips on machines without one (CPU suite)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU in this environment")
    return torch.device("cuda:0")


def to_np(t) -> np.ndarray:
    """Torch tensor (any device/dtype) -> float32 or integer numpy array."""
    import torch

    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.numpy()


def attention_errors(actual, expected, valid=None) -> dict:
    """Max-abs, mean-abs and max-relative (reference style) errors."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if valid is not None:
        a, e = a[valid], e[valid]
    diff = np.abs(a - e)
    return {
        "max_abs": float(diff.max()),
        "mean_abs": float(diff.mean()),
        "rel": float(diff.max() / max(np.abs(e).max(), 1e-8)),
    }


def oracle_select_parallel(q, pooled_k, *, scale, config, offset=0, query_length=None):
    """The oracle's selection of a whole call on the host's cores (at most 16
    threads), over tile ranges.  Returns ``(selected, ratio)``."""
    import os

    from oracle import fpv2_oracle as orc

    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    return orc.select_tile_ranges(q, pooled_k, scale=scale, config=config, offset=offset,
                                  query_length=query_length, workers=workers)
