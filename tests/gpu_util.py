"""Helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np

# Tolerance of the parity bar: outputs within max-abs 1e-2 / rel 1e-3 of the
# oracle's fp16-dequant-then-fp32-accumulate result (fp16 outputs).
ATOL = 1e-2
RTOL = 1e-3


def to_dev(a: np.ndarray, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_np(t) -> np.ndarray:
    return t.detach().cpu().numpy()


def assert_close_f16(got: np.ndarray, ref: np.ndarray, atol: float = ATOL, rtol: float = RTOL, what: str = ""):
    g = np.asarray(got).astype(np.float64)
    r = np.asarray(ref).astype(np.float64)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - r)
    bad = err > atol + rtol * np.abs(r)
    if bad.any():
        idx = np.argwhere(bad)[:5].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside tol; max abs err {err.max():.3e}; e.g. {idx}")
    return float((g == r).mean())


def print_case(*parts) -> None:
    print("[case]", *parts, flush=True)
