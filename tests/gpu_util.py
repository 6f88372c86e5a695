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


def assert_exact_scale(got: np.ndarray, ref: np.ndarray, exact: np.ndarray, what: str = ""):
    """Grouped scales: the kernel multiplies each group's fp32 sum of x*(q-8) by
    the scale once, where the reference rounds every fp16 (q-8)*s product before
    accumulating.  Against the float64 value of the same sum (``exact``), the
    kernel must be at least as accurate as the reference is (RMS), and no
    element may be off by more than one fp16 step plus twice the reference's
    own RMS rounding noise."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    e = np.asarray(exact, dtype=np.float64)
    rms_got = float(np.sqrt(np.mean((g - e) ** 2)))
    rms_ref = float(np.sqrt(np.mean((r - e) ** 2)))
    assert rms_got <= rms_ref + 1e-12, f"{what}: rms error vs exact {rms_got:.3e} > reference's {rms_ref:.3e}"
    step = np.spacing(np.abs(np.asarray(exact, dtype=np.float16))).astype(np.float64)
    bad = np.abs(g - e) > step + 2.0 * rms_ref
    assert not bad.any(), f"{what}: {int(bad.sum())} outputs off the exact value by more than 1 step + 2 rms"


def f16_ulp_distance(got: np.ndarray, ref: np.ndarray) -> np.ndarray:
    """Distance in fp16 steps (adjacent representable values) between two fp16 arrays."""
    def key(a):
        b = np.asarray(a, dtype=np.float16).view(np.int16).astype(np.int32)
        return np.where(b < 0, -(b & 0x7FFF), b)

    return np.abs(key(got) - key(ref))


def print_case(*parts) -> None:
    print("[case]", *parts, flush=True)
