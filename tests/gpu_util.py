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


def assert_reference_rounding(got: np.ndarray, ref: np.ndarray, x: np.ndarray, qweight: np.ndarray,
                              scales: np.ndarray, group: int, what: str = ""):
    """Kernels that round every weight as the reference does (fp16 (q - 8) * s,
    then fp32 accumulation) differ from the oracle's float64-accumulated sum
    only by fp32 summation order: every output within one fp16 step plus the
    fp32 summation bound 2^-20 * sum_k |x_k w_k| (about sqrt(K) roundings of
    the partial sums), and at least 90 % of them equal."""
    import torch

    from oracle import torch_cpu as T  # equals lowbit_oracle.marlin_dequant_f16 bit for bit (test_oracle_golden)

    w = T.marlin_dequant(torch.from_numpy(np.ascontiguousarray(qweight)),
                         torch.from_numpy(np.ascontiguousarray(scales)), group).abs().to(torch.float64)
    bound = (torch.from_numpy(np.abs(np.asarray(x, dtype=np.float64))) @ w).numpy() * 2.0 ** -20
    g = np.asarray(got).astype(np.float64)
    r = np.asarray(ref).astype(np.float64)
    step = np.spacing(np.abs(np.asarray(ref, dtype=np.float16))).astype(np.float64)
    bad = np.abs(g - r) > step + bound
    assert not bad.any(), f"{what}: {int(bad.sum())} outputs beyond one fp16 step + the fp32 summation bound"
    assert float((g == r).mean()) >= 0.9, f"{what}: only {float((g == r).mean()):.3f} of outputs equal the oracle"


def f16_ulp_distance(got: np.ndarray, ref: np.ndarray) -> np.ndarray:
    """Distance in fp16 steps (adjacent representable values) between two fp16 arrays."""
    def key(a):
        b = np.asarray(a, dtype=np.float16).view(np.int16).astype(np.int32)
        return np.where(b < 0, -(b & 0x7FFF), b)

    return np.abs(key(got) - key(ref))


def print_case(*parts) -> None:
    print("[case]", *parts, flush=True)
