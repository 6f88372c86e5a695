"""Writes tests/golden/quant_golden.npz: input/output vectors of the reference's
float -> code quantisers, which nothing else pins (fp16 opmath of the scale and
the quotient, round-half-to-even ties).

Run once, in the build container only (the reference is not on the GPU box):

    python tests/golden/make_quant_golden.py /root/reference

It loads the one module that holds the quantisers,
langburst/langburst/adapters/qwen36_tools/quantize.py (its own imports are
numpy, torch, safetensors and tqdm), from its file, calls
quantize_marlin4_groupwise (:180-243) and quantize_symmetric_lowbit (:125-177)
on small seeded inputs, and saves inputs and outputs.  The inputs include a
zero row (the scale falls back to 1), groups whose scale is exactly 1 with
values on exact half steps (ties), and random rows.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np


def load_quantize(ref_root: Path):
    path = ref_root / "langburst" / "langburst" / "adapters" / "qwen36_tools" / "quantize.py"
    spec = importlib.util.spec_from_file_location("_ref_quantize", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def marlin_input(rng) -> np.ndarray:
    """fp16 [N = 256, K = 128]: random, one zero row, and rows whose 128-wide
    group has amax 7.5 (scale fp16(7.5 * 2/15) = 1) and half-step values."""
    w = (rng.normal(0.0, 0.02, size=(256, 128))).astype(np.float16)
    w[3] = 0
    ties = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 6.5, -7.5, 7.5], dtype=np.float16)
    for r in (5, 77, 200):
        w[r] = rng.choice(ties, size=128).astype(np.float16)
        w[r, 0] = 7.5
    w[9] = (rng.normal(0.0, 40.0, size=128)).astype(np.float16)  # large magnitudes
    return w


def rowwise_input(rng) -> np.ndarray:
    """fp32 [7, 257]: random rows, a zero row, and a row of half steps with
    amax 1 * qmax per group (scale exactly 1 for every bit width's qmax
    is not possible at once; the rows hold half steps of several scales)."""
    w = rng.normal(0.0, 0.05, size=(7, 257)).astype(np.float32)
    w[2] = 0
    w[4] = rng.choice(np.array([0.5, -0.5, 1.5, -2.5, 3.5, 127.0, -127.0], dtype=np.float32), size=257)
    w[5] = rng.choice(np.array([0.5, -1.5, 2.5, 7.0, -7.0, 3.0, -3.0], dtype=np.float32), size=257)
    w[6, :128] = 0  # one zero group, one live group
    return w


def main() -> None:
    import torch

    ref_root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    q = load_quantize(ref_root)
    rng = np.random.default_rng(20260101)
    out = {}
    mw = marlin_input(rng)
    out["marlin_w"] = mw
    for g in (128, -1):
        packed, scales, meta = q.quantize_marlin4_groupwise(torch.from_numpy(mw.copy()), group_size=g)
        tag = "g128" if g == 128 else "gcol"
        out[f"marlin_{tag}_qweight"] = packed
        out[f"marlin_{tag}_scales"] = scales
        out[f"marlin_{tag}_meta"] = np.array([meta["rows"], meta["cols"], meta["group_size"], meta["n_groups"],
                                              meta["packed_cols"]], dtype=np.int64)
    rw = rowwise_input(rng)
    out["rowwise_w"] = rw
    for bits in (2, 3, 4, 8):
        for g in (8, 128):
            packed, scales, meta = q.quantize_symmetric_lowbit(torch.from_numpy(rw.copy()), group_size=g, bits=bits)
            out[f"rowwise_b{bits}_g{g}_packed"] = packed
            out[f"rowwise_b{bits}_g{g}_scales"] = scales
            out[f"rowwise_b{bits}_g{g}_meta"] = np.array([meta["rows"], meta["cols"], meta["group_size"],
                                                          meta["n_groups"], meta["packed_cols"]], dtype=np.int64)
    dst = Path(__file__).resolve().parent / "quant_golden.npz"
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({dst.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
