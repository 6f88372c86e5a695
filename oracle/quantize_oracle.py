"""CPU restatement of the reference's float -> code quantisers and checkpoint writer.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/`` imports this module: it
produces checkpoints in the reference's on-disk format so that the product
loader (``neurova_amd.store``) and kernels can be checked against them.

Paths are relative to ``/root/reference/langburst``.

Pinning: ``tests/golden/quant_golden.npz`` holds the reference's own outputs
(``adapters/qwen36_tools/quantize.py:125-243`` run once on seeded inputs with
zero rows, exact half-step ties and scale-1 groups, by
``tests/golden/make_quant_golden.py``); ``tests/test_store_cpu.py`` requires
bit equality of codes and scales.  The packing steps reuse the oracle's packers
(``lowbit_oracle.rowwise_pack``, ``marlin_pack_codes``, ``marlin_pack_scales``),
which are pinned by the reference's tables and known-answer vectors.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

from . import lowbit_oracle as O

INDEX_NAME = "langburst_index.json"  # core/platform.py:10


def quantize_symmetric_lowbit(w: np.ndarray, group_size: int = 128, bits: int = 4):
    """Rowwise ``lowbit_symmetric_groupwise`` quantiser (``quantize.py:125-177``).

    Per (row, group): fp32 scale = amax|w| / qmax (1 where that is 0 or not
    finite); code = clamp(round-half-even(w / scale), qmin, qmax) + 2**(bits-1),
    computed with the fp32 scale; the stored scale is fp16(scale).  Columns past
    ``cols`` in the last group are zero padding.  Returns (packed, scales, meta).
    """
    w = np.asarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError(f"expected 2D weight, got {tuple(w.shape)}")
    if bits < 2 or bits > 8:
        raise ValueError(f"bits must be in [2, 8], got {bits}")
    rows, cols = w.shape
    n_groups = math.ceil(cols / group_size)
    padded = np.zeros((rows, n_groups * group_size), dtype=np.float32)
    padded[:, :cols] = w
    grouped = padded.reshape(rows, n_groups, group_size)
    qmin, qmax, zero = -(1 << (bits - 1)), (1 << (bits - 1)) - 1, 1 << (bits - 1)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        scale = (np.abs(grouped).max(axis=2) / np.float32(qmax)).astype(np.float32)
        scale = np.where(np.isfinite(scale) & (scale > 0), scale, np.float32(1.0)).astype(np.float32)
        q = np.clip(np.rint(grouped / scale[:, :, None]), qmin, qmax)
    codes = (q.reshape(rows, -1)[:, :cols] + zero).astype(np.uint8)
    packed = O.rowwise_pack(codes, bits)
    meta = {"rows": rows, "cols": cols, "group_size": group_size, "n_groups": n_groups,
            "packed_cols": O.rowwise_packed_cols(cols, bits), "bits": bits}
    return packed, scale.astype(np.float16), meta


def quantize_marlin4_groupwise(w: np.ndarray, group_size: int = 128):
    """Marlin ``lowbit_marlin_groupwise`` quantiser (``quantize.py:180-243``).

    The weight ``[N, K]`` is rounded to fp16 first.  Per (group, column): fp16
    scale = fp16(fp32(amax|w|) * fp32(2/15)) (1 where 0 or not finite; fp16
    arithmetic of a half tensor with a Python scalar runs in fp32 and rounds
    once); code = clamp(round-half-even(fp16(w / s)) + 8, 0, 15) -- the quotient
    of two halves is itself rounded to fp16 before the rounding to an integer.
    ``group_size == -1``: one scale per column over all of K.
    Returns (qweight int32 [K/16, 2N], scales fp16 [groups, N] permuted, meta).
    """
    w16 = np.asarray(w).astype(np.float16)
    if w16.ndim != 2:
        raise ValueError(f"expected 2D weight, got {tuple(w16.shape)}")
    if group_size not in (-1, 128):
        raise ValueError("Marlin layout supports group_size -1 or 128")
    rows, cols = w16.shape
    if cols % 128 != 0 or rows % 256 != 0:
        raise ValueError(f"Marlin requires cols % 128 == 0 and rows % 256 == 0, got {rows}x{cols}")
    eff = cols if group_size == -1 else group_size
    wc = np.ascontiguousarray(w16.T)  # [K, N]
    grouped = wc.reshape(cols // eff, eff, rows)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        amax = np.abs(grouped).max(axis=1).astype(np.float32)  # [groups, N], exact halves
        s = (amax * np.float32(2.0 / 15.0)).astype(np.float16)
        s = np.where(np.isfinite(s) & (s > 0), s, np.float16(1.0)).astype(np.float16)
        quot = (grouped.astype(np.float32) / s.astype(np.float32)[:, None, :]).astype(np.float16)
        q = np.clip(np.rint(quot.astype(np.float32)) + 8, 0, 15)
    codes = q.reshape(cols, rows).astype(np.uint8)
    qweight = O.marlin_pack_codes(codes)
    scales = O.marlin_pack_scales(s, per_column=(eff == cols))
    meta = {"rows": rows, "cols": cols, "group_size": eff, "n_groups": cols // eff, "packed_cols": rows * 16 // 8,
            "bits": 4, "exec_bits": 4, "layout": "marlin_v1"}
    return qweight, scales, meta


def new_index(bits: int = 4, layout: str = "marlin", group_size: int = 128) -> dict:
    """The index header ``convert`` writes (``quantize.py:362-371``)."""
    return {"format": f"langburst-q{bits}-{layout}-v1" if layout != "rowwise" else f"langburst-q{bits}-v4",
            "group_size": group_size, "bits": bits, "layout": layout, "hybrid_policy": "none",
            "fuse_projections": False, "fp16_embed": False, "tensors": {}}


def _write(path: Path, arr: np.ndarray) -> None:  # quantize.py:246-249
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_bytes(np.ascontiguousarray(arr).tobytes(order="C"))


def write_fp16_tensor(out_dir: Path, index: dict, name: str, arr: np.ndarray) -> None:
    """``write_fp16_tensor`` (``quantize.py:252-262``)."""
    rel = name.replace(".", "__")
    raw = Path("fp16") / f"{rel}.fp16.bin"
    _write(out_dir / raw, np.asarray(arr).astype(np.float16))
    index["tensors"][name] = {"kind": "fp16_raw", "path": str(raw), "shape": list(np.shape(arr)), "dtype": "float16"}


def write_quantized_tensor(out_dir: Path, index: dict, name: str, w: np.ndarray, group_size: int, bits: int,
                           marlin: bool) -> None:
    """``write_quantized_tensor`` (``quantize.py:312-340``) with the layout chosen by the caller."""
    rel = name.replace(".", "__")
    if marlin:
        packed, scales, meta = quantize_marlin4_groupwise(w, group_size=group_size)
        q_path, s_path = Path("marlin_q4") / f"{rel}.marlin.int32.bin", Path("marlin_q4") / f"{rel}.scale.fp16.bin"
    else:
        packed, scales, meta = quantize_symmetric_lowbit(w, group_size=group_size, bits=bits)
        q_path, s_path = Path(f"q{bits}") / f"{rel}.q{bits}.bin", Path(f"q{bits}") / f"{rel}.scale.fp16.bin"
    _write(out_dir / q_path, packed)
    _write(out_dir / s_path, scales)
    index["tensors"][name] = {"kind": "lowbit_marlin_groupwise" if marlin else "lowbit_symmetric_groupwise",
                              "qweight": str(q_path), "scales": str(s_path), **meta}


def write_index(out_dir: Path, index: dict) -> Path:
    """``langburst_index.json`` (``quantize.py:429-430``)."""
    path = Path(out_dir) / INDEX_NAME
    path.write_text(json.dumps(index, indent=2), encoding="utf-8")
    return path
