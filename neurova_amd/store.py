"""Loader for the reference's quantised checkpoint format.

A checkpoint directory holds ``langburst_index.json`` (``core/platform.py:10``)
and raw little-endian C-order arrays (``adapters/qwen36_tools/quantize.py:246-340``):

* ``lowbit_marlin_groupwise``: ``qweight`` int32 ``[cols/16, packed_cols]``
  (``packed_cols = 2 * rows``) and ``scales`` fp16 ``[n_groups, rows]``, in
  the Marlin tile order (layout ``marlin_v1``);
* ``lowbit_symmetric_groupwise``: ``qweight`` uint8 ``[rows, packed_cols]``
  and ``scales`` fp16 ``[rows, n_groups]``;
* ``fp16_raw``: an fp16 array of ``shape``.

:class:`QuantizedStore` mirrors the reference's ``QuantizedStore``
(``langburst/loader.py:474-528``): same index resolution, kinds and returned
tensor shapes.  There is no repack: the gfx950 kernels read both layouts as
stored, so a tensor is the file's bytes copied to the device.  Unlike the
reference, every file's size is checked against the shape its index entry
declares, and Marlin tensors against the kernels' shape rules, before any
upload; a mismatch raises ``ValueError``.

The tensor objects call the ``langburst_cuda`` ops of this package on their
device; there is no CPU execution path.  Differences from the reference's
wrappers (``loader.py:148-424``): ``gemm``/``gemv`` return a new tensor per
call (the reference reuses one cached output buffer per batch size), and a
Marlin batch of any size runs as one GEMM (the reference evaluates batches
above ``marlin_direct_max_batch`` row by row).
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass
from pathlib import Path

import numpy as np

INDEX_FILENAMES = ("langburst_index.json",)


def resolve_index_file(root: str | Path) -> Path:
    """The first of ``INDEX_FILENAMES`` present in ``root`` (``core/platform.py:26-33``)."""
    base = Path(root)
    for name in INDEX_FILENAMES:
        path = base / name
        if path.exists():
            return path
    raise FileNotFoundError(f"runtime index not found in {base}; expected one of: {', '.join(INDEX_FILENAMES)}")


def _ops():
    from . import load_extension

    return load_extension()


def _require_device(t, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what}: tensors must be on the GPU (this build has no CPU execution path)")


@dataclass
class FP16Tensor:
    name: str
    value: "object"


@dataclass
class LowBitTensor:
    """Rowwise symmetric groupwise tensor (``loader.py:148-201``)."""

    name: str
    qweight: "object"  # uint8 [rows, packed_cols]
    scales: "object"   # fp16 [rows, n_groups]
    cols: int
    group_size: int
    bits: int = 4

    @property
    def rows(self) -> int:
        return int(self.qweight.shape[0])

    def gemv(self, x, rows_per_cta: int = 8):
        _require_device(self.qweight, self.name)
        return _ops().lowbit_gemv(self.qweight, self.scales, x.contiguous(), self.cols, self.group_size, self.bits,
                                  rows_per_cta)

    def gemm(self, x, rows_per_cta: int = 8):
        if x.ndim != 2:
            raise ValueError("gemm expects x [batch, cols]")
        _require_device(self.qweight, self.name)
        return _ops().lowbit_gemm(self.qweight, self.scales, x.contiguous(), self.cols, self.group_size, self.bits,
                                  rows_per_cta)

    def row_dequant(self, row):
        import torch

        _require_device(self.qweight, self.name)
        if not torch.is_tensor(row):
            row = torch.tensor(int(row), device=self.qweight.device, dtype=torch.long)
        else:
            row = row.to(device=self.qweight.device, dtype=torch.long).reshape(())
        return _ops().lowbit_row_dequant(self.qweight, self.scales, row, self.cols, self.group_size, self.bits)


@dataclass
class LowBitMarlinTensor:
    """Marlin W4 tensor (``loader.py:204-424``)."""

    name: str
    qweight: "object"  # int32 [cols/16, 2*rows]
    scales: "object"   # fp16 [n_groups, rows]
    cols: int
    group_size: int
    bits: int = 4
    exec_bits: int = 4

    @property
    def rows(self) -> int:
        return int(self.qweight.shape[1] // 2)

    def _workspace(self):
        import torch

        return torch.zeros((max(1, self.rows // 128 * 16),), dtype=torch.int32, device=self.qweight.device)

    def gemm(self, x):
        import torch

        if x.ndim != 2:
            raise ValueError("gemm expects x [batch, cols]")
        _require_device(self.qweight, self.name)
        x = x.to(device=self.qweight.device, dtype=torch.float16).contiguous()
        out = torch.empty((x.shape[0], self.rows), dtype=torch.float16, device=self.qweight.device)
        _ops().lowbit_marlin_gemm_out(self.qweight, self.scales, x, out, self._workspace(), self.cols, self.group_size)
        return out

    def gemv(self, x):
        return self.gemm(x.reshape(1, -1)).reshape(-1)

    def gemm_silu_packed(self, mixed):
        """``out = fp16(silu(mixed[:, :cols]) * mixed[:, cols:]) @ W^T`` (``loader.py:337-368``)."""
        import torch

        if mixed.ndim == 1:
            mixed = mixed.reshape(1, -1)
        _require_device(self.qweight, self.name)
        mixed = mixed.to(device=self.qweight.device, dtype=torch.float16).contiguous()
        out = torch.empty((mixed.shape[0], self.rows), dtype=torch.float16, device=self.qweight.device)
        _ops().lowbit_marlin_gemm_silu_packed_out(self.qweight, self.scales, mixed, out, self._workspace(), self.cols,
                                                  self.group_size)
        return out


def _check_file(path: Path, shape: tuple[int, ...], itemsize: int, name: str) -> None:
    want = int(np.prod(shape)) * itemsize
    if not path.exists():
        raise ValueError(f"{name}: missing file {path}")
    have = path.stat().st_size
    if have != want:
        raise ValueError(f"{name}: {path.name} holds {have} bytes, its index entry declares {shape} ({want} bytes)")


class QuantizedStore:
    """Tensors of a quantised checkpoint directory, loaded on first use and cached."""

    def __init__(self, root: str | Path, device="cuda"):
        import torch

        self.root = Path(root)
        with open(resolve_index_file(self.root), "r", encoding="utf-8") as f:
            self.index = json.load(f)
        self.device = torch.device(device)
        self.cache: dict[str, object] = {}

    def names(self) -> list[str]:
        return sorted(self.index["tensors"])

    def _array(self, rel: str, dtype, shape: tuple[int, ...], name: str):
        import torch

        path = self.root / rel
        _check_file(path, shape, np.dtype(dtype).itemsize, name)
        arr = np.fromfile(path, dtype=dtype).reshape(shape)
        return torch.from_numpy(arr).to(self.device, non_blocking=False).contiguous()

    def tensor(self, name: str):
        if name in self.cache:
            return self.cache[name]
        meta = self.index["tensors"][name]
        kind = meta["kind"]
        if kind == "lowbit_symmetric_groupwise":
            bits, rows, cols = int(meta["bits"]), int(meta["rows"]), int(meta["cols"])
            group, n_groups, packed_cols = int(meta["group_size"]), int(meta["n_groups"]), int(meta["packed_cols"])
            if not 2 <= bits <= 8 or group <= 0:
                raise ValueError(f"{name}: bits {bits} / group_size {group} outside the format")
            if packed_cols < math.ceil(cols * bits / 8) or n_groups < math.ceil(cols / group):
                raise ValueError(f"{name}: packed_cols {packed_cols} / n_groups {n_groups} too small for {cols} columns")
            q = self._array(meta["qweight"], np.uint8, (rows, packed_cols), name)
            s = self._array(meta["scales"], np.float16, (rows, n_groups), name)
            obj = LowBitTensor(name=name, qweight=q, scales=s, cols=cols, group_size=group, bits=bits)
        elif kind == "lowbit_marlin_groupwise":
            rows, cols = int(meta["rows"]), int(meta["cols"])
            group, n_groups, packed_cols = int(meta["group_size"]), int(meta["n_groups"]), int(meta["packed_cols"])
            if rows % 256 or cols % 128 or packed_cols != 2 * rows:
                raise ValueError(f"{name}: Marlin tensor {rows}x{cols} (packed_cols {packed_cols}) is not a "
                                 "multiple of 256 output rows x 128 input columns")
            if not (group == 128 and n_groups == cols // 128) and not (group in (-1, cols) and n_groups == 1):
                raise ValueError(f"{name}: Marlin group_size {group} with {n_groups} groups is not supported")
            q = self._array(meta["qweight"], np.int32, (cols // 16, packed_cols), name)
            s = self._array(meta["scales"], np.float16, (n_groups, rows), name)
            obj = LowBitMarlinTensor(name=name, qweight=q, scales=s, cols=cols, group_size=group,
                                     bits=int(meta.get("bits", 4)), exec_bits=int(meta.get("exec_bits", 4)))
        elif kind == "fp16_raw":
            obj = FP16Tensor(name=name, value=self._array(meta["path"], np.float16, tuple(meta["shape"]), name))
        else:
            raise ValueError(f"unknown tensor kind: {kind}")
        self.cache[name] = obj
        return obj
