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
device; there is no CPU execution path.  Their methods take the reference's
argument lists (``loader.py:148-424``) and honour the same environment knobs,
read by this module: ``LANGBURST_LOWBIT_ROWS_PER_CTA`` (rowwise ops),
``LANGBURST_MARLIN_DIRECT_MAX_BATCH`` (Marlin batches above it run row by
row), and the output-cache policy ``LANGBURST_MARLIN_OUT_CACHE_POLICY`` /
``_MAX_BATCH`` with its budget ``LANGBURST_MARLIN_CACHE_MAX_MIB`` /
``_MIN_FREE_MIB`` (off by default: every call returns a new output tensor;
when on, one output buffer per batch size is reused and returned again, as in
the reference).
"""
from __future__ import annotations

import json
import math
import os
from dataclasses import dataclass, field
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


_MIB = 1024 * 1024


def _env_int(name: str, default: int) -> int:
    raw = os.environ.get(name, "").strip()
    return int(raw) if raw else int(default)


def lowbit_rows_per_cta() -> int:
    """``rows_per_cta`` the rowwise ops receive: ``LANGBURST_LOWBIT_ROWS_PER_CTA``,
    one of 4, 8, 16 (unset or empty: 8), as the reference's ``LowBitTensor``
    passes it (``loader.py:168,198``; knob defined at ``tuning.py:44-52``)."""
    value = _env_int("LANGBURST_LOWBIT_ROWS_PER_CTA", 8)
    if value not in (4, 8, 16):
        raise ValueError("lowbit rows_per_cta must be one of: 4, 8, 16")
    return value


def marlin_direct_max_batch() -> int:
    """Largest batch ``LowBitMarlinTensor.gemm`` runs as one GEMM:
    ``LANGBURST_MARLIN_DIRECT_MAX_BATCH`` (>= 1; unset or empty: 256).  Larger
    batches run row by row, as the reference does (``loader.py:315-320``)."""
    value = _env_int("LANGBURST_MARLIN_DIRECT_MAX_BATCH", 256)
    if value < 1:
        raise ValueError("Marlin direct max batch must be >= 1")
    return value


class _OutputCache:
    """Admission rule and byte budget of the reference's Marlin output cache
    (``loader.py:25-136``), read from the same environment variables:

    * ``LANGBURST_MARLIN_OUT_CACHE_POLICY``: ``off`` (default; also ``0``,
      ``false``, ``none``, ``no_cache``) caches nothing; ``decode_only`` caches
      batch 1; ``decode_small`` / ``small`` / ``bounded`` cache batches up to
      ``LANGBURST_MARLIN_OUT_CACHE_MAX_BATCH`` (default 2); anything else
      caches every batch;
    * ``LANGBURST_MARLIN_CACHE_MAX_MIB`` (default 384; 0 = unlimited): total
      bytes of every tensor's cached buffers;
    * ``LANGBURST_MARLIN_CACHE_MIN_FREE_MIB`` (default 384; 0 = no check):
      device memory that must stay free after a new buffer.
    """

    bytes_used = 0

    @staticmethod
    def wants(batch: int) -> bool:
        policy = os.environ.get("LANGBURST_MARLIN_OUT_CACHE_POLICY", "off").strip().lower()
        if policy in ("0", "false", "off", "none", "no_cache"):
            return False
        if policy == "decode_only":
            return int(batch) == 1
        if policy in ("decode_small", "small", "bounded"):
            return int(batch) <= max(1, _env_int("LANGBURST_MARLIN_OUT_CACHE_MAX_BATCH", 2))
        return True

    @classmethod
    def admits(cls, batch: int, device, new_bytes: int) -> bool:
        import torch

        if not cls.wants(batch):
            return False
        max_mib = _env_int("LANGBURST_MARLIN_CACHE_MAX_MIB", 384)
        min_free_mib = _env_int("LANGBURST_MARLIN_CACHE_MIN_FREE_MIB", 384)
        if max_mib < 0 or min_free_mib < 0:
            raise ValueError("LANGBURST_MARLIN_CACHE_MAX_MIB / _MIN_FREE_MIB must be >= 0")
        if max_mib > 0 and cls.bytes_used + int(new_bytes) > max_mib * _MIB:
            return False
        if min_free_mib == 0 or device.type != "cuda":
            return True
        free, _ = torch.cuda.mem_get_info(device)
        return int(free) - int(new_bytes) >= min_free_mib * _MIB

    @classmethod
    def account(cls, delta: int) -> None:
        cls.bytes_used = max(0, cls.bytes_used + int(delta))


def _nbytes(t) -> int:
    return 0 if t is None else int(t.numel() * t.element_size())


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

    def gemv(self, x):
        import torch

        _require_device(self.qweight, self.name)
        with torch.cuda.device(self.qweight.device):
            return _ops().lowbit_gemv(self.qweight, self.scales, x.contiguous(), self.cols, self.group_size, self.bits,
                                      lowbit_rows_per_cta())

    def gemm(self, x):
        import torch

        if x.ndim != 2:
            raise ValueError("gemm expects x [batch, cols]")
        _require_device(self.qweight, self.name)
        with torch.cuda.device(self.qweight.device):
            return _ops().lowbit_gemm(self.qweight, self.scales, x.contiguous(), self.cols, self.group_size, self.bits,
                                      lowbit_rows_per_cta())

    def row_dequant(self, row):
        import torch

        _require_device(self.qweight, self.name)
        if not torch.is_tensor(row):
            row = torch.tensor(int(row), device=self.qweight.device, dtype=torch.long)
        else:
            row = row.to(device=self.qweight.device, dtype=torch.long).reshape(())
        with torch.cuda.device(self.qweight.device):
            return _ops().lowbit_row_dequant(self.qweight, self.scales, row, self.cols, self.group_size, self.bits)


@dataclass
class LowBitMarlinTensor:
    """Marlin W4 tensor (``loader.py:204-424``): ``gemm``/``gemv``,
    ``gemm_silu_packed(mixed, hidden, out=None)`` and ``gemm_argmax(x, out=None)``
    with the reference's argument checks, output and workspace caching rules
    and argmax epoch.  The workspace (int32, ``rows // 128 * 16`` entries) is
    zeroed before every call, as the reference's wrapper does."""

    name: str
    qweight: "object"  # int32 [cols/16, 2*rows]
    scales: "object"   # fp16 [n_groups, rows]
    cols: int
    group_size: int
    bits: int = 4
    exec_bits: int = 4
    _out_cache: dict = field(default_factory=dict, init=False, repr=False)
    _argmax_cache: dict = field(default_factory=dict, init=False, repr=False)
    _argmax_state_cache: dict = field(default_factory=dict, init=False, repr=False)
    _argmax_sync: "object" = field(default=None, init=False, repr=False)
    _argmax_epoch: int = field(default=0, init=False, repr=False)
    _workspace: "object" = field(default=None, init=False, repr=False)

    @property
    def rows(self) -> int:
        return int(self.qweight.shape[1] // 2)

    # -- runtime buffers -------------------------------------------------
    def _cached(self, cache: dict, batch: int, shape: tuple, dtype):
        import torch

        dev = self.qweight.device
        have = cache.get(batch)
        if have is not None and have.device == dev and tuple(have.shape) == shape and have.dtype == dtype:
            return have
        nbytes = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
        # admission is decided before the allocation, so that the free-memory
        # check sees the device as it is (loader.py:254-264)
        if _OutputCache.admits(batch, dev, nbytes):
            out = torch.empty(shape, device=dev, dtype=dtype)
            _OutputCache.account(nbytes - _nbytes(have))
            cache[batch] = out
            return out
        return torch.empty(shape, device=dev, dtype=dtype)

    def _cached_workspace(self):
        import torch

        size = max(1, self.rows // 128 * 16)
        dev = self.qweight.device
        ws = self._workspace
        if ws is not None and ws.device == dev and ws.numel() >= size:
            ws[:size].zero_()
            return ws
        if _OutputCache.admits(1, dev, size * 4):  # before the allocation (loader.py:290-302)
            fresh = torch.zeros((size,), device=dev, dtype=torch.int32)
            _OutputCache.account(size * 4 - _nbytes(ws))
            self._workspace = fresh
            return fresh
        return torch.zeros((size,), device=dev, dtype=torch.int32)

    def runtime_cache_bytes(self) -> int:
        total = _nbytes(self._workspace) + _nbytes(self._argmax_sync)
        for cache in (self._out_cache, self._argmax_cache, self._argmax_state_cache):
            total += sum(_nbytes(t) for t in cache.values())
        return total

    def clear_runtime_cache(self) -> None:
        _OutputCache.account(-self.runtime_cache_bytes())
        self._out_cache.clear()
        self._argmax_cache.clear()
        self._argmax_state_cache.clear()
        self._argmax_sync = None
        self._workspace = None

    # -- projections -----------------------------------------------------
    def _check_device(self) -> None:
        _require_device(self.qweight, self.name)

    def gemv(self, x):
        return self.gemm(x.reshape(1, -1).contiguous()).reshape(-1)

    def gemm(self, x):
        import torch

        if x.ndim != 2:
            raise ValueError("gemm expects x [batch, cols]")
        self._check_device()
        x = x.to(device=self.qweight.device, dtype=torch.float16).contiguous()
        batch = int(x.size(0))
        if batch > marlin_direct_max_batch():
            rows = [self.gemm(r.reshape(1, -1)).reshape(-1).clone() for r in x]
            return torch.stack(rows, dim=0).contiguous()
        out = self._cached(self._out_cache, batch, (batch, self.rows), torch.float16)
        ws = self._cached_workspace()
        with torch.cuda.device(self.qweight.device):
            _ops().lowbit_marlin_gemm_out(self.qweight, self.scales, x, out, ws, self.cols, self.group_size)
        return out

    def gemm_silu_packed(self, mixed, hidden: int, out=None):
        """``out = fp16(silu(mixed[:, :hidden]) * mixed[:, hidden:]) @ W^T``; ``hidden``
        must equal this tensor's input columns (``loader.py:337-368``)."""
        import torch

        if mixed.ndim == 1:
            mixed = mixed.reshape(1, -1)
        if mixed.ndim != 2:
            raise ValueError("gemm_silu_packed expects mixed [batch, 2*hidden]")
        if int(hidden) != int(self.cols):
            raise ValueError("hidden must match this Marlin tensor's input cols")
        if mixed.size(1) != 2 * int(hidden):
            raise ValueError("mixed width must be 2*hidden")
        self._check_device()
        mixed = mixed.to(device=self.qweight.device, dtype=torch.float16).contiguous()
        batch = int(mixed.size(0))
        if out is None:
            out = self._cached(self._out_cache, batch, (batch, self.rows), torch.float16)
        elif out.device != self.qweight.device or tuple(out.shape) != (batch, self.rows) or out.dtype != torch.float16:
            raise ValueError("out must be fp16 CUDA tensor with shape [batch, rows]")
        ws = self._cached_workspace()
        with torch.cuda.device(self.qweight.device):
            _ops().lowbit_marlin_gemm_silu_packed_out(self.qweight, self.scales, mixed, out, ws, int(hidden),
                                                      self.group_size)
        return out

    def gemm_argmax(self, x, out=None):
        """Per-row argmax of ``x @ W^T`` (first index on ties) without writing the
        logits (``loader.py:370-413``); the epoch wraps to 1 after 2e9 calls."""
        import torch

        if x.ndim == 1:
            x = x.reshape(1, -1)
        if x.ndim != 2:
            raise ValueError("gemm_argmax expects x [batch, cols]")
        self._check_device()
        dev = self.qweight.device
        x = x.to(device=dev, dtype=torch.float16).contiguous()
        batch = int(x.size(0))
        scratch_out = self._cached(self._out_cache, batch, (batch, self.rows), torch.float16)
        ws = self._cached_workspace()
        if out is None:
            out = self._cached(self._argmax_cache, batch, (batch,), torch.long)
        else:
            if out.device != dev or out.numel() != batch or out.dtype != torch.long:
                raise ValueError("argmax out must be int64 CUDA tensor with shape [batch]")
            out = out.reshape(batch)
        state = self._cached(self._argmax_state_cache, batch, (batch,), torch.long)
        if self._argmax_sync is None or self._argmax_sync.device != dev:
            sync = torch.empty((2,), device=dev, dtype=torch.int32)
            if _OutputCache.admits(batch, dev, 8):
                _OutputCache.account(8 - _nbytes(self._argmax_sync))
                self._argmax_sync = sync
        else:
            sync = self._argmax_sync
        self._argmax_epoch = 1 if self._argmax_epoch >= 2_000_000_000 else self._argmax_epoch + 1
        with torch.cuda.device(dev):
            _ops().lowbit_marlin_gemm_argmax_out(self.qweight, self.scales, x, scratch_out, ws, state, out, sync,
                                                 self._argmax_epoch, self.cols, self.group_size)
        return out

    def row_dequant(self, row):
        raise RuntimeError("Marlin layout does not support row_dequant; keep embeddings in rowwise layout")


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
