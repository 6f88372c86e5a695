"""Vectorised PyTorch-CPU restatement of the reference's CPU paths, for the
timed CPU baseline.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``bench.py``'s ``cpu_baseline``
leg times these functions, and ``tests/test_oracle_golden.py`` pins them to
the numpy oracle (``lowbit_oracle``): the dequantised weights bit for bit,
the products within the parity tolerance (fp32 accumulation in another
order).  Nothing in ``neurova_amd`` imports this module.

* ``rowwise_dequant_rows`` / ``rowwise_gemv`` restate the reference's CPU
  branch of ``LowBitTensor.gemv`` (``langburst/loader.py:170-171``): the
  dense fp16 matrix of ``dequantize_lowbit_rows`` (``loader.py:427-465``,
  codes per ``lowbit_gemv.cu:4-14``, ``q * fp32(scale)`` rounded to fp16),
  then ``torch.matmul`` with the fp16 activations.  The reference builds the
  matrix with one Python ``.item()`` per code; here the same values come from
  tensor bit operations.
* ``marlin_dequant`` / ``marlin_gemm`` restate the Marlin op's arithmetic
  (``csrc/marlin_cuda_kernel.cu:131-159, 651-659``: ``fp16(fp16(q - 8) * s)``
  weights, fp32 accumulation, fp16 output; per-column scales after that
  rounding).  The reference has no CPU Marlin path (``ops.py:65-79`` raises);
  this is the same arithmetic on the host, for a reported baseline only.
"""
from __future__ import annotations

import numpy as np
import torch


def rowwise_dequant_rows(packed: torch.Tensor, scales: torch.Tensor, cols: int, group_size: int,
                         bits: int) -> torch.Tensor:
    """fp16 ``[rows, cols]``: code ``c`` of a row is bits ``[c*b, c*b+b)`` of its
    LSB-first byte stream (two bytes when it straddles), minus ``2**(b-1)``,
    times the fp32 scale of its group, rounded to fp16 (``loader.py:442-452``)."""
    c = torch.arange(cols, dtype=torch.int64)
    bit = c * bits
    byte = bit >> 3
    shift = bit & 7
    p = packed.to(torch.int32)
    lo = p[:, byte]
    straddle = (shift + bits > 8) & (byte + 1 < packed.shape[1])
    hi = p[:, torch.clamp(byte + 1, max=packed.shape[1] - 1)] * straddle.to(torch.int32)
    word = lo | (hi << 8)
    q = ((word >> shift.to(torch.int32)) & ((1 << bits) - 1)) - (1 << (bits - 1))
    s = scales[:, c // group_size].to(torch.float32)
    return (q.to(torch.float32) * s).to(torch.float16)


def rowwise_gemv(packed: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, cols: int, group_size: int,
                 bits: int) -> torch.Tensor:
    """``torch.matmul(dense, x)`` in fp16, as ``LowBitTensor.gemv`` on the CPU."""
    dense = rowwise_dequant_rows(packed, scales, cols, group_size, bits)
    return torch.matmul(dense, x[:cols].contiguous())


def _unpack_marlin_codes(qweight: torch.Tensor) -> torch.Tensor:
    """Codes ``[K, N]`` (uint8) of a Marlin ``qweight [K/16, 2N]``.

    Word ``(kb, chunk, slot 4c+q, j)`` holds 8 nibbles; nibble ``e`` with
    ``a = e >> 2``, ``h = (e >> 1) & 1``, ``b = e & 1`` is weight
    ``k = 16 kb + 8 b + 2 q + a``, ``n = 64 chunk + 16 j + 8 h + c`` (the
    inverse of ``quantize.py:50-76, 224-230``, cf. ``marlin_mlp_stream.cu:109-121``)."""
    kb_n, words = qweight.shape
    n = words // 2
    w = qweight.reshape(kb_n, n // 64, 8, 4, 4)                                  # kb, chunk, c, q, j
    shifts = 4 * torch.arange(8, dtype=torch.int32)
    nib = ((w.unsqueeze(-1) >> shifts) & 15).to(torch.uint8)                    # ..., e (the mask undoes the sign)
    nib = nib.reshape(kb_n, n // 64, 8, 4, 4, 2, 2, 2)                           # kb, chunk, c, q, j, a, h, b
    nib = nib.permute(0, 7, 3, 5, 1, 4, 6, 2)                                    # kb, b, q, a, chunk, j, h, c
    return nib.reshape(kb_n * 16, n)


def _unpack_marlin_scales(scales: torch.Tensor, k: int, group_size: int) -> torch.Tensor:
    """Natural-order scales: grouped ``[K/128, N]`` (the 64-column chunk stores
    column ``8 jj + i`` at ``8 i + jj``, ``quantize.py:63-65``); per-column
    ``[1, N]`` through the 32-column permutation of ``quantize.py:66-68``."""
    g, n = scales.shape
    if group_size in (-1, 0, k) or group_size <= 0:
        from oracle import lowbit_oracle as O

        nat = O.marlin_unpack_scales(scales.numpy(), per_column=True)
        return torch.from_numpy(np.ascontiguousarray(nat))
    return scales.reshape(g, n // 64, 8, 8).transpose(2, 3).reshape(g, n)


def marlin_dequant(qweight: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp16 ``W^T [K, N]`` with the kernel's rounding (per-column: ``q - 8``)."""
    codes = _unpack_marlin_codes(qweight)
    k, n = codes.shape
    qh = (torch.arange(16, dtype=torch.float32) - 8).to(torch.float16)[codes.to(torch.int64)]
    if group_size <= 0 or group_size == k:
        return qh
    s = _unpack_marlin_scales(scales, k, group_size)
    return (qh.reshape(k // group_size, group_size, n) * s.reshape(k // group_size, 1, n)).reshape(k, n)


def marlin_gemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """``fp16(x @ W)`` with fp32 accumulation (per-column scales after the rounding)."""
    k = x.shape[1]
    w = marlin_dequant(qweight, scales, group_size)
    out = (x.to(torch.float32) @ w.to(torch.float32)).to(torch.float16)
    if group_size <= 0 or group_size == k:
        s = _unpack_marlin_scales(scales, k, group_size).reshape(1, -1)
        out = out * s
    return out
