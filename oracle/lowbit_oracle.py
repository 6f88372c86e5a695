"""CPU oracle for LangBurst's low-bit weight-only projection path.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module, and only as the checker (or, for the CPU baseline, as the
timed restatement of the reference's CPU path).  The shipped package
``neurova_amd`` never calls it; its ops fail loudly when the HIP library is
missing.

Every function restates one piece of the reference algorithm and cites the
reference file:line it follows (paths relative to
``/root/reference/langburst``).  Numerics conventions:

* codes are unsigned integers in ``[0, 2**bits)``; the zero point is implicit:
  ``2**(bits-1)`` for the rowwise layout (``csrc/lowbit_gemv.cu:7``) and ``8``
  for the Marlin layout (``csrc/marlin_cuda_kernel.cu:138-141``);
* dot products are accumulated in float64, i.e. the exact sum of the fp32
  products the reference kernels accumulate in fp32, rounded once to fp16 at
  the end (``lowbit_gemv.cu:67``; ``marlin_cuda_kernel.cu:655-657``).  Any
  fp32 accumulation order lies within a small fraction of one fp16 ulp of it.

Pinning (what checks each function, see ``tests/test_oracle_golden.py``):

* ``rowwise_*`` unpack/pack/dequant: the reference's known-answer vectors
  (``tests/test_v05_cuda_kernels.py:19-32``), its shape invariants
  (``tests/test_quant_lowbit_cpu.py:34-35,63``), the low-nibble-first decode
  (``tests/test_quant_lowbit_cpu.py:18-27``), a brute-force bit-string model
  and round trips; the C restatement ``lowbit_ref.c`` agrees bit for bit.
* ``marlin_perm_tables``/``marlin_unpack_*``: the reference-held inverse tables
  (``csrc/marlin_mlp_stream.cu:7-84``, pinned by SHA-256 in
  ``tests/golden/marlin_tables.json``), bijection/involution invariants and
  ``unpack(pack(c)) == c``; the scalar reader ``marlin_weight_read`` agrees with
  the vectorised unpack.
* ``marlin_gemm``/``rowwise_gemv``: one-hot inputs reproduce single weights,
  linearity in ``x``, and agreement with an independent float64 reference.
* ``silu_mul_packed`` / ``marlin_gemm_argmax`` / ``marlin_mlp_streaming``:
  compositions of the above with closed forms (SiLU) and ``numpy.argmax``'s
  first-index rule, checked on hand-built cases.
"""
from __future__ import annotations

import math

import numpy as np

__all__ = [
    "rowwise_packed_cols",
    "rowwise_code",
    "rowwise_pack",
    "rowwise_unpack",
    "rowwise_dequant_f32",
    "rowwise_row_dequant",
    "rowwise_gemv",
    "rowwise_gemm",
    "marlin_perm_tables",
    "marlin_inverse_tables",
    "marlin_pack_codes",
    "marlin_unpack_codes",
    "marlin_pack_scales",
    "marlin_unpack_scales",
    "marlin_weight_read",
    "marlin_dequant_f16",
    "marlin_gemm",
    "silu_f32",
    "silu_mul_packed",
    "marlin_gemm_silu_packed",
    "argmax_key",
    "marlin_gemm_argmax",
    "marlin_mlp_streaming",
    "make_rowwise_inputs",
    "make_marlin_inputs",
    "marlin_bytes",
    "rowwise_bytes",
]


# ---------------------------------------------------------------------------
# Rowwise "lowbit_symmetric_groupwise" layout
# ---------------------------------------------------------------------------

def rowwise_packed_cols(cols: int, bits: int) -> int:
    """``ceil(cols*bits/8)`` bytes per row (``quantize.py:139``)."""
    return (int(cols) * int(bits) + 7) // 8


def rowwise_code(row: np.ndarray, c: int, bits: int) -> int:
    """Signed code ``c`` of one packed row.

    Restates ``qb_lowbit_value<BITS>`` (``csrc/lowbit_gemv.cu:4-14``) and the
    CPU twin ``lowbit_reference.py:13-21``: read a 16-bit little-endian window
    at byte ``c*bits >> 3``, shift by ``c*bits & 7``, mask ``bits`` bits and
    subtract the zero point ``2**(bits-1)``.
    """
    bit_pos = c * bits
    byte_i = bit_pos >> 3
    shift = bit_pos & 7
    word = int(row[byte_i])
    if shift + bits > 8 and byte_i + 1 < row.shape[0]:
        word |= int(row[byte_i + 1]) << 8
    return ((word >> shift) & ((1 << bits) - 1)) - (1 << (bits - 1))


def rowwise_pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack unsigned codes ``[rows, cols]`` into ``uint8 [rows, ceil(cols*bits/8)]``.

    Restates the LSB-first bitstream writer of ``quantize_symmetric_lowbit``
    (``adapters/qwen36_tools/quantize.py:165-173``): code ``c`` occupies bits
    ``[c*bits, c*bits+bits)`` of the row's little-endian byte stream.
    """
    codes = np.asarray(codes)
    rows, cols = codes.shape
    pc = rowwise_packed_cols(cols, bits)
    out = np.zeros((rows, pc), dtype=np.uint8)
    vals_all = codes.astype(np.uint16)
    for c in range(cols):
        bit_pos = c * bits
        byte_i = bit_pos // 8
        shift = bit_pos % 8
        vals = vals_all[:, c]
        out[:, byte_i] |= ((vals << shift) & 0xFF).astype(np.uint8)
        spill = shift + bits - 8
        if spill > 0 and byte_i + 1 < pc:
            out[:, byte_i + 1] |= (vals >> (bits - spill)).astype(np.uint8)
    return out


def rowwise_unpack(packed: np.ndarray, cols: int, bits: int) -> np.ndarray:
    """Unsigned codes ``uint8 [rows, cols]`` of a packed rowwise matrix.

    Vectorised form of ``qb_lowbit_value`` (``csrc/lowbit_gemv.cu:4-14``)
    without the zero-point subtraction.  Rows may carry padding bytes beyond
    ``ceil(cols*bits/8)`` (the op boundary only requires ``>=``,
    ``lowbit_gemv.cu:267``).
    """
    packed = np.asarray(packed, dtype=np.uint8)
    rows, pc = packed.shape
    c = np.arange(cols, dtype=np.int64)
    bit_pos = c * bits
    byte_i = bit_pos >> 3
    shift = (bit_pos & 7).astype(np.uint16)
    lo = packed[:, byte_i].astype(np.uint16)
    nxt = np.minimum(byte_i + 1, pc - 1)
    straddle = (shift + bits) > 8
    hi = np.where(straddle[None, :], packed[:, nxt].astype(np.uint16) << 8, 0).astype(np.uint16)
    word = lo | hi
    return ((word >> shift[None, :]) & ((1 << bits) - 1)).astype(np.uint8)


def rowwise_dequant_f32(packed: np.ndarray, scales: np.ndarray, cols: int, group_size: int, bits: int) -> np.ndarray:
    """``(q - 2**(bits-1)) * fp32(scale[row, c // group_size])`` as float32.

    Restates ``lowbit_reference.py:7-23``; the product of a small integer and
    an fp16 scale is exact in float32, as in the kernel (``lowbit_gemv.cu:42-43``).
    """
    q = rowwise_unpack(packed, cols, bits).astype(np.int32) - (1 << (bits - 1))
    s = np.asarray(scales, dtype=np.float16).astype(np.float32)
    gidx = np.arange(cols) // int(group_size)
    return q.astype(np.float32) * s[:, gidx]


def rowwise_row_dequant(packed: np.ndarray, scales: np.ndarray, row: int, cols: int, group_size: int, bits: int) -> np.ndarray:
    """One dequantised row as fp16 ``[cols]``.

    Restates ``lowbit_row_dequant_kernel`` (``csrc/lowbit_gemv.cu:226-248``):
    an out-of-range row index yields zeros (``:239-243``); otherwise
    ``fp16_rn(float(q) * float(s))``.
    """
    rows = packed.shape[0]
    if row < 0 or row >= rows:
        return np.zeros((cols,), dtype=np.float16)
    w = rowwise_dequant_f32(packed[row:row + 1], scales[row:row + 1], cols, group_size, bits)[0]
    return w.astype(np.float16)


def rowwise_gemm(packed: np.ndarray, scales: np.ndarray, x: np.ndarray, cols: int, group_size: int, bits: int) -> np.ndarray:
    """``Y[M, N] = fp16(X[:, :cols] @ dequant(W)^T)`` with exact accumulation.

    Restates ``lowbit_gemm_kernel`` (``csrc/lowbit_gemv.cu:145-224``): each
    term ``(q*s)*x`` in fp32, summed in fp32, rounded with
    ``__float2half_rn``.  The sum is taken in float64 here.
    """
    w = rowwise_dequant_f32(packed, scales, cols, group_size, bits).astype(np.float64)
    x64 = np.asarray(x, dtype=np.float16)[:, :cols].astype(np.float64)
    return (x64 @ w.T).astype(np.float16)


def rowwise_gemv(packed: np.ndarray, scales: np.ndarray, x: np.ndarray, cols: int, group_size: int, bits: int) -> np.ndarray:
    """``y[N] = fp16(dequant(W) @ x[:cols])``.

    Restates ``lowbit_gemv_kernel`` (``csrc/lowbit_gemv.cu:16-70``) and the CPU
    fallback ``CPUFallbackOps.lowbit_gemv`` (``langburst/ops.py:16-44``).
    """
    return rowwise_gemm(packed, scales, np.asarray(x).reshape(1, -1), cols, group_size, bits)[0]


# ---------------------------------------------------------------------------
# Marlin "lowbit_marlin_groupwise" / layout "marlin_v1"
# ---------------------------------------------------------------------------

def marlin_perm_tables() -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """The weight permutation (1024), group-scale permutation (64) and
    per-column scale permutation (32) of the Marlin format.

    Restates ``_marlin_perms`` (``adapters/qwen36_tools/quantize.py:50-76``):
    for each of the 32 fragment owners ``i`` the 8 entries
    ``16*row + i//4 + 8*block`` (rows ``2(i%4), 2(i%4)+1, 2(i%4)+8, 2(i%4)+9``,
    blocks 0/1) repeated for the four 256-entry tiles, then each run of 8
    interleaved ``[0,2,4,6,1,3,5,7]``.
    """
    perm = []
    for i in range(32):
        col = i // 4
        perm1 = []
        for block in (0, 1):
            for row in (2 * (i % 4), 2 * (i % 4) + 1, 2 * (i % 4 + 4), 2 * (i % 4 + 4) + 1):
                perm1.append(16 * row + col + 8 * block)
        for j in range(4):
            perm.extend(p + 256 * j for p in perm1)
    perm = np.array(perm, dtype=np.int64).reshape(-1, 8)[:, [0, 2, 4, 6, 1, 3, 5, 7]].ravel()
    scale_perm = np.array([i + 8 * j for i in range(8) for j in range(8)], dtype=np.int64)
    scale_perm_single = np.array([2 * i + j for i in range(4) for j in (0, 1, 8, 9, 16, 17, 24, 25)], dtype=np.int64)
    return perm, scale_perm, scale_perm_single


def marlin_inverse_tables() -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Inverses of :func:`marlin_perm_tables`.

    These are the tables the reference holds as constants in
    ``csrc/marlin_mlp_stream.cu:7-84`` (``LB_MARLIN_INV_PERM``,
    ``LB_MARLIN_INV_SCALE_PERM``, ``LB_MARLIN_INV_SCALE_PERM_SINGLE``).
    """
    out = []
    for p in marlin_perm_tables():
        inv = np.empty_like(p)
        inv[p] = np.arange(p.size)
        out.append(inv)
    return tuple(out)  # type: ignore[return-value]


def marlin_pack_codes(codes_kn: np.ndarray) -> np.ndarray:
    """Pack unsigned 4-bit codes ``[K, N]`` (``W^T``) into ``int32 [K/16, 2N]``.

    Restates ``quantize_marlin4_groupwise`` (``quantize.py:224-230``): 16x16
    tile transpose ``(K/16,16,N/16,16) -> (K/16,N/16,16,16)``, the 1024-entry
    permutation per 1024-nibble run, then eight consecutive nibbles per int32
    (nibble ``i`` at bits ``4i``).  Chunking over output columns
    (``quantize.py:200-231``) does not change the result because chunk widths
    are multiples of 256 columns.
    """
    codes_kn = np.asarray(codes_kn)
    K, N = codes_kn.shape
    if K % 16 or N % 64:
        raise ValueError("Marlin packing needs K % 16 == 0 and N % 64 == 0")
    perm, _, _ = marlin_perm_tables()
    q = codes_kn.astype(np.uint32).reshape(K // 16, 16, N // 16, 16).transpose(0, 2, 1, 3).reshape(K // 16, N * 16)
    q = q.reshape(-1, 1024)[:, perm].reshape(K // 16, N * 16)
    packed = np.zeros((K // 16, N * 2), dtype=np.uint32)
    for i in range(8):
        packed |= q[:, i::8] << np.uint32(4 * i)
    return packed.view(np.int32)


def marlin_unpack_codes(qweight: np.ndarray) -> np.ndarray:
    """Unsigned 4-bit codes ``uint8 [K, N]`` of a Marlin ``qweight``.

    Vectorised form of ``lb_marlin_weight_read`` (``csrc/marlin_mlp_stream.cu:109-133``):
    ``pre = (n>>4)*256 + (k&15)*16 + (n&15)``,
    ``fin = (pre//1024)*1024 + INV_PERM[pre % 1024]``,
    code = nibble ``fin & 7`` of ``qweight[k>>4, fin>>3]``.
    """
    qweight = np.asarray(qweight).view(np.uint32)
    KB, N2 = qweight.shape
    K, N = KB * 16, N2 // 2
    inv, _, _ = marlin_inverse_tables()
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    pre = (n >> 4) * 256 + (k & 15) * 16 + (n & 15)
    fin = (pre // 1024) * 1024 + inv[pre % 1024]
    words = qweight[k >> 4, fin >> 3]
    return ((words >> (4 * (fin & 7)).astype(np.uint32)) & 0xF).astype(np.uint8)


def marlin_pack_scales(scales: np.ndarray, per_column: bool = False) -> np.ndarray:
    """Permute fp16 scales ``[groups, N]`` into the Marlin order.

    Restates ``quantize.py:211-219``: ``s.reshape(-1, 64)[:, scale_perm]`` for
    group-wise scales, ``s.reshape(-1, 32)[:, scale_perm_single]`` for
    per-column scales.
    """
    s = np.asarray(scales, dtype=np.float16)
    _, sp, sps = marlin_perm_tables()
    p = sps if per_column else sp
    return s.reshape(-1, p.size)[:, p].reshape(s.shape).copy()


def marlin_unpack_scales(scales_perm: np.ndarray, per_column: bool = False) -> np.ndarray:
    """Natural-order fp16 scales ``[groups, N]``.

    Restates ``lb_marlin_scale_read`` (``csrc/marlin_mlp_stream.cu:91-107``):
    ``scales[(flat//64)*64 + INV_SCALE_PERM[flat%64]]`` with
    ``flat = group*N + n`` (``//32`` and ``INV_SCALE_PERM_SINGLE`` per column).
    """
    s = np.asarray(scales_perm, dtype=np.float16)
    _, isp, isps = marlin_inverse_tables()
    p = isps if per_column else isp
    flat = s.reshape(-1)
    idx = np.arange(flat.size)
    return flat[(idx // p.size) * p.size + p[idx % p.size]].reshape(s.shape)


def marlin_weight_read(qweight: np.ndarray, scales: np.ndarray, out_col: int, in_col: int, prob_n: int, group_size: int) -> float:
    """Scalar ``(q - 8) * scale`` in float32 for one weight.

    Direct restatement of ``lb_marlin_weight_read`` (``csrc/marlin_mlp_stream.cu:109-133``)
    with ``lb_marlin_scale_read`` (``:91-107``); ``group_size == -1`` means one
    scale per column.
    """
    inv, isp, isps = marlin_inverse_tables()
    kblock, kinner = in_col >> 4, in_col & 15
    nblock, ninner = out_col >> 4, out_col & 15
    pre = nblock * 256 + kinner * 16 + ninner
    fin = (pre // 1024) * 1024 + int(inv[pre % 1024])
    word = int(np.asarray(qweight).view(np.uint32)[kblock, fin >> 3])
    q = ((word >> (4 * (fin & 7))) & 0xF) - 8
    flat_s = np.asarray(scales, dtype=np.float16).reshape(-1)
    if group_size == -1:
        base = (out_col // 32) * 32
        s = flat_s[base + int(isps[out_col - base])]
    else:
        flat = (in_col // group_size) * prob_n + out_col
        base = (flat // 64) * 64
        s = flat_s[base + int(isp[flat - base])]
    return float(np.float32(q) * np.float32(s))


def _normalize_group(group_size: int, K: int) -> int:
    """``groupsize <= 0 or == K`` means per-column (``langburst_ext.cpp:87``)."""
    g = int(group_size)
    return -1 if (g <= 0 or g == K) else g


def marlin_dequant_f16(qweight: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """Dequantised ``W^T`` as fp16 ``[K, N]`` with the kernel's rounding.

    Grouped scales: ``fp16(fp16(q - 8) * s)`` -- the kernel forms ``q - 8``
    exactly in fp16 and multiplies by the fp16 scale with ``__hmul2``
    (``csrc/marlin_cuda_kernel.cu:131-159``).  Per-column scales: the kernel
    multiplies only at the output (``:651-659``), so the weight is ``q - 8``.
    """
    codes = marlin_unpack_codes(qweight)
    K, N = codes.shape
    g = _normalize_group(group_size, K)
    q = (codes.astype(np.int16) - 8).astype(np.float16)
    if g == -1:
        return q
    s = marlin_unpack_scales(scales).astype(np.float16)
    return (q * s[np.arange(K) // g, :]).astype(np.float16)


def marlin_gemm(x: np.ndarray, qweight: np.ndarray, scales: np.ndarray, group_size: int, rows: np.ndarray | None = None) -> np.ndarray:
    """``C[M, N] = A[M, K] @ dequant(B)`` as fp16, the Marlin op's result.

    Restates ``Marlin<>`` (``csrc/marlin_cuda_kernel.cu:227-848``): fp16
    weights as in :func:`marlin_dequant_f16`, fp32 MMA accumulation
    (``:92-104``), ``__float2half`` at write-out (``:651-659``); per-column
    scales are applied after that rounding with an fp16 multiply (``:654-655``).
    ``rows`` optionally restricts the computation to a subset of ``A``'s rows.
    """
    a = np.asarray(x, dtype=np.float16)
    if rows is not None:
        a = a[np.asarray(rows)]
    K = a.shape[1]
    g = _normalize_group(group_size, K)
    w = marlin_dequant_f16(qweight, scales, g).astype(np.float64)
    acc = a.astype(np.float64) @ w
    out = acc.astype(np.float16)
    if g == -1:
        s = marlin_unpack_scales(scales, per_column=True).reshape(-1).astype(np.float16)
        out = (out * s[None, :]).astype(np.float16)
    return out


def marlin_gemm_exact(x: np.ndarray, qweight: np.ndarray, scales: np.ndarray, group_size: int,
                      rows: np.ndarray | None = None) -> np.ndarray:
    """The Marlin product without the reference's per-weight rounding.

    ``fp16(sum_k x * (q - 8) * s)`` with every product and sum in float64 (per
    column scales: as in :func:`marlin_gemm`, applied after the fp16 rounding).
    This is the mathematical value both :func:`marlin_gemm` (which rounds each
    ``fp16((q-8)*s)`` first, ``marlin_cuda_kernel.cu:131-159``) and an
    implementation that scales each group's exact fp32 sum approximate; it
    equals :func:`marlin_gemm` whenever every ``(q-8)*s`` is representable in
    fp16 (e.g. power-of-two scales).
    """
    a = np.asarray(x, dtype=np.float16)
    if rows is not None:
        a = a[np.asarray(rows)]
    K = a.shape[1]
    g = _normalize_group(group_size, K)
    if g == -1:
        return marlin_gemm(x, qweight, scales, group_size, rows)
    q = marlin_unpack_codes(qweight).astype(np.float64) - 8.0
    s = marlin_unpack_scales(scales).astype(np.float64)
    w = q * s[np.arange(K) // g, :]
    return (a.astype(np.float64) @ w).astype(np.float16)


def silu_f32(v: np.ndarray) -> np.ndarray:
    """``x / (1 + exp(-x))`` in float32 (``marlin_cuda_kernel.cu:205-207``)."""
    v = np.asarray(v, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (v / (np.float32(1.0) + np.exp(-v))).astype(np.float32)


def silu_mul_packed(mixed: np.ndarray, cols: int) -> np.ndarray:
    """``fp16(silu(mixed[:, :K]) * mixed[:, K:2K])``.

    Restates ``marlin_silu_packed_a_vec`` (``csrc/marlin_cuda_kernel.cu:209-224``)
    and the CPU composite ``CPUFallbackOps.silu_mul_packed`` (``ops.py:103-114``).
    """
    m = np.asarray(mixed, dtype=np.float16)
    g = m[:, :cols].astype(np.float32)
    u = m[:, cols:2 * cols].astype(np.float32)
    return (silu_f32(g) * u).astype(np.float16)


def marlin_gemm_silu_packed(mixed: np.ndarray, qweight: np.ndarray, scales: np.ndarray, cols: int, group_size: int) -> np.ndarray:
    """Marlin GEMM with the SiLU-gated A prologue (``langburst_ext.cpp:131-185``)."""
    return marlin_gemm(silu_mul_packed(mixed, cols), qweight, scales, group_size)


def argmax_key(values_f16: np.ndarray) -> np.ndarray:
    """Packed ordering key of the fused argmax, per element.

    Restates ``marlin_argmax_ordered_float``/``marlin_argmax_pack``
    (``csrc/marlin_cuda_kernel.cu:189-199``): the float's bits made
    order-preserving in the high word and ``0xffffffff - idx`` in the low word,
    so the maximum key is the largest value with the smallest index.
    """
    v = np.asarray(values_f16, dtype=np.float16).astype(np.float32)
    bits = v.view(np.uint32).astype(np.uint64)
    neg = (bits & np.uint64(0x80000000)) != 0
    ordered = np.where(neg, (~bits) & np.uint64(0xFFFFFFFF), bits ^ np.uint64(0x80000000))
    idx = np.arange(v.shape[-1], dtype=np.uint64)
    return (ordered << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)


def marlin_gemm_argmax(x: np.ndarray, qweight: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """Row-wise argmax of the fp16 Marlin output with the fused-epilogue tie rule.

    Restates the argmax epilogue (``csrc/marlin_cuda_kernel.cu:685-749,833-847``)
    and its CPU composite (``ops.py:116-134``).  For finite outputs without
    signed zeros this equals ``numpy.argmax`` (first maximal index).
    """
    y = marlin_gemm(x, qweight, scales, group_size)
    keys = argmax_key(y)
    best = keys.max(axis=1)
    return (np.uint64(0xFFFFFFFF) - (best & np.uint64(0xFFFFFFFF))).astype(np.int64)


def marlin_mlp_streaming(x: np.ndarray, gate_up_qweight: np.ndarray, gate_up_scales: np.ndarray,
                         down_qweight: np.ndarray, down_scales: np.ndarray, hidden: int, intermediate: int,
                         gate_group_size: int, down_group_size: int) -> np.ndarray:
    """gate_up -> SiLU gate -> down, with the streaming kernel's numerics.

    Restates ``lowbit_marlin_mlp_streaming_kernel``
    (``csrc/marlin_mlp_stream.cu:135-217``): weights are read as float32
    ``(q-8)*s`` without fp16 rounding (``:109-133``), gate/up dot products and
    ``act = silu(gate) * up`` stay in float32 (``:180-198``), the down
    projection accumulates ``w * act`` in float32 (``:200-203``), and only the
    final store rounds to fp16 (``:213-215``).
    """
    gg = _normalize_group(gate_group_size, hidden)
    dg = _normalize_group(down_group_size, intermediate)

    def dense_f32(qw, sc, g, K):
        codes = marlin_unpack_codes(qw).astype(np.float32) - np.float32(8)
        if g == -1:
            s = marlin_unpack_scales(sc, per_column=True).reshape(1, -1).astype(np.float32)
            return codes * s
        s = marlin_unpack_scales(sc).astype(np.float32)
        return codes * s[np.arange(K) // g, :]

    xg = np.asarray(x, dtype=np.float16).astype(np.float64)
    wgu = dense_f32(gate_up_qweight, gate_up_scales, gg, hidden).astype(np.float64)  # [hidden, 2I]
    gu = (xg @ wgu).astype(np.float32)
    act = (silu_f32(gu[:, :intermediate]) * gu[:, intermediate:]).astype(np.float32)
    wd = dense_f32(down_qweight, down_scales, dg, intermediate).astype(np.float64)  # [I, hidden]
    return (act.astype(np.float64) @ wd).astype(np.float16)


# ---------------------------------------------------------------------------
# Synthetic inputs (value distributions of BASELINE.json configs)
# ---------------------------------------------------------------------------

def make_rowwise_inputs(rows: int, cols: int, bits: int, group_size: int, batch: int = 1, seed: int = 0):
    """Seeded rowwise problem: codes uniform in ``[0, 2**bits)``, fp16 scales
    ``|N(0, 0.01)| + 1e-3`` per group, activations fp16 ``N(0, 1)``.
    Draw order: codes, scales, x.  Returns ``(codes, packed, scales, x)``.
    """
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << bits, size=(rows, cols), dtype=np.uint8)
    n_groups = math.ceil(cols / group_size)
    scales = (np.abs(rng.normal(0.0, 0.01, size=(rows, n_groups))) + 1e-3).astype(np.float16)
    x = rng.normal(0.0, 1.0, size=(batch, cols)).astype(np.float16)
    return codes, rowwise_pack(codes, bits), scales, x


def make_marlin_inputs(m: int, k: int, n: int, group_size: int = 128, seed: int = 0):
    """Seeded Marlin problem: codes ``[K, N]`` uniform in ``[0, 16)``, fp16
    scales ``|N(0, 0.01)| + 1e-3`` per (group, column), activations fp16
    ``N(0, 1)``.  Draw order: codes, scales, x.  Returns
    ``(codes_kn, qweight, scales_natural, scales_marlin, x)``.
    """
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, size=(k, n), dtype=np.uint8)
    per_col = group_size <= 0 or group_size == k
    groups = 1 if per_col else k // group_size
    s = (np.abs(rng.normal(0.0, 0.01, size=(groups, n))) + 1e-3).astype(np.float16)
    x = rng.normal(0.0, 1.0, size=(m, k)).astype(np.float16)
    return codes, marlin_pack_codes(codes), s, marlin_pack_scales(s, per_column=per_col), x


# ---------------------------------------------------------------------------
# Algorithmic work per call (roofline numerators)
# ---------------------------------------------------------------------------

def marlin_bytes(m: int, k: int, n: int, group_size: int = 128) -> int:
    """``K*N/2 + (K/g)*N*2 + M*K*2 + M*N*2`` bytes."""
    groups = 1 if (group_size <= 0 or group_size == k) else k // group_size
    return k * n // 2 + groups * n * 2 + m * k * 2 + m * n * 2


def rowwise_bytes(m: int, k: int, n: int, bits: int, group_size: int) -> int:
    """``N*ceil(K*b/8) + N*ceil(K/g)*2 + M*K*2 + M*N*2`` bytes."""
    return n * rowwise_packed_cols(k, bits) + n * math.ceil(k / group_size) * 2 + m * k * 2 + m * n * 2
