"""Parity of the gfx950 rowwise 2..8-bit kernels with the CPU oracle.

Follows the reference's tests langburst/tests/test_lowbit_gemv_cuda.py:14-73
(GEMV vs CPU dequant, pair == two singles, GEMM == repeated GEMV) and
langburst/tests/test_v05_cuda_kernels.py:19-32 (row dequant known answers),
at the reference's odd sizes (K = 513, 257, 259) and the full sizes of BASELINE.json.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from tests.gpu_util import assert_close_f16, print_case, to_dev, to_np

pytestmark = pytest.mark.gpu


def _gemv(dev, packed, scales, x, cols, group, bits):
    import torch
    from neurova_amd import capi

    y = torch.full((packed.shape[0],), float("nan"), dtype=torch.float16, device=dev)
    st = capi.lowbit_gemv(to_dev(packed, dev), to_dev(scales, dev), to_dev(x, dev), y, cols, group, bits)
    assert st == 0, capi.status_string(st)
    return to_np(y)


def test_row_dequant_reference_kats(dev, golden_dir):
    import torch
    import langburst_cuda as lc

    kats = json.loads((golden_dir / "rowwise_kats.json").read_text())
    for case in kats["row_dequant_scale_one"]:
        q = torch.tensor([case["packed"]], dtype=torch.uint8, device=dev)
        s = torch.ones((1, 1), dtype=torch.float16, device=dev)
        row = torch.tensor(0, dtype=torch.long, device=dev)
        out = lc.lowbit_row_dequant(q, s, row, len(case["expected"]), 128, case["bits"])
        assert out.cpu().tolist() == case["expected"]


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 7, 8])
def test_row_dequant_bit_exact(dev, bits):
    import torch
    from neurova_amd import capi

    _, packed, scales, _ = O.make_rowwise_inputs(11, 700, bits, 64, seed=bits)
    q, s = to_dev(packed, dev), to_dev(scales, dev)
    for r in (0, 5, 10, 11, -1):
        out = torch.empty((700,), dtype=torch.float16, device=dev)
        row = torch.tensor([r], dtype=torch.int64, device=dev)
        assert capi.lowbit_row_dequant(q, s, row, out, 700, 64, bits) == 0
        ref = O.rowwise_row_dequant(packed, scales, r, 700, 64, bits)
        assert np.array_equal(to_np(out).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("rows,cols,group", [(37, 513, 128), (41, 257, 128), (64, 1024, 64), (300, 4096, 128), (8, 96, 32)])
def test_gemv_vs_oracle(dev, bits, rows, cols, group):
    print_case("gemv", bits, rows, cols, group)
    _, packed, scales, x = O.make_rowwise_inputs(rows, cols, bits, group, seed=bits * 7 + rows)
    got = _gemv(dev, packed, scales, x[0], cols, group, bits)
    assert_close_f16(got, O.rowwise_gemv(packed, scales, x[0], cols, group, bits), what=f"b{bits} {rows}x{cols} g{group}")


def _pad_rows(packed, mult):
    """Row stride padded to a multiple of `mult` bytes with junk (packed_cols >= need is allowed)."""
    pad = (-packed.shape[1]) % mult
    junk = np.full((packed.shape[0], pad), 0xA5, dtype=np.uint8)
    return np.ascontiguousarray(np.concatenate([packed, junk], axis=1))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("rows,cols,group", [(37, 513, 128), (1, 259, 32), (6, 8192 + 96, 64), (301, 17408 + 7, 128)])
def test_gemv_padded_stride_vs_oracle(dev, bits, rows, cols, group):
    """Dword-multiple row strides take the batch-1 multi-row kernel: a partial last
    32-code unit, an odd row count (last wave half empty), junk past each row's codes."""
    print_case("gemv-padded", bits, rows, cols, group)
    _, packed, scales, x = O.make_rowwise_inputs(rows, cols, bits, group, seed=bits * 11 + rows)
    padded = _pad_rows(packed, 4)
    got = _gemv(dev, padded, scales, x[0], cols, group, bits)
    assert_close_f16(got, O.rowwise_gemv(packed, scales, x[0], cols, group, bits), what=f"b{bits} {rows}x{cols} g{group}")


@pytest.mark.parametrize("bits", [2, 5, 8])
def test_pair_padded_equals_two_singles(dev, bits):
    import torch
    import langburst_cuda as lc

    cols = 1000
    _, pa, sa, x = O.make_rowwise_inputs(33, cols, bits, 64, seed=170 + bits)
    _, pb, sb, _ = O.make_rowwise_inputs(33, cols, bits, 64, seed=180 + bits)
    qa, qb, sca, scb, xd = (to_dev(a, dev) for a in (_pad_rows(pa, 4), _pad_rows(pb, 4), sa, sb, x[0]))
    ya = lc.lowbit_gemv(qa, sca, xd, cols, 64, bits)
    yb = lc.lowbit_gemv(qb, scb, xd, cols, 64, bits)
    pa_out, pb_out = lc.lowbit_gemv_pair(qa, sca, qb, scb, xd, cols, 64, bits)
    torch.cuda.synchronize()
    assert torch.equal(pa_out, ya) and torch.equal(pb_out, yb)
    assert_close_f16(to_np(pb_out), O.rowwise_gemv(pb, sb, x[0], cols, 64, bits))


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("rows,cols,group", [(41, 2048, 128), (7, 5120, 64), (96, 1024, 32), (19, 17408, 128)])
def test_pair_whole_units_equals_two_singles(dev, bits, rows, cols, group):
    """Whole 32-code units and one activation row: the pair takes the LDS-staged
    kernel with both matrices per wave; each output equals its single GEMV.  At
    2 bits, K = 5120 and 17408 end on a step of 32 units, which runs as half
    units (one 16-code word per lane)."""
    import torch
    import langburst_cuda as lc

    print_case("pair-units", bits, rows, cols, group)
    _, pa, sa, x = O.make_rowwise_inputs(rows, cols, bits, group, seed=270 + bits + rows)
    _, pb, sb, _ = O.make_rowwise_inputs(rows, cols, bits, group, seed=280 + bits + rows)
    qa, qb, sca, scb, xd = (to_dev(a, dev) for a in (pa, pb, sa, sb, x[0]))
    ya = lc.lowbit_gemv(qa, sca, xd, cols, group, bits)
    yb = lc.lowbit_gemv(qb, scb, xd, cols, group, bits)
    pa_out, pb_out = lc.lowbit_gemv_pair(qa, sca, qb, scb, xd, cols, group, bits)
    torch.cuda.synchronize()
    assert torch.equal(pa_out, ya) and torch.equal(pb_out, yb)
    assert_close_f16(to_np(pa_out), O.rowwise_gemv(pa, sa, x[0], cols, group, bits), what="pair a")
    assert_close_f16(to_np(pb_out), O.rowwise_gemv(pb, sb, x[0], cols, group, bits), what="pair b")


@pytest.mark.parametrize("bits", [3, 4])
def test_pair_equals_two_singles(dev, bits):
    import torch
    import langburst_cuda as lc

    _, pa, sa, x = O.make_rowwise_inputs(41, 257, bits, 128, seed=70 + bits)
    _, pb, sb, _ = O.make_rowwise_inputs(41, 257, bits, 128, seed=80 + bits)
    qa, qb, sca, scb, xd = (to_dev(a, dev) for a in (pa, pb, sa, sb, x[0]))
    ya = lc.lowbit_gemv(qa, sca, xd, 257, 128, bits)
    yb = lc.lowbit_gemv(qb, scb, xd, 257, 128, bits)
    pa_out, pb_out = lc.lowbit_gemv_pair(qa, sca, qb, scb, xd, 257, 128, bits)
    torch.cuda.synchronize()
    assert torch.equal(pa_out, ya) and torch.equal(pb_out, yb)
    assert_close_f16(to_np(ya), O.rowwise_gemv(pa, sa, x[0], 257, 128, bits))


@pytest.mark.parametrize("bits", [3, 4, 8])
@pytest.mark.parametrize("cols", [259, 2048])
@pytest.mark.parametrize("batch", [1, 2, 5, 16])
def test_gemm_equals_repeated_gemv(dev, bits, cols, batch):
    import torch
    import langburst_cuda as lc

    _, packed, scales, x = O.make_rowwise_inputs(43, cols, bits, 128, batch=batch, seed=90 + bits)
    q, s, xd = to_dev(packed, dev), to_dev(scales, dev), to_dev(x, dev)
    y = lc.lowbit_gemm(q, s, xd, cols, 128, bits)
    rep = torch.stack([lc.lowbit_gemv(q, s, xd[i], cols, 128, bits) for i in range(batch)])
    torch.cuda.synchronize()
    if batch == 1 or cols % 32:
        assert torch.equal(y, rep)  # the same kernel
    else:
        # a single row of whole 32-code units takes the LDS-staged kernel, whose
        # fp32 sums are ordered differently: both within the parity bar
        assert_close_f16(to_np(rep), O.rowwise_gemm(packed, scales, x, cols, 128, bits), what="repeated gemv")
    assert_close_f16(to_np(y), O.rowwise_gemm(packed, scales, x, cols, 128, bits))


def test_cfg1_full_size(dev):
    """N=K=4096, b4, g128, M=1."""
    _, packed, scales, x = O.make_rowwise_inputs(4096, 4096, 4, 128, seed=0)
    got = _gemv(dev, packed, scales, x[0], 4096, 128, 4)
    exact = assert_close_f16(got, O.rowwise_gemv(packed, scales, x[0], 4096, 128, 4), what="cfg1")
    assert exact > 0.95


@pytest.mark.parametrize("bits,rows,cols", [(8, 5127, 2048), (8, 5140, 1056), (4, 4101, 1024), (4, 4096, 2048)])
def test_wide_workgroup_shapes_vs_oracle(dev, bits, rows, cols):
    """Row counts of at least 20 (8 bits) or 16 (4 bits) rows per CU take the
    one-row kernel on 10-wave workgroups of two rows per wave or on 16-wave
    workgroups; ragged counts leave the last workgroup partly empty."""
    print_case("wide workgroups", bits, rows, cols)
    _, packed, scales, x = O.make_rowwise_inputs(rows, cols, bits, 128, seed=rows)
    got = _gemv(dev, packed, scales, x[0], cols, 128, bits)
    exact = assert_close_f16(got, O.rowwise_gemv(packed, scales, x[0], cols, 128, bits), what=f"b{bits} {rows}x{cols}")
    assert exact > 0.95


@pytest.mark.parametrize("bits", [2, 3, 8])
@pytest.mark.parametrize("group", [64, 128])
def test_cfg4_full_size(dev, bits, group):
    """M=1, K=17408, N=5120, b in {2,3,8}, g in {64,128}."""
    print_case("cfg4", bits, group)
    _, packed, scales, x = O.make_rowwise_inputs(5120, 17408, bits, group, seed=bits + group)
    got = _gemv(dev, packed, scales, x[0], 17408, group, bits)
    exact = assert_close_f16(got, O.rowwise_gemv(packed, scales, x[0], 17408, group, bits), what=f"cfg4 b{bits} g{group}")
    assert exact > 0.95


@pytest.mark.parametrize("bits", [4, 8])
def test_embedding_row_dequant_full_table(dev, bits):
    """The embedding lookup (model.py:359-362): one row of a 248320 x 5120 table
    per token.  The table is drawn on the GPU at full size; sampled rows (first,
    last, interior, and out of range) are checked bit-exact against the oracle."""
    import torch
    import langburst_cuda as lc

    rows, cols, group = 248320, 5120, 128
    gen = torch.Generator(device=dev)
    gen.manual_seed(bits)
    q = torch.randint(0, 256, (rows, cols * bits // 8), dtype=torch.uint8, device=dev, generator=gen)
    s = (torch.randn((rows, cols // group), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
    for r in (0, 1, 4097, 123456, rows - 1, rows, -3):
        out = lc.lowbit_row_dequant(q, s, torch.tensor(r, dtype=torch.long, device=dev), cols, group, bits)
        rr = min(max(r, 0), rows - 1)
        ref = O.rowwise_row_dequant(to_np(q[rr:rr + 1]), to_np(s[rr:rr + 1]), 0 if 0 <= r < rows else -1, cols, group, bits)
        assert np.array_equal(to_np(out).view(np.uint16), ref.view(np.uint16)), f"row {r}"


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [64, 128])
def test_in_proj_ba_shapes(dev, bits, group):
    """The GDN in_proj_ba projections (model.py:227-251, 1510-1521): b and a as
    a pair of 48-row GEMVs over K = 5120, the fused 96-row tensor as one GEMV,
    and as a batched GEMM (MTP verification rows)."""
    import torch
    import langburst_cuda as lc

    cols = 5120
    _, pb, sb, x = O.make_rowwise_inputs(48, cols, bits, group, batch=3, seed=200 + bits + group)
    _, pa, sa, _ = O.make_rowwise_inputs(48, cols, bits, group, seed=210 + bits + group)
    qb, qa, scb, sca, xd = (to_dev(t, dev) for t in (pb, pa, sb, sa, x))
    yb, ya = lc.lowbit_gemv_pair(qb, scb, qa, sca, xd[0], cols, group, bits)
    assert_close_f16(to_np(yb), O.rowwise_gemv(pb, sb, x[0], cols, group, bits), what="in_proj_b")
    assert_close_f16(to_np(ya), O.rowwise_gemv(pa, sa, x[0], cols, group, bits), what="in_proj_a")
    pba, sba = np.concatenate([pb, pa]), np.concatenate([sb, sa])
    qba, scba = to_dev(pba, dev), to_dev(sba, dev)
    yba = lc.lowbit_gemv(qba, scba, xd[0], cols, group, bits)
    torch.cuda.synchronize()
    assert torch.equal(yba[:48], yb) and torch.equal(yba[48:], ya)
    ym = lc.lowbit_gemm(qba, scba, xd, cols, group, bits)
    assert_close_f16(to_np(ym), O.rowwise_gemm(pba, sba, x, cols, group, bits), what="in_proj_ba gemm")


def test_dropin_errors(dev):
    import torch
    import langburst_cuda as lc

    q = torch.zeros((4, 8), dtype=torch.uint8, device=dev)
    s = torch.ones((4, 1), dtype=torch.float16, device=dev)
    x = torch.zeros((16,), dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="rows_per_cta must be one of 4, 8, 16"):
        lc.lowbit_gemv(q, s, x, 16, 128, 4, 5)
    with pytest.raises(RuntimeError, match=r"bits must be in \[2, 8\]"):
        lc.lowbit_gemv(q, s, x, 16, 128, 9)
    with pytest.raises(RuntimeError, match="x cols mismatch"):
        lc.lowbit_gemv(q, s, x[:8].contiguous(), 16, 128, 4)
    with pytest.raises(RuntimeError, match="qweight packed_cols too small"):
        lc.lowbit_gemv(q, s, x, 16, 128, 5)
    for r in (4, 8, 16):
        lc.lowbit_gemv(q, s, x, 16, 128, 4, r)
