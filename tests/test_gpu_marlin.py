"""Parity of the gfx950 Marlin-layout kernels with the CPU oracle.

Calls go through the C ABI (neurova_amd.capi -> liblangburst_lowbit.so) and,
for the drop-in surface, through the ``langburst_cuda`` module.  Bar: dequantised
codes bit-exact; outputs within max-abs 1e-2 / rel 1e-3 of the oracle
(tests/gpu_util.py).  Reference tests followed:
langburst/tests/test_lowbit_gemv_cuda.py:76-102 (Marlin vs dequant-matmul).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from tests.gpu_util import assert_close_f16, assert_reference_rounding, print_case, to_dev, to_np

pytestmark = pytest.mark.gpu


def _ws(dev, n, mult=16):
    import torch

    return torch.zeros((max(1, n // 128 * mult),), dtype=torch.int32, device=dev)


def _scratch(dev, m, n, k, g):
    import torch
    from neurova_amd import capi

    return torch.empty((max(1, capi.marlin_scratch_bytes(m, n, k, g)),), dtype=torch.uint8, device=dev)


def _run_gemm(dev, x, qw, sp, g):
    import torch
    from neurova_amd import capi

    m, k = x.shape
    n = qw.shape[1] // 2
    a, b, s = to_dev(x, dev), to_dev(qw, dev), to_dev(sp, dev)
    c = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    ws = _ws(dev, n)
    st = capi.marlin_gemm(a, b, c, s, ws, g, _scratch(dev, m, n, k, g))
    assert st == 0, capi.status_string(st)
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0, "workspace must be left zero"
    return to_np(c)


@pytest.mark.parametrize("group", [128, -1])
def test_dequant_bit_exact(dev, group):
    import torch
    from neurova_amd import capi

    k, n = 512, 768
    print_case("dequant", k, n, group)
    codes, qw, s_nat, sp, _ = O.make_marlin_inputs(1, k, n, group, seed=21)
    w = torch.empty((n, k), dtype=torch.float16, device=dev)
    assert capi.marlin_dequant(to_dev(qw, dev), to_dev(sp, dev), w, k, group) == 0
    ref = O.marlin_dequant_f16(qw, sp, group).T
    assert np.array_equal(to_np(w).view(np.uint16), np.ascontiguousarray(ref).view(np.uint16))


def _assert_per_column_rounding(got, codes, x, sp):
    """Per-column scales: out = fp16(fp16(sum) * s) (langburst_ext.cpp / the
    Marlin write-out).  The kernel's sum is fp32 (one rounding per 32-k MFMA
    plus the final reduction), so it lies within
    delta = (K/32 + 4) * 2^-24 * sum|x * (q - 8)| of the exact sum; every
    output must lie between fp16(fp16(sum - delta) * s) and
    fp16(fp16(sum + delta) * s) (rounding is monotone)."""
    xd = np.asarray(x, dtype=np.float16).astype(np.float64)
    q = codes.astype(np.float64) - 8.0
    exact = xd @ q
    delta = (xd.shape[1] / 32.0 + 4.0) * 2.0 ** -24 * (np.abs(xd) @ np.abs(q))
    s_col = O.marlin_unpack_scales(sp, per_column=True).reshape(-1).astype(np.float16).astype(np.float64)
    lo_acc = np.nextafter((exact - delta).astype(np.float16), np.float16(-np.inf))
    hi_acc = np.nextafter((exact + delta).astype(np.float16), np.float16(np.inf))
    a = (lo_acc.astype(np.float64) * s_col).astype(np.float16).astype(np.float64)
    b = (hi_acc.astype(np.float64) * s_col).astype(np.float16).astype(np.float64)
    g = np.asarray(got, dtype=np.float64)
    ok = (g >= np.minimum(a, b)) & (g <= np.maximum(a, b))
    assert ok.all(), f"{int((~ok).sum())} outputs outside the fp32-accumulation bound of fp16(sum) * s"


@pytest.mark.parametrize("group", [128, -1])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 16, 17, 24, 32])
@pytest.mark.parametrize("k,n", [(256, 256), (1024, 512), (512, 1280)])
def test_skinny_vs_oracle(dev, m, k, n, group):
    print_case("skinny", m, k, n, group)
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, group, seed=100 + m + k + n)
    got = _run_gemm(dev, x, qw, sp, group)
    ref = O.marlin_gemm(x, qw, sp, group)
    exact = assert_close_f16(got, ref, what=f"m={m} k={k} n={n} g={group}")
    if group == -1:  # per-column scales: fp16(sum) * s, the reference's rounding order
        assert exact > 0.9
        _assert_per_column_rounding(got, codes, x, sp)
    else:
        assert_reference_rounding(got, ref, x, qw, sp, group, what=f"m={m} k={k} n={n}")


@pytest.mark.parametrize("group", [128, -1])
@pytest.mark.parametrize("m,k", [(1, 128), (3, 384), (16, 640), (1, 1024), (7, 2048)])
def test_wide_decode_vs_oracle(dev, m, k, group):
    """Wide output (N = 16384, 64 column groups) with few scale groups: K = 128
    (per-column, g == K), 384, 640 (unequal groups per split) and larger K."""
    n = 16384
    print_case("wide", m, k, n, group)
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, group, seed=500 + m + k)
    got = _run_gemm(dev, x, qw, sp, group)
    ref = O.marlin_gemm(x, qw, sp, group)
    exact = assert_close_f16(got, ref, what=f"wide m={m} k={k} g={group}")
    if group <= 0 or group == k:  # per-column scales (g == K counts as per-column, langburst_ext.cpp:87)
        assert exact > 0.9
        _assert_per_column_rounding(got, codes, x, sp)
    else:
        assert_reference_rounding(got, ref, x, qw, sp, group, what=f"wide m={m} k={k}")


@pytest.mark.parametrize("m,k,n,group", [
    (1, 5120, 17408, 128),
    (2, 5120, 17408, -1),
    (1, 5120, 16640, 128),
    (3, 1024, 16640, 128),
    (1, 2048, 16640, -1),
    (8, 1024, 17408, 128),
    (2, 5120, 17408, 128),
    (3, 5120, 17408, 128),
    (4, 2048, 16640, 128),
    (4, 5120, 16384, 128),
    (1, 5120, 34816, 128),
    (2, 4096, 32768, 128),
    (3, 5120, 33280, 128),
])
def test_wide_decode_leftovers_vs_oracle(dev, m, k, n, group):
    """Decode at N just above 64 columns per CU (16384): 256-column tiles that
    do not divide evenly over the CUs, up to M = 8, both scale modes, and
    repeated launches bit-identical.  The grouped cases take the mixed plan
    (one or two whole-K single-chunk tiles per CU, leftover chunks split): A
    staged at M <= 4, loaded per step at M = 8."""
    print_case("wide-left", m, k, n, group)
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, group, seed=900 + m + k + n)
    got = _run_gemm(dev, x, qw, sp, group)
    ref = O.marlin_gemm(x, qw, sp, group)
    exact = assert_close_f16(got, ref, what=f"wide-left m={m} k={k} n={n} g={group}")
    if group <= 0:
        assert exact > 0.9
        _assert_per_column_rounding(got, codes, x, sp)
    else:
        assert_reference_rounding(got, ref, x, qw, sp, group, what=f"wide-left m={m} k={k} n={n}")
    # repeated launches are bit-identical (split partials are summed in split order)
    again = _run_gemm(dev, x, qw, sp, group)
    assert np.array_equal(got.view(np.uint16), again.view(np.uint16))


@pytest.mark.parametrize("m,k,n", [
    (5, 5120, 17408),   # one whole-K tile per CU, 16 leftover chunks split 6 ways
    (13, 2048, 17408),
    (20, 5120, 16640),  # two 16-row MFMA blocks, rows 20..31 masked; 4 leftover chunks
    (32, 1024, 17408),
    (8, 2048, 34816),   # two whole-K tiles per CU
    (7, 1024, 33024),   # eight k groups: two per wave, the leftover chunks split 2 ways
    (16, 5120, 16384),  # whole-K tiles only, no leftover
    (8, 5120, 14336),   # 224 chunks: one whole-K tile each, 32 CUs idle
    (29, 2048, 10240),  # 160 chunks
])
def test_mixed_direct_vs_oracle(dev, m, k, n):
    """The mixed whole-K plan with A loaded per step (M = 5..32): single-chunk
    tiles over the whole K, at most one per CU (two up to M = 8), their four
    waves' k shares summed in LDS, the leftover chunks split over K; ragged M
    in both 16-row blocks; repeated launches bit-identical."""
    from neurova_amd import capi

    plan = capi.marlin_describe_plan(m, n, k, 128)
    chunks, cus = n // 64, plan["cus"]
    assert plan["form"] == "direct" and plan["chunks_or_row_blocks"] == 1, plan
    assert plan["row_blocks_or_full_tiles"] == (m + 15) // 16, plan
    whole = min(chunks // cus, 2) * cus if chunks >= cus else chunks
    assert plan["workgroups"] == whole + (chunks - whole) * plan["splits"], plan
    print_case("mixed-direct", m, k, n)
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=950 + m + k + n)
    got = _run_gemm(dev, x, qw, sp, 128)
    ref = O.marlin_gemm(x, qw, sp, 128)
    assert_close_f16(got, ref, what=f"mixed-direct m={m} k={k} n={n}")
    assert_reference_rounding(got, ref, x, qw, sp, 128, what=f"mixed-direct m={m} k={k} n={n}")
    again = _run_gemm(dev, x, qw, sp, 128)
    assert np.array_equal(got.view(np.uint16), again.view(np.uint16))


@pytest.mark.parametrize("m", [1, 3, 32])
def test_wide_silu_packed_vs_oracle(dev, m):
    import torch
    from neurova_amd import capi

    k, n = 2048, 17408
    print_case("wide-silu", m, k, n)
    _, qw, _, sp, _ = O.make_marlin_inputs(m, k, n, 128, seed=70 + m)
    mixed = np.random.default_rng(70 + m).normal(0, 1, (m, 2 * k)).astype(np.float16)
    c = torch.empty((m, n), dtype=torch.float16, device=dev)
    ws = _ws(dev, n)
    st = capi.marlin_gemm_silu_packed(to_dev(mixed, dev), to_dev(qw, dev), c, to_dev(sp, dev), ws, 128,
                                      _scratch(dev, m, n, k, 128))
    assert st == 0
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0
    assert_close_f16(to_np(c), O.marlin_gemm_silu_packed(mixed, qw, sp, k, 128), what=f"wide-silu m={m}")


@pytest.mark.parametrize("m", [17, 31, 32, 33, 64, 100, 256, 300])
def test_gemm_vs_oracle(dev, m):
    k, n = 1024, 768
    print_case("gemm", m, k, n)
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=300 + m)
    got = _run_gemm(dev, x, qw, sp, 128)
    ref = O.marlin_gemm(x, qw, sp, 128)
    exact = assert_close_f16(got, ref, what=f"m={m}")
    if m <= 32:  # decode kernel (M = 17..32: A fragments loaded per step)
        assert_reference_rounding(got, ref, x, qw, sp, 128, what=f"m={m}")
    else:  # prefill kernel: the reference's fp16 (q - 8) * s weights
        assert exact > 0.95


@pytest.mark.parametrize("m,k,n,group", [(40, 8192, 1024, 128), (64, 17408, 1280, -1), (100, 4096, 2048, 128),
                                         (128, 5120, 4352, 128), (256, 8192, 2048, -1)])
def test_gemm_split_collect_vs_oracle(dev, m, k, n, group):
    """Prefill tiles split over K (3 to 8 ways): below 128 rows the last
    arrival of a tile reads every split (its own included) in batches, on
    128-row tiles one split per round trip with its own from registers; both
    sum in split order.  Both scale modes, repeated launches bit-identical."""
    print_case("gemm-collect", m, k, n, group)
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, group, seed=2100 + m)
    got = _run_gemm(dev, x, qw, sp, group)
    exact = assert_close_f16(got, O.marlin_gemm(x, qw, sp, group), what=f"gemm-collect m={m} k={k} n={n} g={group}")
    assert exact > 0.9
    again = _run_gemm(dev, x, qw, sp, group)
    assert np.array_equal(got.view(np.uint16), again.view(np.uint16))


@pytest.mark.parametrize("m,k,n,group", [(256, 5120, 17408, 128), (384, 17408, 5120, 128), (200, 16384, 4096, -1)])
def test_gemm_all_tiles_split_vs_oracle(dev, m, k, n, group):
    """Fewer 128-row tiles than half the resident workgroups: every tile is
    split over K (3 or 5 ways), a ragged last row block (M = 200), both scale
    modes.  Sampled rows cover every tile; repeated launches are bit-identical
    and the workspace is left zero."""
    from neurova_amd import capi

    plan = capi.marlin_describe_plan(m, n, k, group)
    assert plan["form"] == "prefill" and plan["row_blocks_or_full_tiles"] == 0 and plan["splits"] > 1, plan
    print_case("gemm-all-split", m, k, n, group, plan["splits"])
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, group, seed=2500 + m)
    got = _run_gemm(dev, x, qw, sp, group)
    rows = np.unique(np.concatenate([np.arange(0, m, 37), [1, 127, 128, 129, m - 2, m - 1]]))
    rows = rows[rows < m]
    exact = assert_close_f16(got[rows], O.marlin_gemm(x, qw, sp, group, rows=rows),
                             what=f"gemm-all-split m={m} k={k} n={n} g={group}")
    assert exact > 0.9
    again = _run_gemm(dev, x, qw, sp, group)
    assert np.array_equal(got.view(np.uint16), again.view(np.uint16))


@pytest.mark.parametrize("m,k,n,group", [
    (2048, 17408, 5120, 128),  # 320 tiles, 85 of 136 stages per workgroup
    (1000, 1024, 8448, 128),   # ragged last row block; 4.125 stages per workgroup over 8-stage tiles
    (1536, 2048, 8448, -1),    # per-column scales; 12.375 stages per workgroup over 16-stage tiles
    (2048, 128, 5120, 128),    # one stage per tile: 0 or 1 stage per workgroup, no tile cut
])
def test_gemm_stream_k_vs_oracle(dev, m, k, n, group):
    """The stream-K schedule (128-row tiles filling half to all of one round):
    every resident workgroup runs an equal range of the tiles' scale-group
    stages, and tiles cut between workgroups are finished by the last to
    arrive, summing the parts in k order.  Every output is checked; repeated
    launches are bit-identical; the workspace is left zero."""
    from neurova_amd import capi

    plan = capi.marlin_describe_plan(m, n, k, group)
    assert plan["form"] == "prefill-streamk" and plan["workgroups"] == 2 * plan["cus"], plan
    print_case("gemm-stream-k", m, k, n, group)
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, group, seed=2600 + m + k)
    got = _run_gemm(dev, x, qw, sp, group)
    exact = assert_close_f16(got, O.marlin_gemm(x, qw, sp, group),
                             what=f"gemm-stream-k m={m} k={k} n={n} g={group}")
    assert exact > 0.9
    again = _run_gemm(dev, x, qw, sp, group)
    assert np.array_equal(got.view(np.uint16), again.view(np.uint16))


@pytest.mark.parametrize("m", [1, 4, 16, 32])
def test_decode_shape_cfg2(dev, m):
    """M in {1,4,16}, K=5120, N=17408, g=128 (and configs[4]'s M=32)."""
    k, n = 5120, 17408
    print_case("cfg2", m, k, n)
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=7)
    got = _run_gemm(dev, x, qw, sp, 128)
    ref = O.marlin_gemm(x, qw, sp, 128)
    exact = assert_close_f16(got, ref, what=f"cfg2 m={m}")
    if m <= 16:  # decode kernel
        assert_reference_rounding(got, ref, x, qw, sp, 128, what=f"cfg2 m={m}")
    else:  # prefill kernel, the reference's rounding
        assert exact > 0.95


@pytest.mark.parametrize("m,k,n,group", [
    (1, 5120, 5120, 128),    # 1 chunk per workgroup, 4 waves sharing each k range
    (3, 5120, 7168, -1),
    (16, 5120, 5120, 128),
    (1, 17408, 5120, 128),
    (16, 17408, 5120, 128),  # 2 chunks per workgroup (the LDS limit sets 12 splits)
    (2, 4096, 2048, 128),
    (5, 2560, 1024, -1),
])
def test_narrow_decode_vs_oracle(dev, m, k, n, group):
    """Narrow N (the QKV / O / down projections): the decode kernel's workgroups
    take 1 or 2 chunks and their waves share the k range; both scale modes,
    repeated launches bit-identical."""
    print_case("narrow", m, k, n, group)
    codes, qw, _, sp, x = O.make_marlin_inputs(m, k, n, group, seed=1300 + m + k + n)
    got = _run_gemm(dev, x, qw, sp, group)
    ref = O.marlin_gemm(x, qw, sp, group)
    exact = assert_close_f16(got, ref, what=f"narrow m={m} k={k} n={n} g={group}")
    if group <= 0:
        assert exact > 0.9
        _assert_per_column_rounding(got, codes, x, sp)
    else:
        assert_reference_rounding(got, ref, x, qw, sp, group, what=f"narrow m={m} k={k} n={n}")
    again = _run_gemm(dev, x, qw, sp, group)
    assert np.array_equal(got.view(np.uint16), again.view(np.uint16))


@pytest.mark.parametrize("m,k,n", [(1, 17408, 5120), (4, 5120, 5120)])
def test_narrow_silu_and_argmax_vs_oracle(dev, m, k, n):
    """The SiLU-gated and fused-argmax variants on narrow tiles."""
    import torch
    from neurova_amd import capi

    print_case("narrow-variants", m, k, n)
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=1400 + m + k)
    mixed = np.random.default_rng(1400 + m).normal(0, 1, (m, 2 * k)).astype(np.float16)
    c = torch.empty((m, n), dtype=torch.float16, device=dev)
    ws = _ws(dev, n)
    st = capi.marlin_gemm_silu_packed(to_dev(mixed, dev), to_dev(qw, dev), c, to_dev(sp, dev), ws, 128,
                                      _scratch(dev, m, n, k, 128))
    assert st == 0
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0
    assert_close_f16(to_np(c), O.marlin_gemm_silu_packed(mixed, qw, sp, k, 128), what=f"narrow silu m={m}")
    own = _run_gemm(dev, x, qw, sp, 128).astype(np.float32)
    state = torch.zeros((m,), dtype=torch.int64, device=dev)
    out = torch.full((m,), -1, dtype=torch.int64, device=dev)
    sync = torch.empty((2,), dtype=torch.int32, device=dev)
    st = capi.marlin_gemm_argmax(to_dev(x, dev), to_dev(qw, dev), to_dev(sp, dev), ws, 128, state, out, sync, 1,
                                 _scratch(dev, m, n, k, 128))
    assert st == 0
    torch.cuda.synchronize()
    assert np.array_equal(to_np(out), own.argmax(axis=1))
    assert int(ws.abs().sum()) == 0


@pytest.mark.parametrize("m", [32, 48])
def test_small_m_gemm_many_splits_vs_oracle(dev, m):
    """M above 16 rows on the down projection (K = 17408, N = 5120): at M = 32 the
    decode kernel with A fragments loaded per step (the SiLU-gated activations
    formed once first), at M = 48 the prefill kernel split many ways over K;
    plain and SiLU-gated A, workspace left zero."""
    import torch
    from neurova_amd import capi

    k, n = 17408, 5120
    print_case("small-m-splits", m, k, n)
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=1500 + m)
    got = _run_gemm(dev, x, qw, sp, 128)
    exact = assert_close_f16(got, O.marlin_gemm(x, qw, sp, 128), what=f"small-m m={m}")
    assert exact > 0.95
    mixed = np.random.default_rng(1500 + m).normal(0, 1, (m, 2 * k)).astype(np.float16)
    c = torch.empty((m, n), dtype=torch.float16, device=dev)
    ws = _ws(dev, n)
    st = capi.marlin_gemm_silu_packed(to_dev(mixed, dev), to_dev(qw, dev), c, to_dev(sp, dev), ws, 128,
                                      _scratch(dev, m, n, k, 128))
    assert st == 0
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0
    assert_close_f16(to_np(c), O.marlin_gemm_silu_packed(mixed, qw, sp, k, 128), what=f"small-m silu m={m}")


@pytest.mark.parametrize("k,n", [(5120, 17408), (17408, 5120)])
def test_prefill_shape_cfg3(dev, k, n):
    """M=2048, every output against the oracle (the
    oracle's dequant dominates its cost; its float64 product of all 2048 rows
    takes a few seconds)."""
    m = 2048
    print_case("cfg3", m, k, n)
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=9)
    got = _run_gemm(dev, x, qw, sp, 128)
    exact = assert_close_f16(got, O.marlin_gemm(x, qw, sp, 128), what=f"cfg3 k={k}")
    assert exact > 0.95


def test_deterministic_split_k(dev):
    k, n, m = 17408, 5120, 1
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=3)
    a = _run_gemm(dev, x, qw, sp, 128)
    b = _run_gemm(dev, x, qw, sp, 128)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_m_zero_is_noop(dev):
    import torch
    from neurova_amd import capi

    b = torch.zeros((16, 512), dtype=torch.int32, device=dev)
    s = torch.zeros((2, 256), dtype=torch.float16, device=dev)
    a = torch.zeros((0, 256), dtype=torch.float16, device=dev)
    c = torch.zeros((0, 256), dtype=torch.float16, device=dev)
    assert capi.marlin_gemm(a, b, c, s, _ws(dev, 256), 128) == 0


@pytest.mark.parametrize("m", [1, 5, 24, 40])
def test_silu_packed_vs_oracle(dev, m):
    import torch
    from neurova_amd import capi

    k, n = 1024, 512
    print_case("silu", m, k, n)
    _, qw, _, sp, _ = O.make_marlin_inputs(m, k, n, 128, seed=50 + m)
    mixed = np.random.default_rng(m).normal(0, 1, (m, 2 * k)).astype(np.float16)
    c = torch.empty((m, n), dtype=torch.float16, device=dev)
    st = capi.marlin_gemm_silu_packed(to_dev(mixed, dev), to_dev(qw, dev), c, to_dev(sp, dev), _ws(dev, n), 128,
                                      _scratch(dev, m, n, k, 128))
    assert st == 0
    assert_close_f16(to_np(c), O.marlin_gemm_silu_packed(mixed, qw, sp, k, 128), what=f"silu m={m}")


@pytest.mark.parametrize("m,k,n", [(1, 1024, 65536), (3, 512, 4096), (16, 256, 2048), (20, 1024, 65536), (32, 512, 4096),
                                   (40, 512, 1024), (256, 512, 40960)])
def test_argmax_vs_oracle(dev, m, k, n):
    import torch
    from neurova_amd import capi

    print_case("argmax", m, k, n)
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=60 + m)
    state = torch.zeros((m,), dtype=torch.int64, device=dev)
    out = torch.full((m,), -1, dtype=torch.int64, device=dev)
    sync = torch.empty((2,), dtype=torch.int32, device=dev)
    ws = _ws(dev, n)
    own = _run_gemm(dev, x, qw, sp, 128).astype(np.float32)  # this library's fp16 outputs
    ref = O.marlin_gemm(x, qw, sp, 128).astype(np.float64)
    top2 = np.sort(ref, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * (1e-2 + 1e-3 * np.abs(top2[:, 1]))
    for epoch in (1, 2):  # two calls in a row reuse the workspace
        st = capi.marlin_gemm_argmax(to_dev(x, dev), to_dev(qw, dev), to_dev(sp, dev), ws, 128, state, out, sync,
                                     epoch, _scratch(dev, m, n, k, 128))
        assert st == 0
        torch.cuda.synchronize()
        idx = to_np(out)
        # exactly the first maximum of the same kernel's fp16 outputs
        assert np.array_equal(idx, own.argmax(axis=1))
        # a maximum of the reference's outputs within the parity tolerance ...
        picked = ref[np.arange(m), idx]
        assert (picked >= ref.max(axis=1) - (1e-2 + 1e-3 * np.abs(ref.max(axis=1)))).all()
        # ... and the reference's own index wherever its top two are well apart
        assert np.array_equal(idx[clear], O.marlin_gemm_argmax(x, qw, sp, 128)[clear])
        assert int(ws.abs().sum()) == 0


@pytest.mark.parametrize("batch", [1, 3])
def test_mlp_streaming_vs_oracle(dev, batch):
    import torch
    from neurova_amd import capi

    hidden, inter = 256, 512
    print_case("mlp", batch, hidden, inter)
    rng = np.random.default_rng(batch)
    gu_codes = rng.integers(0, 16, size=(hidden, 2 * inter), dtype=np.uint8)
    d_codes = rng.integers(0, 16, size=(inter, hidden), dtype=np.uint8)
    gu_s = (np.abs(rng.normal(0, 0.01, (hidden // 128, 2 * inter))) + 1e-3).astype(np.float16)
    d_s = (np.abs(rng.normal(0, 0.01, (inter // 128, hidden))) + 1e-3).astype(np.float16)
    gu_q, d_q = O.marlin_pack_codes(gu_codes), O.marlin_pack_codes(d_codes)
    gu_sp, d_sp = O.marlin_pack_scales(gu_s), O.marlin_pack_scales(d_s)
    x = rng.normal(0, 1, (batch, hidden)).astype(np.float16)
    out = torch.empty((batch, hidden), dtype=torch.float16, device=dev)
    accum = torch.empty((batch, hidden), dtype=torch.float32, device=dev)
    sync = torch.zeros((2 * batch,), dtype=torch.int32, device=dev)
    scratch = torch.empty((capi.marlin_mlp_scratch_bytes(batch, hidden, inter),), dtype=torch.uint8, device=dev)
    st = capi.marlin_mlp_streaming(to_dev(gu_q, dev), to_dev(gu_sp, dev), to_dev(d_q, dev), to_dev(d_sp, dev),
                                   to_dev(x, dev), out, accum, sync, hidden, inter, 128, 128, scratch)
    assert st == 0
    ref = O.marlin_mlp_streaming(x, gu_q, gu_sp, d_q, d_sp, hidden, inter, 128, 128)
    assert_close_f16(to_np(out), ref, what="mlp")


def test_dropin_module_marlin_ops(dev):
    """The reference's Python surface: allocating op, _out op, silu_packed_out, argmax_out."""
    import torch
    import langburst_cuda as lc

    m, k, n = 4, 1024, 512
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=77)
    q, s, xd = to_dev(qw, dev), to_dev(sp, dev), to_dev(x, dev)
    ref = O.marlin_gemm(x, qw, sp, 128)
    y = lc.lowbit_marlin_gemm(q, s, xd, k, 128)
    assert_close_f16(to_np(y), ref, what="lowbit_marlin_gemm")
    out = torch.empty((m, n), dtype=torch.float16, device=dev)
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    lc.lowbit_marlin_gemm_out(qweight=q, scales=s, x=xd, out=out, workspace=ws, cols=k, group_size=128)
    assert np.array_equal(to_np(out).view(np.uint16), to_np(y).view(np.uint16))
    mixed = np.random.default_rng(1).normal(0, 1, (m, 2 * k)).astype(np.float16)
    lc.lowbit_marlin_gemm_silu_packed_out(q, s, to_dev(mixed, dev), out, ws, k, 128)
    assert_close_f16(to_np(out), O.marlin_gemm_silu_packed(mixed, qw, sp, k, 128), what="silu_packed_out")
    state = torch.empty((m,), dtype=torch.int64, device=dev)
    am = torch.empty((m,), dtype=torch.int64, device=dev)
    sync = torch.empty((2,), dtype=torch.int32, device=dev)
    lc.lowbit_marlin_gemm_argmax_out(q, s, xd, out, ws, state, am, sync, 1, k, 128)
    assert np.array_equal(to_np(am), to_np(y).astype(np.float32).argmax(axis=1))  # same kernel numerics
    with pytest.raises(RuntimeError, match="Marlin requires K divisible by 128"):
        lc.lowbit_marlin_gemm(q, s, xd[:, :100].contiguous(), 100, 128)
    with pytest.raises(RuntimeError, match="Marlin supports group_size -1 or 128"):
        lc.lowbit_marlin_gemm(q, s, xd, k, 64)
    w = lc.lowbit_marlin_dequant(q, s, k, 128)
    assert np.array_equal(to_np(w).view(np.uint16), np.ascontiguousarray(O.marlin_dequant_f16(qw, sp, 128).T).view(np.uint16))


def test_single_hip_runtime_in_process(dev):
    """The C-ABI library must bind to the HIP runtime PyTorch loaded, not a second copy."""
    import neurova_amd  # noqa: F401
    from neurova_amd import capi

    capi.lib()
    maps = open("/proc/self/maps").read().splitlines()
    hip = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(hip) == 1, hip
    ours = {line.split()[-1] for line in maps if "liblangburst_lowbit" in line or "langburst_cuda" in line}
    assert len(ours) == 2, ours
