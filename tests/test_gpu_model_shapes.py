"""Parity at the model's projection shapes (the
64-layer decode-step sweep) and at the lm_head fused-argmax shape.

Weights are full-size; the oracle (dequant-then-fp32-accumulate,
``oracle/lowbit_oracle.py``) evaluates sampled 64-column chunks of each
output (the Marlin layout slices at 64 columns: ``qweight[:, 2 n0 : 2 n1]``,
``scales[:, n0 : n1]``), and the whole N for the argmax, slice by slice.
Bar: tests/gpu_util.py (max-abs 1e-2 / rel 1e-3).  Reference shapes:
adapters/qwen36_impl/model.py:1371-1482 (MLP), 1994-2034 (lm_head),
configs/ml-dmc8-q4.yaml:62 (fused argmax on)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from tests.gpu_util import assert_close_f16, print_case, to_dev, to_np

pytestmark = pytest.mark.gpu

TOL_ABS, TOL_REL = 1e-2, 1e-3


def _inputs(m, k, n, seed, group=128):
    rng = np.random.default_rng(seed)
    qw = rng.integers(-2**31, 2**31, size=(k // 16, 2 * n), dtype=np.int64).astype(np.int32)
    groups = k // 128 if group == 128 else 1
    s = (np.abs(rng.normal(0, 0.01, (groups, n))) + 1e-3).astype(np.float16)
    x = rng.normal(0, 1, (m, k)).astype(np.float16)
    return qw, s, x


def _chunks(n, count, seed):
    """`count` random 64-column chunks plus fixed ones: the first and last two
    (the mixed plans split the chunks left over after the whole-K tiles, which
    are the last ones) and both sides of the 256- and 512-chunk boundaries
    (one and two whole-K tiles per CU on 256 CUs)."""
    rng = np.random.default_rng(seed)
    total = n // 64
    picks = set(rng.choice(total, size=min(count, total), replace=False).tolist())
    picks |= {c for c in (0, 255, 256, 511, 512, total - 2, total - 1) if 0 <= c < total}
    return [(64 * c, 64 * c + 64) for c in sorted(picks)]


def _oracle_logits(x, qw, s, width=8192):
    """fp16 ``x @ W`` over every column, ``width`` columns at a time: the
    oracle's arithmetic (``O.marlin_gemm``: fp16 ``(q - 8) * s`` weights, float64
    accumulation, one rounding to fp16), with the weights dequantised by the
    vectorised torch-CPU unpack, which equals ``O.marlin_dequant_f16`` bit for
    bit (tests/test_oracle_golden.py); the numpy table-driven unpack takes
    minutes at N = 248320."""
    import torch

    from oracle import torch_cpu as T

    xs = torch.from_numpy(x).to(torch.float64)
    out = []
    for n0 in range(0, qw.shape[1] // 2, width):
        w = T.marlin_dequant(torch.from_numpy(np.ascontiguousarray(qw[:, 2 * n0:2 * (n0 + width)])),
                             torch.from_numpy(np.ascontiguousarray(s[:, n0:n0 + width])), 128)
        out.append((xs @ w.to(torch.float64)).to(torch.float16).numpy())
    return np.concatenate(out, axis=1)


def _gemm(dev, x, qw, s, group, silu=False):
    import torch
    from neurova_amd import capi

    m = x.shape[0]
    k = x.shape[1] // (2 if silu else 1)
    n = qw.shape[1] // 2
    c = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    sc = torch.empty((max(1, capi.marlin_scratch_bytes(m, n, k, group)),), dtype=torch.uint8, device=dev)
    fn = capi.marlin_gemm_silu_packed if silu else capi.marlin_gemm
    st = fn(to_dev(x, dev), to_dev(qw, dev), c, to_dev(s, dev), ws, group, sc)
    assert st == 0, capi.status_string(st)
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0
    return to_np(c)


# QKV 5120 -> 7168, O 5120 -> 5120, gate/up 5120 -> 2 x 17408, down 17408 -> 5120 (SiLU-gated A)
SHAPES = [
    ("qkv", 5120, 7168, False),
    ("o", 5120, 5120, False),
    ("gate_up", 5120, 34816, False),
    ("down_silu", 17408, 5120, True),
]


@pytest.mark.parametrize("m", [1, 5, 16, 24, 32])
@pytest.mark.parametrize("name,k,n,silu", SHAPES)
def test_decode_step_projection_vs_oracle(dev, name, k, n, silu, m):
    """Every decode form at the model's shapes: staged (M = 1), direct-A tiles
    (QKV, O and the SiLU-gated down from M = 5, the last after its gated
    activations are formed once), the LDS ring (gate/up at M = 16, 24, 32),
    16- and 32-row MFMA tiles (M <= 16, M = 24 and 32)."""
    print_case("decode-step shape", name, m, k, n)
    seed = 10 * [sh[0] for sh in SHAPES].index(name) + m
    qw, s, x = _inputs(m, k, n, seed=seed)
    if silu:  # A is SiLU(mixed[:, :K]) * mixed[:, K:]
        x = np.random.default_rng(seed + 1).normal(0, 1, (m, 2 * k)).astype(np.float16)
    got = _gemm(dev, x, qw, s, 128, silu=silu)
    assert np.isfinite(got.astype(np.float32)).all()
    for n0, n1 in _chunks(n, 12, m + k + n):
        qs, ss = qw[:, 2 * n0:2 * n1], s[:, n0:n1]
        ref = O.marlin_gemm_silu_packed(x, qs, ss, k, 128) if silu else O.marlin_gemm(x, qs, ss, 128)
        assert_close_f16(got[:, n0:n1], ref, what=f"{name} m={m} cols {n0}:{n1}")


# The projections the reference publishes M = 1 timings for besides gate/up,
# down and lm_head (langburst/docs/PERFORMANCE_LOG.md:421-427): K = 6144 has 48
# scale groups, N = 14336 fewer 64-column chunks (224) than the device has CUs.
PUBLISHED = [
    ("attn_qkv", 5120, 14336),
    ("gdn_qkvz", 5120, 16384),
    ("gdn_out_attn_o", 6144, 5120),
]


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("name,k,n", PUBLISHED)
def test_published_projection_vs_oracle(dev, name, k, n, m):
    """The reference's other published projection shapes at decode batch
    sizes, against the oracle on 12 sampled 64-column chunks, and with
    per-column scales at M = 1."""
    from neurova_amd import capi

    plan = capi.marlin_describe_plan(m, n, k, 128)
    print_case("published shape", name, m, k, n, plan["form"], plan["chunks_or_row_blocks"], plan["splits"])
    seed = 100 + 10 * [sh[0] for sh in PUBLISHED].index(name) + m
    qw, s, x = _inputs(m, k, n, seed=seed)
    got = _gemm(dev, x, qw, s, 128)
    assert np.isfinite(got.astype(np.float32)).all()
    for n0, n1 in _chunks(n, 12, seed):
        assert_close_f16(got[:, n0:n1], O.marlin_gemm(x, qw[:, 2 * n0:2 * n1], s[:, n0:n1], 128),
                         what=f"{name} m={m} cols {n0}:{n1}")
    if m == 1:
        # (random scales stand for permuted ones; the permutation stays within
        # 32-column blocks, so a 64-column slice is the slice's own layout)
        qw1, s1, x1 = _inputs(m, k, n, seed=seed + 1, group=-1)
        got1 = _gemm(dev, x1, qw1, s1, -1)
        for n0, n1 in _chunks(n, 6, seed + 1):
            ref = O.marlin_gemm(x1, qw1[:, 2 * n0:2 * n1], s1[:, n0:n1], -1)
            assert_close_f16(got1[:, n0:n1], ref, what=f"{name} per-column m={m} cols {n0}:{n1}")


@pytest.mark.parametrize("m", [1, 4])
def test_lm_head_argmax_full_vocab(dev, m):
    """The fused argmax at the lm_head shape, K=5120, N=248320 (970 column
    tiles): equal to the first maximum of the same kernel's fp16 logits, a
    maximum of the oracle's logits within tolerance, and the oracle's index
    wherever its top two are farther apart than twice the tolerance."""
    import torch
    from neurova_amd import capi

    k, n = 5120, 248320
    print_case("lm_head argmax", m, k, n)
    qw, s, x = _inputs(m, k, n, seed=500 + m)
    own = _gemm(dev, x, qw, s, 128).astype(np.float64)
    state = torch.zeros((m,), dtype=torch.int64, device=dev)
    out = torch.full((m,), -1, dtype=torch.int64, device=dev)
    sync = torch.zeros((2,), dtype=torch.int32, device=dev)
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    sc = torch.empty((max(1, capi.marlin_scratch_bytes(m, n, k, 128)),), dtype=torch.uint8, device=dev)
    xd, qd, sd = to_dev(x, dev), to_dev(qw, dev), to_dev(s, dev)
    for epoch in (1, 2):
        st = capi.marlin_gemm_argmax(xd, qd, sd, ws, 128, state, out, sync, epoch, sc)
        assert st == 0, capi.status_string(st)
        torch.cuda.synchronize()
        assert int(ws.abs().sum()) == 0
    idx = to_np(out)
    assert np.array_equal(idx, own.argmax(axis=1))
    ref = _oracle_logits(x, qw, s).astype(np.float64)
    assert ref.shape == (m, n)
    best = ref.max(axis=1)
    tol = TOL_ABS + TOL_REL * np.abs(best)
    assert (ref[np.arange(m), idx] >= best - tol).all()
    top2 = np.sort(ref, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * tol
    assert np.array_equal(idx[clear], ref.argmax(axis=1)[clear])
    # logits themselves, sampled
    for n0, n1 in _chunks(n, 16, m):
        assert_close_f16(own[:, n0:n1], ref[:, n0:n1].astype(np.float16), what=f"lm_head cols {n0}:{n1}")


def test_argmax_agreement_with_reference_rounding(dev):
    """How often the fused argmax picks the oracle's index (the reference's
    rounding: fp16 (q - 8) * s per weight, then fp32 accumulation) over 64
    rows of an lm_head-like problem (K=5120, N=32768).  The kernel rounds the
    weights the same way and differs only in fp32 summation order, so the two
    can differ only where the top two logits are within about one fp16 step;
    outside such near-ties they must agree."""
    import torch
    from neurova_amd import capi

    k, n, m = 5120, 32768, 16
    agree = total = near = 0
    for seed in range(4):
        qw, s, x = _inputs(m, k, n, seed=700 + seed)
        state = torch.zeros((m,), dtype=torch.int64, device=dev)
        out = torch.full((m,), -1, dtype=torch.int64, device=dev)
        sync = torch.zeros((2,), dtype=torch.int32, device=dev)
        ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
        sc = torch.empty((max(1, capi.marlin_scratch_bytes(m, n, k, 128)),), dtype=torch.uint8, device=dev)
        st = capi.marlin_gemm_argmax(to_dev(x, dev), to_dev(qw, dev), to_dev(s, dev), ws, 128, state, out, sync, 1,
                                     sc)
        assert st == 0
        torch.cuda.synchronize()
        idx = to_np(out)
        ref = _oracle_logits(x, qw, s).astype(np.float64)
        want = ref.argmax(axis=1)
        top2 = np.sort(ref, axis=1)[:, -2:]
        step = np.spacing(np.abs(top2[:, 1]).astype(np.float16)).astype(np.float64)
        tie = (top2[:, 1] - top2[:, 0]) <= 2 * step
        assert np.array_equal(idx[~tie], want[~tie])
        agree += int((idx == want).sum())
        total += m
        near += int(tie.sum())
    print(f"[argmax agreement] {agree}/{total} rows pick the reference-rounding index; {near} rows have the top two "
          f"within two fp16 steps", flush=True)
    assert agree >= total - near
