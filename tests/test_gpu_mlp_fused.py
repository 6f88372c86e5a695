"""The decode MLP entry point (``lb_marlin_mlp_fused``: the gate_up launch,
storing fp16(silu(g) * u) where its decode tiles pair gate and up chunks, then
the down launch) against the two projections it replaces, and against the
oracle.

The reference runs its production MLP as the gate_up projection followed by
``down.gemm_silu_packed`` (``adapters/qwen36_impl/model.py:1460-1470``,
``loader.py:337-368``).  The fused entry point must return exactly what
``lb_marlin_gemm`` followed by ``lb_marlin_gemm_silu_packed`` return (with a
workspace large enough that both plan the same tilings), leave its workspace
zero, and meet the parity bar (tests/gpu_util.py) against the oracle's
dequant-then-matmul of the same two steps.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from tests.gpu_util import assert_close_f16, print_case, to_dev, to_np

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 5120, 17408  # the model's MLP (BASELINE.json cfg5)


def _problem(hidden, inter, batch, gg, dg, seed):
    rng = np.random.default_rng(seed)
    gu_codes = rng.integers(0, 16, size=(hidden, 2 * inter), dtype=np.uint8)
    d_codes = rng.integers(0, 16, size=(inter, hidden), dtype=np.uint8)
    gu_groups = 1 if gg == -1 else hidden // 128
    d_groups = 1 if dg == -1 else inter // 128
    # per-column scales apply after the fp16 rounding: keep those outputs in range
    gu_s = (np.abs(rng.normal(0, 0.01, (gu_groups, 2 * inter))) + 1e-3).astype(np.float16)
    d_s = (np.abs(rng.normal(0, 0.01, (d_groups, hidden))) + 1e-3).astype(np.float16)
    x = rng.normal(0, 1, (batch, hidden)).astype(np.float16)
    return (O.marlin_pack_codes(gu_codes), O.marlin_pack_scales(gu_s, per_column=gg == -1),
            O.marlin_pack_codes(d_codes), O.marlin_pack_scales(d_s, per_column=dg == -1), x)


def _problem_dev(hidden, inter, batch, seed, dev):
    """Model-sized problem drawn on the GPU: every int32 pattern is a valid
    Marlin tensor (8 codes per word), scales |N(0, 0.01)| + 1e-3."""
    import torch

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    gu_q = torch.randint(-2**31, 2**31, (hidden // 16, 4 * inter), dtype=torch.int32, device=dev, generator=g)
    d_q = torch.randint(-2**31, 2**31, (inter // 16, 2 * hidden), dtype=torch.int32, device=dev, generator=g)
    gu_s = (torch.randn((hidden // 128, 2 * inter), device=dev, generator=g) * 0.01).abs_().add_(1e-3).half()
    d_s = (torch.randn((inter // 128, hidden), device=dev, generator=g) * 0.01).abs_().add_(1e-3).half()
    x = torch.randn((batch, hidden), device=dev, generator=g).half()
    return [x, gu_q, gu_s, d_q, d_s]


def _two_launches(dev, x, gu_q, gu_s, d_q, d_s, hidden, inter, gg, dg):
    import torch
    from neurova_amd import capi

    batch = x.shape[0]
    mixed = torch.empty((batch, 2 * inter), dtype=torch.float16, device=dev)
    out = torch.empty((batch, hidden), dtype=torch.float16, device=dev)
    ws = torch.zeros((1 << 14,), dtype=torch.int32, device=dev)
    s1 = torch.empty((max(1, capi.marlin_scratch_bytes(batch, 2 * inter, hidden, gg)),), dtype=torch.uint8, device=dev)
    s2 = torch.empty((max(1, capi.marlin_scratch_bytes(batch, hidden, inter, dg)),), dtype=torch.uint8, device=dev)
    assert capi.marlin_gemm(x, gu_q, mixed, gu_s, ws, gg, s1) == 0
    assert capi.marlin_gemm_silu_packed(mixed, d_q, out, d_s, ws, dg, s2) == 0
    torch.cuda.synchronize()
    return to_np(out), to_np(mixed)


def _fused(dev, x, gu_q, gu_s, d_q, d_s, hidden, inter, gg, dg, ws=None):
    import torch
    from neurova_amd import capi

    batch = x.shape[0]
    out = torch.full((batch, hidden), float("nan"), dtype=torch.float16, device=dev)
    if ws is None:
        ws = torch.zeros((capi.marlin_mlp_fused_workspace_len(batch, hidden, inter),), dtype=torch.int32, device=dev)
    scratch = torch.empty((capi.marlin_mlp_fused_scratch_bytes(batch, hidden, inter),), dtype=torch.uint8,
                          device=dev)
    st = capi.marlin_mlp_fused(x, gu_q, gu_s, d_q, d_s, out, hidden, inter, gg, dg, ws, scratch)
    assert st == 0, capi.status_string(st)
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0, f"workspace not left zero: {ws.nonzero().flatten()[:8].tolist()}"
    return to_np(out)


CASES = [
    # hidden, inter, batch, gate group, down group
    (512, 1024, 1, 128, 128),
    (512, 1024, 3, 128, 128),
    (768, 1536, 16, 128, 128),
    (512, 1024, 2, -1, 128),
    (512, 1024, 2, 128, -1),
    (256, 384, 5, 128, 128),
    (512, 1024, 32, 128, 128),  # prefill kernels: the [g | u] round trip
]


@pytest.mark.parametrize("hidden,inter,batch,gg,dg", CASES)
def test_fused_mlp_vs_two_launches_and_oracle(dev, hidden, inter, batch, gg, dg):
    print_case("mlp_fused", hidden, inter, batch, gg, dg)
    gu_q, gu_s, d_q, d_s, x = _problem(hidden, inter, batch, gg, dg, seed=batch + hidden)
    args = [to_dev(a, dev) for a in (x, gu_q, gu_s, d_q, d_s)]
    got = _fused(dev, *args, hidden, inter, gg, dg)
    ref, mixed = _two_launches(dev, *args, hidden, inter, gg, dg)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), "fused != gate_up + silu-gated down"
    # oracle: the gate_up projection, then the SiLU-gated down over the GPU's own [g | u]
    assert_close_f16(mixed, O.marlin_gemm(x, gu_q, gu_s, gg), what="gate_up")
    assert_close_f16(got, O.marlin_gemm_silu_packed(mixed, d_q, d_s, inter, dg), what="down(silu)")


@pytest.mark.parametrize("batch", [1, 4, 16, 24, 32])
def test_fused_mlp_model_shape_vs_two_launches(dev, batch):
    """At the model's shape: the [g | u] round trip at batch 1-4 (the gate_up
    call plans whole-K single-chunk tiles), the gate_up launch storing the
    gated activations from batch 5 on; bit-equal to the two projections."""
    print_case("mlp_fused_model", batch)
    args = _problem_dev(HIDDEN, INTER, batch, 7 + batch, dev)
    got = _fused(dev, *args, HIDDEN, INTER, 128, 128)
    ref, _ = _two_launches(dev, *args, HIDDEN, INTER, 128, 128)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


def test_fused_mlp_back_to_back_calls_share_workspace(dev):
    """Two calls on one workspace, the second with a smaller batch: each as the
    two launches give, and the workspace zero after each."""
    import torch
    from neurova_amd import capi

    print_case("mlp_fused_b2b", HIDDEN, INTER)
    n_ws = max(capi.marlin_mlp_fused_workspace_len(b, HIDDEN, INTER) for b in (16, 1))
    ws = torch.zeros((n_ws,), dtype=torch.int32, device=dev)
    for batch in (16, 1):
        args = _problem_dev(HIDDEN, INTER, batch, 100 + batch, dev)
        got = _fused(dev, *args, HIDDEN, INTER, 128, 128, ws=ws)
        ref, _ = _two_launches(dev, *args, HIDDEN, INTER, 128, 128)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), batch


@pytest.mark.parametrize("batch", [1, 4])
def test_torch_op_matches_reference_op_sequence(dev, batch):
    """``langburst_cuda.lowbit_marlin_mlp_fused_out`` against the two ops the
    reference's ``_fused_marlin_down`` calls (``lowbit_marlin_gemm_out``, then
    ``lowbit_marlin_gemm_silu_packed_out`` with the reference's workspace size,
    ``loader.py:337-368``): bit-equal to the C-ABI two launches, within the
    parity bar of the reference op sequence, workspace left zero."""
    import torch
    import langburst_cuda as lc

    print_case("mlp_fused_op", batch)
    x, gu_q, gu_s, d_q, d_s = _problem_dev(HIDDEN, INTER, batch, 50 + batch, dev)
    ws = torch.zeros((lc.lowbit_marlin_mlp_fused_workspace_len(batch, HIDDEN, INTER),), dtype=torch.int32,
                     device=dev)
    out = torch.empty((batch, HIDDEN), dtype=torch.float16, device=dev)
    lc.lowbit_marlin_mlp_fused_out(gu_q, gu_s, d_q, d_s, x, out, ws, HIDDEN, INTER, 128, 128)
    mixed = torch.empty((batch, 2 * INTER), dtype=torch.float16, device=dev)
    ws_gu = torch.zeros((2 * INTER // 128 * 16,), dtype=torch.int32, device=dev)
    lc.lowbit_marlin_gemm_out(gu_q, gu_s, x, mixed, ws_gu, HIDDEN, 128)
    ws_d = torch.zeros((HIDDEN // 128 * 16,), dtype=torch.int32, device=dev)
    ref_out = torch.empty((batch, HIDDEN), dtype=torch.float16, device=dev)
    lc.lowbit_marlin_gemm_silu_packed_out(d_q, d_s, mixed, ref_out, ws_d, INTER, 128)
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0
    got = to_np(out)
    two, _ = _two_launches(dev, x, gu_q, gu_s, d_q, d_s, HIDDEN, INTER, 128, 128)
    assert np.array_equal(got.view(np.uint16), two.view(np.uint16))
    assert_close_f16(got, to_np(ref_out), what="op vs reference op sequence")
    with pytest.raises(RuntimeError, match="workspace must hold"):
        lc.lowbit_marlin_mlp_fused_out(gu_q, gu_s, d_q, d_s, x, out, ws[:8], HIDDEN, INTER, 128, 128)


def _sample_cols(n, count, seed):
    """`count` 64-column chunks of an N-column Marlin tensor (the layout slices
    at 64 columns: qweight[:, 2 n0 : 2 n1], scales[:, n0 : n1])."""
    rng = np.random.default_rng(seed)
    chunks = np.sort(rng.choice(n // 64, size=count, replace=False))
    return [(64 * c, 64 * c + 64) for c in chunks]


@pytest.mark.parametrize("batch", [1, 4, 16, 32])
def test_fused_mlp_model_shape_vs_oracle(dev, batch):
    """The decode MLP at the model's shape (hidden 5120, intermediate 17408,
    g128) against the oracle, column-sampled: the gate_up stage on 16 chunks of
    its 34816 columns, the SiLU-gated down stage on 16 chunks of its 5120
    outputs over the whole [g | u] row; and bit-equal to the two launches."""
    print_case("mlp_fused_model_oracle", batch)
    rng = np.random.default_rng(900 + batch)
    gu_q = rng.integers(-2**31, 2**31, size=(HIDDEN // 16, 4 * INTER), dtype=np.int64).astype(np.int32)
    d_q = rng.integers(-2**31, 2**31, size=(INTER // 16, 2 * HIDDEN), dtype=np.int64).astype(np.int32)
    gu_s = (np.abs(rng.normal(0, 0.01, (HIDDEN // 128, 2 * INTER))) + 1e-3).astype(np.float16)
    d_s = (np.abs(rng.normal(0, 0.01, (INTER // 128, HIDDEN))) + 1e-3).astype(np.float16)
    x = rng.normal(0, 1, (batch, HIDDEN)).astype(np.float16)
    args = [to_dev(a, dev) for a in (x, gu_q, gu_s, d_q, d_s)]
    got = _fused(dev, *args, HIDDEN, INTER, 128, 128)
    two, mixed = _two_launches(dev, *args, HIDDEN, INTER, 128, 128)
    assert np.array_equal(got.view(np.uint16), two.view(np.uint16))
    for n0, n1 in _sample_cols(2 * INTER, 16, batch):
        assert_close_f16(mixed[:, n0:n1], O.marlin_gemm(x, gu_q[:, 2 * n0:2 * n1], gu_s[:, n0:n1], 128),
                         what=f"gate_up cols {n0}:{n1}")
    for n0, n1 in _sample_cols(HIDDEN, 16, batch + 1):
        assert_close_f16(got[:, n0:n1],
                         O.marlin_gemm_silu_packed(mixed, d_q[:, 2 * n0:2 * n1], d_s[:, n0:n1], INTER, 128),
                         what=f"down(silu) cols {n0}:{n1}")
