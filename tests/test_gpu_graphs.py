"""HIP-graph replay of the path's launches against the same launches run eagerly.

The bench and the decode-step sweep replay their launches from HIP graphs, and
a serving loop would do the same.  The kernels keep their split-K counters in
the caller's workspace and leave them zero, and their scratch holds nothing
across calls, so a captured launch must give on every replay exactly what it
gives eagerly.  Each test captures a few launches, replays the graph several
times with other eager work and synchronisations between the replays, and
compares every replay bit for bit with the eager result; the workspace must
be zero after each replay.
"""
from __future__ import annotations

import pytest

from tests.gpu_util import print_case

pytestmark = pytest.mark.gpu


def _marlin_tensors(torch, dev, k, n, gen):
    q = torch.randint(-2 ** 31, 2 ** 31, (k // 16, 2 * n), dtype=torch.int32, device=dev, generator=gen)
    s = (torch.randn((k // 128, n), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
    return q, s


def _replay_and_check(torch, graph, outs, eager, ws_list, disturb):
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        disturb()  # other eager work on the same buffers' device between replays
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {rep} differs from eager"
        for ws in ws_list:
            assert int(ws.abs().sum()) == 0, f"replay {rep} left the workspace non-zero"


@pytest.mark.parametrize("m,k,n", [(1, 5120, 17408), (4, 17408, 5120), (32, 5120, 7168), (64, 5120, 4096)])
def test_marlin_gemm_graph_replay(dev, m, k, n):
    """Decode (split-K, counters in the workspace; M = 32: A fragments loaded per
    step) and prefill (tail splits) launches."""
    import torch
    import langburst_cuda as lc

    print_case("graph-marlin", m, k, n)
    gen = torch.Generator(device=dev)
    gen.manual_seed(m + k)
    q, s = _marlin_tensors(torch, dev, k, n, gen)
    x = torch.randn((m, k), device=dev, generator=gen).half()
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    out = torch.empty((m, n), dtype=torch.float16, device=dev)
    lc.lowbit_marlin_gemm_out(q, s, x, out, ws, k, 128)
    torch.cuda.synchronize()
    eager = out.clone()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lc.lowbit_marlin_gemm_out(q, s, x, out, ws, k, 128)  # warm the side stream
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        lc.lowbit_marlin_gemm_out(q, s, x, out, ws, k, 128)
    other = torch.empty((m, n), dtype=torch.float16, device=dev)
    _replay_and_check(torch, graph, [out], [eager], [ws],
                      lambda: lc.lowbit_marlin_gemm_out(q, s, x, other, ws, k, 128))


@pytest.mark.parametrize("m", [2, 32])
def test_silu_packed_graph_replay(dev, m):
    """M = 32 captures two launches: the SiLU-gated activations formed once
    into scratch, then the direct-A decode kernel over them."""
    import torch
    import langburst_cuda as lc

    k, n = 17408, 5120
    print_case("graph-silu", m, k, n)
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    q, s = _marlin_tensors(torch, dev, k, n, gen)
    mixed = torch.randn((m, 2 * k), device=dev, generator=gen).half()
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    out = torch.empty((m, n), dtype=torch.float16, device=dev)
    lc.lowbit_marlin_gemm_silu_packed_out(q, s, mixed, out, ws, k, 128)
    torch.cuda.synchronize()
    eager = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lc.lowbit_marlin_gemm_silu_packed_out(q, s, mixed, out, ws, k, 128)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        lc.lowbit_marlin_gemm_silu_packed_out(q, s, mixed, out, ws, k, 128)
    _replay_and_check(torch, graph, [out], [eager], [ws], lambda: torch.cuda.synchronize())


@pytest.mark.parametrize("batch", [1, 16])
def test_mlp_fused_graph_replay(dev, batch):
    """The decode MLP: the [g | u] round trip at batch 1, the gate/up launch
    storing fp16(silu(g) * u) at batch 16 (both keep split counters in the
    workspace)."""
    import torch
    from neurova_amd import capi

    h, it = 5120, 17408
    print_case("graph-mlp", batch)
    gen = torch.Generator(device=dev)
    gen.manual_seed(30 + batch)
    gq, gs = _marlin_tensors(torch, dev, h, 2 * it, gen)
    dq, ds = _marlin_tensors(torch, dev, it, h, gen)
    x = torch.randn((batch, h), device=dev, generator=gen).half()
    ws = torch.zeros((capi.marlin_mlp_fused_workspace_len(batch, h, it),), dtype=torch.int32, device=dev)
    sc = torch.empty((capi.marlin_mlp_fused_scratch_bytes(batch, h, it),), dtype=torch.uint8, device=dev)
    out = torch.empty((batch, h), dtype=torch.float16, device=dev)

    def call(o):
        assert capi.marlin_mlp_fused(x, gq, gs, dq, ds, o, h, it, 128, 128, ws, sc) == 0

    call(out)
    torch.cuda.synchronize()
    eager = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(out)
    other = torch.empty_like(out)
    _replay_and_check(torch, graph, [out], [eager], [ws], lambda: call(other))


@pytest.mark.parametrize("bits", [2, 3, 8])
def test_rowwise_graph_replay(dev, bits):
    """The one-row LDS-staged rowwise GEMV and the pair GEMV."""
    import torch
    import langburst_cuda as lc

    rows, cols, g = 5120, 17408, 128
    print_case("graph-rowwise", bits)
    gen = torch.Generator(device=dev)
    gen.manual_seed(bits)
    pc = cols * bits // 8
    qa = torch.randint(0, 256, (rows, pc), dtype=torch.uint8, device=dev, generator=gen)
    qb = torch.randint(0, 256, (rows, pc), dtype=torch.uint8, device=dev, generator=gen)
    s = (torch.randn((rows, cols // g), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
    x = torch.randn((cols,), device=dev, generator=gen).half()
    y = lc.lowbit_gemv(qa, s, x, cols, g, bits)
    ya, yb = lc.lowbit_gemv_pair(qa, s, qb, s, x, cols, g, bits)
    torch.cuda.synchronize()
    eager = [y.clone(), ya.clone(), yb.clone()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        lc.lowbit_gemv(qa, s, x, cols, g, bits)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        gy = lc.lowbit_gemv(qa, s, x, cols, g, bits)
        gya, gyb = lc.lowbit_gemv_pair(qa, s, qb, s, x, cols, g, bits)
    _replay_and_check(torch, graph, [gy, gya, gyb], eager, [], lambda: lc.lowbit_gemv(qb, s, x, cols, g, bits))
