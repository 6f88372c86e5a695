"""lb_marlin_gemm_noalloc (static per-device scratch, no allocation) against
lb_marlin_gemm (caller scratch) through the C ABI: bit-identical outputs on
calls in a row, the later ones smaller, the workspace left zero, and problems
beyond the static scratch refused before any launch.  The entry point has no
reference counterpart; the oracle check of these shapes is lb_marlin_gemm's
(tests/test_gpu_marlin.py, tests/test_gpu_model_shapes.py)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from tests.gpu_util import assert_close_f16, print_case, to_dev, to_np

pytestmark = pytest.mark.gpu


def _pair(dev, m, k, n, seed):
    import torch
    from neurova_amd import capi

    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128, seed=seed)
    a, b, s = to_dev(x, dev), to_dev(qw, dev), to_dev(sp, dev)
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    ref = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    sc = torch.empty((max(1, capi.marlin_scratch_bytes(m, n, k, 128)),), dtype=torch.uint8, device=dev)
    assert capi.marlin_gemm(a, b, ref, s, ws, 128, sc) == 0
    got = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    st = capi.marlin_gemm_noalloc(a, b, got, s, ws, 128)
    assert st == 0, capi.status_string(st)
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0
    return to_np(got), to_np(ref), (x, qw, sp)


@pytest.mark.parametrize("shapes", [
    [(1, 5120, 17408), (1, 1024, 2048)],      # decode, split K; then a smaller one
    [(32, 5120, 7168), (4, 5120, 5120)],      # prefill tail splits; then decode
    [(16, 17408, 5120), (3, 512, 768)],
])
def test_noalloc_matches_caller_scratch(dev, shapes):
    from neurova_amd import capi

    for i, (m, k, n) in enumerate(shapes):
        print_case("noalloc", i, m, k, n)
        assert capi.marlin_scratch_bytes(m, n, k, 128) <= capi.marlin_noalloc_scratch_limit()
        got, ref, (x, qw, sp) = _pair(dev, m, k, n, seed=40 + i + m)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), (m, k, n)
        if k * n <= 1024 * 2048:
            assert_close_f16(got, O.marlin_gemm(x, qw, sp, 128), what=f"noalloc m={m} k={k} n={n}")


def test_noalloc_refuses_beyond_its_scratch(dev):
    """M = 2048, K = 17408, N = 5120 (the stream-K schedule, two 128 KiB partial
    slots per resident workgroup) needs 128 MiB of partials: refused with
    LB_ERR_NOALLOC_LIMIT, nothing launched, the output untouched."""
    import torch
    from neurova_amd import capi

    m, k, n = 2048, 17408, 5120
    print_case("noalloc limit", m, k, n)
    assert capi.marlin_scratch_bytes(m, n, k, 128) > capi.marlin_noalloc_scratch_limit()
    a = torch.zeros((m, k), dtype=torch.float16, device=dev)
    b = torch.zeros((k // 16, 2 * n), dtype=torch.int32, device=dev)
    s = torch.ones((k // 128, n), dtype=torch.float16, device=dev)
    c = torch.full((m, n), 7.0, dtype=torch.float16, device=dev)
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    assert capi.marlin_gemm_noalloc(a, b, c, s, ws, 128) == capi.LB_ERR_NOALLOC_LIMIT
    torch.cuda.synchronize()
    assert bool((c == 7.0).all()) and int(ws.abs().sum()) == 0


def _capture_inputs(torch, dev, m, k, n, seed):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    q = torch.randint(-2 ** 31, 2 ** 31, (k // 16, 2 * n), dtype=torch.int32, device=dev, generator=gen)
    s = (torch.randn((k // 128, n), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
    x = torch.randn((m, k), device=dev, generator=gen).half()
    return q, s, x


def test_noalloc_graph_replay(dev):
    """Two noalloc calls captured in one HIP graph (the second smaller), each
    replay bit-equal to lb_marlin_gemm run eagerly, with eager work on the
    same static scratch between the replays, the workspace zero after each."""
    import torch
    from neurova_amd import capi

    shapes = [(1, 5120, 17408), (4, 1024, 2048)]
    print_case("noalloc graph", shapes)
    cases = []
    for i, (m, k, n) in enumerate(shapes):
        q, s, x = _capture_inputs(torch, dev, m, k, n, 60 + i)
        ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
        ref = torch.empty((m, n), dtype=torch.float16, device=dev)
        sc = torch.empty((max(1, capi.marlin_scratch_bytes(m, n, k, 128)),), dtype=torch.uint8, device=dev)
        assert capi.marlin_gemm(x, q, ref, s, ws, 128, sc) == 0
        cases.append((q, s, x, ws, ref, torch.empty((m, n), dtype=torch.float16, device=dev)))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream
        for q, s, x, ws, _, out in cases:
            assert capi.marlin_gemm_noalloc(x, q, out, s, ws, 128) == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for q, s, x, ws, _, out in cases:
            assert capi.marlin_gemm_noalloc(x, q, out, s, ws, 128) == 0
    other = torch.empty_like(cases[0][5])
    for rep in range(3):
        for c in cases:
            c[5].fill_(float("nan"))
        graph.replay()
        q, s, x, ws, _, _ = cases[0]
        assert capi.marlin_gemm_noalloc(x, q, other, s, ws, 128) == 0  # eager use of the same scratch
        torch.cuda.synchronize()
        for q, s, x, ws, ref, out in cases:
            assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
            assert int(ws.abs().sum()) == 0


_FIRST_CALL_IN_CAPTURE = r"""
import sys
import torch
from neurova_amd import capi

dev = torch.device("cuda:0")
m, k, n = 1, 5120, 17408
gen = torch.Generator(device=dev)
gen.manual_seed(77)
q = torch.randint(-2 ** 31, 2 ** 31, (k // 16, 2 * n), dtype=torch.int32, device=dev, generator=gen)
s = (torch.randn((k // 128, n), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
x = torch.randn((m, k), device=dev, generator=gen).half()
ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
ref = torch.empty((m, n), dtype=torch.float16, device=dev)
sc = torch.empty((capi.marlin_scratch_bytes(m, n, k, 128),), dtype=torch.uint8, device=dev)
assert capi.marlin_gemm(x, q, ref, s, ws, 128, sc) == 0
torch.cuda.synchronize()
out = torch.empty((m, n), dtype=torch.float16, device=dev)
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=side):
    st = capi.marlin_gemm_noalloc(x, q, out, s, ws, 128)  # this process's first noalloc call
assert st == 0, capi.status_string(st)
for rep in range(3):
    out.fill_(float("nan"))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), rep
    assert int(ws.abs().sum()) == 0
print("first-call-in-capture ok", flush=True)
"""


def test_noalloc_first_call_inside_capture(dev):
    """A fresh process whose first lb_marlin_gemm_noalloc call (the one that
    looks up the static scratch's device address) is made inside a HIP graph
    capture: the capture succeeds and every replay equals lb_marlin_gemm."""
    import os
    import subprocess
    import sys

    print_case("noalloc first call in capture")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    proc = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE], cwd=root, capture_output=True, text=True,
                          timeout=100)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-4000:]
    assert "first-call-in-capture ok" in proc.stdout
