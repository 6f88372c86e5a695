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
    """M = 2048, K = 17408, N = 5120 needs about 120 MiB of partials: refused
    with LB_ERR_NOALLOC_LIMIT, nothing launched, the output untouched."""
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
