"""One layer of the 64-layer decode step through the
drop-in ops in the production call order (``adapters/qwen36_impl/model.py``
:1414-1482, the sequence bench.py's decode step times): QKV 5120 -> 7168,
O 5120 -> 5120, gate/up 5120 -> 2 x 17408 into the ``[gate | up]`` row, then
down 17408 -> 5120 through the SiLU-gated op on that row, with one workspace
shared by the four calls.  Every output is checked against the oracle in full
(the down projection on the kernel's own ``[gate | up]`` row, as the model
composes it), and the shared workspace is left zero.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from tests.gpu_util import assert_close_f16, print_case, to_dev, to_np

pytestmark = pytest.mark.gpu

HIDDEN, INTER, QKV = 5120, 17408, 7168


@pytest.mark.parametrize("m", [1, 32])
def test_decode_layer_vs_oracle(dev, m):
    import torch
    import langburst_cuda as lc

    print_case("decode layer", m)
    shapes = {"qkv": (HIDDEN, QKV), "o": (HIDDEN, HIDDEN), "gate_up": (HIDDEN, 2 * INTER), "down": (INTER, HIDDEN)}
    host, weights = {}, {}
    for i, (name, (k, n)) in enumerate(shapes.items()):
        _, qw, _, sp, xs = O.make_marlin_inputs(m, k, n, 128, seed=4100 + 10 * i + m)
        host[name] = (qw, sp)
        weights[name] = (to_dev(qw, dev), to_dev(sp, dev))
        if name == "qkv":
            x = xs
    xd = to_dev(x, dev)
    ws = torch.zeros((2 * INTER // 128 * 16,), dtype=torch.int32, device=dev)
    out = {name: torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
           for name, (_, n) in shapes.items()}
    lc.lowbit_marlin_gemm_out(*weights["qkv"], xd, out["qkv"], ws, HIDDEN, 128)
    lc.lowbit_marlin_gemm_out(*weights["o"], xd, out["o"], ws, HIDDEN, 128)
    lc.lowbit_marlin_gemm_out(*weights["gate_up"], xd, out["gate_up"], ws, HIDDEN, 128)
    lc.lowbit_marlin_gemm_silu_packed_out(*weights["down"], out["gate_up"], out["down"], ws, INTER, 128)
    torch.cuda.synchronize()
    assert int(ws.abs().sum()) == 0, "the shared workspace must be left zero"

    got = {name: to_np(t) for name, t in out.items()}
    for name in ("qkv", "o", "gate_up"):
        qw, sp = host[name]
        assert_close_f16(got[name], O.marlin_gemm(x, qw, sp, 128), what=f"{name} m={m}")
    qw, sp = host["down"]
    assert_close_f16(got["down"], O.marlin_gemm_silu_packed(got["gate_up"], qw, sp, INTER, 128), what=f"down m={m}")
