"""Checkpoints in the reference's format (written by the oracle's restated
quantisers and writer), loaded onto the GPU by neurova_amd.store and run through
its tensor wrappers, against the oracle on the same bytes.  Same parity bar as
the kernel tests (tests/gpu_util.py)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from oracle import quantize_oracle as Q
from tests.gpu_util import assert_close_f16, print_case, to_np

pytestmark = pytest.mark.gpu


def test_store_round_trip_on_gpu(dev, tmp_path):
    import torch
    from neurova_amd.store import QuantizedStore

    print_case("store", str(tmp_path))
    rng = np.random.default_rng(5)
    index = Q.new_index()
    specs = {
        "gate_up": (rng.normal(0, 0.02, (1024, 512)).astype(np.float32), 128, 4, True),
        "o_percol": (rng.normal(0, 0.02, (256, 768)).astype(np.float32), -1, 4, True),
        "ba": (rng.normal(0, 0.02, (96, 640)).astype(np.float32), 128, 4, False),
        "embed": (rng.normal(0, 0.02, (50, 640)).astype(np.float32), 64, 8, False),
    }
    for name, (w, g, b, marlin) in specs.items():
        Q.write_quantized_tensor(tmp_path, index, name, w, g, b, marlin)
    Q.write_index(tmp_path, index)
    st = QuantizedStore(tmp_path, device=dev)

    gu = st.tensor("gate_up")
    q, s = to_np(gu.qweight), to_np(gu.scales)
    x = rng.normal(0, 1, (3, 512)).astype(np.float16)
    xd = torch.from_numpy(x).to(dev)
    assert_close_f16(to_np(gu.gemm(xd)), O.marlin_gemm(x, q, s, 128), what="store marlin gemm")
    assert_close_f16(to_np(gu.gemv(xd[0]))[None], O.marlin_gemm(x[:1], q, s, 128), what="store marlin gemv")
    op = st.tensor("o_percol")
    xo = rng.normal(0, 1, (2, 768)).astype(np.float16)
    assert_close_f16(to_np(op.gemm(torch.from_numpy(xo).to(dev))),
                     O.marlin_gemm(xo, to_np(op.qweight), to_np(op.scales), -1), what="store marlin per-column")
    mixed = rng.normal(0, 1, (2, 2 * 512)).astype(np.float16)
    assert_close_f16(to_np(gu.gemm_silu_packed(torch.from_numpy(mixed).to(dev))),
                     O.marlin_gemm_silu_packed(mixed, q, s, 512, 128), what="store silu packed")

    ba = st.tensor("ba")
    xb = rng.normal(0, 1, (2, 640)).astype(np.float16)
    qb, sb = to_np(ba.qweight), to_np(ba.scales)
    assert_close_f16(to_np(ba.gemv(torch.from_numpy(xb[0]).to(dev))), O.rowwise_gemv(qb, sb, xb[0], 640, 128, 4),
                     what="store rowwise gemv")
    assert_close_f16(to_np(ba.gemm(torch.from_numpy(xb).to(dev))), O.rowwise_gemm(qb, sb, xb, 640, 128, 4),
                     what="store rowwise gemm")
    em = st.tensor("embed")
    for r in (0, 17, 49):
        got = to_np(em.row_dequant(r))
        ref = O.rowwise_row_dequant(to_np(em.qweight), to_np(em.scales), r, 640, 64, 8)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), r
