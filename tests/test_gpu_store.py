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
    assert_close_f16(to_np(gu.gemm_silu_packed(torch.from_numpy(mixed).to(dev), 512)),
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


def test_marlin_wrapper_reference_calls(dev, tmp_path, monkeypatch):
    """LowBitMarlinTensor called exactly as the reference's model code calls it:
    ``down.gemm_silu_packed(mixed, intermediate_size)`` (model.py:1469),
    ``w.gemm_argmax(x, out=out)`` (model.py:333), ``gemm`` above
    ``marlin_direct_max_batch`` (loader.py:315-320), the output cache policy
    and the argmax epoch wrap (loader.py:398)."""
    import torch
    from neurova_amd.store import QuantizedStore

    print_case("store wrapper calls", str(tmp_path))
    rng = np.random.default_rng(11)
    index = Q.new_index()
    inter, hidden, vocab = 768, 512, 1024
    Q.write_quantized_tensor(tmp_path, index, "down", rng.normal(0, 0.02, (hidden, inter)).astype(np.float32), 128, 4,
                             True)
    Q.write_quantized_tensor(tmp_path, index, "lm_head", rng.normal(0, 0.02, (vocab, hidden)).astype(np.float32), 128,
                             4, True)
    Q.write_index(tmp_path, index)
    st = QuantizedStore(tmp_path, device=dev)
    down, head = st.tensor("down"), st.tensor("lm_head")
    dq, ds = to_np(down.qweight), to_np(down.scales)
    hq, hs = to_np(head.qweight), to_np(head.scales)

    mixed = rng.normal(0, 1, (3, 2 * inter)).astype(np.float16)
    got = down.gemm_silu_packed(torch.from_numpy(mixed).to(dev), inter)
    assert_close_f16(to_np(got), O.marlin_gemm_silu_packed(mixed, dq, ds, inter, 128), what="gemm_silu_packed")
    out = torch.empty((1, hidden), dtype=torch.float16, device=dev)
    r = down.gemm_silu_packed(torch.from_numpy(mixed[0]).to(dev), inter, out=out)
    assert r is out
    assert_close_f16(to_np(out), O.marlin_gemm_silu_packed(mixed[:1], dq, ds, inter, 128), what="silu out=")
    with pytest.raises(ValueError, match="out must be fp16"):
        down.gemm_silu_packed(torch.from_numpy(mixed).to(dev), inter, out=out)

    x = rng.normal(0, 1, (4, hidden)).astype(np.float16)
    ref = O.marlin_gemm(x, hq, hs, 128)
    ids = head.gemm_argmax(torch.from_numpy(x).to(dev))
    assert ids.dtype == torch.long and ids.shape == (4,)
    logits = to_np(head.gemm(torch.from_numpy(x).to(dev))).astype(np.float64)
    assert np.array_equal(to_np(ids), np.argmax(logits, axis=1))          # first maximum of the same logits
    assert np.all(np.abs(ref.astype(np.float64)[np.arange(4), to_np(ids)] - ref.astype(np.float64).max(axis=1)) <= 2e-2)
    o = torch.full((1,), -1, dtype=torch.long, device=dev)
    r = head.gemm_argmax(torch.from_numpy(x[2]).to(dev), out=o)
    assert int(r.reshape(-1)[0]) == int(to_np(ids)[2]) and int(o[0]) == int(to_np(ids)[2])
    with pytest.raises(ValueError, match="argmax out must be int64"):
        head.gemm_argmax(torch.from_numpy(x).to(dev), out=o)
    head._argmax_epoch = 2_000_000_000
    head.gemm_argmax(torch.from_numpy(x[:1]).to(dev))
    assert head._argmax_epoch == 1

    monkeypatch.setenv("LANGBURST_MARLIN_DIRECT_MAX_BATCH", "2")
    rows = head.gemm(torch.from_numpy(x[:3]).to(dev))             # 3 > 2: one row at a time
    assert_close_f16(to_np(rows), ref[:3], what="row-by-row gemm")
    monkeypatch.delenv("LANGBURST_MARLIN_DIRECT_MAX_BATCH")
    a = head.gemm(torch.from_numpy(x).to(dev))
    b = head.gemm(torch.from_numpy(x).to(dev))
    assert a.data_ptr() != b.data_ptr()                           # cache policy off by default
    monkeypatch.setenv("LANGBURST_MARLIN_OUT_CACHE_POLICY", "decode_only")
    a = head.gemv(torch.from_numpy(x[0]).to(dev))
    b = head.gemv(torch.from_numpy(x[1]).to(dev))
    assert a.data_ptr() == b.data_ptr()                           # batch 1 reuses one buffer, as the reference does
    assert_close_f16(to_np(b)[None], ref[1:2], what="cached gemv")
    head.clear_runtime_cache()
    assert head.runtime_cache_bytes() == 0
