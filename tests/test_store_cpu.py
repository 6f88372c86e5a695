"""The quantised checkpoint format: the oracle's quantisers pinned to the
reference's own outputs, and the product loader (neurova_amd.store) checked
on checkpoints the oracle writes.  CPU only.

Reference: adapters/qwen36_tools/quantize.py:125-340 (quantisers, writer),
loader.py:474-528 (QuantizedStore), core/platform.py:10-33 (index file).
Fixtures: tests/golden/quant_golden.npz, written by tests/golden/make_quant_golden.py
from the reference's quantisers.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import lowbit_oracle as O
from oracle import quantize_oracle as Q


@pytest.fixture(scope="module")
def golden(golden_dir):
    return np.load(golden_dir / "quant_golden.npz")


def _meta(meta: dict) -> list[int]:
    return [meta["rows"], meta["cols"], meta["group_size"], meta["n_groups"], meta["packed_cols"]]


@pytest.mark.parametrize("group,tag", [(128, "g128"), (-1, "gcol")])
def test_marlin_quantiser_matches_reference(golden, group, tag):
    q, s, meta = Q.quantize_marlin4_groupwise(golden["marlin_w"], group)
    assert np.array_equal(q, golden[f"marlin_{tag}_qweight"])
    assert np.array_equal(s.view(np.uint16), golden[f"marlin_{tag}_scales"].view(np.uint16))
    assert _meta(meta) == golden[f"marlin_{tag}_meta"].tolist()


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("group", [8, 128])
def test_rowwise_quantiser_matches_reference(golden, bits, group):
    p, s, meta = Q.quantize_symmetric_lowbit(golden["rowwise_w"], group, bits)
    assert np.array_equal(p, golden[f"rowwise_b{bits}_g{group}_packed"])
    assert np.array_equal(s.view(np.uint16), golden[f"rowwise_b{bits}_g{group}_scales"].view(np.uint16))
    assert _meta(meta) == golden[f"rowwise_b{bits}_g{group}_meta"].tolist()


def _marlin_mutant(w, group, mode):
    """The oracle's Marlin quantiser with one plausible mistake planted."""
    w16 = np.asarray(w).astype(np.float16)
    rows, cols = w16.shape
    eff = cols if group == -1 else group
    grouped = np.ascontiguousarray(w16.T).reshape(cols // eff, eff, rows)
    amax = np.abs(grouped).max(axis=1).astype(np.float32)
    k = np.float32(np.float16(2.0 / 15.0)) if mode == "scalar_in_fp16" else np.float32(2.0 / 15.0)
    s = (amax * k).astype(np.float16)
    s = np.where(s > 0, s, np.float16(1.0)).astype(np.float16)
    quot = grouped.astype(np.float32) / s.astype(np.float32)[:, None, :]
    if mode != "quotient_in_fp32":
        quot = quot.astype(np.float16).astype(np.float32)
    r = np.sign(quot) * np.floor(np.abs(quot) + 0.5) if mode == "ties_away" else np.rint(quot)
    codes = np.clip(r + 8, 0, 15).reshape(cols, rows).astype(np.uint8)
    return O.marlin_pack_codes(codes), O.marlin_pack_scales(s, per_column=(eff == cols))


def _rowwise_mutant(w, group, bits, mode):
    w = np.asarray(w, dtype=np.float32)
    rows, cols = w.shape
    ng = -(-cols // group)
    pad = np.zeros((rows, ng * group), np.float32)
    pad[:, :cols] = w
    g = pad.reshape(rows, ng, group)
    qmax = (1 << (bits - 1)) - 1
    scale = (np.abs(g).max(axis=2) / np.float32(qmax)).astype(np.float32)
    scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
    sq = scale.astype(np.float16).astype(np.float32) if mode == "fp16_scale_for_codes" else scale
    quot = g / sq[:, :, None]
    r = np.sign(quot) * np.floor(np.abs(quot) + 0.5) if mode == "ties_away" else np.rint(quot)
    codes = (np.clip(r, -qmax - 1, qmax).reshape(rows, -1)[:, :cols] + (1 << (bits - 1))).astype(np.uint8)
    return O.rowwise_pack(codes, bits), scale.astype(np.float16)


@pytest.mark.parametrize("mode", ["quotient_in_fp32", "scalar_in_fp16", "ties_away"])
def test_marlin_fixture_catches_planted_mistakes(golden, mode):
    """The fixture must tell the reference's fp16 opmath and ties from plausible alternatives."""
    caught = False
    for group, tag in ((128, "g128"), (-1, "gcol")):
        q, s = _marlin_mutant(golden["marlin_w"], group, mode)
        caught |= not (np.array_equal(q, golden[f"marlin_{tag}_qweight"])
                       and np.array_equal(s.view(np.uint16), golden[f"marlin_{tag}_scales"].view(np.uint16)))
    assert caught, mode


@pytest.mark.parametrize("mode", ["fp16_scale_for_codes", "ties_away"])
def test_rowwise_fixture_catches_planted_mistakes(golden, mode):
    caught = False
    for bits in (2, 3, 4, 8):
        for group in (8, 128):
            p, _ = _rowwise_mutant(golden["rowwise_w"], group, bits, mode)
            caught |= not np.array_equal(p, golden[f"rowwise_b{bits}_g{group}_packed"])
    assert caught, mode


def test_quantiser_round_trip_error_bound():
    """Dequantising the codes gives back the weights within half a step."""
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (256, 256)).astype(np.float16)
    q, s, _ = Q.quantize_marlin4_groupwise(w, 128)
    wd = O.marlin_dequant_f16(q, s, 128).astype(np.float32)  # [K, N]
    step = O.marlin_unpack_scales(s).astype(np.float32)       # [groups, N]
    err = np.abs(wd - w.T.astype(np.float32)).reshape(2, 128, 256)
    assert (err <= 0.5 * step[:, None, :] * 1.01 + 1e-6).all()


def _checkpoint(tmp_path):
    rng = np.random.default_rng(11)
    index = Q.new_index()
    tensors = {
        "model.layers.0.mlp.gate_up_proj.weight": (rng.normal(0, 0.02, (512, 256)).astype(np.float32), 128, 4, True),
        "model.layers.0.self_attn.o_proj.weight": (rng.normal(0, 0.02, (256, 384)).astype(np.float32), -1, 4, True),
        "model.layers.0.linear_attn.in_proj_ba.weight": (rng.normal(0, 0.02, (37, 257)).astype(np.float32), 128, 3, False),
        "model.embed_tokens.weight": (rng.normal(0, 0.02, (64, 320)).astype(np.float32), 64, 8, False),
    }
    for name, (w, g, b, marlin) in tensors.items():
        Q.write_quantized_tensor(tmp_path, index, name, w, g, b, marlin)
    norm = rng.normal(0, 1, (320,)).astype(np.float16)
    Q.write_fp16_tensor(tmp_path, index, "model.norm.weight", norm)
    Q.write_index(tmp_path, index)
    return tensors, norm


def test_store_loads_what_the_writer_wrote(tmp_path):
    from neurova_amd.store import FP16Tensor, LowBitMarlinTensor, LowBitTensor, QuantizedStore

    tensors, norm = _checkpoint(tmp_path)
    st = QuantizedStore(tmp_path, device="cpu")
    assert st.names() == sorted(list(tensors) + ["model.norm.weight"])
    for name, (w, g, b, marlin) in tensors.items():
        t = st.tensor(name)
        if marlin:
            q, s, meta = Q.quantize_marlin4_groupwise(w, g)
            assert isinstance(t, LowBitMarlinTensor)
            assert t.rows == w.shape[0] and t.cols == w.shape[1] and t.group_size == meta["group_size"]
        else:
            q, s, meta = Q.quantize_symmetric_lowbit(w, g, b)
            assert isinstance(t, LowBitTensor)
            assert (t.rows, t.cols, t.group_size, t.bits) == (w.shape[0], w.shape[1], g, b)
        assert np.array_equal(t.qweight.numpy(), q)
        assert np.array_equal(t.scales.numpy().view(np.uint16), s.view(np.uint16))
        assert st.tensor(name) is t  # cached
    n = st.tensor("model.norm.weight")
    assert isinstance(n, FP16Tensor) and np.array_equal(n.value.numpy().view(np.uint16), norm.view(np.uint16))


def test_store_rejects_inconsistent_checkpoints(tmp_path):
    from neurova_amd.store import QuantizedStore

    with pytest.raises(FileNotFoundError, match="runtime index not found"):
        QuantizedStore(tmp_path, device="cpu")
    _checkpoint(tmp_path)
    idx_path = tmp_path / "langburst_index.json"
    idx = json.loads(idx_path.read_text())
    # a truncated file
    q_rel = idx["tensors"]["model.layers.0.mlp.gate_up_proj.weight"]["qweight"]
    data = (tmp_path / q_rel).read_bytes()
    (tmp_path / q_rel).write_bytes(data[:-4])
    with pytest.raises(ValueError, match="holds .* bytes"):
        QuantizedStore(tmp_path, device="cpu").tensor("model.layers.0.mlp.gate_up_proj.weight")
    (tmp_path / q_rel).write_bytes(data)
    # a Marlin entry whose output rows are not a multiple of 256, an unknown kind
    bad = dict(idx["tensors"]["model.layers.0.self_attn.o_proj.weight"], rows=200, packed_cols=400)
    idx["tensors"]["bad"] = bad
    idx["tensors"]["odd"] = {"kind": "lowbit_fp8", "path": "x"}
    idx_path.write_text(json.dumps(idx))
    st = QuantizedStore(tmp_path, device="cpu")
    with pytest.raises(ValueError, match="not a multiple of 256"):
        st.tensor("bad")
    with pytest.raises(ValueError, match="unknown tensor kind"):
        st.tensor("odd")


def test_wrappers_refuse_cpu_execution(tmp_path):
    import torch
    from neurova_amd.store import QuantizedStore

    _checkpoint(tmp_path)
    st = QuantizedStore(tmp_path, device="cpu")
    with pytest.raises(RuntimeError, match="no CPU execution path"):
        st.tensor("model.layers.0.mlp.gate_up_proj.weight").gemv(torch.zeros(256, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="no CPU execution path"):
        st.tensor("model.embed_tokens.weight").row_dequant(3)


def test_marlin_wrapper_argument_checks(tmp_path, monkeypatch):
    """LowBitMarlinTensor's reference argument checks (loader.py:337-413) run
    before any device work; the environment knobs are validated."""
    import torch
    from neurova_amd import store
    from neurova_amd.store import QuantizedStore

    _checkpoint(tmp_path)
    st = QuantizedStore(tmp_path, device="cpu")
    down = st.tensor("model.layers.0.mlp.gate_up_proj.weight")
    k = down.cols
    with pytest.raises(ValueError, match="expects mixed"):
        down.gemm_silu_packed(torch.zeros((1, 1, 2 * k), dtype=torch.float16), k)
    with pytest.raises(ValueError, match="hidden must match"):
        down.gemm_silu_packed(torch.zeros((1, 2 * k), dtype=torch.float16), k + 128)
    with pytest.raises(ValueError, match="mixed width must be 2\\*hidden"):
        down.gemm_silu_packed(torch.zeros((1, 2 * k + 2), dtype=torch.float16), k)
    with pytest.raises(RuntimeError, match="no CPU execution path"):
        down.gemm_silu_packed(torch.zeros((2 * k,), dtype=torch.float16), k)
    with pytest.raises(ValueError, match="expects x"):
        down.gemm_argmax(torch.zeros((1, 1, k), dtype=torch.float16))
    with pytest.raises(ValueError, match="expects x"):
        down.gemm(torch.zeros((k,), dtype=torch.float16))
    with pytest.raises(RuntimeError, match="does not support row_dequant"):
        down.row_dequant(0)

    assert store.lowbit_rows_per_cta() == 8 and store.marlin_direct_max_batch() == 256
    monkeypatch.setenv("LANGBURST_LOWBIT_ROWS_PER_CTA", "16")
    monkeypatch.setenv("LANGBURST_MARLIN_DIRECT_MAX_BATCH", "4")
    assert store.lowbit_rows_per_cta() == 16 and store.marlin_direct_max_batch() == 4
    monkeypatch.setenv("LANGBURST_LOWBIT_ROWS_PER_CTA", "5")
    with pytest.raises(ValueError, match="rows_per_cta must be one of: 4, 8, 16"):
        store.lowbit_rows_per_cta()
    monkeypatch.setenv("LANGBURST_MARLIN_DIRECT_MAX_BATCH", "0")
    with pytest.raises(ValueError, match=">= 1"):
        store.marlin_direct_max_batch()


@pytest.mark.parametrize("policy,batch,cached", [("off", 1, False), ("", 1, True), ("decode_only", 1, True),
                                                 ("decode_only", 2, False), ("small", 2, True), ("small", 3, False),
                                                 ("all", 64, True)])
def test_output_cache_policy(monkeypatch, policy, batch, cached):
    """The admission rule of the reference's Marlin output cache (loader.py:29-62); an empty
    policy string is not one of the "off" spellings there, so it caches."""
    from neurova_amd.store import _OutputCache

    monkeypatch.setenv("LANGBURST_MARLIN_OUT_CACHE_POLICY", policy)
    monkeypatch.delenv("LANGBURST_MARLIN_OUT_CACHE_MAX_BATCH", raising=False)
    assert _OutputCache.wants(batch) is cached


def test_output_cache_admits_before_allocating(monkeypatch):
    """The cache decides admission before it allocates, as the reference does
    (loader.py:254-302): with free memory exactly the minimum plus the new
    buffer, the buffer is cached; checking after the allocation would count it
    twice and refuse.  Device allocation and the free-memory query are mocked
    (no GPU here); each mocked allocation lowers the free memory."""
    import torch
    from neurova_amd import store

    mib = 1 << 20
    out_bytes = 4 * 512 * 2  # batch 4 x 512 rows of fp16
    ws_bytes = (512 // 128 * 16) * 4
    free = {"bytes": 384 * mib + out_bytes}
    real_empty, real_zeros = torch.empty, torch.zeros

    def fake_alloc(real):
        def alloc(shape, device=None, dtype=None):
            t = real(shape, dtype=dtype)
            if device is not None:
                free["bytes"] -= t.numel() * t.element_size()
            return t
        return alloc

    monkeypatch.setattr(torch, "empty", fake_alloc(real_empty))
    monkeypatch.setattr(torch, "zeros", fake_alloc(real_zeros))
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (free["bytes"], 1 << 40))
    monkeypatch.setenv("LANGBURST_MARLIN_OUT_CACHE_POLICY", "all")
    monkeypatch.setenv("LANGBURST_MARLIN_CACHE_MAX_MIB", "0")
    monkeypatch.setenv("LANGBURST_MARLIN_CACHE_MIN_FREE_MIB", "384")
    monkeypatch.setattr(store._OutputCache, "bytes_used", 0)

    class FakeQ:
        device = torch.device("cuda", 0)
        shape = (320, 1024)  # 512 rows

    t = store.LowBitMarlinTensor("w", FakeQ(), None, 5120, 128)
    out = t._cached(t._out_cache, 4, (4, 512), torch.float16)
    assert t._out_cache.get(4) is out  # admitted at exactly the threshold
    free["bytes"] = 384 * mib + ws_bytes
    ws = t._cached_workspace()
    assert t._workspace is ws
    free["bytes"] = 384 * mib + out_bytes - 1  # one byte short: not cached
    other = t._cached(t._out_cache, 8, (4, 512), torch.float16)
    assert t._out_cache.get(8) is None and other is not out
