"""Pins the CPU oracle before it is trusted as the checker of the HIP kernels.

Each check is chosen so that a plausible mistake in the oracle (wrong shift,
swapped nibble, transposed tile, wrong permutation direction, dropped zero
point, missing fp16 rounding) fails at least one of them:

* the reference's own known-answer vectors and shape invariants
  (tests/golden/rowwise_kats.json, from langburst/tests/test_v05_cuda_kernels.py:19-32
  and langburst/tests/test_quant_lowbit_cpu.py:34-35,63);
* the reference-held Marlin inverse tables (SHA-256 in tests/golden/marlin_tables.json,
  from langburst/csrc/marlin_mlp_stream.cu:7-84);
* independent formulations: a big-integer bitstream model of the rowwise
  layout, a closed-form (k, n) -> (word, nibble) map of the Marlin layout
  derived from the MMA fragment structure, the scalar reader, and the C
  restatement oracle/lowbit_ref.c;
* mathematics: bijection / involution of the permutations, round trips,
  one-hot inputs that reproduce single dequantised weights, exact fp16
  products, SiLU closed form, argmax ordering.
"""
from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest

from oracle import cref
from oracle import lowbit_oracle as O


# --------------------------------------------------------------- rowwise ----

def test_reference_kats_rowwise(golden_dir):
    kats = json.loads((golden_dir / "rowwise_kats.json").read_text())
    for case in kats["row_dequant_scale_one"]:
        packed = np.array([case["packed"]], dtype=np.uint8)
        cols = len(case["expected"])
        scales = np.ones((1, 1), dtype=np.float16)
        got = O.rowwise_row_dequant(packed, scales, 0, cols, 128, case["bits"])
        assert got.astype(np.float32).tolist() == case["expected"]
        # scalar restatement and the C restatement agree
        assert [O.rowwise_code(packed[0], c, case["bits"]) for c in range(cols)] == case["expected"]
        lib = cref.lib()
        assert [lib.orc_rowwise_value(packed.ctypes.data, packed.shape[1], c, case["bits"]) for c in range(cols)] == case["expected"]


def test_reference_shape_invariants(golden_dir):
    kats = json.loads((golden_dir / "rowwise_kats.json").read_text())
    for s in kats["shapes"]:
        codes = np.zeros((s["rows"], s["cols"]), dtype=np.uint8)
        packed = O.rowwise_pack(codes, s["bits"])
        assert list(packed.shape) == s["packed"]
        assert O.rowwise_packed_cols(s["cols"], s["bits"]) == s["packed"][1]
        n_groups = -(-s["cols"] // s["group_size"])
        assert [s["rows"], n_groups] == s["scales"]


def test_low_nibble_first():
    # code 0 in bits 0-3, code 1 in bits 4-7 (langburst/tests/test_quant_lowbit_cpu.py:18-27)
    packed = O.rowwise_pack(np.array([[1, 2, 15]], dtype=np.uint8), 4)
    assert packed.tolist() == [[0x21, 0x0F]]


def _bitstream_model(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack with Python big integers: row value = sum(code_c << (c*bits)), little-endian bytes."""
    rows, cols = codes.shape
    nbytes = (cols * bits + 7) // 8
    out = np.zeros((rows, nbytes), dtype=np.uint8)
    for r in range(rows):
        v = 0
        for c in range(cols):
            v |= int(codes[r, c]) << (c * bits)
        out[r] = np.frombuffer(v.to_bytes(nbytes, "little"), dtype=np.uint8)
    return out


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 7, 8])
def test_rowwise_pack_matches_bitstream_model_and_roundtrips(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(5, 77), dtype=np.uint8)
    packed = O.rowwise_pack(codes, bits)
    assert np.array_equal(packed, _bitstream_model(codes, bits))
    assert np.array_equal(O.rowwise_unpack(packed, 77, bits), codes)
    # padding bytes beyond ceil(cols*bits/8) do not change the decode
    padded = np.concatenate([packed, rng.integers(0, 256, size=(5, 3), dtype=np.uint8)], axis=1)
    assert np.array_equal(O.rowwise_unpack(padded, 77, bits), codes)
    # scalar reader == vectorised reader
    z = 1 << (bits - 1)
    for c in (0, 1, 7, 8, 31, 32, 76):
        assert O.rowwise_code(packed[2], c, bits) == int(codes[2, c]) - z


@pytest.mark.parametrize("bits,group", [(2, 64), (3, 128), (4, 32), (8, 128), (5, 8)])
def test_rowwise_gemm_oracle_vs_c_restatement(bits, group):
    codes, packed, scales, x = O.make_rowwise_inputs(29, 300, bits, group, batch=3, seed=11 + bits)
    y_np = O.rowwise_gemm(packed, scales, x, 300, group, bits)
    y_c = cref.rowwise_gemm(packed, scales, x, 300, group, bits)
    assert np.array_equal(y_np.view(np.uint16), y_c.view(np.uint16))


def test_rowwise_dequant_exact_products():
    # (q - z) * s is exact in fp32: compare against float64
    codes, packed, scales, _ = O.make_rowwise_inputs(7, 200, 4, 64, seed=3)
    w = O.rowwise_dequant_f32(packed, scales, 200, 64, 4)
    ref = (codes.astype(np.float64) - 8) * scales.astype(np.float64)[:, np.arange(200) // 64]
    assert np.array_equal(w.astype(np.float64), ref)


def test_rowwise_one_hot_reproduces_weight():
    codes, packed, scales, _ = O.make_rowwise_inputs(9, 256, 3, 128, seed=5)
    w = O.rowwise_dequant_f32(packed, scales, 256, 128, 3)
    for k in (0, 5, 127, 128, 255):
        x = np.zeros((1, 256), dtype=np.float16)
        x[0, k] = 1.0
        y = O.rowwise_gemm(packed, scales, x, 256, 128, 3)[0]
        assert np.array_equal(y, w[:, k].astype(np.float16))


def test_rowwise_row_dequant_out_of_range_is_zero():
    _, packed, scales, _ = O.make_rowwise_inputs(4, 64, 4, 32, seed=1)
    assert not O.rowwise_row_dequant(packed, scales, 4, 64, 32, 4).any()
    assert not O.rowwise_row_dequant(packed, scales, -1, 64, 32, 4).any()


# ---------------------------------------------------------------- marlin ----

TABLE_NAMES = ("LB_MARLIN_INV_PERM", "LB_MARLIN_INV_SCALE_PERM", "LB_MARLIN_INV_SCALE_PERM_SINGLE")


def test_marlin_inverse_tables_match_reference(golden_dir):
    gold = json.loads((golden_dir / "marlin_tables.json").read_text())["tables"]
    for name, table in zip(TABLE_NAMES, O.marlin_inverse_tables()):
        g = gold[name]
        assert table.size == g["length"]
        assert hashlib.sha256(table.astype("<i4").tobytes()).hexdigest() == g["sha256_le_int32"]
        for i, v in g["samples"].items():
            assert int(table[int(i)]) == v
    for a, b in zip(cref.marlin_inverse_tables(), O.marlin_inverse_tables()):
        assert np.array_equal(a, b)


def test_marlin_perm_invariants():
    perm, sp, sps = O.marlin_perm_tables()
    assert sorted(perm.tolist()) == list(range(1024))
    assert sorted(sps.tolist()) == list(range(32))
    assert np.array_equal(sp[sp], np.arange(64))  # 8x8 transpose is an involution
    # the permutation mixes the four 256-entry tiles: each run of 32 entries spans all four
    assert all(sorted(set((perm[i:i + 32] // 256).tolist())) == [0, 1, 2, 3] for i in range(0, 1024, 32))


def _closed_form_position(k: int, n: int, N: int):
    """(row, int32 column, nibble) of weight (k, n), from the MMA fragment structure:
    slot 4c+q of a 64-column chunk holds column c (+8) of tiles j at k = 2q, 2q+1, 2q+8, 2q+9."""
    kb, ki = k >> 4, k & 15
    nn = n & 63
    j, c, h = nn >> 4, nn & 7, (nn >> 3) & 1
    q = (ki & 7) >> 1
    nib = 4 * (ki & 1) + 2 * h + (ki >> 3)
    return kb, (n >> 6) * 128 + (4 * c + q) * 4 + j, nib


def test_marlin_pack_closed_form_and_roundtrip():
    rng = np.random.default_rng(0)
    K, N = 256, 512
    codes = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    qw = O.marlin_pack_codes(codes)
    assert qw.shape == (K // 16, 2 * N) and qw.dtype == np.int32
    assert np.array_equal(O.marlin_unpack_codes(qw), codes)
    u = qw.view(np.uint32)
    for k, n in [(0, 0), (1, 0), (8, 0), (9, 0), (2, 3), (15, 63), (16, 64), (37, 200), (255, 511)]:
        r, col, nib = _closed_form_position(k, n, N)
        assert (int(u[r, col]) >> (4 * nib)) & 15 == codes[k, n]
    # C restatement of the scalar reader agrees everywhere on a sample
    lib = cref.lib()
    qc = np.ascontiguousarray(qw)
    for k, n in zip(rng.integers(0, K, 300), rng.integers(0, N, 300)):
        assert lib.orc_marlin_code(qc.ctypes.data, N, int(k), int(n)) == codes[k, n]


def test_marlin_scales_roundtrip_and_layout():
    rng = np.random.default_rng(1)
    s = rng.random((4, 256)).astype(np.float16)
    sp = O.marlin_pack_scales(s)
    assert np.array_equal(O.marlin_unpack_scales(sp), s)
    # column 8jj+i of a 64-column chunk is stored at 8i+jj
    for n in (0, 1, 8, 9, 63, 64, 200):
        nn = n & 63
        assert sp[2, (n >> 6) * 64 + 8 * (nn & 7) + (nn >> 3)] == s[2, n]
    s1 = rng.random((1, 256)).astype(np.float16)
    s1p = O.marlin_pack_scales(s1, per_column=True)
    assert np.array_equal(O.marlin_unpack_scales(s1p, per_column=True), s1)


@pytest.mark.parametrize("group", [128, -1])
def test_marlin_scalar_reader_matches_dequant(group):
    K, N = 256, 256
    _, qw, s_nat, s_perm, _ = O.make_marlin_inputs(1, K, N, group, seed=4)
    codes = O.marlin_unpack_codes(qw).astype(np.float32) - 8
    if group == -1:
        dense = codes * s_nat.astype(np.float32)
    else:
        dense = codes * s_nat.astype(np.float32)[np.arange(K) // 128]
    rng = np.random.default_rng(2)
    for k, n in zip(rng.integers(0, K, 200), rng.integers(0, N, 200)):
        assert O.marlin_weight_read(qw, s_perm, int(n), int(k), N, group) == dense[k, n]


def test_marlin_dequant_rounds_to_fp16_product():
    K, N = 256, 256  # K == group_size would mean per-column scales (langburst_ext.cpp:87)
    codes, qw, s_nat, s_perm, _ = O.make_marlin_inputs(1, K, N, 128, seed=6)
    w = O.marlin_dequant_f16(qw, s_perm, 128)
    exact = (codes.astype(np.float64) - 8) * s_nat.astype(np.float64)[np.arange(K) // 128]
    assert np.array_equal(w, exact.astype(np.float16))  # single rounding of the exact product
    assert np.abs(w.astype(np.float64) - exact).max() <= np.abs(exact).max() * 2.0 ** -11


@pytest.mark.parametrize("group", [128, -1])
def test_marlin_gemm_one_hot_and_c_restatement(group):
    K, N = 256, 256
    codes, qw, s_nat, s_perm, x = O.make_marlin_inputs(3, K, N, group, seed=8)
    w = O.marlin_dequant_f16(qw, s_perm, group)
    for k in (0, 1, 9, 130, 255):
        e = np.zeros((1, K), dtype=np.float16)
        e[0, k] = 1.0
        y = O.marlin_gemm(e, qw, s_perm, group)[0]
        if group == -1:
            expect = (w[k].astype(np.float32) * s_nat[0].astype(np.float32)).astype(np.float16)
        else:
            expect = w[k]
        assert np.array_equal(y, expect)
    y_np = O.marlin_gemm(x, qw, s_perm, group)
    y_c = cref.marlin_gemm(x, qw, s_perm, group)
    assert np.array_equal(y_np.view(np.uint16), y_c.view(np.uint16))
    # an independent float64 evaluation lies within half an fp16 ulp (+ fp32 noise)
    if group != -1:
        wd = ((codes.astype(np.float64) - 8) * s_nat.astype(np.float64)[np.arange(K) // 128]).astype(np.float16)
        ref = x.astype(np.float64) @ wd.astype(np.float64)
        assert np.array_equal(ref.astype(np.float16), y_np)


def test_marlin_gemm_exact_pins():
    """The exact-scale product: equal to the natural-layout float64 product,
    and to the reference rounding wherever (q-8)*s is exact in fp16."""
    K, N = 512, 256
    codes, qw, s_nat, s_perm, x = O.make_marlin_inputs(4, K, N, 128, seed=21)
    got = O.marlin_gemm_exact(x, qw, s_perm, 128)
    natural = x.astype(np.float64) @ ((codes.astype(np.float64) - 8) * s_nat.astype(np.float64)[np.arange(K) // 128])
    assert np.array_equal(got.view(np.uint16), natural.astype(np.float16).view(np.uint16))
    # power-of-two scales: every fp16 (q-8)*s is exact, so both rounding orders agree
    rng = np.random.default_rng(22)
    s2 = (2.0 ** rng.integers(-8, -2, size=s_nat.shape)).astype(np.float16)
    s2_perm = O.marlin_pack_scales(s2, per_column=False)
    assert np.array_equal(O.marlin_gemm_exact(x, qw, s2_perm, 128).view(np.uint16),
                          O.marlin_gemm(x, qw, s2_perm, 128).view(np.uint16))
    # general scales: the two differ only by the per-weight rounding noise
    ref = O.marlin_gemm(x, qw, s_perm, 128).astype(np.float64)
    assert np.abs(got.astype(np.float64) - ref).max() < 1e-2


def test_silu_closed_form():
    g = np.array([[0.0, 1.0, -1.0, 4.0, -10.0, 0.5]], dtype=np.float16)
    u = np.array([[1.0, 2.0, 3.0, 0.5, 1.0, -2.0]], dtype=np.float16)
    mixed = np.concatenate([g, u], axis=1)
    got = O.silu_mul_packed(mixed, 6)[0].astype(np.float64)
    gd, ud = g[0].astype(np.float64), u[0].astype(np.float64)
    exact = gd / (1 + np.exp(-gd)) * ud
    assert np.allclose(got, exact, rtol=1e-3, atol=1e-4)
    assert got[0] == 0.0


def test_argmax_key_ordering():
    v = np.array([1.0, 3.0, -2.0, 3.0, 0.5], dtype=np.float16)
    k = O.argmax_key(v)
    assert int(np.uint64(0xFFFFFFFF) - (k.max() & np.uint64(0xFFFFFFFF))) == 1  # first of the tied maxima
    neg = np.array([-5.0, -1.0, -3.0], dtype=np.float16)
    assert int(np.uint64(0xFFFFFFFF) - (O.argmax_key(neg).max() & np.uint64(0xFFFFFFFF))) == 1
    zeros = np.array([-0.0, 0.0], dtype=np.float16)  # +0 orders above -0
    assert int(np.uint64(0xFFFFFFFF) - (O.argmax_key(zeros).max() & np.uint64(0xFFFFFFFF))) == 1
    rng = np.random.default_rng(0)
    vals = rng.standard_normal((4, 999)).astype(np.float16)
    keys = O.argmax_key(vals)
    got = (np.uint64(0xFFFFFFFF) - (keys.max(axis=1) & np.uint64(0xFFFFFFFF))).astype(np.int64)
    assert np.array_equal(got, vals.argmax(axis=1))


def test_marlin_gemm_argmax_matches_argmax_of_gemm():
    _, qw, _, s_perm, x = O.make_marlin_inputs(5, 256, 512, 128, seed=9)
    y = O.marlin_gemm(x, qw, s_perm, 128)
    assert np.array_equal(O.marlin_gemm_argmax(x, qw, s_perm, 128), y.astype(np.float32).argmax(axis=1))


def test_mlp_streaming_oracle_against_scalar_reader():
    hidden, inter = 256, 256  # group 128 == K would select per-column scales
    rng = np.random.default_rng(3)
    gu_codes = rng.integers(0, 16, size=(hidden, 2 * inter), dtype=np.uint8)
    d_codes = rng.integers(0, 16, size=(inter, hidden), dtype=np.uint8)
    gu_s = (np.abs(rng.normal(0, 0.01, (hidden // 128, 2 * inter))) + 1e-3).astype(np.float16)
    d_s = (np.abs(rng.normal(0, 0.01, (inter // 128, hidden))) + 1e-3).astype(np.float16)
    gu_q, d_q = O.marlin_pack_codes(gu_codes), O.marlin_pack_codes(d_codes)
    gu_sp, d_sp = O.marlin_pack_scales(gu_s), O.marlin_pack_scales(d_s)
    x = rng.normal(0, 1, (2, hidden)).astype(np.float16)
    got = O.marlin_mlp_streaming(x, gu_q, gu_sp, d_q, d_sp, hidden, inter, 128, 128)
    # float64 restatement through the scalar reader
    wgu = np.array([[O.marlin_weight_read(gu_q, gu_sp, n, k, 2 * inter, 128) for n in range(2 * inter)] for k in range(hidden)])
    wd = np.array([[O.marlin_weight_read(d_q, d_sp, n, k, hidden, 128) for n in range(hidden)] for k in range(inter)])
    gu = x.astype(np.float64) @ wgu
    act = gu[:, :inter] / (1 + np.exp(-gu[:, :inter])) * gu[:, inter:]
    ref = act @ wd
    assert np.allclose(got.astype(np.float64), ref, rtol=2e-3, atol=2e-3)


def test_byte_formulas():
    assert O.marlin_bytes(1, 5120, 17408) == 46_002_176
    assert O.marlin_bytes(4, 5120, 17408) == 46_137_344
    assert O.marlin_bytes(16, 5120, 17408) == 46_678_016
    assert O.rowwise_bytes(1, 4096, 4096, 4, 128) == 8_667_136
    assert O.rowwise_bytes(1, 17408, 5120, 3, 128) == 34_861_056
    assert O.rowwise_bytes(1, 17408, 5120, 8, 64) == 91_959_296


# ---- the vectorised torch-CPU restatement timed as the CPU baseline ----

@pytest.mark.parametrize("bits,group,cols", [(4, 128, 4096), (2, 64, 513), (3, 128, 257), (8, 32, 300)])
def test_torch_cpu_rowwise_matches_oracle(bits, group, cols):
    """oracle/torch_cpu.py's dense fp16 matrix is the numpy oracle's fp32
    ``q * s`` rounded to fp16, bit for bit (``loader.py:442-452``); its GEMV is
    within the parity tolerance of the oracle's fp32-accumulated one."""
    import torch

    from oracle import torch_cpu as T

    rows = 64
    _, packed, scales, x = O.make_rowwise_inputs(rows, cols, bits, group, seed=bits + cols)
    dense = T.rowwise_dequant_rows(torch.from_numpy(packed), torch.from_numpy(scales), cols, group, bits)
    want = O.rowwise_dequant_f32(packed, scales, cols, group, bits).astype(np.float16)
    assert np.array_equal(dense.numpy().view(np.uint16), want.view(np.uint16))
    y = T.rowwise_gemv(torch.from_numpy(packed), torch.from_numpy(scales), torch.from_numpy(x[0]), cols, group, bits)
    ref = O.rowwise_gemv(packed, scales, x[0], cols, group, bits).astype(np.float64)
    assert np.all(np.abs(y.numpy().astype(np.float64) - ref) <= 1e-2 + 1e-3 * np.abs(ref) + 2e-3 * np.abs(ref).max())


@pytest.mark.parametrize("group", [128, -1])
def test_torch_cpu_marlin_matches_oracle(group):
    """The torch-CPU Marlin unpack and fp16 dequant equal the oracle's bit for
    bit; the product is within the parity tolerance."""
    import torch

    from oracle import torch_cpu as T

    m, k, n = 3, 512, 768
    _, qw, _, sp, x = O.make_marlin_inputs(m, k, n, 128 if group == 128 else -1, seed=31)
    if group == -1:
        s = (np.abs(np.random.default_rng(2).normal(0, 0.01, (1, n))) + 1e-3).astype(np.float16)
        sp = O.marlin_pack_scales(s, per_column=True)
    w = T.marlin_dequant(torch.from_numpy(qw), torch.from_numpy(sp), group)
    assert np.array_equal(w.numpy().view(np.uint16), O.marlin_dequant_f16(qw, sp, group).view(np.uint16))
    y = T.marlin_gemm(torch.from_numpy(x), torch.from_numpy(qw), torch.from_numpy(sp), group).numpy()
    ref = O.marlin_gemm(x, qw, sp, group).astype(np.float64)
    assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-2 + 1e-3 * np.abs(ref))
