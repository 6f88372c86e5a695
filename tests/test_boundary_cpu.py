"""The drop-in boundary without a GPU: the C-ABI library and the ``langburst_cuda`` module.

Checks that ``lib/liblangburst_lowbit.so`` loads and exports exactly the entry
points ``include/langburst_lowbit.h`` declares, that argument validation
returns the documented status codes before any device work (fake, never
dereferenced pointers), and that the PyTorch module exposes the reference's op
names and rejects host tensors with the reference's messages
(``langburst/csrc/langburst_ext.cpp:68-94``, ``csrc/kernels.cuh:17-18``).
No kernel is launched here.
"""
from __future__ import annotations

import ctypes

import pytest

from neurova_amd import capi

FAKE = 0x10000  # 64 KiB aligned, never dereferenced: validation fails or returns first
MIS = 0x10002   # 2-byte aligned only


def _gpu_present() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


# The fake pointers below are never meant to reach a kernel; with a GPU present
# a mistake in a case could launch on them, so these checks run on CPU hosts only.
pytestmark = pytest.mark.skipif(_gpu_present(), reason="host-side validation checks use fake device pointers")


@pytest.fixture(scope="module")
def L(built):
    return capi.lib()


def test_exports_match_header(L):
    declared = capi.declared_symbols()
    assert declared, "no declarations parsed from the header"
    assert sorted(capi._SIGNATURES) == declared
    for name in declared:
        assert hasattr(L, name), name


def test_version_and_status_strings(L):
    assert L.lb_abi_version() == 1
    assert L.lb_status_string(capi.LB_OK) == b"ok"
    assert L.lb_status_string(capi.LB_ERR_PROB_SHAPE) == b"problem shape not supported"
    assert L.lb_status_string(capi.LB_ERR_WORKSPACE) == b"workspace too small"
    assert L.lb_status_string(99) == b"unknown status"


def _marlin(L, m=1, n=256, k=256, g=128, a=FAKE, b=FAKE, c=FAKE, s=FAKE, ws=FAKE, ws_len=64, scratch=FAKE,
            scratch_bytes=1 << 30):
    return L.lb_marlin_gemm(a, b, c, s, m, n, k, ws, ws_len, g, scratch, scratch_bytes, None)


def test_marlin_shape_and_argument_rejection(L):
    assert _marlin(L, n=300) == capi.LB_ERR_PROB_SHAPE   # N % 256
    assert _marlin(L, k=100) == capi.LB_ERR_PROB_SHAPE   # K % 128
    assert _marlin(L, g=64) == capi.LB_ERR_PROB_SHAPE    # group 64 unsupported (langburst_ext.cpp:88)
    assert _marlin(L, m=-1) == capi.LB_ERR_ARG
    assert _marlin(L, m=0) == capi.LB_OK                 # empty batch is a no-op
    assert _marlin(L, a=None) == capi.LB_ERR_ARG
    assert _marlin(L, c=None) == capi.LB_ERR_ARG
    assert _marlin(L, a=MIS) == capi.LB_ERR_ALIGN
    assert _marlin(L, s=MIS) == capi.LB_ERR_ALIGN


def test_marlin_workspace_and_scratch_rejection(L):
    m, n, k = 1, 17408, 5120
    need = L.lb_marlin_scratch_bytes(m, n, k, 128)
    assert need > 0 and need % 256 == 0
    # with the reference-sized workspace the decode plan splits K, so it needs the partials
    ws = n // 128 * 16
    assert _marlin(L, m=m, n=n, k=k, ws_len=ws, scratch=None, scratch_bytes=0) == capi.LB_ERR_SCRATCH
    assert _marlin(L, m=m, n=n, k=k, ws_len=ws, scratch=FAKE, scratch_bytes=16) == capi.LB_ERR_SCRATCH
    assert _marlin(L, m=m, n=n, k=k, ws_len=ws, scratch=MIS, scratch_bytes=need) == capi.LB_ERR_ALIGN
    # argmax needs its arrival counter even without a split
    assert L.lb_marlin_gemm_argmax(FAKE, FAKE, FAKE, m, n, k, FAKE, 0, 128, FAKE, FAKE, FAKE, 1, FAKE, need,
                                   None) == capi.LB_ERR_WORKSPACE


def test_scratch_sizes(L):
    assert L.lb_marlin_scratch_bytes(0, 256, 256, 128) == 0
    assert L.lb_marlin_scratch_bytes(1, 300, 256, 128) == 0
    # decode: S * M * N * 4 partials + M * (N/256) * 8 argmax keys, both 256-byte aligned
    s1 = L.lb_marlin_scratch_bytes(1, 17408, 5120, 128)
    s16 = L.lb_marlin_scratch_bytes(16, 17408, 5120, 128)
    assert s16 > s1 >= 17408 * 4
    assert L.lb_marlin_mlp_scratch_bytes(1, 256, 512) > 0
    assert L.lb_marlin_mlp_scratch_bytes(0, 256, 512) == 0


def _mlp_fused(L, batch=1, hidden=5120, inter=17408, gg=128, dg=128, x=FAKE, out=FAKE, ws_len=None, scratch=FAKE,
               scratch_bytes=None):
    ws_len = L.lb_marlin_mlp_fused_workspace_len(1, hidden, inter) if ws_len is None else ws_len
    sb = L.lb_marlin_mlp_fused_scratch_bytes(1, hidden, inter) if scratch_bytes is None else scratch_bytes
    return L.lb_marlin_mlp_fused(x, FAKE, FAKE, FAKE, FAKE, out, batch, hidden, inter, gg, dg, FAKE, ws_len,
                                 scratch, sb, None)


def test_mlp_fused_rejection_and_sizes(L):
    h, i = 5120, 17408
    ws = L.lb_marlin_mlp_fused_workspace_len(1, h, i)
    sb = L.lb_marlin_mlp_fused_scratch_bytes(1, h, i)
    # each projection's counters; [g | u] (or the activations) then either launch's partials fit in scratch
    assert ws >= 2 + (2 * i) // 256 and sb % 256 == 0 and sb >= 2 * i * 2
    assert L.lb_marlin_mlp_fused_scratch_bytes(0, h, i) == 0
    assert _mlp_fused(L, batch=0) == capi.LB_OK
    assert _mlp_fused(L, batch=-1) == capi.LB_ERR_ARG
    assert _mlp_fused(L, hidden=300) == capi.LB_ERR_PROB_SHAPE   # hidden % 256
    assert _mlp_fused(L, inter=1000) == capi.LB_ERR_PROB_SHAPE   # intermediate % 128
    assert _mlp_fused(L, gg=64) == capi.LB_ERR_PROB_SHAPE
    assert _mlp_fused(L, x=None) == capi.LB_ERR_ARG
    assert _mlp_fused(L, x=MIS) == capi.LB_ERR_ALIGN
    assert _mlp_fused(L, ws_len=ws - 1) == capi.LB_ERR_WORKSPACE
    assert _mlp_fused(L, scratch_bytes=16) == capi.LB_ERR_SCRATCH
    assert _mlp_fused(L, scratch=FAKE + 16) == capi.LB_ERR_ALIGN


def test_marlin_dequant_rejection(L):
    assert L.lb_marlin_dequant(FAKE, FAKE, FAKE, 300, 256, 128, None) == capi.LB_ERR_PROB_SHAPE
    assert L.lb_marlin_dequant(FAKE, FAKE, FAKE, 256, 256, 64, None) == capi.LB_ERR_PROB_SHAPE
    assert L.lb_marlin_dequant(None, FAKE, FAKE, 256, 256, 128, None) == capi.LB_ERR_ARG
    assert L.lb_marlin_dequant(FAKE, FAKE, FAKE, 0, 256, 128, None) == capi.LB_OK


def test_rowwise_argument_rejection(L):
    # lb_lowbit_gemv(q, rows, packed_cols, s, scale_cols, x, y, cols, group, bits, rows_per_cta, stream)
    ok_args = dict(rows=64, packed_cols=2048, scale_cols=32, cols=4096, group=128, bits=4, rpc=8)

    def gemv(q=FAKE, s=FAKE, x=FAKE, y=FAKE, **kw):
        a = {**ok_args, **kw}
        return L.lb_lowbit_gemv(q, a["rows"], a["packed_cols"], s, a["scale_cols"], x, y, a["cols"], a["group"],
                                a["bits"], a["rpc"], None)

    assert gemv(bits=1) == capi.LB_ERR_ARG
    assert gemv(bits=9) == capi.LB_ERR_ARG
    assert gemv(group=0) == capi.LB_ERR_ARG
    assert gemv(scale_cols=31) == capi.LB_ERR_ARG       # fewer scale columns than groups
    assert gemv(packed_cols=2047) == capi.LB_ERR_ARG    # fewer packed bytes than cols * bits / 8
    assert gemv(q=None) == capi.LB_ERR_ARG
    assert gemv(x=None) == capi.LB_ERR_ARG
    assert gemv(rpc=5) == capi.LB_ERR_ARG               # rows_per_cta in {4, 8, 16}
    assert gemv(rows=0) == capi.LB_OK


def test_module_surface_and_host_tensor_messages(built):
    import torch

    import neurova_amd

    lc = neurova_amd.load_extension()
    for name in ("lowbit_gemv", "lowbit_row_dequant", "lowbit_gemv_pair", "lowbit_gemm", "lowbit_marlin_gemm",
                 "lowbit_marlin_gemm_out", "lowbit_marlin_mlp_streaming_out", "lowbit_marlin_gemm_silu_packed_out",
                 "lowbit_marlin_gemm_argmax_out"):
        assert callable(getattr(lc, name)), name
    q = torch.zeros((64, 2048), dtype=torch.uint8)
    s = torch.zeros((64, 32), dtype=torch.float16)
    x = torch.zeros((4096,), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="qweight must be CUDA"):
        lc.lowbit_gemv(q, s, x, 4096, 128, 4)
    qm = torch.zeros((16, 512), dtype=torch.int32)
    sm = torch.zeros((2, 256), dtype=torch.float16)
    xm = torch.zeros((1, 256), dtype=torch.float16)
    with pytest.raises(RuntimeError, match="must be CUDA"):
        lc.lowbit_marlin_gemm(qm, sm, xm, 256, 128)
    # the one-call decode MLP (no reference op of its own) checks like the streaming op
    assert lc.lowbit_marlin_mlp_fused_workspace_len(1, 5120, 17408) == capi.lib().lb_marlin_mlp_fused_workspace_len(
        1, 5120, 17408)
    gu = torch.zeros((16, 4 * 512), dtype=torch.int32)
    with pytest.raises(RuntimeError, match="must be CUDA"):
        lc.lowbit_marlin_mlp_fused_out(gu, sm, qm, sm, xm, xm, torch.zeros(8, dtype=torch.int32), 256, 512, 128,
                                       128)


def test_ops_never_fall_back_to_cpu(monkeypatch, built):
    from neurova_amd import ops

    ops.cuda_ops.cache_clear()
    monkeypatch.setenv("LANGBURST_CPU_FALLBACK", "1")
    with pytest.raises(ops.ExtensionMissingError, match="no CPU fallback"):
        ops.cuda_ops()
    ops.cuda_ops.cache_clear()
    monkeypatch.delenv("LANGBURST_CPU_FALLBACK")
    assert ops.cuda_ops() is not None  # the compiled module itself
    ops.cuda_ops.cache_clear()


def test_product_path_does_not_import_the_oracle():
    """Only tests, smoke() and bench.py's CPU baseline may use oracle/."""
    import pathlib

    pkg = pathlib.Path(capi.__file__).resolve().parent
    for path in list(pkg.rglob("*.py")) + list(pkg.rglob("*.cpp")) + list(pkg.rglob("*.hip")) + list(
            pkg.rglob("*.hpp")):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path
        assert "lowbit_oracle" not in text and "lowbit_ref" not in text, path
