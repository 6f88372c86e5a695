"""ctypes binding of the C ABI (``include/langburst_lowbit.h``).

This is the binding a non-PyTorch host (or a test) uses: raw device pointers,
sizes and a ``hipStream_t``.  The helpers accept torch tensors for convenience
and pass ``tensor.data_ptr()`` and the current PyTorch stream; every call
returns the library's status code (0 == LB_OK).
"""
from __future__ import annotations

import ctypes
import re
from functools import lru_cache
from pathlib import Path

from . import library_path

HEADER = Path(__file__).resolve().parent.parent / "include" / "langburst_lowbit.h"

LB_OK = 0
LB_ERR_PROB_SHAPE = 1
LB_ERR_KERN_SHAPE = 2
LB_ERR_ARG = 3
LB_ERR_ALIGN = 4
LB_ERR_WORKSPACE = 5
LB_ERR_SCRATCH = 6
LB_ERR_HIP = 7
LB_ERR_NOALLOC_LIMIT = 9

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
SZ = ctypes.c_size_t

_SIGNATURES = {
    "lb_status_string": ([ctypes.c_int], ctypes.c_char_p),
    "lb_abi_version": ([], ctypes.c_int),
    "lb_lowbit_gemv": ([P, I64, I64, P, I64, P, P, I64, I64, I64, I64, P], ctypes.c_int),
    "lb_lowbit_gemv_pair": ([P, P, P, P, I64, I64, I64, P, P, P, I64, I64, I64, I64, P], ctypes.c_int),
    "lb_lowbit_gemm": ([P, I64, I64, P, I64, P, I64, I64, P, I64, I64, I64, I64, P], ctypes.c_int),
    "lb_lowbit_row_dequant": ([P, I64, I64, P, I64, P, P, I64, I64, I64, P], ctypes.c_int),
    "lb_marlin_scratch_bytes": ([I64, I64, I64, I64], SZ),
    "lb_marlin_describe_plan": ([I64, I64, I64, I64, ctypes.c_int32, I64, P], ctypes.c_int),
    "lb_marlin_gemm": ([P, P, P, P, I64, I64, I64, P, I64, I64, P, SZ, P], ctypes.c_int),
    "lb_marlin_gemm_silu_packed": ([P, P, P, P, I64, I64, I64, P, I64, I64, P, SZ, P], ctypes.c_int),
    "lb_marlin_gemm_argmax": ([P, P, P, I64, I64, I64, P, I64, I64, P, P, P, I32, P, SZ, P], ctypes.c_int),
    "lb_marlin_mlp_scratch_bytes": ([I64, I64, I64], SZ),
    "lb_marlin_mlp_streaming": ([P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, SZ, P], ctypes.c_int),
    "lb_marlin_dequant": ([P, P, P, I64, I64, I64, P], ctypes.c_int),
    "lb_probe_stream_read": ([P, SZ, P, I32, P], ctypes.c_int),
    "lb_marlin_noalloc_scratch_limit": ([], SZ),
    "lb_marlin_gemm_noalloc": ([P, P, P, P, I64, I64, I64, P, I64, I64, P], ctypes.c_int),
    "lb_marlin_mlp_fused_scratch_bytes": ([I64, I64, I64], SZ),
    "lb_marlin_mlp_fused_workspace_len": ([I64, I64, I64], I64),
    "lb_marlin_mlp_fused": ([P, P, P, P, P, P, I64, I64, I64, I64, I64, P, I64, P, SZ, P], ctypes.c_int),
}


def declared_symbols() -> list[str]:
    """Entry points declared in ``include/langburst_lowbit.h``."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(lb_\w+)\s*\(", text, flags=re.M)))


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    path = library_path()
    if not path.exists():
        raise OSError(f"{path} is not built; run `python -m neurova_amd.build`")
    try:
        import torch  # noqa: F401  (share PyTorch's HIP runtime when present)
    except ImportError:
        pass
    cdll = ctypes.CDLL(str(path))
    for name, (argtypes, restype) in _SIGNATURES.items():
        fn = getattr(cdll, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return cdll


def _ptr(t) -> int | None:
    return None if t is None else int(t.data_ptr())


def _stream(t) -> int:
    import torch

    return int(torch.cuda.current_stream(t.device).cuda_stream)


def status_string(code: int) -> str:
    return lib().lb_status_string(int(code)).decode()


def lowbit_gemv(qweight, scales, x, y, cols, group_size, bits, rows_per_cta=8) -> int:
    return lib().lb_lowbit_gemv(_ptr(qweight), qweight.shape[0], qweight.shape[1], _ptr(scales), scales.shape[1],
                                _ptr(x), _ptr(y), cols, group_size, bits, rows_per_cta, _stream(x))


def lowbit_gemv_pair(qa, sa, qb, sb, x, ya, yb, cols, group_size, bits, rows_per_cta=8) -> int:
    return lib().lb_lowbit_gemv_pair(_ptr(qa), _ptr(sa), _ptr(qb), _ptr(sb), qa.shape[0], qa.shape[1], sa.shape[1],
                                     _ptr(x), _ptr(ya), _ptr(yb), cols, group_size, bits, rows_per_cta, _stream(x))


def lowbit_gemm(qweight, scales, x, y, cols, group_size, bits, rows_per_cta=8) -> int:
    return lib().lb_lowbit_gemm(_ptr(qweight), qweight.shape[0], qweight.shape[1], _ptr(scales), scales.shape[1],
                                _ptr(x), x.shape[0], x.shape[1], _ptr(y), cols, group_size, bits, rows_per_cta,
                                _stream(x))


def lowbit_row_dequant(qweight, scales, row, out, cols, group_size, bits) -> int:
    return lib().lb_lowbit_row_dequant(_ptr(qweight), qweight.shape[0], qweight.shape[1], _ptr(scales),
                                       scales.shape[1], _ptr(row), _ptr(out), cols, group_size, bits, _stream(out))


def marlin_scratch_bytes(m, n, k, group_size) -> int:
    return int(lib().lb_marlin_scratch_bytes(m, n, k, group_size))


PLAN_FIELDS = ("form", "chunks_or_row_blocks", "splits", "row_blocks_or_full_tiles", "workgroups", "lds_bytes",
               "scratch_bytes", "workspace_entries", "launches", "cus")
PLAN_FORMS = ("staged", "direct", "ring", "prefill", "prefill-streamk")


def marlin_describe_plan(m, n, k, group_size, variant=0, workspace_len=None) -> dict:
    """The plan lb_marlin_gemm (variant 0), the SiLU-gated op (1) or the argmax
    op (2) makes for this problem; no device work.  Raises on a rejected shape."""
    out = (ctypes.c_int64 * 10)()
    ws = n // 128 * 16 if workspace_len is None else workspace_len
    st = lib().lb_marlin_describe_plan(m, n, k, group_size, variant, ws, ctypes.cast(out, ctypes.c_void_p))
    if st != LB_OK:
        raise ValueError(f"lb_marlin_describe_plan: {status_string(st)}")
    d = dict(zip(PLAN_FIELDS, (int(v) for v in out)))
    d["form"] = PLAN_FORMS[d["form"]]
    return d


def marlin_gemm(a, b, c, s, workspace, group_size, scratch=None) -> int:
    m, k = a.shape
    n = b.shape[1] // 2
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    return lib().lb_marlin_gemm(_ptr(a), _ptr(b), _ptr(c), _ptr(s), m, n, k, _ptr(workspace), workspace.numel(),
                                group_size, _ptr(scratch), nbytes, _stream(a))


def marlin_gemm_silu_packed(mixed, b, c, s, workspace, group_size, scratch=None) -> int:
    m = mixed.shape[0]
    k = mixed.shape[1] // 2
    n = b.shape[1] // 2
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    return lib().lb_marlin_gemm_silu_packed(_ptr(mixed), _ptr(b), _ptr(c), _ptr(s), m, n, k, _ptr(workspace),
                                            workspace.numel(), group_size, _ptr(scratch), nbytes, _stream(mixed))


def marlin_gemm_argmax(a, b, s, workspace, group_size, state, out, sync, epoch, scratch=None) -> int:
    m, k = a.shape
    n = b.shape[1] // 2
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    return lib().lb_marlin_gemm_argmax(_ptr(a), _ptr(b), _ptr(s), m, n, k, _ptr(workspace), workspace.numel(),
                                       group_size, _ptr(state), _ptr(out), _ptr(sync), epoch, _ptr(scratch), nbytes,
                                       _stream(a))


def marlin_mlp_scratch_bytes(batch, hidden, intermediate) -> int:
    return int(lib().lb_marlin_mlp_scratch_bytes(batch, hidden, intermediate))


def marlin_mlp_streaming(gu_q, gu_s, d_q, d_s, x, out, accum, sync, hidden, intermediate, gg, dg, scratch) -> int:
    nbytes = scratch.numel() * scratch.element_size()
    return lib().lb_marlin_mlp_streaming(_ptr(gu_q), _ptr(gu_s), _ptr(d_q), _ptr(d_s), _ptr(x), _ptr(out),
                                         _ptr(accum), _ptr(sync), x.shape[0], hidden, intermediate, gg, dg,
                                         _ptr(scratch), nbytes, _stream(x))


def marlin_mlp_fused_scratch_bytes(batch, hidden, intermediate) -> int:
    return int(lib().lb_marlin_mlp_fused_scratch_bytes(batch, hidden, intermediate))


def marlin_mlp_fused_workspace_len(batch, hidden, intermediate) -> int:
    return int(lib().lb_marlin_mlp_fused_workspace_len(batch, hidden, intermediate))


def marlin_mlp_fused(x, gu_q, gu_s, d_q, d_s, out, hidden, intermediate, gg, dg, workspace, scratch) -> int:
    nbytes = scratch.numel() * scratch.element_size()
    return lib().lb_marlin_mlp_fused(_ptr(x), _ptr(gu_q), _ptr(gu_s), _ptr(d_q), _ptr(d_s), _ptr(out), x.shape[0],
                                     hidden, intermediate, gg, dg, _ptr(workspace), workspace.numel(),
                                     _ptr(scratch), nbytes, _stream(x))


def marlin_dequant(b, s, w_nk, k, group_size) -> int:
    n = b.shape[1] // 2
    return lib().lb_marlin_dequant(_ptr(b), _ptr(s), _ptr(w_nk), n, k, group_size, _stream(w_nk))


def probe_stream_read(src, sink, workgroups) -> int:
    return lib().lb_probe_stream_read(_ptr(src), src.numel() * src.element_size(), _ptr(sink), int(workgroups),
                                      _stream(src))


def marlin_noalloc_scratch_limit() -> int:
    return int(lib().lb_marlin_noalloc_scratch_limit())


def marlin_gemm_noalloc(a, b, c, s, workspace, group_size) -> int:
    m, k = a.shape
    n = b.shape[1] // 2
    return lib().lb_marlin_gemm_noalloc(_ptr(a), _ptr(b), _ptr(c), _ptr(s), m, n, k, _ptr(workspace),
                                        workspace.numel(), group_size, _stream(a))
