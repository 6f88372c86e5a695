"""Environment-resolved knobs of the low-bit path.

Mirrors ``langburst/langburst/tuning.py:6-8,44-62``: ``rows_per_cta`` for the
rowwise ops (choices 4/8/16, default 8; the gfx950 kernels validate it but pick
their own tiling) and the batch above which ``LowBitMarlinTensor.gemm`` splits
a batch into single rows (default 256).
"""
from __future__ import annotations

import os

LOWBIT_ROWS_PER_CTA_CHOICES = (4, 8, 16)
DEFAULT_LOWBIT_ROWS_PER_CTA = 8
DEFAULT_MARLIN_DIRECT_MAX_BATCH = 256


def lowbit_rows_per_cta(value: int | str | None = None) -> int:
    raw = value if value is not None else os.environ.get("LANGBURST_LOWBIT_ROWS_PER_CTA")
    if raw is None or raw == "":
        return DEFAULT_LOWBIT_ROWS_PER_CTA
    rows = int(raw)
    if rows not in LOWBIT_ROWS_PER_CTA_CHOICES:
        choices = ", ".join(str(v) for v in LOWBIT_ROWS_PER_CTA_CHOICES)
        raise ValueError(f"lowbit rows_per_cta must be one of: {choices}")
    return rows


def marlin_direct_max_batch(value: int | str | None = None) -> int:
    raw = value if value is not None else os.environ.get("LANGBURST_MARLIN_DIRECT_MAX_BATCH")
    if raw is None or raw == "":
        return DEFAULT_MARLIN_DIRECT_MAX_BATCH
    batch = int(raw)
    if batch < 1:
        raise ValueError("Marlin direct max batch must be >= 1")
    return batch
