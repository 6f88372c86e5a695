"""Writes the golden fixtures under tests/golden/ from the reference's own data.

Run in the build container only (it reads /root/reference as text; nothing is
imported or executed from there).  The outputs are committed; tests never read
the reference at run time.

Fixtures written:

* ``marlin_tables.json`` -- SHA-256 (little-endian int32 bytes), length and a
  few sampled entries of the three inverse-permutation tables the reference
  holds as constants in ``langburst/csrc/marlin_mlp_stream.cu:7-84``
  (``LB_MARLIN_INV_PERM``, ``LB_MARLIN_INV_SCALE_PERM``,
  ``LB_MARLIN_INV_SCALE_PERM_SINGLE``).  Only hashes and samples are stored.
* ``rowwise_kats.json`` -- the reference's known-answer vectors for the
  rowwise decode (``langburst/tests/test_v05_cuda_kernels.py:19-32``) and its
  packed-shape invariants (``langburst/tests/test_quant_lowbit_cpu.py:34-35,63``),
  transcribed as data.
"""
from __future__ import annotations

import hashlib
import json
import re
from pathlib import Path

import numpy as np

REF = Path("/root/reference/langburst")
OUT = Path(__file__).resolve().parent


def _table(src: str, name: str) -> np.ndarray:
    m = re.search(name + r"\[(\d+)\]\s*=\s*\{([^}]*)\}", src)
    if m is None:
        raise RuntimeError(f"table {name} not found")
    vals = [int(v) for v in m.group(2).replace("\n", " ").split(",") if v.strip()]
    if len(vals) != int(m.group(1)):
        raise RuntimeError(f"table {name}: expected {m.group(1)} entries, got {len(vals)}")
    return np.array(vals, dtype="<i4")


def main() -> None:
    src = (REF / "csrc" / "marlin_mlp_stream.cu").read_text()
    tables = {}
    for name in ("LB_MARLIN_INV_PERM", "LB_MARLIN_INV_SCALE_PERM", "LB_MARLIN_INV_SCALE_PERM_SINGLE"):
        t = _table(src, name)
        sample_idx = [0, 1, 7, 8, 31, 32, len(t) // 2, len(t) - 1]
        tables[name] = {
            "length": int(t.size),
            "sha256_le_int32": hashlib.sha256(t.tobytes()).hexdigest(),
            "samples": {str(i): int(t[i]) for i in sample_idx if i < t.size},
        }
    (OUT / "marlin_tables.json").write_text(json.dumps({
        "source": "langburst/csrc/marlin_mlp_stream.cu:7-84",
        "tables": tables,
    }, indent=2) + "\n")

    kats = {
        "source": "langburst/tests/test_v05_cuda_kernels.py:19-32",
        "row_dequant_scale_one": [
            {"bits": 4, "packed": [0x80, 0x97, 0x0F], "expected": [-8.0, 0.0, -1.0, 1.0, 7.0]},
            {"bits": 3, "packed": [0xE0, 0x01], "expected": [-4.0, 0.0, 3.0, -4.0]},
        ],
        "shape_source": "langburst/tests/test_quant_lowbit_cpu.py:34-35,63",
        "shapes": [
            {"rows": 7, "cols": 257, "bits": 4, "group_size": 128, "packed": [7, 129], "scales": [7, 3]},
            {"rows": 5, "cols": 17, "bits": 3, "group_size": 8, "packed": [5, 7], "scales": [5, 3]},
        ],
    }
    (OUT / "rowwise_kats.json").write_text(json.dumps(kats, indent=2) + "\n")
    print("wrote", OUT / "marlin_tables.json", OUT / "rowwise_kats.json")


if __name__ == "__main__":
    main()
