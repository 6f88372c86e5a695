"""The Marlin host planner's choices, without a GPU (``lb_marlin_describe_plan``).

Each entry point plans its launch on the host: the decode form (A staged whole,
A fragments loaded per step, A through an LDS ring) or the prefill GEMM, the
tile width, the k splits, the LDS, scratch and workspace it needs.  These tests
sweep the BASELINE.json shapes and edge shapes and check the invariants the kernels
rely on (every wave gets a scale group, LDS within a workgroup's 64 KB, the
workspace within the reference's N/128*16 entries, the split arithmetic within
32 bits) and the rules the measurements chose (``make_plan`` in
``neurova_amd/csrc/lb_marlin.hip``).  No kernel is launched.
"""
from __future__ import annotations

import itertools

import pytest

from neurova_amd import capi

MS = [1, 2, 3, 4, 5, 8, 15, 16, 17, 20, 24, 31, 32, 33, 48, 64, 100, 256, 2048]
NS = [256, 512, 1280, 5120, 7168, 16384, 17408, 34816, 248320]
KS = [128, 256, 640, 2048, 5120, 17408]
LDS_LIMIT = 64 * 1024


@pytest.fixture(scope="module")
def L(built):
    return capi.lib()


def _plan(m, n, k, g=128, variant=0, ws=None):
    return capi.marlin_describe_plan(m, n, k, g, variant, ws)


@pytest.mark.parametrize("variant", [0, 1, 2])
def test_plan_invariants(L, variant):
    for m, n, k in itertools.product(MS, NS, KS):
        if variant == 1 and m > 64 and n > 17408:
            continue  # the SiLU-gated op at prefill sizes is covered by the BASELINE.json shapes below
        p = _plan(m, n, k, 128, variant)
        what = f"m={m} n={n} k={k} variant={variant}: {p}"
        assert p["workgroups"] >= 1, what
        assert p["workspace_entries"] <= n // 128 * 16, what  # the reference's workspace
        assert p["scratch_bytes"] <= L.lb_marlin_scratch_bytes(m, n, k, 128), what
        if p["form"] == "prefill":
            assert m > 16, what
            assert p["chunks_or_row_blocks"] in (2, 4, 8), what
            assert p["launches"] == 1, what
            continue
        if p["form"] == "prefill-streamk":
            # 128-row tiles filling between half of one round of the resident slots and all of it
            tiles, slots = -(-m // 128) * (n // 256), 2 * p["cus"]
            assert m >= 128 and p["chunks_or_row_blocks"] == 8 and p["launches"] == 1, what
            assert tiles < slots <= 2 * tiles and p["workgroups"] == slots, what
            assert p["workspace_entries"] == 1 + tiles, what
            continue
        cpw, s, mr = p["chunks_or_row_blocks"], p["splits"], p["row_blocks_or_full_tiles"]
        assert cpw in (1, 2, 4) and 1 <= s <= 256, what
        chunks, cus = n // 64, p["cus"]
        if cpw == 1 and p["workgroups"] != chunks * s:
            # mixed: one or two whole-K single-chunk tiles per CU, the leftover chunks split s ways;
            # A staged up to M = 4, loaded per step (direct) for M = 5..32 with one whole-K tile
            # per CU, or two up to M = 8
            whole = min(chunks // cus, 2) * cus
            assert cus < chunks and (chunks - whole) * 8 <= cus and k <= 5120, what
            if m <= 4:
                assert p["form"] == "staged", what
            else:
                assert p["form"] == "direct" and m <= 32 and (chunks < 2 * cus or m <= 8), what
                assert p["row_blocks_or_full_tiles"] == (m + 15) // 16, what
            assert m <= 3 or s <= 6, what  # M >= 4: at most 6 leftover splits
            assert p["workgroups"] == whole + (chunks - whole) * s, what
        else:
            assert p["workgroups"] == (n // (64 * cpw)) * s, what
        assert p["lds_bytes"] <= LDS_LIMIT, what
        # every wave of a tile gets at least one scale group of its split
        assert (k // 128) // s >= 4 // cpw, what
        assert (k // 128) * s < 2 ** 32, what
        assert mr == (1 if p["form"] == "staged" else (m + 15) // 16), what
        assert m <= 32 and (m <= 16 or p["form"] != "staged"), what
        if variant == 2:
            assert p["form"] == "staged", what  # the argmax epilogue runs on staged tiles only
        if p["form"] == "ring":
            assert cpw == 4, what
        if p["form"] == "direct":
            assert cpw in (1, 2) and (m <= 16 or cpw == 1), what
        assert p["launches"] == (2 if variant == 1 and p["form"] != "staged" else 1), what


def test_plan_rules_at_baseline_shapes(L):
    # headline (cfg2): one whole-K single-chunk tile per CU (256), the 16
    # leftover chunks split 10 ways: 416 workgroups; N = 16384: 256 whole tiles
    p = _plan(1, 17408, 5120)
    assert (p["form"], p["chunks_or_row_blocks"], p["splits"], p["workgroups"]) == ("staged", 1, 10, 416)
    p = _plan(1, 16384, 5120)
    assert (p["form"], p["chunks_or_row_blocks"], p["splits"], p["workgroups"]) == ("staged", 1, 1, 256)
    # M = 2 and 3 take the mixed plan too; M = 4 with at most 6 leftover splits
    for m in (2, 3):
        assert _plan(m, 17408, 5120)["workgroups"] == 416
    p = _plan(4, 17408, 5120)
    assert (p["form"], p["chunks_or_row_blocks"], p["splits"], p["workgroups"]) == ("staged", 1, 6, 256 + 16 * 6)
    assert _plan(4, 16384, 5120)["workgroups"] == 256 and _plan(4, 16640, 2048)["workgroups"] == 256 + 4 * 4
    # gate/up (N = 34816): two whole-K tiles per CU, the 32 leftover chunks split 8 ways
    p = _plan(1, 34816, 5120)
    assert (p["form"], p["chunks_or_row_blocks"], p["splits"], p["workgroups"]) == ("staged", 1, 8, 768)
    # K = 17408 keeps the split 4-chunk tiles
    assert _plan(1, 17408, 17408)["chunks_or_row_blocks"] == 4
    # narrow decode projections take 64-column direct tiles
    for m in (1, 4, 16):
        assert _plan(m, 7168, 5120)["form"] == "direct"
        assert _plan(m, 5120, 5120)["form"] == "direct"
    # SiLU-gated down: staged up to 4 rows (the gating launch does not pay), direct from 5
    assert _plan(4, 5120, 17408, variant=1)["form"] == "staged"
    d = _plan(5, 5120, 17408, variant=1)
    assert d["form"] == "direct" and d["launches"] == 2
    # gate/up at M = 16: staging the slice would force 4 splits (544 workgroups); the ring plans 3
    r = _plan(16, 34816, 5120)
    assert (r["form"], r["splits"], r["workgroups"]) == ("ring", 3, 408)
    # M = 17..32: 64-column direct tiles, the ring on 4-chunk tiles, 2-chunk tiles to the prefill kernel
    assert _plan(32, 7168, 5120)["form"] == "direct"
    assert _plan(32, 34816, 5120)["form"] == "ring"
    # N = 17408 at M = 5..32: one whole-K single-chunk tile per CU, A loaded per step, the 16
    # leftover chunks split 6 ways
    h = _plan(32, 17408, 5120)
    assert (h["form"], h["chunks_or_row_blocks"], h["row_blocks_or_full_tiles"], h["splits"], h["workgroups"]) == \
        ("direct", 1, 2, 6, 256 + 16 * 6)
    assert _plan(16, 17408, 5120)["workgroups"] == 256 + 16 * 6
    # two whole-K tiles per CU only up to M = 8 (gate/up)
    assert _plan(8, 34816, 5120)["workgroups"] == 512 + 32 * 6 and _plan(9, 34816, 5120)["form"] != "direct"
    assert _plan(33, 7168, 5120)["form"] == "prefill"
    # prefill (cfg3): N = 17408, K = 5120: 1088 128-row tiles, 1024 whole, the tail split over K;
    # N = 5120, K = 17408: 320 tiles on the stream-K schedule, one range per resident slot
    g = _plan(2048, 17408, 5120)
    assert (g["form"], g["chunks_or_row_blocks"], g["row_blocks_or_full_tiles"], g["splits"]) == ("prefill", 8, 1024, 3)
    g2 = _plan(2048, 5120, 17408)
    assert (g2["form"], g2["workgroups"], g2["scratch_bytes"]) == ("prefill-streamk", 512, 2 * 512 * 128 * 256 * 4)
    # fewer tiles than half the slots: split tail; a whole number of rounds: whole tiles
    t = _plan(256, 17408, 5120)
    assert (t["form"], t["row_blocks_or_full_tiles"], t["splits"]) == ("prefill", 0, 3)
    w = _plan(2048, 16384, 5120)
    assert (w["form"], w["row_blocks_or_full_tiles"], w["splits"], w["workgroups"]) == ("prefill", 1024, 1, 1024)
    # lm_head argmax (N = 248320): staged tiles, one split
    a = _plan(1, 248320, 5120, variant=2)
    assert a["form"] == "staged" and a["workgroups"] >= 256


def test_plan_without_workspace_does_not_split(L):
    for m, n, k in ((1, 17408, 5120), (16, 5120, 17408), (32, 7168, 5120), (4, 34816, 5120)):
        p = _plan(m, n, k, 128, 0, ws=0)
        assert p["splits"] == 1 and p["workspace_entries"] == 0, p
        p1 = _plan(m, n, k, 128, 0, ws=1)
        assert p1["workspace_entries"] <= 1, p1


def test_plan_rejects_what_the_entry_points_reject(L):
    with pytest.raises(ValueError):
        _plan(1, 300, 256)
    with pytest.raises(ValueError):
        _plan(1, 256, 200)
    with pytest.raises(ValueError):
        _plan(1, 256, 256, g=64)
    assert _plan(0, 256, 256)["workgroups"] == 0


# The decode projections of BASELINE.json configs[4] and the ones the reference
# publishes timings for (langburst/docs/PERFORMANCE_LOG.md:421-427), K x N.
NOALLOC_SHAPES = {"qkv": (5120, 7168), "o": (5120, 5120), "gate_up": (5120, 34816), "down": (17408, 5120),
                  "attn_qkv": (5120, 14336), "gdn_qkvz": (5120, 16384), "gdn_out": (6144, 5120),
                  "lm_head": (5120, 248320)}


@pytest.mark.parametrize("name", sorted(NOALLOC_SHAPES))
def test_noalloc_scratch_covers_decode_shapes(L, name):
    """lb_marlin_gemm_noalloc's static scratch holds the partials of every plan
    of these shapes up to M = 64 (the header's claim), grouped or per-column scales."""
    k, n = NOALLOC_SHAPES[name]
    limit = capi.marlin_noalloc_scratch_limit()
    for m in range(1, 65):
        for g in (128, -1):
            assert capi.marlin_scratch_bytes(m, n, k, g) <= limit, (name, m, g)
