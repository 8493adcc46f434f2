"""Host logic of bench.py's GEMM phase summary (no GPU): per-tile phases and
the gap between consecutive tiles on one CU, from synthetic stamp words."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _hw_id(se, sh, cu):
    return (se << 13) | (sh << 12) | (cu << 8)


def test_stamp_phases_known_schedule():
    # two CUs (XCC 0 / SE 1 / CU 3 and XCC 2 / SE 0 / CU 5), two tiles each,
    # the second tile on a CU starting 700 / 900 cycles after the first ends
    rows = []
    for xcc, hw, starts in ((0, _hw_id(1, 0, 3), (1000, None)), (2, _hw_id(0, 1, 5), (5000, None))):
        t0 = starts[0]
        for j in range(2):
            t = [t0, t0 + 100, t0 + 1100, t0 + 1300, t0 + 1600, hw, xcc, len(rows)]
            rows.append(t)
            t0 = t[4] + (700 if xcc == 0 else 900)
    stamps = np.zeros(64 * 8, dtype=np.uint64)
    stamps[: len(rows) * 8] = np.array(rows, dtype=np.uint64).reshape(-1)
    r = bench.stamp_phases(stamps, len(rows))
    assert r["prologue"] == 100 and r["main_loop"] == 1000
    assert r["first_staging"] == 200 and r["rest_of_epilogue"] == 300 and r["total"] == 1600
    assert r["gap_to_next_tile_on_cu"] == 800 and r["cus"] == 2 and r["tiles"] == 4


def test_stamp_phases_separates_cus_by_xcc():
    # the same HW_ID on two XCCs are two CUs: no gap is taken across them
    hw = _hw_id(2, 1, 7)
    rows = [[0, 10, 20, 30, 40, hw, 0, 0], [41, 51, 61, 71, 81, hw, 1, 1]]
    stamps = np.array(rows, dtype=np.uint64).reshape(-1)
    r = bench.stamp_phases(stamps, 2)
    assert r["cus"] == 2 and r["gap_to_next_tile_on_cu"] is None
