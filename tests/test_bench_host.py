"""bench.py's host-side bookkeeping (no GPU): the HBM traffic that the bench
line reports is read from the committed rocprofv3 summary, and it is
consistent with the per-kernel rows of that summary."""

import os
import re
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

L3 = "edge_tp_bwd:uvu|0,1,2,3|0,1,2,3|0,1,2,3"


def _row(text, kernel_prefix):
    for line in text.splitlines():
        if line.startswith("| `" + kernel_prefix):
            cells = [c.strip() for c in line.strip("|").split("|")]
            return float(cells[2]), float(cells[3])
    raise AssertionError(f"no row for {kernel_prefix}")


def test_water_traffic_lines_present_and_match_the_table():
    kern = bench.measured_traffic("water12k", L3 + " kernel")
    entry = bench.measured_traffic("water12k", L3)
    fwd = bench.measured_traffic("water12k", L3.replace("bwd", "fwd"))
    assert kern and entry and fwd
    text = open(os.path.join(ROOT, "profiles", "water12k_hbm_traffic.md")).read()
    r, w = _row(text, "void k_uvu_0123_0123_0123_bwd")
    assert abs(kern - (r + w) * 1e9) < 0.02e9
    rs, ws = _row(text, "void k_seg_rowsum")
    # entry point = kernel + sender row sum + the grad_y part sum (stated in the summary)
    gy = float(re.search(r"= ([0-9.]+) GB\)", text).group(1))
    assert abs(entry - kern - (rs + ws + gy) * 1e9) < 0.02e9
    r, w = _row(text, "void k_uvu_0123_0123_0123_fwd")
    assert abs(fwd - (r + w) * 1e9) < 0.02e9
    assert bench.measured_traffic("water12k", "no such entry") is None
