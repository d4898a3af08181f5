"""bench.py takes each prefill kernel's average duration and HBM traffic per
launch from the committed rocprofv3 summaries under profiles/.  A kernel
renamed in the source (a template argument added, say) would silently drop
out of those readers; these checks fail instead."""
import re

import bench

KERNELS = ("gdn_prep_kernel", "gdn_scan_kernel")


def test_trace_rows_of_both_kernels_parse():
    t = bench.trace_from_profiles()
    assert set(t) == set(KERNELS), t
    for name, us in t.items():
        assert 1.0 < us < 100.0, (name, us)


def test_trace_rows_match_the_summary_table():
    """The parsed averages are the table's rows at the T=1141 HV=32 grids
    (576 prep groups, 256 scan groups)."""
    text = (bench.ROOT / "profiles" / "gdn_prefill_T1141_HV32_kernel_trace.md").read_text()
    rows = {}
    for m in re.finditer(r"^\| (gdn_(?:prep|scan)_kernel)<([^>]*)> \| \d+ \| ([0-9.]+) \|.*\| (\d+)x1 \|",
                         text, flags=re.M):
        rows.setdefault((m.group(1), m.group(2), int(m.group(4))), float(m.group(3)))
    t = bench.trace_from_profiles()
    assert t["gdn_prep_kernel"] == rows[("gdn_prep_kernel", "false,0,false", 576)]
    assert t["gdn_scan_kernel"] == rows[("gdn_scan_kernel", "0,false,false", 256)]


def test_traffic_of_both_kernels_parses():
    for name in KERNELS:
        b = bench.traffic_from_profiles(name)
        assert b is not None, name
        assert 1e7 < b < 1e9, (name, b)
