"""The committed rocprofv3 summaries that bench.py reads stay consistent.

bench.py copies `roofline.traffic` from the `bytes_per_launch:` line of
profiles/exact_route_c2_traffic.md when its run is the configuration that
summary measured.  These checks recompute that line from the summary's own
per-launch FETCH_SIZE / WRITE_SIZE table and calibration factors, so a hand
edit of one without the other fails here.
"""
from __future__ import annotations

import re

import bench

PROFILE = bench.ROOT / "profiles" / "exact_route_c2_traffic.md"


def _table(text: str):
    fetch, write, calib = [], [], None
    for line in text.splitlines():
        m = re.match(r"\| exact route, launch \d+ \| ([0-9,]+) \| ([0-9,]+) \|", line)
        if m:
            fetch.append(int(m.group(1).replace(",", "")))
            write.append(int(m.group(2).replace(",", "")))
        m = re.match(r"\| neg, 1 GiB in / 1 GiB out \| ([0-9,]+) \| ([0-9,]+) \|", line)
        if m:
            calib = tuple(int(x.replace(",", "")) for x in m.groups())
    return fetch, write, calib


def test_traffic_line_matches_its_table():
    text = PROFILE.read_text()
    fetch, write, calib = _table(text)
    assert len(fetch) == 3 and len(write) == 3 and calib is not None
    # a copy of 1 GiB moves 1 GiB in and 1 GiB out: the counters' scale factors
    f_fac = (1 << 20) / calib[0]
    w_fac = (1 << 20) / calib[1]
    assert abs(f_fac - 2.0) < 0.01 and abs(w_fac - 1.0) < 0.01
    expect = (sum(fetch) / 3 * 2.0 + sum(write) / 3 * 1.0) * 1024
    got = bench.measured_traffic("exact_route_c2_traffic.md", True)
    assert got is not None
    assert abs(got - expect) / expect < 1e-6, (got, expect)


def test_traffic_is_only_copied_for_the_measured_configuration():
    assert bench.measured_traffic("exact_route_c2_traffic.md", False) is None
    assert bench.measured_traffic("no_such_summary.md", True) is None


def test_traffic_is_not_below_the_algorithmic_bytes():
    # 138,300 routes at Q = 80 move 123.9 GB algorithmically; the measured
    # traffic includes every row segment, so it cannot be smaller
    text = PROFILE.read_text()
    m = re.search(r"bench\.py `exact_route_bytes`\): ([0-9,]+) B", text)
    assert m, "algorithmic bytes line missing"
    alg = int(m.group(1).replace(",", ""))
    got = bench.measured_traffic("exact_route_c2_traffic.md", True)
    assert alg <= got <= 2 * alg
