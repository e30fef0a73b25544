"""The committed rocprofv3 traffic summary that bench.py reads stays consistent.

bench.py copies each leg's `traffic` from the `traffic:` lines of
profiles/bench_kernels_traffic.md when its run is the configuration that
summary measured (same leg, kernel, beams and algorithmic bytes).  These
checks recompute every line's bytes from its own FETCH_SIZE / WRITE_SIZE
figures and the summary's copy calibration, so a hand edit of one without
the other fails here, and check the lookup's matching rule.
"""
from __future__ import annotations

import re

import bench

PROFILE = bench.ROOT / "profiles" / bench.TRAFFIC_PROFILE


def _fields(line: str) -> dict:
    return dict(kv.split("=", 1) for kv in (x.strip() for x in line[8:].split(";")) if "=" in kv)


def _lines():
    text = PROFILE.read_text()
    cal = re.search(r"^calibration: neg_fetch_kib=(\d+); neg_write_kib=(\d+)", text, re.M)
    assert cal, "calibration line missing"
    rows = [_fields(l.strip()) for l in text.splitlines() if l.strip().startswith("traffic:")]
    return (int(cal.group(1)), int(cal.group(2))), rows


def test_calibration_is_a_copy_of_one_gib():
    (fk, wk), _ = _lines()
    # a copy of 1 GiB reads 1 GiB and writes 1 GiB: the counters' scale factors
    assert abs((1 << 20) / fk - 2.0) < 0.01
    assert abs((1 << 20) / wk - 1.0) < 0.01


def test_every_traffic_line_matches_its_counters():
    (fk, wk), rows = _lines()
    assert len(rows) >= 10
    ff, wf = round((1 << 20) / fk, 3), round((1 << 20) / wk, 3)
    for f in rows:
        expect = (float(f["fetch_kib"]) * ff + float(f["write_kib"]) * wf) * 1024
        assert abs(float(f["bytes"]) - expect) <= 1e-6 * expect + 1, f
        # counter bytes are of the order of the algorithmic bytes: L2 hits can
        # put them below, re-read lines above, never by orders of magnitude
        alg = float(f["algorithmic"])
        assert 0.3 * alg <= float(f["bytes"]) <= 30 * alg, f


def test_lookup_matches_leg_kernel_beams_and_bytes():
    _, rows = _lines()
    f = rows[0]
    beams = [int(b) for b in f["beams"].split(",")]
    alg = float(f["algorithmic"])
    got = bench.measured_traffic(f["leg"], f["kernel"], beams, alg)
    assert got == float(f["bytes"])
    # a different walk (algorithmic bytes 2% off), beam or leg is not this run
    assert bench.measured_traffic(f["leg"], f["kernel"], beams, alg * 1.02) is None
    assert bench.measured_traffic(f["leg"], f["kernel"], [b + 1 for b in beams], alg) is None
    assert bench.measured_traffic("no such leg", f["kernel"], beams, alg) is None
