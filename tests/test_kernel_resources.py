"""Register budgets of the route kernels, from the compiler's resource report.

The graph-route kernels are latency-bound: their speed on MI355X comes from
routes resident per CU (waves per SIMD) without spills reloaded every step.
These tests compile the hot instantiations for gfx950 with the library's own
flags and `-Rpass-analysis=kernel-resource-usage`, and check the occupancy and
VGPR spill counts each was measured at (C2: exact route 6 waves, 46 ms; the
same kernel with 10 spilled VGPRs took 50.8 ms).  CPU only: hipcc
cross-compiles without a GPU.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "go-fann_amd" / "csrc"

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and
                                not Path("/opt/rocm/bin/hipcc").exists(),
                                reason="hipcc not installed")


def _resources(src: str, out_dir: Path) -> dict:
    """{mangled kernel name: {"vgprs", "occupancy", "vgpr_spill"}} of one source."""
    import build  # go-fann_amd/build.py: the library's own compile flags

    cmd = [build.HIPCC, *build.COMMON, "-x", "hip", *build.DEVICE, "--cuda-device-only",
           "-Rpass-analysis=kernel-resource-usage", "-c", str(CSRC / src),
           "-o", str(out_dir / (Path(src).stem + ".o"))]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    out, cur = {}, None
    for line in res.stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        if cur is None:
            continue
        for key, pat in (("vgprs", r"remark:\s+VGPRs: (\d+)"),
                         ("occupancy", r"remark:\s+Occupancy \[waves/SIMD\]: (\d+)"),
                         ("vgpr_spill", r"remark:\s+VGPRs Spill: (\d+)")):
            m = re.search(pat, line)
            if m:
                cur[key] = int(m.group(1))
    return out


@pytest.fixture(scope="module")
def report(tmp_path_factory):
    d = tmp_path_factory.mktemp("res")
    srcs = ("exact_route.hip", "pq_search_m48.hip", "pq_search_m32.hip", "rabitq_search.hip")
    with ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        return dict(zip(srcs, ex.map(lambda s: _resources(s, d), srcs)))


def _kernels(rep: dict, needle: str) -> dict:
    ks = {k: v for k, v in rep.items() if needle in k}
    assert ks, f"no kernel matching {needle}"
    return ks


def test_exact_route_six_waves_without_step_spills(report):
    # every visited-set placement of the u8 kernels (last template argument
    # 0); the headline one (<2, 0, 0>: spilling LDS visited table) keeps at
    # most the one spilled VGPR it was measured with.  The f32 / f16 kernels
    # (1, 2), the long-row ones (middle argument -1, mangled "n1") included,
    # are built for 4 waves (their LDS allows about that many routes) and
    # spill nothing.
    for name, r in _kernels(report["exact_route.hip"], "exact_route_kernel").items():
        elem = int(re.search(r"ILi\d+ELin?\d+ELi(\d+)EEE", name).group(1))
        if elem == 0:
            assert r["occupancy"] >= 6, (name, r)
            assert r["vgprs"] <= 80, (name, r)
            assert r["vgpr_spill"] <= 1, (name, r)
        else:
            assert r["occupancy"] >= 4, (name, r)
            assert r["vgpr_spill"] == 0, (name, r)


@pytest.mark.parametrize("src,needle", [
    ("pq_search_m48.hip", "PqScorerILi48ELi4EEE"),
    ("pq_search_m32.hip", "PqScorerILi32ELi4EEE"),
    ("rabitq_search.hip", "traversal_kernelINS_12RabitqScorer"),
])
def test_traversal_four_waves_without_spills(report, src, needle):
    for name, r in _kernels(report[src], needle).items():
        assert r["occupancy"] >= 4, (name, r)
        assert r["vgpr_spill"] == 0, (name, r)
