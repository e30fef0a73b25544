"""Shared test setup: import paths, the `gpu` marker, library builds.

CPU tests (-m "not gpu") pin the oracle against the reference's own fixtures,
closed forms and brute force, and check the C-ABI library's exports.  GPU
tests (-m gpu) compare the HIP path with the oracle through the C ABI.
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "go-fann_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libgofann_hip.so)")


def _ensure_oracle():
    lib = ROOT / "oracle" / "libgofann_oracle.so"
    if not lib.exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


_ensure_oracle()


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def hip_lib_path():
    lib = ROOT / "go-fann_amd" / "libgofann_hip.so"
    if not lib.exists():
        from build import build  # go-fann_amd/build.py
        build(verbose=False)
    return lib


@pytest.fixture(scope="session")
def gpu_ctx(hip_lib_path):
    if not _gpu_available():
        pytest.skip("no GPU visible")
    from gofann_amd import _lib
    ctx = _lib.Context(0)
    yield ctx
    ctx.close()


def load_golden(name: str):
    import json
    return json.loads((GOLDEN / name).read_text())
