"""Shared pytest setup.

Markers: ``gpu`` tests need an MI355X (gfx950) and call the HIP library through its C ABI;
everything else runs on the CPU.  GPU tests skip only when no GPU exists at all; a GPU
that is present but fails engine bring-up is a failure (crates/hayai-opencl/src/
compute.rs:1020-1032, init_engine_or_skip).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def engine():
    import hayai_amd

    if hayai_amd.device_count() == 0:
        pytest.skip("no GPU device")
    eng = hayai_amd.HipEngine(0)
    print(f"[engine] {eng.device_name} {eng.arch} CUs={eng.device_info.compute_units}", flush=True)
    yield eng
    eng.close()
