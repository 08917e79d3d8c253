"""The C-ABI library loads, exports every symbol include/hayai_hip.h declares, and applies
the reference's pre-launch validation (compute.rs:877-949) without touching a device."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import hayai_amd
from hayai_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        for m in re.finditer(r"\b(hh_[a-z0-9_]+)\s*\(", txt):
            names.add(m.group(1))
    return names


def test_library_is_built_in_tree():
    assert os.path.exists(_abi.LIB_PATH), "run python -m hayai_amd.build"


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = names - exported
    assert not missing, missing
    lib = _abi.load()
    for n in names:
        assert getattr(lib, n) is not None
    # the ctypes table covers the whole header (tests call through every entry point)
    assert names == set(_abi.SIGNATURES), names ^ set(_abi.SIGNATURES)


def test_abi_version_and_status_names():
    lib = _abi.load()
    assert lib.hh_abi_version() == 1
    for code, name in _abi.STATUS_NAMES.items():
        assert lib.hh_status_name(code).decode() == name


def test_row_bytes_table():
    # compute.rs:877-907
    assert hayai_amd.row_bytes(hayai_amd.Q4_K, 4096) == 2304
    assert hayai_amd.row_bytes(hayai_amd.Q4_K, 14336) == 8064
    assert hayai_amd.row_bytes(hayai_amd.Q4_0, 576) == 324
    assert hayai_amd.row_bytes(hayai_amd.Q4_0, 1536) == 864
    assert hayai_amd.row_bytes(hayai_amd.IQ2_XXS, 8192) == 2112
    assert hayai_amd.row_bytes(hayai_amd.IQ2_XXS, 28672) == 7392
    assert hayai_amd.row_bytes(hayai_amd.IQ3_XXS, 4096) == 1568
    assert hayai_amd.row_bytes(hayai_amd.F32, 7) == 28
    assert hayai_amd.row_bytes(hayai_amd.F16, 7) == 14


def test_validation_errors():
    with pytest.raises(hayai_amd.HipError) as e:
        hayai_amd.validate_gemv_shape(hayai_amd.Q4_K, 0, 256)
    assert e.value.status_name == "HH_ERR_INVALID" and "empty shape" in str(e.value)
    with pytest.raises(hayai_amd.HipError) as e:
        hayai_amd.validate_gemv_shape(hayai_amd.Q4_K, 4, 300)
    assert "not a valid column count" in str(e.value)
    with pytest.raises(hayai_amd.HipError) as e:
        hayai_amd.validate_gemv_weights(hayai_amd.Q4_K, 4, 256, 575)
    assert "weight buffer 575 B < 576 B" in str(e.value)
    hayai_amd.validate_gemv_weights(hayai_amd.Q4_K, 4, 256, 576)
    # a type with no kernel is a hard error, never a fallback (orchestrator.rs:403-409)
    with pytest.raises(hayai_amd.HipError) as e:
        hayai_amd.validate_gemv_shape(13, 4, 256)  # Q5_K
    assert e.value.status_name == "HH_ERR_KERNEL_MISSING"


def test_validation_matches_oracle():
    import oracle

    rng = np.random.default_rng(0)
    for _ in range(300):
        t = int(rng.choice([0, 1, 2, 8, 12, 14, 16, 18]))
        m = int(rng.integers(0, 5))
        n = int(rng.choice([0, 1, 31, 32, 64, 255, 256, 512, 1000]))
        ok_shape = oracle.validate_shape(t, m, n)
        try:
            hayai_amd.validate_gemv_shape(t, m, n)
            lib_shape = True
        except hayai_amd.HipError:
            lib_shape = False
        assert ok_shape == lib_shape, (t, m, n)
        if n % oracle.BLOCK[t][0] == 0:
            rb = oracle.row_bytes(t, n)
            for ln in (m * rb, max(m * rb - 1, 0)):
                ok = oracle.validate_weights(t, m, n, ln)
                try:
                    hayai_amd.validate_gemv_weights(t, m, n, ln)
                    lib_ok = True
                except hayai_amd.HipError:
                    lib_ok = False
                assert ok == lib_ok, (t, m, n, ln)


def test_no_device_here_is_an_error_not_a_fallback():
    if hayai_amd.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(hayai_amd.HipError) as e:
        hayai_amd.HipEngine(0)
    assert e.value.status_name == "HH_ERR_NO_DEVICE"


def test_null_arguments_rejected():
    lib = _abi.load()
    assert lib.hh_row_bytes(12, 256, None) == 2
    assert lib.hh_device_count(None) == 2
    assert lib.hh_engine_create(0, None) == 2
    assert b"NULL" in lib.hh_last_error()


def test_product_does_not_reference_oracle():
    # the shipped package and sources never import/link the test oracle
    for dirpath, _, files in os.walk(os.path.join(ROOT, "hayai_amd")):
        for f in files:
            if f.endswith((".py", ".cpp", ".h", ".hip")):
                txt = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in txt and "hayai_oracle" not in txt, f
