"""The GGUF catalog (runtime/gguf.cpp) under AddressSanitizer + UndefinedBehaviorSanitizer.

Host code only: the parser and its readers are built with g++ together with a small driver
(tests/sanitize/gguf_catalog_main.cpp; no GPU code, no HIP runtime) and run over valid files
and 300 mutated or truncated copies, through io_uring and through positioned reads.  Any
memory error, leak or undefined behaviour aborts the driver with a report; every file must
either open (its directory walked, its small tensors read) or be rejected with a status.
"""
import os
import shutil
import subprocess

import numpy as np
import pytest

from hayai_amd import gguf
from hayai_amd.gguf import write_gguf

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM_INCLUDE = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "include")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if shutil.which("g++") is None or not os.path.isdir(ROCM_INCLUDE):
        pytest.skip("g++ or the ROCm headers are not available")
    out = str(tmp_path_factory.mktemp("asan") / "gguf_catalog_asan")
    cmd = ["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__", "-I" + ROCM_INCLUDE, "-I" + os.path.join(REPO, "include"),
           os.path.join(REPO, "tests", "sanitize", "gguf_catalog_main.cpp"),
           os.path.join(REPO, "hayai_amd", "csrc", "runtime", "gguf.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


def _files(tmp_path):
    base = str(tmp_path / "base.gguf")
    write_gguf(base, [("general.architecture", "llama"), ("n", (gguf.U32, 7)),
                      ("arr", (gguf.ARRAY, (gguf.I32, [1, -2, 3]))), ("s", "abc")],
               [("a.weight", (256, 2), 12, np.arange(288, dtype=np.uint8)),
                ("b.weight", (32, 3), 8, np.arange(102, dtype=np.uint8)),
                ("blk.0.ffn_gate.weight", (256, 4), 12, np.arange(576, dtype=np.uint8)),
                ("blk.0.ffn_up.weight", (256, 4), 12, np.arange(576, dtype=np.uint8)),
                ("blk.0.ffn_down.weight", (256, 4), 12, np.arange(576, dtype=np.uint8))])
    blob = open(base, "rb").read()
    rng = np.random.default_rng(321)
    paths = [base]
    for i in range(300):
        b = bytearray(blob)
        for _ in range(int(rng.integers(1, 5))):
            pos = int(rng.integers(0, len(b)))
            b[pos] = int(rng.integers(0, 256))
        if i % 7 == 0:
            b = b[: int(rng.integers(0, len(b)))]
        q = str(tmp_path / f"m{i}.gguf")
        with open(q, "wb") as f:
            f.write(b)
        paths.append(q)
    return paths


@pytest.mark.parametrize("force_file_io", ["0", "1"])
def test_gguf_catalog_is_clean_under_sanitizers(driver, tmp_path, force_file_io):
    paths = _files(tmp_path)
    env = dict(os.environ, HAYAI_FORCE_FILE_IO=force_file_io,
               ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([driver, *paths], capture_output=True, text=True, env=env, timeout=300)
    report = r.stderr[-4000:]
    assert r.returncode == 0, report
    assert "AddressSanitizer" not in r.stderr and "LeakSanitizer" not in r.stderr, report
    assert "runtime error" not in r.stderr, report
    opened, rejected = (int(v) for v in r.stdout.split()[1::2])
    assert opened >= 1 and opened + rejected == len(paths)
