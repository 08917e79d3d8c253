"""GPU parity of the Q4 LUT GEMV (hayai's 4-bit dictionary format) through the C ABI.

Reference: cpu_lut_matmul_q4 (crates/hayai-cpu/src/matmul.rs:48-82), OpenClEngine::
lut_matmul_q4 (crates/hayai-opencl/src/compute.rs:45-128).  Its own tests: matmul.rs:103-135
(LUT matmul vs the fp32 matmul of the unpacked weights, max_abs_diff < 1e-4; the SmolLM
shape smoke test) and the GPU-vs-CPU check compute.rs:1034-1061 / main.rs:648-696 (< 1e-4).
Float work: the bar is max|y - ref| / max|ref| <= 1e-5 against the oracle's sequential f32
sum, plus the reference's absolute 1e-4 where it states one.
"""
import os

import numpy as np
import pytest

import hayai_amd
import oracle

pytestmark = pytest.mark.gpu

FIX = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_fixtures.npz"))
SAMPLE_LUT = np.array([-0.5, -0.4, -0.3, -0.2, -0.1, 0.0, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9, 1.0],
                      np.float32)
REL_TOL = 1e-5


def rel_err(y, ref):
    y, ref = np.asarray(y, np.float64), np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def dense(m, n, w, lut):
    d = np.empty((m, n), np.float64)
    d[:, 0::2] = lut[(w & 15).reshape(m, n // 2)]
    d[:, 1::2] = lut[(w >> 4).reshape(m, n // 2)]
    return d


def test_reference_matches_fp32(engine):
    # matmul.rs:103-122
    m, n = 32, 64
    w = (np.arange(m * n // 2) % 256).astype(np.uint8)
    x = (np.arange(n) * 0.01).astype(np.float32)
    y = engine.lut_matmul_q4(m, n, w, SAMPLE_LUT, x)
    assert np.max(np.abs(y - dense(m, n, w, SAMPLE_LUT) @ x)) < 1e-4


def test_reference_smollm_shape_smoke(engine):
    # matmul.rs:124-135: 0xAB bytes, x = 1 -> every row = 32 * (lut[11] + lut[10]) = 35.2
    m, n = 96, 64
    y = engine.lut_matmul_q4(m, n, np.full(m * n // 2, 0xAB, np.uint8), SAMPLE_LUT, np.ones(n, np.float32))
    assert np.isfinite(y).all()
    assert np.max(np.abs(y - 35.2)) < 1e-4


def test_golden_fixture(engine):
    m, n = FIX["lut/shape"].tolist()
    y = engine.lut_matmul_q4(m, n, FIX["lut/w"], FIX["lut/lut"], FIX["lut/x"])
    assert rel_err(y, FIX["lut/y"]) <= REL_TOL


@pytest.mark.parametrize("m,n", [(1536, 576), (576, 1536), (4096, 4096), (7, 70), (33, 2), (1, 4098)])
def test_matches_oracle(engine, m, n):
    # 1536x576 is `hayai bench`'s LUT shape (main.rs:601-646); n=70 and n=2 give rows whose
    # byte length is not a multiple of 4 (bytewise path)
    print(f"[case] lut {m}x{n}", flush=True)
    rng = np.random.default_rng(m * 7 + n)
    w = rng.integers(0, 256, m * n // 2, dtype=np.uint8)
    lut = rng.standard_normal(16).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    y = engine.lut_matmul_q4(m, n, w, lut, x)
    assert rel_err(y, oracle.lut_matmul_q4(m, n, w, lut, x)) <= REL_TOL
    assert np.max(np.abs(y - dense(m, n, w, lut) @ x)) < 1e-4 * max(1.0, np.sqrt(n) / 8)


def test_hayai_bench_case(engine):
    # main.rs:601-646: weights 0xAB, x = 1.0 at 1536x576 -> 288 * (lut[11] + lut[10]) per row
    m, n = 1536, 576
    y = engine.lut_matmul_q4(m, n, np.full(m * n // 2, 0xAB, np.uint8), SAMPLE_LUT, np.ones(n, np.float32))
    assert np.max(np.abs(y - 288 * 1.1)) < 1e-3


def test_device_buffers_and_offsets(engine):
    m, n = 300, 1000
    rng = np.random.default_rng(3)
    w = rng.integers(0, 256, m * n // 2, dtype=np.uint8)
    lut = rng.standard_normal(16).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    wb = engine.alloc(m * n // 2 + 8)
    wb.write(w, 8)  # rows start 4-aligned but the tensor at an offset
    lb = engine.alloc(16 * 4 + 4)
    lb.write(lut, 4)
    xb = engine.alloc(4 * n + 4)
    xb.write(x, 4)  # x not 16-byte aligned: scalar x loads
    yb = engine.alloc(4 * m + 12)
    engine.lut_gemv_dev(m, n, wb, 8, lb, 4, xb, 4, yb, 12)
    y = yb.read(np.float32, m, 12)
    assert rel_err(y, oracle.lut_matmul_q4(m, n, w, lut, x)) <= REL_TOL
    # deterministic: the same call twice is bit-identical
    engine.lut_gemv_dev(m, n, wb, 8, lb, 4, xb, 4, yb, 12)
    assert np.array_equal(yb.read(np.float32, m, 12).view(np.uint32), y.view(np.uint32))


def test_validation(engine):
    # the reference's assertions (compute.rs:54-58) as status codes
    with pytest.raises(hayai_amd.HipError) as e:
        engine.lut_matmul_q4(4, 5, np.zeros(10, np.uint8), SAMPLE_LUT, np.zeros(5, np.float32))
    assert e.value.status_name == "HH_ERR_INVALID"
    with pytest.raises(hayai_amd.HipError) as e:
        engine.lut_matmul_q4(4, 8, np.zeros(15, np.uint8), SAMPLE_LUT, np.zeros(8, np.float32))
    assert e.value.status_name == "HH_ERR_INVALID"
    with pytest.raises(hayai_amd.HipError):
        engine.lut_matmul_q4(0, 8, np.zeros(0, np.uint8), SAMPLE_LUT, np.zeros(8, np.float32))
