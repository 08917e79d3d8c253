"""Regenerate the committed golden fixtures under tests/golden/.

Run from the repository root:  python tests/golden/make_golden.py

What it writes (data only; no reference source text is copied):
  tables.json       sha256 of the IQ2_XXS / IQ3_XXS grids and the sign table exactly as
                    the reference spells them (parsed from the reference's Rust source and
                    cross-checked against its OpenCL copy when /root/reference is present),
                    plus the 128 sign-table bytes.  The oracle and the HIP library are
                    checked against these.
  ref_fixtures.npz  the inputs of the reference's own GPU-vs-CPU parity tests
                    (crates/hayai-opencl/src/compute.rs:1034-1670, including the Q6_K and Q8_0
                    tests at :1146-1190 and :1235-1272; their byte/input formulas
                    reproduced), with two expected outputs per case: the oracle's fp32 result
                    and an fp64 dot product of the oracle's bit-exact dequant.
"""
from __future__ import annotations

import hashlib
import json
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

REF = "/root/reference/crates"


def _parse_rust_array(path: str, name: str, count: int) -> list[int]:
    txt = open(path).read()
    i = txt.index(f"pub static {name}")
    body = txt[txt.index("= [", i) + 3: txt.index("];", i)]
    vals = [int(v, 16) if v.startswith("0x") else int(v) for v in re.findall(r"0x[0-9a-fA-F]+|\b\d+\b", body)]
    assert len(vals) == count, (name, len(vals))
    return vals


def _parse_cl_array(path: str, name: str, count: int) -> list[int]:
    txt = open(path).read()
    i = txt.index(name)
    body = txt[txt.index("{", i) + 1: txt.index("};", i)]
    vals = [int(v, 16) if v.startswith("0x") else int(v) for v in re.findall(r"0x[0-9a-fA-F]+|\b\d+\b", body)]
    assert len(vals) == count, (name, len(vals))
    return vals


def tables() -> dict:
    iq2 = _parse_rust_array(f"{REF}/hayai-model/src/iq2.rs", "IQ2XXS_GRID", 256)
    iq3 = _parse_rust_array(f"{REF}/hayai-model/src/iq3.rs", "IQ3XXS_GRID", 256)
    ks = _parse_rust_array(f"{REF}/hayai-model/src/iq2.rs", "KSIGNS_IQ2XS", 128)
    cl = f"{REF}/hayai-kernels/kernels/ggml_gemv_q4.cl"
    assert iq2 == _parse_cl_array(cl, "__constant ulong hayai_iq2xxs_grid", 256)
    assert iq3 == _parse_cl_array(cl, "__constant uint hayai_iq3xxs_grid", 256)
    assert ks == _parse_cl_array(cl, "__constant uchar hayai_ksigns_iq2xs", 128)
    assert ks == _parse_rust_array(f"{REF}/hayai-model/src/iq3.rs", "KSIGNS_IQ2XS", 128)
    return {
        "source": "crates/hayai-model/src/iq2.rs:18-95, iq3.rs:29-63 (equal to the OpenCL copies)",
        "iq2xxs_grid_sha256": hashlib.sha256(np.array(iq2, dtype="<u8").tobytes()).hexdigest(),
        "iq3xxs_grid_sha256": hashlib.sha256(np.array(iq3, dtype="<u4").tobytes()).hexdigest(),
        "ksigns_sha256": hashlib.sha256(bytes(ks)).hexdigest(),
        "ksigns": ks,
    }


# ------------------------------------------------------------ reference test inputs ----

def q4_0_fixture():
    """compute.rs:1063-1098: d=0x2E66, qs=(row+b+j)%256, x=i*0.01-0.4, m=64, n=128."""
    m, n = 64, 128
    nb = n // 32
    w = np.zeros(m * nb * 18, np.uint8)
    for row in range(m):
        for b in range(nb):
            base = (row * nb + b) * 18
            w[base], w[base + 1] = 0x66, 0x2E
            for j in range(16):
                w[base + 2 + j] = (row + b + j) % 256
    x = (np.arange(n, dtype=np.float32) * np.float32(0.01) - np.float32(0.4)).astype(np.float32)
    return oracle.Q4_0, m, n, w, x


def q4_k_fixture():
    """compute.rs:1100-1143: d=1.0, dmin=0, scales=1, q=(row+q)%256, x=i*0.005-0.2."""
    m, n = 32, 256
    w = np.zeros(m * 144, np.uint8)
    for row in range(m):
        base = row * 144
        w[base:base + 4] = [0x00, 0x3C, 0x00, 0x00]
        w[base + 4:base + 16] = 1
        for q in range(16, 144):
            w[base + q] = (row + q) % 256
    x = (np.arange(n, dtype=np.float32) * np.float32(0.005) - np.float32(0.2)).astype(np.float32)
    return oracle.Q4_K, m, n, w, x


def q6_k_fixture():
    """compute.rs:1146-1190: ql=(row+q)%256, qh=(row*3+q)%256 (q = byte index), scales=1,
    d=1.0, x=i*0.005-0.2, m=32, n=256."""
    m, n = 32, 256
    w = np.zeros(m * 210, np.uint8)
    for row in range(m):
        base = row * 210
        for q in range(128):
            w[base + q] = (row + q) % 256
        for q in range(128, 192):
            w[base + q] = (row * 3 + q) % 256
        w[base + 192:base + 208] = 1
        w[base + 208], w[base + 209] = 0x00, 0x3C
    x = (np.arange(n, dtype=np.float32) * np.float32(0.005) - np.float32(0.2)).astype(np.float32)
    return oracle.Q6_K, m, n, w, x


def q8_0_fixture():
    """compute.rs:1235-1272: d=0x2E66, qs=(row+b+j)%256, x=i*0.01-0.4, m=32, n=256."""
    m, n = 32, 256
    nb = n // 32
    w = np.zeros(m * nb * 34, np.uint8)
    for row in range(m):
        for b in range(nb):
            base = (row * nb + b) * 34
            w[base], w[base + 1] = 0x66, 0x2E
            for j in range(32):
                w[base + 2 + j] = (row + b + j) % 256
    x = (np.arange(n, dtype=np.float32) * np.float32(0.01) - np.float32(0.4)).astype(np.float32)
    return oracle.Q8_0, m, n, w, x


def parity_fixture(t):
    """compute.rs:1370-1394 gemv_parity: bytes (i*131+17)&0x1F, x=i*0.003-0.2, m=32, n=256."""
    m, n = 32, 256
    rb = oracle.row_bytes(t, n)
    i = np.arange(m * rb, dtype=np.int64)
    w = ((i * 131 + 17) & 0x1F).astype(np.uint8)
    x = (np.arange(n, dtype=np.float32) * np.float32(0.003) - np.float32(0.2)).astype(np.float32)
    return t, m, n, w, x


def f16_fixture():
    """compute.rs:1524-1545: f16 bytes (i*131+17)&0x1F, m=16, n=64, x=i*0.01-0.3."""
    m, n = 16, 64
    i = np.arange(m * n * 2, dtype=np.int64)
    w = ((i * 131 + 17) & 0x1F).astype(np.uint8)
    x = (np.arange(n, dtype=np.float32) * np.float32(0.01) - np.float32(0.3)).astype(np.float32)
    return oracle.F16, m, n, w, x


def batched_fixture():
    """compute.rs:1648-1670: Q4_K m=32 n=256 B=3, bytes (i*131+17)&0x1F, X=i*0.003-0.2."""
    m, n, b = 32, 256, 3
    i = np.arange(m * 144, dtype=np.int64)
    w = ((i * 131 + 17) & 0x1F).astype(np.uint8)
    X = (np.arange(b * n, dtype=np.float32) * np.float32(0.003) - np.float32(0.2)).astype(np.float32)
    return oracle.Q4_K, m, n, w, X.reshape(b, n)


def lut_fixture():
    """compute.rs:1034-1061: m=64 n=128, weights (i*17)%256, x=i*0.01-0.5, sample LUT."""
    m, n = 64, 128
    lut = np.array([-0.5, -0.4, -0.3, -0.2, -0.1, 0.0, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9, 1.0],
                   np.float32)
    w = ((np.arange(m * n // 2) * 17) % 256).astype(np.uint8)
    x = (np.arange(n, dtype=np.float32) * np.float32(0.01) - np.float32(0.5)).astype(np.float32)
    return m, n, w, lut, x


def main():
    os.makedirs(HERE, exist_ok=True)
    if os.path.isdir(REF):
        with open(os.path.join(HERE, "tables.json"), "w") as f:
            json.dump(tables(), f, indent=1)
    oracle.build()
    out = {}
    cases = {
        "q4_0": q4_0_fixture(),
        "q4_k": q4_k_fixture(),
        "parity_q4_0": parity_fixture(oracle.Q4_0),
        "parity_q4_k": parity_fixture(oracle.Q4_K),
        "parity_iq2_xxs": parity_fixture(oracle.IQ2_XXS),
        "parity_iq3_xxs": parity_fixture(oracle.IQ3_XXS),
        "f16": f16_fixture(),
        "q6_k": q6_k_fixture(),
        "q8_0": q8_0_fixture(),
    }
    for name, (t, m, n, w, x) in cases.items():
        out[f"{name}/type"] = np.array([t, m, n], np.int64)
        out[f"{name}/w"] = w
        out[f"{name}/x"] = x
        out[f"{name}/y"] = oracle.gemv(t, m, n, w, x)
        out[f"{name}/y64"] = oracle.gemv_f64(t, m, n, w, x.astype(np.float64))
    t, m, n, w, X = batched_fixture()
    out["batched_q4_k/type"] = np.array([t, m, n], np.int64)
    out["batched_q4_k/w"] = w
    out["batched_q4_k/x"] = X
    out["batched_q4_k/y"] = oracle.gemv_batched(t, m, n, w, X)
    m, n, w, lut, x = lut_fixture()
    out["lut/shape"] = np.array([m, n], np.int64)
    out["lut/w"] = w
    out["lut/lut"] = lut
    out["lut/x"] = x
    out["lut/y"] = oracle.lut_matmul_q4(m, n, w, lut, x)
    np.savez_compressed(os.path.join(HERE, "ref_fixtures.npz"), **out)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
