"""Pin the CPU oracle (oracle/hayai_oracle.c) before trusting it as the parity checker.

Each check is chosen so a plausible transcription mistake (wrong nibble half, wrong scale
byte, dropped min term, sign flipped, transposed operand) fails it; none re-types the
oracle's own formula.  Sources of truth: IEEE conversions in numpy, the reference's own
known-answer tests and fixtures, inverse maps taken from other reference functions (the
Q4_K quantizer's packing), closed-form special cases, fp64 brute force, linearity.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_f16_exhaustive_matches_ieee():
    # gguf.rs:521-545 vs numpy's IEEE binary16 -> binary32 conversion, all 65536 codes.
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()
    # payload kept, sign kept, no quieting (gguf.rs:539-540)
    gb = got[nan].view(np.uint32)
    assert np.array_equal((gb >> 13) & 0x3FF, codes[nan].astype(np.uint32) & 0x3FF)
    assert oracle.f16_to_f32(np.array([0x3C00], np.uint16))[0] == 1.0  # gguf.rs:835-839


def test_f32_to_f16_ref_roundtrip():
    # q4k.rs:307-317 (f16_roundtrip)
    for v in [0.0, 1.0, -1.0, 0.5, 123.45, 0.0001, -9876.5, 1.2345]:
        back = oracle.f16_to_f32(np.array([oracle.f32_to_f16_ref(v)], np.uint16))[0]
        assert abs(v - back) < 0.01 * max(abs(v), 1e-3)


def _blocks(n_blocks, bb, rng):
    return rng.integers(0, 256, n_blocks * bb, dtype=np.uint8)


def test_q4_0_closed_form_d_0x2e66():
    # compute.rs:1063-1098 fixture scale: d = 0x2E66 = 0.0999755859375 exactly
    rng = np.random.default_rng(1)
    w = _blocks(8, 18, rng)
    w.reshape(8, 18)[:, 0:2] = [0x66, 0x2E]
    y = oracle.dequant(oracle.Q4_0, w, 256)
    qs = w.reshape(8, 18)[:, 2:]
    q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.int64) - 8  # j, j+16
    assert np.array_equal(y, (q.reshape(-1) * 0.0999755859375).astype(np.float32))
    w.reshape(8, 18)[:, 0:2] = [0x00, 0x3C]  # d = 1 -> integers
    assert np.array_equal(oracle.dequant(oracle.Q4_0, w, 256), q.reshape(-1).astype(np.float32))


def test_q4_0_tail_block():
    # gguf.rs:363-368: n not a multiple of 32 writes only the first n values
    rng = np.random.default_rng(2)
    w = _blocks(2, 18, rng)
    full = oracle.dequant(oracle.Q4_0, w, 64)
    assert np.array_equal(oracle.dequant(oracle.Q4_0, w, 40), full[:40])


def test_q4_k_reference_fixture_gives_nibbles():
    # compute.rs:1108-1127: d=1, dmin=0, scales=1 -> w = nibble, low nibble of qs[32g+l]
    # at 64g+l and high nibble at 64g+32+l (q4k.rs:188-198)
    rng = np.random.default_rng(3)
    w = _blocks(4, 144, rng).reshape(4, 144)
    w[:, 0:4] = [0x00, 0x3C, 0x00, 0x00]
    w[:, 4:16] = 1
    y = oracle.dequant(oracle.Q4_K, w.reshape(-1), 1024).reshape(4, 4, 64)
    qs = w[:, 16:].reshape(4, 4, 32)
    assert np.array_equal(y[:, :, :32], (qs & 15).astype(np.float32))
    assert np.array_equal(y[:, :, 32:], (qs >> 4).astype(np.float32))


def _pack_scales(sc, m):
    """Scale packing of the reference quantizer, q4k.rs:140-152 (independent of the
    unpack get_scale_min_k4 under test)."""
    sp = [0] * 12
    for j in range(8):
        if j < 4:
            sp[j] = sc[j]
            sp[j + 4] = m[j]
        else:
            sp[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            sp[j - 4] |= (sc[j] >> 4) << 6
            sp[j] |= (m[j] >> 4) << 6
    return np.array(sp, np.uint8)


def test_q4_k_scale_unpack_inverts_reference_packing():
    rng = np.random.default_rng(4)
    for trial in range(400):
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        if trial < 64:  # sweep every value through every slot
            sc = [(trial + 7 * j) % 64 for j in range(8)]
            m = [(63 - trial + 3 * j) % 64 for j in range(8)]
        s = _pack_scales(sc, m)
        for j in range(8):
            assert oracle.get_scale_min_k4(j, s) == (sc[j], m[j])


def test_q4_k_dequant_uses_scale_and_min_per_subblock():
    # Exact special case: d=1, dmin=1 -> w = sc*q - m for the (sc, m) packed into slot j.
    rng = np.random.default_rng(5)
    for _ in range(20):
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        blk = np.zeros(144, np.uint8)
        blk[0:4] = [0x00, 0x3C, 0x00, 0x3C]
        blk[4:16] = _pack_scales(sc, m)
        blk[16:] = rng.integers(0, 256, 128, dtype=np.uint8)
        y = oracle.dequant(oracle.Q4_K, blk, 256)
        qs = blk[16:].reshape(4, 32).astype(np.int64)
        for g in range(4):
            lo = sc[2 * g] * (qs[g] & 15) - m[2 * g]
            hi = sc[2 * g + 1] * (qs[g] >> 4) - m[2 * g + 1]
            assert np.array_equal(y[64 * g:64 * g + 32], lo.astype(np.float32))
            assert np.array_equal(y[64 * g + 32:64 * g + 64], hi.astype(np.float32))


def test_q4_k_quantize_roundtrip_reference_test():
    # q4k.rs:319-350 (q4k_quantize_roundtrip_error_small), same input formula
    x = np.zeros(1024, np.float32)
    for i in range(1024):
        b, j = divmod(i, 256)
        if b == 0:
            x[i] = (j - 128.0) * 0.01
        elif b == 1:
            x[i] = (j % 17) * 0.5 - 4.0
        elif b == 2:
            x[i] = np.float32(np.sin(np.float32(j))) * 3.0
        else:
            x[i] = 1.0 if j % 2 == 0 else -1.0
    back = oracle.dequant(oracle.Q4_K, oracle.quantize_q4_k(x), 1024)
    rel = np.max(np.abs(x - back)) / max(x.max() - min(x.min(), 0.0), 1e-6)
    assert rel < 0.2, rel


def test_q4_k_quantize_roundtrip_error_bound():
    # Stronger: per element |x - deq| <= d1/2 + rounding of the f16 scales, per sub-block.
    rng = np.random.default_rng(6)
    x = rng.normal(size=4096).astype(np.float32)
    back = oracle.dequant(oracle.Q4_K, oracle.quantize_q4_k(x), 4096)
    sub = x.reshape(-1, 32)
    step = (sub.max(1) - sub.min(1)) / 15.0
    err = np.abs(x - back).reshape(-1, 32).max(1)
    assert np.all(err <= step * 0.75 + 0.02), (err / step).max()


def test_tables_match_reference():
    t = json.load(open(os.path.join(GOLDEN, "tables.json")))
    g2, g3, ks = oracle.iq2xxs_grid(), oracle.iq3xxs_grid(), oracle.ksigns()
    assert hashlib.sha256(g2.astype("<u8").tobytes()).hexdigest() == t["iq2xxs_grid_sha256"]
    assert hashlib.sha256(g3.astype("<u4").tobytes()).hexdigest() == t["iq3xxs_grid_sha256"]
    assert ks.tolist() == t["ksigns"]
    assert hashlib.sha256(ks.tobytes()).hexdigest() == t["ksigns_sha256"]
    b2 = g2.view(np.uint8)
    assert set(np.unique(b2).tolist()) <= {8, 25, 43}
    assert set(np.unique(g3.view(np.uint8)).tolist()) <= {4, 12, 20, 28, 36, 44, 52, 62}
    # every sign pattern has an even number of minus signs
    assert all(bin(v).count("1") % 2 == 0 for v in ks.tolist())


def _iq_expected(t, blk, grid, ks, scale):
    """Closed form for d = 1 and scale nibble 0: w = +-scale * grid (iq2.rs:504-523,
    iq3.rs:147-173), assembled from the tables and byte map of Appendix A."""
    out = np.zeros(256, np.float64)
    for ib in range(8):
        if t == oracle.IQ2_XXS:
            aux0 = int.from_bytes(blk[2 + 8 * ib:6 + 8 * ib].tobytes(), "little")
            aux1 = int.from_bytes(blk[6 + 8 * ib:10 + 8 * ib].tobytes(), "little")
            for l in range(4):
                g = int(grid[(aux0 >> (8 * l)) & 255])
                s = ks[(aux1 >> (7 * l)) & 127]
                for j in range(8):
                    out[32 * ib + 8 * l + j] = scale * ((g >> (8 * j)) & 255) * (-1 if (s >> j) & 1 else 1)
        else:
            aux = int.from_bytes(blk[66 + 4 * ib:70 + 4 * ib].tobytes(), "little")
            for l in range(4):
                s = ks[(aux >> (7 * l)) & 127]
                g1 = int(grid[blk[2 + 8 * ib + 2 * l]])
                g2 = int(grid[blk[2 + 8 * ib + 2 * l + 1]])
                for j in range(4):
                    out[32 * ib + 8 * l + j] = scale * ((g1 >> (8 * j)) & 255) * (-1 if (s >> j) & 1 else 1)
                    out[32 * ib + 8 * l + 4 + j] = scale * ((g2 >> (8 * j)) & 255) * (-1 if (s >> (j + 4)) & 1 else 1)
    return out.astype(np.float32)


@pytest.mark.parametrize("t,bb,scale", [(oracle.IQ2_XXS, 66, 0.125), (oracle.IQ3_XXS, 98, 0.25)])
def test_iq_closed_form(t, bb, scale):
    t_ = json.load(open(os.path.join(GOLDEN, "tables.json")))
    ks = t_["ksigns"]
    grid = oracle.iq2xxs_grid() if t == oracle.IQ2_XXS else oracle.iq3xxs_grid()
    rng = np.random.default_rng(7)
    for _ in range(10):
        blk = rng.integers(0, 256, bb, dtype=np.uint8)
        blk[0:2] = [0x00, 0x3C]
        if t == oracle.IQ2_XXS:
            for ib in range(8):
                blk[9 + 8 * ib] &= 0x0F  # scale nibble (aux1 >> 28) = 0
        else:
            for ib in range(8):
                blk[69 + 4 * ib] &= 0x0F
        y = oracle.dequant(t, blk, 256)
        assert np.array_equal(y, _iq_expected(t, blk, grid, ks, scale))


@pytest.mark.parametrize("t,bb,scale", [(oracle.IQ2_XXS, 66, 0.25), (oracle.IQ3_XXS, 98, 0.5)])
def test_iq_scale_nibble(t, bb, scale):
    # db = d*(0.5+s)*k: with d=1, every scale nibble s gives an exact multiple
    rng = np.random.default_rng(8)
    blk = rng.integers(0, 256, bb, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    base = blk.copy()
    for ib in range(8):
        base[(9 + 8 * ib) if t == oracle.IQ2_XXS else (69 + 4 * ib)] &= 0x0F
    y0 = oracle.dequant(t, base, 256).reshape(8, 32)
    y = oracle.dequant(t, blk, 256).reshape(8, 32)
    for ib in range(8):
        s = (blk[(9 + 8 * ib) if t == oracle.IQ2_XXS else (69 + 4 * ib)] >> 4)
        assert np.array_equal(y[ib], (y0[ib] * np.float32(0.5 + s) * np.float32(2.0)).astype(np.float32))


def test_q8_0_closed_form_d_0x2e66():
    # compute.rs:1235-1272 fixture scale d = 0x2E66; gguf.rs:401-420: value = (i8 q) * d
    rng = np.random.default_rng(21)
    w = _blocks(8, 34, rng)
    w.reshape(8, 34)[:, 0:2] = [0x66, 0x2E]
    q = w.reshape(8, 34)[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(oracle.dequant(oracle.Q8_0, w, 256), (q * np.float32(0.0999755859375)).reshape(-1))
    # a tail block: n not a multiple of 32 writes only the first n values (gguf.rs:412-416)
    assert np.array_equal(oracle.dequant(oracle.Q8_0, w, 40), oracle.dequant(oracle.Q8_0, w, 64)[:40])


def _q6_k_encode(codes, scales, d_bits):
    """Pack per-element 6-bit codes (256 per block), 16 i8 scales and an f16 d into Q6_K
    blocks, walking the layout element by element: element e = 128h + 32r + l takes the low
    (r = 0, 1) or high (r = 2, 3) nibble of ql[64h + l + 32(r & 1)] and bits 2r, 2r+1 of
    qh[32h + l] (q6k.rs:31-55 read in the packing direction)."""
    nb = codes.shape[0]
    out = np.zeros((nb, 210), np.uint8)
    for b in range(nb):
        for e in range(256):
            h, r, l = e // 128, (e % 128) // 32, e % 32
            c = int(codes[b, e])
            qi = 64 * h + l + 32 * (r & 1)
            out[b, qi] |= (c & 15) << (4 if r >= 2 else 0)
            out[b, 128 + 32 * h + l] |= (c >> 4) << (2 * r)
        out[b, 192:208] = scales[b].astype(np.int8).view(np.uint8)
        out[b, 208], out[b, 209] = d_bits & 0xFF, d_bits >> 8
    return out.reshape(-1)


def test_q6_k_codes_round_trip():
    # scales = 1, d = 1: every element must come back as its 6-bit code - 32
    rng = np.random.default_rng(22)
    codes = rng.integers(0, 64, (4, 256))
    w = _q6_k_encode(codes, np.ones((4, 16), np.int64), 0x3C00)
    assert np.array_equal(oracle.dequant(oracle.Q6_K, w, 1024), (codes - 32).reshape(-1).astype(np.float32))


def test_q6_k_scale_per_16_columns():
    # code 33 (q = 1) everywhere, scales[k] = k + 1 (k = 0..15) and one negative: element
    # e = 128h + 32r + l uses scales[8h + l/16 + 2r] (q6k.rs:36-48), d = 2 doubles it
    codes = np.full((1, 256), 33)
    sc = np.arange(1, 17)[None, :].copy()
    sc[0, 5] = -7
    w = _q6_k_encode(codes, sc, 0x4000)
    e = np.arange(256)
    idx = 8 * (e // 128) + (e % 32) // 16 + 2 * ((e % 128) // 32)
    assert np.array_equal(oracle.dequant(oracle.Q6_K, w, 256), (2.0 * sc[0, idx]).astype(np.float32))


def test_q6_k_reference_fixture_is_code_minus_32():
    # compute.rs:1146-1190 bytes (scales 1, d 1): values are integers in [-32, 31], each
    # equal to what the element-wise packing of those codes gives back
    w = FIX["q6_k/w"]
    y = oracle.dequant(oracle.Q6_K, w, 32 * 256).reshape(32, 256)
    assert np.array_equal(y, np.round(y)) and y.min() >= -32 and y.max() <= 31
    codes = (y + 32).astype(np.int64)
    blk = w.reshape(32, 210)
    again = _q6_k_encode(codes, np.ones((32, 16), np.int64), 0x3C00).reshape(32, 210)
    assert np.array_equal(again[:, :192], blk[:, :192])


FIX = np.load(os.path.join(GOLDEN, "ref_fixtures.npz"))
CASES = ["q4_0", "q4_k", "parity_q4_0", "parity_q4_k", "parity_iq2_xxs", "parity_iq3_xxs", "f16", "q6_k", "q8_0"]


@pytest.mark.parametrize("name", CASES)
def test_gemv_reference_fixtures(name):
    t, m, n = FIX[f"{name}/type"].tolist()
    w, x = FIX[f"{name}/w"], FIX[f"{name}/x"]
    y = oracle.gemv(t, m, n, w, x)
    assert np.array_equal(y, FIX[f"{name}/y"])  # regression pin of the oracle itself
    y64 = oracle.gemv_f64(t, m, n, w, x.astype(np.float64))
    assert np.allclose(y64, FIX[f"{name}/y64"], rtol=0, atol=0)
    # fp32 accumulation bound: |y - y64| <= n * eps * sum|w x|
    wd = oracle.dequant(t, w, m * n).reshape(m, n).astype(np.float64)
    bound = n * 2.0 ** -23 * (np.abs(wd) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(y - y64) <= bound)


@pytest.mark.parametrize("t", [oracle.Q4_0, oracle.Q4_K, oracle.IQ2_XXS, oracle.IQ3_XXS, oracle.Q8_0, oracle.Q6_K,
                               oracle.F16, oracle.F32])
def test_gemv_fp64_bound_and_linearity(t):
    import hayai_amd.synth as synth

    rng = np.random.default_rng(9)
    m, n = 24, 512
    if t == oracle.F32:
        w = rng.normal(size=m * n).astype(np.float32).view(np.uint8)
    elif t == oracle.F16:
        w = rng.normal(size=m * n).astype(np.float16).view(np.uint8)
    else:
        w = synth.matrix(t, m, n, 1234 + t)
    x1 = rng.normal(size=n).astype(np.float32)
    x2 = rng.normal(size=n).astype(np.float32)
    wd = oracle.dequant(t, w, m * n).reshape(m, n).astype(np.float64)
    y64 = oracle.gemv_f64(t, m, n, w, x1.astype(np.float64))
    assert np.allclose(y64, wd @ x1.astype(np.float64), rtol=1e-12, atol=1e-12)
    y1 = oracle.gemv(t, m, n, w, x1)
    bound = n * 2.0 ** -23 * (np.abs(wd) @ np.abs(x1.astype(np.float64)))
    assert np.all(np.abs(y1 - y64) <= bound)
    # linearity in x (the GEMV is linear; fp32 rounding only)
    a, b = np.float32(0.75), np.float32(-1.5)
    y12 = oracle.gemv(t, m, n, w, (a * x1 + b * x2).astype(np.float32))
    y2 = oracle.gemv(t, m, n, w, x2)
    scale = np.abs(wd) @ (np.abs(x1) + np.abs(x2)).astype(np.float64)
    assert np.all(np.abs(y12 - (a * y1 + b * y2)) <= 4 * n * 2.0 ** -23 * scale)


def test_gemv_batched_matches_per_token():
    t, m, n = FIX["batched_q4_k/type"].tolist()
    w, X = FIX["batched_q4_k/w"], FIX["batched_q4_k/x"]
    Y = oracle.gemv_batched(t, m, n, w, X)
    assert np.array_equal(Y, FIX["batched_q4_k/y"])
    for b in range(X.shape[0]):
        assert np.array_equal(Y[b], oracle.gemv(t, m, n, w, X[b]))


def test_lut_matmul_reference_tests():
    # matmul.rs:103-122: LUT matmul vs fp32 matmul of the unpacked weights, < 1e-4
    lut = np.array([-0.5, -0.4, -0.3, -0.2, -0.1, 0.0, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9, 1.0], np.float32)
    m, n = 32, 64
    w = (np.arange(m * n // 2) % 256).astype(np.uint8)
    x = (np.arange(n, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    dense = np.empty((m, n), np.float32)
    dense[:, 0::2] = lut[(w & 15).reshape(m, n // 2)]
    dense[:, 1::2] = lut[(w >> 4).reshape(m, n // 2)]
    y = oracle.lut_matmul_q4(m, n, w, lut, x)
    assert np.max(np.abs(y - dense.astype(np.float64) @ x.astype(np.float64))) < 1e-4
    # main.rs:648-696 (hayai validate): m=128 n=256, weights (i*31)%256, x=i*0.01-0.25
    m, n = 128, 256
    w = ((np.arange(m * n // 2) * 31) % 256).astype(np.uint8)
    x = (np.arange(n, dtype=np.float32) * np.float32(0.01) - np.float32(0.25)).astype(np.float32)
    dense = np.empty((m, n), np.float64)
    dense[:, 0::2] = lut[(w & 15).reshape(m, n // 2)]
    dense[:, 1::2] = lut[(w >> 4).reshape(m, n // 2)]
    assert np.max(np.abs(oracle.lut_matmul_q4(m, n, w, lut, x) - dense @ x)) < 1e-4
    f = FIX
    m, n = f["lut/shape"].tolist()
    assert np.array_equal(oracle.lut_matmul_q4(m, n, f["lut/w"], f["lut/lut"], f["lut/x"]), f["lut/y"])


def test_swiglu_closed_form():
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 3.5, -100.0], np.float32)
    u = np.array([2.0, 1.0, 1.0, 0.5, 3.0, -2.0, 1.0], np.float32)
    h = oracle.swiglu(g, u)
    ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert np.allclose(h, ref, rtol=2e-7, atol=1e-30)
    assert h[0] == 0.0
    hg = oracle.gelu_tanh(g, u)
    x = g.astype(np.float64)
    ref = 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3))) * u
    assert np.allclose(hg, ref, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------- routing (moe_infer.rs:1039-1121)

def test_route_softmax_topk_uses_full_softmax():
    s = np.array([0.1, 0.9, 0.3, 0.7, 0.2], np.float32)
    top, w = oracle.route_experts(s, 2)
    assert top == [1, 3]
    ex = np.exp(s - 0.9)
    assert abs(w[0] - ex[1] / ex.sum()) < 1e-5 and abs(w[1] - ex[3] / ex.sum()) < 1e-5
    assert w.sum() < 1.0


def test_route_norm_topk_prob():
    s = np.array([0.1, 0.9, 0.3, 0.7, 0.2], np.float32)
    _, w = oracle.route_experts(s, 2, norm_topk_prob=True)
    assert abs(w.sum() - 1.0) < 1e-5


def test_route_correction_bias_selects_but_weights_raw():
    s = np.array([1.0, 0.5, 0.0, -1.0], np.float32)
    top, w = oracle.route_experts(s, 1, bias=np.array([0, 10, 0, 0], np.float32))
    assert top == [1]
    ex = np.exp(s)
    assert abs(w[0] - ex[1] / ex.sum()) < 1e-5


def test_route_grouped():
    s = np.array([0.6, 0.5, 0.9, 0.1], np.float32)
    top, _ = oracle.route_experts(s, 1, n_group=2, topk_group=1, gating=1)
    assert top == [0]


def test_route_sigmoid_and_scaling():
    s = np.array([0.0, 1.0, -1.0], np.float32)
    top, w = oracle.route_experts(s, 2, gating=1, routed_scaling_factor=2.0)
    assert top == [1, 0]
    assert abs(w[0] - 2 * 0.7310586) < 1e-4 and abs(w[1] - 1.0) < 1e-4


def test_route_ties_keep_lower_id_first():
    # stable sort (moe_infer.rs:852-862)
    s = np.array([0.5, 0.7, 0.7, 0.5, 0.7], np.float32)
    top, _ = oracle.route_experts(s, 4)
    assert top == [1, 2, 4, 0]


def test_quantize_act_q8_closed_form():
    x = np.zeros(64, np.float32)
    x[:32] = np.linspace(-1.27, 1.27, 32, dtype=np.float32)
    q, s = oracle.quantize_act_q8(x)
    assert s[1] == 0 and not q[32:].any()  # all-zero block
    assert abs(s[0] - np.float32(1.27) / np.float32(127)) < 1e-9
    assert q[0] == -127 and q[31] == 127
    x2 = np.zeros(32, np.float32)
    x2[0], x2[1] = 1.27, 0.005  # 0.005/0.01 = 0.5 -> round half away -> 1
    q2, s2 = oracle.quantize_act_q8(x2)
    assert q2[0] == 127 and q2[1] == 1


def test_validation_rules():
    # compute.rs:877-949
    assert oracle.row_bytes(oracle.Q4_K, 4096) == 16 * 144
    assert oracle.row_bytes(oracle.Q4_0, 576) == 18 * 18
    assert oracle.row_bytes(oracle.IQ2_XXS, 8192) == 32 * 66
    assert oracle.row_bytes(oracle.IQ3_XXS, 256) == 98
    assert not oracle.validate_shape(oracle.Q4_K, 0, 256)
    assert not oracle.validate_shape(oracle.Q4_K, 4, 0)
    assert not oracle.validate_shape(oracle.Q4_K, 4, 300)
    assert oracle.validate_weights(oracle.Q4_K, 4, 256, 4 * 144)
    assert not oracle.validate_weights(oracle.Q4_K, 4, 256, 4 * 144 - 1)
    with pytest.raises(oracle.OracleError):
        oracle.gemv(oracle.Q4_K, 4, 256, np.zeros(100, np.uint8), np.zeros(256, np.float32))


# ------------------------------------------------------------------ RMSNorm / FFN block
@pytest.mark.parametrize("n", [8, 11, 576, 4096, 4099])
def test_rms_norm_matches_fp64(n):
    # rms_norm (attention.rs:142-147) against the formula in float64; n = 11 and 4099 take
    # the scalar tail after the f32x8 body.  A divisor of n-1, eps outside the root or a
    # missing weight moves the result far beyond this bound.
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    for eps in (1e-5, 1e-6, 0.5):
        y = oracle.rms_norm(x, w, eps)
        ref = x.astype(np.float64) * w / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)
        assert np.max(np.abs(y - ref) / np.abs(ref).max()) < 2e-6


def test_rms_norm_scale_invariant_and_constant():
    # eps = 0: scaling x by 4 scales every intermediate by an exact power of two, so the
    # output is identical bit for bit; a constant vector normalizes to +-1 (times the weight).
    rng = np.random.default_rng(5)
    x = rng.standard_normal(1003).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 1003).astype(np.float32)
    np.testing.assert_array_equal(oracle.rms_norm(x, w, 0.0), oracle.rms_norm(4 * x, w, 0.0))
    c = np.full(1003, -3.0, np.float32)
    np.testing.assert_allclose(oracle.rms_norm(c, w, 0.0), -w, rtol=2e-7)
    # large eps dominates: x / sqrt(eps) for tiny x
    t = np.full(64, 1e-4, np.float32)
    np.testing.assert_allclose(oracle.rms_norm(t, np.ones(64, np.float32), 1.0), t, rtol=1e-6)


def test_ffn_block_zero_norm_weight_is_identity_and_composes():
    # ffn_apply = x + FFN(rms_norm(x)): with a zero norm weight the FFN input is 0, SiLU(0) * 0
    # = 0, and y == x exactly; otherwise y - x equals the FFN of the normalized x.
    d_model, d_ff = 256, 512
    rng = np.random.default_rng(9)
    wg, wu, wd = (rng.integers(0, 256, (r * c) // 32 * 18, dtype=np.uint8) for r, c in
                  ((d_ff, d_model), (d_ff, d_model), (d_model, d_ff)))
    for a in (wg, wu, wd):  # finite f16 scales (0x2E66) in every Q4_0 block
        a.reshape(-1, 18)[:, 0] = 0x66
        a.reshape(-1, 18)[:, 1] = 0x2E
    x = rng.standard_normal(d_model).astype(np.float32)
    t = (oracle.Q4_0,) * 3
    y0 = oracle.ffn_block(t, d_model, d_ff, wg, wu, wd, np.zeros(d_model, np.float32), 1e-5, x)
    np.testing.assert_array_equal(y0, x)
    nw = rng.uniform(0.5, 1.5, d_model).astype(np.float32)
    y = oracle.ffn_block(t, d_model, d_ff, wg, wu, wd, nw, 1e-5, x)
    f = oracle.ffn(t, d_model, d_ff, wg, wu, wd, oracle.rms_norm(x, nw, 1e-5))
    np.testing.assert_array_equal(y, x + f)


# ---------------------------------------------------------------------------------------
# or_ffn and or_moe_token pinned by float64 compositions of the pinned pieces.
#
# The reference's FFN (stream_infer.rs:3752-3864: gate and up GEMV, act(g) * u, down GEMV)
# and its MoE token (moe_infer.rs:342-380: per selected expert the same FFN at its own
# weights, acc += w_e * down_e in top order) are composed here from the dequant (pinned
# above), numpy float64 products and numpy's exp/tanh, and the oracle's fp32 result must
# sit inside the rounding bound propagated through the chain.  Planted mistakes in the
# oracle (gate/up swapped, expert id off by one) must fall outside it.

U32 = 2.0 ** -23  # twice the fp32 unit roundoff: the per-term factor of the GEMV bound above


def _mat(t, rows, cols, w):
    return oracle.dequant(t, w, rows * cols).reshape(rows, cols).astype(np.float64)


def _act64(g, act):
    if act == 0:
        return g / (1.0 + np.exp(-g))
    return 0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g + 0.044715 * g ** 3)))


def _ffn64_with_bound(types, d_model, d_ff, wg, wu, wd, x, act):
    """FFN in float64 and a bound on |fp32 oracle - float64| for y and for h."""
    tg, tu, td = types
    Wg, Wu, Wd = _mat(tg, d_ff, d_model, wg), _mat(tu, d_ff, d_model, wu), _mat(td, d_model, d_ff, wd)
    x64 = x.astype(np.float64)
    g, u = Wg @ x64, Wu @ x64
    bg = d_model * U32 * (np.abs(Wg) @ np.abs(x64))
    bu = d_model * U32 * (np.abs(Wu) @ np.abs(x64))
    s = _act64(g, act)
    h = s * u
    # |act'| <= 1.2 for SiLU (max 1.0998) and tanh-GELU (max 1.129); 16 units for the
    # activation's own roundings (exp/tanh, the divide, the products)
    bh = 1.2 * bg * (np.abs(u) + bu) + (np.abs(s) + 1.2 * bg) * bu + 16 * U32 * np.abs(h)
    y = Wd @ h
    by = np.abs(Wd) @ bh + d_ff * U32 * (np.abs(Wd) @ (np.abs(h) + bh))
    return y, by, h, bh


def _ffn_weights(types, d_model, d_ff, seed):
    import hayai_amd.synth as synth

    tg, tu, td = types
    return (synth.matrix(tg, d_ff, d_model, seed), synth.matrix(tu, d_ff, d_model, seed + 1),
            synth.matrix(td, d_model, d_ff, seed + 2))


FFN_PIN_CASES = [
    ((oracle.Q4_0,) * 3, 256, 512, 0),
    ((oracle.Q4_K,) * 3, 256, 512, 0),
    ((oracle.Q4_K, oracle.Q4_K, oracle.Q6_K), 512, 256, 0),
    ((oracle.IQ2_XXS,) * 3, 256, 512, 0),
    ((oracle.IQ3_XXS, oracle.Q8_0, oracle.Q4_K), 256, 256, 1),
    ((oracle.F16, oracle.Q4_0, oracle.Q8_0), 64, 96, 1),
]


def _f16_weights(rng, rows, cols):
    return (rng.normal(size=rows * cols) * 0.05).astype(np.float16).view(np.uint8)


@pytest.mark.parametrize("types,d_model,d_ff,act", FFN_PIN_CASES)
def test_ffn_pinned_by_fp64_composition(types, d_model, d_ff, act):
    rng = np.random.default_rng(31 + d_model + act)
    if types[0] == oracle.F16:
        wg = _f16_weights(rng, d_ff, d_model)
        _, wu, wd = _ffn_weights(types, d_model, d_ff, 501)
    else:
        wg, wu, wd = _ffn_weights(types, d_model, d_ff, 500 + sum(types))
    x = rng.normal(size=d_model).astype(np.float32)
    y, h = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x, act=act, return_h=True)
    y64, by, h64, bh = _ffn64_with_bound(types, d_model, d_ff, wg, wu, wd, x, act)
    assert np.all(np.abs(h - h64) <= bh)
    assert np.all(np.abs(y - y64) <= by)
    # the worst-case bound (no cancellation assumed) stays well under the outputs, and the
    # error actually seen is far tighter (measured <= 6e-7 of max|y| on these cases), so a
    # mistake that moves any output by 1e-5 of the largest one fails as well
    assert np.max(by) < 1e-2 * np.max(np.abs(y64))
    assert np.max(np.abs(y - y64)) <= 1e-5 * np.max(np.abs(y64))


def test_ffn_pin_catches_gate_up_swap():
    types, d_model, d_ff = (oracle.Q4_K,) * 3, 256, 512
    wg, wu, wd = _ffn_weights(types, d_model, d_ff, 700)
    x = np.random.default_rng(5).normal(size=d_model).astype(np.float32)
    y64, by, _, _ = _ffn64_with_bound(types, d_model, d_ff, wg, wu, wd, x, 0)
    assert np.all(np.abs(oracle.ffn(types, d_model, d_ff, wg, wu, wd, x) - y64) <= by)
    oracle.set_mutation(1)
    try:
        ym = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)
    finally:
        oracle.set_mutation(0)
    assert not np.all(np.abs(ym - y64) <= by)


def _moe_setup(t, n_exp, d_model, d_ff, seed):
    """n_exp experts in one buffer; per expert the regions are stored down, up, gate (not
    the offsets' natural order) so a swapped offset reads the wrong matrix."""
    import hayai_amd.synth as synth

    rg, rd = oracle.row_bytes(t, d_model), oracle.row_bytes(t, d_ff)
    d_off, u_off, g_off = 0, d_model * rd, d_model * rd + d_ff * rg
    stride = g_off + d_ff * rg + 64  # padding between experts
    buf = np.zeros(n_exp * stride, np.uint8)
    for e in range(n_exp):
        b = e * stride
        buf[b + g_off:b + g_off + d_ff * rg] = synth.matrix(t, d_ff, d_model, seed + 3 * e)
        buf[b + u_off:b + u_off + d_ff * rg] = synth.matrix(t, d_ff, d_model, seed + 3 * e + 1)
        buf[b + d_off:b + d_off + d_model * rd] = synth.matrix(t, d_model, d_ff, seed + 3 * e + 2)
    return buf, stride, (g_off, u_off, d_off)


def _moe64_with_bound(t, d_model, d_ff, buf, stride, offs, ids, wts, x, acc0):
    g_off, u_off, d_off = offs
    rg, rd = oracle.row_bytes(t, d_model), oracle.row_bytes(t, d_ff)
    acc = acc0.astype(np.float64)
    bound = np.zeros(d_model)
    mag = np.abs(acc)
    for e, w in zip(ids, wts):  # explicit loop over the selected experts, in top order
        b = int(e) * stride
        y, by, _, _ = _ffn64_with_bound((t, t, t), d_model, d_ff, buf[b + g_off:b + g_off + d_ff * rg],
                                        buf[b + u_off:b + u_off + d_ff * rg],
                                        buf[b + d_off:b + d_off + d_model * rd], x, 0)
        acc = acc + float(w) * y
        bound += abs(float(w)) * by
        mag += np.abs(float(w) * y)
    # each acc += w * d rounds twice per selected expert
    return acc, bound + 2 * len(ids) * U32 * (mag + bound)


@pytest.mark.parametrize("t,d_model,d_ff", [(oracle.Q4_K, 256, 256), (oracle.Q4_0, 128, 96)])
def test_moe_token_pinned_by_fp64_loop(t, d_model, d_ff):
    n_exp = 7
    buf, stride, offs = _moe_setup(t, n_exp, d_model, d_ff, 900 + t)
    rng = np.random.default_rng(17)
    x = rng.normal(size=d_model).astype(np.float32)
    ids, wts = oracle.route_experts(rng.normal(size=n_exp - 1).astype(np.float32), 4, norm_topk_prob=True)
    acc0 = rng.normal(size=d_model).astype(np.float32)
    got = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, ids, wts, x, acc=acc0)
    ref, bound = _moe64_with_bound(t, d_model, d_ff, buf, stride, offs, ids, wts, x, acc0)
    assert np.all(np.abs(got - ref) <= bound)
    assert np.max(bound) < 2e-2 * np.max(np.abs(ref - acc0))
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    # accumulated into acc, not overwritten
    zero = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, ids, wts, x)
    assert np.max(np.abs((got - acc0) - zero)) <= 4 * U32 * np.max(np.abs(got))


def test_moe_pin_catches_expert_index_slip():
    t, d_model, d_ff, n_exp = oracle.Q4_K, 256, 256, 6
    buf, stride, offs = _moe_setup(t, n_exp, d_model, d_ff, 1300)
    rng = np.random.default_rng(23)
    x = rng.normal(size=d_model).astype(np.float32)
    ids, wts = [3, 0, 4, 1], np.array([0.4, 0.3, 0.2, 0.1], np.float32)  # every id + 1 exists
    zero = np.zeros(d_model, np.float32)
    ref, bound = _moe64_with_bound(t, d_model, d_ff, buf, stride, offs, ids, wts, x, zero)
    assert np.all(np.abs(oracle.moe_token(t, d_model, d_ff, buf, stride, offs, ids, wts, x) - ref) <= bound)
    oracle.set_mutation(2)
    try:
        bad = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, ids, wts, x)
    finally:
        oracle.set_mutation(0)
    assert not np.all(np.abs(bad - ref) <= bound)


def _shared_setup(t, d_model, d_ff, seed):
    import hayai_amd.synth as synth

    return (synth.matrix(t, d_ff, d_model, seed), synth.matrix(t, d_ff, d_model, seed + 1),
            synth.matrix(t, d_model, d_ff, seed + 2))


@pytest.mark.parametrize("t,d_model,d_ff,sdf", [(oracle.Q4_K, 256, 256, 512), (oracle.Q4_0, 128, 96, 64)])
def test_moe_shared_expert_pinned(t, d_model, d_ff, sdf):
    # or_moe_shared (moe_infer.rs:456-493): the shared expert's SiLU FFN, weight 1, added to
    # the accumulator.  Pinned on its own by the float64 FFN composition under the propagated
    # bound (one more rounding for acc += d), and in the layer: after the routed experts, once,
    # bit for bit fl(routed + shared)
    sg, su, sd = _shared_setup(t, d_model, sdf, 1500 + t)
    rng = np.random.default_rng(41)
    x = rng.normal(size=d_model).astype(np.float32)
    acc0 = rng.normal(size=d_model).astype(np.float32)
    buf, stride, offs = _moe_setup(t, 5, d_model, d_ff, 1400 + t)
    only = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, [], [], x, acc=acc0, shared=(sdf, sg, su, sd))
    y64, by, _, _ = _ffn64_with_bound((t, t, t), d_model, sdf, sg, su, sd, x, 0)
    ref = acc0.astype(np.float64) + y64
    bound = by + U32 * (np.abs(acc0) + np.abs(y64) + by)
    assert np.all(np.abs(only - ref) <= bound)
    assert np.max(np.abs(only - ref)) <= 1e-5 * np.max(np.abs(y64))
    d = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, [], [], x, shared=(sdf, sg, su, sd))
    ids, wts = [2, 0, 4], np.array([0.5, 0.3, 0.2], np.float32)
    routed = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, ids, wts, x)
    both = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, ids, wts, x, shared=(sdf, sg, su, sd))
    np.testing.assert_array_equal(both, routed + d)
    oracle.set_mutation(3)
    try:
        bad = oracle.moe_token(t, d_model, d_ff, buf, stride, offs, [], [], x, acc=acc0, shared=(sdf, sg, su, sd))
    finally:
        oracle.set_mutation(0)
    assert not np.all(np.abs(bad - ref) <= bound)


def test_ffn_q8_composes_the_pinned_pieces():
    # or_ffn_q8 (the batched int8 path's FFN) = or_ffn on x -> q*s, then the down GEMV of
    # h -> q*s, with or_quantize_act_q8, or_ffn and or_gemv each pinned above: bit-exact
    types, d_model, d_ff = (oracle.Q4_K,) * 3, 256, 512
    wg, wu, wd = _ffn_weights(types, d_model, d_ff, 800)
    x = np.random.default_rng(8).normal(size=d_model).astype(np.float32)
    xq = oracle.dequant_act_q8(x)
    q, s = oracle.quantize_act_q8(x)
    assert np.array_equal(xq, q.astype(np.float32) * np.repeat(s, 32))
    _, h = oracle.ffn(types, d_model, d_ff, wg, wu, wd, xq, return_h=True)
    y = oracle.gemv(oracle.Q4_K, d_model, d_ff, wd, oracle.dequant_act_q8(h))
    np.testing.assert_array_equal(oracle.ffn_q8(types, d_model, d_ff, wg, wu, wd, x), y)
    # and the quantization moves the FFN by about the int8 step, not more
    yf = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)
    assert 1e-4 < np.max(np.abs(y - yf)) / np.max(np.abs(yf)) < 3e-2
