"""Host synthetic-input generator: deterministic, well-formed blocks, stated distributions."""
import numpy as np

import oracle
from hayai_amd import synth


def test_splitmix64_reference_values():
    # splitmix64 (Steele, Lea, Flood 2014) from state 0: first outputs of the generator
    # x += 0x9E3779B97F4A7C15; z = mix(x)
    assert int(synth.synth_u64(0, np.array([0], np.uint64))[0]) == 0xE220A8397B1DCDAF
    assert int(synth.synth_u64(0, np.array([1], np.uint64))[0]) == 0x6E789E6AA1B965F4
    assert int(synth.synth_u64(0, np.array([2], np.uint64))[0]) == 0x06C45D188009454F


def test_stream_is_counter_based():
    a = synth.stream_bytes(42, 1000)
    b = synth.stream_bytes(42, 2000)
    assert np.array_equal(a, b[:1000])
    assert not np.array_equal(a, synth.stream_bytes(43, 1000))


def test_q4_k_scales_in_range_and_uniform_codes():
    w = synth.matrix(synth.Q4_K, 256, 4096, seed=7).reshape(-1, 144)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dm = w[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    lo, hi = synth.SCALE_RANGE[synth.Q4_K]
    for v in (d, dm):
        assert v.min() >= np.float16(lo) * 0.999 and v.max() <= np.float16(hi) * 1.001
        assert abs(v.mean() - (lo + hi) / 2) < 0.02 * (hi - lo)
    nib = np.concatenate([w[:, 16:] & 15, w[:, 16:] >> 4]).ravel()
    counts = np.bincount(nib, minlength=16) / nib.size
    assert np.all(np.abs(counts - 1 / 16) < 0.002)
    # dequant stays finite for every block
    y = oracle.dequant(oracle.Q4_K, w.ravel(), w.shape[0] * 256)
    assert np.isfinite(y).all()


def test_normal_moments():
    x = synth.normal(3, 200000)
    assert x.dtype == np.float32
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


def test_iq_formats_well_formed():
    for t in (synth.IQ2_XXS, synth.IQ3_XXS, synth.Q4_0, synth.Q8_0, synth.Q6_K):
        w = synth.matrix(t, 8, 1024, seed=t)
        y = oracle.dequant(t, w, 8 * 1024)
        assert np.isfinite(y).all() and np.abs(y).max() > 0


def test_scale_field_positions():
    # d lands where each format keeps it: the block start, or byte 208 for Q6_K
    for t, at in ((synth.Q8_0, 0), (synth.Q6_K, 208), (synth.Q4_0, 0)):
        block, bb = synth.BLOCK[t]
        w = synth.quant_weights(t, 64, seed=7).reshape(64, bb)
        d = w[:, at:at + 2].copy().view(np.uint16).ravel().view(np.float16).astype(np.float32)
        lo, hi = synth.SCALE_RANGE[t]
        assert (d >= np.float32(lo) * 0.999).all() and (d <= np.float32(hi) * 1.001).all()


def test_seed_for_distinct():
    seeds = {synth.seed_for(c, l, m) for c in range(5) for l in range(80) for m in range(4)}
    assert len(seeds) == 5 * 80 * 4
