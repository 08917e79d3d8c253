"""GPU FFN op parity: hh_ffn / hh_ffn_dev (the fused replacement of
ffn_begin_gate_up_scratch + ffn_finish_scratch, stream_infer.rs:3752-3864) against the
oracle's gate GEMV, up GEMV, SiLU*up, down GEMV in fp32."""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import synth

pytestmark = pytest.mark.gpu
REL_TOL = 1e-3


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def make_pack(engine, types, d_model, d_ff, config_id, layer=0):
    tg, tu, td = types
    gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, tg)
    up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, tu)
    down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, td)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    wg = synth.matrix(tg, d_ff, d_model, synth.seed_for(config_id, layer, synth.GATE))
    wu = synth.matrix(tu, d_ff, d_model, synth.seed_for(config_id, layer, synth.UP))
    wd = synth.matrix(td, d_model, d_ff, synth.seed_for(config_id, layer, synth.DOWN))
    pack = engine.alloc(lay.total)
    pack.write(wg, lay.gate_off)
    pack.write(wu, lay.up_off)
    pack.write(wd, lay.down_off)
    return lay, (wg, wu, wd), pack


FFN_CASES = [
    # (types, d_model, d_ff, act, config id): config 1 SmolLM Q4_0, config 2 8B Q4_K,
    # config 4 expert shape, config 5-like IQ2_XXS (reduced d_ff), IQ3_XXS, mixed formats
    ((2, 2, 2), 576, 1536, 0, 1),
    ((12, 12, 12), 4096, 14336, 0, 2),
    ((12, 12, 12), 2048, 768, 0, 4),
    ((16, 16, 16), 8192, 3584, 0, 5),
    ((18, 18, 18), 4096, 14336, 0, 6),
    ((12, 12, 12), 4096, 14336, 1, 7),   # GELU(tanh) activation
    ((12, 2, 18), 1024, 2048, 0, 8),     # gate/up formats differ -> unfused gate/up path
    ((12, 12, 14), 4096, 14336, 0, 9),   # Q4_K_M layout: gate/up Q4_K, down Q6_K
    ((14, 14, 14), 1024, 2048, 0, 10),   # all Q6_K
    ((8, 8, 8), 1024, 2048, 1, 11),      # all Q8_0, GELU
    # IQ ring kernels with other down formats (h's digits are shared by every ring down
    # kernel), GELU on IQ2_XXS, and widths the ring kernels refuse (odd block counts per row:
    # the generic team kernels)
    ((16, 16, 18), 8192, 3584, 0, 12),   # IQ2_XXS gate/up, IQ3_XXS down
    ((18, 18, 14), 4096, 14336, 0, 13),  # IQ3_XXS gate/up, Q6_K down
    ((16, 16, 12), 8192, 4096, 1, 14),   # IQ2_XXS gate/up, Q4_K down, GELU
    ((18, 18, 16), 1024, 6144, 0, 15),   # IQ3_XXS gate/up, IQ2_XXS down
    ((16, 16, 16), 4352, 1280, 0, 16),   # 17 / 5 blocks per row: no ring kernels
]


@pytest.mark.parametrize("types,d_model,d_ff,act,cfg", FFN_CASES)
def test_ffn_matches_oracle(engine, types, d_model, d_ff, act, cfg):
    oracle.set_threads(min(16, oracle.max_threads()))
    print(f"[case] ffn types={types} d_model={d_model} d_ff={d_ff} act={act}", flush=True)
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, cfg)
    x = synth.normal(synth.seed_for(cfg, 0, synth.ACT), d_model)
    desc = engine.ffn_desc(types, d_model, d_ff, lay, act)
    y = engine.ffn(desc, pack, 0, x)
    ref, h_ref = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x, act=act, return_h=True)
    assert np.isfinite(y).all()
    assert rel_err(y, ref) <= REL_TOL, rel_err(y, ref)
    # per-element check where the output is not near zero
    big = np.abs(ref) > 1e-3 * np.abs(ref).max()
    per = np.abs(y[big] - ref[big]) / np.abs(ref[big])
    print(f"  rel_inf={rel_err(y, ref):.3e} per_elem_max={per.max():.3e}", flush=True)


def test_ffn_dev_chain_and_pack_offset(engine):
    # two layers resident in one buffer at layer * stride (resident scratch addressing,
    # hetero_scratch.rs:915-925); chain y0 -> x1 on the device
    types, d_model, d_ff = (2, 2, 2), 576, 1536
    lay0, w0, pack0 = make_pack(engine, types, d_model, d_ff, 11, layer=0)
    lay1, w1, pack1 = make_pack(engine, types, d_model, d_ff, 11, layer=1)
    stride = lay0.total
    big = engine.alloc(2 * stride)
    for i, (wg, wu, wd) in enumerate((w0, w1)):
        big.write(wg, i * stride + lay0.gate_off)
        big.write(wu, i * stride + lay0.up_off)
        big.write(wd, i * stride + lay0.down_off)
    desc = engine.ffn_desc(types, d_model, d_ff, lay0)
    x = synth.normal(5, d_model)
    xb = engine.upload(x)
    ya = engine.alloc(4 * d_model)
    yb = engine.alloc(4 * d_model)
    engine.ffn_dev(desc, big, 0, xb, 0, ya, 0)
    engine.ffn_dev(desc, big, stride, ya, 0, yb, 0)
    y = yb.read(np.float32, d_model)
    r0 = oracle.ffn(types, d_model, d_ff, *w0, x)
    r1 = oracle.ffn(types, d_model, d_ff, *w1, r0)
    assert rel_err(y, r1) <= REL_TOL


def test_ffn_rejects_bad_pack(engine):
    types, d_model, d_ff = (12, 12, 12), 256, 512
    lay, _, pack = make_pack(engine, types, d_model, d_ff, 12)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    with pytest.raises(hayai_amd.HipError):
        engine.ffn(desc, pack, 512, synth.normal(1, d_model))  # pushes down past the end
    bad = engine.ffn_desc(types, d_model, 500, lay)
    with pytest.raises(hayai_amd.HipError):
        engine.ffn(bad, pack, 0, synth.normal(1, d_model))
    before = engine.ffn_calls
    engine.ffn(desc, pack, 0, synth.normal(1, d_model))
    assert engine.ffn_calls == before + 3


def engine_with_env(**env):
    """A HipEngine created with the given HAYAI_HIP_* switches set (read at creation)."""
    import os

    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return hayai_amd.HipEngine(0)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def two_launch_engine():
    """An engine with the ring kernels off: Q4_K FFNs run as the first two-launch kernels
    (gate/up + activation with per-32 digits of h, then down), IQ formats on the generic f32
    team kernels."""
    eng = engine_with_env(HAYAI_HIP_RING="0")
    yield eng
    eng.close()


Q4K_CASES = [
    # (d_model, d_ff): the 8B shape (1 wave per gate/up row, 4 per down row); d_model 8192
    # (2 waves per gate/up row); d_ff 28672 (8 waves per down row); fewer h granules and
    # down rows than workgroups (the expert shape, and a tiny layer)
    (4096, 14336), (8192, 4096), (1024, 28672), (2048, 768), (256, 512),
]


@pytest.mark.parametrize("d_model,d_ff", Q4K_CASES)
def test_q4k_ffn_ring_matches_oracle_and_two_launch(engine, two_launch_engine, d_model, d_ff):
    # The ring form (two streaming launches, h as granule digits in between) against the
    # oracle and against the first two-launch kernels on the same bytes.
    types = (12, 12, 12)
    eng = engine
    print(f"[case] q4_k ffn (ring) {d_model}x{d_ff}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    lay, (wg, wu, wd), pack = make_pack(eng, types, d_model, d_ff, 20)
    pack2 = two_launch_engine.alloc(lay.total)
    pack2.write(wg, lay.gate_off)
    pack2.write(wu, lay.up_off)
    pack2.write(wd, lay.down_off)
    desc = eng.ffn_desc(types, d_model, d_ff, lay)
    for k in range(2):
        x = synth.normal(synth.seed_for(20, k, synth.ACT), d_model)
        y = eng.ffn(desc, pack, 0, x)
        y2 = two_launch_engine.ffn(desc, pack2, 0, x)
        ref = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)
        assert rel_err(y, ref) <= REL_TOL, rel_err(y, ref)
        assert rel_err(y, y2) <= REL_TOL
        print(f"  rel_err vs oracle {rel_err(y, ref):.2e}, vs two-launch {rel_err(y, y2):.2e}", flush=True)
    eng.sync()  # reports a timed-out wait if one was recorded


Q4KM_CASES = [
    # (d_model, d_ff): the 8B shape; d_model 8192; d_ff 28672 (8 waves per down row); a tiny
    # layer (2 superblocks per down row); d_ff 1280 (an odd number of Q6_K superblocks per
    # row: down rows are not 4-byte aligned, so the generic kernels run instead)
    (4096, 14336), (8192, 4096), (1024, 28672), (256, 512), (512, 1280),
]


@pytest.mark.parametrize("d_model,d_ff", Q4KM_CASES)
def test_q4k_m_ffn_matches_oracle_and_two_launch(engine, two_launch_engine, d_model, d_ff):
    # Q4_K_M layout (gate/up Q4_K, down Q6_K): the ring gate/up kernel and the Q6_K ring down
    # kernel (210-byte superblocks, half of them 2 bytes off a dword) against the oracle and
    # against the generic gate/up + Q6_K GEMV kernels on the same bytes.
    types = (12, 12, 14)
    print(f"[case] q4_k_m ffn {d_model}x{d_ff}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 21)
    pack2 = two_launch_engine.alloc(lay.total)
    pack2.write(wg, lay.gate_off)
    pack2.write(wu, lay.up_off)
    pack2.write(wd, lay.down_off)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    for k in range(2):
        x = synth.normal(synth.seed_for(21, k, synth.ACT), d_model)
        y = engine.ffn(desc, pack, 0, x)
        y2 = two_launch_engine.ffn(desc, pack2, 0, x)
        ref = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)
        assert np.isfinite(y).all()
        assert rel_err(y, ref) <= REL_TOL, rel_err(y, ref)
        assert rel_err(y, y2) <= REL_TOL
        print(f"  rel_err vs oracle {rel_err(y, ref):.2e}, vs two-launch {rel_err(y, y2):.2e}", flush=True)


@pytest.mark.parametrize("form", ["ring", "two-launch"])
def test_q4k_ffn_chain_is_deterministic(engine, two_launch_engine, form):
    # 6 dependent launches with no host sync in between (the h buffer is reused), then the
    # same chain call by call: the results are identical bit for bit, and every step is within
    # tolerance of the oracle.
    types, d_model, d_ff = (12, 12, 12), 4096, 14336
    engine = engine if form == "ring" else two_launch_engine
    print(f"[case] q4_k ffn chain ({form}) {d_model}x{d_ff}", flush=True)
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 2)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    x = synth.normal(synth.seed_for(2, 9, synth.ACT), d_model)
    xb = engine.upload(x)
    bufs = [engine.alloc(4 * d_model) for _ in range(2)]
    src = xb
    for k in range(6):
        engine.ffn_dev(desc, pack, 0, src, 0, bufs[k % 2], 0)
        src = bufs[k % 2]
    yc = src.read(np.float32, d_model)
    r = x
    for k in range(6):
        r = engine.ffn(desc, pack, 0, r)
        if k == 0:
            assert rel_err(r, oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)) <= REL_TOL
    np.testing.assert_array_equal(yc, r)
    engine.sync()  # reports a grid-barrier timeout if one was recorded


@pytest.mark.parametrize("types,d_model,d_ff", [((12, 12, 12), 4096, 14336), ((2, 2, 2), 576, 1536),
                                                 ((12, 2, 18), 1024, 2048), ((12, 12, 14), 4096, 14336)])
def test_ffn_begin_finish_equals_ffn(engine, two_launch_engine, types, d_model, d_ff):
    # The reference's two-call seam (ffn_begin_gate_up_scratch / ffn_finish_scratch) runs the
    # same kernels as the one-call op (the ring kernels for Q4_K, or the first two-launch
    # kernels): identical bits.
    print(f"[case] begin/finish types={types} {d_model}x{d_ff}", flush=True)
    for eng in (engine, two_launch_engine):
        lay, _, pack = make_pack(eng, types, d_model, d_ff, 13)
        desc = eng.ffn_desc(types, d_model, d_ff, lay)
        x = synth.normal(77, d_model)
        xb = eng.upload(x)
        y1 = eng.alloc(4 * d_model)
        y2 = eng.alloc(4 * d_model)
        eng.ffn_dev(desc, pack, 0, xb, 0, y1, 0)
        eng.ffn_begin_dev(desc, pack, 0, xb, 0)
        eng.ffn_finish_dev(desc, pack, 0, y2, 0)
        a, b = y1.read(np.float32, d_model), y2.read(np.float32, d_model)
        np.testing.assert_array_equal(a, b)
        # a finish consumes the pending intermediate; a second one (or one for another shape) fails
        with pytest.raises(hayai_amd.HipError):
            eng.ffn_finish_dev(desc, pack, 0, y2, 0)
        eng.ffn_begin_dev(desc, pack, 0, xb, 0)
        other = eng.ffn_desc(types, d_model, d_ff, lay, 1)
        with pytest.raises(hayai_amd.HipError):
            eng.ffn_finish_dev(other, pack, 0, y2, 0)


IQ_RING_CASES = [
    # (types, d_model, d_ff): config 5's 70B IQ2_XXS layer (8 waves per down row), IQ3_XXS at
    # the 8B shape, a narrow layer (one block pair per gate/up row, fewer h granules than
    # workgroups), and a d_model of 1536 (three lane units left idle in a 64-lane team)
    ((16, 16, 16), 8192, 28672), ((18, 18, 18), 4096, 14336), ((16, 16, 16), 512, 1024),
    ((18, 18, 18), 1536, 4608),
]


@pytest.mark.parametrize("types,d_model,d_ff", IQ_RING_CASES)
def test_iq_ring_ffn_matches_oracle_and_generic(engine, two_launch_engine, types, d_model, d_ff):
    # The IQ2_XXS / IQ3_XXS ring kernels (int8 codebook entries, v_dot4 against the
    # activation digits) and the generic f32 team kernels (ring form off) each meet the
    # FFN bar against the oracle; the two-call seam runs the ring kernels bit for bit.
    oracle.set_threads(min(16, oracle.max_threads()))
    print(f"[case] iq ring ffn types={types} {d_model}x{d_ff}", flush=True)
    x = synth.normal(synth.seed_for(40, d_model, synth.ACT), d_model)
    lay, (wg, wu, wd), pack0 = make_pack(engine, types, d_model, d_ff, 40)
    ys = {}
    for name, eng in (("ring", engine), ("generic", two_launch_engine)):
        pack = pack0
        if eng is not engine:
            pack = eng.alloc(lay.total)
            for w, off in ((wg, lay.gate_off), (wu, lay.up_off), (wd, lay.down_off)):
                pack.write(w, off)
        desc = eng.ffn_desc(types, d_model, d_ff, lay)
        ys[name] = eng.ffn(desc, pack, 0, x)
        if name == "ring":
            xb, y2 = eng.upload(x), eng.alloc(4 * d_model)
            eng.ffn_begin_dev(desc, pack, 0, xb, 0)
            eng.ffn_finish_dev(desc, pack, 0, y2, 0)
            np.testing.assert_array_equal(y2.read(np.float32, d_model), ys[name])
    ref = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)
    for name, y in ys.items():
        err = rel_err(y, ref)
        print(f"  {name}: rel_err {err:.3e}", flush=True)
        assert np.isfinite(y).all()
        assert err <= REL_TOL, (name, err)


BLOCK_CASES = [
    # (types, d_model, d_ff): the ring kernels with the norm and residual fused (8B Q4_K,
    # Q4_K_M, d_model 8192: two x passes per thread, IQ2_XXS, IQ3_XXS), and the generic
    # three-step path (SmolLM Q4_0, IQ2_XXS with an odd block count per row)
    ((12, 12, 12), 4096, 14336), ((12, 12, 14), 4096, 14336), ((12, 12, 12), 8192, 4096),
    ((2, 2, 2), 576, 1536), ((16, 16, 16), 1024, 2048), ((18, 18, 18), 4096, 14336),
    ((16, 16, 16), 8192, 28672), ((16, 16, 16), 768, 2304),
]


@pytest.mark.parametrize("types,d_model,d_ff", BLOCK_CASES)
def test_ffn_block_matches_oracle(engine, types, d_model, d_ff):
    # ffn_apply (hybrid_infer.rs:883-936): y = x + FFN(rms_norm(x)).  The FFN part (y - x) is
    # held to the FFN bar against the oracle; out of place and in place (y = x) agree.
    print(f"[case] ffn block types={types} {d_model}x{d_ff}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 22)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    rng = np.random.default_rng(d_model + d_ff)
    x = (3.0 * rng.standard_normal(d_model)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, d_model).astype(np.float32)
    eps = 1e-5
    ref = oracle.ffn_block(types, d_model, d_ff, wg, wu, wd, nw, eps, x)
    xb, nb, yb = engine.upload(x), engine.upload(nw), engine.alloc(4 * d_model)
    engine.ffn_block_dev(desc, pack, 0, nb, 0, eps, xb, 0, yb, 0)
    y = yb.read(np.float32, d_model)
    assert np.isfinite(y).all()
    err = rel_err(y - x, ref - x)
    print(f"  rel_err of the FFN part {err:.3e}", flush=True)
    assert err <= REL_TOL, err
    engine.ffn_block_dev(desc, pack, 0, nb, 0, eps, xb, 0, xb, 0)  # in place
    np.testing.assert_array_equal(xb.read(np.float32, d_model), y)
    # the host-activation form
    np.testing.assert_array_equal(engine.ffn_block(desc, pack, 0, nw, eps, x), y)


@pytest.mark.parametrize("types,d_model,d_ff", [((12, 12, 12), 4096, 14336), ((12, 12, 14), 4096, 14336),
                                                ((2, 2, 2), 576, 1536), ((16, 16, 16), 1024, 2048),
                                                ((18, 18, 18), 4096, 14336), ((16, 16, 16), 768, 2304)])
def test_ffn_block_begin_finish_equals_block(engine, types, d_model, d_ff):
    # ffn_apply's own two calls (rms_norm + begin, finish + residual) run the block's kernels:
    # bit-identical to the one-call block, out of place and in place.
    print(f"[case] ffn block begin/finish types={types} {d_model}x{d_ff}", flush=True)
    lay, _, pack = make_pack(engine, types, d_model, d_ff, 25)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    rng = np.random.default_rng(d_model)
    x = rng.standard_normal(d_model).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, d_model).astype(np.float32)
    xb, nb, y1, y2 = engine.upload(x), engine.upload(nw), engine.alloc(4 * d_model), engine.alloc(4 * d_model)
    engine.ffn_block_dev(desc, pack, 0, nb, 0, 1e-5, xb, 0, y1, 0)
    engine.ffn_block_begin_dev(desc, pack, 0, nb, 0, 1e-5, xb, 0)
    engine.ffn_block_finish_dev(desc, pack, 0, xb, 0, y2, 0)
    ref = y1.read(np.float32, d_model)
    np.testing.assert_array_equal(y2.read(np.float32, d_model).view(np.uint32), ref.view(np.uint32))
    engine.ffn_block_begin_dev(desc, pack, 0, nb, 0, 1e-5, xb, 0)
    engine.ffn_block_finish_dev(desc, pack, 0, xb, 0, xb, 0)  # in place, as ffn_apply updates x
    np.testing.assert_array_equal(xb.read(np.float32, d_model).view(np.uint32), ref.view(np.uint32))
    with pytest.raises(hayai_amd.HipError) as e:  # the finish consumed the pending intermediate
        engine.ffn_block_finish_dev(desc, pack, 0, xb, 0, y2, 0)
    assert e.value.status_name == "HH_ERR_INVALID"


def test_ffn_block_unaligned_norm_takes_the_three_step_path(engine):
    # A norm weight that is not 16-byte aligned keeps the ring kernels out (their prologue
    # reads it as float4s): the three-step path gives the same block within tolerance.
    types, d_model, d_ff = (12, 12, 12), 4096, 14336
    print(f"[case] ffn block, norm at offset 4, {d_model}x{d_ff}", flush=True)
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 23)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(d_model).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, d_model).astype(np.float32)
    nb = engine.alloc(4 * d_model + 16)
    nb.write(nw, 4)
    xb, yb = engine.upload(x), engine.alloc(4 * d_model)
    engine.ffn_block_dev(desc, pack, 0, nb, 4, 1e-5, xb, 0, yb, 0)
    y = yb.read(np.float32, d_model)
    ref = oracle.ffn_block(types, d_model, d_ff, wg, wu, wd, nw, 1e-5, x)
    assert rel_err(y - x, ref - x) <= REL_TOL
    with pytest.raises(hayai_amd.HipError):
        engine.ffn_block_dev(desc, pack, 0, nb, 2, 1e-5, xb, 0, yb, 0)  # misaligned float offset
    with pytest.raises(hayai_amd.HipError):
        engine.ffn_block_dev(desc, pack, 0, nb, 0, -1.0, xb, 0, yb, 0)  # negative eps


def test_ffn_block_chain_of_layers(engine):
    # Four layers applied in place on one residual stream, as a decode step runs them
    # (x_{l+1} = x_l + FFN_l(rms_norm(x_l, norm_l))), no host sync in between, against the
    # oracle applying the same four blocks.
    types, d_model, d_ff, L = (12, 12, 12), 4096, 14336, 4
    print(f"[case] ffn block chain, {L} layers {d_model}x{d_ff}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    packs = [make_pack(engine, types, d_model, d_ff, 24, layer=l) for l in range(L)]
    rng = np.random.default_rng(3)
    norms = [rng.uniform(0.5, 1.5, d_model).astype(np.float32) for _ in range(L)]
    x = rng.standard_normal(d_model).astype(np.float32)
    xb = engine.upload(x)
    nbs = [engine.upload(n) for n in norms]
    for l, (lay, _, pack) in enumerate(packs):
        engine.ffn_block_dev(engine.ffn_desc(types, d_model, d_ff, lay), pack, 0, nbs[l], 0, 1e-5, xb, 0, xb, 0)
    y = xb.read(np.float32, d_model)
    r = x
    for l, (lay, (wg, wu, wd), _) in enumerate(packs):
        r = oracle.ffn_block(types, d_model, d_ff, wg, wu, wd, norms[l], 1e-5, r)
    err = rel_err(y - x, r - x)
    print(f"  rel_err of the 4-layer update {err:.3e}", flush=True)
    assert err <= REL_TOL, err


@pytest.mark.parametrize("types,d_model,d_ff", [((2, 2, 2), 576, 1536), ((8, 8, 8), 1024, 2048),
                                                ((2, 2, 2), 2048, 4096), ((2, 2, 2), 2048, 8192)])
def test_small_ffn_one_launch_equals_two_launches(engine, types, d_model, d_ff):
    # The one-launch small FFN (gate/up, grid barrier, down; Q4_0 / Q8_0 shapes whose rows fit
    # two per team) gives the two-launch kernels' bits: the same unit dots and team sums.
    # 2048 x 8192 exceeds it (4 down rows per team) and runs the two launches in both engines.
    import os
    print(f"[case] small ffn types={types} {d_model}x{d_ff}", flush=True)
    old = os.environ.get("HAYAI_HIP_SMALL_FFN")
    os.environ["HAYAI_HIP_SMALL_FFN"] = "0"
    try:
        two = hayai_amd.HipEngine(0)
    finally:
        if old is None:
            del os.environ["HAYAI_HIP_SMALL_FFN"]
        else:
            os.environ["HAYAI_HIP_SMALL_FFN"] = old
    try:
        lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 25)
        lay2, _, pack2 = make_pack(two, types, d_model, d_ff, 25)
        desc = engine.ffn_desc(types, d_model, d_ff, lay)
        xb = engine.upload(synth.normal(88, d_model))
        yb = engine.alloc(4 * d_model)
        for k in range(3):  # repeated launches: a new barrier generation each time
            x = synth.normal(100 + k, d_model)
            y1 = engine.ffn(desc, pack, 0, x)
            y2 = two.ffn(two.ffn_desc(types, d_model, d_ff, lay2), pack2, 0, x)
            np.testing.assert_array_equal(y1, y2)
            assert rel_err(y1, oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)) <= REL_TOL
        engine.ffn_dev(desc, pack, 0, xb, 0, yb, 0)
        engine.sync()  # reports a timed-out barrier if one was recorded
    finally:
        two.close()


@pytest.mark.parametrize("batch", [2, 4, 16])
def test_q4k_m_batched_ffn_matches_oracle(engine, batch):
    # Batched tokens through a Q4_K_M layer: gate/up as weight-stream MFMA GEMMs, the
    # activation, the Q6_K ring GEMV per token (batch >= 4; batch 2 runs the one-token op per
    # token); each token against the oracle.
    types, d_model, d_ff = (12, 12, 14), 4096, 14336
    print(f"[case] q4_k_m batched B={batch}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 26)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    X = synth.normal(synth.seed_for(26, batch, synth.ACT), batch * d_model).reshape(batch, d_model)
    Y = engine.ffn_batched(desc, pack, 0, X)
    worst = 0.0
    for b in range(batch):
        ref = oracle.ffn(types, d_model, d_ff, wg, wu, wd, X[b])
        worst = max(worst, rel_err(Y[b], ref))
    print(f"  worst per-token rel_err {worst:.3e}", flush=True)
    assert worst <= REL_TOL, worst
