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


@pytest.fixture(scope="module")
def two_launch_engine():
    """An engine with the persistent one-launch Q4_K FFN switched off (HAYAI_HIP_FFNP=0):
    every FFN runs as the two-launch gate/up(+act) then down path."""
    import os

    old = os.environ.get("HAYAI_HIP_FFNP")
    os.environ["HAYAI_HIP_FFNP"] = "0"
    try:
        eng = hayai_amd.HipEngine(0)
    finally:
        if old is None:
            del os.environ["HAYAI_HIP_FFNP"]
        else:
            os.environ["HAYAI_HIP_FFNP"] = old
    yield eng
    eng.close()


PERSISTENT_CASES = [
    # (d_model, d_ff): the 8B shape (1 wave per gate/up row, 4 per down row); d_model 8192
    # (2 waves per gate/up row); d_ff 28672 (8 waves per down row); fewer h granules and
    # down rows than workgroups (the expert shape, and a tiny layer)
    (4096, 14336), (8192, 4096), (1024, 28672), (2048, 768), (256, 512),
]


@pytest.mark.parametrize("d_model,d_ff", PERSISTENT_CASES)
def test_persistent_ffn_matches_oracle_and_two_launch(engine, two_launch_engine, d_model, d_ff):
    # The persistent kernel (gate/up, grid barrier, down with its weights already in flight)
    # against the oracle and against the two-launch kernels on the same bytes.
    types = (12, 12, 12)
    print(f"[case] persistent ffn {d_model}x{d_ff}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 20)
    pack2 = two_launch_engine.alloc(lay.total)
    pack2.write(wg, lay.gate_off)
    pack2.write(wu, lay.up_off)
    pack2.write(wd, lay.down_off)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    for k in range(2):
        x = synth.normal(synth.seed_for(20, k, synth.ACT), d_model)
        y = engine.ffn(desc, pack, 0, x)
        y2 = two_launch_engine.ffn(desc, pack2, 0, x)
        ref = oracle.ffn(types, d_model, d_ff, wg, wu, wd, x)
        assert rel_err(y, ref) <= REL_TOL, rel_err(y, ref)
        assert rel_err(y, y2) <= REL_TOL
        print(f"  rel_err vs oracle {rel_err(y, ref):.2e}, vs two-launch {rel_err(y, y2):.2e}", flush=True)


def test_persistent_ffn_chain_is_deterministic(engine):
    # 6 dependent launches with no host sync in between (each launch's grid barrier uses a new
    # generation; the h exchange buffer is reused), then the same chain call by call: the
    # results are identical bit for bit, and every step is within tolerance of the oracle.
    types, d_model, d_ff = (12, 12, 12), 4096, 14336
    print(f"[case] persistent ffn chain {d_model}x{d_ff}", flush=True)
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
                                                 ((12, 2, 18), 1024, 2048)])
def test_ffn_begin_finish_equals_ffn(engine, two_launch_engine, types, d_model, d_ff):
    # The reference's two-call seam (ffn_begin_gate_up_scratch / ffn_finish_scratch) runs the
    # same kernels as the two-launch form of the one-call op: identical bits.  (With the
    # persistent Q4_K kernel the one-call op differs from it only by rounding.)
    print(f"[case] begin/finish types={types} {d_model}x{d_ff}", flush=True)
    for eng, exact in ((two_launch_engine, True), (engine, types != (12, 12, 12))):
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
        if exact:
            np.testing.assert_array_equal(a, b)
        else:
            assert rel_err(a, b) <= REL_TOL
        # a finish consumes the pending intermediate; a second one (or one for another shape) fails
        with pytest.raises(hayai_amd.HipError):
            eng.ffn_finish_dev(desc, pack, 0, y2, 0)
        eng.ffn_begin_dev(desc, pack, 0, xb, 0)
        other = eng.ffn_desc(types, d_model, d_ff, lay, 1)
        with pytest.raises(hayai_amd.HipError):
            eng.ffn_finish_dev(other, pack, 0, y2, 0)
