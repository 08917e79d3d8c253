"""GPU tests of the no-allocation FFN entry point (hh_ffn_dev_noalloc).

The entry point runs hh_ffn_dev's kernels with the d_ff intermediate in a fixed per-GPU
scratch array instead of the engine's workspaces.  Its output must equal hh_ffn_dev's bit
for bit (same kernels, same bytes) on two calls in a row, the second smaller than the first
(the array keeps the last call's contents), and the FFN itself must match the oracle.  It
must also run inside a graph capture on a fresh engine, where any workspace allocation is
refused, and reject shapes beyond its limit.
"""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import synth

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4_K, Q6_K = hayai_amd.Q4_0, hayai_amd.Q8_0, hayai_amd.Q4_K, hayai_amd.Q6_K
IQ2, IQ3 = hayai_amd.IQ2_XXS, hayai_amd.IQ3_XXS


def make_layer(engine, types, d_model, d_ff, seed):
    tg, tu, td = types
    gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, tg)
    up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, tu)
    down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, td)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    wg = synth.matrix(tg, d_ff, d_model, seed)
    wu = synth.matrix(tu, d_ff, d_model, seed + 1)
    wd = synth.matrix(td, d_model, d_ff, seed + 2)
    pack = engine.alloc(lay.total)
    pack.write(wg, lay.gate_off)
    pack.write(wu, lay.up_off)
    pack.write(wd, lay.down_off)
    return engine.ffn_desc(types, d_model, d_ff, lay), pack, (wg, wu, wd)


# (types, first shape, second smaller shape): the ring layouts (Q4_K, Q4_K_M), the fused
# two-step form (IQ2_XXS at the 70B shape, Q4_0 at the SmolLM shape) and the unfused form
# with a Q6_K down GEMV (its x digits in the scratch too)
CASES = [
    ((Q4_K, Q4_K, Q4_K), (4096, 14336), (2048, 5632)),
    ((Q4_K, Q4_K, Q6_K), (4096, 14336), (1024, 2048)),
    ((IQ2, IQ2, IQ2), (8192, 28672), (2048, 5632)),
    ((IQ3, Q8_0, Q6_K), (2048, 4096), (1024, 2048)),
    ((Q4_0, Q4_0, Q4_0), (576, 1536), (256, 512)),
]


@pytest.mark.parametrize("types,big,small", CASES)
def test_noalloc_equals_ffn_dev_twice(engine, types, big, small):
    for call, (d_model, d_ff) in enumerate((big, small)):
        print(f"[case] noalloc types={types} {d_model}x{d_ff} call={call}", flush=True)
        desc, pack, mats = make_layer(engine, types, d_model, d_ff, 100 * call + 7 * sum(types))
        x = synth.normal(55 + call, d_model)
        xbuf = engine.upload(x)
        y_ref = engine.alloc(4 * d_model)
        y_na = engine.alloc(4 * d_model)
        y_na.fill(0xFF)
        engine.ffn_dev(desc, pack, 0, xbuf, 0, y_ref, 0)
        engine.ffn_dev_noalloc(desc, pack, 0, xbuf, 0, y_na, 0)
        engine.sync()
        ref = y_ref.read(np.float32, d_model)
        got = y_na.read(np.float32, d_model)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        if call == 1:  # the FFN itself, at the smaller shape (the oracle is quick there)
            r = oracle.ffn(types, d_model, d_ff, *mats, x)
            assert np.max(np.abs(got - r)) / np.max(np.abs(r)) <= 1e-3


# every form the entry point takes: the ring kernels (Q4_K), the fused two-step form
# (IQ2_XXS, Q4_0) and the unfused form with a Q6_K down GEMV
CAPTURE_CASES = [
    ((Q4_K, Q4_K, Q4_K), 2048, 5632),
    ((IQ2, IQ2, IQ2), 2048, 5632),
    ((Q4_0, Q4_0, Q4_0), 576, 1536),
    ((IQ3, Q8_0, Q6_K), 1024, 2048),
]


@pytest.mark.parametrize("types,d_model,d_ff", CAPTURE_CASES)
def test_noalloc_under_capture_on_fresh_engine(types, d_model, d_ff):
    # A fresh engine owns no workspaces, and any allocation inside a capture is refused: the
    # entry point captures and replays anyway, equal to its eager result on every replay.
    print(f"[case] noalloc graph capture types={types} {d_model}x{d_ff}", flush=True)
    eng = hayai_amd.HipEngine(0)
    try:
        desc, pack, mats = make_layer(eng, types, d_model, d_ff, 301)
        x = synth.normal(302, d_model)
        xbuf = eng.upload(x)
        y = eng.alloc(4 * d_model)
        g = eng.capture(lambda: eng.ffn_dev_noalloc(desc, pack, 0, xbuf, 0, y, 0))
        y_eager = eng.alloc(4 * d_model)
        eng.ffn_dev_noalloc(desc, pack, 0, xbuf, 0, y_eager, 0)
        eng.sync()
        ref = y_eager.read(np.float32, d_model)
        r = oracle.ffn(types, d_model, d_ff, *mats, x)
        assert np.max(np.abs(ref - r)) / np.max(np.abs(r)) <= 1e-3
        for rep in range(3):
            y.fill(0)
            g.launch()
            eng.sync()
            assert np.array_equal(y.read(np.float32, d_model).view(np.uint32), ref.view(np.uint32)), f"replay {rep}"
            eng.ffn_dev_noalloc(desc, pack, 0, xbuf, 0, y_eager, 0)  # eager work between replays
            eng.sync()
        g.free()
    finally:
        eng.close()


def test_noalloc_rejects_d_ff_beyond_limit(engine):
    print("[case] noalloc limit", flush=True)
    d_model, d_ff = 32, 32768 + 256
    desc, pack, _ = make_layer(engine, (Q4_0, Q4_0, Q4_0), d_model, d_ff, 401)
    xbuf = engine.upload(synth.normal(402, d_model))
    y = engine.alloc(4 * d_model)
    with pytest.raises(hayai_amd.HipError) as e:
        engine.ffn_dev_noalloc(desc, pack, 0, xbuf, 0, y, 0)
    assert e.value.status_name == "HH_ERR_INVALID"
    assert "d_ff" in str(e.value)
    # the engine and the entry point are still usable
    desc2, pack2, mats2 = make_layer(engine, (Q4_0, Q4_0, Q4_0), 256, 512, 403)
    x2 = synth.normal(404, 256)
    x2buf = engine.upload(x2)
    y2 = engine.alloc(4 * 256)
    engine.ffn_dev_noalloc(desc2, pack2, 0, x2buf, 0, y2, 0)
    engine.sync()
    r = oracle.ffn((Q4_0,) * 3, 256, 512, *mats2, x2)
    assert np.max(np.abs(y2.read(np.float32, 256) - r)) / np.max(np.abs(r)) <= 1e-3
