"""GPU tests of graph capture and replay (hh_graph_begin / hh_graph_end / hh_graph_launch).

A decode loop's FFN launches are the same every token, so the engine can capture a chain of
enqueue-only calls once and replay it.  Every replay must equal the eager chain bit for bit
(same kernels, same bytes), read the buffers' contents at replay time, and survive eager
work and synchronisations between replays.  Calls that cannot be replayed (kernels with
per-launch state, workspace growth) are refused without breaking the engine.
"""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import synth

pytestmark = pytest.mark.gpu

T = hayai_amd.Q4_K
D_MODEL, D_FF = 2048, 5632


def make_layers(engine, n_layers, d_model=D_MODEL, d_ff=D_FF, cfg=31):
    gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, T)
    up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, T)
    down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, T)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    packs, mats = [], []
    for l in range(n_layers):
        wg = synth.matrix(T, d_ff, d_model, synth.seed_for(cfg, l, synth.GATE))
        wu = synth.matrix(T, d_ff, d_model, synth.seed_for(cfg, l, synth.UP))
        wd = synth.matrix(T, d_model, d_ff, synth.seed_for(cfg, l, synth.DOWN))
        p = engine.alloc(lay.total)
        p.write(wg, lay.gate_off)
        p.write(wu, lay.up_off)
        p.write(wd, lay.down_off)
        packs.append(p)
        mats.append((wg, wu, wd))
    return lay, packs, mats


def chain(engine, desc, packs, xbuf, bufs):
    """x -> layer 0 -> layer 1 -> ... on the device; the last layer's output lands in bufs[-1]."""
    src = xbuf
    for l, p in enumerate(packs):
        engine.ffn_dev(desc, p, 0, src, 0, bufs[l], 0)
        src = bufs[l]


def test_graph_replay_equals_eager_chain(engine):
    n = 3
    print(f"[case] graph replay q4_k {D_MODEL}x{D_FF} layers={n}", flush=True)
    lay, packs, mats = make_layers(engine, n)
    desc = engine.ffn_desc((T, T, T), D_MODEL, D_FF, lay)
    x = synth.normal(synth.seed_for(31, 0, synth.ACT), D_MODEL)
    xbuf = engine.upload(x)
    eager = [engine.alloc(4 * D_MODEL) for _ in range(n)]
    chain(engine, desc, packs, xbuf, eager)  # also sizes every workspace the chain needs
    y_eager = eager[-1].read(np.float32, D_MODEL)

    outs = [engine.alloc(4 * D_MODEL) for _ in range(n)]
    g = engine.capture(lambda: chain(engine, desc, packs, xbuf, outs))
    other = engine.alloc(4 * D_MODEL)
    for rep in range(3):
        outs[-1].fill(0)
        g.launch()
        engine.sync()
        y = outs[-1].read(np.float32, D_MODEL)
        assert np.array_equal(y.view(np.uint32), y_eager.view(np.uint32)), f"replay {rep}"
        # eager work and a synchronisation between replays
        engine.ffn_dev(desc, packs[0], 0, xbuf, 0, other, 0)
        engine.sync()

    # the graph reads x at replay time
    x2 = synth.normal(synth.seed_for(31, 1, synth.ACT), D_MODEL)
    xbuf.write(x2)
    g.launch()
    engine.sync()
    chain(engine, desc, packs, xbuf, eager)
    y2 = outs[-1].read(np.float32, D_MODEL)
    assert np.array_equal(y2.view(np.uint32), eager[-1].read(np.float32, D_MODEL).view(np.uint32))
    # and the chain is the FFN: layer 0 against the oracle
    r0 = oracle.ffn((T, T, T), D_MODEL, D_FF, *mats[0], x2)
    y0 = outs[0].read(np.float32, D_MODEL)
    assert np.max(np.abs(y0 - r0)) / np.max(np.abs(r0)) <= 1e-3
    g.free()


def test_graph_refuses_unreplayable_calls(engine):
    print("[case] graph refusals", flush=True)
    lay, packs, _ = make_layers(engine, 1, d_model=256, d_ff=512, cfg=32)
    desc = engine.ffn_desc((T, T, T), 256, 512, lay)
    x = engine.upload(synth.normal(3, 256 * 2))
    y = engine.alloc(4 * 256 * 2)
    # batched FFN: per-launch counters, not capturable
    with pytest.raises(hayai_amd.HipError) as e:
        engine.capture(lambda: engine.ffn_batched_dev(desc, packs[0], 0, x, 0, 2, y, 0))
    assert e.value.status_name == "HH_ERR_INVALID"
    # the engine is usable afterwards, eagerly and for a new capture
    engine.ffn_dev(desc, packs[0], 0, x, 0, y, 0)
    engine.sync()
    g = engine.capture(lambda: engine.ffn_dev(desc, packs[0], 0, x, 0, y, 0))
    g.launch()
    engine.sync()
    g.free()


def test_graph_refuses_workspace_growth():
    # a fresh engine has no workspaces: the first FFN inside a capture would allocate
    print("[case] graph workspace growth", flush=True)
    eng = hayai_amd.HipEngine(0)
    try:
        lay, packs, _ = make_layers(eng, 1, d_model=256, d_ff=512, cfg=33)
        desc = eng.ffn_desc((T, T, T), 256, 512, lay)
        x = eng.upload(synth.normal(4, 256))
        y = eng.alloc(4 * 256)
        with pytest.raises(hayai_amd.HipError) as e:
            eng.capture(lambda: eng.ffn_dev(desc, packs[0], 0, x, 0, y, 0))
        assert e.value.status_name == "HH_ERR_INVALID"
        eng.ffn_dev(desc, packs[0], 0, x, 0, y, 0)  # eagerly: allocates
        eng.sync()
        g = eng.capture(lambda: eng.ffn_dev(desc, packs[0], 0, x, 0, y, 0))
        g.launch()
        eng.sync()
        g.free()
    finally:
        eng.close()
