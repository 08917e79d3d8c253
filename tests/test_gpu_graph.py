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


BARRIER_CASES = [
    # (types, d_model, d_ff, engine switches): the one-launch FFNs with a grid barrier, the
    # small Q4_0 / Q8_0 FFN at SmolLM2-135M's layer.
    ((hayai_amd.Q4_0,) * 3, 576, 1536, {}),
    ((hayai_amd.Q8_0,) * 3, 576, 1536, {}),
]


@pytest.mark.parametrize("types,d_model,d_ff,env", BARRIER_CASES)
def test_graph_replays_grid_barrier_ffns(types, d_model, d_ff, env):
    # The barrier generation is kept on the device (an epoch the releasing workgroup
    # advances), so a graph of one-launch FFNs replays with unchanged arguments.  Several
    # barriers per replay (a chain of layers), eager launches between replays (the epoch
    # keeps counting across both), and every replay equal to the eager chain bit for bit:
    # the same kernel ran, not a fallback captured in its place.
    n = 3
    print(f"[case] graph grid-barrier ffn {types} {d_model}x{d_ff} {env}", flush=True)
    eng = engine_with_env(**env)
    try:
        t = types[0]
        gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, t)
        up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, t)
        down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, t)
        lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
        desc = eng.ffn_desc(types, d_model, d_ff, lay)
        packs, mats = [], []
        for l in range(n):
            wg = synth.matrix(t, d_ff, d_model, synth.seed_for(34, l, synth.GATE))
            wu = synth.matrix(t, d_ff, d_model, synth.seed_for(34, l, synth.UP))
            wd = synth.matrix(t, d_model, d_ff, synth.seed_for(34, l, synth.DOWN))
            p = eng.alloc(lay.total)
            p.write(wg, lay.gate_off)
            p.write(wu, lay.up_off)
            p.write(wd, lay.down_off)
            packs.append(p)
            mats.append((wg, wu, wd))
        x = synth.normal(synth.seed_for(34, 0, synth.ACT), d_model)
        xbuf = eng.upload(x)
        eager = [eng.alloc(4 * d_model) for _ in range(n)]
        chain(eng, desc, packs, xbuf, eager)
        eng.sync()
        y_eager = [b.read(np.float32, d_model) for b in eager]
        r0 = oracle.ffn(types, d_model, d_ff, *mats[0], x)
        assert np.max(np.abs(y_eager[0] - r0)) / np.max(np.abs(r0)) <= 1e-3

        outs = [eng.alloc(4 * d_model) for _ in range(n)]
        g = eng.capture(lambda: chain(eng, desc, packs, xbuf, outs))
        other = [eng.alloc(4 * d_model) for _ in range(n)]
        for rep in range(4):
            for b in outs:
                b.fill(0)
            g.launch()
            if rep % 2:
                chain(eng, desc, packs, xbuf, other)  # eager barriers right behind the replay
            eng.sync()
            for l in range(n):
                y = outs[l].read(np.float32, d_model)
                assert np.array_equal(y.view(np.uint32), y_eager[l].view(np.uint32)), f"replay {rep} layer {l}"
            if rep % 2:
                y = other[-1].read(np.float32, d_model)
                assert np.array_equal(y.view(np.uint32), y_eager[-1].view(np.uint32)), f"eager after replay {rep}"
        g.free()
    finally:
        eng.close()


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


def test_graph_refuses_buffer_operations(engine):
    # fills, copies, writes and reads would record memset/memcpy nodes (or synchronise)
    # inside the capture; they are refused and the engine stays usable
    print("[case] graph buffer operations", flush=True)
    a = engine.alloc(1024)
    b = engine.alloc(1024)
    host = np.arange(256, dtype=np.float32)
    for name, fn in (("fill", lambda: a.fill(0)), ("copy", lambda: a.copy_from(b, 1024)),
                     ("write", lambda: a.write(host)), ("read", lambda: a.read(np.float32, 256))):
        with pytest.raises(hayai_amd.HipError) as e:
            engine.capture(fn)
        assert e.value.status_name == "HH_ERR_INVALID", name
    a.write(host)
    b.copy_from(a, 1024)
    engine.sync()
    assert np.array_equal(b.read(np.float32, 256), host)


def test_graph_replay_after_workspace_growth():
    # A graph holds workspace addresses in its kernels' arguments.  Capture a Q6_K GEMV
    # (its x digits live in a workspace sized for n = 1024), then let a Q4_K_M batched FFN
    # grow that workspace (its per-token Q6_K GEMVs run at n = d_ff = 2048): replays must
    # still equal the eager GEMV, since the old allocation stays alive while the graph does.
    print("[case] graph replay after workspace growth", flush=True)
    eng = hayai_amd.HipEngine(0)
    try:
        m, n = 512, 1024
        w6 = synth.matrix(hayai_amd.Q6_K, m, n, 41)
        wbuf = eng.upload(w6)
        x = synth.normal(42, n)
        xbuf = eng.upload(x)
        y_eager = eng.alloc(4 * m)
        eng.gemv_dev(hayai_amd.Q6_K, m, n, wbuf, 0, xbuf, 0, y_eager, 0)
        eng.sync()
        ref = y_eager.read(np.float32, m)
        assert np.max(np.abs(ref - oracle.gemv(oracle.Q6_K, m, n, w6, x))) <= 1e-3 * np.max(np.abs(ref))
        y = eng.alloc(4 * m)
        g = eng.capture(lambda: eng.gemv_dev(hayai_amd.Q6_K, m, n, wbuf, 0, xbuf, 0, y, 0))
        g.launch()
        eng.sync()
        assert np.array_equal(y.read(np.float32, m).view(np.uint32), ref.view(np.uint32))

        d_model, d_ff, B = 1024, 2048, 8
        Q4, Q6 = hayai_amd.Q4_K, hayai_amd.Q6_K
        gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, Q4)
        up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, Q4)
        down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, Q6)
        lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
        pack = eng.alloc(lay.total)
        pack.write(synth.matrix(Q4, d_ff, d_model, 43), lay.gate_off)
        pack.write(synth.matrix(Q4, d_ff, d_model, 44), lay.up_off)
        pack.write(synth.matrix(Q6, d_model, d_ff, 45), lay.down_off)
        desc = eng.ffn_desc((Q4, Q4, Q6), d_model, d_ff, lay)
        xb = np.stack([synth.normal(46 + b, d_model) for b in range(B)])
        yb = eng.ffn_batched(desc, pack, 0, xb)  # grows the GEMV digit workspace
        assert np.all(np.isfinite(yb))

        for rep in range(3):
            y.fill(0)
            g.launch()
            eng.sync()
            assert np.array_equal(y.read(np.float32, m).view(np.uint32), ref.view(np.uint32)), f"replay {rep}"
            eng.ffn_batched(desc, pack, 0, xb)  # eager work between replays
        g.free()
        # with no graph left, the engine still runs the GEMV eagerly
        eng.gemv_dev(hayai_amd.Q6_K, m, n, wbuf, 0, xbuf, 0, y, 0)
        eng.sync()
        assert np.array_equal(y.read(np.float32, m).view(np.uint32), ref.view(np.uint32))
    finally:
        eng.close()
