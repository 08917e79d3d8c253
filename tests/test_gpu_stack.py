"""GPU tests of hh_ffn_block_stack_dev: n FFN residual blocks back to back,
x_{l+1} = x_l + FFN_l(rms_norm(x_l, norm_l)) (ffn_apply, hybrid_infer.rs:883-936, layer after
layer).  Small Q4_0 / Q8_0 layers run every layer in one persistent launch (small_stack.hip,
tagged-word exchanges between workgroups); other layouts (all-Q4_K among them) run one ring
block per layer.  Each case is held against the oracle's block applied layer by layer, and
against the engine's own per-layer blocks."""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import synth

pytestmark = pytest.mark.gpu
REL_TOL = 1e-3
Q4_0, Q8_0, Q4_K = hayai_amd.Q4_0, hayai_amd.Q8_0, hayai_amd.Q4_K


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def make_stack(engine, types, d_model, d_ff, n_layers, cfg):
    """n_layers packs at a fixed stride in one buffer, plus one norm vector per layer."""
    tg, tu, td = types
    gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, tg)
    up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, tu)
    down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, td)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    stride = (lay.total + 255) // 256 * 256
    pack = engine.alloc(stride * n_layers)
    mats = []
    for l in range(n_layers):
        wg = synth.matrix(tg, d_ff, d_model, synth.seed_for(cfg, l, synth.GATE))
        wu = synth.matrix(tu, d_ff, d_model, synth.seed_for(cfg, l, synth.UP))
        wd = synth.matrix(td, d_model, d_ff, synth.seed_for(cfg, l, synth.DOWN))
        pack.write(wg, l * stride + lay.gate_off)
        pack.write(wu, l * stride + lay.up_off)
        pack.write(wd, l * stride + lay.down_off)
        mats.append((wg, wu, wd))
    rng = np.random.default_rng(cfg)
    norms = rng.uniform(0.5, 1.5, (n_layers, d_model)).astype(np.float32)
    return lay, stride, pack, mats, norms


STACK_CASES = [
    # (types, d_model, d_ff, n_layers): SmolLM2-135M's layer in Q4_0 and
    # Q8_0, 7 layers (more than the ring depth, not a multiple of it); a layer with fewer
    # rows than CUs (grid = min(d_model, d_ff)) and one layer only; the largest persistent
    # shape (64 blocks per row both ways); Q4_K layers (ring kernels, one block per layer)
    ((Q4_0,) * 3, 576, 1536, 7),
    ((Q8_0,) * 3, 576, 1536, 5),
    ((Q4_0,) * 3, 64, 128, 3),
    ((Q4_0,) * 3, 576, 1536, 1),
    ((Q4_0,) * 3, 2048, 2048, 2),
    # all-Q4_K (one ring block per layer): two and four waves per down row; the 8B shape of
    # BASELINE configs[1] (3 layers, and 1)
    ((Q4_K,) * 3, 1024, 2816, 3),
    ((Q4_K,) * 3, 2048, 8192, 4),
    ((Q4_K,) * 3, 4096, 14336, 3),
    ((Q4_K,) * 3, 4096, 14336, 1),
]


@pytest.mark.parametrize("types,d_model,d_ff,n_layers", STACK_CASES)
def test_ffn_block_stack_matches_oracle_chain(engine, types, d_model, d_ff, n_layers):
    print(f"[case] ffn block stack types={types} {d_model}x{d_ff} layers={n_layers}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    lay, stride, pack, mats, norms = make_stack(engine, types, d_model, d_ff, n_layers, 60 + n_layers)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    rng = np.random.default_rng(d_model * n_layers)
    x = (2.0 * rng.standard_normal(d_model)).astype(np.float32)
    eps = 1e-5
    ref = x.copy()
    for l in range(n_layers):
        ref = oracle.ffn_block(types, d_model, d_ff, *mats[l], norms[l], eps, ref)

    xb, nb, yb = engine.upload(x), engine.upload(norms), engine.alloc(4 * d_model)
    engine.ffn_block_stack_dev(desc, pack, 0, stride, n_layers, nb, 0, d_model, eps, xb, 0, yb, 0)
    engine.sync()
    y = yb.read(np.float32, d_model)
    assert np.isfinite(y).all()
    err = rel_err(y - x, ref - x)
    print(f"  rel_err of the FFN part vs the oracle chain {err:.3e}", flush=True)
    assert err <= REL_TOL, err

    # the engine's per-layer blocks (the same math, sums in another order)
    cb = engine.upload(x)
    for l in range(n_layers):
        engine.ffn_block_dev(desc, pack, l * stride, nb, 4 * l * d_model, eps, cb, 0, cb, 0)
    engine.sync()
    yc = cb.read(np.float32, d_model)
    assert rel_err(y - x, yc - x) <= 1e-4
    if types[0] == Q4_K:
        # all-Q4_K stacks run the ring blocks layer by layer: the same kernels, the same bits
        np.testing.assert_array_equal(y.view(np.uint32), yc.view(np.uint32))
    elif d_model >= 576:
        # the persistent small stack ran, not the per-layer blocks it falls back to: its RMSNorm
        # and row sums run in another order (the exchange wave's DPP sums against the norm
        # kernel's workgroup reduction), so over hundreds of outputs some differ in their last
        # bits
        assert not np.array_equal(y, yc)

    # deterministic across launches (the exchange tags advance), and in place (y = x)
    engine.ffn_block_stack_dev(desc, pack, 0, stride, n_layers, nb, 0, d_model, eps, xb, 0, yb, 0)
    engine.sync()
    np.testing.assert_array_equal(yb.read(np.float32, d_model).view(np.uint32), y.view(np.uint32))
    engine.ffn_block_stack_dev(desc, pack, 0, stride, n_layers, nb, 0, d_model, eps, xb, 0, xb, 0)
    engine.sync()
    np.testing.assert_array_equal(xb.read(np.float32, d_model).view(np.uint32), y.view(np.uint32))


def test_ffn_block_stack_shared_norm_and_offsets(engine):
    # norm_stride 0 reuses one norm vector; pack, norm, x and y at nonzero offsets
    types, d_model, d_ff, n_layers = (Q4_0,) * 3, 576, 1536, 4
    print(f"[case] ffn block stack shared norm {d_model}x{d_ff} layers={n_layers}", flush=True)
    lay, stride, pack, mats, norms = make_stack(engine, types, d_model, d_ff, n_layers, 71)
    big = engine.alloc(stride * (n_layers + 1))
    big.copy_from(pack, stride * n_layers, dst_off=stride)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    x = synth.normal(72, d_model)
    eps = 1e-6
    ref = x.copy()
    for l in range(n_layers):
        ref = oracle.ffn_block(types, d_model, d_ff, *mats[l], norms[0], eps, ref)
    nb = engine.alloc(4 * d_model + 64)
    nb.write(norms[0], 64)
    xb = engine.alloc(4 * d_model + 128)
    xb.write(x, 128)
    yb = engine.alloc(4 * d_model + 256)
    engine.ffn_block_stack_dev(desc, big, stride, stride, n_layers, nb, 64, 0, eps, xb, 128, yb, 256)
    engine.sync()
    y = yb.read(np.float32, d_model, 256)
    assert rel_err(y - x, ref - x) <= REL_TOL


def test_ffn_block_stack_rejects_bad_ranges(engine):
    types, d_model, d_ff, n_layers = (Q4_0,) * 3, 576, 1536, 2
    print("[case] ffn block stack validation", flush=True)
    lay, stride, pack, _, norms = make_stack(engine, types, d_model, d_ff, n_layers, 73)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    xb, nb, yb = engine.upload(synth.normal(74, d_model)), engine.upload(norms), engine.alloc(4 * d_model)
    for args in ((0, stride, 0, nb, 0, d_model),          # no layers
                 (0, stride, 3, nb, 0, d_model),          # a third layer past the pack
                 (0, stride, 2, nb, 0, 2 * d_model),      # layer 1's norm past the buffer
                 (0, 1 << 62, 2, nb, 0, d_model)):        # layer offset overflow
        off, st, n, norm, noff, nstr = args
        with pytest.raises(hayai_amd.HipError) as e:
            engine.ffn_block_stack_dev(desc, pack, off, st, n, norm, noff, nstr, 1e-5, xb, 0, yb, 0)
        assert e.value.status_name == "HH_ERR_INVALID", args
    engine.ffn_block_stack_dev(desc, pack, 0, stride, n_layers, nb, 0, d_model, 1e-5, xb, 0, yb, 0)
    engine.sync()
    assert np.isfinite(yb.read(np.float32, d_model)).all()


@pytest.mark.parametrize("types,d_model,d_ff,n_layers", [((Q4_0,) * 3, 576, 1536, 6), ((Q4_K,) * 3, 1024, 2816, 4)])
def test_ffn_block_stack_graph_replay(engine, types, d_model, d_ff, n_layers):
    # The persistent stacks' exchange tags come from an epoch on the device: a captured
    # stack replays with unchanged arguments, between eager stacks, bit for bit.
    print(f"[case] ffn block stack graph types={types} {d_model}x{d_ff} layers={n_layers}", flush=True)
    lay, stride, pack, _, norms = make_stack(engine, types, d_model, d_ff, n_layers, 75)
    desc = engine.ffn_desc(types, d_model, d_ff, lay)
    xb, nb = engine.upload(synth.normal(76, d_model)), engine.upload(norms)
    y_eager, yg, other = engine.alloc(4 * d_model), engine.alloc(4 * d_model), engine.alloc(4 * d_model)

    def run(y):
        engine.ffn_block_stack_dev(desc, pack, 0, stride, n_layers, nb, 0, d_model, 1e-5, xb, 0, y, 0)

    run(y_eager)
    engine.sync()
    ref = y_eager.read(np.float32, d_model)
    g = engine.capture(lambda: run(yg))
    for rep in range(4):
        yg.fill(0)
        g.launch()
        if rep % 2:
            run(other)
        engine.sync()
        np.testing.assert_array_equal(yg.read(np.float32, d_model).view(np.uint32), ref.view(np.uint32))
        if rep % 2:
            np.testing.assert_array_equal(other.read(np.float32, d_model).view(np.uint32), ref.view(np.uint32))
    g.free()
