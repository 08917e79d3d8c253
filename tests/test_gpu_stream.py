"""GPU tests of pinned-host ping-pong weight streaming (StreamingScratch analogue).

Reference: StreamingScratch (crates/hayai-opencl/src/hetero_scratch.rs:48-71,565-571,611-656,
781-849,853-925) with pinned host slots (memory.rs:72-147), driven per layer by the decode
loop: prepare_host_write -> fill the host slot -> DMA the FFN regions into the mirror ->
weight_bind -> FFN GEMVs on the mirror (stream_infer.rs:1665-1722,3752-3864).

The FFN of a streamed layer must equal, bit for bit, the same FFN run on a resident copy of
the layer (same kernels, same bytes): any DMA that overwrote a mirror slot before the FFN of
the layer it held had finished, or an FFN that read a slot before its DMA completed, shows
up as a mismatch.  No host synchronisation happens between layers, so the event ordering
alone is under test.  Two layers are also checked against the oracle (max rel err <= 1e-3).
"""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import synth

pytestmark = pytest.mark.gpu

T = hayai_amd.IQ2_XXS
D_MODEL, D_FF = 2048, 5632


def make_layers(n_layers, t=T, d_model=D_MODEL, d_ff=D_FF, cfg=5):
    gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, t)
    up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, t)
    down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, t)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    packs, mats = [], []
    for l in range(n_layers):
        wg = synth.matrix(t, d_ff, d_model, synth.seed_for(cfg, l, synth.GATE))
        wu = synth.matrix(t, d_ff, d_model, synth.seed_for(cfg, l, synth.UP))
        wd = synth.matrix(t, d_model, d_ff, synth.seed_for(cfg, l, synth.DOWN))
        p = np.zeros(lay.total, np.uint8)
        p[lay.gate_off:lay.gate_off + wg.size] = wg
        p[lay.up_off:lay.up_off + wu.size] = wu
        p[lay.down_off:lay.down_off + wd.size] = wd
        packs.append(p)
        mats.append((wg, wu, wd))
    return lay, packs, mats


def resident_outputs(engine, desc, lay, packs, xbuf, d_model):
    res = engine.alloc(lay.total * len(packs))
    for l, p in enumerate(packs):
        res.write(p, l * lay.total)
    ybuf = engine.alloc(4 * d_model * len(packs))
    for l in range(len(packs)):
        engine.ffn_dev(desc, res, l * lay.total, xbuf, 4 * d_model * l, ybuf, 4 * d_model * l)
    return ybuf.read(np.float32, d_model * len(packs)).reshape(len(packs), d_model)


def streamed_outputs(engine, desc, lay, packs, xbuf, d_model, k_chunk=1, n_slots=2):
    """The reference's decode order: stage layer 0; per layer, stage the next layer while
    the current one's FFN is enqueued on its mirror."""
    st = hayai_amd.StreamingScratch(engine, lay.total, k_chunk=k_chunk, n_slots=n_slots)
    ybuf = engine.alloc(4 * d_model * len(packs))

    def stage(l):
        st.host_slot(l)[:] = packs[l]
        for role in range(3):  # FFN regions one DMA each (dma_ffn_slices_mapped)
            off, ln = lay.ffn_region(role)
            st.dma(l, off, ln)

    ahead = n_slots - 1
    for l in range(min(ahead, len(packs))):
        stage(l)
    for l in range(len(packs)):
        if l + ahead < len(packs):
            stage(l + ahead)
        mirror, off = st.weight_bind(l)
        assert off == st.weight_offset(l, 0)
        engine.ffn_dev(desc, mirror, off, xbuf, 4 * d_model * l, ybuf, 4 * d_model * l)
    y = ybuf.read(np.float32, d_model * len(packs)).reshape(len(packs), d_model)
    st.free()
    return y


@pytest.mark.parametrize("k_chunk,n_slots", [(1, 2), (1, 3), (2, 2)])
def test_streamed_equals_resident(engine, k_chunk, n_slots):
    n_layers = 8
    print(f"[case] stream iq2_xxs {D_MODEL}x{D_FF} layers={n_layers} k_chunk={k_chunk} slots={n_slots}", flush=True)
    lay, packs, mats = make_layers(n_layers)
    desc = engine.ffn_desc((T, T, T), D_MODEL, D_FF, lay)
    xs = np.stack([synth.normal(synth.seed_for(5, l, synth.ACT), D_MODEL) for l in range(n_layers)])
    xbuf = engine.upload(xs)
    ref = resident_outputs(engine, desc, lay, packs, xbuf, D_MODEL)
    if k_chunk == 1:
        got = streamed_outputs(engine, desc, lay, packs, xbuf, D_MODEL, k_chunk, n_slots)
    else:
        # macro-chunk: a slot holds k_chunk consecutive layers; stage whole blocks
        st = hayai_amd.StreamingScratch(engine, lay.total, k_chunk=k_chunk, n_slots=n_slots)
        ybuf = engine.alloc(4 * D_MODEL * n_layers)
        blocks = n_layers // k_chunk

        def stage_block(b):
            for l in range(b * k_chunk, (b + 1) * k_chunk):
                st.host_slot(l)[:] = packs[l]
                st.dma(l)

        stage_block(0)
        for b in range(blocks):
            if b + 1 < blocks:
                stage_block(b + 1)
            for l in range(b * k_chunk, (b + 1) * k_chunk):
                mirror, off = st.weight_bind(l)
                assert off == (l % k_chunk) * lay.total
                engine.ffn_dev(desc, mirror, off, xbuf, 4 * D_MODEL * l, ybuf, 4 * D_MODEL * l)
        got = ybuf.read(np.float32, D_MODEL * n_layers).reshape(n_layers, D_MODEL)
        st.free()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    for l in (0, n_layers - 1):
        wg, wu, wd = mats[l]
        r = oracle.ffn((T, T, T), D_MODEL, D_FF, wg, wu, wd, xs[l])
        assert np.max(np.abs(got[l] - r)) / np.max(np.abs(r)) <= 1e-3


def test_slot_addressing(engine):
    # slot_for / weight_offset (hetero_scratch.rs:565-571,915-925)
    st = hayai_amd.StreamingScratch(engine, 4096, k_chunk=3, n_slots=2)
    for l in range(12):
        assert st.slot_for(l) == (l // 3) % 2
        assert st.weight_offset(l, 100) == (l % 3) * 4096 + 100
    st.free()
    st = hayai_amd.StreamingScratch(engine, 4096, k_chunk=0, n_slots=1)  # clamped to 1 and 2
    assert [st.slot_for(l) for l in range(4)] == [0, 1, 0, 1]
    st.free()


def test_bind_and_dma_validation(engine):
    st = hayai_amd.StreamingScratch(engine, 4096)
    with pytest.raises(hayai_amd.HipError) as e:
        st.weight_bind(0)  # nothing staged
    assert e.value.status_name == "HH_ERR_INVALID"
    st.host_slot(0)[:] = 7
    st.dma(0)
    st.weight_bind(0)
    with pytest.raises(hayai_amd.HipError):
        st.weight_bind(2)  # slot 0 holds layer 0, not 2
    with pytest.raises(hayai_amd.HipError):
        st.dma(1, 4000, 200)  # past the layer
    mirror, off = st.weight_bind(0)
    engine.sync()
    assert (mirror.read(np.uint8, 4096, off) == 7).all()
    st.free()


def test_stream_70b_full_layer(engine):
    # configs[4] at its real shape: 70B IQ2_XXS FFN layers (d_model 8192, d_ff 28672,
    # 181.7 MB per layer) through two pinned slots.  Every region is >= 32 MB, so each DMA
    # goes out as two halves on two copy streams.  Streamed == resident bit for bit, and
    # every layer against the oracle.
    n_layers, d_model, d_ff = 2, 8192, 28672
    print(f"[case] stream iq2_xxs 70B layer {d_model}x{d_ff} layers={n_layers}", flush=True)
    lay, packs, mats = make_layers(n_layers, d_model=d_model, d_ff=d_ff, cfg=5)
    desc = engine.ffn_desc((T, T, T), d_model, d_ff, lay)
    xs = np.stack([synth.normal(synth.seed_for(5, l, synth.ACT), d_model) for l in range(n_layers)])
    xbuf = engine.upload(xs)
    got = streamed_outputs(engine, desc, lay, packs, xbuf, d_model)
    ref = resident_outputs(engine, desc, lay, packs, xbuf, d_model)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    oracle.set_threads(min(16, oracle.max_threads()))
    try:
        for l in range(n_layers):
            r = oracle.ffn((T, T, T), d_model, d_ff, *mats[l], xs[l])
            err = np.max(np.abs(got[l] - r)) / np.max(np.abs(r))
            print(f"[case] layer {l} rel_err={err:.3e}", flush=True)
            assert err <= 1e-3
    finally:
        oracle.set_threads(1)


@pytest.mark.parametrize("split", [1, 0])
def test_large_dma_bytes(split, monkeypatch):
    # A DMA of 32 MB or more is split over two copy streams (HAYAI_HIP_DMA_SPLIT=1, the
    # default): an odd length at an odd offset, into the second layer of a two-layer slot,
    # must land byte for byte, with the switch on and off.
    monkeypatch.setenv("HAYAI_HIP_DMA_SPLIT", str(split))
    print(f"[case] large dma split={split}", flush=True)
    eng = hayai_amd.HipEngine(0)
    try:
        layer_bytes = 80 << 20
        st = hayai_amd.StreamingScratch(eng, layer_bytes, k_chunk=2, n_slots=2)
        off, length = 12345, (70 << 20) + 77
        for layer in (1, 2):  # slot 0 at in-slot offset layer_bytes, then slot 1 at 0
            pat = ((np.arange(layer_bytes, dtype=np.uint64) * (7 + layer)) % 251).astype(np.uint8)
            st.host_slot(layer)[:] = pat
            st.dma(layer, off, length)
            mirror, moff = st.weight_bind(layer)
            assert moff == (layer % 2) * layer_bytes
            eng.sync()
            back = mirror.read(np.uint8, length, moff + off)
            assert np.array_equal(back, pat[off:off + length]), f"layer {layer}"
        st.free()
    finally:
        eng.close()
