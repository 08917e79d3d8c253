"""A model file through the whole path on the GPU: GGUF catalog -> load_layer_pack_into a
pinned streaming slot (io_uring) -> DMA to the device mirror -> the FFN op at the layer
pack's offsets, against the oracle on the tensors' bytes and against the same layer
uploaded directly (bit for bit)."""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import gguf, synth
from hayai_amd.gguf import GgufCatalog, write_gguf

pytestmark = pytest.mark.gpu
REL_TOL = 1e-3


def rel_err(y, ref):
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.fixture(scope="module")
def engine():
    eng = hayai_amd.HipEngine(0)
    yield eng
    eng.close()


@pytest.mark.parametrize("types,d_model,d_ff", [((12, 12, 14), 1024, 2048), ((12, 12, 12), 4096, 14336),
                                                ((16, 16, 16), 1024, 2048), ((2, 2, 2), 576, 1536)])
def test_ffn_from_gguf_file_through_pinned_slots(engine, tmp_path, types, d_model, d_ff):
    print(f"[case] gguf -> pinned slot -> ffn types={types} {d_model}x{d_ff}", flush=True)
    oracle.set_threads(min(16, oracle.max_threads()))
    tg, tu, td = types
    layers, want, tensors = 3, {}, []
    for l in range(layers):
        for name in ("attn_q", "attn_k", "attn_v", "attn_output"):
            tensors.append((f"blk.{l}.{name}.weight", (64, 64), 1, np.zeros(8192, np.uint8)))
        for name, t, mat, rows, cols in (("ffn_gate", tg, synth.GATE, d_ff, d_model),
                                         ("ffn_up", tu, synth.UP, d_ff, d_model),
                                         ("ffn_down", td, synth.DOWN, d_model, d_ff)):
            lo, hi = synth.SCALE_RANGE[t]
            w = synth.matrix(t, rows, cols, synth.seed_for(30, l, mat), lo, hi)
            tensors.append((f"blk.{l}.{name}.weight", (cols, rows), t, w))
            want[(l, name)] = w
    path = str(tmp_path / "m.gguf")
    write_gguf(path, [("general.architecture", "llama")], tensors)
    with GgufCatalog(path) as cat:
        lp = cat.layer_pack(0)
        lay = lp.ffn_layout()
        desc = engine.ffn_desc(types, d_model, d_ff, lay)
        st = hayai_amd.StreamingScratch(engine, lp.total, k_chunk=1, n_slots=2)
        xs = [synth.normal(synth.seed_for(30, l, synth.ACT), d_model) for l in range(layers)]
        xbuf, ybuf = engine.upload(np.concatenate(xs)), engine.alloc(4 * d_model * layers)
        for l in range(layers):
            lpl = cat.load_layer_pack(l, st.host_slot(l))
            assert lpl.ffn_layout() == lay
            st.dma(l, lay.gate_off, lay.down_off + lay.down_len - lay.gate_off)
            mirror, off = st.weight_bind(l)
            engine.ffn_dev(desc, mirror, off, xbuf, 4 * d_model * l, ybuf, 4 * d_model * l)
        ys = ybuf.read(np.float32, d_model * layers).reshape(layers, d_model)
        st.free()
    for l in range(layers):
        wg, wu, wd = want[(l, "ffn_gate")], want[(l, "ffn_up")], want[(l, "ffn_down")]
        ref = oracle.ffn(types, d_model, d_ff, wg, wu, wd, xs[l])
        assert rel_err(ys[l], ref) <= REL_TOL, (l, rel_err(ys[l], ref))
        # the same bytes uploaded directly at the same offsets: identical output
        pack = engine.alloc(lay.total)
        pack.write(wg, lay.gate_off)
        pack.write(wu, lay.up_off)
        pack.write(wd, lay.down_off)
        np.testing.assert_array_equal(engine.ffn(desc, pack, 0, xs[l]), ys[l])
        pack.free()
        print(f"  layer {l}: rel_err {rel_err(ys[l], ref):.2e}", flush=True)
