"""Batched GEMV / FFN on the matrix cores against the oracle.

ggml_gemv_batched_q4_k (crates/hayai-opencl/src/compute.rs:179-257) computes B GEMVs that
share W; execute_quant_gemv_batched (crates/hayai-core/src/orchestrator.rs:240-269) runs
other types token by token.  Two matrix-core paths:
- 17..64 tokens per pass (at 16 tokens the f16 kernels are faster,
  HAYAI_HIP_MMI_MIN=16 moves 16 onto this path): activations quantized to int8 per 32-element
  block, their exact products with sc * q on the matrix cores (q4k_mmi.hip); parity against
  the oracle fed the same quantized activations (oracle.dequant_act_q8 / oracle.ffn_q8), the
  quantization's own error printed beside it;
- 2..16 tokens: f16 operands with f32-level accuracy, against the oracle's f32 restatement.
Both are held to the FFN tolerance (max |y - ref| / max |ref| <= 1e-3 per token).  The int8
path's distance from the f32-activation result (the quantization itself, which configs[2]
prescribes and the public contract states) is bounded too: QERR_GEMM for a GEMM, QERR_FFN for
the FFN (h is heavy-tailed, so its per-block quantization costs more); measured 0.7-1.9% and
3-13% of max|y|, so a wrong prep scale, rounding or clamp (errors of tens of percent) fails.
"""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import synth

pytestmark = pytest.mark.gpu
REL_TOL = 1e-3
QERR_GEMM = 0.04
QERR_FFN = 0.25
Q4_0, Q4_K = 2, 12


def rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def per_token_err(Y, R):
    return max(rel_err(Y[b], R[b]) for b in range(Y.shape[0]))


def int8_tokens(batch):
    """Which tokens go through the int8 path: passes of up to 64 tokens, those of 17 or more."""
    on = np.zeros(batch, bool)
    for b0 in range(0, batch, 64):
        nb = min(64, batch - b0)
        on[b0:b0 + nb] = nb >= 17
    return on


def batched_ref(t, m, n, w, X):
    """Per token: the oracle GEMV of the activation the path computes with."""
    on = int8_tokens(X.shape[0])
    Xq = np.stack([oracle.dequant_act_q8(X[b]) if on[b] else X[b] for b in range(X.shape[0])])
    return oracle.gemv_batched(t, m, n, w, Xq)


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.set_threads(min(16, oracle.max_threads()))


def test_reference_batched_fixture(engine):
    # compute.rs:1648-1670: m=32, n=256, batch=3, bytes (i*131+17)&0x1F, inputs i*0.003-0.2
    m, n, batch = 32, 256, 3
    w = ((np.arange(m * 144) * 131 + 17) & 0x1F).astype(np.uint8)
    x = (np.arange(batch * n, dtype=np.float32) * np.float32(0.003) - np.float32(0.2)).astype(np.float32)
    y = engine.ggml_gemv_batched_q4_k(m, n, w, x, batch)
    ref = oracle.gemv_batched(Q4_K, m, n, w, x.reshape(batch, n)).reshape(-1)
    assert np.max(np.abs(y - ref)) < 1e-3
    assert per_token_err(y.reshape(batch, m), ref.reshape(batch, m)) <= REL_TOL


@pytest.mark.parametrize("m,n,batch", [
    (14336, 4096, 2), (14336, 4096, 4), (14336, 4096, 16), (14336, 4096, 17), (14336, 4096, 64),
    (4096, 14336, 16), (4096, 14336, 64),   # down shape: superblocks split over workgroups
    (4096, 14336, 33), (768, 2048, 8), (100, 512, 5), (48, 256, 70),  # ragged rows, > 64 tokens
])
def test_q4_k_batched_matches_oracle(engine, m, n, batch):
    print(f"[case] batched q4_k m={m} n={n} batch={batch}", flush=True)
    w = synth.matrix(Q4_K, m, n, synth.seed_for(3, batch, m))
    X = synth.normal(synth.seed_for(3, batch, n), batch * n).reshape(batch, n)
    Y = engine.ggml_gemv_batched_q4_k(m, n, w, X, batch).reshape(batch, m)
    R = batched_ref(Q4_K, m, n, w, X)
    err = per_token_err(Y, R)
    qerr = per_token_err(Y, oracle.gemv_batched(Q4_K, m, n, w, X))
    print(f"  per-token max rel err {err:.3e} (vs f32 activations: {qerr:.3e}, "
          f"int8 tokens {int(int8_tokens(batch).sum())})", flush=True)
    assert np.isfinite(Y).all()
    assert err <= REL_TOL
    assert qerr <= (QERR_GEMM if int8_tokens(batch).any() else REL_TOL), qerr


def test_batched_is_deterministic_and_batch1_is_gemv(engine):
    m, n, batch = 4096, 14336, 16
    w = synth.matrix(Q4_K, m, n, 91)
    X = synth.normal(92, batch * n).reshape(batch, n)
    a = engine.ggml_gemv_batched_q4_k(m, n, w, X, batch)
    b = engine.ggml_gemv_batched_q4_k(m, n, w, X, batch)
    np.testing.assert_array_equal(a, b)
    y1 = engine.ggml_gemv_batched_q4_k(m, n, w, X[:1], 1)
    np.testing.assert_array_equal(y1, engine.ggml_gemv_q4_k(m, n, w, X[0]))
    assert engine.ggml_gemv_batched_q4_k(m, n, w, X[:0], 0).size == 0


def test_other_types_run_per_token(engine):
    m, n, batch = 1536, 576, 3
    w = synth.matrix(Q4_0, m, n, 5)
    X = synth.normal(6, batch * n).reshape(batch, n)
    Y = engine.ggml_gemv_batched(Q4_0, m, n, w, X, batch).reshape(batch, m)
    for b in range(batch):
        np.testing.assert_array_equal(Y[b], engine.ggml_gemv_q4_0(m, n, w, X[b]))


def test_batched_dev_offsets(engine):
    m, n, batch = 2048, 768, 8
    rb = hayai_amd.row_bytes(Q4_K, n)
    w = synth.matrix(Q4_K, m, n, 31)
    X = synth.normal(32, batch * n).reshape(batch, n)
    wbuf = engine.alloc(256 + m * rb)
    wbuf.write(w, 256)
    xbuf = engine.alloc(64 + X.nbytes)
    xbuf.write(X, 64)
    ybuf = engine.alloc(128 + 4 * batch * m)
    engine.gemv_batched_dev(Q4_K, m, n, wbuf, 256, xbuf, 64, batch, ybuf, 128)
    Y = ybuf.read(np.float32, batch * m, 128).reshape(batch, m)
    assert per_token_err(Y, batched_ref(Q4_K, m, n, w, X)) <= REL_TOL
    with pytest.raises(hayai_amd.HipError):
        engine.gemv_batched_dev(Q4_K, m, n, wbuf, 256, xbuf, 64, batch + 1, ybuf, 128)  # x too short


def make_pack(engine, types, d_model, d_ff, cfg):
    tg, tu, td = types
    gate = hayai_amd.QuantMatrix("ffn_gate", d_model, d_ff, tg)
    up = hayai_amd.QuantMatrix("ffn_up", d_model, d_ff, tu)
    down = hayai_amd.QuantMatrix("ffn_down", d_ff, d_model, td)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    wg = synth.matrix(tg, d_ff, d_model, synth.seed_for(cfg, 0, synth.GATE))
    wu = synth.matrix(tu, d_ff, d_model, synth.seed_for(cfg, 0, synth.UP))
    wd = synth.matrix(td, d_model, d_ff, synth.seed_for(cfg, 0, synth.DOWN))
    pack = engine.alloc(lay.total)
    pack.write(wg, lay.gate_off)
    pack.write(wu, lay.up_off)
    pack.write(wd, lay.down_off)
    return lay, (wg, wu, wd), pack


@pytest.mark.parametrize("types,d_model,d_ff,batch,act", [
    ((12, 12, 12), 4096, 14336, 4, 0), ((12, 12, 12), 4096, 14336, 16, 0), ((12, 12, 12), 4096, 14336, 64, 0),
    ((12, 12, 12), 2048, 768, 32, 0), ((12, 12, 12), 1024, 2048, 9, 1), ((2, 2, 2), 576, 1536, 3, 0),
    ((12, 12, 12), 8192, 1024, 40, 1),  # three token tiles (run as four), d_model past the LDS stage ring
])
def test_ffn_batched_matches_oracle(engine, types, d_model, d_ff, batch, act):
    print(f"[case] ffn batched types={types} {d_model}x{d_ff} batch={batch} act={act}", flush=True)
    lay, (wg, wu, wd), pack = make_pack(engine, types, d_model, d_ff, 30 + batch)
    desc = engine.ffn_desc(types, d_model, d_ff, lay, act)
    X = synth.normal(synth.seed_for(3, batch, synth.ACT), batch * d_model).reshape(batch, d_model)
    Y = engine.ffn_batched(desc, pack, 0, X)
    on = int8_tokens(batch) if types == (12, 12, 12) else np.zeros(batch, bool)
    R = np.stack([(oracle.ffn_q8 if on[b] else oracle.ffn)(types, d_model, d_ff, wg, wu, wd, X[b], act=act)
                  for b in range(batch)])
    err = per_token_err(Y, R)
    R32 = np.stack([oracle.ffn(types, d_model, d_ff, wg, wu, wd, X[b], act=act) for b in range(batch)])
    qerr = per_token_err(Y, R32)
    print(f"  per-token max rel err {err:.3e} (vs f32 activations: {qerr:.3e})", flush=True)
    assert err <= REL_TOL
    assert qerr <= (QERR_FFN if on.any() else REL_TOL), qerr
    if types == (2, 2, 2):
        for b in range(batch):  # non-Q4_K formats: the single-token op per token
            np.testing.assert_array_equal(Y[b], engine.ffn(desc, pack, 0, X[b]))


@pytest.mark.parametrize("batch", [16, 40, 64])
def test_int8_path_off_keeps_f32_activations(monkeypatch, batch):
    # HAYAI_HIP_MMQ=0: 17..64 tokens run one token at a time on the batch-1 kernels (16 stay
    # on the f16 weight-stream MFMA kernels), held to the oracle fed the original f32
    # activations: no int8 activation quantization on this path
    print(f"[case] batched without int8 batch={batch}", flush=True)
    monkeypatch.setenv("HAYAI_HIP_MMQ", "0")
    eng = hayai_amd.HipEngine(0)
    try:
        m, n = 4096, 14336
        w = synth.matrix(Q4_K, m, n, 71)
        X = synth.normal(72 + batch, batch * n).reshape(batch, n)
        Y = eng.ggml_gemv_batched_q4_k(m, n, w, X, batch).reshape(batch, m)
        assert per_token_err(Y, oracle.gemv_batched(Q4_K, m, n, w, X)) <= REL_TOL
    finally:
        eng.close()


@pytest.mark.parametrize("m,n", [(14336, 4096), (4096, 14336), (300, 768)])
def test_int8_path_at_16_tokens(monkeypatch, m, n):
    # HAYAI_HIP_MMI_MIN=16: one 16-token tile on the int8-activation kernels (whole stages in
    # LDS for the 8B shapes, ragged rows for 300), held to the quantized-activation oracle
    print(f"[case] int8 batched at 16 tokens m={m} n={n}", flush=True)
    monkeypatch.setenv("HAYAI_HIP_MMI_MIN", "16")
    eng = hayai_amd.HipEngine(0)
    try:
        w = synth.matrix(Q4_K, m, n, 81)
        X = synth.normal(82, 16 * n).reshape(16, n)
        Y = eng.ggml_gemv_batched_q4_k(m, n, w, X, 16).reshape(16, m)
        Xq = np.stack([oracle.dequant_act_q8(X[b]) for b in range(16)])
        err = per_token_err(Y, oracle.gemv_batched(Q4_K, m, n, w, Xq))
        print(f"  per-token max rel err {err:.3e}", flush=True)
        assert err <= REL_TOL
        # the FFN at 16 tokens: gate/up with whole rows of x in LDS, h quantized in-kernel
        if m == 14336:
            lay, (wg, wu, wd), pack = make_pack(eng, (Q4_K,) * 3, n, m, 77)
            desc = eng.ffn_desc((Q4_K,) * 3, n, m, lay, 0)
            Xf = synth.normal(83, 16 * n).reshape(16, n)
            Yf = eng.ffn_batched(desc, pack, 0, Xf)
            R = np.stack([oracle.ffn_q8((Q4_K,) * 3, n, m, wg, wu, wd, Xf[b]) for b in range(16)])
            assert per_token_err(Yf, R) <= REL_TOL
    finally:
        eng.close()
