"""MoE routing and the grouped expert FFN on the GPU against the oracle.

Routing: route_experts + top_k_indices (crates/hayai-core/src/moe_infer.rs:852-934); the
known-answer cases are the reference's own tests (moe_infer.rs:1039-1121).  Selected ids must
be identical; weights go through the device expf, so they are compared to 1e-6 relative.
Expert FFN: the expert loop + combine of moe_infer.rs:342-455 against the oracle's
or_moe_token fed the same ids and weights, held to the FFN tolerance (1e-3).
"""
import numpy as np
import pytest

import hayai_amd
import oracle
from hayai_amd import synth

pytestmark = pytest.mark.gpu
Q4_K = 12
REL_TOL = 1e-3


def desc_for(engine, E, k, d_model=256, d_ff=256, **kw):
    return engine.moe_desc(d_model, d_ff, E, k, 0, (0, 0, 0), **kw)


@pytest.mark.parametrize("scores,k,kw,want", [
    ([0.1, 0.9, 0.3, 0.7, 0.2], 2, {}, [1, 3]),
    ([0.1, 0.9, 0.3, 0.7, 0.2], 2, {"norm_topk_prob": True}, [1, 3]),
    ([0.6, 0.5, 0.9, 0.1], 1, {"n_group": 2, "topk_group": 1, "gating": 1}, [0]),
    ([0.0, 1.0, -1.0], 2, {"gating": 1, "routed_scaling_factor": 2.0}, [1, 0]),
    ([0.5, 0.7, 0.7, 0.5, 0.7], 4, {}, [1, 2, 4, 0]),
])
def test_route_reference_cases(engine, scores, k, kw, want):
    s = np.array(scores, np.float32)
    d = desc_for(engine, s.size, k, **kw)
    ids, w = engine.route_experts(d, s)
    assert ids[0].tolist() == want
    ref_ids, ref_w = oracle.route_experts(s, k, **kw)
    assert ref_ids == want
    np.testing.assert_allclose(w[0], ref_w, rtol=1e-6, atol=1e-7)


def test_route_correction_bias_selects_but_weights_raw(engine):
    s = np.array([1.0, 0.5, 0.0, -1.0], np.float32)
    b = np.array([0, 10, 0, 0], np.float32)
    ids, w = engine.route_experts(desc_for(engine, 4, 1), s, bias=b)
    assert ids[0].tolist() == [1]
    ex = np.exp(s.astype(np.float64))
    assert abs(w[0][0] - ex[1] / ex.sum()) < 1e-5


@pytest.mark.parametrize("E,k,kw,levels", [
    (128, 8, {"norm_topk_prob": True}, None),                       # Qwen3-MoE
    (128, 8, {"norm_topk_prob": True}, 7),                          # many ties
    (256, 8, {"n_group": 8, "topk_group": 4, "gating": 1, "norm_topk_prob": True,
              "routed_scaling_factor": 2.5}, None),                 # DeepSeek-V3 style
    (256, 8, {"n_group": 8, "topk_group": 4, "gating": 1}, 5),
    (64, 6, {"n_group": 4, "topk_group": 1}, None),
    (16, 64, {}, None),                                             # top_k > experts
    (16, 12, {"n_group": 4, "topk_group": 2}, None),                # top_k > candidates
    (512, 64, {"routed_scaling_factor": 0.5}, None),
])
def test_route_matches_oracle(engine, E, k, kw, levels):
    T = 64
    rng = np.random.default_rng(E * 131 + k)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if levels:
        logits = (np.round(logits * levels / 3) / levels).astype(np.float32)
    bias = None
    if kw.get("gating") == 1:
        bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    d = desc_for(engine, E, k, **kw)
    ids, w = engine.route_experts(d, logits, bias=bias)
    for t in range(T):
        rid, rw = oracle.route_experts(logits[t], k, bias=bias, **kw)
        n = len(rid)
        assert ids[t, :n].tolist() == rid, t
        assert (ids[t, n:] == -1).all() and (w[t, n:] == 0).all()
        np.testing.assert_allclose(w[t, :n], rw, rtol=2e-6, atol=1e-8)


def make_experts(engine, E, d_model, d_ff, seed):
    rin = hayai_amd.row_bytes(Q4_K, d_model)
    rff = hayai_amd.row_bytes(Q4_K, d_ff)
    g_off, u_off, d_off = 0, d_ff * rin, 2 * d_ff * rin
    stride = 2 * d_ff * rin + d_model * rff
    buf = engine.alloc(E * stride)
    lo, hi = synth.SCALE_RANGE[Q4_K]
    for e in range(E):
        for mat, off, rows, cols in ((synth.GATE, g_off, d_ff, d_model), (synth.UP, u_off, d_ff, d_model),
                                     (synth.DOWN, d_off, d_model, d_ff)):
            engine.synth_weights_dev(Q4_K, buf, e * stride + off, rows * cols // 256,
                                     synth.seed_for(seed, e, mat), lo, hi)
    host = buf.read(np.uint8, E * stride)
    return buf, host, stride, (g_off, u_off, d_off)


@pytest.mark.parametrize("E,k,d_model,d_ff,T", [
    (128, 8, 2048, 768, 1),    # config 4 at one token: 128 experts, routing inside the ring kernels
    (32, 8, 2048, 768, 1),     # Qwen3-30B-A3B expert shape (one token: the ring kernels)
    (32, 8, 2048, 768, 5),
    (8, 2, 4096, 1024, 1),     # one token, 64 lanes per gate/up row
    (16, 4, 1024, 512, 1),     # one token, 4 gate/up rows per wave item
    (8, 2, 4096, 1024, 3),     # wider rows: 64-lane teams, several units per lane on down
    (16, 4, 1024, 512, 2),
    (128, 8, 2048, 768, 32),   # config 4 at 32 tokens: the grouped gather-GEMV
    (4, 2, 1024, 512, 40),     # ~20 tokens per expert: several LDS passes per expert
])
def test_moe_ffn_matches_oracle(engine, E, k, d_model, d_ff, T):
    oracle.set_threads(min(16, oracle.max_threads()))
    print(f"[case] moe E={E} k={k} {d_model}x{d_ff} T={T}", flush=True)
    buf, host, stride, offs = make_experts(engine, E, d_model, d_ff, 40 + E)
    d = engine.moe_desc(d_model, d_ff, E, k, stride, offs, norm_topk_prob=True)
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    x = synth.normal(synth.seed_for(4, T, synth.ACT), T * d_model).reshape(T, d_model)
    lb, xb = engine.upload(logits), engine.upload(x)
    ids_b, w_b = engine.alloc(4 * T * k), engine.alloc(4 * T * k)
    y1, y2 = engine.alloc(4 * T * d_model), engine.alloc(4 * T * d_model)
    engine.route_experts_dev(d, lb, 0, None, 0, T, ids_b, 0, w_b, 0)
    engine.moe_ffn_dev(d, buf, 0, xb, 0, T, ids_b, 0, w_b, 0, y1, 0)
    engine.moe_dev(d, buf, 0, lb, 0, None, 0, xb, 0, T, y2, 0)
    ids = ids_b.read(np.int32, T * k).reshape(T, k)
    w = w_b.read(np.float32, T * k).reshape(T, k)
    Y = y1.read(np.float32, T * d_model).reshape(T, d_model)
    np.testing.assert_array_equal(Y, y2.read(np.float32, T * d_model).reshape(T, d_model))
    for t in range(T):
        rid, _ = oracle.route_experts(logits[t], k, norm_topk_prob=True)
        assert ids[t].tolist() == rid
        ref = oracle.moe_token(Q4_K, d_model, d_ff, host, stride, offs, ids[t], w[t], x[t])
        err = float(np.max(np.abs(Y[t] - ref)) / np.max(np.abs(ref)))
        print(f"  token {t}: rel err {err:.3e}", flush=True)
        assert err <= REL_TOL


@pytest.mark.parametrize("T", [1, 5, 20])
def test_moe_shared_expert_matches_oracle(engine, T):
    # The always-active shared expert (moe_infer.rs:456-493) after the routed experts, weight
    # 1: one token on the ring kernels (down adds into y), several in passes of <= 16 tokens on
    # the f16 MFMA kernels then an add; against the oracle's routed loop + or_moe_shared, in
    # both calls (routing on the device, and ids/weights given)
    E, k, d_model, d_ff, sdf = 16, 4, 2048, 768, 1536
    oracle.set_threads(min(16, oracle.max_threads()))
    print(f"[case] moe + shared expert E={E} k={k} {d_model}x{d_ff} shared {sdf} T={T}", flush=True)
    rin, rsf = hayai_amd.row_bytes(Q4_K, d_model), hayai_amd.row_bytes(Q4_K, sdf)
    buf0, host, stride, offs = make_experts(engine, E, d_model, d_ff, 90)
    base = E * stride
    s_offs = (base, base + sdf * rin, base + 2 * sdf * rin)
    buf = engine.alloc(base + 2 * sdf * rin + d_model * rsf)
    buf.copy_from(buf0, base)
    lo, hi = synth.SCALE_RANGE[Q4_K]
    for mat, off, rows, cols in ((synth.GATE, s_offs[0], sdf, d_model), (synth.UP, s_offs[1], sdf, d_model),
                                 (synth.DOWN, s_offs[2], d_model, sdf)):
        engine.synth_weights_dev(Q4_K, buf, off, rows * cols // 256, synth.seed_for(91, 0, mat), lo, hi)
    sg = buf.read(np.uint8, sdf * rin, s_offs[0])
    su = buf.read(np.uint8, sdf * rin, s_offs[1])
    sd = buf.read(np.uint8, d_model * rsf, s_offs[2])
    d = engine.moe_desc(d_model, d_ff, E, k, stride, offs, norm_topk_prob=True, shared=(sdf, s_offs))
    rng = np.random.default_rng(T)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    x = synth.normal(synth.seed_for(9, T, synth.ACT), T * d_model).reshape(T, d_model)
    lb, xb = engine.upload(logits), engine.upload(x)
    ids_b, w_b = engine.alloc(4 * T * k), engine.alloc(4 * T * k)
    y1, y2 = engine.alloc(4 * T * d_model), engine.alloc(4 * T * d_model)
    engine.moe_dev(d, buf, 0, lb, 0, None, 0, xb, 0, T, y1, 0)
    engine.route_experts_dev(d, lb, 0, None, 0, T, ids_b, 0, w_b, 0)
    engine.moe_ffn_dev(d, buf, 0, xb, 0, T, ids_b, 0, w_b, 0, y2, 0)
    Y1 = y1.read(np.float32, T * d_model).reshape(T, d_model)
    Y2 = y2.read(np.float32, T * d_model).reshape(T, d_model)
    np.testing.assert_array_equal(Y1, Y2)
    ids = ids_b.read(np.int32, T * k).reshape(T, k)
    w = w_b.read(np.float32, T * k).reshape(T, k)
    for t in range(T):
        ref = oracle.moe_token(Q4_K, d_model, d_ff, host, stride, offs, ids[t], w[t], x[t], shared=(sdf, sg, su, sd))
        routed = oracle.moe_token(Q4_K, d_model, d_ff, host, stride, offs, ids[t], w[t], x[t])
        err = float(np.max(np.abs(Y1[t] - ref)) / np.max(np.abs(ref)))
        # the shared expert moves the output (a path that skipped it would fail here)
        assert float(np.max(np.abs(ref - routed)) / np.max(np.abs(ref))) > 50 * REL_TOL
        if t in (0, T - 1):
            print(f"  token {t}: rel err {err:.3e}", flush=True)
        assert err <= REL_TOL


def test_moe_empty_slots_contribute_nothing(engine):
    E, k, d_model, d_ff = 8, 3, 1024, 512
    buf, host, stride, offs = make_experts(engine, E, d_model, d_ff, 77)
    d = engine.moe_desc(d_model, d_ff, E, k, stride, offs)
    x = synth.normal(5, d_model)
    xb = engine.upload(x)
    y = engine.alloc(4 * d_model)
    ids = engine.upload(np.array([3, -1, 6], np.int32))
    w = engine.upload(np.array([0.25, 0.5, 0.75], np.float32))
    engine.moe_ffn_dev(d, buf, 0, xb, 0, 1, ids, 0, w, 0, y, 0)
    got = y.read(np.float32, d_model)
    ref = oracle.moe_token(Q4_K, d_model, d_ff, host, stride, offs, [3, 6], [0.25, 0.75], x)
    assert float(np.max(np.abs(got - ref)) / np.max(np.abs(ref))) <= REL_TOL


def test_moe_rejects_bad_descriptors(engine):
    E, k, d_model, d_ff = 4, 2, 512, 256
    buf, _, stride, offs = make_experts(engine, E, d_model, d_ff, 3)
    xb, y = engine.upload(synth.normal(1, d_model)), engine.alloc(4 * d_model)
    lb = engine.upload(np.zeros(E, np.float32))
    bad = [
        engine.moe_desc(d_model, d_ff, E, k, stride, offs, ggml_type=2),    # not Q4_K
        engine.moe_desc(d_model, d_ff, E, 65, stride, offs),                # top_k > 64
        engine.moe_desc(d_model, d_ff, E + 1, k, stride, offs),             # experts past the buffer
        engine.moe_desc(d_model, d_ff, E, k, stride + 8, offs),             # misaligned stride
        engine.moe_desc(d_model, 300, E, k, stride, offs),                  # d_ff not a block multiple
        engine.moe_desc(d_model, d_ff, E, k, stride, offs, shared=(512, (E * stride, 0, 0))),  # shared past the end
        engine.moe_desc(d_model, d_ff, E, k, stride, offs, shared=(300, (0, 0, 0))),  # shared d_ff not a block multiple
    ]
    for d in bad:
        with pytest.raises(hayai_amd.HipError):
            engine.moe_dev(d, buf, 0, lb, 0, None, 0, xb, 0, 1, y, 0)


def test_moe_grouped_matches_per_token_path_and_skips_empty_slots(engine):
    # Several tokens with some empty slots (id -1, or out of range): the grouped kernels give
    # the per-(token, expert) kernels' result within tolerance and ignore the empty slots.
    import os
    E, k, d_model, d_ff, T = 16, 4, 2048, 768, 6
    print(f"[case] moe grouped vs per-token E={E} k={k} T={T}", flush=True)
    buf, host, stride, offs = make_experts(engine, E, d_model, d_ff, 91)
    d = engine.moe_desc(d_model, d_ff, E, k, stride, offs)
    rng = np.random.default_rng(11)
    ids = rng.integers(0, E, (T, k)).astype(np.int32)
    for t in range(T):  # distinct experts per token, as routing gives
        ids[t] = rng.permutation(E)[:k]
    ids[1, 2] = -1
    ids[4, 0] = E + 3
    w = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    x = synth.normal(17, T * d_model).reshape(T, d_model)
    xb, ib, wb, y1 = engine.upload(x), engine.upload(ids), engine.upload(w), engine.alloc(4 * T * d_model)
    engine.moe_ffn_dev(d, buf, 0, xb, 0, T, ib, 0, wb, 0, y1, 0)
    Y = y1.read(np.float32, T * d_model).reshape(T, d_model)
    old = os.environ.get("HAYAI_HIP_MOE_GROUPED")
    os.environ["HAYAI_HIP_MOE_GROUPED"] = "0"
    try:
        plain = hayai_amd.HipEngine(0)
    finally:
        if old is None:
            del os.environ["HAYAI_HIP_MOE_GROUPED"]
        else:
            os.environ["HAYAI_HIP_MOE_GROUPED"] = old
    try:
        pb = plain.alloc(buf.nbytes)
        pb.write(host)
        d2 = plain.moe_desc(d_model, d_ff, E, k, stride, offs)
        y2 = plain.alloc(4 * T * d_model)
        plain.moe_ffn_dev(d2, pb, 0, plain.upload(x), 0, T, plain.upload(ids), 0, plain.upload(w), 0, y2, 0)
        Y2 = y2.read(np.float32, T * d_model).reshape(T, d_model)
    finally:
        plain.close()
    for t in range(T):
        keep = [(int(e), float(v)) for e, v in zip(ids[t], w[t]) if 0 <= e < E]
        ref = oracle.moe_token(Q4_K, d_model, d_ff, host, stride, offs, [e for e, _ in keep], [v for _, v in keep], x[t])
        for got in (Y[t], Y2[t]):
            assert float(np.max(np.abs(got - ref)) / np.max(np.abs(ref))) <= REL_TOL


def _engine_with_env(**env):
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


@pytest.mark.parametrize("T", [512, 513])
def test_moe_grouped_at_the_pair_limit(engine, T):
    # 512 tokens x top-8 = 4096 (token, slot) pairs, the most the grouped kernels take in one
    # call (every expert active, ~32 pairs each: several LDS passes per expert, records and
    # rank masks at full size); 513 tokens go to the per-(token, expert) kernels instead.
    # Routed on the GPU (hh_moe_dev) and from given ids (hh_moe_ffn_dev): bit-identical, and
    # each token against the oracle.
    E, k, d_model, d_ff = 128, 8, 256, 256
    oracle.set_threads(min(16, oracle.max_threads()))
    print(f"[case] moe pair limit E={E} k={k} {d_model}x{d_ff} T={T}", flush=True)
    buf, host, stride, offs = make_experts(engine, E, d_model, d_ff, 333)
    d = engine.moe_desc(d_model, d_ff, E, k, stride, offs, norm_topk_prob=True)
    rng = np.random.default_rng(T)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    x = synth.normal(synth.seed_for(6, T, synth.ACT), T * d_model).reshape(T, d_model)
    lb, xb = engine.upload(logits), engine.upload(x)
    ids_b, w_b = engine.alloc(4 * T * k), engine.alloc(4 * T * k)
    y1, y2 = engine.alloc(4 * T * d_model), engine.alloc(4 * T * d_model)
    engine.route_experts_dev(d, lb, 0, None, 0, T, ids_b, 0, w_b, 0)
    engine.moe_ffn_dev(d, buf, 0, xb, 0, T, ids_b, 0, w_b, 0, y1, 0)
    engine.moe_dev(d, buf, 0, lb, 0, None, 0, xb, 0, T, y2, 0)
    ids = ids_b.read(np.int32, T * k).reshape(T, k)
    w = w_b.read(np.float32, T * k).reshape(T, k)
    Y = y1.read(np.float32, T * d_model).reshape(T, d_model)
    np.testing.assert_array_equal(Y, y2.read(np.float32, T * d_model).reshape(T, d_model))
    assert len(np.unique(ids)) == E  # every expert has pairs
    worst = 0.0
    for t in range(T):
        ref = oracle.moe_token(Q4_K, d_model, d_ff, host, stride, offs, ids[t], w[t], x[t])
        worst = max(worst, float(np.max(np.abs(Y[t] - ref)) / np.max(np.abs(ref))))
    print(f"  worst token rel err {worst:.3e}", flush=True)
    assert worst <= REL_TOL
