#!/usr/bin/env python3
"""Benchmark of the FFN GEMV hot path on one MI355X (BASELINE.json metric).

Workload: Llama-3-8B-shaped SwiGLU FFN, d_model=4096,
d_ff=14336, 32 layers resident in HBM, batch 1, gate/up/down in Q4_K.  One step = one
token through the FFN of all 32 layers (hh_ffn_dev per layer: the ring gate/up kernel, which
writes h as int8 digits, then the ring down kernel), all on the engine's compute stream.
Inputs are synthetic (seeded splitmix64 Q4_K blocks generated on the device, N(0,1) f32
activations per layer) and are resident in HBM before the timed region starts.

The step is timed eagerly (one dispatch per kernel; value) and also as a HIP graph of the
same 32-layer step captured once and replayed (hh_graph_*), reported beside it.
value = algorithmic bytes per step / time per step, where algorithmic bytes per layer =
packed weights read once (99,090,432 B) + x in (16,384 B) + y out (16,384 B); the d_ff
intermediate is excluded.  FFN tok/s = 1 / time per step.

roofline: the dominant kernel, the ring gate/up kernel (66 MB of the layer's 99 MB), timed
with HIP events on the compute stream around a region of its launches alone (32 layers x
50, back to back): achieved = its algorithmic bytes (W_gate + W_up + x + h as f32) / time per
launch.  traffic = HBM bytes per launch of that kernel from
rocprofv3 FETCH_SIZE / WRITE_SIZE passes (each scaled by what the counter reads for a
256 MiB device copy, --copy-calibration), read from profiles/ when present.  The down kernel
is timed the same way and reported beside it.
cpu_baseline: the oracle's fp32 restatement of hayai-model's gemv_q4_k FFN (oracle/,
OpenMP over rows) on a bounded sample of the same layers, host cores.
configs: the other BASELINE.json configs in compact form (compact_configs), each with its own
roofline, timed in the same run (--no-configs skips them).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

D_MODEL, D_FF, LAYERS = 4096, 14336, 32
Q4_K = 12
PEAK_HBM_GBS = 8000.0
CONFIG_ID = 2
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gu_ring_n_8b_bs1_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_bytes() -> int:
    import hayai_amd

    w = 2 * D_FF * hayai_amd.row_bytes(Q4_K, D_MODEL) + D_MODEL * hayai_amd.row_bytes(Q4_K, D_FF)
    return w + 4 * D_MODEL + 4 * D_MODEL


def gateup_bytes() -> int:
    import hayai_amd

    return 2 * D_FF * hayai_amd.row_bytes(Q4_K, D_MODEL) + 4 * D_MODEL + 4 * D_FF


def gateup_bytes_n() -> int:
    """The gate/up kernel of the residual block: W_gate + W_up + x + the norm weight + h (f32)."""
    return gateup_bytes() + 4 * D_MODEL


def host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_time(fn, budget_s: float, threads: int):
    """Median seconds per fn(i) call of the oracle on `threads` host threads (calls repeat
    for about budget_s seconds, at least 4; the first is a warm-up).  Returns (seconds,
    calls, total seconds)."""
    import oracle

    oracle.build()
    oracle.set_threads(threads)
    times, i, t_end = [], 0, time.time() + budget_s
    while time.time() < t_end or len(times) < 4:
        t0 = time.perf_counter()
        fn(i)
        times.append(time.perf_counter() - t0)
        i += 1
    oracle.set_threads(1)
    return statistics.median(times[1:]), len(times), sum(times)


def cpu_entry(fn, budget_s: float, work_per_call: float, what: str, unit: str = "GB/s") -> dict:
    """cpu_baseline of a workload: the oracle's restatement of the reference's CPU path (rayon
    over rows there, OpenMP over rows here), timed on all host cores (up to 16) for 2/3 of the
    budget and on one core for the rest.  value = work_per_call (bytes, or flops for GFLOPS)
    / median seconds per call / 1e9, in the workload's own unit."""
    cores = host_cores()
    threads = max(1, min(16, cores))
    t_all, n_all, tot_all = cpu_time(fn, budget_s * 2 / 3, threads)
    t_one, n_one, tot_one = cpu_time(fn, budget_s / 3, 1)
    model = cpu_model()
    return {"value": round(work_per_call / t_all / 1e9, 3), "unit": unit, "cores": threads, "kind": "port",
            "sample": (f"{what}: {n_all} calls in {tot_all:.1f}s, median {t_all * 1e3:.3f} ms per call; "
                       f"{threads} OpenMP threads of {cores} host cores ({model})"),
            "cpu_model": model, "host_cores": cores,
            "one_core": {"value": round(work_per_call / t_one / 1e9, 3), "unit": unit, "cores": 1,
                         "sample": f"{n_one} calls in {tot_one:.1f}s, median {t_one * 1e3:.3f} ms per call"}}


LUT_M, LUT_N = 1536, 576  # hayai bench: SmolLM2-135M's FFN layer (crates/hayai-cli/src/main.rs:601-646)
LUT_TABLE = np.array([-0.5, -0.4, -0.3, -0.2, -0.1, 0.0, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9, 1.0],
                     np.float32)


def lut_cpu_baseline(budget_s: float) -> dict:
    """The reference's named CPU baseline: hayai-cpu's cpu_lut_matmul_q4 (matmul.rs:48-82) at
    `hayai bench`'s shape and inputs (1536x576, every weight byte 0xAB, x = 1.0), GFLOPS =
    2*m*n / time per call, as main.rs:601-646 counts them."""
    import oracle

    w = np.full(LUT_M * LUT_N // 2, 0xAB, np.uint8)
    x = np.ones(LUT_N, np.float32)
    e = cpu_entry(lambda i: oracle.lut_matmul_q4(LUT_M, LUT_N, w, LUT_TABLE, x), budget_s,
                  2.0 * LUT_M * LUT_N, f"oracle cpu_lut_matmul_q4 {LUT_M}x{LUT_N} (0xAB weights, x = 1)", "GFLOPS")
    return e


def cpu_baseline(engine, pack, lay, stride, xs, budget_s: float) -> dict:
    """Time the oracle FFN (fp32 restatement of gemv_q4_k, q4k.rs:206-256) on host cores
    over a bounded sample of the benchmark's own layers (copied back from HBM); the
    reference's LUT MatMul baseline is reported beside it."""
    import oracle
    import hayai_amd

    n_layers = 4  # 4 x 99 MB rotating weight sets: far beyond any host LLC
    rg = hayai_amd.row_bytes(Q4_K, D_MODEL)
    rd = hayai_amd.row_bytes(Q4_K, D_FF)
    mats = []
    for l in range(n_layers):
        base = l * stride
        wg = pack.read(np.uint8, D_FF * rg, base + lay.gate_off)
        wu = pack.read(np.uint8, D_FF * rg, base + lay.up_off)
        wd = pack.read(np.uint8, D_MODEL * rd, base + lay.down_off)
        mats.append((wg, wu, wd))
    e = cpu_entry(lambda i: oracle.ffn((Q4_K, Q4_K, Q4_K), D_MODEL, D_FF, *mats[i % n_layers], xs[i % n_layers]),
                  budget_s, layer_bytes(),
                  f"oracle fp32 FFN (gate/up/down gemv_q4_k + SiLU) over {n_layers} of the 32 benchmark layers")
    t_layer = layer_bytes() / (e["value"] * 1e9)
    e["ffn_tok_s"] = round(1.0 / (t_layer * LAYERS), 4)
    e["lut_matmul_q4"] = lut_cpu_baseline(max(3.0, budget_s / 3))
    return e


def roofline_step(gbs: float, what: str) -> dict:
    """Roofline of a secondary workload over its whole step (all its launches): achieved =
    the step's algorithmic bytes / step time."""
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "kernel": what}


def emit(eng, out: dict) -> int:
    """Print a workload's JSON line and release the engine."""
    print(json.dumps(out), flush=True)
    eng.close()
    return 0


def compact_configs(eng, pack, lay, stride, desc) -> dict:
    """The other BASELINE.json configs in compact form, timed in the default run beside the
    headline, on the same box and clock: configs[0] (SmolLM2-135M Q4_0, 30 layers), configs[2]
    (the headline's own 32 resident 8B layers at 16 and 64 tokens), configs[3] (the MoE layer at
    1 and 32 tokens, 4 resident layers) and configs[4] (the 70B IQ2_XXS FFN, 8 layers through
    the two pinned slots, with the host link's plain hipMemcpy rate beside it).  Each entry keeps
    its own roofline; the full forms are --workload smollm / batched / moe / stream."""
    def ns(**kw):
        base = dict(steps=10, warmup=2, no_cpu_baseline=True, cpu_budget=0.0, batch=1, layers=0)
        base.update(kw)
        return argparse.Namespace(**base)

    keep = ("config", "dtype", "steps", "ms_per_step", "value", "unit", "pct_of_peak", "us_per_layer", "ffn_tok_s",
            "tflops", "mfma", "roofline")

    def pick(o, extra=()):
        return {k: o[k] for k in keep + tuple(extra) if k in o}

    t0 = time.perf_counter()
    out = {}
    out["c0_smollm_q4_0_bs1"] = pick(bench_smollm(eng, ns(steps=40, warmup=4)), ("graph_replay", "chained_stack"))
    for B in (16, 64):
        out[f"c2_8b_q4_k_batch{B}"] = pick(bench_batched(eng, pack, lay, stride, desc, ns(batch=B, steps=5, warmup=2)))
    for T in (1, 32):
        out[f"c3_moe_q4_k_t{T}"] = pick(bench_moe(eng, ns(batch=T, steps=20, warmup=3)),
                                         ("mean_distinct_experts_per_layer",))
    out["c4_70b_iq2_xxs_streamed"] = pick(bench_stream(eng, ns(layers=8, steps=3, warmup=1)),
                                          ("h2d_copy_only_gbs", "h2d_pinned_memcpy_peak_gbs", "h2d_frac_of_memcpy_peak",
                                           "overlap_efficiency", "ffn_resident_hbm_gbs", "ffn_resident_pct_of_peak"))
    log(f"[bench] compact configs timed in {time.perf_counter() - t0:.1f}s")
    return out


def bench_batched(eng, pack, lay, stride, desc, args) -> dict:
    """the 8B Q4_K FFN for B tokens per step (all 32 layers
    resident), gate/up(+SiLU) and down on the matrix cores.  value = algorithmic bytes per
    step (weights once per layer + B tokens' f32 x in and y out) / step time."""
    import hayai_amd
    from hayai_amd import synth

    B = args.batch
    X = synth.normal(synth.seed_for(3, B, synth.ACT), B * D_MODEL * LAYERS).reshape(LAYERS, B, D_MODEL)
    xbuf = eng.upload(X)
    ybuf = eng.alloc(X.nbytes)
    row = 4 * B * D_MODEL

    def step():
        for l in range(LAYERS):
            eng.ffn_batched_dev(desc, pack, l * stride, xbuf, l * row, B, ybuf, l * row)

    for _ in range(args.warmup):
        step()
    eng.sync()
    e0, e1 = eng.event(), eng.event()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    eng.sync()
    ms = e0.elapsed_ms(e1) / args.steps
    wbytes = 2 * D_FF * hayai_amd.row_bytes(Q4_K, D_MODEL) + D_MODEL * hayai_amd.row_bytes(Q4_K, D_FF)
    bytes_step = LAYERS * (wbytes + 2 * 4 * B * D_MODEL)
    gbs = bytes_step / (ms / 1e3) / 1e9
    flops = LAYERS * 2.0 * B * 3 * D_MODEL * D_FF
    tflops = flops / (ms / 1e3) / 1e12
    log(f"[bench] batched B={B}: {ms * 1e3:.1f} us/step, {gbs:.1f} GB/s, {tflops:.1f} TFLOP/s, "
        f"{B * 1e3 / ms:.0f} tok/s")
    cpu = None
    if not args.no_cpu_baseline:
        import oracle

        oracle.build()
        cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        threads = max(1, min(16, cores))
        oracle.set_threads(threads)
        rg, rd = hayai_amd.row_bytes(Q4_K, D_MODEL), hayai_amd.row_bytes(Q4_K, D_FF)
        wg = pack.read(np.uint8, D_FF * rg, lay.gate_off)
        wu = pack.read(np.uint8, D_FF * rg, lay.up_off)
        wd = pack.read(np.uint8, D_MODEL * rd, lay.down_off)
        n, t_end, t0 = 0, time.time() + args.cpu_budget, time.perf_counter()
        while time.time() < t_end or n < 2:
            oracle.ffn((Q4_K, Q4_K, Q4_K), D_MODEL, D_FF, wg, wu, wd, X[0][n % B])
            n += 1
        t_tok = (time.perf_counter() - t0) / n
        cpu = {"value": round(1.0 / (t_tok * LAYERS), 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"oracle fp32 FFN of layer 0, {n} tokens one at a time in {n * t_tok:.1f}s "
                         f"({t_tok * 1e3:.1f} ms per token-layer), {threads} OpenMP threads; tok/s for 32 layers"}
    out = {
        "metric": "FFN GEMV achieved HBM GB/s (% of peak) + FFN tok/s, 8B-shape Q4_K batched",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("int8 activations per 32-element block (as configs[2]) x sc*q, exact integer products on the "
                  "f16 matrix cores, f32 scales and accumulation"
                  if B >= 17 else "f16 MFMA operands (x as hi+lo pair), f32 accumulate"),
        "data": "synthetic (seeded Q4_K blocks, N(0,1) f32 activations)",
        "config": {"workload": f"llama3-8b-ffn-q4_k-batch{B}-32layers-resident", "d_model": D_MODEL, "d_ff": D_FF,
                   "layers": LAYERS, "batch": B, "weights": "Q4_K", "act": "silu"},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "ffn_tok_s": round(B * 1e3 / ms, 2),
        "tflops": round(tflops, 2),
        "roofline": roofline_step(gbs, "whole step: token prep + weight-stream f16 MFMA gate/up and down (B <= 16) or "
                                       "the int8-activation kernels (17..64 tokens, f16 MFMA); MFMA rate in tflops"),
        "mfma": {"achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s (f16 dense)",
                 "frac": round(tflops / 2500.0, 5),
                 "counted": "useful multiply-adds only: 2 * B * 3 * d_model * d_ff per layer"},
        "cpu_baseline": cpu,
    }
    return out


def bench_moe(eng, args) -> dict:
    """Qwen3-30B-A3B-shaped MoE layer (128 experts, top-8 softmax
    routing with renormalisation, d_model 2048, expert d_ff 768, Q4_K), T tokens per step.
    4 MoE layers are resident (4 x 340 MB, beyond the 256 MB last-level cache) and each step
    cycles through 16 router-logit sets, so the experts a step reads are not cache-resident.
    value = algorithmic bytes per step / step time, where the bytes count every DISTINCT
    expert a layer's tokens select once (gate + up + down = 2,654,208 B) plus f32 x in, y
    out and the logits."""
    import hayai_amd
    from hayai_amd import synth

    T = args.batch
    E, K, DM, DF, L, SETS = 128, 8, 2048, 768, 4, 16
    rin, rff = hayai_amd.row_bytes(Q4_K, DM), hayai_amd.row_bytes(Q4_K, DF)
    offs = (0, DF * rin, 2 * DF * rin)
    stride = 2 * DF * rin + DM * rff
    experts = eng.alloc(L * E * stride)
    lo, hi = synth.SCALE_RANGE[Q4_K]
    for l in range(L):
        for e in range(E):
            base = (l * E + e) * stride
            for mat, off, rows, cols in ((synth.GATE, offs[0], DF, DM), (synth.UP, offs[1], DF, DM),
                                         (synth.DOWN, offs[2], DM, DF)):
                eng.synth_weights_dev(Q4_K, experts, base + off, rows * cols // 256,
                                      synth.seed_for(4, l * E + e, mat), lo, hi)
    desc = eng.moe_desc(DM, DF, E, K, stride, offs, norm_topk_prob=True)
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((SETS, L, T, E)).astype(np.float32)
    x = synth.normal(synth.seed_for(4, T, synth.ACT), L * T * DM).reshape(L, T, DM)
    lbuf, xbuf = eng.upload(logits), eng.upload(x)
    ybuf = eng.alloc(4 * L * T * DM)
    # distinct experts per (set, layer) from the routing itself
    ids, rw = eng.route_experts(desc, logits.reshape(-1, E))
    ids = ids.reshape(SETS, L, T, K)
    rw = np.asarray(rw).reshape(SETS, L, T, K)
    distinct = [[len(set(ids[s, l].reshape(-1).tolist()) - {-1}) for l in range(L)] for s in range(SETS)]
    eng.sync()
    log(f"[bench] moe T={T}: mean distinct experts per layer {np.mean(distinct):.1f}")
    lstride, xstride = 4 * T * E, 4 * T * DM

    def step(s):
        for l in range(L):
            eng.moe_dev(desc, experts, l * E * stride, lbuf, ((s % SETS) * L + l) * lstride, None, 0, xbuf,
                        l * xstride, T, ybuf, l * xstride)

    for i in range(args.warmup):
        step(i)
    eng.sync()
    e0, e1 = eng.event(), eng.event()
    e0.record()
    for i in range(args.steps):
        step(i)
    e1.record()
    eng.sync()
    ms = e0.elapsed_ms(e1) / args.steps
    bytes_step = np.mean([sum(distinct[i % SETS]) for i in range(args.steps)]) * stride + L * T * (2 * 4 * DM + 4 * E)
    gbs = bytes_step / (ms / 1e3) / 1e9
    log(f"[bench] moe T={T}: {ms * 1e3:.1f} us/step ({ms * 1e3 / L:.1f} us/layer), {gbs:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        host = experts.read(np.uint8, E * stride, 0)  # layer 0's experts

        def moe_layer(i):
            for t in range(T):
                keep = [(int(e), float(v)) for e, v in zip(ids[0, 0, t], rw[0, 0, t]) if e >= 0]
                oracle.moe_token(Q4_K, DM, DF, host, stride, offs, [e for e, _ in keep], [v for _, v in keep], x[0, t])

        import oracle
        cpu = cpu_entry(moe_layer, args.cpu_budget, distinct[0][0] * stride + T * (2 * 4 * DM + 4 * E),
                        f"oracle MoE layer (the {T} tokens' routed experts, expert loop + combine, moe_infer.rs:342-455) "
                        f"over layer 0's {distinct[0][0]} distinct experts")
    out = {
        "metric": "FFN GEMV achieved HBM GB/s (% of peak), Qwen3-30B-A3B-shaped MoE layer",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_K experts, N(0,1) router logits and activations)",
        "config": {"workload": f"qwen3-30b-a3b-moe-q4_k-T{T}", "experts": E, "top_k": K, "d_model": DM,
                   "expert_d_ff": DF, "layers_resident": L, "tokens": T},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "us_per_layer": round(ms * 1e3 / L, 3),
        "mean_distinct_experts_per_layer": round(float(np.mean(distinct)), 2),
        "roofline": roofline_step(gbs, "whole MoE step: routing + grouped expert gate/up and down (T > 1) or the ring "
                                       "kernels (T = 1)"),
        "cpu_baseline": cpu,
    }
    return out


def bench_stream(eng, args) -> dict:
    """Llama-3-70B-shaped FFN (d_model 8192, d_ff 28672) in IQ2_XXS,
    80 layers streamed from pinned host memory through 2 ping-pong slots: the DMA of layer
    l+1 (hipMemcpyAsync on the copy stream) overlaps the FFN of layer l (compute stream).
    The two pinned host slots are filled once with synthetic layer images: the loader that
    would refill them from disk (io_uring) is outside this path, so every layer re-sends a
    slot's bytes.  value = streamed layer bytes per token / token time (host-link bound).
    Also reported: H2D GB/s of the copies alone, overlap efficiency = T(copies alone) /
    T(pipeline), and the FFN kernels' HBM GB/s on a staged (device-resident) layer."""
    import hayai_amd
    from hayai_amd import synth

    T = hayai_amd.IQ2_XXS
    DM, DF = 8192, 28672
    L = getattr(args, "layers", 0) or 80
    gate = hayai_amd.QuantMatrix("ffn_gate", DM, DF, T)
    up = hayai_amd.QuantMatrix("ffn_up", DM, DF, T)
    down = hayai_amd.QuantMatrix("ffn_down", DF, DM, T)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    desc = eng.ffn_desc((T, T, T), DM, DF, lay)
    st = hayai_amd.StreamingScratch(eng, lay.total, k_chunk=1, n_slots=2)
    lo, hi = synth.SCALE_RANGE[T]
    # the two slot images: seeded IQ2_XXS blocks generated on the device (synth.matrix's
    # generator), copied once into the pinned host slots
    img = eng.alloc(lay.total)
    for l in range(2):
        for mat, off, rows, cols in ((synth.GATE, lay.gate_off, DF, DM), (synth.UP, lay.up_off, DF, DM),
                                     (synth.DOWN, lay.down_off, DM, DF)):
            eng.synth_weights_dev(T, img, off, rows * cols // 256, synth.seed_for(5, l, mat), lo, hi)
        st.host_slot(l)[:] = img.read(np.uint8, lay.total)
    img.free()
    wbytes = sum(ln for _, ln in (lay.ffn_region(r) for r in range(3)))
    xs = synth.normal(synth.seed_for(5, 0, synth.ACT), L * DM).reshape(L, DM)
    xbuf = eng.upload(xs)
    ybuf = eng.alloc(4 * DM * L)

    def stage(l):
        for role in range(3):
            off, ln = lay.ffn_region(role)
            st.dma(l, off, ln)

    def token():
        stage(0)
        for l in range(L):
            if l + 1 < L:
                stage(l + 1)
            mirror, off = st.weight_bind(l)
            eng.ffn_dev(desc, mirror, off, xbuf, 4 * DM * l, ybuf, 4 * DM * l)

    def timed(fn, reps):
        a, b = eng.event(), eng.event()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        eng.sync()
        return a.elapsed_ms(b) / reps

    for _ in range(args.warmup):
        token()
    eng.sync()
    ms_tok = timed(token, args.steps)

    def copies_only():
        for l in range(L):
            stage(l)
        st.weight_bind(L - 1)  # the compute stream waits for the last copy

    ms_copy = timed(copies_only, max(1, min(args.steps, 3)))
    # the host link on its own: one hipMemcpyAsync of 256 MiB from pinned host memory to HBM
    # (hh_buf_copy on the compute stream), the best of 3
    pin, dev = eng.alloc(256 << 20, hayai_amd.BUF_PINNED_HOST), eng.alloc(256 << 20)
    dev.copy_from(pin, 256 << 20)
    ms_peak = min(timed(lambda: dev.copy_from(pin, 256 << 20), 1) for _ in range(3))
    h2d_peak = (256 << 20) / (ms_peak / 1e3) / 1e9
    pin.free()
    dev.free()
    # FFN kernels alone on a staged layer (weights device-resident in the mirror)
    stage(0)
    mirror, off0 = st.weight_bind(0)
    eng.sync()

    def ffn_only():
        for l in range(L):
            eng.ffn_dev(desc, mirror, off0, xbuf, 4 * DM * l, ybuf, 4 * DM * l)

    ffn_only()
    ms_ffn = timed(ffn_only, max(1, args.steps))
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        v = np.array(st.host_slot(0))  # layer 0's image, copied out of the pinned slot
        wl = [v[o:o + n] for o, n in (lay.ffn_region(r) for r in range(3))]
        cpu = cpu_entry(lambda i: oracle.ffn((T, T, T), DM, DF, wl[0], wl[1], wl[2], xs[i % L]), args.cpu_budget,
                        wbytes + 2 * 4 * DM, "oracle fp32 IQ2_XXS FFN of one 70B layer from host memory")
    tok_bytes = L * (wbytes + 2 * 4 * DM)
    gbs = tok_bytes / (ms_tok / 1e3) / 1e9
    h2d = L * wbytes / (ms_copy / 1e3) / 1e9
    ffn_gbs = tok_bytes / (ms_ffn / 1e3) / 1e9
    log(f"[bench] stream: {ms_tok:.2f} ms/token ({ms_tok / L * 1e3:.0f} us/layer), {gbs:.2f} GB/s; copies alone "
        f"{ms_copy:.2f} ms ({h2d:.2f} GB/s); FFN alone {ms_ffn * 1e3 / L:.1f} us/layer ({ffn_gbs:.0f} GB/s)")
    out = {
        "metric": "FFN tok/s and streamed GB/s, 70B-shape IQ2_XXS FFN streamed from pinned host (2-slot ping-pong)",
        "value": round(gbs, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_tok, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded IQ2_XXS layer images in 2 pinned host slots, N(0,1) f32 activations)",
        "config": {"workload": f"llama3-70b-ffn-iq2_xxs-bs1-{L}layers-streamed", "d_model": DM, "d_ff": DF,
                   "layers": L, "batch": 1, "weights": "IQ2_XXS", "slots": 2, "layer_bytes": wbytes},
        "ffn_tok_s": round(1e3 / ms_tok, 3),
        "h2d_copy_only_gbs": round(h2d, 3),
        "h2d_pinned_memcpy_peak_gbs": round(h2d_peak, 3),
        "h2d_frac_of_memcpy_peak": round(h2d / h2d_peak, 4),
        "overlap_efficiency": round(ms_copy / ms_tok, 4),
        "ffn_resident_hbm_gbs": round(ffn_gbs, 1),
        "ffn_resident_pct_of_peak": round(100.0 * ffn_gbs / PEAK_HBM_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(ffn_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(ffn_gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "the IQ2_XXS FFN kernels on a staged (device-resident) layer; the token itself is "
                               "host-link bound"},
        "cpu_baseline": cpu,
    }
    st.free()
    return out


def bench_disk(eng, args) -> int:
    """BASELINE.json configs[4] with the reference's real I/O step: the 70B-shaped IQ2_XXS
    FFN layers are read from a GGUF file through the catalog (io_uring, one batch of reads
    per layer, load_layer_pack_into) into the 2 pinned ping-pong slots, then DMAed and run
    as in the stream workload.  The file (written first, under $TMPDIR) holds --disk-layers
    distinct layers (each with small F16 attention tensors ahead of its FFN, as a layer pack
    has them); the 80 layers of a token cycle through them, so after the first pass the
    reads come from the host page cache.  value = streamed bytes per token / token time."""
    import tempfile

    import hayai_amd
    from hayai_amd import synth
    from hayai_amd.gguf import GgufCatalog, write_gguf

    T = hayai_amd.IQ2_XXS
    DM, DF, L, NF = 8192, 28672, 80, max(2, args.disk_layers)
    lo, hi = synth.SCALE_RANGE[T]
    path = os.path.join(os.environ.get("TMPDIR", tempfile.gettempdir()), f"hayai_bench_{os.getpid()}.gguf")

    def tensors():
        for l in range(NF):
            for name in ("attn_q", "attn_k", "attn_v", "attn_output"):
                yield f"blk.{l}.{name}.weight", (64, 64), 1, np.zeros(64 * 64 * 2, np.uint8)
            for name, mat, rows, cols in (("ffn_gate", synth.GATE, DF, DM), ("ffn_up", synth.UP, DF, DM),
                                          ("ffn_down", synth.DOWN, DM, DF)):
                yield f"blk.{l}.{name}.weight", (cols, rows), T, synth.matrix(T, rows, cols,
                                                                               synth.seed_for(5, l, mat), lo, hi)

    if args.o_direct:  # the reference's HAYAI_O_DIRECT: reads bypass the page cache
        os.environ["HAYAI_O_DIRECT"] = "1"
    t0 = time.perf_counter()
    write_gguf(path, [("general.architecture", "llama")], list(tensors()))
    log(f"[bench] wrote {os.path.getsize(path) / 2**30:.2f} GiB GGUF ({NF} layers) in {time.perf_counter() - t0:.1f} s")
    try:
        cat = GgufCatalog(path)
        lp = cat.layer_pack(0)
        lay = lp.ffn_layout()
        desc = eng.ffn_desc((T, T, T), DM, DF, lay)
        st = hayai_amd.StreamingScratch(eng, lp.total, k_chunk=1, n_slots=2)
        xs = synth.normal(synth.seed_for(5, 0, synth.ACT), L * DM).reshape(L, DM)
        xbuf = eng.upload(xs)
        ybuf = eng.alloc(4 * DM * L)
        ffn_bytes = lay.gate_len + lay.up_len + lay.down_len
        read_s = [0.0]

        def load(l):
            view = st.host_slot(l)  # waits for the DMA still reading this slot
            r0 = time.perf_counter()
            cat.load_layer_pack(l % NF, view)
            read_s[0] += time.perf_counter() - r0
            st.dma(l, lay.gate_off, lay.down_off + lay.down_len - lay.gate_off)

        def token():
            load(0)
            for l in range(L):
                if l + 1 < L:
                    load(l + 1)
                mirror, off = st.weight_bind(l)
                eng.ffn_dev(desc, mirror, off, xbuf, 4 * DM * l, ybuf, 4 * DM * l)

        for _ in range(args.warmup):
            token()
        eng.sync()
        steps = max(1, min(args.steps, 20))
        read_s[0] = 0.0
        a, b = eng.event(), eng.event()
        w0 = time.perf_counter()
        a.record()
        for _ in range(steps):
            token()
        b.record()
        eng.sync()
        wall = (time.perf_counter() - w0) / steps
        ms_tok = a.elapsed_ms(b) / steps
        read_gbs = L * lp.total / (read_s[0] / steps) / 1e9
        cpu = None
        if not args.no_cpu_baseline:
            import oracle
            v = np.zeros(lp.total, np.uint8)
            cat.load_layer_pack(0, v)
            wl = [v[lay.gate_off:lay.gate_off + lay.gate_len], v[lay.up_off:lay.up_off + lay.up_len],
                  v[lay.down_off:lay.down_off + lay.down_len]]
            cpu = cpu_entry(lambda i: (cat.load_layer_pack(i % NF, v),
                                       oracle.ffn((T, T, T), DM, DF, wl[0], wl[1], wl[2], xs[i % L])), args.cpu_budget,
                            lp.total + 2 * 4 * DM, "one layer read from the GGUF file (io_uring) + the oracle's fp32 "
                                                   "IQ2_XXS FFN on host cores")
        tok_bytes = L * (lp.total + 2 * 4 * DM)
        gbs = tok_bytes / (ms_tok / 1e3) / 1e9
        log(f"[bench] disk: {ms_tok:.2f} ms/token ({ms_tok / L * 1e3:.0f} us/layer), {gbs:.2f} GB/s; file reads alone "
            f"{read_s[0] / steps * 1e3:.2f} ms/token ({read_gbs:.2f} GB/s, io_uring={int(cat.io_uring)}, "
            f"o_direct={int(cat.o_direct)}); "
            f"wall {wall * 1e3:.2f} ms/token")
        out = {
            "metric": "FFN tok/s and streamed GB/s, 70B-shape IQ2_XXS FFN read from a GGUF file (io_uring) into "
                      "2 pinned slots",
            "value": round(gbs, 3),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms_tok, 4),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "f32",
            "data": (f"synthetic GGUF file of {NF} distinct IQ2_XXS layers ("
                     + ("read from the device with O_DIRECT" if cat.o_direct else
                        "page-cache resident after the first pass") + "), N(0,1) f32 activations"),
            "config": {"workload": "llama3-70b-ffn-iq2_xxs-bs1-80layers-gguf-io_uring", "d_model": DM, "d_ff": DF,
                       "layers": L, "file_layers": NF, "batch": 1, "weights": "IQ2_XXS", "slots": 2,
                       "layer_pack_bytes": lp.total, "ffn_bytes": ffn_bytes},
            "ffn_tok_s": round(1e3 / ms_tok, 3),
            "file_read_gbs": round(read_gbs, 3),
            "io_uring": bool(cat.io_uring),
            "o_direct": bool(cat.o_direct),
            "roofline": {"bound": "host link", "achieved": round(gbs, 2), "peak": None, "unit": "GB/s", "frac": None,
                         "traffic": None, "kernel": "file -> pinned slot -> HBM per layer pack; PCIe-bound, see the "
                                                    "stream workload for the H2D copy rate"},
            "cpu_baseline": cpu,
        }
        print(json.dumps(out), flush=True)
        st.free()
        cat.close()
    finally:
        os.unlink(path)
    eng.close()
    return 0


def bench_lmhead(eng, args) -> int:
    """The LM head of a Q4_K_M 8B model (stream_infer.rs:2003-2019: execute_quant_gemv of
    output.weight after the final norm): Q6_K, vocab 128256 x d_model 4096, batch 1, as x
    digits + the Q6_K ring kernel.  Reported beside the f32 team kernel (ring off)."""
    import hayai_amd
    from hayai_amd import synth

    T, M, N = (hayai_amd.Q4_K if args.lm_type == "q4_k" else hayai_amd.Q6_K), 128256, 4096
    bb = 144 if T == hayai_amd.Q4_K else 210
    w = eng.alloc(M * (N // 256) * bb)
    lo, hi = synth.SCALE_RANGE[T]
    eng.synth_weights_dev(T, w, 0, M * N // 256, synth.seed_for(6, 0, synth.DOWN), lo, hi)
    x = eng.upload(synth.normal(synth.seed_for(6, 0, synth.ACT), N))
    y = eng.alloc(4 * M)

    def timed(e, reps):
        for _ in range(args.warmup):
            e.gemv_dev(T, M, N, w, 0, x, 0, y, 0)
        e.sync()
        a, b = e.event(), e.event()
        a.record()
        for _ in range(reps):
            e.gemv_dev(T, M, N, w, 0, x, 0, y, 0)
        b.record()
        e.sync()
        return a.elapsed_ms(b) / reps

    ms = timed(eng, args.steps)
    nbytes = M * (N // 256) * bb + 4 * N + 4 * M
    gbs = nbytes / (ms / 1e3) / 1e9
    os.environ["HAYAI_HIP_RING"] = "0"
    plain = hayai_amd.HipEngine(0)
    del os.environ["HAYAI_HIP_RING"]
    wp, xp, yp = plain.alloc(w.nbytes), plain.upload(synth.normal(synth.seed_for(6, 0, synth.ACT), N)), plain.alloc(4 * M)
    plain.synth_weights_dev(T, wp, 0, M * N // 256, synth.seed_for(6, 0, synth.DOWN), lo, hi)
    for _ in range(args.warmup):
        plain.gemv_dev(T, M, N, wp, 0, xp, 0, yp, 0)
    plain.sync()
    a, b = plain.event(), plain.event()
    a.record()
    for _ in range(args.steps):
        plain.gemv_dev(T, M, N, wp, 0, xp, 0, yp, 0)
    b.record()
    plain.sync()
    ms_plain = a.elapsed_ms(b) / args.steps
    plain.close()
    log(f"[bench] lm head {args.lm_type} {M}x{N}: {ms * 1e3:.1f} us ({gbs:.1f} GB/s); ring off {ms_plain * 1e3:.1f} us "
        f"({nbytes / (ms_plain / 1e3) / 1e9:.1f} GB/s)")
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        wh, xh = w.read(np.uint8, w.nbytes), x.read(np.float32, N)
        cpu = cpu_entry(lambda i: oracle.gemv(T, M, N, wh, xh), args.cpu_budget, nbytes,
                        f"oracle fp32 gemv of the {M}x{N} matrix")
    out = {
        "metric": "LM-head GEMV achieved HBM GB/s, Q6_K 128256x4096 (Llama-3 8B Q4_K_M output.weight) bs=1",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q6_K blocks, N(0,1) f32 activations)",
        "config": {"workload": "llama3-8b-lm-head-q6_k-bs1", "vocab": M, "d_model": N, "weights": "Q6_K"},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "team_kernel_us": round(ms_plain * 1e3, 2),
        "roofline": roofline_step(gbs, "x digits + the Q6_K ring kernel" if T != hayai_amd.Q4_K else "Q4_K GEMV kernel"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_smollm(eng, args) -> dict:
    """SmolLM2-135M-shaped SwiGLU FFN (d_model 576, d_ff 1536) in
    Q4_0, 30 layers, batch 1.  The 30-layer stack is 45 MB; 8 copies (360 MB, beyond the
    256 MB last-level cache) rotate across steps so weights come from HBM.  value =
    algorithmic bytes per step / step time; this shape is launch-latency bound."""
    import hayai_amd
    from hayai_amd import synth

    T = hayai_amd.Q4_0
    DM, DF, L, COPIES = 576, 1536, 30, 8
    gate = hayai_amd.QuantMatrix("ffn_gate", DM, DF, T)
    up = hayai_amd.QuantMatrix("ffn_up", DM, DF, T)
    down = hayai_amd.QuantMatrix("ffn_down", DF, DM, T)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    desc = eng.ffn_desc((T, T, T), DM, DF, lay)
    stride = lay.total
    pack = eng.alloc(stride * L * COPIES)
    lo, hi = synth.SCALE_RANGE[T]
    for c in range(COPIES):
        for l in range(L):
            for mat, off, rows, cols in ((synth.GATE, lay.gate_off, DF, DM), (synth.UP, lay.up_off, DF, DM),
                                         (synth.DOWN, lay.down_off, DM, DF)):
                eng.synth_weights_dev(T, pack, (c * L + l) * stride + off, rows * cols // 32,
                                      synth.seed_for(1, l, mat), lo, hi)
    xs = synth.normal(synth.seed_for(1, 0, synth.ACT), L * DM).reshape(L, DM)
    xbuf = eng.upload(xs)
    ybuf = eng.alloc(4 * DM * L)

    def step(s):
        base = (s % COPIES) * L * stride
        for l in range(L):
            eng.ffn_dev(desc, pack, base + l * stride, xbuf, 4 * DM * l, ybuf, 4 * DM * l)

    for i in range(args.warmup):
        step(i)
    eng.sync()
    a, b = eng.event(), eng.event()
    a.record()
    for i in range(args.steps):
        step(i)
    b.record()
    eng.sync()
    ms = a.elapsed_ms(b) / args.steps
    wb = gate.nbytes + up.nbytes + down.nbytes
    bytes_step = L * (wb + 2 * 4 * DM)
    gbs = bytes_step / (ms / 1e3) / 1e9
    log(f"[bench] smollm: {ms * 1e3:.1f} us/step ({ms * 1e3 / L:.2f} us/layer), {gbs:.1f} GB/s")
    # the same steps as HIP graphs: one 30-layer graph per weight copy, captured once and
    # replayed in rotation (the one-launch FFN's grid barrier keeps its state on the device)
    graphs = [eng.capture(lambda c=c: step(c)) for c in range(COPIES)]
    for i in range(args.warmup):
        graphs[i % COPIES].launch()
    eng.sync()
    a.record()
    for i in range(args.steps):
        graphs[i % COPIES].launch()
    b.record()
    eng.sync()
    ms_graph = a.elapsed_ms(b) / args.steps
    for g in graphs:
        g.free()
    log(f"[bench] smollm graph replay: {ms_graph * 1e3:.1f} us/step ({ms_graph * 1e3 / L:.2f} us/layer)")
    # The 30 layers as chained residual blocks (x_{l+1} = x_l + FFN_l(rms_norm(x_l))): one
    # persistent launch per step (hh_ffn_block_stack_dev), and the same chain as 30 block
    # calls for comparison.
    norms = synth.normal(synth.seed_for(1, 0, synth.ACT) + 7, L * DM) * 0.1 + 1.0
    nbuf = eng.upload(norms.astype(np.float32))
    sbuf = eng.alloc(4 * DM)

    def stack(s):
        eng.ffn_block_stack_dev(desc, pack, (s % COPIES) * L * stride, stride, L, nbuf, 0, DM, 1e-5, xbuf, 0,
                                sbuf, 0)

    def blocks(s):
        base = (s % COPIES) * L * stride
        for l in range(L):
            eng.ffn_block_dev(desc, pack, base + l * stride, nbuf, 4 * DM * l, 1e-5, xbuf if l == 0 else sbuf, 0,
                              sbuf, 0)

    chained = {}
    for name, fn in (("stack", stack), ("blocks", blocks)):
        for i in range(args.warmup):
            fn(i)
        eng.sync()
        a.record()
        for i in range(args.steps):
            fn(i)
        b.record()
        eng.sync()
        chained[name] = a.elapsed_ms(b) / args.steps
        log(f"[bench] smollm chained {name}: {chained[name] * 1e3:.1f} us/step "
            f"({chained[name] * 1e3 / L:.2f} us/layer)")
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        mats = [[pack.read(np.uint8, m.nbytes, l * stride + o) for m, o in ((gate, lay.gate_off), (up, lay.up_off),
                                                                            (down, lay.down_off))] for l in range(4)]
        cpu = cpu_entry(lambda i: oracle.ffn((T, T, T), DM, DF, *mats[i % 4], xs[i % L]), args.cpu_budget,
                        wb + 2 * 4 * DM, "oracle fp32 Q4_0 FFN over 4 of the 30 layers in rotation")
    out = {
        "metric": "FFN GEMV achieved HBM GB/s (% of peak) + FFN tok/s, SmolLM2-135M-shape Q4_0 bs=1",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_0 blocks, N(0,1) f32 activations), 8 rotating copies of the 30 layers",
        "config": {"workload": "smollm2-135m-ffn-q4_0-bs1-30layers", "d_model": DM, "d_ff": DF, "layers": L,
                   "batch": 1, "weights": "Q4_0", "act": "silu"},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "ffn_tok_s": round(1e3 / ms, 2),
        "us_per_layer": round(ms * 1e3 / L, 3),
        "graph_replay": {"ms_per_step": round(ms_graph, 5), "us_per_layer": round(ms_graph * 1e3 / L, 3),
                         "value": round(bytes_step / (ms_graph / 1e3) / 1e9, 2)},
        "chained_stack": {"ms_per_step": round(chained["stack"], 5),
                          "us_per_layer": round(chained["stack"] * 1e3 / L, 3),
                          "value": round((bytes_step + L * 4 * DM) / (chained["stack"] / 1e3) / 1e9, 2)},
        "chained_blocks": {"ms_per_step": round(chained["blocks"], 5),
                           "us_per_layer": round(chained["blocks"] * 1e3 / L, 3)},
        "roofline": roofline_step(gbs, "whole step: the one-launch Q4_0 FFN kernel per layer (launch-latency bound)"),
        "cpu_baseline": cpu,
    }
    return out


def bench_q4km(eng, args) -> int:
    """The 8B FFN in the Q4_K_M layout: gate/up Q4_K, down Q6_K (llama.cpp's Q4_K_M keeps
    ffn_down of many layers in Q6_K), 32 layers resident, batch 1.  Not a BASELINE.json
    config: it measures the path a real Q4_K_M file takes through the FFN op."""
    import hayai_amd
    from hayai_amd import synth

    Q6_K = hayai_amd.Q6_K
    gate = hayai_amd.QuantMatrix("ffn_gate", D_MODEL, D_FF, Q4_K)
    up = hayai_amd.QuantMatrix("ffn_up", D_MODEL, D_FF, Q4_K)
    down = hayai_amd.QuantMatrix("ffn_down", D_FF, D_MODEL, Q6_K)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    stride = (lay.total + 255) // 256 * 256
    pack = eng.alloc(stride * LAYERS)
    for l in range(LAYERS):
        for t, mat, off, rows, cols in ((Q4_K, synth.GATE, lay.gate_off, D_FF, D_MODEL),
                                        (Q4_K, synth.UP, lay.up_off, D_FF, D_MODEL),
                                        (Q6_K, synth.DOWN, lay.down_off, D_MODEL, D_FF)):
            lo, hi = synth.SCALE_RANGE[t]
            eng.synth_weights_dev(t, pack, l * stride + off, rows * cols // 256, synth.seed_for(9, l, mat), lo, hi)
    xs = [synth.normal(synth.seed_for(9, l, synth.ACT), D_MODEL) for l in range(LAYERS)]
    xbuf = eng.upload(np.concatenate(xs))
    ybuf = eng.alloc(4 * D_MODEL * LAYERS)
    desc = eng.ffn_desc((Q4_K, Q4_K, Q6_K), D_MODEL, D_FF, lay)

    def step():
        for l in range(LAYERS):
            eng.ffn_dev(desc, pack, l * stride, xbuf, 4 * D_MODEL * l, ybuf, 4 * D_MODEL * l)

    for _ in range(args.warmup):
        step()
    eng.sync()
    a, b = eng.event(), eng.event()
    a.record()
    for _ in range(args.steps):
        step()
    b.record()
    eng.sync()
    ms = a.elapsed_ms(b) / args.steps
    wb = gate.nbytes + up.nbytes + down.nbytes
    bytes_step = LAYERS * (wb + 2 * 4 * D_MODEL + 2 * 4 * D_FF)
    gbs = bytes_step / (ms / 1e3) / 1e9
    log(f"[bench] q4_k_m: {ms * 1e3:.1f} us/step ({ms * 1e3 / LAYERS:.2f} us/layer), {gbs:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        mats = [[pack.read(np.uint8, m.nbytes, l * stride + o) for m, o in ((gate, lay.gate_off), (up, lay.up_off),
                                                                            (down, lay.down_off))] for l in range(4)]
        cpu = cpu_entry(lambda i: oracle.ffn((Q4_K, Q4_K, Q6_K), D_MODEL, D_FF, *mats[i % 4], xs[i % 4]),
                        args.cpu_budget, bytes_step / LAYERS, "oracle fp32 Q4_K_M FFN over 4 of the 32 layers")
    out = {
        "metric": "FFN GEMV achieved HBM GB/s (% of peak) + FFN tok/s, 8B-shape Q4_K_M (Q6_K down) bs=1",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_K / Q6_K blocks, N(0,1) f32 activations)",
        "config": {"workload": "llama3-8b-ffn-q4_k_m-bs1-32layers-resident", "d_model": D_MODEL, "d_ff": D_FF,
                   "layers": LAYERS, "batch": 1, "weights": "Q4_K gate/up, Q6_K down", "act": "silu"},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "ffn_tok_s": round(1e3 / ms, 2),
        "us_per_layer": round(ms * 1e3 / LAYERS, 3),
        "roofline": roofline_step(gbs, "ring gate/up (Q4_K) + Q6_K ring down, per layer"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    eng.close()
    return 0


def bench_block(eng, pack, lay, stride, desc, args) -> int:
    """The 8B decode step's FFN half as a model runs it: 32 residual blocks chained in place
    on one residual stream, x_{l+1} = x_l + FFN_l(rms_norm(x_l, norm_l)) (ffn_apply,
    hybrid_infer.rs:883-936), the RMSNorm and the residual add fused into the ring kernels.
    Reported beside the plain FFN op on the same weights (independent per-layer x)."""
    import hayai_amd
    from hayai_amd import synth

    norms = eng.upload(np.concatenate([synth.normal(synth.seed_for(CONFIG_ID, l, 7), D_MODEL) * 0.1 + 1.0
                                       for l in range(LAYERS)]).astype(np.float32))
    x0 = synth.normal(synth.seed_for(CONFIG_ID, 0, synth.ACT), D_MODEL)
    xres = eng.upload(x0)
    xs = eng.upload(np.tile(x0, LAYERS))
    ys = eng.alloc(4 * D_MODEL * LAYERS)

    def block_step():
        for l in range(LAYERS):
            eng.ffn_block_dev(desc, pack, l * stride, norms, 4 * D_MODEL * l, 1e-5, xres, 0, xres, 0)

    def ffn_step():
        for l in range(LAYERS):
            eng.ffn_dev(desc, pack, l * stride, xs, 4 * D_MODEL * l, ys, 4 * D_MODEL * l)

    def stack_step():  # the same chain as one hh_ffn_block_stack_dev call
        eng.ffn_block_stack_dev(desc, pack, 0, stride, LAYERS, norms, 0, D_MODEL, 1e-5, xres, 0, xres, 0)

    def timed(run, n):
        e0, e1 = eng.event(), eng.event()
        e0.record()
        for _ in range(n):
            run()
        e1.record()
        eng.sync()
        return e0.elapsed_ms(e1) / n

    for _ in range(args.warmup):
        xres.write(x0)
        block_step()
        ffn_step()
        stack_step()
    eng.sync()
    xres.write(x0)
    block_step()
    eng.sync()
    y_block = xres.read(np.float32, D_MODEL)
    xres.write(x0)
    stack_step()
    eng.sync()
    y_stack = xres.read(np.float32, D_MODEL)
    stack_diff = float(np.max(np.abs(y_stack - y_block)) / max(float(np.max(np.abs(y_block - x0))), 1e-30))
    xres.write(x0)
    ms_block = timed(block_step, args.steps)
    ms_ffn = timed(ffn_step, args.steps)
    ms_stack = timed(stack_step, args.steps)
    bytes_step = LAYERS * (layer_bytes() + 4 * D_MODEL)  # + the norm weights
    gbs = bytes_step / (ms_block / 1e3) / 1e9
    log(f"[bench] block: {ms_block * 1e3:.1f} us/step ({ms_block * 1e3 / LAYERS:.2f} us/layer), {gbs:.1f} GB/s; "
        f"plain FFN op {ms_ffn * 1e3 / LAYERS:.2f} us/layer; one stack call "
        f"(blocks per layer) {ms_stack * 1e3 / LAYERS:.2f} us/layer, "
        f"max diff vs the blocks {stack_diff:.2e} of max|FFN part|")
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        rg, rd = hayai_amd.row_bytes(Q4_K, D_MODEL), hayai_amd.row_bytes(Q4_K, D_FF)
        mats = [(pack.read(np.uint8, D_FF * rg, l * stride + lay.gate_off), pack.read(np.uint8, D_FF * rg, l * stride + lay.up_off),
                 pack.read(np.uint8, D_MODEL * rd, l * stride + lay.down_off)) for l in range(4)]
        nw = norms.read(np.float32, D_MODEL * 4).reshape(4, D_MODEL)
        cpu = cpu_entry(lambda i: oracle.ffn_block((Q4_K,) * 3, D_MODEL, D_FF, *mats[i % 4], nw[i % 4], 1e-5, x0),
                        args.cpu_budget, layer_bytes() + 4 * D_MODEL,
                        "oracle ffn_apply (rms_norm + fp32 Q4_K FFN + residual) over 4 of the 32 layers")
    out = {
        "metric": "FFN residual block (RMSNorm + FFN + residual) achieved HBM GB/s, 8B-shape Q4_K bs=1",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_block, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Q4_K blocks, N(0,1) f32 residual stream, norm weights 1 + 0.1 N(0,1))",
        "config": {"workload": "llama3-8b-ffn-block-q4_k-bs1-32layers-chained", "d_model": D_MODEL, "d_ff": D_FF,
                   "layers": LAYERS, "batch": 1, "weights": "Q4_K", "act": "silu", "eps": 1e-5},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "us_per_layer": round(ms_block * 1e3 / LAYERS, 3),
        "plain_ffn_us_per_layer": round(ms_ffn * 1e3 / LAYERS, 3),
        "stack_call": {"us_per_layer": round(ms_stack * 1e3 / LAYERS, 3),
                       "max_rel_diff_vs_blocks": stack_diff},
        "roofline": roofline_step(gbs, "ring gate/up with the RMSNorm prologue + ring down with the residual epilogue"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_lut(eng, args) -> int:
    """`hayai bench` (crates/hayai-cli/src/main.rs:601-646) on the GPU: the Q4 LUT MatMul
    (Hayai's 4-bit dictionary format) at SmolLM2-135M's FFN layer shape, 1536x576, every
    weight byte 0xAB, x = 1.0, GFLOPS = 2*m*n / time per call.  value: device-resident
    operands, kernel launches back to back (events on the compute stream); host_io: the
    reference's execute_lut_matmul form (host arrays in and out, blocking, PCIe included).
    The 442 KB weight matrix stays in cache, so the HBM roofline is taken on the same kernel
    at the 8B gate shape (14336x4096, 29 MB) over 10 rotating copies (294 MB, beyond the
    256 MB last-level cache).  cpu_baseline: the oracle's cpu_lut_matmul_q4 at the bench
    shape (the reference's named CPU baseline), all host cores and one core."""
    M, N = LUT_M, LUT_N
    w = np.full(M * N // 2, 0xAB, np.uint8)
    x = np.ones(N, np.float32)
    wb, tb, xb, yb = eng.upload(w), eng.upload(LUT_TABLE), eng.upload(x), eng.alloc(4 * M)
    inner = 100

    def run():
        for _ in range(inner):
            eng.lut_gemv_dev(M, N, wb, 0, tb, 0, xb, 0, yb, 0)

    for _ in range(args.warmup):
        run()
    eng.sync()
    e0, e1 = eng.event(), eng.event()
    e0.record()
    for _ in range(args.steps):
        run()
    e1.record()
    eng.sync()
    ms = e0.elapsed_ms(e1) / (args.steps * inner)
    y = yb.read(np.float32, M)
    flops = 2.0 * M * N
    gflops = flops / (ms / 1e3) / 1e9
    # host-array form (compute.rs:45-128 uploads W, LUT and x and reads y back per call)
    reps = max(20, args.steps)
    for _ in range(5):
        eng.lut_matmul_q4(M, N, w, LUT_TABLE, x)
    t0 = time.perf_counter()
    for _ in range(reps):
        yh = eng.lut_matmul_q4(M, N, w, LUT_TABLE, x)
    host_s = (time.perf_counter() - t0) / reps
    assert np.array_equal(yh, y)
    # the kernel streaming from HBM
    BM, BN, COPIES = 14336, 4096, 10
    wbig = eng.alloc(BM * BN // 2 * COPIES)
    for c in range(COPIES):
        eng.synth_weights_dev(0, wbig, c * BM * BN // 2, BM * BN // 8, 77 + c, 0.0, 0.0)
    xbig = eng.upload(np.ones(BN, np.float32))
    ybig = eng.alloc(4 * BM)
    for c in range(COPIES):
        eng.lut_gemv_dev(BM, BN, wbig, c * BM * BN // 2, tb, 0, xbig, 0, ybig, 0)
    eng.sync()
    n_big = max(COPIES, (args.steps // COPIES) * COPIES)
    e0.record()
    for i in range(n_big):
        eng.lut_gemv_dev(BM, BN, wbig, (i % COPIES) * BM * BN // 2, tb, 0, xbig, 0, ybig, 0)
    e1.record()
    eng.sync()
    big_us = e0.elapsed_ms(e1) / n_big * 1e3
    big_bytes = BM * BN // 2 + 4 * BN + 4 * BM + 64
    big_gbs = big_bytes / (big_us / 1e6) / 1e9
    log(f"[bench] lut {M}x{N}: {ms * 1e3:.2f} us per call, {gflops:.1f} GFLOPS (device), "
        f"{flops / host_s / 1e9:.2f} GFLOPS host-io; {BM}x{BN}: {big_us:.2f} us, {big_gbs:.0f} GB/s")
    cpu = None if args.no_cpu_baseline else lut_cpu_baseline(args.cpu_budget)
    out = {
        "metric": "Q4 LUT MatMul GFLOPS (hayai bench: SmolLM2-135M FFN layer 1536x576)",
        "value": round(gflops, 2),
        "unit": "GFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms * inner, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "hayai bench inputs (weights 0xAB, x = 1.0, the reference's 16-entry LUT)",
        "config": {"workload": "hayai-bench-lut-matmul-q4-1536x576", "m": M, "n": N, "calls_per_step": inner},
        "us_per_call": round(ms * 1e3, 3),
        "host_io": {"gflops": round(flops / host_s / 1e9, 3), "us_per_call": round(host_s * 1e6, 2),
                    "note": "host arrays in/out per call, blocking (PCIe included)"},
        "roofline": {"bound": "hbm", "achieved": round(big_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(big_gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": f"hh_lut_gemv at {BM}x{BN} over {COPIES} rotating weight copies",
                     "mean_us": round(big_us, 3), "algorithmic_bytes": big_bytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    eng.close()
    return 0


SHAPES = {"8b": (4096, 14336, 32), "70b": (8192, 28672, 80), "smollm": (576, 1536, 30)}


def bench_ffn_resident(eng, args) -> int:
    """One format through the FFN op, every layer resident in HBM, batch 1: --fmt (q4_0,
    q8_0, q4_k, q6_k, iq2_xxs, iq3_xxs) at --shape (8b: 4096x14336 x 32 layers; 70b:
    8192x28672 x 80 layers; smollm: 576x1536 x 30).  Shows each format's own kernel where it is
    the whole cost (a resident 70B IQ2_XXS model is 14.5 GB, well inside 288 GB of HBM).
    value = algorithmic bytes per step (weights once + x in + y out per layer) / step time."""
    import hayai_amd
    from hayai_amd import synth

    T = FMTS[args.fmt]
    DM, DF, L = SHAPES[args.shape]
    if args.layers:
        L = args.layers
    gate = hayai_amd.QuantMatrix("ffn_gate", DM, DF, T)
    up = hayai_amd.QuantMatrix("ffn_up", DM, DF, T)
    down = hayai_amd.QuantMatrix("ffn_down", DF, DM, T)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    stride = (lay.total + 255) // 256 * 256
    pack = eng.alloc(stride * L)
    blk = synth.BLOCK[T][0]
    lo, hi = synth.SCALE_RANGE[T]
    for l in range(L):
        for mat, off, rows, cols in ((synth.GATE, lay.gate_off, DF, DM), (synth.UP, lay.up_off, DF, DM),
                                     (synth.DOWN, lay.down_off, DM, DF)):
            eng.synth_weights_dev(T, pack, l * stride + off, rows * cols // blk, synth.seed_for(20 + T, l, mat), lo, hi)
    xs = synth.normal(synth.seed_for(20 + T, 0, synth.ACT), L * DM).reshape(L, DM)
    xbuf = eng.upload(xs)
    ybuf = eng.alloc(4 * DM * L)
    desc = eng.ffn_desc((T, T, T), DM, DF, lay)

    def step():
        for l in range(L):
            eng.ffn_dev(desc, pack, l * stride, xbuf, 4 * DM * l, ybuf, 4 * DM * l)

    for _ in range(args.warmup):
        step()
    eng.sync()
    a, b = eng.event(), eng.event()
    a.record()
    for _ in range(args.steps):
        step()
    b.record()
    eng.sync()
    ms = a.elapsed_ms(b) / args.steps
    wb = gate.nbytes + up.nbytes + down.nbytes
    bytes_layer = wb + 2 * 4 * DM
    gbs = bytes_layer * L / (ms / 1e3) / 1e9
    log(f"[bench] ffn {args.fmt} {args.shape}: {ms * 1e3:.1f} us/step ({ms * 1e3 / L:.2f} us/layer), {gbs:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        nl = min(2, L)
        mats = [[pack.read(np.uint8, m.nbytes, l * stride + o) for m, o in ((gate, lay.gate_off), (up, lay.up_off),
                                                                            (down, lay.down_off))] for l in range(nl)]
        cpu = cpu_entry(lambda i: oracle.ffn((T, T, T), DM, DF, *mats[i % nl], xs[i % nl]), args.cpu_budget,
                        bytes_layer, f"oracle fp32 {args.fmt} FFN over {nl} of the {L} layers")
    out = {
        "metric": f"FFN GEMV achieved HBM GB/s (% of peak) + FFN tok/s, {args.shape}-shape {args.fmt} bs=1, resident",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": FMT_DTYPE.get(args.fmt, "f32"),
        "data": f"synthetic (seeded {args.fmt} blocks, N(0,1) f32 activations)",
        "config": {"workload": f"{args.shape}-ffn-{args.fmt}-bs1-{L}layers-resident", "d_model": DM, "d_ff": DF,
                   "layers": L, "batch": 1, "weights": args.fmt, "act": "silu"},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "ffn_tok_s": round(1e3 / ms, 2),
        "us_per_layer": round(ms * 1e3 / L, 3),
        "roofline": roofline_step(gbs, f"{args.fmt} gate/up + down, per layer"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    eng.close()
    return 0


def bench_gemv(eng, args) -> int:
    """One GEMV, --fmt at --m x --n (default: hayai's calibration probe, Q4_K 4096x4096,
    crates/hayai-core/src/calibration.rs:175-196), over rotating weight copies that exceed the
    256 MB last-level cache.  value = (weights + x + y) bytes / time per GEMV."""
    import hayai_amd
    from hayai_amd import synth

    T = FMTS[args.fmt]
    M, N = args.m, args.n
    rb = hayai_amd.row_bytes(T, N)
    wbytes = M * rb
    copies = max(2, -(-(300 << 20) // wbytes))
    stride = (wbytes + 255) // 256 * 256
    wbuf = eng.alloc(stride * copies)
    blk = synth.BLOCK[T][0]
    lo, hi = synth.SCALE_RANGE.get(T, (0.0, 0.0))
    for c in range(copies):
        eng.synth_weights_dev(T, wbuf, c * stride, M * N // blk, 300 + c, lo, hi)
    x = synth.normal(301, N)
    xb, yb = eng.upload(x), eng.alloc(4 * M)
    for c in range(copies):
        eng.gemv_dev(T, M, N, wbuf, c * stride, xb, 0, yb, 0)
    eng.sync()
    n = max(copies, args.steps // copies * copies)
    a, b = eng.event(), eng.event()
    a.record()
    for i in range(n):
        eng.gemv_dev(T, M, N, wbuf, (i % copies) * stride, xb, 0, yb, 0)
    b.record()
    eng.sync()
    us = a.elapsed_ms(b) / n * 1e3
    nbytes = wbytes + 4 * N + 4 * M
    gbs = nbytes / (us / 1e6) / 1e9
    log(f"[bench] gemv {args.fmt} {M}x{N}: {us:.2f} us, {gbs:.0f} GB/s over {copies} copies")
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        wh = wbuf.read(np.uint8, wbytes, 0)
        wh2 = wbuf.read(np.uint8, wbytes, stride)
        cpu = cpu_entry(lambda i: oracle.gemv(T, M, N, wh if i % 2 == 0 else wh2, x), args.cpu_budget, nbytes,
                        f"oracle fp32 {args.fmt} GEMV {M}x{N}, two weight copies in rotation")
    out = {
        "metric": f"GEMV achieved HBM GB/s, {args.fmt} {M}x{N}",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": copies,
        "ms_per_step": round(us / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": FMT_DTYPE.get(args.fmt, "f32"),
        "data": f"synthetic (seeded {args.fmt} blocks, N(0,1) f32 x), {copies} rotating weight copies",
        "config": {"workload": f"gemv-{args.fmt}-{M}x{N}", "m": M, "n": N},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "roofline": roofline_step(gbs, f"{args.fmt} GEMV kernel"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    eng.close()
    return 0


FMTS = {"q4_0": 2, "q8_0": 8, "q4_k": 12, "q6_k": 14, "iq2_xxs": 16, "iq3_xxs": 18}
FMT_DTYPE = {"q4_k": "q4_k x int8-digit activations (v_dot4 i32 sums, f32 scales)",
             "q6_k": "q6_k x int8-digit activations (v_dot4 i32 sums, f32 scales)"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="default workload: skip the compact forms of the other BASELINE.json configs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one 256 MiB device copy before timing (reference point for HBM counters)")
    ap.add_argument("--workload", default="bs1", choices=["bs1", "batched", "moe", "stream", "smollm", "q4km", "block", "disk",
                                                          "lmhead", "lut", "ffn", "gemv"],
                    help="bs1: BASELINE.json configs[1] (the headline); batched: configs[2], --batch tokens per "
                         "step; moe: configs[3], --batch tokens per step; stream: configs[4] (70B IQ2_XXS "
                         "streamed from pinned host); smollm: configs[0]; q4km: the 8B FFN with a Q6_K down "
                         "projection (Q4_K_M layout); block: the 8B FFN residual block (RMSNorm + FFN + "
                         "residual) chained over 32 layers; disk: configs[4] read from a GGUF file through "
                         "io_uring into the pinned slots; lmhead: the 8B Q4_K_M LM head (Q6_K 128256x4096); "
                         "lut: hayai bench's Q4 LUT MatMul (1536x576, GFLOPS); ffn: --fmt at --shape, every "
                         "layer resident; gemv: one --fmt GEMV at --m x --n (default: the calibration probe, "
                         "Q4_K 4096x4096)")
    ap.add_argument("--disk-layers", type=int, default=8, help="distinct layers in the --workload disk file")
    ap.add_argument("--o-direct", action="store_true",
                    help="--workload disk: read the file with O_DIRECT (HAYAI_O_DIRECT), bypassing the page cache")
    ap.add_argument("--lm-type", default="q6_k", choices=["q6_k", "q4_k"], help="--workload lmhead weight format")
    ap.add_argument("--batch", type=int, default=16, help="tokens per step for --workload batched")
    ap.add_argument("--fmt", default="q4_k", choices=["q4_0", "q8_0", "q4_k", "q6_k", "iq2_xxs", "iq3_xxs"],
                    help="--workload ffn / gemv weight format")
    ap.add_argument("--shape", default="8b", choices=["8b", "70b", "smollm"], help="--workload ffn shape")
    ap.add_argument("--layers", type=int, default=0, help="--workload ffn: layers (0: the shape's own count)")
    ap.add_argument("--m", type=int, default=4096, help="--workload gemv rows")
    ap.add_argument("--n", type=int, default=4096, help="--workload gemv columns")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the FFN path would shard "
              "d_ff across GPUs with one d_model all-reduce per layer, which is not built here.", file=sys.stderr)
        return 2

    import hayai_amd
    from hayai_amd import synth

    eng = hayai_amd.HipEngine(0)
    log(f"[bench] device {eng.device_name} {eng.arch} CUs={eng.device_info.compute_units}")
    if args.workload == "moe":
        return emit(eng, bench_moe(eng, args))
    if args.workload == "stream":
        return emit(eng, bench_stream(eng, args))
    if args.workload == "smollm":
        return emit(eng, bench_smollm(eng, args))
    if args.workload == "q4km":
        return bench_q4km(eng, args)
    if args.workload == "disk":
        return bench_disk(eng, args)
    if args.workload == "lmhead":
        return bench_lmhead(eng, args)
    if args.workload == "lut":
        return bench_lut(eng, args)
    if args.workload == "ffn":
        return bench_ffn_resident(eng, args)
    if args.workload == "gemv":
        return bench_gemv(eng, args)
    gate = hayai_amd.QuantMatrix("ffn_gate", D_MODEL, D_FF, Q4_K)
    up = hayai_amd.QuantMatrix("ffn_up", D_MODEL, D_FF, Q4_K)
    down = hayai_amd.QuantMatrix("ffn_down", D_FF, D_MODEL, Q4_K)
    lay = hayai_amd.LayerPackLayout.ffn_only(gate, up, down)
    stride = lay.total
    pack = eng.alloc(stride * LAYERS)
    lo, hi = synth.SCALE_RANGE[Q4_K]
    for l in range(LAYERS):
        for mat, off, rows, cols in ((synth.GATE, lay.gate_off, D_FF, D_MODEL), (synth.UP, lay.up_off, D_FF, D_MODEL),
                                     (synth.DOWN, lay.down_off, D_MODEL, D_FF)):
            eng.synth_weights_dev(Q4_K, pack, l * stride + off, rows * cols // 256,
                                  synth.seed_for(CONFIG_ID, l, mat), lo, hi)
    xs = [synth.normal(synth.seed_for(CONFIG_ID, l, synth.ACT), D_MODEL) for l in range(LAYERS)]
    xbuf = eng.upload(np.concatenate(xs))
    ybuf = eng.alloc(4 * D_MODEL * LAYERS)
    eng.sync()
    log(f"[bench] {LAYERS} layers resident: {stride * LAYERS / 2**30:.2f} GiB of Q4_K weights")
    desc = eng.ffn_desc((Q4_K, Q4_K, Q4_K), D_MODEL, D_FF, lay)
    if args.workload == "batched":
        return emit(eng, bench_batched(eng, pack, lay, stride, desc, args))
    if args.workload == "block":
        return bench_block(eng, pack, lay, stride, desc, args)

    # One decode step's FFN half: the 32 layers chained on one residual stream, as ffn_apply
    # runs them (hybrid_infer.rs:883-938): x_{l+1} = x_l + FFN_l(rms_norm(x_l, norm_l)).  A
    # chain of bare FFNs diverges (the FFN is about quadratic in x), so the decode's RMSNorm
    # and residual, fused into the two ring kernels, carry the chain.
    norms = eng.upload(np.concatenate([synth.normal(synth.seed_for(CONFIG_ID, l, 7), D_MODEL) * 0.1 + 1.0
                                       for l in range(LAYERS)]).astype(np.float32))
    xres = eng.upload(xs[0])
    EPS = 1e-5

    def step():
        for l in range(LAYERS):
            eng.ffn_block_dev(desc, pack, l * stride, norms, 4 * D_MODEL * l, EPS, xres, 0, xres, 0)

    def ffn_unchained():  # the plain FFN op per layer on independent inputs (no norm/residual)
        for l in range(LAYERS):
            eng.ffn_dev(desc, pack, l * stride, xbuf, 4 * D_MODEL * l, ybuf, 4 * D_MODEL * l)

    if args.copy_calibration:
        cal = eng.alloc(256 << 20)
        cal.copy_from(pack, 256 << 20)
        eng.sync()
        cal.free()

    def timed(run, n) -> float:  # ms per call of run(), events on the compute stream
        e0, e1 = eng.event(), eng.event()
        e0.record()
        for _ in range(n):
            run()
        e1.record()
        eng.sync()
        return e0.elapsed_ms(e1) / n

    for _ in range(args.warmup):
        step()
        ffn_unchained()
    eng.sync()
    xres.write(xs[0])
    t0 = time.perf_counter()
    ms_eager = timed(step, args.steps)
    wall = time.perf_counter() - t0
    y_end = xres.read(np.float32, D_MODEL)
    finite = bool(np.isfinite(y_end).all())
    log(f"[bench] chained residual stream after {args.steps} steps: finite={finite}, "
        f"max|x|={float(np.max(np.abs(y_end))):.3e}")
    xres.write(xs[0])
    graph = eng.capture(step)
    for _ in range(3):
        graph.launch()
    eng.sync()
    ms_graph = timed(graph.launch, args.steps)
    graph.free()
    ms_plain = timed(ffn_unchained, args.steps)
    ms = ms_eager
    bytes_layer = layer_bytes() + 4 * D_MODEL  # + the norm weight
    bytes_step = bytes_layer * LAYERS
    gbs = bytes_step / (ms / 1e3) / 1e9
    gbs_graph = bytes_step / (ms_graph / 1e3) / 1e9
    gbs_plain = layer_bytes() * LAYERS / (ms_plain / 1e3) / 1e9
    log(f"[bench] {ms * 1e3:.1f} us/step (event), wall {wall / args.steps * 1e6:.1f} us/step, {gbs:.1f} GB/s; "
        f"graph replay {ms_graph * 1e3:.1f} us/step, {gbs_graph:.1f} GB/s; plain FFN op (unchained) "
        f"{ms_plain * 1e3:.1f} us/step, {gbs_plain:.1f} GB/s")

    # Each kernel of the step on its own, through ffn_apply's two-call form (it issues exactly
    # the kernels of the one-call block): a region of gate/up launches alone over all layers,
    # then one of gate/up + down, each bracketed by events on the compute stream;
    # down = (gate/up + down) - gate/up.  Back-to-back launches of one kernel: the time per
    # launch includes the dispatch gap between launches.
    n_prof = max(1, min(args.steps, 50))

    def region(with_down: bool) -> float:
        def run():
            for l in range(LAYERS):
                base = l * stride
                eng.ffn_block_begin_dev(desc, pack, base, norms, 4 * D_MODEL * l, EPS, xbuf, 4 * D_MODEL * l)
                if with_down:
                    eng.ffn_block_finish_dev(desc, pack, base, xbuf, 4 * D_MODEL * l, ybuf, 4 * D_MODEL * l)
        return timed(run, n_prof) / LAYERS

    gu = region(False)
    dn = region(True) - gu
    gu_gbs = gateup_bytes_n() / (gu / 1e3) / 1e9
    dn_gbs = (D_MODEL * hayai_amd.row_bytes(Q4_K, D_FF) + 4 * D_FF + 2 * 4 * D_MODEL) / (dn / 1e3) / 1e9
    log(f"[bench] per kernel: gate/up {gu * 1e3:.2f} us ({gu_gbs:.0f} GB/s), down {dn * 1e3:.2f} us "
        f"({dn_gbs:.0f} GB/s)")
    layer_us = ms * 1e3 / LAYERS

    configs = None if args.no_configs else compact_configs(eng, pack, lay, stride, desc)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(eng, pack, lay, stride, xs, args.cpu_budget)
        log(f"[bench] cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads, {cpu['one_core']['value']} GB/s "
            f"on one core; LUT MatMul {cpu['lut_matmul_q4']['value']} GFLOPS")

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        traffic = int(t["hbm_bytes_per_launch"])
    out = {
        "metric": "FFN GEMV achieved HBM GB/s (% of peak) + FFN tok/s, 8B-shape Q4_K bs=1",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x int8-digit activations (v_dot4 i32 sums, f32 scales)",
        "data": "synthetic (seeded Q4_K blocks, N(0,1) f32 activations, norm weights 1 + 0.1 N(0,1))",
        "config": {"workload": "llama3-8b-ffn-q4_k-bs1-32layers-resident", "d_model": D_MODEL, "d_ff": D_FF,
                   "layers": LAYERS, "batch": 1, "weights": "Q4_K", "act": "silu",
                   "step": "32 layers chained on one residual stream (RMSNorm + FFN + residual, ffn_apply); "
                           "a bandwidth harness: random weights, the stream carried from step to step "
                           "(its values grow; the kernels' time does not depend on them)",
                   "launch": "eager, 2 kernels per layer"},
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "ffn_tok_s": round(1e3 / ms, 2),
        "us_per_layer": round(layer_us, 3),
        "output_finite": finite,
        "graph_replay": {"ms_per_step": round(ms_graph, 5), "value": round(gbs_graph, 2),
                         "ffn_tok_s": round(1e3 / ms_graph, 2)},
        "ffn_op_unchained": {"ms_per_step": round(ms_plain, 5), "value": round(gbs_plain, 2),
                             "us_per_layer": round(ms_plain * 1e3 / LAYERS, 3)},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": gateup_bytes_n(),
                     "kernel": "hh_q4k_gu_ring_g1_n: ring gate/up with the RMSNorm + SwiGLU, h as int8 digits",
                     "mean_us": round(gu * 1e3, 3)},
        "down_kernel": {"kernel": "hh_q4k_dn_ring_d4 (residual epilogue)", "us": round(dn * 1e3, 3),
                        "gbs": round(dn_gbs, 1)},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)
    eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
