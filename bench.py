"""MoE-layer decode throughput on one MI355X.

Workload: one Mixtral-shape MoE FFN layer — d_model 4096, 8 experts, top-2, expert FFN
14336 SwiGLU, gate/up/down quantised to Q4_K (build-side quantiser) from N(0, 0.02^2)
weights, f32 router N(0, 0.02^2), N(0, 1) activations — decoded at a batch of tokens.
A step is one call of the layer (route -> dispatch -> gate/up -> down -> combine) on
inputs already resident in HBM. Steps rotate over `--layers` distinct copies of the
layer in HBM (different router weights, separate slab copies of the experts) so each
step streams its experts from HBM rather than from the 256 MB MALL.

Each batch is timed twice over the same steps: bare, for `value` and `ms_per_step`, and
with HIP events recorded on the stream around every gate/up and down launch, for the
kernel times (the events themselves add about 3 us per launch to a step).

Prints one JSON line with `roofline` (the gate/up kernel: algorithmic bytes per launch /
its average duration from HIP events on its stream; `layer_frac`: the whole layer step's
algorithmic bytes over its bare time, against the same peak) and `cpu_baseline` (the oracle's
restatement of the reference's packed CPU path, threaded over rows, on a bounded sample).
`roofline.traffic` is the HBM bytes per gate/up launch that rocprofv3's FETCH_SIZE and
WRITE_SIZE counters measured on this same workload, scaled by what they read for a copy of
known size (`--calibrate-copy`), as recorded in profiles/ (TRAFFIC_FILE); it is null for
any other configuration.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

D, F, NE, K = 4096, 14336, 8, 2
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
TRAFFIC_FILE = ROOT / "profiles" / "k_gu_units_q4k_c2_b8_traffic.md"
SEED = 0x6761_7275_6461_2000  # build-side seeds, "garuda" + tag


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_median(fn, calls=10, budget_s=20.0):
    """fn() once as a warm-up (not counted), then at least `calls` timed calls, or as many as
    fit `budget_s` but at least three; returns (median seconds, calls timed)."""
    import statistics
    fn()
    ts, t_end = [], time.time() + budget_s
    while len(ts) < calls and (len(ts) < 3 or time.time() < t_end):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), len(ts)


def cpu_record(value, unit, threads, sample):
    return {"value": value, "unit": unit, "cores": threads, "cpu": cpu_model(), "kind": "port", "sample": sample}


def make_experts(threads):
    import garuda_amd as G
    from garuda_amd import moe as M
    mats = {}
    for p, (name, rows, cols) in enumerate((("gate", F, D), ("up", F, D), ("down", D, F))):
        parts = []
        for e in range(NE):
            x = M.fill_gaussian(SEED + 16 * e + p, rows * cols, 0.0, 0.02, threads)
            parts.append(M.quantize(G.Q4_K, x, threads))
            del x
        mats[name] = np.concatenate(parts)
    return mats


def measured_traffic(batch, math, layers):
    """HBM bytes per gate/up launch from the committed counter summary, if it covers this run."""
    try:
        text = TRAFFIC_FILE.read_text()
    except OSError:
        return None
    vals = {}
    for line in text.splitlines():
        if ":" in line and line.strip().startswith("- "):
            key, _, v = line.strip()[2:].partition(":")
            vals[key.strip()] = v.strip()
    try:
        if int(vals["batch"]) != batch or vals["math"] != math or int(vals["layers"]) != layers:
            return None
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


# BASELINE configs 4 and 5 (the per-layer slice of C5): name -> shape, types, batch
EXTRA_CONFIGS = {
    "c4": dict(d=2048, f=768, ne=128, k=8, n=64, qts=("Q6_K", "Q6_K", "Q8_0"), logits_scale=4.0,
               workload="C4 fine-grained MoE layer: d2048 f768 128 experts top-8, Q6_K gate/up, Q8_0 down, "
                        "64 tokens, router logits uniform x4 given"),
    "c5_layer": dict(d=4096, f=14336, ne=8, k=2, n=8, qts=("Q3_K", "Q3_K", "Q4_K"), logits_scale=None,
                     workload="C5 per-layer slice: Mixtral-shape layer with Q3_K gate/up and Q4_K down "
                              "(Q3_K_M-style mix), 8 concurrent decode tokens"),
}


def extra_leg(name, a, dev, threads, stream, timed, cpu):
    """One decode leg of a further BASELINE configuration: tokens/s and the layer's HBM rate
    (touched experts' packed bytes + router + activations per call over the call time)."""
    import torch
    import garuda_amd as G
    from garuda_amd import moe as M

    c = EXTRA_CONFIGS[name]
    d, f, ne, k, n = c["d"], c["f"], c["ne"], c["k"], c["n"]
    qts = tuple(getattr(G, q) for q in c["qts"])
    seed = SEED + 0x1000 * (1 + list(EXTRA_CONFIGS).index(name))
    mats = {}
    for p, (nm, rows, cols) in enumerate((("gate", f, d), ("up", f, d), ("down", d, f))):
        mats[nm] = M.quantize(qts[p], M.fill_gaussian(seed + p, ne * rows * cols, 0.0, 0.02, threads), threads)
    expert_bytes = sum(M.byte_size(qts[p], rows * cols) for p, (rows, cols) in enumerate(((f, d), (f, d), (d, f))))
    layers = []
    for l in range(2):
        router = M.fill_gaussian(seed + 0x10 + l, ne * d, 0.0, 0.02, threads)
        layers.append(G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], qts,
                                 math=G.MATH_PACKED))
    keep = mats if cpu else {}
    hs = torch.from_numpy(M.fill_gaussian(seed + 0x20, n * d, 0.0, 1.0, threads).reshape(n, d)).cuda()
    lg = None
    if c["logits_scale"] is not None:
        rng = np.random.default_rng(seed & 0xffffffff)
        lg = torch.from_numpy((rng.random((n, ne), dtype=np.float32) * np.float32(c["logits_scale"]))).cuda()
    out = torch.empty((n, d), dtype=torch.float32, device="cuda")
    ids = torch.empty((len(layers), n, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((len(layers), n, k), dtype=torch.float32, device="cuda")
    sh = stream.cuda_stream

    def step(i):
        l = i % len(layers)
        layers[l].forward_async(hs.data_ptr(), n, out.data_ptr(), ids[l].data_ptr(), wts[l].data_ptr(),
                                lg.data_ptr() if lg is not None else 0, sh)

    steps = max(50, a.steps // 2)
    for i in range(max(5, a.warmup // 2)):
        step(i)
    torch.cuda.synchronize()
    ms, _ = timed(step, steps, False)
    touched = float(np.mean([len(np.unique(ids[l].cpu().numpy())) for l in range(len(layers))]))
    step_s = ms / steps / 1e3
    nbytes = touched * expert_bytes + (0 if lg is not None else ne * d * 4) + 2 * n * d * 4
    log(f"{name}: {n / step_s:.0f} tok/s, {step_s * 1e6:.1f} us/call, {touched:.1f} experts touched, "
        f"{nbytes / step_s / 1e9:.0f} GB/s")
    res = {"workload": c["workload"], "tokens_per_s": n / step_s, "us_per_call": step_s * 1e6,
           "experts_touched": touched, "layer_bytes": nbytes, "layer_GBs": nbytes / step_s / 1e9,
           "hbm_frac": nbytes / step_s / 1e9 / HBM_PEAK_GBS, "math": "packed", "steps": steps, "cpu_baseline": None}
    if cpu:
        from oracle import oracle as O  # the checker's restatement, timed as the CPU path
        L = dict(d=d, f=f, ne=ne, k=k, packed=1, router=layers[0].router, qtypes=qts, **keep)
        hs_np = hs.cpu().numpy()
        lg_np = lg.cpu().numpy() if lg is not None else None
        med, calls = cpu_median(lambda: O.feed_forward_batch(L, hs_np, lg_np, threads=threads))
        res["cpu_baseline"] = cpu_record(n / med, "tokens/s", threads,
                                         f"median of {calls} calls (one warm-up call before) of this layer at batch "
                                         f"{n}, oracle restatement of the packed int8 path, {threads} threads")
        log(f"{name} cpu: {n / med:.1f} tok/s")
    for l in layers:
        l.release()
    return res


def prefill_leg(a, dev, mats, threads, stream, timed, cpu, packed=False):
    """the same Q4_K layer at a prefill of `a.prefill_tokens` tokens,
    routing skewed to Zipf(1.1) expert loads through one shared activation direction.
    f32 math (Weight::Full) runs k_pf for gate/up and down; packed math (Weight::Packed,
    mmap = true) runs k_pq for gate/up and k_pf for down over the dequantised h; all on
    MFMA. Returns the JSON object of the leg."""
    import torch
    import garuda_amd as G
    from garuda_amd import moe as M

    math = G.MATH_PACKED if packed else G.MATH_F32
    mname = "packed" if packed else "f32"
    n = a.prefill_tokens
    u = M.skew_direction(SEED + 0x300, D)
    layers = []
    for l in range(a.prefill_layers):
        router = M.skew_router(M.fill_gaussian(SEED + 0x100 + l, NE * D, 0.0, 0.02, threads), NE, D, u)
        layers.append(G.MoeLayer(dev, D, F, NE, K, router, mats["gate"], mats["up"], mats["down"],
                                 (G.Q4_K,) * 3, math=math))
    hs_np = M.skew_tokens(M.fill_gaussian(SEED + 0x400, n * D, 0.0, 1.0, threads).reshape(n, D), u)
    hs = torch.from_numpy(hs_np).cuda()
    out = torch.empty((n, D), dtype=torch.float32, device="cuda")
    ids = torch.empty((len(layers), n, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((len(layers), n, K), dtype=torch.float32, device="cuda")
    sh = stream.cuda_stream

    def step(i):
        l = i % len(layers)
        layers[l].forward_async(hs.data_ptr(), n, out.data_ptr(), ids[l].data_ptr(), wts[l].data_ptr(), 0, sh)

    for i in range(max(3, a.warmup // 4)):
        step(i)
    torch.cuda.synchronize()
    ms, _ = timed(step, a.prefill_steps, False)
    _, (gu_ms, dn_ms, _) = timed(step, a.prefill_steps, True)
    loads = [np.bincount(ids[l].cpu().numpy().reshape(-1), minlength=NE) for l in range(len(layers))]
    flops = float(np.mean([ld.sum() for ld in loads])) * 6 * D * F  # 2 flops per MAC, 3 matrices
    ex_s = (gu_ms + dn_ms) / 1e3
    step_s = ms / a.prefill_steps / 1e3
    tflops = flops / ex_s / 1e12
    log(f"prefill ({mname}) n={n}: {n / step_s:.0f} tok/s, {step_s * 1e6:.0f} us/call, gate/up {gu_ms * 1e3:.0f} us, "
        f"down {dn_ms * 1e3:.0f} us, {tflops:.0f} TFLOP/s algorithmic ({tflops / MFMA_PEAK_TFLOPS:.1%} of peak), "
        f"loads {loads[0].tolist()}")
    cpu_rec = None
    if cpu and packed:
        # Weight::Packed: quant::matmul's int8 path over a sample of the same tokens
        from oracle import oracle as O  # the checker's restatement, timed as the CPU path
        sample = max(1, a.prefill_cpu_tokens)
        pick = np.linspace(0, n - 1, sample).astype(np.int64)
        L = dict(d=D, f=F, ne=NE, k=K, packed=1, router=layers[0].router, qtypes=(G.Q4_K,) * 3, **mats)
        med, calls = cpu_median(lambda: O.feed_forward_batch(L, hs_np[pick], threads=threads), calls=5)
        cpu_rec = cpu_record(sample / med, "tokens/s", threads,
                             f"median of {calls} calls (one warm-up call before) on {sample} of the {n} skewed "
                             f"tokens, oracle restatement of quant::matmul's packed int8 path, {threads} threads")
        log(f"prefill cpu (packed path): {sample / med:.1f} tok/s")
    elif cpu:
        # Weight::Full (llama/mod.rs:170-173): the experts expanded to f32 once, as the
        # reference does at load, then simd::matmul over a sample of the same tokens
        from oracle import oracle as O  # the checker's restatement, timed as the CPU path
        sample = max(1, a.prefill_cpu_tokens)
        pick = np.linspace(0, n - 1, sample).astype(np.int64)
        full = {f"{nm}_f32": O.dequantize(G.Q4_K, mats[nm], mats[nm].size // 144 * 256, checked=False)
                for nm in ("gate", "up", "down")}
        L = dict(d=D, f=F, ne=NE, k=K, packed=0, router=layers[0].router, qtypes=(G.Q4_K,) * 3, **mats, **full)
        med, calls = cpu_median(lambda: O.feed_forward_batch(L, hs_np[pick], threads=threads), calls=5)
        del full, L
        cpu_rec = cpu_record(sample / med, "tokens/s", threads,
                             f"median of {calls} calls (one warm-up call before) on {sample} of the {n} skewed "
                             f"tokens, oracle restatement of the f32 Weight::Full path (simd::matmul over the "
                             f"dequantised experts), {threads} threads")
        log(f"prefill cpu (f32 Full path): {sample / med:.1f} tok/s")
    for l in layers:
        l.release()
    kernels = "k_pq<Q4_K> (gate/up) + k_pf<Q4_K, down>" if packed else "k_pf<Q4_K, gate/up> + k_pf<Q4_K, down>"
    note = ("algorithmic flops (sum of expert tokens x 6 d f) over the two MFMA launches' time; the reference's "
            "packed arithmetic adds one float term per 32-value sub-block per (row, token) of gate/up, five VALU "
            "operations evaluated in K order, which bound k_pq near 20% of peak" if packed else
            "algorithmic flops (sum of expert tokens x 6 d f) over the two MFMA launches' "
            "time; the exact-product scheme issues two fp16 MFMA passes per product (with the min-term "
            "passes and padded token tiles 2.46x the algorithmic work), which bound k_pf near 36% of peak")
    return {
        "cpu_baseline": cpu_rec,
        "workload": f"C3 prefill: the C2 layer at {n} tokens, Zipf(1.1)-skewed routing, {mname} math, "
                    f"{len(layers)} HBM copies rotated",
        "tokens_per_s": n / step_s, "ms_per_call": step_s * 1e3, "steps": a.prefill_steps,
        "expert_loads": [int(x) for x in loads[0]],
        "gateup_us": gu_ms * 1e3, "down_us": dn_ms * 1e3,
        "roofline": {"bound": "mfma", "kernels": kernels,
                     "achieved": tflops, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tflops / MFMA_PEAK_TFLOPS,
                     "flops_per_call": flops, "note": note},
    }


def dense_leg(a, dev, threads, stream, timed):
    """Dense projections (Weight::matmul_rows) through the same kernels, at C5's shapes
    and a decode batch of 8 (packed math): one layer's attention projections q, k, v, o
    (4096x4096, 1024x4096, 1024x4096, 4096x4096, Q4_K) and the output head (32000x4096,
    Q6_K). Copies are rotated so each step's weights come from HBM, not the 256 MB MALL."""
    import torch
    import garuda_amd as G
    from garuda_amd import moe as M

    n = 8
    shapes = {"q": (4096, 4096, G.Q4_K), "k": (1024, 4096, G.Q4_K), "v": (1024, 4096, G.Q4_K),
              "o": (4096, 4096, G.Q4_K), "head": (32000, 4096, G.Q6_K)}
    copies = {"attn": 16, "head": 4}
    seed = SEED + 0x600
    raws = {nm: M.quantize(qt, M.fill_gaussian(seed + i, r * c, 0.0, 0.02, threads), threads)
            for i, (nm, (r, c, qt)) in enumerate(shapes.items())}
    attn = [[G.DenseWeight(dev, shapes[nm][2], shapes[nm][0], shapes[nm][1], raws[nm]) for nm in "qkvo"]
            for _ in range(copies["attn"])]
    # as the model step runs them: q, k and v stacked into one 6144-row weight (the packed
    # rows laid end to end, what the model's stacking of the three makes), then o
    qkv_raw = np.concatenate([raws["q"], raws["k"], raws["v"]])
    stacked = [(G.DenseWeight(dev, G.Q4_K, 6144, 4096, qkv_raw),
                G.DenseWeight(dev, G.Q4_K, 4096, 4096, raws["o"])) for _ in range(copies["attn"])]
    del qkv_raw
    head = [G.DenseWeight(dev, G.Q6_K, 32000, 4096, raws["head"]) for _ in range(copies["head"])]
    del raws
    x = torch.from_numpy(M.fill_gaussian(seed + 0x10, n * 4096, 0.0, 1.0, threads).reshape(n, 4096)).cuda()
    outs = {nm: torch.empty((n, shapes[nm][0]), dtype=torch.float32, device="cuda") for nm in shapes}
    outs["qkv"] = torch.empty((n, 6144), dtype=torch.float32, device="cuda")
    # the model step's form: the K slices left for the next launch to add (rope/append, the
    # feed-forward's residual add), so no launch of their own
    parts = {nm: torch.empty((G.DenseWeight.MAX_SLICES, n, r), dtype=torch.float32, device="cuda")
             for nm, r in (("qkv", 6144), ("o", 4096))}
    sh = stream.cuda_stream

    def attn_step(i):
        for W, nm in zip(attn[i % len(attn)], "qkvo"):
            W.forward_async(x.data_ptr(), n, outs[nm].data_ptr(), sh)

    def stacked_step(i):
        Wqkv, Wo = stacked[i % len(stacked)]
        Wqkv.forward_async(x.data_ptr(), n, outs["qkv"].data_ptr(), sh)
        Wo.forward_async(x.data_ptr(), n, outs["o"].data_ptr(), sh)

    def slices_step(i):
        Wqkv, Wo = stacked[i % len(stacked)]
        Wqkv.forward_slices_async(x.data_ptr(), n, parts["qkv"].data_ptr(), sh)
        Wo.forward_slices_async(x.data_ptr(), n, parts["o"].data_ptr(), sh)

    def head_step(i):
        head[i % len(head)].forward_async(x.data_ptr(), n, outs["head"].data_ptr(), sh)

    res = {}
    steps = max(64, a.steps // 4)
    for name, step, nbytes in (
            ("attention q,k,v,o", attn_step, sum(M.byte_size(qt, r * c) for nm, (r, c, qt) in shapes.items()
                                                 if nm != "head")),
            ("attention qkv stacked + o", stacked_step,
             sum(M.byte_size(qt, r * c) for nm, (r, c, qt) in shapes.items() if nm != "head")),
            ("attention qkv stacked + o, slices to the next launch", slices_step,
             sum(M.byte_size(qt, r * c) for nm, (r, c, qt) in shapes.items() if nm != "head")),
            ("output head", head_step, M.byte_size(G.Q6_K, 32000 * 4096))):
        for i in range(8):
            step(i)
        torch.cuda.synchronize()
        ms, _ = timed(step, steps, False)
        us = ms / steps * 1e3
        gbs = (nbytes + n * 4096 * 4) / (us / 1e6) / 1e9
        log(f"dense {name}: {us:.1f} us per call at batch {n}, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM peak)")
        res[name] = {"us_per_call": us, "weight_bytes": nbytes, "GB_s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS}
    for ws in attn:
        for W in ws:
            W.release()
    for W in head:
        W.release()
    for ws in stacked:
        for W in ws:
            W.release()
    return {"workload": "C5 dense projections at decode batch 8, packed math: one layer's q,k,v,o "
                        "(Q4_K; 4096x4096, 1024x4096 x2, 4096x4096) as four calls, stacked (q,k,v in one "
                        "6144-row call, then o) with the K slices added by a launch of their own, and "
                        "stacked as the model step runs them (the slices left to the next launch, which "
                        "adds them: rope/append, the feed-forward's residual add), and the 32000x4096 "
                        f"Q6_K output head; {copies['attn']} and {copies['head']} copies rotated",
            "batch": n, "legs": res}


def prefetch_leg(a, mats, threads):
    """Predictor-driven prefetch into a slab that holds 6 of the C2
    layer's 8 experts, over a decode stream whose tokens drift (h_t = 0.9 h_{t-1} + 0.45
    noise, so consecutive steps route alike). The same steps run without and with the
    PrefetchEngine (depth = top-k); each step is the synchronous forward (staging what it
    misses) plus, with prefetch, observe_step staging the predicted experts."""
    import garuda_amd as G
    from garuda_amd import moe as M
    from garuda_amd.predict import ExpertPredictor, PrefetchEngine

    expert_bytes = 3 * M.byte_size(G.Q4_K, F * D)
    router = M.fill_gaussian(SEED + 0x700, NE * D, 0.0, 0.02, threads)
    steps = a.prefetch_steps
    res = {}
    # each mode twice, alternating; the second run of each is kept (the first pays the
    # process's one-time costs, which would fall on whichever mode ran first)
    for mode in ("off", "on", "off", "on"):
        dev2 = G.Device(0, slab_bytes=6 * (expert_bytes + (1 << 20)))
        layer = G.MoeLayer(dev2, D, F, NE, K, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        eng = PrefetchEngine(dev2, ExpertPredictor(NE), enabled=True, depth=K) if mode == "on" else None
        rng = np.random.default_rng(SEED & 0xffff)
        h = rng.normal(0, 1, D).astype(np.float32)
        prev, last = [], []
        # untimed first steps: each mode starts on a fresh device, whose first calls load
        # the kernels and fill the slab
        for _ in range(10):
            h = (0.9 * h + 0.45 * rng.normal(0, 1, D)).astype(np.float32)
            layer.feed_forward_batch(h.reshape(1, D))
        s0 = dev2.slab_stats()
        t0 = time.perf_counter()
        for _ in range(steps):
            h = (0.9 * h + 0.45 * rng.normal(0, 1, D)).astype(np.float32)
            _, ids, _ = layer.feed_forward_batch(h.reshape(1, D))
            if eng is not None:
                used = [int(x) for x in ids.reshape(-1)]
                last = eng.observe_step(layer, 0, prev, used, last)
                prev = used
        dt = time.perf_counter() - t0
        s1 = dev2.slab_stats()
        r = {"ms_per_step": dt / steps * 1e3, "forward_misses": s1.misses - s0.misses,
             "staged_GB": (s1.h2d_bytes - s0.h2d_bytes) / 1e9}
        if eng is not None:
            st = eng.predictor_stats()
            r.update(precision=st.precision(), recall=st.recall(), prefetched=eng.launched, already_resident=eng.skipped)
        res[mode] = r
        layer.release()
        dev2.close()
    on, off = res["on"], res["off"]
    log(f"prefetch: {steps} steps, slab of 6/8 experts: without {off['ms_per_step']:.2f} ms/step, "
        f"{off['forward_misses']} forward misses; with {on['ms_per_step']:.2f} ms/step, {on['forward_misses']} "
        f"misses, {on['prefetched']} prefetched, precision {on['precision']:.2f} recall {on['recall']:.2f}")
    return {"workload": "C2 layer, slab of 6 of 8 experts, batch-1 decode stream with drifting tokens; "
                        "synchronous forward per step (+ observe_step with prefetch)",
            "steps": steps, "without": off, "with": on}


def attention_leg(a, dev, threads, stream, timed):
    """Decode attention over the paged KV cache at C5's shape (32 query
    heads on 8 kv heads of 128, pages of 16 positions, 8 concurrent sequences), one layer:
    the sequences' prompts are prefilled to a context, then batch-8 decode steps (one
    token per sequence) are timed. Bytes per step: every sequence's keys and values over
    its context, the kernel's HBM floor."""
    import torch
    import garuda_amd as G
    from garuda_amd.attention import KvCache

    nh, nkv, hd, nseq = 32, 8, 128, 8
    res = {}
    for ctx_len in (128, 2048):
        steps = 64
        kv = KvCache(dev, 1, nh, nkv, hd, block_size=16, max_positions=ctx_len + steps + 8, max_seqs=nseq)
        seqs = [kv.open_seq() for _ in range(nseq)]
        g = torch.Generator(device="cpu").manual_seed(SEED & 0xffff)
        chunk = 256
        for p0 in range(0, ctx_len, chunk):  # prefill every sequence to ctx_len
            m = min(chunk, ctx_len - p0)
            ids = [s for s in seqs for _ in range(m)]
            q = torch.randn(len(ids), nh * hd, generator=g).cuda()
            k = torch.randn(len(ids), nkv * hd, generator=g).cuda()
            v = torch.randn(len(ids), nkv * hd, generator=g).cuda()
            o = torch.empty(len(ids), nh * hd, device="cuda")
            kv.attention_async(0, ids, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), stream.cuda_stream)
        torch.cuda.synchronize()
        q = torch.randn(nseq, nh * hd, generator=g).cuda()
        k = torch.randn(nseq, nkv * hd, generator=g).cuda()
        v = torch.randn(nseq, nkv * hd, generator=g).cuda()
        o = torch.empty(nseq, nh * hd, device="cuda")

        def step(i):
            kv.attention_async(0, seqs, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), stream.cuda_stream)

        ms, _ = timed(step, steps, False)
        us = ms / steps * 1e3
        nbytes = nseq * nkv * hd * 4 * 2 * (ctx_len + steps // 2)
        gbs = nbytes / (us / 1e6) / 1e9
        log(f"attention ctx {ctx_len}: {us:.1f} us per batch-{nseq} decode step of one layer, {gbs:.0f} GB/s "
            f"of K/V ({gbs / HBM_PEAK_GBS:.1%} of HBM peak)")
        res[str(ctx_len)] = {"us_per_step": us, "kv_bytes_per_step": nbytes, "GB_s": gbs, "hbm_frac": gbs / HBM_PEAK_GBS}
        kv.close()
    return {"workload": "C5 attention, one layer: 8 sequences decoding (one token each) over a paged KV cache, "
                        "32 query / 8 kv heads of 128, pages of 16, f32 K/V", "contexts": res}


def e2e_leg(a, threads, cpu):
    """C5 end to end: a 32-layer Mixtral-shape model (Q3_K gate/up, Q4_K down, Q4_K
    attention projections, Q6_K output head, f32 token table; GQA 32/8 of 128, paged KV
    cache, rope theta 1e6) decoding 8 sequences at once through gmoe_model_decode: each
    sequence is fed a 128-token prompt one token per step, then decodes greedily while
    the steps are timed (each step returns its tokens to the host). The layers cycle over
    8 HBM copies of one synthetic layer, so every layer's weights come from HBM, not the
    MALL. With `cpu`, one batch-8 step of the same model at the middle of the GPU's timed
    contexts (each cache filled with random keys and values to that length) runs through
    the oracle's restatement on the host threads."""
    import garuda_amd as G
    from garuda_amd import moe as M
    from garuda_amd.attention import KvCache

    d, f, ne, k, nh, nkv, hd, vocab, nseq = 4096, 14336, 8, 2, 32, 8, 128, 32000, 8
    nl, copies, prompt, steps = a.e2e_layers, min(8, a.e2e_layers), a.e2e_prompt, a.e2e_steps
    seed = SEED + 0x5000
    t0 = time.time()

    def q(qt, rows, cols, sd, std=0.02):
        return M.quantize(qt, M.fill_gaussian(sd, rows * cols, 0.0, std, threads), threads)

    ex = {nm: q(qt, ne * rows, cols, seed + i) for i, (nm, qt, rows, cols) in
          enumerate((("gate", G.Q3_K, f, d), ("up", G.Q3_K, f, d), ("down", G.Q4_K, d, f)))}
    att = {nm: q(G.Q4_K, rows, cols, seed + 8 + i) for i, (nm, rows, cols) in
           enumerate((("wq", nh * hd, d), ("wk", nkv * hd, d), ("wv", nkv * hd, d), ("wo", d, nh * hd)))}
    head_raw = q(G.Q6_K, vocab, d, seed + 16)
    table = M.fill_gaussian(seed + 17, vocab * d, 0.0, 1.0, threads).reshape(vocab, d)
    norms = [M.fill_gaussian(seed + 32 + i, d, 1.0, 0.05, threads) for i in range(2 * copies + 1)]
    routers = [M.fill_gaussian(seed + 64 + c, ne * d, 0.0, 0.02, threads) for c in range(copies)]
    gen_s = time.time() - t0
    expert_bytes = sum(M.byte_size(qt, r * c) for qt, r, c in ((G.Q3_K, f, d), (G.Q3_K, f, d), (G.Q4_K, d, f)))
    dev = G.Device(0, slab_bytes=copies * ne * (expert_bytes + 4096) + (64 << 20))
    moe = [G.MoeLayer(dev, d, f, ne, k, routers[c], ex["gate"], ex["up"], ex["down"], (G.Q3_K, G.Q3_K, G.Q4_K))
           for c in range(copies)]
    dense = {nm: [G.DenseWeight(dev, G.Q4_K, r, cc, att[nm]) for _ in range(copies)]
             for nm, r, cc in (("wq", nh * hd, d), ("wk", nkv * hd, d), ("wv", nkv * hd, d), ("wo", d, nh * hd))}
    head = G.DenseWeight(dev, G.Q6_K, vocab, d, head_raw)
    # the window is C5's context (2048): graph-replayed steps attend over the live
    # context's chunk bucket, whatever the window
    kv = KvCache(dev, nl, nh, nkv, hd, block_size=16, max_positions=max(2048, prompt + steps + 8), max_seqs=nseq,
                 rope_theta=1e6)
    pick = [l % copies for l in range(nl)]
    # the token table kept packed (Q6_K rows, 107 MB instead of 524 MB of f32), a row
    # dequantised per token
    embd_raw = M.quantize(G.Q6_K, table.reshape(-1), threads)
    model = G.DecodeModel(dev, kv, [moe[c] for c in pick], *[[dense[nm][c] for c in pick] for nm in ("wq", "wk", "wv", "wo")],
                          head, np.stack([norms[2 * c] for c in pick]), np.stack([norms[2 * c + 1] for c in pick]),
                          norms[-1], (G.Q6_K, embd_raw, vocab, d))
    seqs = [kv.open_seq() for _ in range(nseq)]
    toks = np.random.default_rng(seed & 0xffffffff).integers(0, vocab, (nseq, prompt)).astype(np.uint32)
    # the prompts through gmoe_model_prefill (forward_tail): one call a sequence, its 128
    # tokens one chunk, every layer over the chunk at once (the MFMA/packed prefill paths)
    model.prefill(seqs[0], toks[0, :8])  # warm-up (scratch sizing), on a sequence of its own
    kv.close_seq(seqs[0])
    seqs[0] = kv.open_seq()
    t0 = time.perf_counter()
    nxt = np.array([model.prefill(s, toks[i])[0] for i, s in enumerate(seqs)], np.uint32)
    prompt_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(steps):
        nxt = model.decode_step(seqs, nxt)
    dt = time.perf_counter() - t0
    tps = nseq * steps / dt
    log(f"c5 end to end: {tps:.0f} tok/s ({dt / steps * 1e3:.2f} ms per batch-{nseq} step of {nl} layers, "
        f"contexts {prompt + 1}-{prompt + steps}); prompts prefilled at {nseq * prompt / prompt_s:.0f} tok/s "
        f"({prompt_s * 1e3 / nseq:.1f} ms per {prompt}-token prompt), weights made in {gen_s:.1f}s")
    res = {"workload": f"C5 end to end: {nl} Mixtral-shape layers (Q3_K gate/up, Q4_K down and attention "
                       f"projections, Q6_K head, Q6_K token table kept packed, GQA 32/8 of 128, paged KV cache "
                       f"with a 2048-position window) cycling over {copies} HBM copies of one synthetic layer; "
                       f"{nseq} sequences, {prompt}-token prompts prefilled one sequence a call (chunks run "
                       f"layer-major), then {steps} timed greedy decode steps of all {nseq}",
           "tokens_per_s": tps, "ms_per_step": dt / steps * 1e3, "layers": nl, "sequences": nseq,
           "prompt": prompt, "steps": steps, "prefill_tokens_per_s": nseq * prompt / prompt_s,
           "prefill_ms_per_prompt": prompt_s * 1e3 / nseq, "cpu": None}
    model.close()
    kv.close()
    for ws in dense.values():
        for w in ws:
            w.release()
    head.release()
    for m in moe:
        m.release()
    dev.close()
    if cpu:
        from oracle import oracle as O  # the checker's restatement, timed as the CPU path
        from oracle.model import ModelOracle
        layers = [dict(attn_norm=norms[2 * c], ffn_norm=norms[2 * c + 1],
                       wq=(O.Q4_K, att["wq"], nh * hd, d), wk=(O.Q4_K, att["wk"], nkv * hd, d),
                       wv=(O.Q4_K, att["wv"], nkv * hd, d), wo=(O.Q4_K, att["wo"], d, nh * hd),
                       moe=dict(d=d, f=f, ne=ne, k=k, router=routers[c], qtypes=(O.Q3_K, O.Q3_K, O.Q4_K), packed=1,
                                gate=ex["gate"], up=ex["up"], down=ex["down"]))
                  for c in pick]
        ctx = prompt + steps // 2  # the middle of the GPU's timed steps
        orc = ModelOracle(layers, (O.Q6_K, head_raw, vocab, d), norms[-1], table, nh, nkv, hd,
                          max_positions=ctx + 2, rope_theta=1e6, threads=threads)
        # every sequence's cache holds ctx positions (random keys and values: only the
        # step's cost is measured), so the step attends over as many as the GPU's do
        kr = np.random.default_rng(SEED & 0xFFFF)
        for sq in range(nseq):
            for l in range(nl):
                K_, V_ = orc.kv._kv(sq, l)
                K_.extend(kr.normal(0, 1, (ctx, nkv * hd)).astype(np.float32))
                V_.extend(kr.normal(0, 1, (ctx, nkv * hd)).astype(np.float32))
        t0 = time.time()
        orc.decode_step(list(range(nseq)), toks[:, 0])
        wall = time.time() - t0
        res["cpu"] = cpu_record(nseq / wall, "tokens/s", threads,
                                f"one batch-{nseq} decode step of the {nl}-layer model at context {ctx + 1} (the "
                                f"middle of the GPU's timed steps), oracle restatement of logits_batch (packed int8 "
                                f"products), {threads} threads, {wall:.1f}s")
        log(f"c5 end to end on the CPU: {nseq / wall:.2f} tok/s on {threads} threads")
    return res


def c1_leg(a, dev, threads, cpu):
    """garuda's synthetic engine (MoeEngine) generalised to 4 layers,
    d 256, 8 query / 2 kv heads of 32, 8 experts top-2 of 512, vocab 512, its f32 weights from
    the engine's seeded generator and its experts through the L2 tier (synthesised into a
    temporary directory, then staged into the slab). Batch-1 greedy decode of 64 tokens
    after a 16-token prompt fed one token per step, on the GPU and, as the CPU figure, in
    the oracle's restatement (configuration 1 is not runnable on the reference itself: its
    engine is one MHA block)."""
    import tempfile

    from garuda_amd.synthetic import SyntheticEngine

    dims = dict(n_layers=4, d_model=256, n_heads=8, n_kv_heads=2, head_dim=32, d_ff=512, n_experts=8, top_k=2,
                vocab=512)
    prompt = np.random.default_rng(SEED & 0xFFFFFFFF).integers(0, dims["vocab"], 16)
    n_new = a.c1_tokens

    def run(step, open_seq):
        seq = open_seq()
        t0 = time.perf_counter()
        for t in prompt:
            nxt = step(seq, int(t))
        t1 = time.perf_counter()
        toks = []
        for _ in range(n_new):
            toks.append(int(nxt))
            nxt = step(seq, int(nxt))
        return toks, t1 - t0, time.perf_counter() - t1

    with tempfile.TemporaryDirectory() as td, SyntheticEngine(dev, td, max_positions=2048, **dims) as eng:
        gstep = lambda seq, t: eng.step([seq], [t])[0]
        run(gstep, eng.open_seq)  # warm-up pass (its own sequence)
        gtoks, gp, gd = run(gstep, eng.open_seq)
    out = {"workload": "C1 synthetic engine restated: 4 layers d256 GQA 8/2 hd32, 8 experts top-2 of 512, "
                       "vocab 512, f32 seeded weights, experts through the L2 tier; batch-1 greedy decode",
           "prompt_tokens": len(prompt), "decode_tokens": n_new,
           "prompt_tokens_per_s": len(prompt) / gp, "decode_tokens_per_s": n_new / gd,
           "ms_per_decode_step": gd / n_new * 1e3}
    log(f"c1: {out['decode_tokens_per_s']:.0f} decode tok/s ({out['ms_per_decode_step']:.3f} ms a step), "
        f"prompt {out['prompt_tokens_per_s']:.0f} tok/s")
    if cpu:
        from oracle.model import synthetic_engine
        orc = synthetic_engine(dims["n_layers"], dims["d_model"], dims["n_heads"], dims["n_kv_heads"],
                               dims["head_dim"], dims["d_ff"], dims["n_experts"], dims["top_k"], dims["vocab"],
                               max_positions=256, threads=threads)
        cseq = iter(range(1 << 30))
        ctoks, cp, cd = run(lambda seq, t: orc.decode_step([seq], [t])[0][0], lambda: next(cseq))
        same = sum(1 for x, y in zip(gtoks, ctoks) if x == y)
        out["cpu_restatement"] = {"value": n_new / cd, "unit": "tokens/s", "cores": threads, "kind": "port",
                                  "sample": f"the same {len(prompt)}-token prompt and {n_new} greedy tokens through "
                                            f"the oracle's restatement (oracle.model.synthetic_engine), "
                                            f"{cd:.2f}s for the decode tokens"}
        out["greedy_tokens_equal"] = f"{same}/{n_new}"
        log(f"c1 cpu restatement: {n_new / cd:.1f} tok/s; greedy tokens equal {same}/{n_new}")
    return out


def gguf_leg(a, dev, mats, threads):
    """The slab's source, a GGUF checkpoint: the C2 layer written as a one-layer GGUF
    checkpoint (stacked Q4_K experts, F32 router), then Gguf.open + MoeLayer.from_gguf timed
    to the end of staging: the mapped file's expert bytes copied through the pinned double
    buffer, over the host link, and tiled into the HBM slab. Beside it, the host link's own
    rate for a pinned copy of one expert's bytes, with HIP events."""
    import shutil
    import tempfile

    import torch
    import garuda_amd as G
    from garuda_amd import gguf as gg
    from garuda_amd import moe as M

    tmp = Path(tempfile.mkdtemp(prefix="gmoe_gguf_"))
    try:
        router = M.fill_gaussian(SEED + 0x500, NE * D, 0.0, 0.02, threads)
        meta = [("general.architecture", gg.STRING, "llama"), ("llama.embedding_length", gg.U32, D),
                ("llama.feed_forward_length", gg.U32, F), ("llama.block_count", gg.U32, 1),
                ("llama.expert_count", gg.U32, NE), ("llama.expert_used_count", gg.U32, K)]
        tensors = [("blk.0.ffn_gate_inp.weight", [D, NE], G.F32, router),
                   ("blk.0.ffn_gate_exps.weight", [D, F, NE], G.Q4_K, mats["gate"]),
                   ("blk.0.ffn_up_exps.weight", [D, F, NE], G.Q4_K, mats["up"]),
                   ("blk.0.ffn_down_exps.weight", [F, D, NE], G.Q4_K, mats["down"])]
        path = tmp / "c2_layer.gguf"
        size = gg.write_gguf_file(path, meta, tensors)
        staged = NE * 3 * M.byte_size(G.Q4_K, F * D)
        times = []
        for _ in range(a.gguf_reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with G.Gguf.open(path) as g:
                layer = G.MoeLayer.from_gguf(dev, g, 0)
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
                layer.release()
        nb = staged // NE
        host = torch.empty(nb, dtype=torch.uint8, pin_memory=True)
        devb = torch.empty(nb, dtype=torch.uint8, device="cuda")
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        link = []
        for _ in range(3):
            ev0.record()
            devb.copy_(host, non_blocking=True)
            ev1.record()
            torch.cuda.synchronize()
            link.append(nb / (ev0.elapsed_time(ev1) / 1e3) / 1e9)
        del host, devb
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    best = min(times)
    gbs, link_gbs = staged / best / 1e9, max(link)
    log(f"gguf: {size / 1e6:.0f} MB file, {staged / 1e6:.0f} MB of experts staged into HBM in "
        f"{best * 1e3:.0f} ms ({gbs:.1f} GB/s; pinned host->device copy {link_gbs:.1f} GB/s)")
    return {"workload": "C2 layer as a one-layer GGUF checkpoint (stacked Q4_K experts): open + register, "
                        "mapped file -> pinned double buffer -> HBM slab, page-cache resident file",
            "file_bytes": size, "staged_bytes": staged, "seconds": best, "reps": len(times),
            "GB_s": gbs, "link_GB_s": link_gbs, "frac_of_link": gbs / link_gbs}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--batch", type=int, default=8, help="tokens per step for the headline value")
    ap.add_argument("--sweep", default="1,2,4,8", help="other decode batch sizes to report")
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--math", choices=("packed", "f32"), default="packed")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-calls", type=int, default=10, help="timed calls of the CPU baseline (median)")
    ap.add_argument("--kernel-events", choices=("on", "off"), default="on",
                    help="also time the steps with HIP events around every gate/up and down launch "
                         "(the roofline's kernel times); off skips that second pass")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="also run one device-to-device copy of MB MiB (the counter calibration of profiles/)")
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="tokens of the C3 prefill legs (Zipf-skewed routing, f32 and packed math on MFMA); 0 skips them")
    ap.add_argument("--prefill-steps", type=int, default=40)
    ap.add_argument("--prefill-cpu-tokens", type=int, default=32,
                    help="tokens of the C3 CPU sample (the f32 path runs about 30 ms a token on 16 threads)")
    ap.add_argument("--prefill-layers", type=int, default=2)
    ap.add_argument("--dense", type=int, default=1, help="run the dense-projection leg (0: skip)")
    ap.add_argument("--attention", type=int, default=1, help="run the paged-attention leg (0: skip)")
    ap.add_argument("--prefetch-steps", type=int, default=200,
                    help="decode steps of the prefetch leg, each way (0: skip it)")
    ap.add_argument("--gguf-reps", type=int, default=3,
                    help="timed open+register passes of the GGUF staging leg (0: skip it)")
    ap.add_argument("--e2e-layers", type=int, default=32,
                    help="layers of the C5 end-to-end decode leg (0: skip it)")
    ap.add_argument("--e2e-prompt", type=int, default=128, help="prompt tokens per sequence of the end-to-end leg")
    ap.add_argument("--e2e-steps", type=int, default=32, help="timed decode steps of the end-to-end leg")
    ap.add_argument("--c1-tokens", type=int, default=64,
                    help="greedy decode tokens of the C1 synthetic-engine leg after its 16-token prompt (0: skip)")
    ap.add_argument("--extra", default="c4,c5_layer",
                    help="further BASELINE configurations to time at decode (c4, c5_layer); empty skips")
    a = ap.parse_args()

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(the path would shard by expert, one exchange each way). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import garuda_amd as G
    from garuda_amd import moe as M

    threads = len(os.sched_getaffinity(0))
    t0 = time.time()
    mats = make_experts(threads)
    log(f"experts generated and quantised in {time.time() - t0:.1f}s ({sum(m.size for m in mats.values()) / 1e6:.0f} MB packed)")

    math = G.MATH_PACKED if a.math == "packed" else G.MATH_F32
    expert_bytes = 3 * M.byte_size(G.Q4_K, F * D)
    n_pf_layers = a.prefill_layers if a.prefill_tokens else 0
    # + the further configurations' 2 copies each (C4 ~0.55 GB, C5 slice ~0.67 GB per copy)
    slab = (a.layers + n_pf_layers) * NE * (expert_bytes + 3 * 4096) + (256 << 20) + (3 << 30)
    dev = G.Device(0, slab_bytes=slab)
    layers = []
    t0 = time.time()
    for l in range(a.layers):
        router = M.fill_gaussian(SEED + 0x100 + l, NE * D, 0.0, 0.02, threads)
        layers.append(G.MoeLayer(dev, D, F, NE, K, router, mats["gate"], mats["up"], mats["down"],
                                 (G.Q4_K,) * 3, math=math))
    log(f"{a.layers} layers staged into HBM in {time.time() - t0:.1f}s")

    # a stream of its own (default priority): torch's default stream is the null stream,
    # which the library's non-blocking streams do not order against
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    sh = stream.cuda_stream

    def timed(step, steps, events):
        """`steps` calls of step(i) between two synchronisations; with events, also the
        gate/up and down launch times (HIP events on the stream around each launch)."""
        dev.kernel_time(0)  # drain
        base = [dev.kernel_time(w) for w in range(3)]
        dev.set_kernel_timing(events)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record(stream)
        for i in range(steps):
            step(i)
        ev1.record(stream)
        torch.cuda.synchronize()
        dev.set_kernel_timing(False)
        kt = [dev.kernel_time(w) for w in range(3)]
        cnt = max(kt[0][1] - base[0][1], 1)
        return ev0.elapsed_time(ev1), [(kt[w][0] - base[w][0]) / cnt for w in range(3)]

    results = {}
    batches = sorted(set([a.batch] + [int(b) for b in a.sweep.split(",") if b]))
    for n in batches:
        hs = torch.from_numpy(M.fill_gaussian(SEED + 0x200 + n, n * D, 0.0, 1.0, threads).reshape(n, D)).cuda()
        out = torch.empty((n, D), dtype=torch.float32, device="cuda")
        ids = torch.empty((len(layers), n, K), dtype=torch.int32, device="cuda")
        wts = torch.empty((len(layers), n, K), dtype=torch.float32, device="cuda")

        def step(i):
            l = i % len(layers)
            layers[l].forward_async(hs.data_ptr(), n, out.data_ptr(), ids[l].data_ptr(), wts[l].data_ptr(),
                                    0, sh)

        for i in range(a.warmup):
            step(i)
        torch.cuda.synchronize()
        # the throughput is timed bare (the per-launch events cost ~3 us each); the kernel
        # times come from a second pass over the same steps with events around each launch
        ms, _ = timed(step, a.steps, False)
        ms_ev, kms = timed(step, a.steps, a.kernel_events == "on")
        nan = float("nan")
        gu_ms, dn_ms, ex_ms = kms if a.kernel_events == "on" else (nan, nan, nan)
        touched = [len(np.unique(ids[l].cpu().numpy())) for l in range(len(layers))]
        # steps cycle through the layers evenly
        e_avg = float(np.mean([touched[i % len(layers)] for i in range(a.steps)]))
        gu_bytes = e_avg * 2 * M.byte_size(G.Q4_K, F * D) + n * D + n * K * F  # weights + int8 x in + int8 h out
        dn_bytes = e_avg * M.byte_size(G.Q4_K, D * F) + n * K * F + n * K * D * 4
        layer_bytes = e_avg * expert_bytes + NE * D * 4 + 2 * n * D * 4
        results[n] = dict(
            tokens_per_s=n * a.steps / (ms / 1e3), ms_per_step=ms / a.steps, experts_touched=e_avg,
            gateup_us=gu_ms * 1e3, down_us=dn_ms * 1e3, experts_us=ex_ms * 1e3,
            gateup_GBs=gu_bytes / (gu_ms / 1e3) / 1e9, down_GBs=dn_bytes / (dn_ms / 1e3) / 1e9,
            layer_GBs=layer_bytes / (ms / a.steps / 1e3) / 1e9, gateup_bytes=gu_bytes)
        log(f"n={n}: {results[n]['tokens_per_s']:.0f} tok/s, {ms / a.steps * 1e3:.1f} us/step, "
            f"E={e_avg:.2f}, gate/up {gu_ms * 1e3:.1f} us ({results[n]['gateup_GBs']:.0f} GB/s), "
            f"down {dn_ms * 1e3:.1f} us ({results[n]['down_GBs']:.0f} GB/s), layer {results[n]['layer_GBs']:.0f} GB/s")

    prefill = prefill_packed = None
    if a.prefill_tokens:
        prefill = prefill_leg(a, dev, mats, threads, stream, timed, not a.no_cpu)
        prefill_packed = prefill_leg(a, dev, mats, threads, stream, timed, not a.no_cpu, packed=True)
    extra = {}
    for name in [x for x in a.extra.split(",") if x]:
        extra[name] = extra_leg(name, a, dev, threads, stream, timed, not a.no_cpu)

    dense = dense_leg(a, dev, threads, stream, timed) if a.dense else None
    prefetch = prefetch_leg(a, mats, threads) if a.prefetch_steps > 0 else None
    attention = attention_leg(a, dev, threads, stream, timed) if a.attention else None
    gguf = gguf_leg(a, dev, mats, threads) if a.gguf_reps > 0 else None
    e2e = e2e_leg(a, threads, not a.no_cpu) if a.e2e_layers > 0 else None
    c1 = c1_leg(a, dev, threads, not a.no_cpu) if a.c1_tokens > 0 else None

    if a.calibrate_copy:
        src = torch.empty(a.calibrate_copy << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {a.calibrate_copy} MiB read, {a.calibrate_copy} MiB written")
        del src, dst

    cpu = None
    if not a.no_cpu:
        from oracle import oracle as O
        n = a.batch
        hs_np = M.fill_gaussian(SEED + 0x200 + n, n * D, 0.0, 1.0, threads).reshape(n, D)
        L = dict(d=D, f=F, ne=NE, k=K, packed=1 if math == G.MATH_PACKED else 0,
                 router=layers[0].router, qtypes=(G.Q4_K,) * 3, **mats)
        med, calls = cpu_median(lambda: O.feed_forward_batch(L, hs_np, threads=threads), calls=a.cpu_calls)
        cpu = cpu_record(n / med, "tokens/s", threads,
                         f"median of {calls} calls (one warm-up call before) of the C2 layer at batch {n} "
                         f"(layer 0), oracle restatement of quant::matmul's packed int8 path, rows split over "
                         f"{threads} threads")
        log(f"cpu baseline: {cpu['value']:.1f} tok/s on {threads} threads")

    r = results[a.batch]
    gu_s = r["gateup_us"] / 1e6
    line = {
        "metric": "MoE-layer tokens/s (Q4_K Mixtral-shape decode, 1 MI355X)",
        "value": r["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if math == G.MATH_PACKED else "f32",
        "data": "synthetic (N(0,0.02^2) weights quantised to Q4_K by this build; N(0,1) activations)",
        "config": {"workload": f"C2 decode: Mixtral-shape MoE layer d4096 f14336 8 experts top-2 Q4_K, "
                               f"batch {a.batch}, {a.layers} HBM copies rotated",
                   "batch": a.batch, "d_model": D, "d_ff": F, "n_experts": NE, "top_k": K, "qtype": "Q4_K",
                   "math": a.math},
        "roofline": {"bound": "hbm", "kernel": f"k_gu_units<Q4_K, {a.math} math>",
                     "achieved": r["gateup_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": r["gateup_GBs"] / HBM_PEAK_GBS,
                     "traffic": measured_traffic(a.batch, a.math, a.layers),
                     "bytes_per_launch": r["gateup_bytes"], "avg_launch_us": r["gateup_us"],
                     # the whole layer step (front end, gate/up, down) against the same peak:
                     # its algorithmic bytes over the bare step time
                     "layer_achieved": r["layer_GBs"], "layer_frac": r["layer_GBs"] / HBM_PEAK_GBS},
        "cpu_baseline": cpu,
        "prefill": prefill,
        "prefill_packed": prefill_packed,
        "configs": extra,
        "dense_projections": dense,
        "prefetch": prefetch,
        "attention": attention,
        "gguf_staging": gguf,
        "c5_end_to_end": e2e,
        "c1_synthetic_engine": c1,
        "sweep": {str(n): {k: (round(v, 3) if isinstance(v, float) else v) for k, v in res.items()}
                  for n, res in results.items()},
    }
    print(json.dumps(line), flush=True)
    for l in layers:
        l.release()
    dev.close()


if __name__ == "__main__":
    main()
