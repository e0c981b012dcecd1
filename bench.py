#!/usr/bin/env python3
"""bench.py -- one DeepSeek-R1 MoE layer (loki's fused_layer MoE block) on one MI355X.

Default workload (the north star's target config, configs[0]): one MoE layer decoding 1 token:
x [1, 7168] ~ N(0,1), fp32 router [256, 7168] ~ N(0, 0.02^2), bias ~ N(0, 0.01^2), grouped sigmoid routing
(8 groups, top-4 groups, top-8, x2.5), 256 routed + 1 shared IQ2_XXS experts (gate/up [2048, 7168], down [7168, 2048],
qs uniform bytes, d = fp16(|N(0, 0.002^2)|)). All inputs are generated on the device and resident in HBM before the
timed region. Before each workload's warm-up steps the GPU runs the same workload untimed for --preheat-ms (default
100 ms): a cold GPU's first ~20-30 ms of load run at lower clocks. Each step takes a fresh x (so different experts) and the steps rotate over --copies independently seeded
layers (default 8 x 2.9 GB), so the 256 MB MALL cannot serve repeated weights.

Prints ONE JSON line: value = microseconds per token of the whole block (router, dispatch, experts, combine), plus the
achieved HBM bandwidth, the roofline of the dominant kernel (decode: the whole block in one launch, k_moe_decode1
for one token, k_moe_decode for batches; prefill: the gate/up expert kernel), timed live with HIP events recorded on the stream the kernel runs on, and
the CPU checker timed on this host's cores on a bounded sample of every config. decode-8, prefill-512, prefill-2048,
the 58-layer stack and the real-shard formats are reported under `extra`. Every timed loop ends with fl_sync: a
device-side failure (a bounded wait of the decode block that timed out) makes the run exit non-zero instead of
recording a fast invalid step.
"""
import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0         # MI355X dense int8 MFMA, published
MAT_BYTES = 2048 * (7168 // 256) * 66   # one IQ2_XXS expert matrix: 3,784,704 B
EXPERT_BYTES = 3 * MAT_BYTES            # 11,354,112 B
ROUTER_BYTES = 256 * 7168 * 4 + 256 * 4  # router W + bias
E, H = 7168, 2048

WORKLOADS = {
    # name: (tokens, bias sigma, hot experts, description)
    "decode1": (1, 0.01, 0, "decode-1: one MoE layer, 1 token"),
    "decode8": (8, 0.01, 0, "decode-8: one MoE layer, batch of 8 tokens"),
    "prefill512": (512, 0.05, 0, "prefill-512: one MoE layer, 512 tokens"),
    "prefill2048": (2048, 0.05, 16, "prefill-2048: one MoE layer, 2048 tokens, 16 hot experts (+0.5 bias)"),
}
STACK_LAYERS = 58   # configs[3]: DeepSeek-R1's MoE layers, every expert of every layer resident (~169 GB)


class no_gc:
    """The drop-in flows' warm-up and host-timed loops run with Python's garbage collector off, collected once before
    the warm-up: a collection pass in a process holding many objects stalled one library call per full run by tens of
    ms of host time, which is the harness's, not the library's. (The device-timed loops keep the collector: a
    collection right before them idles the GPU and lowers its clocks for the first timed steps.)"""
    def __enter__(self):
        import gc
        gc.collect(); self.was = gc.isenabled(); gc.disable()
        return self

    def __exit__(self, *exc):
        import gc
        if self.was:
            gc.enable()
        return False


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def step_bytes(n, U):
    """Algorithmic HBM bytes of one block call: every used expert (and the shared one) read once, the router once,
    x read and y written once."""
    return (U + 1) * EXPERT_BYTES + ROUTER_BYTES + 2 * n * E * 4


def gateup_bytes(n, U, topk=8):
    """Algorithmic bytes of one gate/up launch: gate+up of every used expert and the shared one, Q8_K x, h written."""
    P = n * topk
    return 2 * (U + 1) * MAT_BYTES + n * (E + E // 256 * 4) + (P + n) * H * 4


def routing_margins(probs, bias, n_group=8, topk_group=4, topk=8):
    """How close the routing of these rows came to a tie: per row, the gap between the topk-th and the next eligible
    biased score c = p + bias (inside the kept groups), and the gap between the topk_group-th and the next group score
    (top1 + top2 of c per group). Returns the minimum of each over the rows (fp32, as the selection compares them)."""
    import numpy as np
    c = (np.asarray(probs, np.float32) + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    n, ne = c.shape
    per = ne // n_group
    g = np.sort(c.reshape(n, n_group, per), axis=2)[:, :, ::-1]
    gs = (g[:, :, 0] + g[:, :, 1]).astype(np.float32)
    order = np.argsort(-gs, axis=1, kind="stable")
    gsort = np.take_along_axis(gs, order, axis=1)
    gmargin = gsort[:, topk_group - 1] - gsort[:, topk_group] if topk_group < n_group else np.full(n, np.inf)
    keep = np.zeros((n, n_group), bool)
    np.put_along_axis(keep, order[:, :topk_group], True, axis=1)
    ce = np.where(np.repeat(keep, per, axis=1), c, -np.inf)
    cs = -np.sort(-ce, axis=1)
    kmargin = cs[:, topk - 1] - cs[:, topk]
    return float(np.min(kmargin)), float(np.min(gmargin))


def distinct_experts(ctx, layer, xs):
    """Number of distinct routed experts per x (routing recomputed outside the timed region)."""
    out = []
    for x in xs:
        _, _, sel, _ = ctx.route(layer.gate_inp, layer.probs_b, x)
        out.append(int(sel.unique().numel()))
    return out


PREHEAT_MS = 100.0   # --preheat-ms


def preheat(torch, step):
    """Runs step(i) untimed for PREHEAT_MS of wall time before a workload's warm-up steps. An idle MI355X runs its first
    ~20-30 ms of load at lower clocks (measured: decode-8 per-50-step averages 216, 184, 174, 171, 170 us from a cold
    start, decode-1 41.5, 33.5, 33.9, 32.6, 31.6, 30.8, 30.4, 30.2 us), so a handful of warm-up steps would time the
    power management's ramp rather than the kernels; the timed steps themselves are unchanged."""
    t0 = time.perf_counter()
    i = 0
    while True:
        step(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= PREHEAT_MS:
                return i


def run_workload(ctx, torch, name, steps, warmup, copies, seed=20260101):
    from loki_amd import MoeLayerWeights
    n, bias_sigma, nhot, desc = WORKLOADS[name]
    layers = []
    for c in range(copies):
        hot = None
        if nhot:
            g = torch.Generator().manual_seed(seed + 7 * c)
            hot = torch.randperm(256, generator=g)[:nhot].tolist()
        layers.append(MoeLayerWeights.synthetic(ctx, seed + 1000 * c, bias_sigma=bias_sigma, hot=hot))
    nx = steps + warmup
    xs = []
    for i in range(nx):
        x = torch.empty((n, E), dtype=torch.float32, device="cuda")
        ctx.synth_normal(x, seed + 17, 1000 + i, 0.0, 1.0)
        xs.append(x)
    y = torch.empty((n, E), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    preheat(torch, lambda i: ctx.moe_layer(layers[i % copies], xs[i % nx], y))
    for i in range(warmup):
        ctx.moe_layer(layers[i % copies], xs[i], y)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    h0 = time.perf_counter()
    for i in range(steps):
        ctx.moe_layer(layers[(warmup + i) % copies], xs[warmup + i], y)
    host_us = (time.perf_counter() - h0) * 1e6 / steps
    end.record()
    torch.cuda.synchronize()
    ctx.sync()   # a device-side failure in any timed step raises here
    ms = start.elapsed_time(end) / steps
    dbg = ctx.debug()
    fused, dkernel = bool(dbg.fused), dbg.kernel
    if fused:
        # one launch per step, issued back to back on the library's stream: the timed region's per-step time is the
        # launch's average duration
        stage = {"gate_up": ms}
    else:
        # same steps again with per-stage HIP events (stage durations for the roofline; not used for `value`)
        ctx.stage_ms(reset=True)
        ctx.set_profile(True)
        for i in range(steps):
            ctx.moe_layer(layers[(warmup + i) % copies], xs[warmup + i], y)
        ctx.set_profile(False)
        calls, stage = ctx.stage_ms(reset=True)
        ctx.sync()
        stage = {k: v / max(calls, 1) for k, v in stage.items()}
    U, km, gm = [], [], []
    for i in range(steps):
        L = layers[(warmup + i) % copies]
        _, probs, sel, _ = ctx.route(L.gate_inp, L.probs_b, xs[warmup + i])
        U.append(int(sel.unique().numel()))
        k, g = routing_margins(probs.cpu().numpy(), L.probs_b.cpu().numpy())
        km.append(k); gm.append(g)
    ctx.sync()
    mean_U = sum(U) / len(U)
    res = dict(name=name, desc=desc, n=n, ms=ms, U=mean_U, stage_ms=stage, fused=fused, dkernel=dkernel, host_us=host_us,
               margins={"topk_min": min(km), "group_min": min(gm)},
               bytes=sum(step_bytes(n, u) for u in U) / len(U),
               gu_bytes=sum(gateup_bytes(n, u) for u in U) / len(U))
    res["gbs"] = res["bytes"] / (ms * 1e-3) / 1e9
    res["layers"], res["xs"] = layers, xs
    return res


def run_stack(ctx, torch, steps, warmup, nlayers=STACK_LAYERS, seed=20260301, cpu_sample=False):
    """one token through nlayers independently seeded MoE layers, x_{L+1} = RMSNorm(y_L) (weights 1,
    eps 1e-6; the norm runs inside the next layer's block). A step is the whole chain for one fresh x; bytes = nlayers
    x the decode-1 bytes of a layer."""
    from loki_amd import MoeLayerWeights
    t0 = time.perf_counter()
    layers = [MoeLayerWeights.synthetic(ctx, seed + 1000 * L, bias_sigma=0.01) for L in range(nlayers)]
    torch.cuda.synchronize()
    t_synth = time.perf_counter() - t0
    xs = []
    for i in range(steps + warmup):
        x = torch.empty((1, E), dtype=torch.float32, device="cuda")
        ctx.synth_normal(x, seed + 17, 2000 + i, 0.0, 1.0)
        xs.append(x)
    ys = [torch.empty((1, E), dtype=torch.float32, device="cuda") for _ in range(2)]

    def token(x):   # layer L > 0 normalises y_{L-1} inside its block (fl_moe_layer_normed)
        ctx.moe_layer(layers[0], x, ys[0])
        for i, L in enumerate(layers[1:]):
            ctx.moe_layer_normed(L, ys[i % 2], None, 1e-6, ys[(i + 1) % 2])

    preheat(torch, lambda i: token(xs[i % len(xs)]))
    for i in range(warmup):
        token(xs[i])
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        token(xs[warmup + i])
    end.record()
    torch.cuda.synchronize()
    ctx.sync()
    ms = start.elapsed_time(end) / steps
    nbytes = nlayers * step_bytes(1, 8)
    cpu = cpu_stack_sample(ctx, layers, xs[warmup]) if cpu_sample else None
    del layers
    torch.cuda.empty_cache()
    return {"layers": nlayers, "us_per_token": round(ms * 1e3, 1), "ms_per_step": round(ms, 4), "cpu": cpu,
            "bytes_per_token": nbytes, "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "us_per_layer": round(ms * 1e3 / nlayers, 2),
            "resident_weight_gb": round(nlayers * (257 * EXPERT_BYTES + ROUTER_BYTES) / 1e9, 1),
            "synth_s": round(t_synth, 1)}


# K-quant formats of the reference's real shards: block bytes and fp16 d / dmin offsets (FL_* codes)
KQ = {5: ("q2_K", 84, 80, 82), 6: ("q3_K", 110, 108, None), 3: ("q5_K", 176, 0, 2), 1: ("q6_K", 210, 208, None)}


def kq_random(torch, fmt, R, K, seed):
    """random K-quant matrix bytes on the device: uniform quant/scale bytes, fp16 d (and dmin) in [6e-5, 4e-3]"""
    _, bs, od, om = KQ[fmt]
    nb = R * (K // 256)
    g = torch.Generator(device="cuda").manual_seed(seed)
    blk = torch.randint(0, 256, (nb, bs), dtype=torch.uint8, device="cuda", generator=g)
    for off in (od, om):
        if off is not None:
            d = torch.randint(0x0C00, 0x1C00, (nb,), dtype=torch.int32, device="cuda", generator=g).to(torch.int16)
            blk[:, off:off + 2] = d.view(torch.uint8).view(nb, 2)
    return blk.view(-1)


def run_kquant(ctx, torch, iters=20, seed=20260401):
    """fl_kq_matvec_dev on the decode shapes of the reference's real formats, each launch reading weights from HBM
    (copies rotated past the 256 MB MALL): the routed down of 64 experts x 1 token as one 458,752-row matrix (Q2_K,
    Q3_K), and the shared expert's gate (Q5_K, [2048, 7168]) and down (Q6_K, [7168, 2048]) on 8 tokens."""
    out = {}
    cases = (("routed_down_q2_K_64x1", 5, 64 * E, H, 1, 1), ("routed_down_q3_K_64x1", 6, 64 * E, H, 1, 1),
             ("shared_gate_q5_K_x8", 3, H, E, 8, 32), ("shared_down_q6_K_x8", 1, E, H, 8, 24))
    for name, fmt, R, K, n, copies in cases:
        ws = [kq_random(torch, fmt, R, K, seed + 31 * c + fmt) for c in range(copies)]
        x = torch.empty((n, K), dtype=torch.float32, device="cuda")
        ctx.synth_normal(x, seed, fmt, 0.0, 1.0)
        q, d = ctx.quant_q8k(x)
        y = torch.empty((n, R), dtype=torch.float32, device="cuda")
        for i in range(3):
            ctx.kq_matvec(fmt, ws[i % copies], R, K, q, d, y)
        torch.cuda.synchronize()
        reps = max(iters, copies)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(reps):
            ctx.kq_matvec(fmt, ws[i % copies], R, K, q, d, y)
        t1.record()
        torch.cuda.synchronize()
        ctx.sync()
        us = t0.elapsed_time(t1) * 1e3 / reps
        wb = R * (K // 256) * KQ[fmt][1]
        out[name] = {"us_per_launch": round(us, 2), "weight_bytes": wb, "hbm_gbs": round(wb / us / 1e3, 1),
                     "hbm_frac": round(wb / us / 1e3 / HBM_PEAK_GBS, 4)}
        log("[bench] kquant %s: %s" % (name, json.dumps(out[name])))
        del ws, x, q, d, y
        torch.cuda.empty_cache()
    return out


def run_dropin(ctx, torch, steps=60, warmup=5, ggml_steps=3, seed=20260601):
    """The reference-named path at decode-1, as the engine drives it (src/server_core_fused.cpp:946-953): per token
    fl_ffn_begin (router input and residual from the host; routing and shared expert) -> fl_fetch (routing to the host,
    waited) -> fl_moe on the layer's resident 256-expert arena (ids = expert ids, waited; h and moe to the host). The
    arena and the shared expert are tiled and declared (fl_register_tiled), so fl_moe reads them in place; the same
    layer in ggml's layout (undeclared: repacked on every call, the reference's refilled-arena contract) is timed over a
    few tokens for comparison. Times are host wall clock per token (every step ends in a host wait): medians over the
    tokens (the measurement protocol's statistic; an occasional host stall of a few ms moves the mean), the mean beside
    them."""
    import ctypes
    import numpy as np
    from loki_amd import FLOut, FLW, MoeLayerWeights, lib
    L = MoeLayerWeights.synthetic(ctx, seed)
    mats = (L.gate, L.up, L.down, L.sh_gate, L.sh_up, L.sh_down)
    for t in mats:
        ctx.register_tiled(t)
    rng = np.random.default_rng(seed)
    xs = rng.standard_normal((steps + warmup, E)).astype(np.float32)
    fis = rng.standard_normal((steps + warmup, E)).astype(np.float32)
    out = FLOut()
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)

    def flw(sh):
        w = FLW()
        w.gate_inp = L.gate_inp.data_ptr(); w.probs_b = L.probs_b.data_ptr(); w.gate_f16 = 0
        w.sh_gate, w.sh_up, w.sh_down = (m.data_ptr() for m in sh)
        return w

    def token(i, w, g, u, d, split):
        t0 = time.perf_counter()
        ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(w), 1, ptr(xs[i]), ptr(fis[i]), -1))
        t1 = time.perf_counter()
        lib().fl_fetch(ctx.ctx, 1, 1, ctypes.byref(out))
        t2 = time.perf_counter()
        sel = np.ctypeslib.as_array(out.sel, shape=(8,)).astype(np.int32)   # the resident arena: slot id = expert id
        wts = np.ctypeslib.as_array(out.wts, shape=(8,)).copy()
        lib().fl_moe(ctx.ctx, g.data_ptr(), u.data_ptr(), d.data_ptr(), 256, 4, ptr(sel), ptr(wts), 8, 1, ctypes.byref(out))
        t3 = time.perf_counter()
        split.append((t1 - t0, t2 - t1, t3 - t2))

    res = {}
    try:
        w = flw((L.sh_gate, L.sh_up, L.sh_down))
        split = []
        with no_gc():   # collected before the warm-up tokens
            for i in range(warmup):
                token(i, w, L.gate, L.up, L.down, [])
            g0 = ctx.gpu_ms(1)
            for i in range(steps):
                token(warmup + i, w, L.gate, L.up, L.down, split)
            g1 = ctx.gpu_ms(1)
        sp = np.array(split) * 1e6
        # the experts' GPU time per token as the library accounts it (fl_gpu_ms(1): HIP events around each launch, or
        # the one-token launch's own device clock when fl_ffn_begin ran the block): the rest of us_per_token is host
        # calls and launch latency
        res["gpu_moe_us"] = round((g1 - g0) * 1e3 / steps, 1)
        res["us_per_token"] = round(float(np.median(sp.sum(axis=1))), 1)
        res["ffn_begin_us"], res["fetch_us"], res["moe_us"] = (round(float(v), 1) for v in np.median(sp, axis=0))
        res["mean_us_per_token"] = round(float(sp.sum(axis=1).mean()), 1)
        res["tokens"] = steps
    finally:
        for t in mats:
            ctx.unregister_tiled(t)
    # the same layer in ggml's layout, undeclared: fl_ffn_begin packs the shared expert once (cached by pointer) and
    # fl_moe repacks the 256-expert arena on every call
    gg = [ctx.unpack(m, r, c, n) for m, (r, c, n) in zip(mats, ((2048, E, 256), (2048, E, 256), (E, 2048, 256), (2048, E, 1), (2048, E, 1), (E, 2048, 1)))]
    torch.cuda.synchronize()
    w = flw(gg[3:])
    split = []
    token(0, w, gg[0], gg[1], gg[2], [])
    for i in range(ggml_steps):
        token(1 + i, w, gg[0], gg[1], gg[2], split)
    res["ggml_arena_us_per_token"] = round(float(np.median(np.array(split).sum(axis=1))) * 1e6, 1)
    res["ggml_arena_tokens"] = ggml_steps
    del gg, L
    torch.cuda.empty_cache()
    return res


def run_dropin_rows(ctx, torch, n=8, steps=30, warmup=5, seed=20260621):
    """The reference-named path at decode-8 (src/server_core_fused.cpp:946-953 with n = 8 rows): per step fl_ffn_begin
    (8 rows) -> fl_fetch -> fl_moe on the resident, declared 256-expert arena (ids = expert ids). Medians of the host
    wall clock per step over the steps."""
    import ctypes
    import numpy as np
    from loki_amd import FLOut, FLW, MoeLayerWeights, lib
    L = MoeLayerWeights.synthetic(ctx, seed)
    mats = (L.gate, L.up, L.down, L.sh_gate, L.sh_up, L.sh_down)
    for t in mats:
        ctx.register_tiled(t)
    rng = np.random.default_rng(seed)
    xs = rng.standard_normal((steps + warmup, n, E)).astype(np.float32)
    fis = rng.standard_normal((steps + warmup, n, E)).astype(np.float32)
    out = FLOut()
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    w = FLW()
    w.gate_inp = L.gate_inp.data_ptr(); w.probs_b = L.probs_b.data_ptr(); w.gate_f16 = 0
    w.sh_gate, w.sh_up, w.sh_down = (m.data_ptr() for m in (L.sh_gate, L.sh_up, L.sh_down))
    res = {}
    try:
        split = []
        with no_gc():
            for i in range(steps + warmup):
                t0 = time.perf_counter()
                ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(w), n, ptr(xs[i]), ptr(fis[i]), -1))
                t1 = time.perf_counter()
                lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
                t2 = time.perf_counter()
                sel = np.ctypeslib.as_array(out.sel, shape=(n * 8,)).astype(np.int32)
                wts = np.ctypeslib.as_array(out.wts, shape=(n * 8,)).copy()
                lib().fl_moe(ctx.ctx, L.gate.data_ptr(), L.up.data_ptr(), L.down.data_ptr(), 256, 4, ptr(sel), ptr(wts), 8, n, ctypes.byref(out))
                t3 = time.perf_counter()
                if i >= warmup:
                    split.append((t1 - t0, t2 - t1, t3 - t2))
        sp = np.array(split) * 1e6
        step_us = float(np.median(sp.sum(axis=1)))
        res = {"us_per_step": round(step_us, 1), "us_per_token": round(step_us / n, 2), "ffn_begin_us": round(float(np.median(sp[:, 0])), 1),
               "fetch_us": round(float(np.median(sp[:, 1])), 1), "moe_us": round(float(np.median(sp[:, 2])), 1), "tokens": n, "steps": steps}
        log("[bench] drop-in decode-%d: %s" % (n, json.dumps(res)))
    finally:
        for t in mats:
            ctx.unregister_tiled(t)
    del L
    torch.cuda.empty_cache()
    return res


def run_dropin_wide(ctx, torch, n=512, steps=10, warmup=2, seed=20260611):
    """The reference-named prefill path (the engine's wide pass, src/server_core_fused.cpp:733-744, 931-949) at
    prefill-512: per 64-row group fl_ffn_begin(wrow) -> fl_fetch; then the pairs in slots of <= 8 rows per expert (the
    engine's byexp order) as one fl_wide_moe on the layer's resident 256-expert arena (declared tiled; ids = expert ids),
    then fl_wide_finish. The slot tables are built on the host outside the timed calls (the engine's own dispatch); the
    time is the host wall clock of the library calls per step, median over the steps. The same x / ffn_inp every step
    (fresh inputs would only change the routing)."""
    import ctypes
    import numpy as np
    from loki_amd import FLOut, FLW, MoeLayerWeights, lib
    KE, G = 8, 64
    L = MoeLayerWeights.synthetic(ctx, seed, bias_sigma=0.05)
    mats = (L.gate, L.up, L.down, L.sh_gate, L.sh_up, L.sh_down)
    for t in mats:
        ctx.register_tiled(t)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, E)).astype(np.float32)
    fi = rng.standard_normal((n, E)).astype(np.float32)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    w = FLW()
    w.gate_inp = L.gate_inp.data_ptr(); w.probs_b = L.probs_b.data_ptr(); w.gate_f16 = 0
    w.sh_gate, w.sh_up, w.sh_down = (m.data_ptr() for m in (L.sh_gate, L.sh_up, L.sh_down))
    out = FLOut()
    res = {}
    try:
        assert lib().fl_wide_init(ctx.ctx, n, KE) == 1

        def step():
            t_lib = 0.0
            sel = np.empty((n, KE), np.int32); wts = np.empty((n, KE), np.float32)
            for r0 in range(0, n, G):
                t0 = time.perf_counter()
                ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(w), G, ptr(x[r0:r0 + G]), ptr(fi[r0:r0 + G]), r0))
                lib().fl_fetch(ctx.ctx, G, 1, ctypes.byref(out))
                t_lib += time.perf_counter() - t0
                sel[r0:r0 + G] = np.ctypeslib.as_array(out.sel, shape=(G, KE))
                wts[r0:r0 + G] = np.ctypeslib.as_array(out.wts, shape=(G, KE))
            # slots: each expert's (row, k) pairs in row-major order, 8 per slot (vectorised host dispatch)
            fe = sel.ravel()
            order = np.argsort(fe, kind="stable")
            es = fe[order]
            cnt = np.bincount(es, minlength=256)
            first = np.concatenate([[0], np.cumsum(cnt)[:-1]])
            rank = np.arange(es.size) - first[es]
            nsl = (cnt + 7) // 8
            soff = np.concatenate([[0], np.cumsum(nsl)[:-1]])
            slot = soff[es] + rank // 8
            ns = int(nsl.sum())
            midx = np.repeat(np.arange(256, dtype=np.int32), nsl)
            rows = np.full(ns * 8, -1, np.int32); kidx = np.zeros(ns * 8, np.int32); wk = np.zeros(ns * 8, np.float32)
            pos = slot * 8 + rank % 8
            rows[pos] = (order // KE).astype(np.int32); kidx[pos] = (order % KE).astype(np.int32); wk[pos] = wts.ravel()[order]
            t0 = time.perf_counter()
            lib().fl_wide_moe(ctx.ctx, L.gate.data_ptr(), L.up.data_ptr(), L.down.data_ptr(), 4, 256, ptr(midx), ptr(rows), ptr(kidx),
                              ptr(wk), ns, KE, 0)
            lib().fl_wide_finish(ctx.ctx, n, KE, ctypes.byref(out))
            return t_lib + time.perf_counter() - t0

        with no_gc():   # collected before the warm-up steps
            for _ in range(warmup):
                step()
            ts = [step() for _ in range(steps)]
        torch.cuda.synchronize()
        ctx.sync()
        ms = float(np.median(ts)) * 1e3
        res = {"ms_per_step": round(ms, 3), "tokens_per_s": round(n / (ms * 1e-3)), "tokens": n, "steps": steps}
        log("[bench] drop-in prefill-%d (wide pass): %s" % (n, json.dumps(res)))
    finally:
        for t in mats:
            ctx.unregister_tiled(t)
    del L
    torch.cuda.empty_cache()
    return res


def run_realfmt(ctx, torch, steps=20, warmup=3, copies=2, seed=20260501):
    """fl_moe_layer on the reference's real-shard formats, device-resident: IQ2_XXS routed gate/up (tiled), Q3_K routed
    down and a Q5_K / Q5_K / Q6_K shared expert read in place (fl_set_layer_formats); decode-8, decode-1 and prefill-512
    (routed gate/up on the MFMA GEMM, the K-quants on their mat-vecs), fresh x per step, layer copies rotated.
    Algorithmic bytes: U * (2 IQ2_XXS + 1 Q3_K matrix) + the shared expert + the router."""
    from loki_amd import MoeLayerWeights
    layers = []
    for c in range(copies):
        base = MoeLayerWeights.synthetic(ctx, seed + 1000 * c)
        down = kq_random(torch, 6, 256 * E, H, seed + 1000 * c + 1)
        shg, shu, shd = (kq_random(torch, 3, H, E, seed + 1000 * c + 2), kq_random(torch, 3, H, E, seed + 1000 * c + 3),
                         kq_random(torch, 1, E, H, seed + 1000 * c + 4))
        layers.append(MoeLayerWeights(base.gate_inp, base.probs_b, base.gate, base.up, down, shg, shu, shd))
    ctx.set_layer_formats(6, 3, 3, 1)
    out = {}
    try:
        for name, n in (("decode8", 8), ("decode1", 1), ("prefill512", 512)):
            xs = []
            for i in range(steps + warmup):
                x = torch.empty((n, E), dtype=torch.float32, device="cuda")
                ctx.synth_normal(x, seed + 17, 3000 + i, 0.0, 1.0)
                xs.append(x)
            y = torch.empty((n, E), dtype=torch.float32, device="cuda")
            for i in range(warmup):
                ctx.moe_layer(layers[i % copies], xs[i], y)
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for i in range(steps):
                ctx.moe_layer(layers[(warmup + i) % copies], xs[warmup + i], y)
            t1.record()
            torch.cuda.synchronize()
            ctx.sync()
            ms = t0.elapsed_time(t1) / steps
            U = sum(distinct_experts(ctx, layers[(warmup + i) % copies], [xs[warmup + i]])[0] for i in range(steps)) / steps
            b = U * (2 * MAT_BYTES + E * (H // 256) * 110) + 2 * H * (E // 256) * 176 + E * (H // 256) * 210 + ROUTER_BYTES
            out[name] = {"us_per_token": round(ms * 1e3 / n, 2), "ms_per_step": round(ms, 4), "distinct_experts": round(U, 1),
                         "tokens_per_s": round(n / (ms * 1e-3)),
                         "bytes_per_step": int(b), "hbm_gbs": round(b / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            log("[bench] real formats %s: %s" % (name, json.dumps(out[name])))
    finally:
        ctx.set_layer_formats()
    del layers
    torch.cuda.empty_cache()
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """All-cores thread count: the host cores this process may use, capped at 16 (a one-GPU box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def time_oracle(ctx, layer, x, threads, n_group=8, topk_group=4):
    """Seconds of one oracle block call on x (numpy [n, E]) with the layer's weights; the selected experts are copied to
    the host first, outside the timed call."""
    from oracle import oracle as orc
    from tests._helpers import host_layer
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, sel, _ = orc.router(W, b, x, n_group, topk_group)
    _, _, gate, up, down, sh = host_layer(ctx, layer, sel.ravel())
    t0 = time.perf_counter()
    out = orc.moe_forward(x, W, b, gate, up, down, *sh, n_group=n_group, topk_group=topk_group, nthreads=threads)
    return time.perf_counter() - t0, out["y"]


def cpu_sample(ctx, res, rows, threads):
    """us/token of the oracle on the first `rows` tokens of the workload's first step, at `threads` threads."""
    x = res["xs"][0].cpu().numpy()[:rows]
    dt, _ = time_oracle(ctx, res["layers"][0], x, threads)
    return dt * 1e6 / x.shape[0]


def cpu_stack_sample(ctx, layers, x0, nlayers=2):
    """The first `nlayers` layers of the stack chain for one token on the CPU (the oracle's own chain: x_{L+1} =
    RMSNorm(y_L)); per-token time scaled to all layers. Each layer's selected experts are copied to the host outside
    the timed call."""
    from oracle import oracle as orc
    out = {}
    for threads in (cpu_threads(), 1):
        x = x0.cpu().numpy()
        tot = 0.0
        for L in layers[:nlayers]:
            dt, y = time_oracle(ctx, L, x, threads)
            tot += dt
            x = orc.rmsnorm(y)
        out["us_per_token_%dt" % threads] = round(tot / nlayers * len(layers) * 1e6, 1)
    return out


_LIB_SHA = None


def lib_sha16():
    """SHA-256 prefix of the library this process loads: profiles/ summaries carry the one their run loaded."""
    global _LIB_SHA
    if _LIB_SHA is None:
        import hashlib
        from loki_amd import LIB_PATH
        with open(LIB_PATH, "rb") as f:
            _LIB_SHA = hashlib.sha256(f.read()).hexdigest()[:16]
    return _LIB_SHA


# roofline kernel -> the key of its profiles/ summaries
PROFILE_KEY = {"k_moe_decode1": "k_moe_decode1", "k_moe_decode": "k_moe_decode", "k_pf_gemm<gate_up>": "k_pf_gemm_gate_up",
               "k_experts<gate_up>": "k_experts_gate_up"}


def load_profile(kind, kernel, workload):
    """A committed profiles/<kind>_<key>_<workload>.json, if it was made with this very library (else None, and why)."""
    p = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                     "%s_%s_%s.json" % (kind, PROFILE_KEY.get(kernel, kernel), workload))
    if not os.path.exists(p):
        return None, "no %s" % os.path.basename(p)
    with open(p) as f:
        js = json.load(f)
    if js.get("lib_sha16") != lib_sha16():
        return None, "%s was made with library %s, this run loads %s" % (os.path.basename(p), js.get("lib_sha16"), lib_sha16())
    return js, os.path.join("profiles", os.path.basename(p))


def kernel_roofline(res):
    """Dominant kernel of a workload's step, its algorithmic bytes and average duration: the single decode launch
    (its bytes are the step's), else the gate/up stage (grouped GEMM on MFMA above 8 tokens, else the mat-vec kernel)."""
    n = res["n"]
    if res["fused"]:
        kname = "k_moe_decode1" if res["dkernel"] == 2 else "k_moe_decode"
        k_ms, k_bytes = res["stage_ms"]["gate_up"], res["bytes"]
        stages = {"block": k_ms}
    else:
        kname = "k_pf_gemm<gate_up>" if n > 8 else "k_experts<gate_up>"
        k_ms, k_bytes = res["stage_ms"]["gate_up"], res["gu_bytes"]
        stages = res["stage_ms"]
    k_gbs = k_bytes / (k_ms * 1e-3) / 1e9
    tr, tr_src = load_profile("traffic", kname, res["name"])
    kt, kt_src = load_profile("trace", kname, res["name"])
    roof = {"kernel": kname, "bound": "hbm", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": tr["bytes_per_launch"] if tr else None,
            "algorithmic_bytes_per_launch": int(k_bytes), "avg_launch_us": round(k_ms * 1e3, 2),
            "lib_sha16": lib_sha16(), "traffic_source": tr_src,
            # the same kernel's average duration over the timed steps of a committed rocprofv3 kernel trace made with
            # this library (profiles/trace_*.json): the frac it implies, to set beside the live one
            "profile_avg_us": kt["avg_us_last"] if kt else None,
            # (the median of the same launches: the protocol's statistic; an event between steps, the other way to
            # get per-step times, adds microseconds to each)
            "profile_median_us": kt["median_us_last"] if kt else None,
            "profile_frac": round(k_bytes / (kt["avg_us_last"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if kt else None,
            "profile_source": kt_src}
    return roof, stages


def summary(res):
    roof, stages = kernel_roofline(res)
    return {"us_per_token": round(res["ms"] * 1e3 / res["n"], 3), "ms_per_step": round(res["ms"], 4),
            "tokens_per_s": round(res["n"] / (res["ms"] * 1e-3), 1), "hbm_gbs": round(res["gbs"], 1),
            "hbm_frac": round(res["gbs"] / HBM_PEAK_GBS, 4), "distinct_experts": round(res["U"], 1),
            "host_us_per_call": round(res["host_us"], 2), "routing_margin": res["margins"], "roofline": roof,
            "stage_us": {k: round(v * 1e3, 2) for k, v in stages.items()}}


def bench(args, ctx, torch):
    if args.fused is not None:
        ctx.set_fused(args.fused)
    if args.only_kquant:
        print(json.dumps({"kquant": run_kquant(ctx, torch), "real_formats": run_realfmt(ctx, torch), "lib_sha16": lib_sha16()}), flush=True)
        return
    if args.only_dropin:
        print(json.dumps({"dropin_decode1": run_dropin(ctx, torch), "dropin_decode8": run_dropin_rows(ctx, torch),
                          "dropin_prefill512": run_dropin_wide(ctx, torch), "lib_sha16": lib_sha16()}), flush=True)
        return
    thr = cpu_threads()
    cpu_per = {}

    def cpu_leg(res):
        if args.no_cpu:
            return
        rows = min(res["n"], 8)
        cpu_per[res["name"]] = {"us_per_token_%dt" % thr: round(cpu_sample(ctx, res, rows, thr), 1),
                                "us_per_token_1t": round(cpu_sample(ctx, res, rows, 1), 1), "tokens": rows}
        log("[bench] cpu %s: %s" % (res["name"], json.dumps(cpu_per[res["name"]])))

    res = run_workload(ctx, torch, args.workload, args.steps, args.warmup, args.copies)
    n = res["n"]
    head = summary(res)
    log("[bench] %s: %s" % (args.workload, json.dumps(head)))
    cpu_leg(res)
    if args.copy_probe:
        a = torch.empty(1 << 28, dtype=torch.float32, device="cuda"); b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log("[bench] copy probe: 3 x %d bytes read + written" % (a.numel() * 4))
        del a, b
    extra = {}
    if not args.no_extra:
        for wl, st in (("decode8", 30), ("decode1", 30), ("prefill512", 5), ("prefill2048", 3)):
            if wl == args.workload:
                continue
            r = run_workload(ctx, torch, wl, st, 2, args.copies)
            extra[wl] = summary(r)
            log("[bench] %s: %s" % (wl, json.dumps(extra[wl])))
            cpu_leg(r)
            del r
            torch.cuda.empty_cache()
        extra["dropin_decode1"] = run_dropin(ctx, torch)
        extra["dropin_decode8"] = run_dropin_rows(ctx, torch)
        extra["dropin_prefill512"] = run_dropin_wide(ctx, torch)
        log("[bench] dropin_decode1: %s" % json.dumps(extra["dropin_decode1"]))
        extra["kquant"] = run_kquant(ctx, torch)
        extra["real_formats"] = run_realfmt(ctx, torch)
    if not args.no_stack:
        torch.cuda.empty_cache()
        extra["stack58"] = run_stack(ctx, torch, args.stack_steps, 2, cpu_sample=not args.no_cpu)
        if extra["stack58"].get("cpu"):
            cpu_per["stack58"] = extra["stack58"].pop("cpu")
        log("[bench] stack58: %s" % json.dumps(extra["stack58"]))
    cpu = None
    if not args.no_cpu:
        key = "us_per_token_%dt" % thr
        cpu = {"value": cpu_per[args.workload][key], "unit": "us/token", "cores": thr, "kind": "port",
               "sample": "%s: %d token(s) of the first step through oracle/moe_oracle.c (restated ggml CPU semantics: "
                         "Q8_K, vec_dot_iq2_xxs_q8_K, grouped router, swiglu, k-ordered combine), OpenMP %d threads, "
                         "same x and weights as the GPU steps; per_config holds every config at %d threads and at 1 "
                         "thread (prefill: the batch's first 8 tokens; stack58: 2 layers of the chain, scaled to 58)"
                         % (args.workload, cpu_per[args.workload]["tokens"], thr, thr),
               "cpu_model": cpu_model(), "nproc": os.cpu_count(), "per_config": cpu_per}
        log("[bench] cpu baseline: %s" % json.dumps(cpu))
    out = {
        "metric": "MoE-layer decode µs/token (HBM GB/s, % peak); prefill-512 tokens/s",
        "value": round(res["ms"] * 1e3 / n, 3),
        "unit": "us/token",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(res["ms"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (device-generated, seeded; the benchmark configs' distribution)",
        "config": {"workload": res["desc"], "tokens": n, "hidden": E, "expert_ffn": H, "routed_experts": 256,
                   "shared_experts": 1, "routing": "sigmoid, 8 groups, top-4 groups, top-8, x2.5",
                   "weights": "IQ2_XXS (activations Q8_K)", "layer_copies": args.copies, "preheat_ms": args.preheat_ms},
        "hbm_gbs": head["hbm_gbs"],
        "hbm_frac": head["hbm_frac"],
        "distinct_experts": head["distinct_experts"],
        "routing_margin": head["routing_margin"],
        "host_us_per_call": head["host_us_per_call"],
        "roofline": head["roofline"],
        "stage_us": head["stage_us"],
        "lib_sha16": lib_sha16(),
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode1", choices=sorted(WORKLOADS))
    ap.add_argument("--copies", type=int, default=8,
                    help="independently seeded layers rotated over the steps (8 x 2.9 GB: a layer's router and shared "
                         "expert recur after 7 other layers' ~770 MB, well past the 256 MB MALL)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the other decode / prefill workloads and the K-quant legs")
    ap.add_argument("--no-stack", action="store_true", help="skip the 58-layer resident stack (configs[3], ~169 GB)")
    ap.add_argument("--stack-steps", type=int, default=10)
    ap.add_argument("--only-kquant", action="store_true",
                    help="run only the K-quant mat-vec leg (the reference's real-shard formats) and print its JSON")
    ap.add_argument("--only-dropin", action="store_true",
                    help="run only the reference-named path (fl_ffn_begin -> fl_fetch -> fl_moe) and print its JSON")
    ap.add_argument("--fused", type=int, default=None, choices=(0, 1, 2),
                    help="decode path: 2 regular single launch (library default), 1 cooperative single launch, 0 per pass")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 1 GiB device copy (the reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--preheat-ms", type=float, default=PREHEAT_MS,
                    help="untimed load before each decode / prefill / stack workload's warm-up steps, so the timed steps run "
                         "at the clocks of a loaded GPU (0: none)")
    args = ap.parse_args()
    globals()["PREHEAT_MS"] = args.preheat_ms
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py: this build runs on one GPU only (the MoE block is not sharded across GPUs); got --gpus %d, "
            "WORLD_SIZE %d" % (args.gpus, world))
        sys.exit(2)
    import torch
    from loki_amd import Context, LokiError
    ctx = Context()
    rc = 0
    try:
        bench(args, ctx, torch)
    except LokiError as e:   # a device-side failure reported by fl_sync: no bench line
        log("bench.py: %s" % e)
        rc = 3
    finally:
        # the context's HIP objects are released before interpreter exit (exit-time destructors would otherwise run
        # them after a profiler's own teardown)
        torch.cuda.synchronize()
        ctx.close()
    sys.exit(rc)


if __name__ == "__main__":
    main()
