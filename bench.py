#!/usr/bin/env python3
"""I2_S ternary GEMV throughput on one MI355X.

Workload (one "step"): the BitNet-2B FFN GEMVs at batch 1 over 32 distinct,
independently seeded weight sets -- per set, gate and up (6912 x 2560) share
one int8-quantised activation, down (2560 x 6912) has its own. 424.7 MB of
packed ternary weights, rotated every step, so HBM (not the 256 MB Infinity
Cache) feeds them. A step is one plan run on the library stream: a single
slab-kernel launch over all 96 matrices in which every workgroup quantises
its f32 activation (int8 absmax per token) in LDS, streams its slab of
packed weights and writes the f32 epilogue. Inputs are resident in HBM
before the timed region.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Beside the headline line the JSON carries (each GPU figure also as the
median and best of several batches or runs):
  batches  the headline launch in ten batches of 100;
  cfg0     one 2560 x 2560 GEMV per launch, hot and rotated over 192 tensors,
           and the 192 as one launch;
  ffn_sets the headline workload one weight set per launch (gate + up +
           down), the 32 sets rotated;
  dropin   the same FFN workload through the host-pointer row that a patched
           reference forward.c calls (sllm_kdispatch_*), each call copying
           across PCIe and waiting: what the drop-in costs per GEMV;
  block30  the decode GEMVs of 30 independently seeded 2B blocks, one launch;
  decode   a random-init BitNet-b1.58-2B decode step (30 blocks, F16 output,
           greedy argmax) after a 1024-position binary16 KV prefix, tokens/s
           on the device's own token loop, its first token checked bit for bit
           (logits, every int32 dot and activation) against the oracle, and the
           reference's own sllm_forward timed on this host from the same
           prefix (restored through its state file);
  gemm     several tokens against one tensor (4, 16, 64 and the 512-token
           prefill chunk) on int8 MFMA beside the GEMV path, with sampled
           tokens checked against the oracle.

Prints ONE JSON line. `value` is algorithmic bytes per step / wall time per
step. `roofline` is the slab kernel, the step's only launch: its average
launch duration is the time between two HIP events recorded on the library
stream at the edges of the timed region, divided by the step count (so it
includes the short gaps between back-to-back launches; an event per launch
would add a wait of several microseconds to every step). `cpu_baseline` is the reference's own CPU path
(oracle/_ref, built from its sources) or the oracle's restatement of it,
timed on this host over a bounded sample of the same workload.
"""
import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "I2_S GEMV achieved HBM GB/s (% of peak) + 2B-shape decode tokens/s, batch 1"
PEAK_HBM_GBS = 8000.0
SETS = 32
K_UP, N_FF = 2560, 6912
SHAPES = [("gate", N_FF, K_UP), ("up", N_FF, K_UP), ("down", K_UP, N_FF)]


def load_package():
    spec = importlib.util.spec_from_file_location("saphira_llm_amd", os.path.join(ROOT, "saphira-llm_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["saphira_llm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class Workload:
    """Config: BitNet-2B FFN GEMVs, batch 1, 32 rotated weight sets."""

    def __init__(self, amd, dev, sets=SETS):
        self.amd, self.dev, self.sets = amd, dev, sets
        t0 = time.perf_counter()
        self.host_w = []          # per set: [gate, up, down] packed bytes (kept for the CPU leg)
        self.bufs = []
        jobs = []
        x_up = np.stack([amd.synth_normal(amd.synth_seed(1, s, 0, 100), K_UP) for s in range(sets)])
        x_dn = np.stack([amd.synth_normal(amd.synth_seed(1, s, 0, 101), N_FF) for s in range(sets)])
        self.x_up, self.x_dn = x_up, x_dn
        self.b_xup, self.b_xdn = dev.put(x_up), dev.put(x_dn)
        self.b_y = []
        w_bytes = 0
        out_elems = 0
        for s in range(sets):
            ws = []
            for m, (name, n_rows, n) in enumerate(SHAPES):
                w = amd.synth_i2s(amd.synth_seed(1, s, 0, m), n_rows, n)
                ws.append(w)
                bw = dev.put(w)
                by = dev.alloc(4 * n_rows)
                self.bufs += [bw, by]
                self.b_y.append(by)
                # each job carries its f32 activation (gate and up share
                # one row; each of their workgroups quantises it in-kernel)
                x = self.b_xup.at(4 * s * K_UP) if n == K_UP else self.b_xdn.at(4 * s * N_FF)
                jobs.append(amd.GemvJob(bw.ptr, n_rows, n, x.value, None, None, by.ptr, None))
                w_bytes += n_rows * n // 4 + 4          # codes + the f32 scale
                out_elems += n_rows
            self.host_w.append(ws)
        self.jobs = jobs
        self.plan = dev.plan(jobs)
        # algorithmic bytes
        self.weight_bytes = w_bytes
        act_in = sets * (K_UP + N_FF)                   # distinct activation vectors (gate/up share)
        self.step_bytes = w_bytes + 4 * act_in + 4 * out_elems          # f32 in, f32 out
        self.ops = sum(2 * n_rows * n for _, n_rows, n in SHAPES) * sets
        # one launch reads the weights and f32 activations and writes f32 outputs
        self.gemv_bytes = self.step_bytes
        log(f"workload ready in {time.perf_counter() - t0:.1f}s: {len(jobs)} GEMVs, "
            f"{w_bytes / 1e6:.1f} MB weights")

    def step(self):
        """One step: the plan's launch."""
        self.dev.plan_run(self.plan)

    def outputs(self, sets):
        """(weights, N, K, x, GPU output, label) of every GEMV in `sets`, for
        the oracle check in the CPU leg (parity is the tests' job; this guards
        the timed configuration itself)."""
        out = []
        for s in sets:
            for m, (name, n_rows, n) in enumerate(SHAPES):
                x = self.x_up[s] if n == K_UP else self.x_dn[s]
                out.append((self.host_w[s][m], n_rows, n, x,
                            self.b_y[3 * s + m].download(np.float32, n_rows), f"set {s} {name}"))
        return out


# one BitNet-b1.58-2B block: (name, N, K, activation slot); q/k/v share the
# attention input, gate/up the FFN input (src/forward.c:645-793)
BLOCK = [("q", 2560, 2560, 0), ("k", 640, 2560, 0), ("v", 640, 2560, 0), ("o", 2560, 2560, 1),
         ("gate", N_FF, K_UP, 2), ("up", N_FF, K_UP, 2), ("down", K_UP, N_FF, 3)]


def measure_block_plan(amd, dev, layers=30, steps=200):
    """The per-block decode GEMVs of 30 independently seeded layers (521 MB of
    packed weights), f32 N(0,1) inputs quantised in-kernel, as one plan: one
    launch of 210 GEMVs, timed like the main workload. Returns the figures and
    the inputs / outputs of layers 0 and 29 for the oracle check."""
    bufs, jobs, keep = [], [], []
    w_bytes = act_bytes = out_bytes = 0
    for il in range(layers):
        xs = {}
        for slot, n in ((0, K_UP), (1, K_UP), (2, K_UP), (3, N_FF)):
            x = amd.synth_normal(amd.synth_seed(2, 0, il, 200 + slot), n)
            xs[slot] = (x, dev.put(x))
            bufs.append(xs[slot][1])
            act_bytes += 4 * n
        for m, (name, n_rows, n, slot) in enumerate(BLOCK):
            w = amd.synth_i2s(amd.synth_seed(2, 0, il, m), n_rows, n)
            bw, by = dev.put(w), dev.alloc(4 * n_rows)
            bufs += [bw, by]
            jobs.append(amd.GemvJob(bw.ptr, n_rows, n, xs[slot][1].ptr, None, None, by.ptr, None))
            w_bytes += n_rows * n // 4 + 4
            out_bytes += 4 * n_rows
            if il in (0, layers - 1):
                keep.append((w, n_rows, n, xs[slot][0], by, f"layer {il} {name}"))
    plan = dev.plan(jobs)
    for _ in range(20):
        dev.plan_run(plan)
    dev.sync()
    checks = [(w, n_rows, n, x, by.download(np.float32, n_rows), what) for w, n_rows, n, x, by, what in keep]
    dev.events(2)
    dev.sync()
    t0 = time.perf_counter()
    dev.record(0)
    for _ in range(steps):
        dev.plan_run(plan)
    dev.record(1)
    dev.sync()
    wall_us = (time.perf_counter() - t0) * 1e6 / steps
    ev_us = dev.elapsed(0, 1) * 1e3 / steps
    bt = timed_batches(dev, lambda: dev.plan_run(plan), 10, steps // 10)
    dev.plan_destroy(plan)
    for b in bufs:
        b.free()
    total = w_bytes + act_bytes + out_bytes
    return checks, {"workload": "30 independently seeded BitNet-2B blocks (q/o 2560x2560, k/v 640x2560, gate/up 6912x2560, "
                        "down 2560x6912), 210 GEMVs in one launch, f32 inputs quantised in-kernel",
            "weight_bytes": w_bytes, "bytes_per_launch": total, "us_per_launch": round(ev_us, 2),
            "GBps": round(total / (ev_us * 1e-6) / 1e9, 1), "wall_us_per_launch": round(wall_us, 2),
            "frac_of_peak": round(total / (ev_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4), "steps": steps,
            "batches": with_rate(bt, total)}


CFG0_N = 2560
CFG0_COPIES = 192      # 192 x 1.64 MB = 315 MB: more than the 256 MB Infinity Cache


def measure_cfg0(amd, dev, calls=2000):
    """One 2560 x 2560 I2_S GEMV at batch 1 (quantise -> GEMV -> epilogue,
    one launch per call, sllm_gfx950_linear): hot (the same tensor every
    call, resident in the caches) and rotated over CFG0_COPIES distinct
    tensors (so HBM feeds them); and the rotated copies as one plan (every
    GEMV of the set in one launch, each with its own activation), the
    bandwidth-bound form. Returns the figures and two outputs for the oracle
    check."""
    n = CFG0_N
    ws = [amd.synth_i2s(amd.synth_seed(0, s_, 0, 0), n, n) for s_ in range(CFG0_COPIES)]
    xs = np.stack([amd.synth_normal(amd.synth_seed(0, s_, 0, 1), n) for s_ in range(CFG0_COPIES)])
    bws = [dev.put(w) for w in ws]
    bx = dev.put(xs)
    bq, ba = dev.alloc(n), dev.alloc(8)
    by = dev.alloc(4 * n * CFG0_COPIES)
    per_call = n * n // 4 + 4 + 4 * n + 4 * n
    res = {}
    for label, rot in (("hot", 1), ("rotated", CFG0_COPIES)):
        for i in range(64):
            dev.linear(bws[i % rot].vp, n, n, bx.at(4 * n * (i % rot)), bq.vp, ba.vp, by.at(4 * n * (i % rot)))
        dev.events(2)
        dev.sync()
        dev.record(0)
        for i in range(calls):
            dev.linear(bws[i % rot].vp, n, n, bx.at(4 * n * (i % rot)), bq.vp, ba.vp, by.at(4 * n * (i % rot)))
        dev.record(1)
        us = dev.elapsed(0, 1) * 1e3 / calls
        it = iter(range(1 << 40))

        def call():
            i = next(it) % rot
            dev.linear(bws[i].vp, n, n, bx.at(4 * n * i), bq.vp, ba.vp, by.at(4 * n * i))
        res[label] = {"us_per_call": round(us, 2), "GBps": round(per_call / us / 1e3, 1),
                      "batches": with_rate(timed_batches(dev, call, 10, calls // 10), per_call)}
        log(f"cfg0 2560x2560 {label}: {us:.2f} us per call, {per_call / us / 1e3:.1f} GB/s")
    checks = []
    for i in (0, CFG0_COPIES - 1):
        checks.append((ws[i], n, n, xs[i], by.download(np.float32, n, 4 * n * i), f"cfg0 copy {i}"))
    plan = dev.plan([amd.GemvJob(bws[i].ptr, n, n, bx.ptr + 4 * n * i, None, None, by.ptr + 4 * n * i, None)
                     for i in range(CFG0_COPIES)])
    for _ in range(20):
        dev.plan_run(plan)
    reps = 200
    dev.sync()
    dev.record(0)
    for _ in range(reps):
        dev.plan_run(plan)
    dev.record(1)
    us = dev.elapsed(0, 1) * 1e3 / reps
    bt = timed_batches(dev, lambda: dev.plan_run(plan), 10, reps // 10)
    dev.plan_destroy(plan)
    for b in bws + [bx, bq, ba, by]:
        b.free()
    total = per_call * CFG0_COPIES
    res["batched"] = {"us_per_launch": round(us, 2), "GBps": round(total / us / 1e3, 1),
                      "frac_of_peak": round(total / us / 1e3 / PEAK_HBM_GBS, 4), "gemvs_per_launch": CFG0_COPIES,
                      "batches": with_rate(bt, total)}
    log(f"cfg0 2560x2560, {CFG0_COPIES} rotated GEMVs in one launch: {us:.2f} us, {total / us / 1e3:.1f} GB/s")
    return checks, (ws, xs), dict(res, workload=(f"I2_S GEMV 2560x2560 batch 1, uniform ternary, per-tensor scale U(0.5,2), "
                                       f"f32 N(0,1) activation int8-absmax quantised in-kernel, f32 output; one "
                                       f"launch per call (sllm_gfx950_linear), hot and rotated over "
                                       f"{CFG0_COPIES} tensors ({CFG0_COPIES * (n * n // 4 + 32) / 1e6:.0f} MB); "
                                       f"and the {CFG0_COPIES} as one launch"),
                        bytes_per_call=per_call, calls=calls)


def measure_dropin(amd, wl, passes=2):
    """The drop-in row's cost on the FFN workload: what the reference's own
    forward pass pays per GEMV once its sllm_gemv and quantiser calls go to
    the gfx950 row (sllm_kdispatch_*, host pointers, src/forward.c:196-205 and
    :651-788). Every tensor of the 32 sets is registered once (uploaded under
    its host address); then per set, as the reference orders it: quantise the
    FFN input, GEMV gate, GEMV up, quantise the down input, GEMV down --
    each call copies its q / rows across PCIe and waits for the result.
    Host wall clock; the epilogue is the reference's, on the host. Returns
    the figures and the outputs of sets 0 and 31 for the oracle check."""
    lib = amd.lib()
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    for ws in wl.host_w:
        for w, (_, n_rows, n) in zip(ws, SHAPES):
            amd.check(lib.sllm_gfx950_tensor_register(P(w), n_rows, n), "tensor_register")
    amd.check(lib.sllm_kdispatch_select(b"gfx950"), "kdispatch_select")
    q = np.empty(N_FF, np.int8)
    dots = [np.empty(n_rows, np.int32) for _, n_rows, _ in SHAPES]
    acts = [amd.Act(), amd.Act()]
    checks = []

    def one_set(s):
        ws = wl.host_w[s]
        lib.sllm_kdispatch_quant_act(P(wl.x_up[s]), K_UP, P(q), ctypes.byref(acts[0]))
        lib.sllm_kdispatch_gemv(P(ws[0]), N_FF, K_UP, P(q), P(dots[0]))
        lib.sllm_kdispatch_gemv(P(ws[1]), N_FF, K_UP, P(q), P(dots[1]))
        lib.sllm_kdispatch_quant_act(P(wl.x_dn[s]), N_FF, P(q), ctypes.byref(acts[1]))
        lib.sllm_kdispatch_gemv(P(ws[2]), K_UP, N_FF, P(q), P(dots[2]))

    try:
        for s in range(wl.sets):
            one_set(s)
        t0 = time.perf_counter()
        for _ in range(passes):
            for s in range(wl.sets):
                one_set(s)
        dt = time.perf_counter() - t0
        for s in (0, wl.sets - 1):
            one_set(s)
            for m, (name, n_rows, n) in enumerate(SHAPES):
                w = wl.host_w[s][m]
                a = acts[0] if m < 2 else acts[1]
                w_scale = np.frombuffer(w[n_rows * n // 4:n_rows * n // 4 + 4].tobytes(), np.float32)[0]
                pq = np.float32(w_scale) / np.float32(a.scale)
                y = (dots[m] - np.int32(a.sum)).astype(np.float32) * pq
                x = wl.x_up[s] if n == K_UP else wl.x_dn[s]
                checks.append((w, n_rows, n, x, y, f"drop-in row set {s} {name}"))
    finally:
        lib.sllm_kdispatch_reset()
        for ws in wl.host_w:
            for w in ws:
                lib.sllm_gfx950_tensor_unregister(P(w))
    gemvs = passes * wl.sets * len(SHAPES)
    us_per_gemv = dt * 1e6 / gemvs
    us_per_set = dt * 1e6 / (passes * wl.sets)
    set_bytes = wl.step_bytes / wl.sets
    log(f"drop-in row: {us_per_set:.1f} us per FFN set ({us_per_gemv:.1f} us per GEMV incl. its share of "
        f"the quantiser calls), {set_bytes / us_per_set / 1e3:.1f} GB/s")
    return checks, {
        "workload": ("the FFN workload through the host-pointer row the patched reference forward.c "
                     "calls (sllm_kdispatch_quant_act / sllm_kdispatch_gemv): per set 2 quantiser calls "
                     "and 3 GEMVs, each copying q / int32 rows across PCIe and synchronising; host epilogue"),
        "us_per_set": round(us_per_set, 1), "us_per_gemv": round(us_per_gemv, 1),
        "GBps": round(set_bytes / us_per_set / 1e3, 1), "sets_timed": passes * wl.sets,
        "clock": "host wall clock"}


# the decode workload: random-init BitNet-b1.58-2B, a 1024-position KV prefix
# of binary16 N(0,1) values (held as f32, as the reference's cache holds it)
DECODE_PREFIX = 1024


def decode_prefix(amd, cfg, n_pos):
    """K and V caches [layer][head_kv][pos][head_dim] of binary16 N(0,1)."""
    hd = cfg["n_embd"] // cfg["n_head"]
    shape = (cfg["n_layer"], cfg["n_head_kv"], n_pos, hd)
    n = int(np.prod(shape))
    k = amd.synth_normal_f16(amd.synth_seed(5, 0, 0, 1), n).view(np.float16).astype(np.float32).reshape(shape)
    v = amd.synth_normal_f16(amd.synth_seed(5, 0, 0, 2), n).view(np.float16).astype(np.float32).reshape(shape)
    return k, v


def decode_bytes_per_token(cfg, npast):
    """Algorithmic HBM bytes of one decode token: every I2_S matrix (codes and
    tail), the F16 output projection, the norm weights, the K and V cache rows
    attended (f32) and the new K / V rows written."""
    e, f, L = cfg["n_embd"], cfg["n_ff"], cfg["n_layer"]
    hd = e // cfg["n_head"]
    gqa = hd * cfg["n_head_kv"]
    i2s = L * ((2 * e * e + 2 * gqa * e + 3 * f * e) // 4 + 7 * 32)
    lm = cfg["n_vocab"] * e * 2
    norms = L * (3 * e + f) * 4 + e * 4
    kv = L * 2 * cfg["n_head_kv"] * npast * hd * 4 + L * 2 * gqa * 4
    return i2s + lm + norms + kv, {"i2s": i2s, "lm_head": lm, "norms": norms, "kv": kv}


def measure_decode(amd, dev, tokens=128, warm=8, graph=True, inflight=None, runs=3):
    """The decode step at BitNet-2B shape on the device's own greedy loop
    (one HIP graph per token, the argmax kernel feeding the next token): the
    first token after the prefix is traced for the CPU leg's bit-exact check,
    then `warm` untimed tokens and `runs` timed runs of `tokens` tokens each,
    one after the other (tokens/s: the median run, and the best). Every
    generated id is kept for the CPU leg's token witness. inflight: tokens
    the loop keeps enqueued ahead of the host (the library's default when
    None)."""
    cfg = dict(amd.BITNET_2B)
    t0 = time.perf_counter()
    model = amd.synth_model(cfg, 0)
    k, v = decode_prefix(amd, cfg, DECODE_PREFIX)
    g = amd.DeviceDecoder(dev, model, DECODE_PREFIX + 1 + warm + runs * tokens + 8)
    g.kv_load(k, v, DECODE_PREFIX)
    log(f"decode model and {DECODE_PREFIX}-position prefix ready in {time.perf_counter() - t0:.1f}s")
    tok0 = 128000 % cfg["n_vocab"]
    g.trace_start()
    logits0 = g.forward(tok0, DECODE_PREFIX)
    dots0, acts0 = g.trace_read()
    g.trace_stop()
    g.set_graph(graph)
    if inflight is not None:
        g.set_inflight(inflight)
    warm_ids = g.generate([], warm)
    dev.events(2)
    ids, run_ms, walls = [], [], []
    for _ in range(runs):
        dev.sync()
        t0 = time.perf_counter()
        dev.record(0)
        ids += list(g.generate([], tokens))
        dev.record(1)
        walls.append(time.perf_counter() - t0)
        run_ms.append(dev.elapsed(0, 1))
    g.close()
    ms = float(np.median(run_ms))
    tok_s = tokens / (ms * 1e-3)
    wall = float(np.median(walls))
    pos_first = DECODE_PREFIX + 1 + warm
    npast_mean = pos_first + 1 + (runs * tokens - 1) / 2
    bpt, parts = decode_bytes_per_token(cfg, npast_mean)
    # the same token with a binary16 KV cache (the bytes BASELINE's 6,360
    # tokens/s roofline is quoted on): parity needs the f32 cache
    bpt16 = bpt - parts["kv"] // 2
    check = {"model": model, "k": k, "v": v, "token": tok0, "logits": logits0, "dots": dots0, "acts": acts0,
             "ids": [int(x) for x in warm_ids] + [int(x) for x in ids]}
    return check, {
        "workload": (f"random-init BitNet-b1.58-2B (30 blocks, 2560/6912, 20x128 heads, 5 KV heads, F16 128256 x 2560 "
                     f"output), KV cache of {DECODE_PREFIX} binary16 N(0,1) positions, greedy decode at positions "
                     f"{pos_first}..{pos_first + runs * tokens - 1} ({runs} runs of {tokens}), batch 1, "
                     + ("one HIP graph per token" if graph else "the token's launches enqueued one by one")
                     + ("" if inflight is None else f", at most {inflight} token(s) enqueued ahead")),
        "tokens_per_s": round(tok_s, 1), "us_per_token": round(ms * 1e3 / tokens, 1),
        "tokens_per_s_best": round(tokens / (min(run_ms) * 1e-3), 1),
        "run_tokens_per_s": [round(tokens / (r_ * 1e-3), 1) for r_ in run_ms],
        "wall_tokens_per_s": round(tokens / wall, 1), "tokens": tokens, "runs": runs,
        "bytes_per_token": int(bpt), "bytes_parts": {a: int(b) for a, b in parts.items()},
        "effective_GBps": round(bpt * tok_s / 1e9, 1), "roofline_tokens_per_s": round(PEAK_HBM_GBS * 1e9 / bpt, 1),
        "frac_of_roofline": round(tok_s * bpt / (PEAK_HBM_GBS * 1e9), 4),
        "roofline_f16kv_tokens_per_s": round(PEAK_HBM_GBS * 1e9 / bpt16, 1),
        "frac_of_f16kv_roofline": round(tok_s * bpt16 / (PEAK_HBM_GBS * 1e9), 4),
        "launches_per_token": 6 * cfg["n_layer"] + 2,
    }


PREFILL_TOKENS = 512
PREFILL_CHECK = 16
# positions whose logits the reference's own chunked forward checks: one in
# every eight-token scores block, the offset inside the block advancing by
# one from block to block (positions 0, 9, 18, ..., 511)
PREFILL_CHECK_POS = tuple(8 * i + i % 8 for i in range(PREFILL_TOKENS // 8))


def measure_prefill(amd, dev, model, reps=5):
    """The chunked forward at BitNet-2B shape: PREFILL_TOKENS tokens as one
    chunk from position 0 (every projection one int8-MFMA GEMM over the
    chunk), after untimed chunks until the time settles, timed with HIP
    events on the library stream -- with the output
    head for the last token only (a prompt's prefill), and for every token
    (sllm_forward_chunk's full output, its copy to host memory included).
    Rows 0..PREFILL_CHECK-1 of the full output go to the CPU leg's bit-exact
    check against the oracle, and the rows at PREFILL_CHECK_POS to its check
    against the reference's own chunked forward over the same 512 tokens."""
    cfg = dict(amd.BITNET_2B)
    n = PREFILL_TOKENS
    toks = [int(t) for t in np.random.default_rng(90).integers(0, cfg["n_vocab"], n)]
    g = amd.DeviceDecoder(dev, model, n + 8)
    res, med, warm = {}, {}, {}
    for label, logits in (("last", False), ("all", True)):
        # untimed chunks until three in a row agree within 1 % (the clocks
        # and caches take a few chunks to settle), at most 12
        seen = []
        for _ in range(12):
            g.reset()
            dev.events(2)
            dev.sync()
            dev.record(0)
            g.forward_chunk(toks, 0, logits=logits)
            dev.record(1)
            dev.sync()
            seen.append(dev.elapsed(0, 1))
            if len(seen) >= 3 and max(seen[-3:]) <= 1.01 * min(seen[-3:]):
                break
        warm[label] = [round(t, 3) for t in seen]
        times = []
        for _ in range(reps):
            g.reset()
            dev.events(2)
            dev.sync()
            dev.record(0)
            g.forward_chunk(toks, 0, logits=logits)
            dev.record(1)
            dev.sync()
            times.append(dev.elapsed(0, 1))
        res[label], med[label] = min(times), float(np.median(times))
    g.reset()
    full = g.forward_chunk(toks, 0, logits=True)
    g.close()
    check = {"model": model, "tokens": toks, "logits": full[:PREFILL_CHECK].copy(),
             "strided": full[list(PREFILL_CHECK_POS)].copy()}
    del full
    return check, {
        "workload": (f"random-init BitNet-b1.58-2B, one chunk of {n} tokens at positions 0..{n - 1} "
                     f"(sllm_gfx950_forward_chunk), batch 1"),
        "tokens": n,
        "ms_last_logits": round(res["last"], 3), "ms_last_logits_median": round(med["last"], 3), "reps": reps,
        "warmup_ms": warm,
        "tokens_per_s": round(n / (res["last"] * 1e-3), 1),
        "ms_all_logits_incl_host_copy": round(res["all"], 3),
        "ms_all_logits_incl_host_copy_median": round(med["all"], 3),
        "all_logits_tokens_per_s": round(n / (res["all"] * 1e-3), 1),
    }


PEAK_INT8_TOPS = 5000.0
GEMM_SETS = 64


def measure_gemm(amd, dev):
    """Several tokens against one tensor: the int8-MFMA GEMM (q quantised
    beforehand, timed alone) against the GEMV path (one plan of M jobs
    sharing the tensor, each quantising its own token in-kernel), over
    GEMM_SETS rotated weight sets (283 MB: HBM, not the Infinity Cache).
    Token counts 4, 16, 64 at both FFN shapes, and the 512-token prefill
    chunk at 6912 x 2560."""
    rows, checks = [], []
    for n_rows, k, ms in ((6912, 2560, (4, 16, 64, 512)), (2560, 6912, (4, 16, 64))):
        ws = [amd.synth_i2s(amd.synth_seed(6, s_, n_rows, k), n_rows, k) for s_ in range(GEMM_SETS)]
        bws = [dev.put(w) for w in ws]
        for m in ms:
            x = np.concatenate([amd.synth_normal(amd.synth_seed(6, 0, t, 77), k) for t in range(m)]).astype(np.float32)
            bx, bq, ba = dev.put(x), dev.alloc(m * k), dev.alloc(8 * m)
            by, bi = dev.alloc(4 * m * n_rows), dev.alloc(4 * m * n_rows)
            dev.quant_act(bx.vp, k, m, bq.vp, ba.vp)
            for i in range(GEMM_SETS):
                dev.gemm(bws[i].vp, n_rows, k, bq.vp, ba.vp, m, by.vp)
            dev.gemm(bws[0].vp, n_rows, k, bq.vp, ba.vp, m, by.vp, bi.vp)
            dev.sync()
            pick = sorted({0, m // 2, m - 1})
            yd = by.download(np.float32, m * n_rows).reshape(m, n_rows)
            dd = bi.download(np.int32, m * n_rows).reshape(m, n_rows)
            checks.append((ws[0], n_rows, k, x, m, pick, yd[pick], dd[pick], f"gemm {n_rows}x{k} m={m}"))
            rot = iter(range(1 << 30))
            settle(dev, lambda: dev.gemm(bws[next(rot) % GEMM_SETS].vp, n_rows, k, bq.vp, ba.vp, m, by.vp))
            bt_m = timed_batches(dev, lambda: dev.gemm(bws[next(rot) % GEMM_SETS].vp, n_rows, k, bq.vp, ba.vp, m, by.vp),
                           8, GEMM_SETS)
            mfma_us = bt_m["median_us"]
            plans = [dev.plan([amd.GemvJob(bws[i].ptr, n_rows, k, bx.ptr + 4 * k * t, None, None, by.ptr + 4 * n_rows * t,
                                           None) for t in range(m)]) for i in range(GEMM_SETS)]
            for p in plans:
                dev.plan_run(p)
            dev.sync()
            bt_g = timed_batches(dev, lambda: dev.plan_run(plans[next(rot) % GEMM_SETS]), 4, GEMM_SETS)
            gemv_us = bt_g["median_us"]
            for p in plans:
                dev.plan_destroy(p)
            for b in (bx, bq, ba, by, bi):
                b.free()
            ops = 2.0 * m * n_rows * k
            byts = n_rows * k // 4 + 32 + m * k + 8 * m + 4 * m * n_rows
            rows.append({"n_rows": n_rows, "k": k, "tokens": m, "mfma_us": round(mfma_us, 2),
                         "mfma_TOPS": round(ops / mfma_us / 1e6, 1),
                         "mfma_frac_int8_peak": round(ops / mfma_us / 1e6 / PEAK_INT8_TOPS, 4),
                         "mfma_GBps": round(byts / mfma_us / 1e3, 1), "gemv_plan_us": round(gemv_us, 2),
                         "mfma_best_us": bt_m["best_us"], "mfma_batch_us": bt_m["batch_us"],
                         "gemv_plan_best_us": bt_g["best_us"],
                         "faster": "mfma" if mfma_us < gemv_us else "gemv"})
            log(f"gemm {n_rows}x{k} m={m}: mfma {mfma_us:.2f} us ({ops / mfma_us / 1e6:.1f} TOPS), gemv plan {gemv_us:.2f} us")
        for b in bws:
            b.free()
    return checks, rows


def measure_gemm_plan(amd, dev, wl, token_counts=(4, 16, 64)):
    """The multi-tensor form: the FFN workload's 96 tensors (32 rotated sets
    of gate / up / down, 424.7 MB) against m tokens each, as one GEMM plan
    launch -- every tensor with its own quantised rows (gate and up share
    theirs) -- beside the GEMV plan doing the same work (one job per tensor
    and token, each quantising its token in-kernel). Bytes: packed weights,
    int8 rows and f32 outputs. The plan's outputs of sets 0 and 31 are
    checked bit for bit against sllm_gfx950_gemm tensor by tensor."""
    rows = []
    for m in token_counts:
        xs_up = [np.concatenate([amd.synth_normal(amd.synth_seed(7, s, t, 100), K_UP) for t in range(m)])
                 for s in range(wl.sets)]
        xs_dn = [np.concatenate([amd.synth_normal(amd.synth_seed(7, s, t, 101), N_FF) for t in range(m)])
                 for s in range(wl.sets)]
        bxu, bxd = dev.put(np.concatenate(xs_up)), dev.put(np.concatenate(xs_dn))
        bqu, bqd = dev.alloc(wl.sets * m * K_UP), dev.alloc(wl.sets * m * N_FF)
        bau, bad = dev.alloc(wl.sets * m * 8), dev.alloc(wl.sets * m * 8)
        dev.quant_act(bxu.vp, K_UP, wl.sets * m, bqu.vp, bau.vp)
        dev.quant_act(bxd.vp, N_FF, wl.sets * m, bqd.vp, bad.vp)
        outs = [dev.alloc(4 * m * n_rows) for s in range(wl.sets) for _, n_rows, _ in SHAPES]
        jobs = []
        for s in range(wl.sets):
            for t_, (name, n_rows, n) in enumerate(SHAPES):
                up = n == K_UP
                q = (bqu if up else bqd).ptr + s * m * n
                a = (bau if up else bad).ptr + s * m * 8
                jobs.append((wl.jobs[3 * s + t_].w, n_rows, n, q, a, outs[3 * s + t_].ptr, None))
        plan = dev.gemm_plan(jobs, m)
        settle(dev, lambda: dev.gemm_plan_run(plan), batch=10)
        bt_p = timed_batches(dev, lambda: dev.gemm_plan_run(plan), 8, 10)
        plan_us = bt_p["median_us"]
        # the same tensors one sllm_gfx950_gemm at a time, for the check
        ref = dev.alloc(4 * m * N_FF)
        for s in (0, wl.sets - 1):
            for t_, (name, n_rows, n) in enumerate(SHAPES):
                j = jobs[3 * s + t_]
                dev.gemm(j[0], n_rows, n, j[3], j[4], m, ref.vp)
                dev.sync()
                got = outs[3 * s + t_].download(np.float32, m * n_rows)
                want = ref.download(np.float32, m * n_rows)
                if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
                    raise SystemExit(f"bench: GEMM plan output differs from sllm_gfx950_gemm (set {s} {name}, m={m})")
        ref.free()
        dev.gemm_plan_destroy(plan)
        # the GEMV plan over the same tensors and tokens
        gjobs = []
        for s in range(wl.sets):
            for t_, (name, n_rows, n) in enumerate(SHAPES):
                bx = bxu if n == K_UP else bxd
                for t in range(m):
                    gjobs.append(amd.GemvJob(wl.jobs[3 * s + t_].w, n_rows, n, bx.ptr + 4 * (s * m + t) * n, None, None,
                                             outs[3 * s + t_].ptr + 4 * t * n_rows, None))
        gplan = dev.plan(gjobs)
        dev.plan_run(gplan)
        bt_g = timed_batches(dev, lambda: dev.plan_run(gplan), 3, 1)
        gemv_us = bt_g["median_us"]
        dev.plan_destroy(gplan)
        for b in [bxu, bxd, bqu, bqd, bau, bad] + outs:
            b.free()
        byts = wl.weight_bytes + wl.sets * m * (K_UP + N_FF) + wl.sets * m * 8 * 2 + \
            4 * m * sum(n_rows for _, n_rows, _ in SHAPES) * wl.sets
        ops = 2.0 * m * sum(n_rows * n for _, n_rows, n in SHAPES) * wl.sets
        rows.append({"tokens": m, "tensors": len(jobs), "plan_us": round(plan_us, 2),
                     "plan_GBps": round(byts / plan_us / 1e3, 1), "plan_TOPS": round(ops / plan_us / 1e6, 1),
                     "plan_best_us": bt_p["best_us"], "plan_GBps_best": round(byts / bt_p["best_us"] / 1e3, 1),
                     "plan_batch_us": bt_p["batch_us"], "bytes": byts,
                     "gemv_plan_us": round(gemv_us, 2), "gemv_plan_best_us": bt_g["best_us"],
                     "faster": "mfma" if plan_us < gemv_us else "gemv"})
        log(f"gemm plan, 96 tensors x {m} tokens: {plan_us:.1f} us ({byts / plan_us / 1e3:.0f} GB/s), "
            f"GEMV plan {gemv_us:.1f} us")
    return rows


def settle(dev, launch, batch=25, max_batches=80, tol=0.005, min_ms=25.0):
    """Run `launch` (one launch of the timed work) untimed until its duration
    is steady: batches of `batch` launches (HIP events on the stream) until
    three batches in a row agree with the one before within `tol` and at
    least `min_ms` of launches have run, or `max_batches` batches.
    From idle clocks the launch starts near 65 us, rises to about 76 us and
    only then comes down to its steady 64 us, about 375 launches (25 ms) in;
    the W warm-up steps alone (5 in the driver's runs) stop inside that ramp.
    Measured over four seconds of back-to-back launches the steady figure
    holds (no later throttling)."""
    dev.events(2)
    hist, calm = [], 0
    for _ in range(max_batches):
        dev.record(0)
        for _ in range(batch):
            launch()
        dev.record(1)
        dev.sync()
        hist.append(dev.elapsed(0, 1) * 1e3 / batch)
        if len(hist) > 1 and abs(hist[-1] - hist[-2]) <= tol * hist[-1]:
            calm += 1
            if calm >= 3 and sum(hist) * batch / 1e3 >= min_ms:
                break
        else:
            calm = 0
    return {"launches": batch * len(hist), "first_batch_us": round(hist[0], 2), "max_batch_us": round(max(hist), 2),
            "last_batch_us": round(hist[-1], 2)}


def timed_batches(dev, run, n_batches, per_batch):
    """Microseconds per call of `run`: n_batches batches of per_batch
    back-to-back calls, HIP events on the library stream at each batch's
    edges. Returns median, best and every batch's mean (the reference's
    tgbench reports best / median / spread the same way,
    bench/tg_bench.c:256-333)."""
    dev.events(2)
    us = []
    for _ in range(n_batches):
        dev.sync()
        dev.record(0)
        for _ in range(per_batch):
            run()
        dev.record(1)
        dev.sync()
        us.append(dev.elapsed(0, 1) * 1e3 / per_batch)
    return {"median_us": round(float(np.median(us)), 2), "best_us": round(min(us), 2),
            "batch_us": [round(u, 2) for u in us], "per_batch": per_batch}


def with_rate(b, byts):
    """A timed_batches() record with GB/s at its median and best."""
    return dict(b, GBps_median=round(byts / b["median_us"] / 1e3, 1), GBps_best=round(byts / b["best_us"] / 1e3, 1))


def measure_ffn_sets(amd, dev, wl):
    """Config 1 in its per-set form: one launch per weight set (gate, up and
    down of one set as a three-job plan, gate and up sharing the quantised
    input), the 32 sets rotated launch after launch, many back-to-back
    launches. Bytes per launch: one set's share of the headline's."""
    plans = [dev.plan(wl.jobs[3 * s_:3 * s_ + 3]) for s_ in range(wl.sets)]
    rot = iter(range(1 << 40))
    run = lambda: dev.plan_run(plans[next(rot) % wl.sets])  # noqa: E731
    st = settle(dev, run)
    b = timed_batches(dev, run, 10, 10 * wl.sets)
    for p_ in plans:
        dev.plan_destroy(p_)
    per_set = wl.step_bytes // wl.sets
    return dict(with_rate(b, per_set), bytes_per_launch=per_set, settle=st,
                frac_of_peak_median=round(per_set / b["median_us"] / 1e3 / PEAK_HBM_GBS, 4),
                workload=("the FFN workload one set per launch: gate + up (shared int8 input) + down of one of the "
                          f"{wl.sets} sets, sets rotated, {10 * wl.sets} launches per batch"))


def measure_copy_bandwidth(dev, nbytes=2 << 30, reps=20):
    """Plain device copy and read-only checksum of known size: the achievable
    HBM figure beside the GEMV."""
    src, dst = dev.alloc(nbytes), dev.alloc(nbytes)
    part = dev.alloc(4 * 2048)
    dev.copy(dst.vp, src.vp, nbytes)
    dev.checksum(src.vp, nbytes, part.vp, 2048)
    dev.sync()
    dev.timer_start()
    for _ in range(reps):
        dev.copy(dst.vp, src.vp, nbytes)
    copy_ms = dev.timer_stop() / reps
    dev.timer_start()
    for _ in range(reps):
        dev.checksum(src.vp, nbytes, part.vp, 2048)
    read_ms = dev.timer_stop() / reps
    for b in (src, dst, part):
        b.free()
    return {"copy_GBps": round(2 * nbytes / copy_ms / 1e6, 1),
            "read_GBps": round(nbytes / read_ms / 1e6, 1), "bytes": nbytes}


def host_cpu():
    """The host's CPU model, the logical CPUs this process may run on and the
    physical cores among them (distinct (package, core) pairs in
    /proc/cpuinfo), and the thread counts the CPU baselines use: 1, 4 and
    all (at most 16: the host's share of CPUs per GPU)."""
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except AttributeError:
        allowed = list(range(os.cpu_count() or 1))
    model, cores, ident, flags = "", set(), {}, set()
    try:
        for block in open("/proc/cpuinfo").read().split("\n\n"):
            d = {}
            for line in block.splitlines():
                if ":" in line:
                    key, val = line.split(":", 1)
                    d[key.strip()] = val.strip()
            if "processor" not in d or int(d["processor"]) not in allowed:
                continue
            model = model or d.get("model name", "")
            if not ident:
                ident = {k_: d.get(k_) for k_ in ("vendor_id", "cpu family", "model", "stepping", "microcode",
                                                  "cache size", "cpu MHz")}
                flags = set(d.get("flags", "").split())
            cores.add((d.get("physical id", "0"), d.get("core id", d["processor"])))
    except OSError:
        pass
    top = min(16, len(allowed))
    # the ISA the reference's dot selects on (src/i2s_gemm.c:292-363)
    isa = [f for f in ("avx2", "fma", "f16c", "avx_vnni", "avx512f", "avx512_vnni", "avx512_bf16") if f in flags]
    return {"cpu": model, "cpu_id": ident, "isa": isa, "logical_cpus": len(allowed),
            "physical_cores": len(cores) or None, "thread_counts": sorted({1, min(4, top), top})}


def cpu_decode(dec_check, seconds=10.0, thread_counts=(16,)):
    """The decode parity check, token witness and baseline. Parity: the
    oracle's decode step on the same model and prefix at the same position --
    logits, every int32 dot and every activation of the GPU's traced token,
    bit for bit. Baseline: the reference's own sllm_forward (oracle/_ref)
    restored to the same prefix through its state file (src/forward.c:963-1100),
    greedy decode timed for about `seconds` at each thread count. Witness (as
    the reference's tgbench checks its token stream, bench/tg_bench.c:300-321):
    every run's greedy ids equal the GPU's ids position by position over the
    positions both generated; a mismatch ends the bench."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    from oracle.gguf_synth import state_image
    import tempfile
    c = dec_check
    model, cfg = c["model"], c["model"]["cfg"]
    n_ctx = DECODE_PREFIX + 512
    o = orc.Decoder(model, n_ctx)
    ok, ov = o.caches()
    ok[:, :, :DECODE_PREFIX] = c["k"]
    ov[:, :, :DECODE_PREFIX] = c["v"]
    want, wdots, wacts = o.forward(c["token"], DECODE_PREFIX, trace=True)
    o.close()
    bits = lambda a: np.ascontiguousarray(a, np.float32).view(np.uint32)
    if not (np.array_equal(bits(want), bits(c["logits"])) and np.array_equal(wdots, c["dots"])
            and np.array_equal(wacts["sum"], c["acts"]["sum"]) and np.array_equal(bits(wacts["scale"]), bits(c["acts"]["scale"]))):
        raise SystemExit("bench: the GPU decode step differs from the oracle")
    log(f"decode at position {DECODE_PREFIX}: logits, {wdots.size} int32 dots and {wacts.size} activations "
        f"match the oracle bit for bit")
    if not orc.ref_available():
        return {"checked": True, "cpu": None, "witness": None}
    fd, path = tempfile.mkstemp(suffix=".slkv")
    os.close(fd)
    runs, witnessed = [], 0
    gpu_ids = c["ids"]
    try:
        with open(path, "wb") as f:
            f.write(state_image(cfg, n_ctx, c["k"], c["v"], want))
        for threads in thread_counts:
            r = orc.RefDecoder(model, n_ctx, threads=threads)
            r.state_load(path)
            tok, pos, ids = int(c["token"]), DECODE_PREFIX, []
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < seconds and pos < n_ctx:
                lg = r.forward(tok, pos)
                tok = int(orc.ref().ref_argmax(orc._p(lg), lg.size))
                ids.append(tok)
                pos += 1
            dt = time.perf_counter() - t0
            r.close()
            n = min(len(ids), len(gpu_ids))
            for i in range(n):
                if ids[i] != gpu_ids[i]:
                    raise SystemExit(f"bench: token witness: the reference's greedy id at position "
                                     f"{DECODE_PREFIX + 1 + i} is {ids[i]}, the GPU's {gpu_ids[i]}")
            witnessed = max(witnessed, n)
            runs.append({"threads": threads, "tokens_per_s": round(len(ids) / dt, 2), "tokens": len(ids),
                         "seconds": round(dt, 1)})
            log(f"reference decode, {threads} threads: {len(ids) / dt:.2f} tokens/s; "
                f"{n} greedy ids equal to the GPU's")
    finally:
        os.remove(path)
    best = max(runs, key=lambda r_: r_["tokens_per_s"])
    return {"checked": True, "witness": witnessed,
            "cpu": dict(best, kind="reference", runs=runs,
                        sample=f"sllm_forward greedy from position {DECODE_PREFIX} after the same prefix, "
                               f"at {', '.join(str(r_['threads']) for r_ in runs)} threads; the fastest")}


def cpu_prefill(pre_check, seconds=10.0, thread_counts=(16,)):
    """Parity: rows 0..15 of the chunk's logits against the oracle's
    token-by-token logits, and the rows at PREFILL_CHECK_POS (one in every
    eight-token scores block, 511 included) against the reference's own
    sllm_forward_chunk (oracle/_ref) over the same 512 tokens, bit for bit.
    Baseline: that reference chunked forward, chunks of 16 from position 0 --
    at the highest thread count over all 512 tokens (the run the strided
    check reads), at the others as many chunks as fit in about `seconds`."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    c = pre_check
    model = c["model"]
    o = orc.Decoder(model, PREFILL_CHECK + 8)
    want = np.stack([o.forward(t, p) for p, t in enumerate(c["tokens"][:PREFILL_CHECK])])
    o.close()
    if not np.array_equal(want.view(np.uint32), np.ascontiguousarray(c["logits"], np.float32).view(np.uint32)):
        raise SystemExit("bench: the GPU chunk's logits differ from the oracle")
    log(f"prefill chunk: logits of positions 0..{PREFILL_CHECK - 1} match the oracle bit for bit")
    if not orc.ref_available():
        return {"checked": True, "strided": False, "cpu": None}
    toks = np.asarray(c["tokens"], np.int32)
    pos = list(PREFILL_CHECK_POS)
    runs = []
    for threads in sorted(thread_counts, reverse=True):
        whole = threads == max(thread_counts)
        r = orc.RefDecoder(model, PREFILL_TOKENS + 8, threads=threads)
        rows = {}
        done, t0 = 0, time.perf_counter()
        while done + 16 <= PREFILL_TOKENS and (whole or time.perf_counter() - t0 < seconds):
            lg = r.forward_chunk(toks[done:done + 16], done)
            if whole:
                for p_ in pos:
                    if done <= p_ < done + 16:
                        rows[p_] = lg[p_ - done].copy()
            done += 16
        dt = time.perf_counter() - t0
        r.close()
        runs.append({"threads": threads, "tokens_per_s": round(done / dt, 2), "tokens": done, "seconds": round(dt, 1)})
        log(f"reference chunked prefill, {threads} threads: {done / dt:.2f} tokens/s")
        if whole:
            ref_rows = np.stack([rows[p_] for p_ in pos])
            got = np.ascontiguousarray(c["strided"], np.float32)
            if not np.array_equal(ref_rows.view(np.uint32), got.view(np.uint32)):
                bad = [p_ for i, p_ in enumerate(pos) if not np.array_equal(ref_rows[i].view(np.uint32),
                                                                           got[i].view(np.uint32))]
                raise SystemExit(f"bench: the GPU chunk's logits differ from the reference's at positions {bad[:8]}")
            log(f"prefill chunk: logits of {len(pos)} positions (one per eight-token block, 0..511) match the "
                "reference's own chunked forward bit for bit")
    best = max(runs, key=lambda r_: r_["tokens_per_s"])
    return {"checked": True, "strided": True,
            "cpu": dict(best, kind="reference", runs=runs,
                        sample="sllm_forward_chunk, chunks of 16 from position 0, every token's logits; at "
                               f"{max(thread_counts)} threads all {PREFILL_TOKENS} tokens, at the others as many "
                               "chunks as fit in the time allowed; the fastest")}


def cpu_gemm_check(checks):
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    n = 0
    for w, n_rows, k, x, m, pick, yd, dd, what in checks:
        for i, t in enumerate(pick):
            yo, qo, do, so, su = orc.linear(w, n_rows, k, x[t * k:(t + 1) * k])
            if not (np.array_equal(dd[i], do) and np.array_equal(yd[i].view(np.uint32), yo.view(np.uint32))):
                raise SystemExit(f"bench: {what} token {t} differs from the oracle")
            n += 1
    log(f"{n} GEMM tokens (first, middle, last of every run) match the oracle bit for bit")


def cpu_baseline(wl, checks, seconds=6.0, cfg0=None, host=None):
    """The CPU leg. First the parity check: the GPU outputs kept in `checks`
    against the oracle, bit for bit. Then the baseline: the reference's CPU
    path (or the oracle's restatement) over a bounded sample of the same
    workload -- passes over the 32 sets, each set quantise -> GEMV ->
    epilogue for gate/up/down, row-parallel over the reference's pool --
    timed at 1 thread and at all threads; at all threads both with the
    reference's own split policy (src/forward.c:145-205, which keeps GEMVs
    below 512 rows per thread on one thread) and with every GEMV
    distributed; the faster all-thread figure is the baseline. cfg0: (the
    2560 x 2560 tensors, their activations) timed the same way."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as orc
    for w, n_rows, n, x, got, what in checks:
        want = orc.linear(w, n_rows, n, x, orc.DOT_VNNI)[0]
        if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
            raise SystemExit(f"bench: output mismatch against the oracle ({what})")
    log(f"{len(checks)} GPU outputs (sets 0 and 31, block layers 0 and 29, cfg0 copies, drop-in row) "
        f"match the oracle bit for bit")
    use_ref = orc.ref_available()
    host = host or host_cpu()
    threads = host["thread_counts"][-1]
    Act = orc.Act
    q_buf = np.empty(N_FF, np.int8)
    dots = np.empty(N_FF, np.int32)
    y = np.empty(N_FF, np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)

    def timed(nt, distribute_all, unit):
        """unit(quant, run, i): the i-th unit of work (quantise + GEMVs);
        returns the units done in about `seconds`."""
        if use_ref:
            r = orc.ref()
            r.sllm_i2s_select_auto()
            pool = r.ref_pool_create(nt)
            quant = r.sllm_i2s_quant_act
            run = lambda w, n_rows, n, q, a: r.ref_gemv_epilogue(pool, P(w), n_rows, n, P(q), ctypes.byref(a),
                                                                 P(dots), P(y), distribute_all)
        else:
            o = orc.orc()
            pool = o.orc_pool_create(nt)
            path = orc.DOT_VNNI if o.orc_vnni_supported() else orc.DOT_V3
            quant = o.orc_quant_act
            run = lambda w, n_rows, n, q, a: o.orc_gemv_epilogue_parallel(pool, P(w), n_rows, n, P(q), ctypes.byref(a),
                                                                          P(dots), P(y), path)
        done = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            unit(quant, run, done)
            done += 1
        dt = time.perf_counter() - t0
        if use_ref:
            orc.ref().sllm_pool_destroy(pool)
            isa = {0: "v3", 1: "vnni"}.get(orc.ref().sllm_i2s_dot_isa(), "other")
        else:
            orc.orc().orc_pool_destroy(pool)
            isa = "vnni" if orc.orc().orc_vnni_supported() else "v3"
        return {"units": done, "seconds": dt, "dot": isa}

    def ffn_set(quant, run, i):
        s = i % wl.sets
        ws, a = wl.host_w[s], Act()
        quant(P(wl.x_up[s]), K_UP, P(q_buf), ctypes.byref(a))
        run(ws[0], N_FF, K_UP, q_buf, a)
        run(ws[1], N_FF, K_UP, q_buf, a)
        quant(P(wl.x_dn[s]), N_FF, P(q_buf), ctypes.byref(a))
        run(ws[2], K_UP, N_FF, q_buf, a)

    def sweep(unit, unit_bytes):
        one = timed(1, 0, unit)
        policy = timed(threads, 0, unit)
        spread = timed(threads, 1, unit) if use_ref else policy
        gbps = lambda t: t["units"] * unit_bytes / t["seconds"] / 1e9
        best = max((policy, "reference split policy"), (spread, "every GEMV distributed"), key=lambda t: gbps(t[0]))
        return one, policy, spread, best, gbps

    one, policy, spread, best, gbps = sweep(ffn_set, wl.step_bytes / wl.sets)
    b = best[0]
    out = {
        "value": round(gbps(b), 3), "unit": "GB/s", "cores": threads,
        "kind": "reference" if use_ref else "port",
        "sample": (f"{b['units']} FFN sets (gate+up+down: quantise+GEMV+epilogue) cycling over the same "
                   f"{wl.sets} weight sets in {b['seconds']:.1f}s, {threads} threads, {best[1]}, dot={b['dot']}"),
        "one_thread_GBps": round(gbps(one), 3),
        "policy_GBps": round(gbps(policy), 3),
        "all_distributed_GBps": round(gbps(spread), 3),
        "host": host,
    }
    if cfg0 is not None:
        ws0, xs0 = cfg0
        n = CFG0_N

        def cfg0_call(quant, run, i):
            a = Act()
            quant(P(xs0[i % len(ws0)]), n, P(q_buf), ctypes.byref(a))
            run(ws0[i % len(ws0)], n, n, q_buf, a)

        one, policy, spread, best, gbps = sweep(cfg0_call, n * n // 4 + 4 + 8 * n)
        out["cfg0"] = {"one_thread_GBps": round(gbps(one), 3), "policy_GBps": round(gbps(policy), 3),
                       "all_distributed_GBps": round(gbps(spread), 3), "threads": threads,
                       "best_us_per_call": round(best[0]["seconds"] / best[0]["units"] * 1e6, 1),
                       "sample": f"quantise + GEMV + epilogue of the 2560x2560 tensors rotated over {len(ws0)}, "
                                 f"{best[1]} at {threads} threads, dot={best[0]['dot']}"}
        log(f"cfg0 reference CPU: {gbps(one):.2f} GB/s on 1 thread, {gbps(best[0]):.2f} GB/s on {threads}")
    return out


I2S_CODE_OBJECT = os.path.join(ROOT, "saphira-llm_amd", "build", "i2s_gfx950.hsaco")
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "gemv_slab_ffn32_traffic.json")


def code_object_sha256():
    """SHA-256 of the GEMV code object embedded in the library (the build's
    i2s_gfx950.hsaco), or None when it is not on disk."""
    import hashlib
    try:
        with open(I2S_CODE_OBJECT, "rb") as f:
            return hashlib.sha256(f.read()).hexdigest()
    except OSError:
        return None


def profiled_traffic():
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes over this same workload (scaled by the counters'
    reading of a copy of known size) -- only when they were taken on the code
    object this run uses (its SHA-256 is stored with them); else None."""
    if not os.path.exists(TRAFFIC_JSON):
        return None, "no traffic profile"
    with open(TRAFFIC_JSON) as f:
        t = json.load(f)
    cur = code_object_sha256()
    if cur is None or t.get("code_object_sha256") != cur:
        return None, "traffic profile taken on another build of the GEMV code object"
    return t.get("hbm_bytes_per_launch"), "rocprofv3 FETCH_SIZE / WRITE_SIZE of this code object (profiles/)"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-graph", action="store_true",
                    help="decode leg: enqueue each token's launches instead of replaying a HIP graph "
                         "(rocprofv3's kernel tracer does not survive graph replay)")
    ap.add_argument("--inflight", type=int, default=None,
                    help="decode leg: tokens the device greedy loop keeps enqueued ahead of the host "
                         "(default: the library's)")
    ap.add_argument("--sustain", type=float, default=0.0,
                    help="after the timed steps, keep the headline launch running this many seconds in "
                         "batches of 2000 and report each batch's mean (a sustained-clock check; 0: off)")
    ap.add_argument("--legs", default="cfg0,sets,dropin,block,decode,prefill,gemm",
                    help="comma-separated legs to run beside the headline GEMV (cfg0, sets, dropin, block, decode, "
                         "prefill, gemm); for profiling one leg")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the I2_S GEMV path runs on a single MI355X and "
              "the library has no multi-GPU path (--gpus must be 1).", file=sys.stderr)
        sys.exit(2)

    amd = load_package()
    dev = amd.Device(0)
    log(f"device {dev.name}, {dev.cu} CUs, {dev.hbm / 2**30:.0f} GiB")
    wl = Workload(amd, dev)

    # steady clocks first (the launch's own ramp from idle), then the W
    # warm-up steps; the copy / read calibration runs after every other leg:
    # its 86 GB of copies leave the launch about 4 % slower for some 100 ms
    st = settle(dev, wl.step)
    log(f"settled after {st['launches']} launches: {st['first_batch_us']} us per launch at first, "
        f"{st['max_batch_us']} at most, {st['last_batch_us']} at the end")
    for _ in range(args.warmup):
        wl.step()
    dev.sync()

    K = args.steps
    dev.events(2)
    dev.sync()
    t0 = time.perf_counter()
    dev.record(0)
    for _ in range(K):
        wl.step()
    dev.record(1)
    dev.sync()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / K
    value = wl.step_bytes / (ms_per_step * 1e-3) / 1e9
    gemv_avg = dev.elapsed(0, 1) / K
    achieved = wl.gemv_bytes / (gemv_avg * 1e-3) / 1e9
    log(f"step {ms_per_step * 1e3:.1f} us wall, slab GEMV {gemv_avg * 1e3:.1f} us per launch "
        f"(events on the stream), {achieved:.0f} GB/s")
    sustained = None
    if args.sustain > 0:
        batches, t_end = [], time.perf_counter() + args.sustain
        while time.perf_counter() < t_end:
            dev.record(0)
            for _ in range(2000):
                wl.step()
            dev.record(1)
            dev.sync()
            batches.append(round(dev.elapsed(0, 1) / 2000 * 1e3, 2))
        sustained = {"batch_launches": 2000, "batch_us": batches, "mean_us": round(sum(batches) / len(batches), 2),
                     "GBps_at_mean": round(wl.gemv_bytes / (sum(batches) / len(batches) * 1e-6) / 1e9, 1)}
        log(f"sustained {args.sustain:.0f} s: {len(batches)} batches of 2000 launches, "
            f"{min(batches)}..{max(batches)} us per launch, mean {sustained['mean_us']}")

    # the same launch in ten batches of 100, for its median and best
    head_batches = with_rate(timed_batches(dev, wl.step, 10, 100), wl.gemv_bytes)
    log(f"headline in batches of 100: median {head_batches['median_us']} us, best {head_batches['best_us']} us")
    traffic, traffic_note = profiled_traffic()

    checks = wl.outputs([0, wl.sets - 1])
    legs = set(args.legs.split(","))
    block_checks, block30, dec_check, decode, gemm_checks, gemm = [], None, None, None, [], None
    pre_check, prefill = None, None
    cfg0_checks, cfg0_host, cfg0 = [], None, None
    dropin_checks, dropin = [], None
    if "cfg0" in legs:
        cfg0_checks, cfg0_host, cfg0 = measure_cfg0(amd, dev)
    ffn_sets = None
    if "sets" in legs:
        ffn_sets = measure_ffn_sets(amd, dev, wl)
        log(f"FFN sets one per launch: median {ffn_sets['median_us']} us ({ffn_sets['GBps_median']} GB/s), "
            f"best {ffn_sets['best_us']} us ({ffn_sets['GBps_best']} GB/s)")
    if "dropin" in legs:
        dropin_checks, dropin = measure_dropin(amd, wl)
        dropin["device_resident_us_per_set"] = round(gemv_avg * 1e3 / SETS, 2)
        dropin["x_device_resident"] = round(dropin["us_per_set"] / (gemv_avg * 1e3 / SETS), 1)
    if "block" in legs:
        block_checks, block30 = measure_block_plan(amd, dev)
        log(f"block plan (30 layers, 210 GEMVs): {block30['us_per_launch']} us per launch, {block30['GBps']} GB/s")
    if "decode" in legs:
        dec_check, decode = measure_decode(amd, dev, graph=not args.no_graph, inflight=args.inflight)
        log(f"decode: {decode['tokens_per_s']} tokens/s ({decode['us_per_token']} us per token, "
            f"{decode['effective_GBps']} GB/s effective)")
    if "prefill" in legs:
        pre_model = dec_check["model"] if dec_check is not None else amd.synth_model(dict(amd.BITNET_2B), 0)
        pre_check, prefill = measure_prefill(amd, dev, pre_model)
        log(f"prefill: {prefill['tokens']}-token chunk {prefill['ms_last_logits']} ms "
            f"({prefill['tokens_per_s']} tokens/s); with every token's logits {prefill['ms_all_logits_incl_host_copy']} ms")
    if "gemm" in legs:
        gemm_checks, gemm = measure_gemm(amd, dev)
        gemm = {"per_tensor": gemm, "plan_96_tensors": measure_gemm_plan(amd, dev, wl)}
    # last: its copies leave the GPU slower for some 100 ms
    calib = measure_copy_bandwidth(dev)
    log(f"calibration: copy {calib['copy_GBps']} GB/s, read {calib['read_GBps']} GB/s")

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": K, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {
            "workload": "BitNet-2B FFN GEMVs batch 1: gate+up 6912x2560 (shared activation) and "
                        "down 2560x6912, 32 independently seeded I2_S weight sets rotated per step "
                        "(424.7 MB packed), f32 N(0,1) activations int8-absmax quantised per token, "
                        "f32 outputs",
            "sets": SETS, "weight_bytes": wl.weight_bytes, "step_bytes": wl.step_bytes,
            "launches_per_step": 1, "hbm_frac_of_peak": round(value / PEAK_HBM_GBS, 4),
            "tops": round(wl.ops / (ms_per_step * 1e-3) / 1e12, 3),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic, "traffic_source": traffic_note,
            "kernel": "sllm_k_gemv_slab (96 GEMVs with in-kernel quantisation, one launch)",
            "avg_launch_us": round(gemv_avg * 1e3, 2), "bytes_per_launch": wl.gemv_bytes,
        },
        "settle": st,
        "batches": head_batches,
        "sustained": sustained,
        "ffn_sets": ffn_sets,
        "calibration": calib,
        "cfg0": cfg0,
        "dropin": dropin,
        "block30": block30,
        "decode": decode,
        "prefill": prefill,
        "gemm": gemm,
    }
    if not args.no_cpu:
        log("timing the CPU baseline")
        host = host_cpu()
        out["cpu_baseline"] = cpu_baseline(wl, checks + block_checks + cfg0_checks + dropin_checks, args.cpu_seconds, cfg0_host, host)
        cpu_gemm_check(gemm_checks)
        if dec_check is not None:
            dec = cpu_decode(dec_check, seconds=args.cpu_seconds, thread_counts=host["thread_counts"])
            out["decode"]["parity"] = ("logits, int32 dots and activations of the first token bit-identical to the "
                                       "oracle; greedy ids equal to the reference's own at every position both "
                                       "generated")
            out["decode"]["token_witness"] = dec["witness"]
            out["decode"]["cpu_baseline"] = dec["cpu"]
        if pre_check is not None:
            pre = cpu_prefill(pre_check, seconds=args.cpu_seconds, thread_counts=host["thread_counts"])
            out["prefill"]["parity"] = (f"logits of positions 0..{PREFILL_CHECK - 1} bit-identical to the oracle"
                                        + (f"; of {len(PREFILL_CHECK_POS)} positions, one per eight-token block "
                                           f"(0, 9, 18, ..., {PREFILL_CHECK_POS[-1]}), bit-identical to the "
                                           "reference's own chunked forward over the same tokens"
                                           if pre["strided"] else ""))
            out["prefill"]["cpu_baseline"] = pre["cpu"]
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
