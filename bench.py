"""Benchmark of the hip backend's quantized MUL_MAT path on one MI355X.

Workload (the config the metric is quoted on): a synthetic Qwen3-8B
Q4_K_M decode token -- 36 layers x 7 matvecs at bs=1: Q, O 4096x4096 Q4_K; K, V 1024x4096 Q4_K;
gate, up 12288x4096 Q4_K; down 4096x12288 Q6_K. Weights ~ N(0, 0.02) generated and quantized on the
device (bit-identical to the reference quantizer), stored R32 in 252 distinct buffers (4.37 GB, far
beyond the 256 MB MALL). A step = one token = the 252 matvecs, replayed from one plan.

Reported on one JSON line:
  value         weight GB/s of the whole token (all 252 kernels, wall clock over the timed steps)
  roofline      the token's largest product, gate+up (2 x 12288x4096 Q4_K as one MUL_MAT_MULTI):
                algorithmic weight bytes per launch / mean launch duration from HIP events on its
                stream (the 36 layers' gate+up launches as one HIP graph, replayed right after the
                timed region), vs 8 TB/s;
                `traffic` = HBM bytes per launch from the committed rocprofv3 PMC summary
  prefill       Q4_K M=512 (N=512 tokens) MFMA TFLOP/s on the two MLP shapes, vs 2.5 PFLOP/s dense f16/bf16
  cpu_baseline  the reference's CPU MUL_MAT (oracle/_ref; the oracle when absent), 1 thread, one gate matrix, N=1
  configs       BASELINE.json's other workloads, one line each at their own shapes (Q4_0 4096x4096;
                Q8_0 Llama-7B MLP at N=1,4,8; Q4_K prefill at N=64..2048; the Q6_K LM head at
                N=1,8,64; the 70B-class Q4_K MLP), decode weights cycled over distinct copies that
                exceed the MALL, each with the reference CPU MUL_MAT (1 thread) timed beside it
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import scrapgpulibrary_amd as sg  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the dominant kernel, measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# profiling runs (their commands are recorded in the file itself)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_matvec_decode_token.json")
F16_PEAK_TFLOPS = 2500.0

HIDDEN, KV, FFN, LAYERS = 4096, 1024, 12288, 36
LAYER_SHAPES = [  # (name, dtype, K, M)
    ("q", sg.Q4_K, HIDDEN, HIDDEN),
    ("k", sg.Q4_K, HIDDEN, KV),
    ("v", sg.Q4_K, HIDDEN, KV),
    ("o", sg.Q4_K, HIDDEN, HIDDEN),
    ("gate", sg.Q4_K, HIDDEN, FFN),
    ("up", sg.Q4_K, HIDDEN, FFN),
    ("down", sg.Q6_K, FFN, HIDDEN),
]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(dtype, K, M):
    return sg.row_bytes(dtype, K) * M


class Model:
    """36 layers of R32 weights plus the activation / output vectors, all resident in HBM."""

    def __init__(self, dev, st, layers, fuse=True):
        self.dev, self.st = dev, st
        self.bufs = []
        tmp = dev.alloc(4 * FFN * HIDDEN)
        self.weights = []  # per layer: list of (name, dtype, K, M, desc)
        t0 = time.time()
        for li in range(layers):
            row = []
            for si, (name, dt, K, M) in enumerate(LAYER_SHAPES):
                b = dev.alloc(weight_bytes(dt, K, M))
                self.bufs.append(b)
                f = sg.tdesc(sg.F32, (K, M), tmp)
                st.fill_normal(f, seed=1000 * li + si, mean=0.0, std=0.02)
                q = sg.tdesc(dt, (K, M), b, layout=sg.R32)
                st.quantize(f, q)
                row.append((name, dt, K, M, q))
            self.weights.append(row)
            if li == 0:
                log(f"layer 0 generated+quantized in {time.time() - t0:.2f}s")
        st.sync()
        log(f"{layers} layers ready in {time.time() - t0:.1f}s")
        self.tmp = tmp
        self.xh_buf = dev.alloc(4 * HIDDEN)
        self.xf_buf = dev.alloc(4 * FFN)
        self.xh = sg.tdesc(sg.F32, (HIDDEN, 1), self.xh_buf)
        self.xf = sg.tdesc(sg.F32, (FFN, 1), self.xf_buf)
        st.fill_normal(self.xh, seed=7)
        st.fill_normal(self.xf, seed=8)
        self.y_bufs = {n: dev.alloc(4 * M) for n, _, _, M in LAYER_SHAPES}
        self.keep = []
        self.by_group = {}  # "q+k+v", "o", "gate+up", "down" (or one name per weight) -> ops of all layers
        nodes = []
        for row in self.weights:
            by = {name: (q, sg.tdesc(sg.F32, (M, 1), self.y_bufs[name])) for name, dt, K, M, q in row}
            # the decode step of one layer as the reference's ggml adapter issues it: q/k/v and
            # gate/up each share x (MUL_MAT_MULTI), o and down are single MUL_MATs
            groups = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)] if fuse else [(n,) for n, *_ in LAYER_SHAPES]
            for g in groups:
                x = self.xf if g[0] == "down" else self.xh
                if len(g) == 1:
                    op, keep = sg.mul_mat_op(by[g[0]][0], x, by[g[0]][1])
                else:
                    op, keep = sg.multi_op([by[n][0] for n in g], x, [by[n][1] for n in g])
                self.keep.append((op, keep))
                self.by_group.setdefault("+".join(g), []).append(op)
                nodes.append(sg.PlanNode(C.sizeof(sg.PlanNode), op, 0))
        self.nodes = (sg.PlanNode * len(nodes))(*nodes)
        self.pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), self.nodes, len(nodes))
        plan = C.c_void_p()
        sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(self.pdesc), C.byref(plan)), "plan_build")
        self.plan = plan.value
        self.bytes_per_token = sum(weight_bytes(dt, K, M) for _, dt, K, M in LAYER_SHAPES) * layers

    def token(self):
        sg.check(sg.lib().scrapgpu_plan_execute(self.st.handle, self.plan), "plan_execute")


def hip_runtime():
    """The HIP runtime the library itself runs on (already loaded in this process), for events."""
    h = C.CDLL("libamdhip64.so.7")  # the soname libscrapgpu_hip.so links: the same loaded runtime
    for f in ("hipEventCreate", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime", "hipEventDestroy"):
        getattr(h, f).restype = C.c_int
    h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    h.hipEventSynchronize.argtypes = [C.c_void_p]
    h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    h.hipEventDestroy.argtypes = [C.c_void_p]
    return h


def hip_check(err, what):
    if err != 0:
        raise RuntimeError(f"{what}: hipError {err}")


def profile_group(model, group, replays):
    """Mean launch time of one product of the token: the 36 layers' instances recorded as one plan
    (a HIP graph) and replayed `replays` times between two HIP events on the model's stream."""
    ops = model.by_group[group]
    nodes = (sg.PlanNode * len(ops))(*[sg.PlanNode(C.sizeof(sg.PlanNode), op, 0) for op in ops])
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, len(ops))
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(model.dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    hip = hip_runtime()
    stream = C.c_void_p(sg.lib().scrapgpu_hip_stream_native(model.st.handle))
    ev = [C.c_void_p(), C.c_void_p()]
    try:
        for e in ev:
            hip_check(hip.hipEventCreate(C.byref(e)), "hipEventCreate")
        for _ in range(2):
            sg.check(sg.lib().scrapgpu_plan_execute(model.st.handle, plan), "plan_execute")
        model.st.sync()
        hip_check(hip.hipEventRecord(ev[0], stream), "hipEventRecord")
        for _ in range(replays):
            sg.check(sg.lib().scrapgpu_plan_execute(model.st.handle, plan), "plan_execute")
        hip_check(hip.hipEventRecord(ev[1], stream), "hipEventRecord")
        hip_check(hip.hipEventSynchronize(ev[1]), "hipEventSynchronize")
        ms = C.c_float()
        hip_check(hip.hipEventElapsedTime(C.byref(ms), ev[0], ev[1]), "hipEventElapsedTime")
        ms = ms.value / (replays * len(ops))
    finally:
        for e in ev:
            if e.value:
                hip.hipEventDestroy(e)
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    name = {"q+k+v": "matvec_multi_q4_k", "gate+up": "matvec_multi_q4_k", "down": "matvec_q6_k"}.get(group, "matvec_q4_k")
    weights = {"q+k+v": ("q", "k", "v"), "gate+up": ("gate", "up")}.get(group, (group,))
    by = sum(weight_bytes(dt, K, M) for n, dt, K, M in LAYER_SHAPES if n in weights)
    return name, ms, by


def bench_layer_prefill(dev, st, model, n_tokens, reps):
    """One Qwen3-8B Q4_K_M layer's products at prefill (layer 0's weights: q/k/v and gate/up as
    MUL_MAT_MULTI, o, down in Q6_K) over n_tokens tokens, recorded as one plan; TFLOP/s of the plan
    replay from HIP events. x: synthetic activations of the products' input widths."""
    by = {name: (dt, K, M, q) for name, dt, K, M, q in model.weights[0]}
    bufs = [dev.alloc(4 * HIDDEN * n_tokens), dev.alloc(4 * FFN * n_tokens)]
    xh = sg.tdesc(sg.F32, (HIDDEN, n_tokens), bufs[0])
    xf = sg.tdesc(sg.F32, (FFN, n_tokens), bufs[1])
    st.fill_normal(xh, seed=31)
    st.fill_normal(xf, seed=32)
    ys = {}
    for name, (_, _, M, _) in by.items():
        bufs.append(dev.alloc(4 * M * n_tokens))
        ys[name] = sg.tdesc(sg.F32, (M, n_tokens), bufs[-1])
    keep, nodes = [], []
    for group in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
        x = xf if group[0] == "down" else xh
        if len(group) == 1:
            op, k = sg.mul_mat_op(by[group[0]][3], x, ys[group[0]])
        else:
            op, k = sg.multi_op([by[n][3] for n in group], x, [ys[n] for n in group])
        keep.append((op, k))
        nodes.append(sg.PlanNode(C.sizeof(sg.PlanNode), op, 0))
    arr = (sg.PlanNode * len(nodes))(*nodes)
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), arr, len(nodes))
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    try:
        run = lambda: [sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute") for _ in range(reps)]
        run()
        ms = hip_events_ms(st, run, 3) / reps
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
        st.sync()
        for b in bufs:
            b.free()
    flops = 2.0 * n_tokens * sum(K * M for dt, K, M, _ in by.values())
    return {"workload": f"Qwen3-8B Q4_K_M layer products (q/k/v, o, gate/up Q4_K; down Q6_K) at {n_tokens} tokens, one plan",
            "ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}


def bench_prefill(dev, st, n_tokens, reps):
    """Q4_K prefill: W 12288x4096 and 4096x12288 with x [n_tokens, K]; TFLOP/s from HIP events."""
    L = sg.lib()
    out = {}
    for K, M in ((HIDDEN, FFN), (FFN, HIDDEN)):
        wb = dev.alloc(weight_bytes(sg.Q4_K, K, M))
        f = sg.tdesc(sg.F32, (K, M), dev.alloc(4 * K * M))
        st.fill_normal(f, seed=K + M, std=0.02)
        w = sg.tdesc(sg.Q4_K, (K, M), wb, layout=sg.R32)
        st.quantize(f, w)
        xb = dev.alloc(4 * K * n_tokens)
        x = sg.tdesc(sg.F32, (K, n_tokens), xb)
        st.fill_normal(x, seed=3)
        yb = dev.alloc(4 * M * n_tokens)
        y = sg.tdesc(sg.F32, (M, n_tokens), yb)
        op, keep = sg.mul_mat_op(w, x, y)
        for _ in range(3):
            st.execute(op)
        st.sync()
        L.scrapgpu_hip_profile_reset()
        L.scrapgpu_hip_profile_enable(1)
        for _ in range(reps):
            st.execute(op)
        st.sync()
        L.scrapgpu_hip_profile_enable(0)
        rows = sg.profile_table()
        L.scrapgpu_hip_profile_reset()
        r = [r for r in rows if r["name"].startswith("matmul")][0]
        ms = r["ms"] / r["launches"]
        out[f"{M}x{K}"] = {"kernel": r["name"], "ms": round(ms, 4), "tflops": round(2.0 * M * K * n_tokens / (ms * 1e-3) / 1e12, 1)}
        for b in (wb, xb, yb):
            b.free()
    return out


MOE_E, MOE_USED, MOE_HIDDEN, MOE_FFN, MOE_LAYERS = 128, 8, 2048, 768, 48


def hip_events_ms(st, fn, reps):
    """Mean time of fn() (enqueued work on the model's stream) between two HIP events, over reps."""
    hip = hip_runtime()
    stream = C.c_void_p(sg.lib().scrapgpu_hip_stream_native(st.handle))
    ev = [C.c_void_p(), C.c_void_p()]
    total = 0.0
    try:
        for e in ev:
            hip_check(hip.hipEventCreate(C.byref(e)), "hipEventCreate")
        for _ in range(reps):
            st.sync()
            hip_check(hip.hipEventRecord(ev[0], stream), "hipEventRecord")
            fn()
            hip_check(hip.hipEventRecord(ev[1], stream), "hipEventRecord")
            hip_check(hip.hipEventSynchronize(ev[1]), "hipEventSynchronize")
            ms = C.c_float()
            hip_check(hip.hipEventElapsedTime(C.byref(ms), ev[0], ev[1]), "hipEventElapsedTime")
            total += ms.value
    finally:
        for e in ev:
            if e.value:
                hip.hipEventDestroy(e)
    return total / reps


def bench_moe(dev, st, tokens):
    """MUL_MAT_ID: a Qwen3-30B-A3B-shaped MoE decode token, bs = 1: per layer the gate and up experts
    (Q4_K, 2048 -> 768) and the down experts (Q6_K, 768 -> 2048) of 128, 8 selected, as three
    MUL_MAT_ID ops sharing the layer's ids; MOE_LAYERS layers, the model's 48 (18.8 GB of experts,
    far past the 256 MB MALL; one plan replay per token, so its fixed launch cost is spread over the
    token's 96 launches as in the model); fresh random ids every token (read on the device by the
    recorded plan)."""
    rng = np.random.default_rng(17)
    bufs = []
    tmp = dev.alloc(4 * MOE_HIDDEN * MOE_FFN * MOE_E)
    bufs.append(tmp)
    shapes = (("gate", sg.Q4_K, MOE_HIDDEN, MOE_FFN), ("up", sg.Q4_K, MOE_HIDDEN, MOE_FFN), ("down", sg.Q6_K, MOE_FFN, MOE_HIDDEN))
    xh = sg.tdesc(sg.F32, (MOE_HIDDEN, 1, 1), dev.alloc(4 * MOE_HIDDEN))
    st.fill_normal(xh, seed=21)
    xf = sg.tdesc(sg.F32, (MOE_FFN, MOE_USED, 1), dev.alloc(4 * MOE_FFN * MOE_USED))
    st.fill_normal(xf, seed=22)
    ids_buf = dev.alloc(4 * MOE_USED * MOE_LAYERS)
    bufs += [ids_buf]
    keep, nodes = [], []
    for li in range(MOE_LAYERS):
        ids = sg.tdesc(sg.I32, (MOE_USED, 1), ids_buf, offset=4 * MOE_USED * li)
        for name, dt, K, M in shapes:
            b = dev.alloc(weight_bytes(dt, K, M) * MOE_E)
            bufs.append(b)
            f = sg.tdesc(sg.F32, (K, M * MOE_E), tmp)
            st.fill_normal(f, seed=100 * li + len(nodes), mean=0.0, std=0.02)
            st.quantize(f, sg.tdesc(dt, (K, M * MOE_E), b, layout=sg.R32))
            w = sg.tdesc(dt, (K, M, MOE_E), b, layout=sg.R32)
            y = sg.tdesc(sg.F32, (M, MOE_USED, 1), dev.alloc(4 * M * MOE_USED))
            op, k = sg.mul_mat_id_op(w, xf if name == "down" else xh, ids, y, MOE_USED)
            keep.append((op, k))
            nodes.append(sg.PlanNode(C.sizeof(sg.PlanNode), op, 0))
    st.sync()
    arr = (sg.PlanNode * len(nodes))(*nodes)
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), arr, len(nodes))
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    ids_all = sg.tdesc(sg.I32, (MOE_USED * MOE_LAYERS,), ids_buf)

    def token():
        sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute")

    try:
        times = []
        for t in range(tokens + 3):
            sel = np.concatenate([rng.permutation(MOE_E)[:MOE_USED] for _ in range(MOE_LAYERS)]).astype(np.int32)
            st.upload(ids_all, sel)
            ms = hip_events_ms(st, token, 1)
            if t >= 3:
                times.append(ms)
        # launches per token: one eager replay under the event profiler (the plan launches a
        # layer's gate and up, which share x and ids, as one kernel)
        st.sync()
        sg.lib().scrapgpu_hip_profile_reset()
        sg.lib().scrapgpu_hip_profile_enable(1)
        try:
            token()
            st.sync()
        finally:
            sg.lib().scrapgpu_hip_profile_enable(0)
        launches = sum(r["launches"] for r in sg.profile_table())
        sg.lib().scrapgpu_hip_profile_reset()
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    ms = float(np.mean(times))
    by = MOE_LAYERS * MOE_USED * sum(weight_bytes(dt, K, M) for _, dt, K, M in shapes)
    return {"workload": f"Qwen3-30B-A3B MoE experts: {MOE_LAYERS} layers x (gate, up Q4_K {MOE_HIDDEN}->{MOE_FFN}; down Q6_K "
                        f"{MOE_FFN}->{MOE_HIDDEN}) x {MOE_E} experts, {MOE_USED} used, bs=1, MUL_MAT_ID with device ids",
            "ms_per_token": round(ms, 4), "selected_weight_bytes_per_token": by, "GBps": round(by / (ms * 1e-3) / 1e9, 1),
            "ops_per_token": len(nodes), "launches_per_token": launches}


def bench_moe_prefill(dev, st, n_tokens, reps):
    """MUL_MAT_ID at prefill size: the Qwen3-30B-A3B gate experts (Q4_K 2048->768, 128 experts,
    8 used) over n_tokens tokens with random distinct ids per token (the grouped MFMA path)."""
    K, M, E, U = MOE_HIDDEN, MOE_FFN, MOE_E, MOE_USED
    wb = dev.alloc(weight_bytes(sg.Q4_K, K, M) * E)
    tmp = dev.alloc(4 * K * M)
    for e in range(E):
        f = sg.tdesc(sg.F32, (K, M), tmp)
        st.fill_normal(f, seed=5000 + e, std=0.02)
        st.quantize(f, sg.tdesc(sg.Q4_K, (K, M), wb, layout=sg.R32, offset=weight_bytes(sg.Q4_K, K, M) * e))
    w = sg.tdesc(sg.Q4_K, (K, M, E), wb, layout=sg.R32)
    xb = dev.alloc(4 * K * n_tokens)
    x = sg.tdesc(sg.F32, (K, 1, n_tokens), xb)
    st.fill_normal(x, seed=6)
    rng = np.random.default_rng(7)
    ids = np.stack([rng.permutation(E)[:U] for _ in range(n_tokens)]).astype(np.int32)
    ib = dev.alloc(ids.nbytes)
    it = sg.tdesc(sg.I32, (U, n_tokens), ib)
    st.upload(it, ids)
    yb = dev.alloc(4 * M * U * n_tokens)
    y = sg.tdesc(sg.F32, (M, U, n_tokens), yb)
    op, keep = sg.mul_mat_id_op(w, x, it, y, U)
    st.execute(op)
    st.sync()
    ms = hip_events_ms(st, lambda: [st.execute(op) for _ in range(reps)], 3) / reps
    for b in (wb, tmp, xb, ib, yb):
        b.free()
    flops = 2.0 * M * K * U * n_tokens
    used = len(np.unique(ids))
    return {"workload": f"Qwen3-30B-A3B gate experts (Q4_K {K}->{M}) x {E}, {U} used, {n_tokens} tokens, MUL_MAT_ID (device-grouped MFMA)",
            "us": round(ms * 1e3, 2), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "experts_read": used, "weight_GBps": round(used * weight_bytes(sg.Q4_K, K, M) / (ms * 1e-3) / 1e9, 1)}


def bench_moe_prefill_layer(dev, st, n_tokens, reps, order=("gate", "up", "down")):
    """MUL_MAT_ID at prefill size over a whole MoE layer's experts: a plan of the Qwen3-30B-A3B
    gate and up (Q4_K 2048->768, the same x and ids: one x pre-pass and routing for both) and down
    (Q6_K 768->2048, x per slot) of 128 experts, 8 used, over n_tokens tokens with random distinct
    ids per token; time per replay of the plan (a HIP graph)."""
    E, U = MOE_E, MOE_USED
    specs = {"gate": (sg.Q4_K, MOE_HIDDEN, MOE_FFN), "up": (sg.Q4_K, MOE_HIDDEN, MOE_FFN), "down": (sg.Q6_K, MOE_FFN, MOE_HIDDEN)}
    bufs, keep, nodes = [], [], []
    tmp = dev.alloc(4 * MOE_HIDDEN * MOE_FFN * E)
    bufs.append(tmp)
    bufs += [dev.alloc(4 * MOE_HIDDEN * n_tokens), dev.alloc(4 * MOE_FFN * U * n_tokens)]
    xh = sg.tdesc(sg.F32, (MOE_HIDDEN, 1, n_tokens), bufs[-2])
    xf = sg.tdesc(sg.F32, (MOE_FFN, U, n_tokens), bufs[-1])
    st.fill_normal(xh, seed=41)
    st.fill_normal(xf, seed=42)
    rng = np.random.default_rng(43)
    ids = np.stack([rng.permutation(E)[:U] for _ in range(n_tokens)]).astype(np.int32)
    bufs.append(dev.alloc(ids.nbytes))
    it = sg.tdesc(sg.I32, (U, n_tokens), bufs[-1])
    st.upload(it, ids)
    flops = 0.0
    for i, name in enumerate(order):
        dt, K, M = specs[name]
        b = dev.alloc(weight_bytes(dt, K, M) * E)
        bufs.append(b)
        f = sg.tdesc(sg.F32, (K, M * E), tmp)
        st.fill_normal(f, seed=300 + i, std=0.02)
        st.quantize(f, sg.tdesc(dt, (K, M * E), b, layout=sg.R32))
        bufs.append(dev.alloc(4 * M * U * n_tokens))
        y = sg.tdesc(sg.F32, (M, U, n_tokens), bufs[-1])
        op, k = sg.mul_mat_id_op(sg.tdesc(dt, (K, M, E), b, layout=sg.R32), xf if name == "down" else xh, it, y, U)
        keep.append((op, k))
        nodes.append(sg.PlanNode(C.sizeof(sg.PlanNode), op, 0))
        flops += 2.0 * M * K * U * n_tokens
    arr = (sg.PlanNode * len(nodes))(*nodes)
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), arr, len(nodes))
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")

    def layer():
        sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute")

    try:
        layer()
        st.sync()
        ms = hip_events_ms(st, lambda: [layer() for _ in range(reps)], 3) / reps
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
        st.sync()
        for b in bufs:
            b.free()
    return {"workload": f"Qwen3-30B-A3B MoE layer experts (gate, up Q4_K {MOE_HIDDEN}->{MOE_FFN}; down Q6_K {MOE_FFN}->{MOE_HIDDEN}) x {E}, "
                        f"{U} used, {n_tokens} tokens, MUL_MAT_ID plan (device-grouped MFMA)",
            "us": round(ms * 1e3, 2), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}


def bench_get_rows(dev, st, n_rows, reps):
    """GET_ROWS: n_rows random rows of a Q6_K 151936 x 4096 table (the Qwen3 LM head / embedding
    shape, 510 MB, R32) dequantized to f32."""
    K, R = HIDDEN, 151936
    tmp = dev.alloc(4 * K * R)
    st.fill_normal(sg.tdesc(sg.F32, (K, R), tmp), seed=31, std=0.02)
    wb = dev.alloc(weight_bytes(sg.Q6_K, K, R))
    w = sg.tdesc(sg.Q6_K, (K, R), wb, layout=sg.R32)
    st.quantize(sg.tdesc(sg.F32, (K, R), tmp), w)
    tmp.free()
    rng = np.random.default_rng(33)
    ib = dev.alloc(4 * n_rows)
    ids = sg.tdesc(sg.I32, (n_rows, 1, 1), ib)
    st.upload(ids, rng.integers(0, R, n_rows).astype(np.int32))
    yb = dev.alloc(4 * K * n_rows)
    y = sg.tdesc(sg.F32, (K, n_rows, 1, 1), yb)
    op, keep = sg.get_rows_op(w, ids, y)
    for _ in range(3):
        st.execute(op)
    ms = hip_events_ms(st, lambda: [st.execute(op) for _ in range(10)], reps) / 10
    rb = weight_bytes(sg.Q6_K, K, 1) * n_rows
    for b in (wb, ib, yb):
        b.free()
    return {"workload": f"{n_rows} rows of a Q6_K {R}x{K} R32 table -> f32", "us": round(ms * 1e3, 2),
            "rows_read_bytes": rb, "f32_written_bytes": 4 * K * n_rows, "GBps_read_plus_write": round((rb + 4 * K * n_rows) / (ms * 1e-3) / 1e9, 1)}


def cpu_baseline(dev, st, model, seconds):
    """The reference's own CPU MUL_MAT (oracle/_ref, compiled from the reference sources; its CPU
    backend runs one thread) on one gate matrix at N=1; the oracle's C restatement of it when
    that library was not built."""
    import oracle as O

    name, dt, K, M, q = model.weights[0][4]
    nat = st.download(q, np.uint8)
    x = st.download(model.xh)[:K].reshape(1, K).copy()
    use_ref = O.ref_available()
    run = (lambda: O.ref_mul_mat(dt, nat, K, M, x)) if use_ref else (lambda: O.mul_mat(dt, nat, K, M, x))
    run()  # warm-up
    times = []
    t_end = time.time() + seconds
    while time.time() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    what = "reference CPU backend (oracle/_ref)" if use_ref else "oracle (C restatement)"
    return {"value": round(weight_bytes(dt, K, M) / med / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "reference" if use_ref else "port",
            "sample": f"{what} MUL_MAT Q4_K {M}x{K} N=1 (one layer's gate), median of {len(times)} runs of {med * 1e3:.1f} ms; "
                      f"host {cpu}, nproc {os.cpu_count()}"}


# ---- BASELINE.json's other workloads, one line each ---------------------------------------------

MALL_BYTES = 256 << 20


def device_weights(dev, st, dtype, K, M, copies, seed):
    """`copies` distinct R32 weights M x K ~ N(0, 0.02), quantized on the device (the reference
    quantizer's bytes); copies > 1 so that a timing loop over them streams from HBM, not the MALL."""
    tmp = dev.alloc(4 * K * M)
    out = []
    for c in range(copies):
        b = dev.alloc(weight_bytes(dtype, K, M))
        st.fill_normal(sg.tdesc(sg.F32, (K, M), tmp), seed=seed + c, mean=0.0, std=0.02)
        d = sg.tdesc(dtype, (K, M), b, layout=sg.R32)
        st.quantize(sg.tdesc(sg.F32, (K, M), tmp), d)
        out.append((b, d))
    st.sync()
    tmp.free()
    return out


def copies_for(nbytes):
    """Distinct copies whose total exceeds the 256 MB MALL 1.5 times over (at least one)."""
    return max(1, -(-int(1.5 * MALL_BYTES) // nbytes))


def time_plan(dev, st, ops, replays):
    """Mean ms per op of `ops` recorded as one plan (a HIP graph) and replayed between HIP events.
    The plan holds the ops in order, repeated until it has 16 nodes or more (each node a full
    execution of its op), so that one graph launch's fixed cost is spread over many ops as in the
    decode token's 144-node plan; the replays shrink by the same factor."""
    rep = max(1, -(-16 // len(ops)))
    ops = list(ops) * rep
    replays = max(2, -(-replays // rep))
    nodes = (sg.PlanNode * len(ops))(*[sg.PlanNode(C.sizeof(sg.PlanNode), op, 0) for op in ops])
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, len(ops))
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    try:
        run = lambda: [sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute") for _ in range(replays)]
        run()
        ms = hip_events_ms(st, run, 3) / (replays * len(ops))
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    return ms


def cpu_ms(dtype, nat, K, M, x, budget_s):
    """Median ms of the reference's CPU MUL_MAT (oracle/_ref; the oracle's C restatement when that
    library is absent), one thread, over as many calls as fit `budget_s` (at least one)."""
    import oracle as O

    run = (lambda: O.ref_mul_mat(dtype, nat, K, M, x)) if O.ref_available() else (lambda: O.mul_mat(dtype, nat, K, M, x))
    times = []
    t_end = time.time() + budget_s
    while not times or (time.time() < t_end and len(times) < 7):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e3, len(times)


def decode_line(dev, st, dtype, K, M, N, copies, seed, cpu_budget):
    """GB/s of weights for W x at N columns (weights streamed from HBM: distinct copies cycled),
    with the CPU reference beside it."""
    ws = device_weights(dev, st, dtype, K, M, copies, seed)
    xb, yb = dev.alloc(4 * K * N), dev.alloc(4 * M * N)
    xt, yt = sg.tdesc(sg.F32, (K, N), xb), sg.tdesc(sg.F32, (M, N), yb)
    st.fill_normal(xt, seed=seed + 99)
    keep = [sg.mul_mat_op(d, xt, yt) for _, d in ws]
    st.execute(keep[0][0])
    st.sync()
    form = sg.last_launch()[0]
    ms = time_plan(dev, st, [op for op, _ in keep], max(3, 40 // len(keep)))
    by = weight_bytes(dtype, K, M)
    out = {"kernel": form, "us": round(ms * 1e3, 2), "GBps": round(by / (ms * 1e-3) / 1e9, 1),
           "hbm_frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "GFLOPs": round(2.0 * M * K * N / (ms * 1e-3) / 1e9, 1)}
    if cpu_budget > 0:
        nat = st.download(ws[0][1], np.uint8)
        x = st.download(xt).reshape(N, K).copy()
        cms, n = cpu_ms(dtype, nat, K, M, x, cpu_budget)
        out["cpu"] = {"ms": round(cms, 2), "GBps": round(by / (cms * 1e-3) / 1e9, 3), "GFLOPs": round(2.0 * M * K * N / (cms * 1e-3) / 1e9, 2),
                      "runs": n}
    for b, _ in ws:
        b.free()
    xb.free()
    yb.free()
    return out


def prefill_line(dev, st, dtype, K, M, N, seed, cpu_budget):
    """TFLOP/s of W x at N tokens on the MFMA path, with the CPU reference beside it."""
    ws = device_weights(dev, st, dtype, K, M, 2, seed)
    xb, yb = dev.alloc(4 * K * N), dev.alloc(4 * M * N)
    xt, yt = sg.tdesc(sg.F32, (K, N), xb), sg.tdesc(sg.F32, (M, N), yb)
    st.fill_normal(xt, seed=seed + 99)
    keep = [sg.mul_mat_op(d, xt, yt) for _, d in ws]
    st.execute(keep[0][0])
    st.sync()
    form = sg.last_launch()[0]
    ms = time_plan(dev, st, [op for op, _ in keep], 10)
    fl = 2.0 * M * K * N
    out = {"kernel": form, "us": round(ms * 1e3, 2), "TFLOPs": round(fl / (ms * 1e-3) / 1e12, 1),
           "mfma_frac": round(fl / (ms * 1e-3) / 1e12 / F16_PEAK_TFLOPS, 4)}
    if cpu_budget > 0:
        nat = st.download(ws[0][1], np.uint8)
        x = st.download(xt).reshape(N, K).copy()
        cms, n = cpu_ms(dtype, nat, K, M, x, cpu_budget)
        out["cpu"] = {"ms": round(cms, 1), "GFLOPs": round(fl / (cms * 1e-3) / 1e9, 2), "runs": n}
    for b, _ in ws:
        b.free()
    xb.free()
    yb.free()
    return out


def bench_configs(dev, st, cpu_budget):
    """BASELINE.json configs[0], [1], [3], [4] (configs[2] is the main line)."""
    res = {}
    by = weight_bytes(sg.Q4_0, 4096, 4096)
    res["1_q4_0_4096x4096"] = {"N1": decode_line(dev, st, sg.Q4_0, 4096, 4096, 1, copies_for(by), 100, cpu_budget)}
    log("config 1 done")
    c2 = {}
    for K, M in ((4096, 11008), (11008, 4096)):
        by = weight_bytes(sg.Q8_0, K, M)
        c2[f"{M}x{K}"] = {f"N{N}": decode_line(dev, st, sg.Q8_0, K, M, N, copies_for(by), 200 + N, cpu_budget) for N in (1, 4, 8)}
    res["2_q8_0_llama7b_mlp"] = c2
    log("config 2 done")
    c4 = {}
    for K, M in ((4096, 12288), (12288, 4096)):
        c4[f"{M}x{K}"] = {f"N{N}": prefill_line(dev, st, sg.Q4_K, K, M, N, 300 + N, cpu_budget) for N in (64, 128, 512, 2048)}
    res["4_q4_k_prefill"] = c4
    log("config 4 done")
    by = weight_bytes(sg.Q6_K, 4096, 151936)
    res["5_q6_k_lm_head_151936x4096"] = {f"N{N}": (decode_line(dev, st, sg.Q6_K, 4096, 151936, N, 1, 400 + N, cpu_budget) if N <= 8
                                                   else prefill_line(dev, st, sg.Q6_K, 4096, 151936, N, 400 + N, cpu_budget)) for N in (1, 8, 64)}
    by = weight_bytes(sg.Q4_K, 8192, 28672)
    res["5_q4_k_70b_mlp_28672x8192"] = {"N1": decode_line(dev, st, sg.Q4_K, 8192, 28672, 1, copies_for(by), 500, cpu_budget)}
    log("config 5 done")
    return res


def traffic_of(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary, or None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            t = json.load(fh)
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(kernel)
    return None if k is None else k.get("hbm_bytes_per_launch")


def bench_float(dev, st):
    """Float weights (natural layout, no quantization): an F16 12288x4096 decode product at one
    column (GB/s, 4 weight copies cycled so that they stream from HBM) and F16 / BF16 prefill at 512
    tokens (TFLOP/s)."""
    K, M = 4096, 12288
    w = (np.random.default_rng(9000).standard_normal(M * K, dtype=np.float32) * 0.02).reshape(M, K)
    out = {}
    for name, dt, bits in (("f16", sg.F16, w.astype(np.float16).view(np.uint16)),
                           ("bf16", sg.BF16, (w.view(np.uint32) >> 16).astype(np.uint16))):
        copies = 4 if name == "f16" else 1
        bufs = []
        for _ in range(copies):
            b = dev.alloc(bits.nbytes)
            st.write(b, 0, bits.view(np.uint8).reshape(-1))
            bufs.append(b)
        for N in ((1, 512) if name == "f16" else (512,)):
            xb, yb = dev.alloc(4 * K * N), dev.alloc(4 * M * N)
            xt, yt = sg.tdesc(sg.F32, (K, N), xb), sg.tdesc(sg.F32, (M, N), yb)
            st.fill_normal(xt, seed=9001)
            keep = [sg.mul_mat_op(sg.tdesc(dt, (K, M), b), xt, yt) for b in bufs]
            st.execute(keep[0][0])
            st.sync()
            form = sg.last_launch()[0]
            ms = time_plan(dev, st, [op for op, _ in keep], 10)
            line = {"kernel": form, "us": round(ms * 1e3, 2)}
            if N == 1:
                line["GBps"] = round(bits.nbytes / (ms * 1e-3) / 1e9, 1)
                line["hbm_frac"] = round(bits.nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            else:
                tf = 2.0 * M * K * N / (ms * 1e-3) / 1e12
                line["TFLOPs"] = round(tf, 1)
                line["mfma_frac"] = round(tf / F16_PEAK_TFLOPS, 4)
            out[f"{name}_{M}x{K}_N{N}"] = line
            xb.free()
            yb.free()
        for b in bufs:
            b.free()
    log("float weights done")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-moe", action="store_true", help="skip the MUL_MAT_ID (MoE decode and prefill) lines")
    ap.add_argument("--no-get-rows", action="store_true", help="skip the GET_ROWS line")
    ap.add_argument("--no-configs", action="store_true", help="skip the lines of BASELINE.json's other workloads")
    ap.add_argument("--no-float", action="store_true", help="skip the float-weight (F16 / BF16) lines")
    ap.add_argument("--config-cpu-seconds", type=float, default=2.0, help="CPU reference budget per config line (at least one call)")
    ap.add_argument("--no-fuse", action="store_true", help="one MUL_MAT per weight instead of MUL_MAT_MULTI for q/k/v and gate/up")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one MI355X per run); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    dev = sg.Device(0)
    st = dev.stream()
    info = dev.info()
    log("device:", info.name.decode(), info.compute_units, "CUs")
    model = Model(dev, st, args.layers, fuse=not args.no_fuse)
    for _ in range(args.warmup):
        model.token()
    st.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.token()
    st.sync()
    dt = time.perf_counter() - t0
    ms_step = dt / args.steps * 1e3
    gbs = model.bytes_per_token * args.steps / dt / 1e9

    # the roofline kernel: the token's largest product (gate+up fused, 2 x 12288x4096 Q4_K)
    dom_group = "gate+up" if "gate+up" in model.by_group else "gate"
    groups = {}
    for g in model.by_group:
        g_name, g_ms, g_bytes = profile_group(model, g, 10)
        groups[g] = {"kernel": g_name, "mean_us": round(g_ms * 1e3, 3), "bytes": g_bytes, "GBps": round(g_bytes / (g_ms * 1e-3) / 1e9, 1)}
    dom_name, dom_bytes = groups[dom_group]["kernel"], groups[dom_group]["bytes"]
    dom_ms = groups[dom_group]["mean_us"] * 1e-3
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9

    prefill = None if args.no_prefill else bench_prefill(dev, st, 512, 10)
    layer_pf = None if args.no_prefill else bench_layer_prefill(dev, st, model, 512, 5)
    moe = None if args.no_moe else bench_moe(dev, st, 20)
    moe_pf = None if args.no_moe else bench_moe_prefill(dev, st, 512, 10)
    moe_pf_layer = None if args.no_moe else bench_moe_prefill_layer(dev, st, 512, 10)
    get_rows = None if args.no_get_rows else bench_get_rows(dev, st, 512, 5)
    cpu = None if args.no_cpu else cpu_baseline(dev, st, model, args.cpu_seconds)
    configs = None if args.no_configs else bench_configs(dev, st, 0.0 if args.no_cpu else args.config_cpu_seconds)
    float_w = None if args.no_float else bench_float(dev, st)

    result = {
        "metric": "Q4_K matvec weight GB/s (% HBM peak) at bs=1; prefill TFLOP/s at M=512",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "decode: q4_k/q6_k weight codes x int8 three-plane x (x = f*(253*a + b + c/253) per 32 elements, |err| <= 1.03*2^-24*max|x_seg|; non-finite segments in fp32) on i8 MFMA, int32 sums scaled and accumulated in f32; prefill: f16 MFMA, f32 accumulate",
        "data": "synthetic: weights ~N(0,0.02) quantized on device (bit-identical to the reference quantizer), x ~N(0,1)",
        "config": {"workload": f"Qwen3-8B Q4_K_M decode token: {args.layers} layers x 7 matvecs (q,k,v,o,gate,up in Q4_K; down in Q6_K), bs=1"
                               + ("; q/k/v and gate/up as MUL_MAT_MULTI" if not args.no_fuse else ""),
                   "weight_bytes_per_token": model.bytes_per_token, "parallelism": "single GPU"},
        "tokens_per_s_equiv": round(1e3 / ms_step, 1),
        "products": groups,
        "roofline": {"bound": "hbm", "kernel": f"{dom_name} ({dom_group})", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_of(dom_group),
                     "bytes_per_launch": dom_bytes, "mean_launch_us": round(dom_ms * 1e3, 3)},
        "prefill_M512": prefill,
        "prefill_layer_M512": layer_pf,
        "prefill_peak_frac": None if prefill is None else round(max(v["tflops"] for v in prefill.values()) / F16_PEAK_TFLOPS, 4),
        "moe_decode_mul_mat_id": moe,
        "moe_prefill_mul_mat_id": moe_pf,
        "moe_prefill_layer_mul_mat_id": moe_pf_layer,
        "get_rows": get_rows,
        "cpu_baseline": cpu,
        "configs": configs,
        "float_weights": float_w,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
