"""Benchmark: decode attention + KV append, µs per layer-step and achieved HBM
GB/s on one MI355X.

Workload: one full-depth batch-1 decode step = 48 layers in
gemma4 order (40 sliding layers with 1024-slot rings, page 1; 8 global layers,
page 64), 8 KV heads x 256, 16 query heads, bf16, context 8192 prefilled with
N(0,1) K/V. Each layer appends the current token (position 8192) and attends
over its live keys. The step runs as one persistent launch
(gemma4_decode_step_layers_bf16) that walks the 48 layers in order; layer i
reads its q/k/v only after layer i-1's output is complete. Every timed step
does the full work; the appended position is the same each step so the
per-step work is constant.

`value` = algorithmic HBM bytes of a step / step time, with all inputs
resident in HBM. Also reported: the per-layer-launch path (48 fused launches
replayed from a hipGraph), the per-launch split kernels, the batch-64
global-layer rate, the config-5 prefill chunk (TFLOP/s and
MFMA utilisation), the roofline of the dominant kernel measured live with HIP
events, and the CPU oracle baseline.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "gemma.c_amd"))
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
NUM_LAYERS = 48
HEADS, DIM, QH = 8, 256, 16
HIDDEN = 3840  # gemma4 hidden width (reference src/gemma4.h:6)
CONTEXT = 8192
WINDOW = 1024
GLOBAL_PAGE = 64
ROW_BYTES = HEADS * DIM * 2  # one token's K (or V) row, all KV heads


def is_global_layer(layer: int) -> bool:
    """gemma4 5:1 cadence with the last layer global (src/gemma4.h:105-108)."""
    return layer == NUM_LAYERS - 1 or (layer + 1) % 6 == 0


def layer_bytes(live_keys: int, batch: int = 1) -> int:
    """Algorithmic HBM bytes of one fused layer step: K+V of every live key
    (the new key included), the appended K/V row write, and q/out rows."""
    kv_read = live_keys * 2 * ROW_BYTES
    append = batch * 2 * ROW_BYTES
    q_out = batch * 2 * QH * DIM * 2
    return kv_read + append + q_out


class Layer:
    pass


def build_config2(torch, gk, dev, seed=0):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    seq_len = CONTEXT + 1
    sliding_pages = WINDOW  # page size 1 -> exactly 1024 ring slots
    global_pages = (seq_len + GLOBAL_PAGE - 1) // GLOBAL_PAGE
    n_sliding = sum(1 for l in range(NUM_LAYERS) if not is_global_layer(l))
    n_global = NUM_LAYERS - n_sliding
    s_cfg = gk.make_config(n_sliding, sliding_pages, 1, sliding_pages, 1, HEADS, DIM, WINDOW)
    g_cfg = gk.make_config(n_global, global_pages, GLOBAL_PAGE, global_pages, 1, HEADS, DIM, 0)

    def randn_bf16(shape):
        return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32).bfloat16().view(torch.int16)

    caches = {
        "sk": randn_bf16((n_sliding * sliding_pages, HEADS, DIM)),
        "sv": randn_bf16((n_sliding * sliding_pages, HEADS, DIM)),
        "gk": randn_bf16((n_global * global_pages * GLOBAL_PAGE, HEADS, DIM)),
        "gv": randn_bf16((n_global * global_pages * GLOBAL_PAGE, HEADS, DIM)),
    }
    i32 = dict(dtype=torch.int32, device=dev)
    meta = {
        "s_pt": torch.arange(sliding_pages, **i32),
        "g_pt": torch.arange(global_pages, **i32),
        "seq": torch.tensor([seq_len], **i32),
        "pos": torch.tensor([CONTEXT], **i32),
    }
    s_split, s_n = gk.decode_split_plan(s_cfg, 1, WINDOW)
    g_split, g_n = gk.decode_split_plan(g_cfg, 1, seq_len)
    max_n = max(s_n, g_n)
    scratch = {
        "pm": torch.empty(QH * max_n, device=dev),
        "pl": torch.empty(QH * max_n, device=dev),
        "pa": torch.empty(QH * max_n * DIM, device=dev),
        "cnt": torch.zeros(HEADS, **i32),
    }
    layers = []
    si = gi = 0
    for l in range(NUM_LAYERS):
        L = Layer()
        L.is_global = is_global_layer(l)
        if L.is_global:
            L.cfg, L.cache_layer, L.ck, L.cv, L.pt = g_cfg, gi, caches["gk"], caches["gv"], meta["g_pt"]
            L.split, L.n_splits, L.live = g_split, g_n, seq_len
            gi += 1
        else:
            L.cfg, L.cache_layer, L.ck, L.cv, L.pt = s_cfg, si, caches["sk"], caches["sv"], meta["s_pt"]
            L.split, L.n_splits, L.live = s_split, s_n, WINDOW
            si += 1
        L.q = randn_bf16((1, QH, DIM))
        L.k = randn_bf16((1, HEADS, DIM))
        L.v = randn_bf16((1, HEADS, DIM))
        L.out = torch.zeros((1, QH, DIM), dtype=torch.int16, device=dev)
        L.bytes = layer_bytes(L.live)
        layers.append(L)
    return layers, caches, meta, scratch


def launch_layer(gk, L, meta, scratch, stream):
    return gk.flash_attention_append_decode_paged_bf16(
        L.out, scratch["pm"], scratch["pl"], scratch["pa"], L.q, L.ck, L.cv, L.pt,
        meta["seq"], meta["pos"], L.k, L.v, L.cfg, L.cache_layer, 1.0 / math.sqrt(DIM),
        L.split, L.n_splits, 1, stream=stream, split_counters=None)


def launch_split_only(gk, L, meta, scratch, stream):
    """Phase 1 alone (fused append + split partials): the dominant kernel."""
    return gk.flash_attention_decode_split_paged_bf16(
        L.out, scratch["pm"], scratch["pl"], scratch["pa"], L.q, L.ck, L.cv, L.pt,
        meta["seq"], meta["pos"], L.k, L.v, L.cfg, L.cache_layer, 1.0 / math.sqrt(DIM),
        L.split, L.n_splits, 1, stream=stream)


def time_graph(torch, fn, reps, warmup):
    """Capture fn() once as a HIP graph; replay `reps` times between events."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(s.cuda_stream)  # warm the code objects outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn(torch.cuda.current_stream().cuda_stream)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps, g


def warm_clock(torch, fn, seconds=0.3):
    """Run fn(stream) back to back for `seconds`: a fresh process runs its
    first ~0.1 s of sustained work up to 15% slower (clock ramp)."""
    import time as _time
    st = torch.cuda.current_stream().cuda_stream
    t_end = _time.perf_counter() + seconds
    while _time.perf_counter() < t_end:
        for _ in range(10):
            fn(st)
        torch.cuda.synchronize()


def time_graph_calls(torch, fn, calls, reps=5, warmup=2):
    """Capture `calls` back-to-back invocations fn(stream, i) as one HIP graph
    and replay it; returns ms per invocation. For kernels of a few to tens of
    microseconds, whose eager launches would be paced by the host."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(s.cuda_stream, 0)  # warm the code objects outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = torch.cuda.current_stream().cuda_stream
        for i in range(calls):
            fn(st, i)
    import time as _time
    t_end = _time.perf_counter() + 0.2  # past the clock ramp of a fresh process
    n = 0
    while n < warmup or _time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
        n += 1
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / (reps * calls)


class StepRunner:
    """The whole config-2 step as one persistent launch."""

    def __init__(self, torch, gk, dev, layers, caches, meta):
        self.gk = gk
        self.q = torch.stack([L.q for L in layers])
        self.k = torch.stack([L.k for L in layers])
        self.v = torch.stack([L.v for L in layers])
        self.out = torch.zeros((NUM_LAYERS, 1, QH, DIM), dtype=torch.int16, device=dev)
        self.s_cfg = next(L.cfg for L in layers if not L.is_global)
        self.g_cfg = next(L.cfg for L in layers if L.is_global)
        self.caches, self.meta = caches, meta
        nbytes = gk.decode_step_workspace_bytes(1)
        self.ws = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
        gk.check(gk.decode_step_workspace_init(self.ws, 1), "decode_step_workspace_init")

    def __call__(self, stream):
        c, m = self.caches, self.meta
        self.gk.check(self.gk.decode_step_layers_bf16(
            self.out, self.q, self.k, self.v, c["sk"], c["sv"], m["s_pt"], self.s_cfg,
            c["gk"], c["gv"], m["g_pt"], self.g_cfg, m["seq"], m["pos"], 0, NUM_LAYERS,
            1.0 / math.sqrt(DIM), 1, self.ws, stream=stream), "decode_step_layers")

    def status(self):
        return self.gk.decode_step_status(self.ws)


def bench_step_ref_geometry(torch, gk, dev, layers, caches, meta, steps):
    """Config 2 with the reference model's global geometry (1 KV head x 512,
    src/gemma4.h:17-21) in place of 8 x 256: the same 40 sliding layers, 8
    global layers over 8193 keys at 1 x 512. The step entry point runs the
    sliding runs as persistent launches and each global layer as one fused
    append + split-K launch (16 launches per step)."""
    seq_len = CONTEXT + 1
    g_pages = (seq_len + GLOBAL_PAGE - 1) // GLOBAL_PAGE
    g_cfg = gk.make_config(8, g_pages, GLOBAL_PAGE, g_pages, 1, 1, 512, 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)

    def rnd(shape):
        return torch.randn(shape, generator=gen, device=dev).bfloat16().view(torch.int16)

    gk_c, gv_c = rnd((8 * g_pages * GLOBAL_PAGE, 1, 512)), rnd((8 * g_pages * GLOBAL_PAGE, 1, 512))
    qs, ks, vs, total = [], [], [], 0
    for l in range(NUM_LAYERS):
        h, d = (1, 512) if is_global_layer(l) else (HEADS, DIM)
        qs.append(rnd((QH * d,)))
        ks.append(rnd((h * d,)))
        vs.append(rnd((h * d,)))
        live = seq_len if is_global_layer(l) else WINDOW
        total += live * 2 * h * d * 2 + 2 * h * d * 2 + 2 * QH * d * 2
    q, k, v = torch.cat(qs), torch.cat(ks), torch.cat(vs)
    out = torch.zeros_like(q)
    s_cfg = next(L.cfg for L in layers if not L.is_global)
    ws = torch.empty(gk.decode_step_workspace_bytes(1) // 4, dtype=torch.int32, device=dev)
    gk.check(gk.decode_step_workspace_init(ws, 1), "workspace_init")

    def fn(st):
        gk.check(gk.decode_step_layers_bf16(
            out, q, k, v, caches["sk"], caches["sv"], meta["s_pt"], s_cfg, gk_c, gv_c,
            meta["g_pt"], g_cfg, meta["seq"], meta["pos"], 0, NUM_LAYERS, 1.0 / math.sqrt(DIM),
            1, ws, stream=st), "decode_step 1x512")

    warm_clock(torch, fn, 0.2)
    ms = time_eager(torch, fn, steps, 3)
    assert gk.decode_step_status(ws) == 0
    del gk_c, gv_c
    return {"workload": "config2 with 1x512 global layers (the reference model's geometry)",
            "ms_per_step": round(ms, 4), "us_per_layer_step": round(ms * 1e3 / NUM_LAYERS, 3),
            "achieved_GBs": round(total / (ms * 1e-3) / 1e9, 1), "bytes_per_step": total,
            "timing": "eager back-to-back steps: 8 persistent sliding runs + 8 fused "
                      "global launches per step"}


def bench_step_prep(torch, gk, runner, steps):
    """Config 2 from the layers' raw projections
    (gemma4_decode_step_layers_prep_bf16): the same persistent step with each
    layer's Q/K RMSNorm + RoPE and V RMSNorm done in-kernel after the previous
    layer completes, as the reference's fused decode layer does."""
    dev = runner.q.device
    gen = torch.Generator(device=dev)
    gen.manual_seed(12)
    w = (1.0 + 0.1 * torch.randn((2, NUM_LAYERS, DIM), generator=gen, device=dev)).bfloat16()
    w = w.view(torch.int16)
    npos = CONTEXT + 1
    ang = torch.rand((2, 2, npos, DIM // 2), generator=gen, device=dev) * 6.28
    cos, sin = torch.cos(ang), torch.sin(ang)
    c, m = runner.caches, runner.meta

    def fn(st):
        gk.check(gk.decode_step_layers_prep_bf16(
            runner.out, runner.q, runner.k, runner.v, c["sk"], c["sv"], m["s_pt"], runner.s_cfg,
            c["gk"], c["gv"], m["g_pt"], runner.g_cfg, m["seq"], m["pos"], w[0], w[1],
            cos[0, 0], sin[0, 0], cos[1, 0], sin[1, 0], 0, NUM_LAYERS, 1.0 / math.sqrt(DIM), 1,
            runner.ws, stream=st), "decode_step_layers_prep")

    warm_clock(torch, fn, 0.2)
    ms = time_eager(torch, fn, steps, 3)
    assert runner.status() == 0
    return {"workload": "config2 from raw projections (in-step Q/K norm+RoPE, V norm)",
            "ms_per_step": round(ms, 4), "us_per_layer_step": round(ms * 1e3 / NUM_LAYERS, 3),
            "timing": "eager back-to-back steps, one persistent launch each"}


def bench_prefill(torch, gk, dev, reps):
    """a 2048-row prefill chunk on one sliding layer (window
    1024, 1024-slot page-1 ring after a 1536-token prior) and one global layer
    (prior 6144, page 64); bf16 MFMA QK^T and PV. FLOPs = 4*D per (query row,
    query head, visible key)."""
    import numpy as np
    lq = 2048
    res = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    for kind, window, page, prior in (("sliding", WINDOW, 1, 1536), ("global", 0, GLOBAL_PAGE, 6144)):
        max_pages = WINDOW if window else (prior + lq) // page
        cfg = gk.make_config(1, max_pages, page, max_pages, 1, HEADS, DIM, window)
        rows = max_pages * page

        def rnd(shape):
            return torch.randn(shape, generator=gen, device=dev).bfloat16().view(torch.int16)

        ck, cv = rnd((rows, HEADS, DIM)), rnd((rows, HEADS, DIM))
        q, k, v = rnd((1, lq, QH, DIM)), rnd((1, lq, HEADS, DIM)), rnd((1, lq, HEADS, DIM))
        pt = torch.arange(max_pages, dtype=torch.int32, device=dev)
        out = torch.zeros((1, lq, QH, DIM), dtype=torch.int16, device=dev)
        pr = torch.tensor([prior], dtype=torch.int32, device=dev)

        args = [gk.ptr(t) for t in (out, q, k, v, ck, cv, pt, pr)] + [cfg, 0, 1, lq, 1 / 16]
        if window or os.environ.get("GEMMA_KV_PREFILL_PLAIN"):
            raw = gk.lib().gemma4_flash_attention_prefill_chunk_paged_bf16
        else:
            # The global chunk's causal work balanced over workgroups.
            nbytes = gk.flash_attention_prefill_chunk_workspace_bytes(1, lq, cfg)
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
            raw = gk.lib().gemma4_flash_attention_prefill_chunk_paged_bf16_ws
            args += [gk.ptr(ws), nbytes]

        def fn(st):
            code = raw(*args, st)
            if code:
                raise gk.HipError(code, "prefill")

        # Back-to-back eager launches through the raw C-ABI call, after a
        # time-based warm-up (50 short chunks are shorter than the clock ramp).
        warm_clock(torch, fn)
        ms = time_eager(torch, fn, max(reps, 50), 10)
        plain_ms = None
        if not window and raw is not gk.lib().gemma4_flash_attention_prefill_chunk_paged_bf16:
            # The same chunk through the entry point without a workspace.
            plain = gk.lib().gemma4_flash_attention_prefill_chunk_paged_bf16
            plain_args = args[:13]

            def fn_plain(st):
                code = plain(*plain_args, st)
                if code:
                    raise gk.HipError(code, "prefill")
            plain_ms = time_eager(torch, fn_plain, max(reps, 50), 10)
        keys = np.arange(lq) + prior + 1
        if window:
            keys = np.minimum(keys, window)
        flops = 4 * DIM * QH * int(keys.sum())
        tflops = flops / (ms * 1e-3) / 1e12
        res[kind] = {"us_per_chunk": round(ms * 1e3, 2), "gflop": round(flops / 1e9, 2),
                     "tflops": round(tflops, 1),
                     "mfma_util_vs_bf16_dense_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
        if plain_ms is not None:
            res[kind]["entry_point"] = "gemma4_flash_attention_prefill_chunk_paged_bf16_ws (balanced)"
            res[kind]["us_per_chunk_unbalanced"] = round(plain_ms * 1e3, 2)
    return res


def time_each(torch, fn, reps):
    """Median time of single launches, each bracketed by its own pair of HIP
    events on the launch stream (the kernel's own duration as the stream
    sees it, without the gap to the next launch)."""
    import statistics
    st = torch.cuda.current_stream()
    pairs = []
    for _ in range(reps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn(st.cuda_stream)
        b.record()
        pairs.append((a, b))
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in pairs)


def time_eager(torch, fn, reps, warmup):
    st = torch.cuda.current_stream().cuda_stream
    for _ in range(warmup):
        fn(st)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn(st)
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def read_traffic(kernel_tag: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = REPO / "profiles" / f"{kernel_tag}_pmc.md"
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text())
    return float(m.group(1)) if m else None


def bench_config1(torch, gk, dev, reps=3):
    """BASELINE config 1 on the GPU: one sliding layer, 1024-slot page-1 ring,
    2048 sequential steps from an empty cache, each one fused append + decode
    launch (the ring slot of position t is mapped from the start: the slots a
    step cannot see yet are never read, so the work equals the reference
    loop's). Step t's seq_len/position come from per-step device arrays. The
    2048 launches are captured once as a graph and replayed (every replay
    redoes the same 2048 appends and attentions)."""
    steps = 2048
    cfg = gk.make_config(1, WINDOW, 1, WINDOW, 1, HEADS, DIM, WINDOW)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)

    def rnd(shape):
        return torch.randn(shape, generator=gen, device=dev).bfloat16().view(torch.int16)

    q, k, v = rnd((steps, QH, DIM)), rnd((steps, HEADS, DIM)), rnd((steps, HEADS, DIM))
    ck = torch.zeros((WINDOW, HEADS, DIM), dtype=torch.int16, device=dev)
    cv = torch.zeros_like(ck)
    pt = torch.arange(WINDOW, dtype=torch.int32, device=dev)
    seq = torch.arange(1, steps + 1, dtype=torch.int32, device=dev)
    pos = torch.arange(steps, dtype=torch.int32, device=dev)
    out = torch.zeros((steps, QH, DIM), dtype=torch.int16, device=dev)
    split, n = gk.decode_split_plan(cfg, 1, WINDOW)
    pm = torch.empty(QH * n, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(QH * n * DIM, device=dev)
    qrow, kvrow = QH * DIM * 2, HEADS * DIM * 2
    lib = gk.lib()
    base = [gk.ptr(t) for t in (out, pm, pl, pa, q, ck, cv, pt, seq, pos, k, v)]

    def fn(st, i=0):
        for t in range(steps):
            code = lib.gemma4_flash_attention_append_decode_paged_bf16(
                base[0] + t * qrow, base[1], base[2], base[3], base[4] + t * qrow, base[5],
                base[6], base[7], base[8] + 4 * t, base[9] + 4 * t, base[10] + t * kvrow,
                base[11] + t * kvrow, 0, cfg, 0, 1.0 / 16, split, n, 1, st)
            if code:
                raise gk.HipError(code, f"config1 step {t}")

    ms = time_graph_calls(torch, fn, 1, reps=reps, warmup=1)
    total = sum(layer_bytes(min(t + 1, WINDOW)) for t in range(steps))

    # The same 2048 steps as one persistent walk (gemma4_decode_walk_bf16):
    # step t reads its q/k/v after step t-1's output is complete. The walk
    # advances the device length itself, so it is reset before each launch
    # (outside the events, which bracket the walk launch alone).
    ws = torch.empty(gk.decode_step_workspace_bytes(1) // 4, dtype=torch.int32, device=dev)
    gk.check(gk.decode_step_workspace_init(ws, 1), "decode_step_workspace_init")
    wseq = torch.zeros(1, dtype=torch.int32, device=dev)
    wpos = torch.zeros(1, dtype=torch.int32, device=dev)
    wout = torch.zeros_like(out)
    walk_ms = []
    for r in range(reps + 1):
        wseq.zero_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gk.check(gk.decode_walk_bf16(wout, q, k, v, ck, cv, pt, cfg, 0, wseq, wpos, steps,
                                     1.0 / 16, 1, ws), "decode_walk")
        e1.record()
        torch.cuda.synchronize()
        if r > 0:  # the first launch is a warm-up
            walk_ms.append(e0.elapsed_time(e1))
    assert gk.decode_step_status(ws) == 0
    assert int(wseq.item()) == steps
    wms = statistics.median(walk_ms)
    return {"workload": "config1: 1 sliding layer, ring 1024 page 1, 2048 sequential "
                        "append+attend steps from an empty cache",
            "us_per_layer_step": round(wms * 1e3 / steps, 3), "ms_2048_steps": round(wms, 3),
            "achieved_GBs": round(total / (wms * 1e-3) / 1e9, 1), "bytes_2048_steps": total,
            "timing": "one persistent walk launch (gemma4_decode_walk_bf16) between HIP events, "
                      f"median of {reps}",
            "per_step_launches": {
                "us_per_layer_step": round(ms * 1e3 / steps, 3), "ms_2048_steps": round(ms, 3),
                "achieved_GBs": round(total / (ms * 1e-3) / 1e9, 1),
                "split_size": split, "num_splits": n,
                "timing": "hipGraph of the 2048 fused append+decode launches, replayed"}}


def batch64_seq():
    import numpy as np
    rng = np.random.default_rng(64)
    seq = rng.integers(512, 32769, size=64).astype(np.int32)
    max_pages = (int(seq.max()) + GLOBAL_PAGE - 1) // GLOBAL_PAGE
    return seq, max_pages, 64 * max_pages * GLOBAL_PAGE


def alloc_kv(torch, dev, rows):
    """A K and a V cache of `rows` token rows (8 x 256 bf16). The full bench
    allocates the batch-64 and long-context caches at its start, as a
    serving runtime allocates its KV caches once at start-up: device memory
    allocated later, after other legs freed theirs, measured up to 6% slower
    to stream for the strided per-head reads of these legs."""
    ck = torch.empty((rows, HEADS, DIM), dtype=torch.bfloat16, device=dev)
    return ck, torch.empty_like(ck)


def bench_batch64(torch, gk, dev, steps, warmup, kv=None):
    """one global layer, 64 sequences, contexts U[512, 32768]."""
    seq, max_pages, rows = batch64_seq()
    page = GLOBAL_PAGE
    cfg = gk.make_config(1, 64 * max_pages, page, max_pages, 64, HEADS, DIM, 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    ck, cv = kv if kv is not None else alloc_kv(torch, dev, rows)
    assert ck.shape == (rows, HEADS, DIM)
    for t in (ck, cv):  # fill in slices to bound the fp32 temporary
        for r0 in range(0, rows, 1 << 20):
            t[r0:r0 + (1 << 20)] = torch.randn((min(1 << 20, rows - r0), HEADS, DIM),
                                               generator=gen, device=dev).bfloat16()
    ck, cv = ck.view(torch.int16), cv.view(torch.int16)
    pt = torch.arange(64 * max_pages, dtype=torch.int32, device=dev)
    seq_t = torch.from_numpy(seq).to(dev)
    pos_t = torch.from_numpy(seq - 1).to(dev)
    q = torch.randn((64, QH, DIM), generator=gen, device=dev).bfloat16().view(torch.int16)
    k = torch.randn((64, HEADS, DIM), generator=gen, device=dev).bfloat16().view(torch.int16)
    v = torch.randn((64, HEADS, DIM), generator=gen, device=dev).bfloat16().view(torch.int16)
    out = torch.zeros((64, QH, DIM), dtype=torch.int16, device=dev)
    split, n = gk.decode_split_plan(cfg, 64, int(seq.max()))
    pm = torch.empty(64 * QH * n, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(64 * QH * n * DIM, device=dev)

    def fn(st):  # fused append + split kernel, then the combine kernel
        gk.check(gk.flash_attention_append_decode_paged_bf16(
            out, pm, pl, pa, q, ck, cv, pt, seq_t, pos_t, k, v, cfg, 0, 1 / 16, split, n, 64,
            stream=st, split_counters=None), "batch64 decode")

    # Back-to-back eager launches (steady-state serving loop; the next step's
    # launch overlaps the current one). A graph replay per step measured
    # ~60 us slower per 1.4 ms step on this path.
    warm_clock(torch, fn)
    ms = time_eager(torch, fn, max(steps, 20), max(warmup, 10))
    total = sum(layer_bytes(int(s)) for s in seq)
    gbs = total / (ms * 1e-3) / 1e9
    del ck, cv
    return {"workload": "config3: 1 global layer, 64 seqs, ctx U[512,32768] seed 64",
            "us_per_layer_step": ms * 1e3, "achieved_GBs": gbs,
            "frac_of_peak": gbs / HBM_PEAK_GBS, "split_size": split, "num_splits": n,
            "bytes_per_step": total, "traffic": read_traffic("decode_batch64_config3")}


def bench_long(torch, gk, dev, steps, warmup, target_workgroups=0, counters=False, ctx=131072,
               kv=None):
    """one global layer, one sequence of 131072 keys (1 GiB
    of K/V), 1% of the keys scaled x8; fused append + split kernel, then the
    log-sum-exp combine (a second kernel, or in-kernel with counters)."""
    page = GLOBAL_PAGE
    max_pages = ctx // page
    cfg = gk.make_config(1, max_pages, page, max_pages, 1, HEADS, DIM, 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    ck, cv = kv if kv is not None else alloc_kv(torch, dev, ctx)
    assert ck.shape == (ctx, HEADS, DIM)
    for t in (ck, cv):
        for r0 in range(0, ctx, 1 << 15):
            n_rows = min(1 << 15, ctx - r0)
            t[r0:r0 + n_rows] = torch.randn((n_rows, HEADS, DIM), generator=gen,
                                            device=dev).bfloat16()
    hot = torch.randperm(ctx, generator=gen, device=dev)[:ctx // 100]
    ck[hot] *= 8
    ck, cv = ck.view(torch.int16), cv.view(torch.int16)
    pt = torch.arange(max_pages, dtype=torch.int32, device=dev)
    seq_t = torch.tensor([ctx], dtype=torch.int32, device=dev)
    pos_t = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    q = torch.randn((1, QH, DIM), generator=gen, device=dev).bfloat16().view(torch.int16)
    k = torch.randn((1, HEADS, DIM), generator=gen, device=dev).bfloat16().view(torch.int16)
    v = torch.randn((1, HEADS, DIM), generator=gen, device=dev).bfloat16().view(torch.int16)
    out = torch.zeros((1, QH, DIM), dtype=torch.int16, device=dev)
    split, n = gk.decode_split_plan(cfg, 1, ctx, target_workgroups)
    pm = torch.empty(QH * n, device=dev)
    pl = torch.empty_like(pm)
    pa = torch.empty(QH * n * DIM, device=dev)
    cnt = torch.zeros(HEADS, dtype=torch.int32, device=dev) if counters else None

    def fn(st):
        gk.check(gk.flash_attention_append_decode_paged_bf16(
            out, pm, pl, pa, q, ck, cv, pt, seq_t, pos_t, k, v, cfg, 0, 1 / 16, split, n, 1,
            stream=st, split_counters=cnt), "long-context decode")

    warm_clock(torch, fn)
    ms = time_eager(torch, fn, max(steps, 20), max(warmup, 10))
    total = layer_bytes(ctx)
    gbs = total / (ms * 1e-3) / 1e9
    del ck, cv
    return {"workload": "config4: 1 global layer, 1 seq, ctx 131072, 1% keys x8",
            "us_per_layer_step": ms * 1e3, "achieved_GBs": gbs,
            "frac_of_peak": gbs / HBM_PEAK_GBS, "split_size": split, "num_splits": n,
            "in_kernel_combine": counters, "bytes_per_step": total,
            "traffic": read_traffic("decode_long_context_config4")}


def bench_oproj(torch, gk, dev, rnd, rows_list=(1, 4, 8, 16, 64)):
    """Attention output projection + post-attention norm + residual, per call
    (projection + tail launches) from a graph of back-to-back calls. The
    weights rotate over copies that together exceed the 256 MiB MALL, so
    every call streams its weights from HBM."""
    oproj = {}
    for width in (4096, 8192):
        wbytes = HIDDEN * width * 2
        copies = max(2, -(-384 * 2**20 // wbytes))
        ws = [rnd((HIDDEN, width)) for _ in range(copies)]
        g = rnd((HIDDEN,))
        for rows in rows_list:
            attn, x = rnd((rows, width)), rnd((rows, HIDDEN))
            outs = [torch.empty((rows, HIDDEN), dtype=torch.int16, device=dev) for _ in range(3)]

            def fn(st, i):
                gk.check(gk.attention_o_projection_post_norm_bf16(
                    *outs, attn, ws[i % copies], g, x, rows, width, stream=st), "o projection")
            us = time_graph_calls(torch, fn, 4 * copies) * 1e3
            nbytes = wbytes + rows * (width + 4 * HIDDEN) * 2
            oproj[f"width{width}_rows{rows}"] = {"us": round(us, 2),
                                                 "GBs": round(nbytes / (us * 1e-6) / 1e9, 1)}
        del ws
    return oproj


def bench_widened(torch, gk, dev):
    """The rows around the hot path, each timed on its own: the decode-token
    prep + append (both geometries, batch 1 and 64), the prefill norm+RoPE
    launchers (prep + attention, 2048 rows), the attention output projection,
    a decode layer from raw projections (two launches vs the fused one), and
    the runtime's decode-step bookkeeping on the host vs on the device.
    Synthetic N(0,1) inputs."""
    import time as _time
    import numpy as np
    res = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)

    def rnd(shape):
        return torch.randn(shape, generator=gen, device=dev).bfloat16().view(torch.int16)

    # Decode prep + append: one token per sequence into a paged cache.
    prep = {}
    for name, heads, dim, rot, theta in (("sliding_8x256", 8, 256, 256, 10000.0),
                                         ("global_1x512", 1, 512, 128, 1_000_000.0)):
        for batch in (1, 64):
            page, max_pages = 16, 64
            cfg = gk.make_config(1, batch * max_pages, page, max_pages, batch, heads, dim,
                                 0 if heads == 1 else 1024)
            ck = torch.zeros((batch * max_pages * page, heads, dim), dtype=torch.int16, device=dev)
            cv = torch.zeros_like(ck)
            pt = torch.arange(batch * max_pages, dtype=torch.int32, device=dev)
            pos = torch.full((batch,), 100, dtype=torch.int32, device=dev)
            q, k, v = rnd((batch, QH, dim)), rnd((batch, heads, dim)), rnd((batch, heads, dim))
            qp = torch.empty_like(q)
            w = rnd((dim,))
            cos = torch.rand((1024, rot // 2), device=dev)
            sin = torch.rand((1024, rot // 2), device=dev)

            def fn(st, i):
                gk.check(gk.decode_prep_append_bf16(qp, ck, cv, cfg, pt, pos, 0, q, k,
                                                    v if heads > 1 else None, w, w, cos, sin,
                                                    batch, stream=st), "decode prep")
            us = time_graph_calls(torch, fn, 20) * 1e3
            nbytes = batch * (2 * QH * dim * 2 + 4 * heads * dim * 2)  # q in/out, k,v in, cache rows out
            prep[f"{name}_batch{batch}"] = {"us": round(us, 2),
                                            "GBs": round(nbytes / (us * 1e-6) / 1e9, 1)}
    res["decode_prep_append"] = prep

    # Prefill launchers: prep + causal attention over 2048 rows.
    lq = 2048
    launch = {}
    for name in ("sliding_8x256_window1024", "global_1x512"):
        heads, dim, rot = (8, 256, 256) if name.startswith("sliding") else (1, 512, 128)
        q, k, v = rnd((lq, QH, dim)), rnd((lq, heads, dim)), rnd((lq, heads, dim))
        qp, kp, vp, out = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(q)
        w = rnd((dim,))
        cos = torch.rand((lq, rot // 2), device=dev)
        sin = torch.rand((lq, rot // 2), device=dev)
        pos = torch.arange(lq, dtype=torch.int32, device=dev)
        scale = 1 / math.sqrt(dim)
        if heads == 8:
            def fn(st):
                gk.check(gk.flash_attention_sliding_fwd_bf16_norm_rope(
                    out, qp, kp, vp, q, k, v, w, w, cos, sin, pos, 1, lq, lq, 1024, scale,
                    stream=st), "sliding launcher")
            keys = np.minimum(np.arange(lq) + 1, 1024)
        else:
            def fn(st):
                gk.check(gk.flash_attention_global_fwd_bf16_norm_rope(
                    out, qp, kp, vp, q, k, w, w, cos, sin, pos, 1, lq, lq, scale, stream=st),
                    "global launcher")
            keys = np.arange(lq) + 1
        ms = time_graph_calls(torch, lambda st, i: fn(st), 10)
        flops = 4 * dim * QH * int(keys.sum())
        launch[name] = {"us": round(ms * 1e3, 1), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
    res["prefill_norm_rope_launchers"] = launch

    res["attention_o_projection"] = bench_oproj(torch, gk, dev, rnd)

    # Decode layer from raw projections, config-2 shapes at batch 1: the
    # token prep + append launch followed by the attention, against the
    # fused call that prepares inside the attention launch.
    fused = {}
    for name, page, max_pages, window in (("sliding_ring1024", 1, WINDOW, WINDOW),
                                          ("global_ctx8192", GLOBAL_PAGE,
                                           (CONTEXT + GLOBAL_PAGE) // GLOBAL_PAGE, 0)):
        cfg = gk.make_config(1, max_pages, page, max_pages, 1, HEADS, DIM, window)
        rows = max_pages * page
        ck, cv = rnd((rows, HEADS, DIM)), rnd((rows, HEADS, DIM))
        pt = torch.arange(max_pages, dtype=torch.int32, device=dev)
        seq_t = torch.tensor([CONTEXT + 1], dtype=torch.int32, device=dev)
        pos_t = torch.tensor([CONTEXT], dtype=torch.int32, device=dev)
        q, k, v = rnd((1, QH, DIM)), rnd((1, HEADS, DIM)), rnd((1, HEADS, DIM))
        qp, out = torch.empty_like(q), torch.empty_like(q)
        w = rnd((DIM,))
        cos = torch.rand((CONTEXT + 1, DIM // 2), device=dev)
        sin = torch.rand((CONTEXT + 1, DIM // 2), device=dev)
        split, n = gk.decode_split_plan(cfg, 1, window if window else CONTEXT + 1)
        pm = torch.empty(QH * n, device=dev)
        pl = torch.empty_like(pm)
        pa = torch.empty(QH * n * DIM, device=dev)

        def two(st, i=0):
            gk.check(gk.decode_prep_append_bf16(qp, ck, cv, cfg, pt, pos_t, 0, q, k, v, w, w, cos,
                                                sin, 1, stream=st), "prep")
            gk.check(gk.flash_attention_decode_paged_bf16(out, pm, pl, pa, qp, ck, cv, pt, seq_t,
                                                          cfg, 0, 1 / 16, split, n, 1,
                                                          stream=st), "decode")

        def one(st, i=0):
            gk.check(gk.flash_attention_prep_append_decode_paged_bf16(
                out, pm, pl, pa, q, ck, cv, pt, seq_t, pos_t, k, v, w, w, cos, sin, cfg, 0,
                1 / 16, split, n, 1, stream=st), "fused")
        two(torch.cuda.current_stream().cuda_stream)
        one(torch.cuda.current_stream().cuda_stream)
        fused[name] = {"prep_then_attention_us": round(time_graph_calls(torch, two, 20) * 1e3, 2),
                       "fused_us": round(time_graph_calls(torch, one, 20) * 1e3, 2)}
        del ck, cv
    res["decode_layer_from_raw_projections"] = fused

    # Runtime decode-step bookkeeping: host (validate, map, H2D copies) vs
    # device (one kernel), wall time per step with the stream drained.
    rt_res = {}
    for batch in (1, 64):
        rt_h, rt_d = gk.Runtime(batch, 1100, 16), gk.Runtime(batch, 1100, 16)
        gk.check(rt_h.init_code)
        gk.check(rt_d.init_code)
        gk.check(rt_h.prepare_prefill(900))
        gk.check(rt_d.prepare_prefill(900))
        torch.cuda.synchronize()
        t0 = _time.perf_counter()
        for _ in range(100):
            gk.check(rt_h.prepare_decode_step())
        torch.cuda.synchronize()
        t1 = _time.perf_counter()
        for _ in range(100):
            gk.check(rt_d.prepare_decode_step_device())
        torch.cuda.synchronize()
        t2 = _time.perf_counter()
        assert rt_d.device_step_status() == 0
        rt_res[f"batch{batch}"] = {"host_us": round((t1 - t0) * 1e4, 1),
                                   "device_us": round((t2 - t1) * 1e4, 1)}
        rt_h.close()
        rt_d.close()
    res["runtime_decode_step"] = rt_res
    return res


def _stats(values):
    import statistics
    return {"median": statistics.median(values), "min": min(values), "max": max(values),
            "runs": len(values)}


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(runs_1core: int = 3, runs_all: int = 5, quick: bool = False):
    """The oracle's append + decode attention timed in C on the host cores,
    on one thread (the reference's own host reference is single-threaded)
    and on a pool of all host threads split over (sequence, KV head) tasks.

    Primary row: BASELINE config 1 in full -- one sliding layer, 8x256 KV, 16
    q heads, 1024-slot page-1 ring, 2048 sequential append+attend steps from
    an empty cache, N(0,1) inputs, scale 1/16 -- the 2048-step loop timed
    inside C. One-step rows for configs 2 (48 layers, context 8192), 3 (64
    sequences, contexts U[512, 32768], one global layer) and 4 (131072 keys,
    1% x8). Reported per row: median / min / max seconds over the runs."""
    import numpy as np
    from oracle import oracle
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, threads)
    fill_threads = threads
    scale = 1.0 / 16.0
    rows = {}

    # ---- config 1: the full 2048-step loop.
    steps = 256 if quick else 2048
    q = oracle.fill_normal_bf16((steps, QH, DIM), 101, threads=fill_threads)
    k = oracle.fill_normal_bf16((steps, HEADS, DIM), 102, threads=fill_threads)
    v = oracle.fill_normal_bf16((steps, HEADS, DIM), 103, threads=fill_threads)
    c1 = (1, WINDOW, 1, WINDOW, 1, HEADS, DIM, WINDOW)
    c1_bytes = sum(layer_bytes(min(t + 1, WINDOW)) for t in range(steps))
    ref_out = None
    for name, th, runs in (("1core", 1, runs_1core), ("all_cores", threads, runs_all)):
        secs = []
        for r in range(runs):
            _log(f"cpu config1 {name} run {r + 1}/{runs}")
            sec, out, *_ = oracle.time_config1(q, k, v, c1, scale, th)
            assert sec > 0
            if ref_out is None:
                ref_out = out
            assert np.array_equal(out, ref_out), "threaded CPU run differs from 1-core run"
            secs.append(sec)
        st = _stats(secs)
        rows[f"config1_{name}"] = {
            "threads": min(th, HEADS),  # one task per KV head
            "seconds": st, "us_per_layer_step": st["median"] / steps * 1e6,
            "GBs": c1_bytes / st["median"] / 1e9}
    del q, k, v

    # ---- one-step rows for configs 2-4 (caches filled once per config).
    def fill_caches(cfgs):
        """Seeded N(0,1) K and V caches for each config."""
        rng_seed = 200
        caches = []
        for c in cfgs:
            n = c[0] * c[1] * c[2] * c[5] * c[6]
            caches.append((oracle.fill_normal_bf16((n,), rng_seed, threads=fill_threads),
                           oracle.fill_normal_bf16((n,), rng_seed + 1, threads=fill_threads)))
            rng_seed += 2
        return caches

    def run_rows(name, cfgs, pts, caches, layer_list, seq, pos, batch, bytes_per_step,
                 runs_single):
        """Time one step: for each (config index, cache layer) of layer_list,
        the append + attention of `batch` sequences."""
        q = oracle.fill_normal_bf16((batch, QH, DIM), 301, threads=fill_threads)
        kn = oracle.fill_normal_bf16((batch, HEADS, DIM), 302, threads=fill_threads)
        vn = oracle.fill_normal_bf16((batch, HEADS, DIM), 303, threads=fill_threads)
        out = np.zeros_like(q)
        for tag, th, runs in (("1core", 1, runs_single), ("all_cores", threads, runs_all)):
            secs = []
            for r in range(runs):
                _log(f"cpu {name} {tag} run {r + 1}/{runs}")
                total = 0.0
                for ci, cl in layer_list:
                    ck, cv = caches[ci]
                    total += oracle.time_decode_layer(out, q, ck, cv, pts[ci], seq, pos, kn, vn,
                                                      cfgs[ci], cl, scale, th)
                secs.append(total)
            st = _stats(secs)
            rows[f"{name}_{tag}"] = {"threads": th, "seconds": st,
                                     "us_per_layer_step": st["median"] / len(layer_list) * 1e6,
                                     "GBs": bytes_per_step / st["median"] / 1e9}

    # config 2: 48 layers, batch 1, context 8192 (+ the appended token).
    seq_len = CONTEXT + 1
    g_pages = (seq_len + GLOBAL_PAGE - 1) // GLOBAL_PAGE
    s_cfg = (40, WINDOW, 1, WINDOW, 1, HEADS, DIM, WINDOW)
    g_cfg = (8, g_pages, GLOBAL_PAGE, g_pages, 1, HEADS, DIM, 0)
    caches = fill_caches((s_cfg, g_cfg))
    pts = (np.arange(WINDOW, dtype=np.int32), np.arange(g_pages, dtype=np.int32))
    layer_list, si, gi, c2_bytes = [], 0, 0, 0
    for l in range(NUM_LAYERS):
        if is_global_layer(l):
            layer_list.append((1, gi)); gi += 1
            c2_bytes += layer_bytes(seq_len)
        else:
            layer_list.append((0, si)); si += 1
            c2_bytes += layer_bytes(WINDOW)
    run_rows("config2_step", (s_cfg, g_cfg), pts, caches, layer_list,
             np.array([seq_len], np.int32), np.array([CONTEXT], np.int32), 1, c2_bytes,
             1 if quick else runs_1core)
    del caches

    if not quick:
        # config 3: 64 sequences, contexts U[512, 32768] (the GPU leg's seed),
        # pages allocated per sequence back to back.
        rng = np.random.default_rng(64)
        seq = rng.integers(512, 32769, size=64).astype(np.int32)
        max_pages = (int(seq.max()) + GLOBAL_PAGE - 1) // GLOBAL_PAGE
        need = (seq + GLOBAL_PAGE - 1) // GLOBAL_PAGE
        pt = np.full(64 * max_pages, -1, np.int32)
        nxt = 0
        for b in range(64):
            pt[b * max_pages: b * max_pages + need[b]] = np.arange(nxt, nxt + need[b])
            nxt += int(need[b])
        c3 = (1, nxt, GLOBAL_PAGE, max_pages, 64, HEADS, DIM, 0)
        caches = fill_caches((c3,))
        run_rows("config3_step", (c3,), (pt,), caches, [(0, 0)], seq, seq - 1, 64,
                 sum(layer_bytes(int(s)) for s in seq), runs_1core)
        del caches

        # config 4: 131072 keys, 1% of them x8.
        ctx = 131072
        c4 = (1, ctx // GLOBAL_PAGE, GLOBAL_PAGE, ctx // GLOBAL_PAGE, 1, HEADS, DIM, 0)
        caches = fill_caches((c4,))
        hot = np.random.default_rng(4).permutation(ctx)[:ctx // 100]
        ck = caches[0][0].reshape(ctx, HEADS * DIM)
        ck[hot] = oracle.f32_to_bf16(oracle.bf16_to_f32(ck[hot]) * 8)
        run_rows("config4_step", (c4,), (np.arange(ctx // GLOBAL_PAGE, dtype=np.int32),), caches,
                 [(0, 0)], np.array([ctx], np.int32), np.array([ctx - 1], np.int32), 1,
                 layer_bytes(ctx), runs_1core)
        del caches

    head = rows["config1_all_cores"]
    return {"value": round(head["GBs"], 3), "unit": "GB/s", "cores": head["threads"],
            "kind": "port",
            "us_per_layer_step": round(head["us_per_layer_step"], 1),
            "sample": (f"config1 in full: {steps} sequential append+attend steps from an empty "
                       f"1024-slot ring (8x256 KV, 16 q heads), the loop timed inside C; value = "
                       f"median of {runs_all} runs on {min(threads, HEADS)} threads (one "
                       f"task per KV head of the one sequence); 1-core and configs 2-4 one-step rows in 'rows'"),
            "rows": rows, "cpu_model": _cpu_model(), "nproc": os.cpu_count(),
            "threads_available": threads}


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it, with family / model / stepping
    (some hosts report only a short model name)."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                if k in ("model name", "cpu family", "model", "stepping", "cpu MHz") and k not in fields:
                    fields[k] = v
            elif fields:
                break
    except OSError:
        pass
    if not fields:
        return "unknown"
    extra = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping", "cpu MHz")
                      if k in fields)
    return f"{fields.get('model name', 'unknown')} ({extra})"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-quick", action="store_true",
                    help="CPU baseline on a 256-step sample of config 1 and config 2 only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batch64", action="store_true")
    ap.add_argument("--no-long", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-widened", action="store_true")
    ap.add_argument("--only", choices=["step", "persistent", "global", "copy", "prefill",
                                       "widened", "oproj", "batch64", "long", "config1", "cpu",
                                       "refgeo"],
                    default=None,
                    help="profiling helper: run one leg only")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the KV-cache path runs on a single MI355X and "
              f"has no multi-GPU leg (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    if args.only == "cpu":
        print(json.dumps(cpu_baseline(quick=args.cpu_quick)))
        return

    import torch
    import gemma_kv as gk
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    gk.lib()
    dev = torch.device("cuda:0")

    if args.only == "copy":
        # Calibration kernel for the PMC byte counters: a 1 GiB device copy.
        src = torch.empty(1 << 29, dtype=torch.int16, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2}))
        return

    if args.only == "prefill":
        print(json.dumps(bench_prefill(torch, gk, dev, args.steps)))
        return
    if args.only == "widened":
        print(json.dumps(bench_widened(torch, gk, dev)))
        return
    if args.only == "batch64":
        print(json.dumps(bench_batch64(torch, gk, dev, args.steps, args.warmup)))
        return
    if args.only == "long":
        print(json.dumps(bench_long(torch, gk, dev, args.steps, args.warmup)))
        return
    if args.only == "config1":
        print(json.dumps(bench_config1(torch, gk, dev)))
        return
    if args.only == "oproj":
        gen = torch.Generator(device=dev)
        gen.manual_seed(7)
        rnd = lambda shape: torch.randn(shape, generator=gen, device=dev).bfloat16().view(torch.int16)
        print(json.dumps(bench_oproj(torch, gk, dev, rnd, rows_list=(1, 64))))
        return

    # The batch-64 and long-context KV caches first (see alloc_kv).
    kv_long = alloc_kv(torch, dev, 131072) if not args.only and not args.no_long else None
    kv_b64 = alloc_kv(torch, dev, batch64_seq()[2]) if not args.only and not args.no_batch64 else None
    layers, caches, meta, scratch = build_config2(torch, gk, dev)
    step_bytes = sum(L.bytes for L in layers)
    runner = StepRunner(torch, gk, dev, layers, caches, meta)
    if args.only == "refgeo":
        print(json.dumps(bench_step_ref_geometry(torch, gk, dev, layers, caches, meta,
                                                 args.steps)))
        return
    if args.only == "persistent":
        for _ in range(args.steps):
            runner(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert runner.status() == 0
        return

    def step(stream):
        for L in layers:
            code = launch_layer(gk, L, meta, scratch, stream)
            if code:
                raise gk.HipError(code, "append_decode")

    if args.only == "step":
        for _ in range(args.steps):
            step(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        return

    # ---- per-kernel timing, live with HIP events on the launch stream: the
    # split phase (fused append + partials) of the global and of the sliding
    # layers, each replayed back-to-back from a graph.
    g_layers = [L for L in layers if L.is_global]
    s_layers = [L for L in layers if not L.is_global]

    def split_round(Ls):
        def fn(stream):
            for L in Ls:
                gk.check(launch_split_only(gk, L, meta, scratch, stream), "split phase")
        return fn

    if args.only == "global":
        for _ in range(args.steps):
            split_round(g_layers)(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        return

    # ---- the headline: the whole step as one persistent launch, K launches
    # back to back between events on the launch stream (so the time includes
    # each launch's start-up), after W untimed ones.
    torch.cuda.synchronize()
    ms_step = time_eager(torch, runner, args.steps, args.warmup)
    status = runner.status()
    if status != 0:
        raise RuntimeError(f"decode step reported status {status}")
    gbs = step_bytes / (ms_step * 1e-3) / 1e9
    # Each timed step is one launch of the step kernel, so the K back-to-back
    # launches give its average launch duration; value and roofline share
    # that one timing. Single launches between events are reported beside it.
    ms_single = time_each(torch, runner, max(5, args.steps // 2))

    result = {
        "metric": "decode attn+KV-append µs/layer-step and achieved HBM GB/s at batch 1 and 64",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "us_per_layer_step": round(ms_step * 1e3 / NUM_LAYERS, 3),
        "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) K/V/q from a fixed seed",
        "config": {"workload": "config2: 48 layers (40 sliding ring-1024 page-1 + 8 global page-64), "
                               "8 KV heads x 256, 16 q heads, batch 1, context 8192, fused append+decode",
                   "batch": 1, "context": CONTEXT, "layers": NUM_LAYERS,
                   "bytes_per_step": step_bytes,
                   "timing": "one persistent launch per step (layer i waits for layer i-1's output)"},
        "roofline": {"kernel": "decode_step_kernel (the whole 48-layer step, one launch)",
                     "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("decode_step_config2"),
                     "avg_launch_us": round(ms_step * 1e3, 2),
                     "timing": ("the K timed steps, one kernel launch each, back to back "
                                "between HIP events on the launch stream (the same timing "
                                "as value)"),
                     "single_launch_us_median": round(ms_single * 1e3, 2),
                     "algorithmic_bytes_per_launch": step_bytes},
    }
    result["step_with_prep"] = bench_step_prep(torch, gk, runner, max(10, args.steps // 2))
    result["step_reference_global_geometry"] = bench_step_ref_geometry(
        torch, gk, dev, layers, caches, meta, max(10, args.steps // 2))
    if not args.no_batch64:
        b64 = bench_batch64(torch, gk, dev, max(3, args.steps // 5), 2, kv=kv_b64)
        result["batch64"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in b64.items()}
    if not args.no_long:
        lc = bench_long(torch, gk, dev, max(10, args.steps // 2), 3, kv=kv_long)
        result["long_context"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                  for k, v in lc.items()}
    del runner, kv_b64, kv_long
    if not args.no_prefill:
        result["prefill_config5"] = bench_prefill(torch, gk, dev, max(5, args.steps // 2))
    # The legs timed by graph replay come last. Each graph leg also runs on a
    # second stream (warm-up outside capture, the capture itself); once a
    # kernel has run on another stream, the eager launches of the first
    # measured 4-5% slower for the rest of the process (long context 157.6
    # -> 164.8 us after one small kernel on a side stream).
    result["config1_gpu"] = bench_config1(torch, gk, dev)
    if not args.no_widened:
        result["widened"] = bench_widened(torch, gk, dev)
    rounds = 20
    g_ms, _ = time_graph(torch, lambda st: [split_round(g_layers)(st) for _ in range(rounds)], 3, 1)
    s_ms, _ = time_graph(torch, lambda st: [split_round(s_layers)(st) for _ in range(4)], 3, 1)
    g_launch_us = g_ms * 1e3 / (rounds * len(g_layers))
    s_launch_us = s_ms * 1e3 / (4 * len(s_layers))
    g_bytes = g_layers[0].bytes
    s_bytes = s_layers[0].bytes
    g_gbs = g_bytes / (g_launch_us * 1e-6) / 1e9
    s_gbs = s_bytes / (s_launch_us * 1e-6) / 1e9
    result["global_split_kernel"] = {
        "kernel": "decode_split_kernel<8x256>, global layer (8193 keys, fused append)",
        "avg_launch_us": round(g_launch_us, 3), "achieved_GBs": round(g_gbs, 1),
        "frac": round(g_gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic("decode_split_global_ctx8192"),
        "algorithmic_bytes_per_launch": g_bytes,
        "split_size": g_layers[0].split, "num_splits": g_layers[0].n_splits}
    result["sliding_split_kernel"] = {
        "avg_launch_us": round(s_launch_us, 3), "achieved_GBs": round(s_gbs, 1),
        "algorithmic_bytes_per_launch": s_bytes,
        "split_size": s_layers[0].split, "num_splits": s_layers[0].n_splits}
    ms_graph, _ = time_graph(torch, step, max(5, args.steps // 2), 2)
    gbs_graph = step_bytes / (ms_graph * 1e-3) / 1e9
    result["per_layer_launches"] = {"ms_per_step": round(ms_graph, 4),
                                    "us_per_layer_step": round(ms_graph * 1e3 / NUM_LAYERS, 3),
                                    "achieved_GBs": round(gbs_graph, 1),
                                    "timing": "hipGraph replay of 48 fused append+decode launches"}
    del caches
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(quick=args.cpu_quick)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
