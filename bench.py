#!/usr/bin/env python3
"""Tree-verification attention benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

A step is one ragged verify attention call (``varlen_tree_attention``) over
the Qwen3-8B-shaped workload B=8 requests x (prefix 8192 + tree of 128
packed tokens), 32 query / 8 KV heads, head_dim 128, bf16, inputs resident
in HBM.  K/V come from rotating buffer sets (3 x 273 MB) so the 256 MB
Infinity Cache cannot serve a call's keys from the previous call.  Each call
is bracketed by HIP events on the launch stream: attention kernel, split-K
combine.  One JSON line goes to stdout; progress goes to stderr.

Also reported: the roofline of the attention kernel (binding side from the
algorithmic bytes and flops), the HBM fraction the metric names, the MFMA
ceiling of the kernel's launch shape timed right after the headline calls
(what the part sustains in that clock state, and the kernel's fraction of
it), the CPU oracle timed on host cores on a one-request sample, and
secondary workloads (bitmask and greedy-accept kernels, the other benchmark
shapes).
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "tree-verify attn µs/call + % HBM roofline, Qwen3-8B shape, N=128, ctx 8k, B=8"
PEAK_HBM = 8.0e12          # B/s, MI355X HBM3E
PEAK_MFMA_BF16 = 2.5e15    # FLOP/s, dense bf16
PEAK_MFMA_FP32 = 157.3e12  # FLOP/s, dense fp32
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"
BENCH_LIB = ROOT / "cast_amd" / "libcast_bench.so"
_bench_lib = None


def bench_lib():
    """The measurement aids of cast_amd/csrc/bench/cast_bench.h (built by
    cast_amd.build into libcast_bench.so beside the product library)."""
    global _bench_lib
    if _bench_lib is None:
        import ctypes
        import torch  # noqa: F401  (map torch's HIP runtime first)
        if not BENCH_LIB.exists():
            raise RuntimeError(f"{BENCH_LIB} is missing: build it with `python -m cast_amd.build`")
        lib = ctypes.CDLL(str(BENCH_LIB))
        P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        lib.cast_clock_sample.argtypes = [P, I32, I32, P]
        lib.cast_clock_sample.restype = ctypes.c_int
        lib.cast_mfma_ceiling.argtypes = [P, I64, P, P, I32, I32, I32, P]
        lib.cast_mfma_ceiling.restype = ctypes.c_int
        _bench_lib = lib
    return _bench_lib


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def roofline(wl, seconds):
    """Binding-side roofline of one attention call over ``wl``."""
    byt, flo = wl.algorithmic_bytes(), wl.algorithmic_flops()
    peak = PEAK_MFMA_FP32 if wl.dtype == "fp32" else PEAK_MFMA_BF16
    t_hbm, t_mfma = byt / PEAK_HBM, flo / peak
    if t_mfma >= t_hbm:
        ach = flo / seconds / 1e12
        return dict(bound="mfma", achieved=round(ach, 2), peak=peak / 1e12, unit="TFLOP/s",
                    frac=round(ach / (peak / 1e12), 4))
    ach = byt / seconds / 1e9
    return dict(bound="hbm", achieved=round(ach, 1), peak=PEAK_HBM / 1e9, unit="GB/s",
                frac=round(ach / (PEAK_HBM / 1e9), 4))


def traffic_of(name):
    """HBM bytes of one call over workload ``name`` as the profiler's FETCH_SIZE
    and WRITE_SIZE counters read them, per kernel, scaled by the same
    counters over a plain elementwise kernel (profiles/traffic.json), or
    None when that workload was not profiled."""
    try:
        return json.loads(TRAFFIC_FILE.read_text()).get(name)
    except (ValueError, OSError):
        return None


def whole_call_traffic(wl, entry):
    """Attention kernel plus split-K combine: bytes and their ratio to the
    workload's algorithmic bytes (Q, K, V, out and the ancestor words once)."""
    if not entry:
        return None
    total = entry["hbm_bytes_per_launch"] + entry.get("combine_bytes", 0)
    return dict(bytes=total, ratio=round(total / wl.algorithmic_bytes(), 3),
                attention_bytes=entry["hbm_bytes_per_launch"], combine_bytes=entry.get("combine_bytes", 0),
                algorithmic_bytes=wl.algorithmic_bytes())


class Harness:
    """Resident inputs of one workload, with rotated K/V sets."""

    def __init__(self, wl, dev, sets, kv_split):
        import numpy as np
        import torch
        from cast_amd import tree_bitmask
        self.wl, self.dev, self.kv_split = wl, dev, kv_split
        self.meta = wl.meta_tensors(dev)
        self.mask = tree_bitmask(self.meta["parent"], self.meta["cu_q"], 2)
        self.sets = []
        for s in range(sets):
            wl.seed = 1000 + s
            self.sets.append(wl.qkv(device=dev, generator_device=dev))
        wl.seed = 0
        self.out = torch.empty_like(self.sets[0][0])
        from cast_amd.tree_attn import plan
        p = plan(wl.B, wl.total_q, wl.total_kv, wl.Hq, wl.Hkv, wl.D, kv_split=kv_split)
        self.plan = p
        self.ws = torch.empty(max(p.workspace_bytes, 256), dtype=torch.uint8, device=dev)
        del np

    def call(self, i, hook=None):
        from cast_amd import varlen_tree_attention
        q, k, v = self.sets[i % len(self.sets)]
        m = self.meta
        return varlen_tree_attention(q, k, v, m["cu_q"], m["cu_kv"], m["prefix_len"], m["pack_len"], self.mask,
                                     return_lse=True, kv_split=self.kv_split, out=self.out, workspace=self.ws,
                                     _stage_hook=hook)

    def time(self, steps, warmup):
        import torch
        for i in range(warmup):
            self.call(i)
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            self.call(i, hook=lambda s, e=ev[i]: e[s].record())
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        attn = [e[0].elapsed_time(e[1]) * 1e3 for e in ev]     # us
        comb = [e[1].elapsed_time(e[2]) * 1e3 for e in ev]
        call = [e[0].elapsed_time(e[2]) * 1e3 for e in ev]
        w = 5
        return dict(call_us=statistics.median(call), call_mean_us=statistics.fmean(call),
                    attn_us=statistics.median(attn), attn_mean_us=statistics.fmean(attn),
                    combine_us=statistics.median(comb), wall_us=wall / steps * 1e6,
                    first_calls_us=statistics.median(call[:w]),
                    windows_us=[round(statistics.median(call[i:i + w]), 1) for i in range(0, steps, w)],
                    min_call_us=min(call))


def time_kernel(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        ev[i][0].record()
        fn()
        ev[i][1].record()
    torch.cuda.synchronize()
    return statistics.median(e[0].elapsed_time(e[1]) * 1e3 for e in ev)


def cpu_baseline(wl, budget_s=12.0):
    """The oracle (dense fp32 torch on host cores) on request 0, scaled to B."""
    import torch
    from oracle import attn as oracle_attn
    from oracle import bitmask as oracle_bitmask
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, k, v = wl.qkv(device="cpu")
    words = oracle_bitmask.chain_walk_words(wl.packed.parent, wl.cu_q)
    qf, kf, vf = q.float(), k.float(), v.float()

    def run():
        oracle_attn.dense_tree_attention(qf, kf, vf, wl.cu_q, wl.cu_kv, wl.prefix_len, wl.pack_len, words,
                                         requests=[0])

    run()
    times, t_end = [], time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 150):   # ~12 s of CPU work
        t = time.perf_counter()
        run()
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    S0, P0 = int(wl.prefix_len[0]), int(wl.pack_len[0])
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return dict(value=round(med * wl.B * 1e6, 1), unit="us/call", cores=cores, kind="port", cpu=model,
                sample=f"request 0 of {wl.B} (S={S0}, P={P0}, {wl.Hq}/{wl.Hkv} heads, D={wl.D}): dense fp32 "
                       f"torch oracle on the bf16-rounded inputs, median of {len(times)} runs "
                       f"({med * 1e3:.1f} ms each), scaled x{wl.B}")


def cpu_baseline_sample(wl, budget_s=2.0, min_runs=10, warmup=3):
    """The oracle on host cores over a bounded sample of ``wl``'s requests:
    after ``warmup`` untimed runs of request 0, requests 0, 1, ... are each
    run once per pass until ``budget_s`` is spent and at least ``min_runs``
    runs are timed; the median per request is scaled to the whole batch by
    the requests' score counts P_b * (S_b + P_b)."""
    import torch
    from oracle import attn as oracle_attn
    from oracle import bitmask as oracle_bitmask
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q, k, v = wl.qkv(device="cpu")
    words = oracle_bitmask.chain_walk_words(wl.packed.parent, wl.cu_q)
    qf, kf, vf = q.float(), k.float(), v.float()
    work = [int(wl.pack_len[b]) * (int(wl.prefix_len[b]) + int(wl.pack_len[b])) for b in range(wl.B)]

    def run(b):
        oracle_attn.dense_tree_attention(qf, kf, vf, wl.cu_q, wl.cu_kv, wl.prefix_len, wl.pack_len, words,
                                         requests=[b])

    for _ in range(warmup):
        run(0)
    times = {}
    t_end = time.perf_counter() + budget_s
    b, runs = 0, 0
    while True:
        t = time.perf_counter()
        run(b)
        times.setdefault(b, []).append(time.perf_counter() - t)
        runs += 1
        b = (b + 1) % wl.B
        if (time.perf_counter() > t_end and runs >= min_runs) or len(times.get(b, [])) >= 50:
            break
    sampled = sorted(times)
    med = sum(statistics.median(times[r]) for r in sampled)
    scale = sum(work) / sum(work[r] for r in sampled)
    return dict(value=round(med * scale * 1e6, 1), unit="us/call", cores=cores, kind="port",
                sample=f"requests {sampled[0]}-{sampled[-1]} of {wl.B} ({runs} timed runs after {warmup} "
                       f"warmups, median per request), dense fp32 torch oracle, scaled x{scale:.3g} by score count")


def store_layout(dev, steps, warmup):
    """The attention hook's per-layer work on the headline shapes, prefix in a
    per-request store [B, Hkv, cap, D] (cap = S + 320, three stores rotated
    per call) and the pack as HF
    hands it over ([Hkv, total_q, D]): the in-place call vs assembling the
    ragged K/V first, as cast_trees/serving.py:61-66 does (gather + scatter;
    the reference's fp32 up-cast on top is not included)."""
    import torch
    from cast_amd import scenarios
    from cast_amd.tree_attn import store_tree_attention
    from cast_amd import tree_bitmask, varlen_tree_attention
    wl = scenarios.qwen3_headline()
    meta = wl.meta_tensors(dev)
    mask = tree_bitmask(meta["parent"], meta["cu_q"], 2)
    B, Hkv, D, S = wl.B, wl.Hkv, wl.D, int(wl.prefix_len[0])
    cap = S + 320
    g = torch.Generator(device=dev).manual_seed(5)
    # three store sets, rotated per call like the headline's K/V (no cache reuse across calls)
    stores = [tuple(torch.randn((B, Hkv, cap, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(2))
              for _ in range(3)]
    kst, vst = stores[0]
    kpk = torch.randn((wl.total_q, Hkv, D), generator=g, device=dev).to(torch.bfloat16).transpose(0, 1)
    vpk = torch.randn((wl.total_q, Hkv, D), generator=g, device=dev).to(torch.bfloat16).transpose(0, 1)
    q = torch.randn((wl.Hq, wl.total_q, D), generator=g, device=dev).to(torch.bfloat16).transpose(0, 1)
    total_kv = wl.total_kv
    ws = torch.empty(1 << 27, dtype=torch.uint8, device=dev)
    # the reference's gather / scatter indices (serving.py:234-240)
    pl = torch.from_numpy(wl.prefix_len.astype("int64")).to(dev)
    cu_kv = meta["cu_kv"].long()
    pre_b = torch.repeat_interleave(torch.arange(B, device=dev), pl)
    cu_pre = torch.cat([pl.new_zeros(1), pl.cumsum(0)])
    pre_pos = torch.arange(int(cu_pre[-1]), device=dev) - cu_pre[:-1].repeat_interleave(pl)
    pre_dst = cu_kv[:-1].repeat_interleave(pl) + pre_pos
    pkl = torch.from_numpy(wl.pack_len.astype("int64")).to(dev)
    within = torch.arange(wl.total_q, device=dev) - meta["cu_q"].long()[:-1].repeat_interleave(pkl)
    pack_dst = (cu_kv[:-1] + pl).repeat_interleave(pkl) + within

    turn = [0]

    def inplace():
        k_st, v_st = stores[turn[0] % 3]
        turn[0] += 1
        store_tree_attention(q, k_st, v_st, kpk, vpk, meta["cu_q"], meta["prefix_len"], meta["pack_len"], mask,
                             total_kv=total_kv, workspace=ws)

    def assembled():
        k_rag = torch.empty((total_kv, Hkv, D), dtype=torch.bfloat16, device=dev)
        v_rag = torch.empty_like(k_rag)
        k_rag[pre_dst] = kst[pre_b, :, pre_pos, :]
        v_rag[pre_dst] = vst[pre_b, :, pre_pos, :]
        k_rag[pack_dst] = kpk.transpose(0, 1)
        v_rag[pack_dst] = vpk.transpose(0, 1)
        varlen_tree_attention(q, k_rag, v_rag, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"],
                              mask, workspace=ws)

    t_in = time_kernel(inplace, steps, warmup)
    t_as = time_kernel(assembled, steps, warmup)
    del stores
    log(f"  store layout: in place {t_in:.1f} us/call, ragged assembly + attention {t_as:.1f} us/call")
    return dict(inplace_us=round(t_in, 2), assembled_us=round(t_as, 2), cap=cap)


def kv_append(dev, steps, warmup, layers=36):
    """The accepted-path KV append after a verify round (cast_trees/serving.py:
    264-289) at Qwen3-8B shapes: 36 layers, B=8, 8 KV heads, D=128, stores of
    8192 + 320 slots, packs of 128, a planted accepted path per request: one
    fused launch driven by greedy_accept's device outputs, against the
    reference's two indexed copies per layer."""
    import torch
    from cast_amd import greedy_accept, scenarios, serving
    wl = scenarios.qwen3_headline()
    meta = wl.meta_tensors(dev)
    logits, _ = scenarios.planted_logits(wl, seed=0)
    path, plen, _, _ = greedy_accept(logits.to(dev), meta["cu_q"], meta["parent"],
                                     torch.from_numpy(wl.packed.token).to(dev))
    del logits
    B, Hkv, D, cap = wl.B, wl.Hkv, wl.D, int(wl.prefix_len[0]) + 320
    g = torch.Generator(device=dev).manual_seed(3)
    buf_k = [torch.empty((B, Hkv, cap, D), dtype=torch.bfloat16, device=dev) for _ in range(layers)]
    buf_v = [torch.empty_like(x) for x in buf_k]
    pack_k = [torch.randn((Hkv, wl.total_q, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
    pack_v = [torch.randn((Hkv, wl.total_q, D), generator=g, device=dev).to(torch.bfloat16) for _ in range(layers)]
    store_len = torch.from_numpy(wl.prefix_len.astype("int32")).to(dev)
    plen_h, path_h = plen.cpu().tolist(), path.cpu().tolist()
    src, dst_b, dst_p = [], [], []
    for b in range(B):
        for j, pk in enumerate([0] + [i + 1 for i in path_h[b][:plen_h[b]]]):
            src.append(int(wl.cu_q[b]) + pk)
            dst_b.append(b)
            dst_p.append(int(wl.prefix_len[b]) + j)
    src, dst_b, dst_p = (torch.tensor(x, dtype=torch.long, device=dev) for x in (src, dst_b, dst_p))

    # a decode loop hands over new pack tensors every round (key[0] / value[0]
    # of that round's forward): every call gets its own fresh views, made
    # before the timed region, so no per-tensor cache can hit
    rounds = [([x[:] for x in pack_k], [x[:] for x in pack_v]) for _ in range(steps + warmup)]
    turn = [0]

    def explicit():
        pk, pv = rounds[turn[0] % len(rounds)]
        turn[0] += 1
        serving.append_accepted(buf_k, buf_v, store_len, meta["cu_q"], path, plen, pk, pv)

    def hooked(n, w):
        # the serving flow: the attention hook recorded each layer's pack
        # K/V as the forward ran (serving._PACK_REC, done here before the
        # events), and the append reads PACK_KV
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(n)]
        for i in range(w + n):
            pk, pv = rounds[i % len(rounds)]
            serving.PACK_KV["k"], serving.PACK_KV["v"] = pk, pv
            serving._PACK_REC.begin(layers)
            for li in range(layers):
                serving._PACK_REC.note(li, pk[li], pv[li])
            if i >= w:
                ev[i - w][0].record()
            serving.append_accepted(buf_k, buf_v, store_len, meta["cu_q"], path, plen)
            if i >= w:
                ev[i - w][1].record()
        torch.cuda.synchronize()
        return statistics.median(a.elapsed_time(b) * 1e3 for a, b in ev)

    def per_layer():
        for li in range(layers):
            buf_k[li][dst_b, :, dst_p] = pack_k[li][:, src].permute(1, 0, 2)
            buf_v[li][dst_b, :, dst_p] = pack_v[li][:, src].permute(1, 0, 2)

    t_f = hooked(steps, warmup)
    t_x = time_kernel(explicit, steps, warmup)
    t_r = time_kernel(per_layer, steps, warmup)
    log(f"  kv append ({layers} layers, {len(src)} rows): fused {t_f:.1f} us (explicit pack lists {t_x:.1f} us), "
        f"per-layer indexing {t_r:.1f} us")
    return dict(fused_us=round(t_f, 2), fused_explicit_packs_us=round(t_x, 2), per_layer_indexing_us=round(t_r, 2),
                layers=layers, rows=len(src))


def cache_gather(dev, steps, warmup, layers=36):
    """The batch-one decoder's accepted-path cache compaction (cast_trees/
    verify.py:48-60) at Qwen3-8B shapes: 36 layers, 8 KV heads, D=128, bf16,
    a cached prefix of 4096 plus a packed pass of 128, 6 kept entries.  In
    place on the device (one launch) against the reference's index_select of
    every layer."""
    import torch
    from transformers import DynamicCache
    from cast_amd.verify import cache_layers, gather_cache
    n_prefix, n_pack, Hkv, D = 4096, 128, 8, 128
    g = torch.Generator(device=dev).manual_seed(5)
    full = [tuple(torch.randn((1, Hkv, n_prefix + n_pack, D), generator=g, device=dev).to(torch.bfloat16)
                  for _ in range(2)) for _ in range(layers)]
    cache = DynamicCache()
    for i, (k, v) in enumerate(full):
        cache.update(k, v, i)
    n_layers, get, put = cache_layers(cache)
    keep = [0, 1, 5, 9, 20, 33]

    def restore():
        for i, (k, v) in enumerate(full):
            put(i, k, v)

    def device():
        restore()
        gather_cache(cache, n_prefix, keep)

    def reference_flow():
        # what cast_trees/verify.py:48-60 does: one position index, then every
        # layer's K and V gathered whole along the sequence axis
        restore()
        positions = torch.cat([torch.arange(n_prefix, device=dev),
                               torch.tensor([n_prefix + j for j in keep], device=dev)])
        for layer in range(n_layers):
            k_old, v_old = get(layer)
            put(layer, torch.index_select(k_old, 2, positions), torch.index_select(v_old, 2, positions))

    t_d = time_kernel(device, steps, warmup)
    t_r = time_kernel(reference_flow, steps, warmup)
    log(f"  gather_cache ({layers} layers, prefix {n_prefix}, keep {len(keep)}): in place {t_d:.1f} us, "
        f"index_select {t_r:.1f} us")
    return dict(in_place_us=round(t_d, 2), index_select_us=round(t_r, 2), layers=layers, prefix=n_prefix,
                kept=len(keep))


def verify_round(dev, steps, warmup, layers=36):
    """One verify round's device work at the headline shapes (Qwen3-8B, 36
    layers, B=8 x (8192 + 128)): the ancestor words, the attention of every
    layer reading its KV store in place, the greedy accept over 1024 x 151936
    logits and the accepted-path KV append of all layers.  The model's own
    projections and MLPs are not part of it.  Timed as eager launches and as
    one replay of a HIP graph that captured the same round."""
    import torch
    from cast_amd import greedy_accept, scenarios, serving, tree_bitmask
    from cast_amd.tree_attn import plan, store_tree_attention
    wl = scenarios.qwen3_headline()
    meta = wl.meta_tensors(dev)
    B, Hkv, Hq, D, S = wl.B, wl.Hkv, wl.Hq, wl.D, int(wl.prefix_len[0])
    cap = S + 320
    g = torch.Generator(device=dev).manual_seed(11)
    bf = torch.bfloat16
    k_st = [torch.randn((B, Hkv, cap, D), generator=g, device=dev).to(bf) for _ in range(layers)]
    v_st = [torch.randn((B, Hkv, cap, D), generator=g, device=dev).to(bf) for _ in range(layers)]
    k_pk = [torch.randn((wl.total_q, Hkv, D), generator=g, device=dev).to(bf).transpose(0, 1) for _ in range(layers)]
    v_pk = [torch.randn((wl.total_q, Hkv, D), generator=g, device=dev).to(bf).transpose(0, 1) for _ in range(layers)]
    q = (torch.randn((wl.total_q, Hq, D), generator=g, device=dev) / math.sqrt(D)).to(bf)
    outs = [torch.empty_like(q) for _ in range(layers)]
    logits, _ = scenarios.planted_logits(wl, seed=0)
    logits = logits.to(dev)
    token = torch.from_numpy(wl.packed.token).to(dev)
    store_len = torch.from_numpy(wl.prefix_len.astype("int32")).to(dev)
    p = plan(B, wl.total_q, wl.total_kv, Hq, Hkv, D)
    ws = torch.empty(max(p.workspace_bytes, 256), dtype=torch.uint8, device=dev)

    def round_():
        mask = tree_bitmask(meta["parent"], meta["cu_q"], 2)
        for li in range(layers):
            store_tree_attention(q, k_st[li], v_st[li], k_pk[li], v_pk[li], meta["cu_q"], meta["prefix_len"],
                                 meta["pack_len"], mask, total_kv=wl.total_kv, out=outs[li], workspace=ws)
        path, plen, _, _ = greedy_accept(logits, meta["cu_q"], meta["parent"], token)
        # the append writes the accepted rows at fixed slots each round
        serving.append_accepted(k_st, v_st, store_len, meta["cu_q"], path, plen, k_pk, v_pk)

    eager = time_kernel(round_, steps, warmup)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        round_()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        round_()
    replay = time_kernel(graph.replay, steps, warmup)
    log(f"  verify round ({layers} layers, headline shapes): eager {eager / 1e3:.2f} ms, graph replay "
        f"{replay / 1e3:.2f} ms")
    res = dict(layers=layers, eager_ms=round(eager / 1e3, 3), graph_replay_ms=round(replay / 1e3, 3))
    del k_st, v_st, k_pk, v_pk, graph
    torch.cuda.empty_cache()
    return res


def graph_replay(dev, steps, warmup, layers=36):
    """The verify attention of one request (S=2048, P=16: launch-bound) over
    36 layers: 36 eager calls against one replay of a HIP graph that
    captured the same 36 calls (split-K partials and combine each)."""
    import torch
    from cast_amd import scenarios, tree_bitmask, varlen_tree_attention
    from cast_amd.tree_attn import plan
    wl = scenarios.qwen3_single()
    meta = wl.meta_tensors(dev)
    mask = tree_bitmask(meta["parent"], meta["cu_q"], 2)
    q, k, v = wl.qkv(device=dev)
    out = torch.empty_like(q)
    p = plan(wl.B, wl.total_q, wl.total_kv, wl.Hq, wl.Hkv, wl.D)
    ws = torch.empty(max(p.workspace_bytes, 256), dtype=torch.uint8, device=dev)

    def calls():
        for _ in range(layers):
            varlen_tree_attention(q, k, v, meta["cu_q"], meta["cu_kv"], meta["prefix_len"], meta["pack_len"], mask,
                                  out=out, workspace=ws)

    eager = time_kernel(calls, steps, warmup)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    replay = time_kernel(graph.replay, steps, warmup)
    log(f"  single-request attention x {layers} layers: eager {eager:.1f} us, graph replay {replay:.1f} us")
    return dict(layers=layers, eager_us=round(eager, 2), graph_replay_us=round(replay, 2),
                per_layer_eager_us=round(eager / layers, 2), per_layer_graph_us=round(replay / layers, 2))


def draft_trees(dev, steps, warmup):
    """Drafting at Qwen3-8B shapes: B=8 requests x 15 future positions x the
    151936-entry vocabulary (bf16 logits), top-8 per position, one best-first
    tree of 127 nodes per request.  The device path (cast_draft_topk +
    cast_build_trees) against the reference flow: torch log_softmax + topk on
    the GPU, a copy to the host, and the heap of cast_trees/tree.py:29-49."""
    import numpy as np
    import torch
    from cast_amd import tree as T
    from cast_amd.draft import build_trees, topk_marginals
    B, L, V = 8, 15, 151936
    g = torch.Generator(device=dev).manual_seed(11)
    x = (torch.randn((B * L, V), generator=g, device=dev) * 4).to(torch.bfloat16)
    bud = torch.full((B,), 127, dtype=torch.int32, device=dev)

    def device():
        idx, lp = topk_marginals(x, 8, on_device=True)
        build_trees(idx.view(B, L, 8), lp.view(B, L, 8), bud)

    def reference_flow():
        top = torch.topk(torch.nn.functional.log_softmax(x.float(), dim=-1), 8, dim=-1)
        ti, tl = top.indices.cpu().numpy(), top.values.cpu().numpy()
        for b in range(B):
            T.build_tree(ti[b * L:(b + 1) * L], tl[b * L:(b + 1) * L], 127)

    t_d = time_kernel(device, steps, warmup)
    idx, lp = topk_marginals(x, 8, on_device=True)
    t_k = time_kernel(lambda: topk_marginals(x, 8, on_device=True), steps, warmup)
    t_t = time_kernel(lambda: build_trees(idx.view(B, L, 8), lp.view(B, L, 8), bud), steps, warmup)
    t_tt = time_kernel(lambda: torch.topk(torch.nn.functional.log_softmax(x.float(), dim=-1), 8, dim=-1), steps,
                       warmup)
    t_r = time_kernel(reference_flow, max(3, steps // 5), 2)
    log(f"  draft trees (B={B}, 127 nodes): device {t_d:.1f} us (top-k {t_k:.1f}, trees {t_t:.1f}), "
        f"torch topk + host heap {t_r:.1f} us (torch log_softmax + topk alone {t_tt:.1f} us)")
    return dict(device_us=round(t_d, 2), topk_us=round(t_k, 2), trees_us=round(t_t, 2),
                torch_topk_host_heap_us=round(t_r, 2), torch_log_softmax_topk_us=round(t_tt, 2), batch=B, nodes=127,
                topk_gbps=round(B * L * V * 2 / (t_k * 1e-6) / 1e9, 1))


def bitmask_lines(dev, steps, warmup):
    """K1 (ancestor words) on the headline trees (1024 rows) and on the B=32
    stress trees (4096 rows), and K3 (greedy accept) on the headline trees
    with full Qwen3-vocabulary bf16 logits."""
    import torch
    from cast_amd import greedy_accept, scenarios, tree_bitmask
    res = {}
    for key, wl in (("tree_bitmask", scenarios.qwen3_headline()), ("tree_bitmask_b32", scenarios.stress_mixed())):
        meta = wl.meta_tensors(dev)
        t_bm = time_kernel(lambda: tree_bitmask(meta["parent"], meta["cu_q"], 2), steps, warmup)
        res[key] = dict(us_per_call=round(t_bm, 2), rows=int(wl.total_q))
        log(f"  {key}: {t_bm:.1f} us for {wl.total_q} rows")
    wl = scenarios.qwen3_headline()
    meta = wl.meta_tensors(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    logits = torch.randn(wl.total_q, wl.vocab, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    tok = torch.from_numpy(wl.packed.token).to(dev)
    t_acc = time_kernel(lambda: greedy_accept(logits, meta["cu_q"], meta["parent"], tok), steps, warmup)
    lb = wl.total_q * wl.vocab * 2
    res["greedy_accept"] = dict(us_per_call=round(t_acc, 2), logits_bytes=lb,
                                hbm_frac=round(lb / (t_acc * 1e-6) / PEAK_HBM, 4))
    log(f"  greedy_accept {t_acc:.1f} us ({lb / t_acc / 1e3:.0f} GB/s)")
    return res


ATTN_WORKLOADS = ("cpu-plumbing", "qwen3-8b-single", "qwen3-8b-ragged", "llama31-8b-ctx32k-p128",
                  "qwen3-8b-stress-b32", "qwen3-8b-stress-b32-trees", "qwen3-8b-b8-ctx8k-p128-fp32",
                  "qwen3-8b-b8-ctx8k-p128-fp16", "d256-b8-ctx8k-p128", "d256-b8-ctx8k-p128-fp32")
# the benchmark's five named configurations, each with a CPU oracle figure
CPU_SAMPLED = ("cpu-plumbing", "qwen3-8b-single", "qwen3-8b-ragged", "llama31-8b-ctx32k-p128",
               "qwen3-8b-stress-b32")


def attn_workload(dev, name, steps, warmup, cpu=False):
    """One attention workload timed like the headline (2 rotated K/V sets)."""
    import torch
    from cast_amd import scenarios
    if name.endswith(("-fp32", "-fp16")):
        # a workload's shapes in fp32 (what the unchanged reference hook hands
        # the kernel, cast_trees/serving.py:68-71) or in fp16 (same MFMA rate
        # as bf16 on this part)
        wl = dataclasses.replace(scenarios.CONFIGS[name[:-5]](), dtype=name[-4:], name=name)
    else:
        wl = scenarios.CONFIGS[name]()
    h = Harness(wl, dev, sets=2, kv_split=0)
    t = h.time(steps, warmup)
    rl = roofline(wl, t["attn_us"] * 1e-6)
    res = dict(us_per_call=round(t["call_us"], 2), attn_us=round(t["attn_us"], 2),
               combine_us=round(t["combine_us"], 2), steps=steps, warmup=warmup, dtype=wl.dtype,
               bound=rl["bound"], frac=rl["frac"],
               hbm_frac=round(wl.algorithmic_bytes() / (t["call_us"] * 1e-6) / PEAK_HBM, 4),
               tokens=int(wl.total_q), kv_tokens=int(wl.total_kv), kv_split=h.plan.kv_split,
               algorithmic_bytes=wl.algorithmic_bytes(), algorithmic_flops=wl.algorithmic_flops(),
               whole_call_traffic=whole_call_traffic(wl, traffic_of(name)))
    log(f"  {name}: {t['call_us']:.1f} us/call (attn {t['attn_us']:.1f}, combine {t['combine_us']:.1f}), "
        f"{rl['bound']} frac {rl['frac']:.3f} ({steps} timed after {warmup})")
    del h
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = cpu_baseline_sample(wl)
        log(f"    cpu oracle: {res['cpu_baseline']['value']:.0f} us/call ({res['cpu_baseline']['sample']})")
    return res


def secondary(dev, steps, warmup, cpu=True):
    """Every other workload, each entry with the timed and untimed call
    counts it used.  A workload that raises is recorded with its error, so
    that it cannot take the headline line down with it."""
    import torch
    res = {}

    def guarded(key, fn):
        try:
            return fn()
        except Exception as e:   # noqa: BLE001  (reported in the line, not swallowed)
            log(f"  {key}: FAILED {type(e).__name__}: {e}")
            try:   # release what the failed workload held before the next one
                torch.cuda.synchronize()
                torch.cuda.empty_cache()
            except Exception:   # noqa: BLE001
                pass
            return dict(error=f"{type(e).__name__}: {e}")

    for name in ATTN_WORKLOADS:
        res[name] = guarded(name, lambda: attn_workload(dev, name, steps, warmup, cpu=cpu and name in CPU_SAMPLED))
    # fresh stores settle over ~20 calls
    runs = [("store_layout", store_layout, max(steps, 60), max(warmup, 20)),
            ("kv_append", kv_append, steps, warmup), ("cache_gather", cache_gather, steps, warmup),
            ("draft_trees", draft_trees, steps, warmup), ("graph_replay", graph_replay, steps, warmup),
            ("verify_round", verify_round, steps, warmup)]
    for key, fn, n, w in runs:
        res[key] = guarded(key, lambda: dict(fn(dev, n, w), steps=n, warmup=w))
    lines = guarded("tree_bitmask", lambda: bitmask_lines(dev, steps, warmup))
    if "error" in lines:
        res["tree_bitmask"] = lines
    else:
        for key, r in lines.items():
            res[key] = dict(r, steps=steps, warmup=warmup)
    return res


class CeilingLoop:
    """cast_mfma_ceiling at the headline attention kernel's launch shape:
    `grid` workgroups x 8 waves x 65 tiles x 32 v_mfma_f32_32x32x16_bf16
    (at grid 256, the headline's exact MFMA count)."""
    TILES = 65

    def __init__(self, dev):
        import torch
        from cast_amd import _lib
        self.lib, self._lib = bench_lib(), _lib
        g = torch.Generator(device=dev).manual_seed(5)
        self.src = torch.randn(1 << 20, generator=g, device=dev).to(torch.bfloat16)
        self.out = torch.empty(256 * 512, dtype=torch.float32, device=dev)
        self.clk = torch.zeros(2 * 256, dtype=torch.int64, device=dev)
        self.stream = _lib.stream_of(self.src)

    def run(self, mode, steps, warmup, grid=256):
        import torch
        L = self._lib

        def launch():
            L.check(self.lib.cast_mfma_ceiling(L.ptr(self.src), self.src.numel() // 8, L.ptr(self.out),
                                               L.ptr(self.clk), grid, self.TILES, mode, self.stream),
                    "cast_mfma_ceiling")
        for _ in range(warmup):
            launch()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
        torch.cuda.synchronize()
        for e in ev:
            e[0].record()
            launch()
            e[1].record()
        torch.cuda.synchronize()
        us = statistics.fmean(e[0].elapsed_time(e[1]) * 1e3 for e in ev)
        cw = self.clk[:2 * grid].view(grid, 2).cpu().tolist()
        ghz = sorted(c / (w / 100.0) / 1e3 for c, w in cw if w > 0)
        if not torch.isfinite(self.out[:grid * 512]).all():
            raise RuntimeError("mfma ceiling: non-finite accumulators")
        flop = grid * 8 * self.TILES * 32 * 32 * 32 * 16 * 2
        tf = flop / us / 1e6
        return dict(us=round(us, 2), tflops=round(tf, 1), frac=round(tf / (PEAK_MFMA_BF16 / 1e12), 4),
                    ghz_median=round(statistics.median(ghz), 3), ghz_min=round(ghz[0], 3), ghz_max=round(ghz[-1], 3))


def mfma_ceiling(dev, steps, warmup, sets=3):
    """What the matrix pipes sustain at the headline attention kernel's launch
    shape (cast_mfma_ceiling): 256 workgroups x 8 waves x 65 tiles x 32
    v_mfma_f32_32x32x16_bf16, the headline's exact MFMA count, with operands in
    registers, then read from LDS, then with the per-tile barrier as well.  The
    headline attention kernel is timed in the same process before and after,
    so the ratio does not depend on the box's sustained clock."""
    from cast_amd import scenarios
    wl = scenarios.qwen3_headline()
    h = Harness(wl, dev, sets=sets, kv_split=0)
    loop = CeilingLoop(dev)
    flop = 256 * 8 * loop.TILES * 32 * 32 * 32 * 16 * 2

    def attention():
        t = h.time(steps, warmup)
        return dict(us=round(t["attn_mean_us"], 2), tflops=round(wl.algorithmic_flops() / t["attn_mean_us"] / 1e6, 1))

    before = attention()
    log(f"  attention kernel {before['us']} us = {before['tflops']} TFLOP/s")
    modes = {}
    for name, mode in (("registers", 0), ("lds_operands", 1), ("lds_operands_barrier", 3)):
        modes[name] = r = loop.run(mode, steps, warmup)
        log(f"  mfma ceiling, {name}: {r['us']} us = {r['tflops']} TFLOP/s ({r['frac']} of peak) "
            f"at {r['ghz_median']} GHz ({r['ghz_min']}-{r['ghz_max']})")
    # the register loop on fewer CUs (one workgroup per CU): a clock that rises
    # as CUs go idle is set by the power limit, not by a fixed MFMA clock
    fewer = {}
    for g in (128, 64, 32):
        r = loop.run(0, steps, warmup, grid=g)
        fewer[str(g)] = dict(us=r["us"], ghz_median=r["ghz_median"])
        log(f"  mfma ceiling, registers, {g} workgroups: {r['us']} us at {r['ghz_median']} GHz")
    after = attention()
    log(f"  attention kernel {after['us']} us = {after['tflops']} TFLOP/s")
    best = max(before["tflops"], after["tflops"])
    return dict(workload=wl.name, grid=256, tiles=loop.TILES, waves=8, flop_per_launch=flop,
                algorithmic_flop=wl.algorithmic_flops(), steps=steps, warmup=warmup, modes=modes,
                registers_on_fewer_workgroups=fewer,
                attention_before=before, attention_after=after,
                attention_of_register_ceiling=round(best / modes["registers"]["tflops"], 3),
                attention_of_lds_ceiling=round(best / modes["lds_operands_barrier"]["tflops"], 3))


def clock_trace(dev, n, sets):
    """The headline call n times from a cold start, each followed by a shader
    clock sample (cast_clock_sample): per call the event time, the clock and
    their product, the shader cycles per call.  Flat cycles under a moving
    time mean the clock moved, not the kernel."""
    import torch
    from cast_amd import _lib, scenarios
    lib = bench_lib()
    wl = scenarios.qwen3_headline()
    h = Harness(wl, dev, sets=sets, kv_split=0)
    buf = torch.zeros(2 * n, dtype=torch.int64, device=dev)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(n)]
    stream = _lib.stream_of(buf)
    torch.cuda.synchronize()
    for i in range(n):
        ev[i][0].record()
        h.call(i)
        ev[i][1].record()
        _lib.check(lib.cast_clock_sample(_lib.ptr(buf), i, 1000, stream), "cast_clock_sample")
    torch.cuda.synchronize()
    us = [a.elapsed_time(b) * 1e3 for a, b in ev]
    cw = buf.view(n, 2).cpu().tolist()
    ghz = [c / (w / 100.0) / 1e3 for c, w in cw]          # cycles per ns
    mcyc = [t * f / 1e3 for t, f in zip(us, ghz)]
    win = 10
    windows = [dict(calls=f"{lo}-{min(lo + win, n) - 1}", us=round(statistics.median(us[lo:lo + win]), 1),
                    ghz=round(statistics.median(ghz[lo:lo + win]), 3),
                    mcycles=round(statistics.median(mcyc[lo:lo + win]), 4)) for lo in range(0, n, win)]
    for w in windows:
        log(f"  calls {w['calls']:>9s}: {w['us']:7.1f} us  {w['ghz']:.3f} GHz  {w['mcycles']:.4f} Mcycles")
    return dict(workload=wl.name, calls=n, window=win, windows=windows,
                per_call=[[round(t, 1), round(f, 3)] for t, f in zip(us, ghz)])


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200,
                    help="untimed calls first (the clock settles over ~150 calls of this workload)")
    ap.add_argument("--sets", type=int, default=3, help="rotated K/V buffer sets")
    ap.add_argument("--kv-split", type=int, default=0, help="keys per split-K chunk (0: library choice)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--only", choices=["kv_append", "cache_gather", "draft_trees", "store_layout", "tree_bitmask",
                                       "graph_replay", "verify_round",
                                       *ATTN_WORKLOADS],
                    help="only run one secondary workload (for kernel profiles); prints its JSON")
    ap.add_argument("--clock-trace", type=int, default=0, metavar="N",
                    help="only run N headline calls from a cold start, each followed by a shader clock sample")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only time the MFMA ceiling loops at the headline kernel's launch shape, bracketed by "
                         "the headline attention kernel")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 launches), to scale HBM byte counters")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the verify path shards by request and KV head with no exchange, so no multi-GPU figure "
              "is produced", file=sys.stderr)
        sys.exit(2)

    import torch
    from cast_amd import scenarios
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        # an elementwise kernel (negation), not copy_(): a same-dtype copy_
        # may go to a DMA engine that the shader counters do not see
        n = args.copy_calibration << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "launches": 5}), flush=True)
        return
    if args.mfma_ceiling:
        print(json.dumps({"mfma_ceiling": mfma_ceiling(dev, args.steps, args.warmup, args.sets)}), flush=True)
        return
    if args.clock_trace:
        print(json.dumps({"clock_trace": clock_trace(dev, args.clock_trace, args.sets)}), flush=True)
        return
    if args.only:
        if args.only in ATTN_WORKLOADS:
            print(json.dumps({args.only: attn_workload(dev, args.only, args.steps, args.warmup)}), flush=True)
            return
        fn = {"kv_append": kv_append, "cache_gather": cache_gather, "draft_trees": draft_trees,
              "store_layout": store_layout, "tree_bitmask": bitmask_lines, "graph_replay": graph_replay,
              "verify_round": verify_round}[args.only]
        print(json.dumps({args.only: fn(dev, args.steps, args.warmup)}), flush=True)
        return
    log(f"device: {torch.cuda.get_device_name(dev)}")
    wl = scenarios.qwen3_headline()
    h = Harness(wl, dev, sets=args.sets, kv_split=args.kv_split)
    log(f"workload {wl.name}: total_q={wl.total_q} total_kv={wl.total_kv} kv_split={h.plan.kv_split} "
        f"workspace={h.plan.workspace_bytes / 2**20:.1f} MiB")
    t = h.time(args.steps, args.warmup)
    log(f"  call {t['call_us']:.1f} us (mean {t['call_mean_us']:.1f}), attention kernel {t['attn_us']:.1f} us, "
        f"combine {t['combine_us']:.1f} us, host wall {t['wall_us']:.1f} us/call")
    # achieved = algorithmic work per launch / mean launch duration (HIP events
    # on the launch stream), comparable with the profiler's average duration
    rl = roofline(wl, t["attn_mean_us"] * 1e-6)
    entry = traffic_of(wl.name)
    rl["traffic"] = entry["hbm_bytes_per_launch"] if entry else None
    call_s = t["call_us"] * 1e-6
    line = {
        "metric": METRIC, "value": round(t["call_us"], 2), "unit": "us/call", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(t["call_us"] / 1e3, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded Gaussian Q/K/V, trees from seeded N(0,5) 15x151936 block scores)",
        "config": {"workload": wl.name, "batch": wl.B, "prefix": int(wl.prefix_len[0]),
                   "pack": int(wl.pack_len[0]), "q_heads": wl.Hq, "kv_heads": wl.Hkv, "head_dim": wl.D,
                   "kv_split": h.plan.kv_split, "kv_sets": args.sets},
        "roofline": rl,
        "hbm_frac": round(wl.algorithmic_bytes() / call_s / PEAK_HBM, 4),
        "tokens_per_s": round(wl.total_q / call_s, 1),
        # the shader clock falls under sustained MFMA load and recovers over
        # ~100 calls: the first timed calls and the per-5-call medians show
        # where in that transient the timed region sat
        "first_calls_us": round(t["first_calls_us"], 2), "call_windows_us": t["windows_us"],
        "min_call_us": round(t["min_call_us"], 2),
        "attn_kernel_us": round(t["attn_us"], 2), "combine_us": round(t["combine_us"], 2),
        "call_mean_us": round(t["call_mean_us"], 2), "host_wall_us": round(t["wall_us"], 2),
        "algorithmic_bytes": wl.algorithmic_bytes(), "algorithmic_flops": wl.algorithmic_flops(),
        # the attention kernel's bytes (roofline.traffic) plus the combine's
        "whole_call_traffic": whole_call_traffic(wl, entry),
    }
    # the practical MFMA ceiling of this launch shape, timed right after the
    # headline calls with the same step and warmup counts: the headline's MFMA
    # count with LDS operand reads and the per-tile barrier, no softmax and no
    # loads.  Its clock depends on the load before it, as the kernel's does.
    ceil = CeilingLoop(dev).run(3, args.steps, args.warmup)
    ceil["attention_frac_of_ceiling"] = round(rl["achieved"] / ceil["tflops"], 4)
    ceil["loop"] = "lds_operands_barrier"
    line["mfma_ceiling"] = ceil
    log(f"  mfma ceiling (LDS operands + barrier): {ceil['tflops']} TFLOP/s ({ceil['frac']} of peak) at "
        f"{ceil['ghz_median']} GHz; attention kernel at {ceil['attention_frac_of_ceiling']} of it")
    del h
    torch.cuda.empty_cache()
    if not args.no_secondary:
        log("secondary workloads:")
        # at least 50 timed calls each, whatever the headline's counts
        line["secondary"] = secondary(dev, max(50, args.steps // 2), max(20, args.warmup // 4),
                                      cpu=not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle on host cores)...")
        line["cpu_baseline"] = cpu_baseline(wl)
        log(f"  {line['cpu_baseline']}")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
