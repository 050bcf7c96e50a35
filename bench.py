#!/usr/bin/env python3
"""Benchmark of the quantized paged decode attention hot path on one MI355X.

Workload (the metric's config): Llama-3-8B-shaped
single-layer decode — 32 query / 8 KV heads (GQA 4), head_dim 128, batch 16,
every sequence at 32,768 tokens = 32 FP16 sinks + 255 INT2/INT4 pages of 128
tokens + 96 FP16 tail tokens; 12.5% of key channels INT4 (16 outlier channels
per head scaled x8, chosen by 256 seeded calibration tokens).  K/V are fp16
N(0,1), quantised into the pools by the HIP quantize kernel; pages are placed
through a shuffled free list.  Three independent pool copies (~953 MB) rotate
step to step so no step is served from the 256 MB MALL.

One step = one decode layer-step for all 16 sequences: kitty_paged_decode,
i.e. the split-K kernel (pages + FP16 segments) and the merge kernel.  After
at least --warmup steps and --warmup-seconds of them (steady clock whatever
--steps is), `value` is microseconds per layer-step over exactly --steps
back-to-back steps (host clock; inputs resident in HBM).  The roofline entry
is for the split-K kernel: bursts of back-to-back launches between two HIP
events on the launch stream, right after `value` at the same settled clock
(per-launch event pairs in the alternating step pattern are reported as
upper bounds).

`value_window_r128` times the same step in the layout the pipeline decodes
with its 128-token FP16 value window (one value page fewer per sequence, a
224-token value tail); `legs` repeats the headline for configs 4 and 5, each
with its own roofline block and a sampled CPU baseline; `quantize_pack` times
config 2's batch quantize, `spill` the pipeline's spill launch,
`module_forward` KittyPagedAttention.forward decode steps on the GPU and
`module_forward_cfg1_cpu` the same module on CPU tensors (the product's CPU
path), with `cpu_baseline_cfg1` the reference's CPU decode of config 1 beside it;
`reference_items` runs the reference's own benchmark items (one-page key
quantise / dequantise, push_token throughput, memory compression) with its
defaults and timing method, and `widened_rows` times prefill (push_chunk) and
the profiler's |K| accumulation at production shapes; `cpu_baseline` is the
reference's CPU path restated op for op in torch (oracle/torch_reference.py)
on every thread this process may use, `cpu_baseline_c_port` the scalar C
restatement on one thread, both on a bounded sample of the config-3 step.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kitty-kv_amd"))

HBM_PEAK_GBPS = 8000.0

CONFIGS = {
    # config 1: the reference's CPU-runnable case (one sequence, 8 Q / 8 KV heads, 1K context), here on the GPU
    "cfg1": dict(B=1, Hq=8, Hkv=8, ctx=1024, boost=0.125, outlier=8.0, seed=1),
    "cfg3": dict(B=16, Hq=32, Hkv=8, ctx=32768, boost=0.125, outlier=8.0, seed=3),
    # config 4: ragged contexts drawn uniformly from [512, 65536] (seeded), 25 % INT4
    "cfg4": dict(B=64, Hq=32, Hkv=8, ctx=(512, 65536), boost=0.25, outlier=8.0, seed=4),
    "cfg5": dict(B=4, Hq=64, Hkv=8, ctx=131072, boost=0.125, outlier=16.0, seed=5),
    # config 3's pages with one query head per KV head (multi-head attention, the padded MFMA group)
    "mha": dict(B=16, Hq=8, Hkv=8, ctx=32768, boost=0.125, outlier=8.0, seed=3),
}
D, G, S = 128, 128, 32


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_workload(torch, dev, cfg, copies: int, placement_kind: str = "shuffled", sample_pages=()):
    """Pools of `copies` independent copies of the config's KV, quantised on
    the device from seeded fp16 K/V, with one DecodePlan per copy.  The fp16
    inputs of the pool pages in sample_pages are kept (w["samples"][page] =
    (k, v), each (Hkv, G, D) on the host) for parity checks."""
    from kitty.kernels.ops import DecodePlan, pool_store, quantize_into_pools
    import numpy as np
    B, Hq, Hkv = cfg["B"], cfg["Hq"], cfg["Hkv"]
    if isinstance(cfg["ctx"], tuple):   # ragged: per-sequence contexts from a seeded draw
        ctxs = np.random.default_rng(cfg["seed"]).integers(cfg["ctx"][0], cfg["ctx"][1] + 1, size=B)
    else:
        ctxs = np.full(B, cfg["ctx"])
    dk = round(cfg["boost"] * D)
    sentinel = min(dk + 1, 255)
    np_list = [(int(c) - S) // G for c in ctxs]
    tail_list = [(int(c) - S) % G for c in ctxs]
    n_pages, n_tail = max(np_list), max(tail_list)
    pages_per_copy = sum(np_list)
    gen = torch.Generator(device="cpu").manual_seed(cfg["seed"])
    chans = torch.stack([torch.randperm(D, generator=gen)[:dk] for _ in range(Hkv)])
    calib = torch.randn(256, Hkv, D, generator=gen)
    for h in range(Hkv):
        calib[:, h, chans[h]] *= cfg["outlier"]
    score = calib.abs().mean(0)
    order = torch.argsort(score, dim=-1, descending=True, stable=True)
    bi = torch.full((Hkv, D), sentinel, dtype=torch.uint8)
    for r in range(dk):
        bi[torch.arange(Hkv), order[:, r]] = r
    bi = bi.to(dev)

    used = copies * pages_per_copy
    P = used + 8
    kb = torch.empty(P, Hkv, D, G // 4, dtype=torch.uint8, device=dev)
    kh = torch.empty(P, Hkv, dk, G // 4, dtype=torch.uint8, device=dev)
    km = torch.empty(P, Hkv, 2, D, dtype=torch.float16, device=dev)
    vp = torch.empty(P, Hkv, G, D // 4, dtype=torch.uint8, device=dev)
    vm = torch.empty(P, Hkv, G, 2, dtype=torch.float16, device=dev)
    store = pool_store(kb, kh, km, vp, vm)
    if placement_kind == "shuffled":      # a fragmented pool: pages from a shuffled free list
        placement = torch.randperm(P, generator=gen)[:used].to(torch.int32)
    elif len(set(np_list)) == 1:          # first-fit, B sequences growing in lockstep: page p of seq b
        placement = torch.arange(used, dtype=torch.int32).view(copies, n_pages, B).transpose(1, 2).reshape(-1)
    else:
        placement = torch.arange(used, dtype=torch.int32)
    g = torch.Generator(device=dev).manual_seed(cfg["seed"] + 100)
    scale = torch.ones(Hkv, D, device=dev)
    for h in range(Hkv):
        scale[h, chans[h].to(dev)] = cfg["outlier"]
    chunk = 1024
    samples = {}
    want = {int(x) for x in sample_pages}
    for p0 in range(0, used, chunk):
        n = min(chunk, used - p0)
        k = (torch.randn(n, Hkv, G, D, device=dev, generator=g) * scale[None, :, None, :]).half()
        v = torch.randn(n, Hkv, G, D, device=dev, generator=g).half()
        quantize_into_pools(store, k, v, bi, placement[p0:p0 + n].to(dev), sentinel)
        for i, pid in enumerate(placement[p0:p0 + n].tolist()):
            if pid in want:
                samples[pid] = (k[i].cpu(), v[i].cpu())
    torch.cuda.synchronize()

    q = torch.randn(B, Hq, D, device=dev, generator=g).half()
    sk = torch.randn(B, Hkv, S, D, device=dev, generator=g).half()
    sv = torch.randn(B, Hkv, S, D, device=dev, generator=g).half()
    tk = torch.randn(B, Hkv, max(n_tail, 1), D, device=dev, generator=g).half()
    tv = torch.randn(B, Hkv, max(n_tail, 1), D, device=dev, generator=g).half()
    npg = torch.tensor(np_list, dtype=torch.int32, device=dev)
    sl = torch.full((B,), S, dtype=torch.int32, device=dev)
    tl = torch.tensor(tail_list, dtype=torch.int32, device=dev)
    out = torch.empty(B, Hq, D, dtype=torch.float16, device=dev)
    plans, tables = [], []
    for c in range(copies):
        bt = torch.zeros(B, n_pages, dtype=torch.int32)
        off = c * pages_per_copy
        for b in range(B):
            bt[b, :np_list[b]] = placement[off:off + np_list[b]]
            off += np_list[b]
        bt = bt.to(dev)
        tables.append(bt)
        plans.append(DecodePlan(q, bt, npg, kb, kh, km, vp, vm, bi, sk, sv, sl, tk, tv, tl, out=out))
    w = dict(B=B, Hq=Hq, Hkv=Hkv, dk=dk, n_pages=n_pages, n_tail=n_tail, np_list=np_list, tail_list=tail_list,
             P=P, pools=(kb, kh, km, vp, vm), tables=tables, q=q, sk=sk, sv=sv, tk=tk, tv=tv, bi=bi, plans=plans,
             out=out, sentinel=sentinel, samples=samples)
    return w


def algorithmic_bytes(w) -> dict:
    B, Hkv, Hq, dk = w["B"], w["Hkv"], w["Hq"], w["dk"]
    pages = sum(w["np_list"])
    per_page_head = D * G // 4 + dk * G // 4 + 2 * D * 2 + G * D // 4 + G * 2 * 2
    packed = Hkv * pages * per_page_head
    fp16 = Hkv * sum(S + t for t in w["tail_list"]) * D * 2 * 2
    small = B * Hq * D * 2 + pages * 4 + Hkv * D + 3 * B * 4   # q, block table, boost_idx, lengths
    return dict(per_page_head=per_page_head, packed=packed, fp16=fp16, total=packed + fp16 + small)


def cpu_threads() -> int:
    """Threads for the torch CPU baseline: every CPU this process may run on,
    capped by OMP_NUM_THREADS when the host sets it (a GPU box's CPU share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(cap))) if cap.isdigit() and int(cap) > 0 else max(1, n)


def _cpu_sequences(w, budget_s: float, run_one) -> dict:
    """Whole sequences of the workload through run_one(b, sub-pools) until
    about budget_s of CPU time; the total is scaled by pages to one
    layer-step (the reference's time is linear in the pages it walks)."""
    kb, kh, km, vp, vm = w["pools"]
    bt = w["tables"][0]
    done, t_total, pages_done = 0, 0.0, 0
    while done < w["B"] and (t_total < budget_s or done == 0):
        b = done
        npb = w["np_list"][b]
        idx = bt[b, :npb].long()
        sub = [t[idx].cpu() for t in (kb, kh, km, vp, vm)]   # the sequence's pages, compacted on the host
        t0 = time.perf_counter()
        run_one(b, sub)
        t_total += time.perf_counter() - t0
        done += 1
        pages_done += npb
    total_pages = sum(w["np_list"])
    return dict(value=t_total * total_pages / max(pages_done, 1), done=done, pages_done=pages_done,
                total_pages=total_pages)


def cpu_baseline_torch(w, budget_s: float) -> dict:
    """The reference's own CPU path, restated op for op in torch
    (oracle/torch_reference.py: paged_attention_reference with its discarded
    first dequantisation pass and per-channel high-bit loop), on whole
    sequences of the workload, with every thread torch may use here."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch
    import torch_reference as TR
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    q, sk, sv, tk, tv, bi = (t.cpu() for t in (w["q"], w["sk"], w["sv"], w["tk"], w["tv"], w["bi"]))

    def run_one(b, sub):
        n = w["tail_list"][b]
        TR.paged_attention(q[b], range(w["np_list"][b]), *sub, bi, w["dk"], sk[b], sv[b], tk[b, :, :n],
                           tv[b, :, :n], w["Hq"], w["Hkv"], D)
    try:
        r = _cpu_sequences(w, budget_s, run_one)
    finally:
        torch.set_num_threads(prev)
    return {"value": round(r["value"] * 1e6, 1), "unit": "us/layer-step", "cores": threads, "kind": "port",
            **host_cpu(),
            "sample": f"{r['done']} of {w['B']} sequences ({r['pages_done']} of {r['total_pages']} pages, all "
                      f"{w['Hkv']} KV heads, {S} sinks + FP16 tail each) through oracle/torch_reference.py "
                      f"(paged_attention_reference restated op for op in torch, CPU, {threads} threads); "
                      f"scaled by pages to one layer-step"}


def cpu_baseline_cfg1(torch, dev, budget_s: float = 3.0) -> dict:
    """The reference's CPU decode at config 1 (one sequence, 8 Q / 8 KV heads,
    1K context): oracle/torch_reference.py's paged_attention (the reference's
    paged_attention_reference restated op for op) on config 1's pools, run
    repeatedly for about budget_s on every thread torch may use here; the
    median run.  Beside it, module_forward_cfg1_cpu times the product's own
    CPU path (the whole module step)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch_reference as TR
    w = build_workload(torch, dev, CONFIGS["cfg1"], 1)
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        kb, kh, km, vp, vm = w["pools"]
        npb, n = w["np_list"][0], w["tail_list"][0]
        idx = w["tables"][0][0, :npb].long()
        sub = [t[idx].cpu() for t in (kb, kh, km, vp, vm)]
        q, sk, sv, tk, tv, bi = (t.cpu() for t in (w["q"], w["sk"], w["sv"], w["tk"], w["tv"], w["bi"]))
        times, t_end = [], time.perf_counter() + budget_s
        while time.perf_counter() < t_end or not times:
            t0 = time.perf_counter()
            TR.paged_attention(q[0], range(npb), *sub, bi, w["dk"], sk[0], sv[0], tk[0, :, :n], tv[0, :, :n],
                               w["Hq"], w["Hkv"], D)
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    return {"value": round(statistics.median(times) * 1e6, 1), "unit": "us/layer-step", "cores": threads,
            "kind": "port", **host_cpu(), "runs": len(times),
            "sample": f"config 1's whole step (1 sequence, {npb} pages, {S} sinks + {n} tail tokens, all "
                      f"{w['Hkv']} KV heads) through oracle/torch_reference.py, median of {len(times)} runs"}


def cpu_baseline_c(w, budget_s: float) -> dict:
    """The scalar C restatement (oracle/kitty_oracle.c) of the same function,
    one thread, for comparison with the torch figure."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    O.build()
    bin_ = w["bi"].cpu().numpy()
    q, sk, sv, tk, tv = (t.cpu().numpy() for t in (w["q"], w["sk"], w["sv"], w["tk"], w["tv"]))

    def run_one(b, sub):
        skb, skh, skm, svp, svm = [t.numpy() for t in sub]
        npb, n = w["np_list"][b], w["tail_list"][b]
        for pg in range(npb):            # the reference's discarded first pass (attention.py:100-132)
            for h in range(w["Hkv"]):
                O.dequantize_key(skb[pg, h], skh[pg, h], skm[pg, h, 0], skm[pg, h, 1], bin_[h], w["dk"])
                O.dequantize_value(svp[pg, h], svm[pg, h, :, 0], svm[pg, h, :, 1])
        O.paged_attention(q[b], np.arange(npb, dtype=np.int32), skb, skh, skm, svp, svm, bin_, w["dk"], sk[b],
                          sv[b], tk[b, :, :n], tv[b, :, :n], w["Hq"], w["Hkv"], D, n_threads=1)
    r = _cpu_sequences(w, budget_s, run_one)
    return {"value": round(r["value"] * 1e6, 1), "unit": "us/layer-step", "cores": 1, "kind": "port",
            **host_cpu(),
            "sample": f"{r['done']} of {w['B']} sequences ({r['pages_done']} of {r['total_pages']} pages) through "
                      f"oracle/kitty_oracle.c (paged_attention_reference restated in scalar C, with its "
                      f"discarded first pass), single thread; scaled by pages to one layer-step"}


def host_cpu() -> dict:
    """Host CPU of this run: /proc/cpuinfo's model string with its family,
    model and stepping numbers (a virtualised host may shorten the string),
    and the threads the OS offers."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break                      # first processor only
                k, _, v = line.partition(":")
                info[k.strip()] = v.strip()
    except OSError:
        pass
    model = info.get("model name", "unknown")
    ident = "family {} model {} stepping {}".format(info.get("cpu family", "?"), info.get("model", "?"),
                                                    info.get("stepping", "?"))
    return {"cpu_model": f"{model} ({info.get('vendor_id', '?')} {ident})", "host_threads": os.cpu_count()}


def quantize_cpu_baseline(k, v, bi, dk: int) -> dict:
    """Oracle C port of quantize_key_page_torch / quantize_value_page_torch,
    one thread, over every block of one config-2 batch (256 key + 256 value
    blocks; a few hundred ms)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    O.build()
    kc, vc, bic = k.cpu().numpy(), v.cpu().numpy(), bi.cpu().numpy()   # (T, H, D), (H, D)
    T, H, _ = kc.shape
    t0 = time.perf_counter()
    for p0 in range(0, T, G):
        for h in range(H):
            O.quantize_key(kc[p0:p0 + G, h].T, bic[h], dk, dk + 1)     # the reference quantises (D, G) keys
            O.quantize_value(vc[p0:p0 + G, h])
    us = (time.perf_counter() - t0) * 1e6
    return {"value": round(us, 1), "unit": "us/batch", "cores": 1, "kind": "port", **host_cpu(),
            "sample": f"all {T // G * H} key + {T // G * H} value blocks of one config-2 batch through "
                      f"oracle/kitty_oracle.c (quantize_key_page_torch / quantize_value_page_torch restated), "
                      f"single thread"}


def quantize_cpu_baseline_torch(k, v, bi, dk: int) -> dict:
    """The reference's quantize_key_page_torch / quantize_value_page_torch,
    restated op for op in torch (oracle/torch_reference.py), over every block
    of one config-2 batch with every thread torch may use here (the
    reference's key loop takes each (D, G) block, its value loop each (G, D)
    block, one call per (page, head))."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch
    import torch_reference as TR
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        kc, vc, bic = k.cpu(), v.cpu(), bi.cpu()                        # (T, H, D), (H, D)
        T, H, _ = kc.shape
        t0 = time.perf_counter()
        for p0 in range(0, T, G):
            for h in range(H):
                TR.quantize_key_page(kc[p0:p0 + G, h].T.contiguous(), bic[h], dk, dk + 1)   # pipeline.py:219
                TR.quantize_value_page(vc[p0:p0 + G, h])
        us = (time.perf_counter() - t0) * 1e6
    finally:
        torch.set_num_threads(prev)
    return {"value": round(us, 1), "unit": "us/batch", "cores": threads, "kind": "port", **host_cpu(),
            "sample": f"all {T // G * H} key + {T // G * H} value blocks of one config-2 batch through "
                      f"oracle/torch_reference.py (quantize_key_page_torch / quantize_value_page_torch restated "
                      f"op for op in torch, CPU, {threads} threads)"}


def bench_quantize(torch, dev, reps: int = 64, cpu: bool = False) -> dict:
    """4096 tokens x 8 KV heads x 128, batch quantize + pack.
    Sixteen input / output sets (309 MB, more than the 256 MB MALL) rotate;
    `reps` launches are enqueued back to back between two HIP events
    (pre-built arguments, so the GPU never waits for the host); the mean per
    launch of the median of five such bursts is reported."""
    from kitty.kernels.ops import QuantizePlan, pool_store
    T, H, dk, sets = 4096, 8, 16, 16
    n = T // G
    g = torch.Generator(device=dev).manual_seed(2)
    pools = [torch.empty(n * sets, H, D, G // 4, dtype=torch.uint8, device=dev),
             torch.empty(n * sets, H, dk, G // 4, dtype=torch.uint8, device=dev),
             torch.empty(n * sets, H, 2, D, dtype=torch.float16, device=dev),
             torch.empty(n * sets, H, G, D // 4, dtype=torch.uint8, device=dev),
             torch.empty(n * sets, H, G, 2, dtype=torch.float16, device=dev)]
    store = pool_store(*pools)
    gcpu = torch.Generator().manual_seed(2)
    bi = torch.full((H, D), dk + 1, dtype=torch.uint8)
    scale = torch.ones(H, D)
    for h in range(H):
        ch = torch.randperm(D, generator=gcpu)[:dk]   # the head's outlier channels, quantised to INT4
        bi[h, ch] = torch.arange(dk, dtype=torch.uint8)
        scale[h, ch] = 8.0
    bi, scale = bi.to(dev), scale.to(dev)
    plans = []
    for i in range(sets):
        k = (torch.randn(T, H, D, device=dev, generator=g) * scale).half()
        v = torch.randn(T, H, D, device=dev, generator=g).half()
        pids = torch.arange(i * n, (i + 1) * n, dtype=torch.int32, device=dev)
        if i == 0:
            k0, v0 = k, v
        plans.append(QuantizePlan(store, k.view(n, G, H, D).permute(0, 2, 1, 3),
                                  v.view(n, G, H, D).permute(0, 2, 1, 3), bi, pids, dk + 1))
    for p in plans:
        p.run()
    torch.cuda.synchronize()

    def burst() -> float:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            plans[i % sets].run()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3
    us = statistics.median(burst() for _ in range(5))
    cpu_base = quantize_cpu_baseline_torch(k0, v0, bi, dk) if cpu else None
    cpu_port = quantize_cpu_baseline(k0, v0, bi, dk) if cpu else None
    read = 2 * T * H * D * 2
    written = n * H * (D * G // 4 + dk * G // 4 + 2 * D * 2 + G * D // 4 + G * 2 * 2)
    out = {"workload": "cfg2: 4096 tok x 8 KV heads x 128, 16 x8 outlier key channels per head as INT4",
           "us": round(us, 2),
           "GBps": round((read + written) / us / 1e3, 1), "frac": round((read + written) / us / 1e3 / HBM_PEAK_GBPS, 4),
           "bytes_read": read, "bytes_written": written}
    if cpu_base:
        out["cpu_baseline"] = cpu_base
        out["cpu_baseline_c_port"] = cpu_port
    return out


def module_leg(torch, dev, cfg_name: str = "cfg3", cycles: int = 2, event_cycles: int = 4) -> dict:
    """KittyPagedAttention.forward decode steps at a config's shape, the
    drop-in module path: per step one token of every sequence through the
    pipeline (append; key and value spills every G steps) and the fused
    decode over key pages, value pages (128-token value window) and FP16
    tails.  Sequences are prefilled to ctx - 2G tokens with push_chunk and
    run G untimed steps (one spill cycle: the first launch of every kernel
    and the first pinned staging buffer are set-up costs), then `cycles` x G
    steps are timed back to back (host clock, events on the stream), so each
    sequence spills its keys and values `cycles` times.  A last pass of
    `event_cycles` x G steps with an event per step separates the spill steps
    (the median over its cycles of each cycle's slowest step)."""
    from kitty import KittyConfig, KittyAttentionFactory
    c = CONFIGS[cfg_name]
    B, Hq, Hkv, ctx = c["B"], c["Hq"], c["Hkv"], c["ctx"]
    kcfg = KittyConfig(num_layers=1, num_kv_heads=Hkv, head_dim=D, q_buffer_size=G, sink_size=S,
                       local_value_window=128, boost_rate=c["boost"], max_seq_len=ctx + (cycles + event_cycles + 1) * G,
                       max_batch_size=B, device=str(dev))
    gen = torch.Generator(device="cpu").manual_seed(c["seed"])
    dk = kcfg.d_boost
    bi = torch.full((1, Hkv, D), kcfg.sentinel, dtype=torch.uint8)
    scale = torch.ones(Hkv, D)
    for h in range(Hkv):
        ch = torch.randperm(D, generator=gen)[:dk]
        bi[0, h, ch] = torch.arange(dk, dtype=torch.uint8)
        scale[h, ch] = c["outlier"]
    layout, pipe, layers = KittyAttentionFactory.from_config(kcfg, bi, Hq)
    attn = layers[0]
    g = torch.Generator(device=dev).manual_seed(c["seed"] + 200)
    scale = scale.to(dev)
    pre = ctx - 2 * G                   # warm-up and timed steps take every sequence across ctx
    chunk = 4096
    for t0 in range(0, pre, chunk):
        n = min(chunk, pre - t0)
        k = (torch.randn(B, Hkv, n, D, device=dev, generator=g) * scale[None, :, None, :]).half()
        v = torch.randn(B, Hkv, n, D, device=dev, generator=g).half()
        pipe.push_chunk(0, k, v, list(range(B)))
    steps = cycles * G
    qs = torch.randn(steps, B, Hq, 1, D, device=dev, generator=g).half()
    ks = (torch.randn(steps, B, Hkv, 1, D, device=dev, generator=g) * scale[None, None, :, None, :]).half()
    vs = torch.randn(steps, B, Hkv, 1, D, device=dev, generator=g).half()
    torch.cuda.synchronize()
    seq_ids = list(range(B))
    # one untimed spill cycle: builds and caches the decode plan, first launches
    for i in range(G):
        attn(qs[i % steps], ks[i % steps], vs[i % steps], seq_id=seq_ids)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        attn(qs[i], ks[i], vs[i], seq_id=seq_ids)
    e1.record()
    torch.cuda.synchronize()
    n_t = steps
    wall_us = (time.perf_counter() - t0) * 1e6 / n_t
    event_us = e0.elapsed_time(e1) * 1e3 / n_t
    # per-step events over event_cycles more cycles of G steps: spill steps vs the rest
    n_ev = event_cycles * G
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev + 1)]
    torch.cuda.synchronize()
    slot0 = pipe.slot(seq_ids[0])
    spills = []
    ev[0].record()
    for i in range(n_ev):
        # the sequences run in lockstep: this step spills them all when the
        # first one's key or value buffer is one token from full
        spills.append(int(pipe._qlen[slot0, 0]) + 1 == G or int(pipe._vlen[slot0, 0]) + 1 == pipe.value_capacity)
        attn(qs[i % steps], ks[i % steps], vs[i % steps], seq_id=seq_ids)
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(n_ev)]
    assert sum(spills) >= event_cycles, "a spill step in every cycle"
    med = statistics.median(p for p, sp in zip(per, spills) if not sp)
    spill_us = statistics.median(p for p, sp in zip(per, spills) if sp)
    # the largest step of each cycle, spill or not (host noise: collector pauses, scheduling)
    worst = statistics.median(max(per[j * G:(j + 1) * G]) for j in range(event_cycles))
    plan = attn._plans.get(tuple(range(B)))
    assert plan is not None, "the decode plan is cached across steps"
    del layers, attn, pipe, layout, qs, ks, vs
    torch.cuda.empty_cache()
    return {"workload": f"KittyPagedAttention.forward decode, {cfg_name} shape: B{B} Hq{Hq} Hkv{Hkv} d{D}, "
                        f"contexts {ctx - G + 1}..{ctx + (cycles - 1) * G}, S{S} G{G} R128 "
                        f"{int(c['boost'] * 1000) / 10}% INT4 keys",
            "us_per_step": round(wall_us, 2), "us_per_step_events": round(event_us, 2), "steps": n_t,
            "step_us_median": round(med, 2), "spill_step_us": round(spill_us, 2),
            "spill_step_extra_us": round(spill_us - med, 2), "spill_steps_timed": sum(spills),
            "cycle_max_step_us": round(worst, 2),
            "note": "each step: append of all B tokens; every G steps a spill (one kitty_store_i32 launch for "
                    "the new pages' ids, block-table entries and counters, then one batch-quantize launch of "
                    "B*Hkv key and B*Hkv value blocks whose value blocks also shift the 128-token value window); "
                    "decode with independent key/value streams (page-pair split kernel, key-only pages in its "
                    "FP16 segments) and merge.  step_us_median: median event time of the steps without a spill; "
                    "spill_step_us: median of the spill steps; cycle_max_step_us: median over cycles of each "
                    "cycle's largest step, spill or not (host noise included); host clock over the timed steps "
                    "includes the Python module overhead"}


def module_leg_cpu(torch, cfg_name: str = "cfg1", steps: int = 256) -> dict:
    """KittyPagedAttention.forward decode steps with every tensor on the CPU
    (the product's own CPU path, kitty/kernels/cpu.py: quantise, spills and
    decode in torch), at config 1's shape: one sequence prefilled to
    ctx - 2G tokens with push_chunk, then `steps` decode steps (two spill
    cycles), host clock, on every thread torch may use here."""
    from kitty import KittyConfig, KittyAttentionFactory
    c = CONFIGS[cfg_name]
    B, Hq, Hkv, ctx = c["B"], c["Hq"], c["Hkv"], c["ctx"]
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        kcfg = KittyConfig(num_layers=1, num_kv_heads=Hkv, head_dim=D, q_buffer_size=G, sink_size=S,
                           local_value_window=128, boost_rate=c["boost"], max_seq_len=ctx + 4 * G,
                           max_batch_size=B, device="cpu")
        gen = torch.Generator().manual_seed(c["seed"])
        bi = torch.full((1, Hkv, D), kcfg.sentinel, dtype=torch.uint8)
        for h in range(Hkv):
            bi[0, h, torch.randperm(D, generator=gen)[:kcfg.d_boost]] = torch.arange(kcfg.d_boost, dtype=torch.uint8)
        layout, pipe, layers = KittyAttentionFactory.from_config(kcfg, bi, Hq)
        attn = layers[0]
        k = torch.randn(B, Hkv, ctx - 2 * G, D, generator=gen).half()
        v = torch.randn(B, Hkv, ctx - 2 * G, D, generator=gen).half()
        pipe.push_chunk(0, k, v, list(range(B)))
        qs = torch.randn(steps, B, Hq, 1, D, generator=gen).half()
        ks = torch.randn(steps, B, Hkv, 1, D, generator=gen).half()
        vs = torch.randn(steps, B, Hkv, 1, D, generator=gen).half()
        per = []
        for i in range(steps):
            t0 = time.perf_counter()
            attn(qs[i], ks[i], vs[i], seq_id=list(range(B)))
            per.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    return {"workload": f"KittyPagedAttention.forward decode on CPU tensors, {cfg_name} shape: B{B} Hq{Hq} Hkv{Hkv} "
                        f"d{D}, contexts {ctx - 2 * G + 1}..{ctx - 2 * G + steps}, S{S} G{G} R128",
            "us_per_step": round(sum(per) / steps * 1e6, 1), "us_per_step_median": round(statistics.median(per) * 1e6, 1),
            "steps": steps, "cores": threads, **host_cpu(),
            "note": "kitty/kernels/cpu.py through the module and pipeline (no oracle): bit-exact quantisation, "
                    "fp32 decode; host clock per step"}


def spill_latency(torch, dev, B: int = 16, Hkv: int = 8, dk: int = 16, reps: int = 64) -> dict:
    """The pipeline's spill launches at their production shape: one
    kitty_quantize_kv_blocks launch over the B * Hkv (G x D) blocks of one
    layer (config-3 batch): key and value into the same pages (R = 0), key
    only, value only, and the spill of the 128-token value window as the
    pipeline makes it (keys into new pages, values into their own pages, the
    value blocks then shifting the window's 128 newest rows to the front of
    the 256-row value buffer), each timed as bursts of `reps` back-to-back
    launches over 8 rotating input / page sets."""
    from kitty.kernels.ops import QuantizePlan, pool_store
    sets = 8
    n = B * sets
    pools = [torch.empty(n, Hkv, D, G // 4, dtype=torch.uint8, device=dev),
             torch.empty(n, Hkv, dk, G // 4, dtype=torch.uint8, device=dev),
             torch.empty(n, Hkv, 2, D, dtype=torch.float16, device=dev),
             torch.empty(n, Hkv, G, D // 4, dtype=torch.uint8, device=dev),
             torch.empty(n, Hkv, G, 2, dtype=torch.float16, device=dev)]
    store = pool_store(*pools)
    g = torch.Generator(device=dev).manual_seed(9)
    bi = torch.full((Hkv, D), dk + 1, dtype=torch.uint8)
    for h in range(Hkv):
        bi[h, torch.randperm(D, generator=torch.Generator().manual_seed(h))[:dk]] = torch.arange(dk, dtype=torch.uint8)
    bi = bi.to(dev)
    res = {}
    R = 128
    for kind in ("key+value", "key only", "value only", "window spill"):
        plans = []
        for i in range(sets):
            k = torch.randn(B, Hkv, G, D, device=dev, generator=g).half()
            v = torch.randn(B, Hkv, G + (R if kind == "window spill" else 0), D, device=dev, generator=g).half()
            pids = torch.arange(i * B, (i + 1) * B, dtype=torch.int32, device=dev)
            if kind == "window spill":
                vids = torch.arange(n - (i + 1) * B, n - i * B, dtype=torch.int32, device=dev)
                plans.append(QuantizePlan(store, k, v[:, :, :G], bi, pids, dk + 1, value_page_ids=vids,
                                          value_shift=R))
                continue
            plans.append(QuantizePlan(store, k if kind != "value only" else None,
                                      v if kind != "key only" else None,
                                      bi if kind != "value only" else None, pids, dk + 1))
        for p in plans:
            p.run()
        torch.cuda.synchronize()

        def burst() -> float:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(reps):
                plans[i % sets].run()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / reps * 1e3
        res[kind] = round(statistics.median(burst() for _ in range(5)), 2)
    return {"blocks": B * Hkv, "us_per_launch": res,
            "workload": f"{B * Hkv} blocks of {G} tokens x {D} channels (B{B} x Hkv{Hkv}, one layer), {dk} INT4 "
                        f"key channels"}


def copy_probe(torch, dev) -> int:
    """A device-to-device copy of known size: its FETCH_SIZE / WRITE_SIZE
    counters per dispatch calibrate the decode kernel's counter readings."""
    n = 256 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "dispatches": 5}), flush=True)
    return 0


def time_decode(torch, plans, steps: int, warm_steps: int, warm_s: float) -> dict:
    """Steady-state timing of kitty_paged_decode steps (split + merge).

    Warm-up: at least warm_steps steps and warm_s seconds of them, so the GPU
    clock has settled whatever --steps is.  `value`: exactly `steps`
    back-to-back steps between two HIP events and by the host clock.  Kernel
    times, right after at the same settled clock: five bursts of at least 100
    back-to-back launches of the split kernel, then of the merge kernel,
    each burst between two HIP events on the launch stream (median burst,
    mean per launch).  A last pass of alternating steps with an event
    around every launch gives per-launch times in the exact step pattern;
    each marker adds a few microseconds, so those are upper bounds."""
    n = len(plans)
    t_end = time.perf_counter() + warm_s
    i = 0
    while i < warm_steps or time.perf_counter() < t_end:
        plans[i % n].run()
        i += 1
        if i % 256 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    warm_done = i
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        plans[i % n].run()
    e1.record()
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - t0) * 1e6 / steps
    event_us = e0.elapsed_time(e1) * 1e3 / steps

    def burst(fn, k) -> float:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for i in range(k):
            fn(plans[i % n])
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / k
    kb = max(steps, 100)
    kernel_us = statistics.median(burst(lambda p: p.run_splits(), kb) for _ in range(5))
    merge_us = statistics.median(burst(lambda p: p.run_merge(), kb) for _ in range(5))
    m = max(steps, 200)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * m + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(m):
        p = plans[i % n]
        p.run_splits()
        ev[2 * i + 1].record()
        p.run_merge()
        ev[2 * i + 2].record()
    torch.cuda.synchronize()
    split = [ev[2 * i].elapsed_time(ev[2 * i + 1]) * 1e3 for i in range(m)]
    merge = [ev[2 * i + 1].elapsed_time(ev[2 * i + 2]) * 1e3 for i in range(m)]
    step_inst = ev[0].elapsed_time(ev[2 * m]) * 1e3 / m
    # the split kernel is part of every step: its time cannot exceed the step's
    assert kernel_us <= event_us, (kernel_us, event_us)
    return dict(wall_us=wall_us, event_us=event_us, kernel_us=kernel_us, merge_us=merge_us,
                kernel_event_us=sum(split) / m, merge_event_us=sum(merge) / m,
                step_instrumented_us=step_inst, instrumented_steps=m, burst_launches=kb, warm_steps=warm_done,
                warm_s=warm_s)


def decode_leg(torch, dev, name: str, copies: int, placement: str, steps: int, warm_steps: int,
               warm_s: float, keep: bool = False):
    """One decode workload: build it, time it, return (record, workload)."""
    cfg = CONFIGS[name]
    log(f"building {name} workload ({copies} pool copies)")
    w = build_workload(torch, dev, cfg, copies, placement)
    nb = algorithmic_bytes(w)
    log(f"{name}: pool {w['P']} pages, {nb['packed'] / 1e6:.1f} MB packed KV per step")
    t = time_decode(torch, w["plans"], steps, warm_steps, warm_s)
    log(f"{name}: {t['wall_us']:.1f} us/step wall ({t['event_us']:.1f} by events); split kernel "
        f"{t['kernel_us']:.1f} us, merge {t['merge_us']:.1f} us (bursts); per-launch events "
        f"{t['kernel_event_us']:.1f} / {t['merge_event_us']:.1f} us in a {t['step_instrumented_us']:.1f} us step")
    kernel_us = t["kernel_us"]
    achieved = nb["total"] / (kernel_us * 1e-6) / 1e9
    packed_gbps = nb["packed"] / (kernel_us * 1e-6) / 1e9
    step_packed = nb["packed"] / (t["wall_us"] * 1e-6) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"decode_{name}_traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    GQ = cfg["Hq"] // cfg["Hkv"]
    rec = {
        "value": round(t["wall_us"], 2), "unit": "us/layer-step", "step_us_events": round(t["event_us"], 2),
        "workload": f"{name}: B{cfg['B']} Hq{cfg['Hq']} Hkv{cfg['Hkv']} d{D} ctx{cfg['ctx']} S{S} G{G} "
                    f"{int(cfg['boost'] * 100 * 10) / 10}% INT4 keys, INT2 values",
        "pages_per_seq": w["n_pages"] if len(set(w["np_list"])) == 1 else sum(w["np_list"]) / cfg["B"],
        "tail_tokens": w["n_tail"], "pool_copies": len(w["plans"]),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": f"decode_mfma_kernel<{GQ}> (split-K phase of kitty_paged_decode)",
                     "kernel_us": round(kernel_us, 2), "merge_us": round(t["merge_us"], 2),
                     "burst_launches": t["burst_launches"],
                     "kernel_event_us": round(t["kernel_event_us"], 2),
                     "merge_event_us": round(t["merge_event_us"], 2),
                     "step_instrumented_us": round(t["step_instrumented_us"], 2),
                     "instrumented_steps": t["instrumented_steps"], "warmup_steps": t["warm_steps"],
                     "warmup_s": t["warm_s"],
                     "algorithmic_bytes": nb["total"], "packed_kv_bytes": nb["packed"],
                     "packed_kv_GBps": round(packed_gbps, 1),
                     "packed_kv_frac": round(packed_gbps / HBM_PEAK_GBPS, 4),
                     "step_packed_kv_frac": round(step_packed / HBM_PEAK_GBPS, 4)},
    }
    return rec, (w if keep else None)


def window_leg(torch, w, steps: int, warm_steps: int, warm_s: float, R: int = 128) -> dict:
    """Config 3's step in the layout the pipeline really decodes with an
    R-token FP16 value window (the reference's KIVI split, local_value_window
    = 128): every key page is packed, the newest value page is not, so each
    sequence reads num_pages key pages, num_pages - 1 value pages and an
    R + tail token FP16 value tail.  Same pools, block tables and query as
    the headline leg; decode-only (split + merge), timed like it."""
    from kitty.kernels.ops import DecodePlan
    dev = w["q"].device
    B, Hkv = w["B"], w["Hkv"]
    g = torch.Generator(device=dev).manual_seed(33)
    tv = torch.randn(B, Hkv, R + w["n_tail"], D, device=dev, generator=g).half()
    npg = torch.tensor(w["np_list"], dtype=torch.int32, device=dev)
    npv = npg - R // G
    tl = torch.tensor(w["tail_list"], dtype=torch.int32, device=dev)
    tlv = tl + R
    sl = torch.full((B,), S, dtype=torch.int32, device=dev)
    kb, kh, km, vp, vm = w["pools"]
    out = torch.empty_like(w["out"])
    plans = [DecodePlan(w["q"], bt, npg, kb, kh, km, vp, vm, w["bi"], w["sk"], w["sv"], sl, w["tk"], tv, tl,
                        out=out, num_pages_v=npv, tail_len_v=tlv) for bt in w["tables"]]
    t = time_decode(torch, plans, steps, warm_steps, warm_s)
    pages = sum(w["np_list"])
    key_part = D * G // 4 + w["dk"] * G // 4 + 2 * D * 2
    val_part = G * D // 4 + G * 2 * 2
    packed = Hkv * (pages * key_part + (pages - B * (R // G)) * val_part)
    fp16 = Hkv * sum(2 * (S + x) + R for x in w["tail_list"]) * D * 2
    small = B * w["Hq"] * D * 2 + pages * 4 + Hkv * D + 5 * B * 4
    total = packed + fp16 + small
    achieved = total / (t["kernel_us"] * 1e-6) / 1e9
    log(f"value window R={R}: {t['wall_us']:.1f} us/step wall; split kernel {t['kernel_us']:.1f} us, "
        f"merge {t['merge_us']:.1f} us")
    return {"value": round(t["wall_us"], 2), "unit": "us/layer-step", "step_us_events": round(t["event_us"], 2),
            "workload": f"cfg3 with a {R}-token FP16 value window: per sequence {w['n_pages']} key pages, "
                        f"{w['n_pages'] - R // G} value pages, {S} sinks, {w['n_tail']}-token key tail and "
                        f"{R + w['n_tail']}-token value tail",
            "kernel_us": round(t["kernel_us"], 2), "merge_us": round(t["merge_us"], 2),
            "algorithmic_bytes": total, "packed_kv_bytes": packed,
            "achieved_GBps": round(achieved, 1), "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "step_packed_kv_frac": round(packed / (t["wall_us"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


def _host_median_ms(torch, fn, runs: int) -> float:
    """Median wall-clock ms of fn() with a synchronisation before and after
    every call (the reference benchmark's _timed_runs,
    benchmark/benchmark_kitty_hardware.py:60-70)."""
    times = []
    for _ in range(runs):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


def _device_us(torch, fn, reps: int = 100) -> float:
    """Mean µs per call of `reps` back-to-back calls between two HIP events
    (median of five bursts): the device time without the host round trip."""
    def burst() -> float:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3
    return statistics.median(burst() for _ in range(5))


def reference_items(torch, dev, runs: int = 100) -> dict:
    """The reference's own benchmark (benchmark/benchmark_kitty_hardware.py)
    on this build, with its defaults (32 layers, 8 KV heads, D = G = 128,
    boost rate 0.125, 8,192-token sequences, :330-352) and its timing (each
    call between two synchronisations, median of `runs`): one-page key
    quantise (:110-147) and dequantise (:159-193) through the
    reference-signature wrappers, push_token throughput for one sequence on
    layer 0 with the same random tokens drawn per step (:200-241), and the
    memory compression against an FP16 cache (:85-107).  The time per call of
    back-to-back calls between HIP events is reported beside the host figures
    (`back_to_back_us`): it is bound by the Python wrappers (reference
    signatures, one call per page), not by the kernels, whose durations are in
    the rocprofv3 kernel trace."""
    from kitty import KittyConfig, KittyInferencePipeline, PageCentricKVLayoutManager
    from kitty.kernels.dequantize_key import dequantize_key_page
    from kitty.kernels.quantize_key import quantize_key_page
    cfg = KittyConfig(num_layers=32, num_kv_heads=8, head_dim=128, boost_rate=0.125, max_seq_len=8192,
                      device=str(dev))
    D, G, K, sent = cfg.head_dim, cfg.q_buffer_size, cfg.d_boost, cfg.sentinel
    bi = torch.full((D,), sent, dtype=torch.uint8, device=dev)
    bi[:K] = torch.arange(K, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev).manual_seed(11)
    key = torch.randn(D, G, dtype=torch.float16, device=dev, generator=g)
    ob = torch.zeros(D, G // 4, dtype=torch.uint8, device=dev)
    oh = torch.zeros(K, G // 4, dtype=torch.uint8, device=dev)
    osc = torch.zeros(D, dtype=torch.float16, device=dev)
    oz = torch.zeros(D, dtype=torch.float16, device=dev)
    out16 = torch.zeros(D, G, dtype=torch.float16, device=dev)

    def quant():
        quantize_key_page(key, bi, K, sent, ob, oh, osc, oz)

    def dequant():
        dequantize_key_page(ob, oh, osc, oz, bi, K, out16)

    res = {"config": "reference benchmark defaults: 32 layers, 8 KV heads, D = G = 128, boost 0.125, "
                     "max_seq_len 8192", "runs": runs}
    for name, fn, nbytes in (("quantize_key_page", quant, D * G * 2), ("dequantize_key_page", dequant, D * G * 2)):
        for _ in range(5):
            fn()
        ms = _host_median_ms(torch, fn, runs)
        res[name] = {"latency_ms": round(ms, 4), "bandwidth_GBps": round(nbytes / (ms * 1e-3) / 1e9, 3),
                     "back_to_back_us": round(_device_us(torch, fn), 2)}

    L, H, T = cfg.num_layers, cfg.num_kv_heads, cfg.max_seq_len
    bidx = torch.full((L, H, D), sent, dtype=torch.uint8, device=dev)
    bidx[:, :, :K] = torch.arange(K, dtype=torch.uint8, device=dev)
    layout = PageCentricKVLayoutManager(cfg, bidx)
    pipe = KittyInferencePipeline(cfg, layout, bidx)

    def token():
        k = torch.randn(H, D, dtype=torch.float16, device=dev, generator=g)
        v = torch.randn(H, D, dtype=torch.float16, device=dev, generator=g)
        pipe.push_token(layer_id=0, key=k, value=v, seq_id=0)

    for _ in range(cfg.sink_size):
        token()
    steps = min(500, cfg.max_seq_len - cfg.sink_size - 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        token()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    # the same again over the sequence's next tokens: first-use costs (the
    # pipeline's first spill, pinned staging) are behind it
    steps2 = min(steps, cfg.max_seq_len - cfg.sink_size - steps - 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps2):
        token()
    torch.cuda.synchronize()
    el2 = time.perf_counter() - t0
    res["decode_throughput"] = {"num_steps": steps, "tokens_per_sec": round(steps / el, 1),
                                "ms_per_token": round(el * 1e3 / steps, 4),
                                "tokens_per_sec_second_pass": round(steps2 / el2, 1) if steps2 > 0 else None,
                                "note": "push_token of one sequence, layer 0 (append, spills every G tokens), "
                                        "the reference's method (sinks filled first, two randn per token "
                                        "inside the timed loop); a second pass over the next tokens"}
    mem = layout.memory_stats()
    S, R = cfg.sink_size, cfg.local_value_window
    fp16_bytes = L * 2 * H * T * D * 2
    kitty = mem["total_MB"] * 1024 ** 2 + L * 2 * H * (S + G + R) * D * 2
    res["memory_compression"] = {"fp16_cache_MB": round(fp16_bytes / 1024 ** 2, 1),
                                 "kitty_total_MB": round(kitty / 1024 ** 2, 1),
                                 "compression_ratio": round(fp16_bytes / kitty, 3)}
    return res


def widened_rows(torch, dev, B: int = 16, T: int = 4096, reps: int = 20) -> dict:
    """The rows next to the decode path at production shapes: prefill (one
    push_chunk of T prompt tokens for each of B sequences, one layer, 8 KV
    heads x 128: sinks, (T - S) // G key pages quantised, FP16 buffers
    written; pipeline.py push_chunk) and the profiler's |K| accumulation (one
    kitty_channel_abs_sum launch over a (B, 8, T, 128) fp16 key tensor;
    sensitivity.py:46-61), each as time per call and GB/s of fp16 input."""
    from kitty import KittyConfig, KittyInferencePipeline, PageCentricKVLayoutManager
    from kitty.sensitivity import _ChannelAccumulator
    H, D = 8, 128
    g = torch.Generator(device=dev).manual_seed(12)
    keys = torch.randn(B, H, T, D, dtype=torch.float16, device=dev, generator=g)
    values = torch.randn(B, H, T, D, dtype=torch.float16, device=dev, generator=g)
    res = {"shape": f"B{B} x Hkv{H} x T{T} x D{D} fp16, one layer"}

    import ctypes
    from kitty import _hip
    acc = _ChannelAccumulator(H, D, dev)
    for _ in range(3):
        acc.update(keys)
    us_module = _device_us(torch, lambda: acc.update(keys), reps)
    L = _hip.load()
    need = ctypes.c_size_t(0)
    _hip.check(L.kitty_channel_abs_sum_workspace_size(B, T, H, D, ctypes.byref(need)))
    ws = torch.empty(max(need.value, 16), dtype=torch.uint8, device=dev)
    sums = torch.zeros(H, D, dtype=torch.float32, device=dev)
    args = (keys.data_ptr(), keys.stride(0), keys.stride(2), keys.stride(1), B, T, H, D, _hip.KITTY_DTYPE_F16,
            sums.data_ptr(), ws.data_ptr(), need.value, _hip.stream_ptr(dev))
    us = _device_us(torch, lambda: L.kitty_channel_abs_sum(*args), reps)
    nbytes = keys.numel() * 2
    _hip.check(L.kitty_channel_abs_sum_deferred_size(H, D, ctypes.byref(need)))
    slots = torch.zeros(need.value, dtype=torch.uint8, device=dev)
    dargs = args[:10] + (slots.data_ptr(), need.value, args[12])
    us_def = _device_us(torch, lambda: L.kitty_channel_abs_sum_deferred(*dargs), reps)
    us_flush = _device_us(torch, lambda: L.kitty_channel_abs_sum_flush(slots.data_ptr(), H, D, sums.data_ptr(),
                                                                       args[12]), reps)
    res["profiler_abs_sum"] = {"us": round(us, 2), "GBps": round(nbytes / us / 1e3, 1),
                               "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBPS, 4), "bytes_read": nbytes,
                               "us_deferred_update": round(us_def, 2),
                               "frac_deferred_update": round(nbytes / us_def / 1e3 / HBM_PEAK_GBPS, 4),
                               "us_flush": round(us_flush, 2),
                               "us_via_accumulator_update": round(us_module, 2),
                               "note": "kitty_channel_abs_sum (two kernels) back to back with pre-built "
                                       "arguments; kitty_channel_abs_sum_deferred (first pass into per-chunk "
                                       "slots, what _ChannelAccumulator.update runs) and the flush that "
                                       "finishes it once per read; the Python update() path"}

    cfg = KittyConfig(num_layers=1, num_kv_heads=H, head_dim=D, boost_rate=0.125, max_seq_len=T + 256,
                      max_batch_size=B, device=str(dev))
    bidx = torch.full((1, H, D), cfg.sentinel, dtype=torch.uint8, device=dev)
    bidx[:, :, :cfg.d_boost] = torch.arange(cfg.d_boost, dtype=torch.uint8, device=dev)
    layout = PageCentricKVLayoutManager(cfg, bidx)
    pipe = KittyInferencePipeline(cfg, layout, bidx)
    seqs = list(range(B))

    def prefill():
        """One push_chunk of new sequences (the B resets before it untimed):
        host ms and device ms between two events on the launch stream."""
        for s in seqs:
            pipe.reset_sequence(s)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        pipe.push_chunk(0, keys, values, seqs)
        e1.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3, e0.elapsed_time(e1)

    for _ in range(2):
        prefill()
    runs = [prefill() for _ in range(reps)]
    ms = statistics.median(r[0] for r in runs)
    dev_ms = statistics.median(r[1] for r in runs)
    nbytes = 2 * keys.numel() * 2
    res["prefill_push_chunk"] = {"ms": round(ms, 3), "device_ms": round(dev_ms, 3),
                                 "tokens_per_sec": round(B * T / (ms * 1e-3)),
                                 "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                 "GBps_device": round(nbytes / (dev_ms * 1e-3) / 1e9, 1),
                                 "pages_per_seq": (T - cfg.sink_size) // cfg.q_buffer_size,
                                 "note": "median of host clock (ms) and of two HIP events (device_ms) around "
                                         "each push_chunk; the resets of the B sequences before it untimed; "
                                         "GB/s of fp16 prompt input"}
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warmup-seconds", type=float, default=1.0,
                    help="minimum seconds of decode steps before any timing (per leg)")
    ap.add_argument("--config", choices=sorted(CONFIGS), default="cfg3")
    ap.add_argument("--legs", default="cfg4,cfg5",
                    help="other decode configs timed after the main one, each with its own roofline "
                         "('' for none)")
    ap.add_argument("--copies", type=int, default=3)
    ap.add_argument("--placement", choices=["shuffled", "first-fit"], default="shuffled",
                    help="page ids: a shuffled free list (fragmented pool) or first-fit order of B sequences "
                         "growing in lockstep")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-quantize", action="store_true")
    ap.add_argument("--no-module", action="store_true", help="skip the KittyPagedAttention.forward leg")
    ap.add_argument("--no-window", action="store_true", help="skip the config-3 value-window decode leg")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the reference benchmark's items and the prefill / profiler rows")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    if args.copy_probe:
        return copy_probe(torch, dev)
    cfg = CONFIGS[args.config]
    main_rec, w = decode_leg(torch, dev, args.config, args.copies, args.placement, args.steps, args.warmup,
                             args.warmup_seconds, keep=True)
    K = args.steps
    result = {
        "metric": "decode-attn µs/layer + achieved HBM GB/s (% peak), 32Q/8KV d128 b16 32K ctx"
        if args.config == "cfg3" else f"decode-attn us/layer-step ({args.config})",
        "value": main_rec["value"],
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(main_rec["value"] / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: fp16 N(0,1) K/V with x{:g} outlier key channels, quantised on device".format(
            cfg["outlier"]),
        "config": {"workload": main_rec["workload"], "batch": cfg["B"],
                   "context": cfg["ctx"] if not isinstance(cfg["ctx"], tuple) else list(cfg["ctx"]),
                   "pages_per_seq": main_rec["pages_per_seq"], "tail_tokens": main_rec["tail_tokens"],
                   "pool_copies": main_rec["pool_copies"], "parallelism": "single GPU"},
        "step_us_events": main_rec["step_us_events"],
        "roofline": main_rec["roofline"],
    }
    if args.config == "cfg3" and not args.no_window:
        result["value_window_r128"] = window_leg(torch, w, K, args.warmup, max(0.5, args.warmup_seconds / 2))
    if not args.no_cpu_baseline:
        log(f"timing CPU baselines ({cpu_threads()} torch threads, then the C port on 1 thread)")
        result["cpu_baseline"] = cpu_baseline_torch(w, args.cpu_seconds)
        result["cpu_baseline_c_port"] = cpu_baseline_c(w, args.cpu_seconds * 2 / 3)
    del w
    torch.cuda.empty_cache()
    legs = {}
    for name in [x for x in args.legs.split(",") if x and x != args.config]:
        rec, lw = decode_leg(torch, dev, name, args.copies, args.placement, K, args.warmup,
                             max(0.5, args.warmup_seconds / 2), keep=not args.no_cpu_baseline)
        if lw is not None:
            log(f"{name}: sampled CPU baseline")
            rec["cpu_baseline"] = cpu_baseline_torch(lw, args.cpu_seconds / 3)
        del lw
        legs[name] = rec
        torch.cuda.empty_cache()
    if legs:
        result["legs"] = legs
    if not args.no_quantize:
        result["quantize_pack"] = bench_quantize(torch, dev, cpu=not args.no_cpu_baseline)
        result["spill"] = spill_latency(torch, dev)
    if not args.no_module:
        log("timing KittyPagedAttention.forward decode steps")
        result["module_forward"] = module_leg(torch, dev, "cfg3")
        result["module_forward_cfg1"] = module_leg(torch, dev, "cfg1")
        log("timing the module on CPU tensors (config 1)")
        result["module_forward_cfg1_cpu"] = module_leg_cpu(torch)
        if not args.no_cpu_baseline:
            result["cpu_baseline_cfg1"] = cpu_baseline_cfg1(torch, dev)
    if not args.no_extra:
        log("timing the reference benchmark's items, prefill and the profiler accumulation")
        result["reference_items"] = reference_items(torch, dev)
        torch.cuda.empty_cache()
        result["widened_rows"] = widened_rows(torch, dev)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
