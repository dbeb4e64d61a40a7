#!/usr/bin/env python3
"""Decode-step benchmark for the INT8 KV-cache decode-attention operator on one MI355X.

A step is what a serving loop runs per generated token at the configuration
named by BASELINE.json's metric (cfg1: B=8, H=32 MHA, d=128, L=4096): quantise
and append one new K/V token per (batch, head), then decode attention of one
query per head over the L cached tokens.  Both happen in one kernel launch
(kvq_decode_launch with a fused append).

Timing protocol:
  * inputs resident in HBM; the caches rotate over R replicas with
    R * KV_bytes >= 512 MiB (R >= 3) so steps read HBM, not the 256 MB
    Infinity Cache; a cache-warm single-replica figure is reported separately;
  * W untimed warm-up steps, then more untimed steps until --settle-ms of
    wall time has passed (sustained load first, so clocks and power state
    are at steady state), then exactly K steps between two HIP events on the
    launch stream, synchronised on both sides -> ms_per_step, value;
  * every step is exactly one launch of the decode kernel, so the timed
    region / K is that kernel's average duration -> roofline.achieved; a
    second pass brackets every launch with its own events (reported as
    kernel_us_isolated: launches spaced by the event records);
  * cpu_baseline: the CPU oracle (same fp32 math as the reference's
    cpu_reference, OpenMP over heads) on the host copy of the same step.

Prints ONE JSON line.  Only --gpus 1 is supported (this build runs on one GPU).
"""
from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
METRIC = "KV-cache read GB/s (% HBM peak) + us/decode step at B8 H32 d128 L4096"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=2000, help="untimed steps first")
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="after the warm-up steps, keep launching untimed steps until this much wall "
                         "time has passed since the warm-up began (MI355X runs this kernel ~15%% slower "
                         "during its first ~20 ms of sustained load than in steady state)")
    ap.add_argument("--config", default="cfg1", help="cfg0..cfg4 (default cfg1, the headline); cfg2m: cfg2's lengths with MHA")
    ap.add_argument("--splits", type=int, default=0, help="splits per sequence (0 = library choice)")
    ap.add_argument("--replicas", type=int, default=0, help="cache replicas (0 = enough for 512 MiB, >= 3)")
    ap.add_argument("--page-size", type=int, default=0,
                    help="run the same step through a paged cache with this many tokens per page "
                         "(0 = contiguous cache)")
    ap.add_argument("--page-order", choices=("shuffled", "sequential"), default="shuffled",
                    help="paged cache: pages scattered in a shuffled pool, or in sequence order")
    ap.add_argument("--seed", type=int, default=17)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="max seconds for the CPU baseline")
    ap.add_argument("--calib", action="store_true",
                    help="also run a plain 1 GiB copy kernel (PMC byte-counter calibration)")
    ap.add_argument("--traffic", default=os.path.join(REPO, "profiles", "traffic.json"),
                    help="measured HBM traffic summary (from rocprofv3 --pmc), if present")
    return ap.parse_args()


def cpu_baseline(prob, budget_s):
    """The oracle (fp32 reference math, OpenMP) on the host copy of one step."""
    import numpy as np
    from oracle import oracle as orc

    o = orc.get()
    h = lambda t: None if t is None else t.cpu().numpy()
    q, k, v, ks, vs = h(prob.q), h(prob.k), h(prob.v), h(prob.ks), h(prob.vs)
    kn, vn = h(prob.k_new), h(prob.v_new)
    lengths = prob.lengths_host.astype(np.int32)

    def step():
        if kn is not None:
            o.append(kn, vn, k, v, ks, vs, positions=lengths - 1)
        return o.decode_f32(q, k, v, ks, vs, lengths=lengths)

    step()  # warm-up
    times, t_start = [], time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < 2.0 and len(times) < 50):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    t = statistics.median(times)
    return {
        "value": round(prob.kv_bytes() / t / 1e9, 3),
        "unit": "GB/s",
        "cores": o.threads,
        "kind": "port",
        "sample": (f"full {prob.name} step ({'append + ' if kn is not None else ''}decode, "
                   f"{prob.B}x{prob.Hq} query heads), median of {len(times)} runs: {t * 1e6:.0f} us/step"),
    }


def paged_decoder(kvq, p, out, page, splits, seed, order="shuffled"):
    """The problem's cache moved into a pool of `page`-token pages, in shuffled
    order (block table = the shuffle) or in sequence order, wrapped in a
    PagedDecoder."""
    import torch

    B, Hkv, cap, d = p.k.shape
    npg = -(-cap // page)
    gen = torch.Generator().manual_seed(seed)
    perm = (torch.randperm(B * npg, generator=gen) if order == "shuffled" else torch.arange(B * npg)).to(p.k.device)

    def pool(x):  # [B, Hkv, cap, ...] -> [B * npg, Hkv, page, ...] in perm order
        pad = torch.zeros((B, Hkv, npg * page) + tuple(x.shape[3:]), dtype=x.dtype, device=x.device)
        pad[:, :, :cap] = x
        pages = pad.view((B, Hkv, npg, page) + tuple(x.shape[3:])).transpose(1, 2)
        pages = pages.reshape((B * npg, Hkv, page) + tuple(x.shape[3:]))
        dst = torch.empty(pages.shape, dtype=pages.dtype, device=pages.device)
        dst[perm] = pages
        return dst

    table = perm.view(B, npg).to(torch.int32).contiguous()
    dec = kvq.PagedDecoder(p.q, pool(p.k), pool(p.v), pool(p.ks), pool(p.vs), table, p.lengths, out,
                           max_seq_len=(0 if p.uniform else p.max_len) or p.cap, num_splits=splits,
                           k_new=p.k_new, v_new=p.v_new)
    return dec


def kernel_name(base, page):
    """The tuned kernel the library's planner picks for this problem."""
    G = base.Hq // base.Hkv
    mfma = base.d in (64, 128) and G % 4 == 0 and (page == 0 or (page & (page - 1) == 0 and page % 32 == 0))
    name = "decode_mfma" if mfma else "decode_fast"
    if base.uniform:
        return name
    # Ragged: a batch of <= 64 sequences that fits one round plans itself in
    # the kernel (matrix-core kernel, or the FMA kernel with <= 2 query heads
    # per kv head); otherwise a schedule_kernel launch precedes it.
    if mfma:
        U, slots = base.Hkv * (G // (8 if G % 8 == 0 else 4)), 256
    else:
        sg = 4 if G % 4 == 0 else (2 if G % 2 == 0 else 1)
        U, slots = (base.Hkv * (G // sg) if sg <= 2 else 0), 512
    if U and base.B <= 64 and base.B <= slots // U:
        return name + " (split plan in-kernel)"
    return name + " (+ schedule_kernel per step)"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(sharding across GPUs is designed, not built)", file=sys.stderr)
        sys.exit(2)

    import torch

    pkg = importlib.import_module("cuda-operators_amd")
    kvq = pkg.kvq
    synth = importlib.import_module("cuda-operators_amd.synth")
    kvq.lib()  # fail loudly if the HIP library is missing
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    base = synth.make(args.config, seed=args.seed, device="cuda")
    kv_bytes = base.kv_bytes()
    alloc_bytes = base.B * base.Hkv * base.cap * (2 * base.d + 8)
    R = args.replicas or max(3, math.ceil(512 * 2**20 / alloc_bytes))
    reps = [base]
    for _ in range(R - 1):
        c = synth.Problem(base.name, base.B, base.Hq, base.Hkv, base.d, base.cap, base.lengths_host,
                          base.q.clone(), base.k.clone(), base.v.clone(), base.ks.clone(), base.vs.clone(),
                          base.lengths, base.k_new, base.v_new)
        reps.append(c)
    outs = [torch.empty_like(base.q) for _ in reps]
    if args.page_size > 0:
        decs = [paged_decoder(kvq, p, o, args.page_size, args.splits, args.seed + i, args.page_order)
                for i, (p, o) in enumerate(zip(reps, outs))]
    else:
        decs = [kvq.Decoder(p.q, p.k, p.v, p.ks, p.vs, o, lengths=p.lengths,
                            max_seq_len=(0 if p.uniform else p.max_len) or p.cap,
                            num_splits=args.splits, k_new=p.k_new, v_new=p.v_new)
                for p, o in zip(reps, outs)]
    torch.cuda.synchronize()

    # Launches go to the current stream by its raw handle: one foreign call
    # per step, so host work between launches stays small (heavier per-launch
    # host work measurably slowed the running kernels on MI355X).
    sh = stream.cuda_stream
    t_warm = time.perf_counter()
    for i in range(args.warmup):
        decs[i % R](sh)
    torch.cuda.synchronize()
    settle = 0
    while (time.perf_counter() - t_warm) * 1e3 < args.settle_ms:
        for _ in range(50):
            decs[(args.warmup + settle) % R](sh)
            settle += 1
        torch.cuda.synchronize()

    # Pass 1: K steps between two events (the contract's timed region).
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        decs[i % R](sh)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps

    # Pass 2: every launch between its own events (kernel duration).
    n2 = min(args.steps, 100)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n2)]
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        decs[i % R](sh)
        b.record(stream)
    torch.cuda.synchronize()
    kern_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)

    # Pass 3: cache-warm (single replica, no rotation), labelled separately.
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(5):
        decs[0](sh)
    w0.record(stream)
    for _ in range(n2):
        decs[0](sh)
    w1.record(stream)
    torch.cuda.synchronize()
    warm_ms = w0.elapsed_time(w1) / n2

    if args.calib:
        x = torch.empty(2**28, dtype=torch.float32, device=dev)  # 1 GiB
        y = torch.empty_like(x)
        x.fill_(1.0)
        torch.cuda.synchronize()
        torch.mul(x, 1.0, out=y)  # reads 1 GiB, writes 1 GiB
        torch.cuda.synchronize()
        del x, y

    gbps = kv_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = gbps  # the step's decode launch(es)
    traffic = None
    if os.path.exists(args.traffic):
        try:
            with open(args.traffic) as f:
                tr = json.load(f)
            entry = tr.get("configs", {}).get(args.config)
            # Measured for the contiguous cache with the library's split choice.
            if entry and args.page_size == 0 and args.splits == 0:
                traffic = entry.get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    line = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_steps": settle,
        "ms_per_step": round(ms_per_step, 6),
        "us_per_step": round(ms_per_step * 1e3, 3),
        "pct_hbm_peak": round(100.0 * gbps / HBM_PEAK_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "storage": "int8 K/V + fp32 per-token scales",
        "data": "synthetic (seeded N(0,1) fp32 quantised per token on device)",
        "config": {
            "workload": f"{args.config}: B{base.B} Hq{base.Hq} Hkv{base.Hkv} d{base.d} "
                        f"L{'U' if not base.uniform else ''}{base.max_len}"
                        f"{' +append' if base.k_new is not None else ''}",
            "kv_bytes_per_step": kv_bytes,
            "replicas": R,
            "splits": decs[0].params.num_splits or "auto",
            "layout": (f"paged, {args.page_size} tokens per page, {args.page_order} pool" if args.page_size > 0
                       else "contiguous"),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name(base, args.page_size),
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel_us": round(ms_per_step * 1e3, 3),
            "kernel_us_isolated": round(kern_ms * 1e3, 3),
            "bytes_per_launch": kv_bytes,
        },
        "cache_warm": {"us_per_step": round(warm_ms * 1e3, 3),
                       "GB/s": round(kv_bytes / (warm_ms * 1e-3) / 1e9, 2),
                       "note": "single replica, Infinity-Cache resident; not the headline"},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(base, args.cpu_budget)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
