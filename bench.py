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

Besides the headline (cfg1), the same protocol runs every configuration of
BASELINE.json (cfg0..cfg4, --configs) and reports each under "configs": us per
step, KV GB/s, fraction of the HBM roofline, the kernel the library planned,
the CPU baseline on a bounded sample, and max |GPU - oracle| of one checked
step (with the fraction of the 1e-4 + 1e-3*|ref| tolerance it uses).
"provenance" records git state, source and library hashes, ROCm/hipcc/torch
versions, the GPU and the host CPU.

Prints ONE JSON line.  Only --gpus 1 is supported (this build runs on one GPU).
"""
from __future__ import annotations

import argparse
import hashlib
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
    ap.add_argument("--configs", default="cfg0,cfg1,cfg2,cfg3,cfg4",
                    help="configurations to time besides the headline, comma-separated ('none': headline only)")
    ap.add_argument("--config-steps", type=int, default=200,
                    help="timed steps per extra configuration (at least --steps)")
    ap.add_argument("--config-cpu-budget", type=float, default=3.0,
                    help="max seconds for each extra configuration's CPU baseline")
    ap.add_argument("--calib", action="store_true",
                    help="also run a plain 1 GiB copy kernel (PMC byte-counter calibration)")
    ap.add_argument("--traffic", default=os.path.join(REPO, "profiles", "traffic.json"),
                    help="measured HBM traffic summary (from rocprofv3 --pmc), if present")
    return ap.parse_args()


def host_info():
    """CPU model and the cores this process may use (the GPU box's host share)."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "nproc": usable, "os_cpu_count": os.cpu_count()}


def cpu_baseline(prob, budget_s, min_runs=5):
    """The oracle (fp32 reference math, OpenMP) on the host copy of one step.
    Returns (baseline dict, the oracle's output of that step)."""
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

    ref = step()  # warm-up; also the checked step's expected output
    times, t_start = [], time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < 2.0 and len(times) < 50):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    t = statistics.median(times)
    base = {
        "value": round(prob.kv_bytes() / t / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(t * 1e6, 1),
        "cores": o.threads,
        "kind": "port",
        "sample": (f"full {prob.name} step ({'append + ' if kn is not None else ''}decode, "
                   f"{prob.B}x{prob.Hq} query heads), median of {len(times)} runs: {t * 1e6:.0f} us/step"),
    }
    base.update(host_info())
    return base, ref


def check_step(got, ref):
    """max |GPU - oracle| of one step and the largest fraction of the parity
    tolerance (1e-4 + 1e-3 * |ref|) any element uses."""
    import numpy as np
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    err = np.abs(g - r)
    finite = bool(np.all(np.isfinite(g)))
    return {"max_abs_err": float(err.max()) if finite else None,
            "max_tol_frac": float((err / (1e-4 + 1e-3 * np.abs(r))).max()) if finite else None,
            "within_tolerance": finite and bool(np.all(err <= 1e-4 + 1e-3 * np.abs(r)))}


def _sha256_files(paths):
    h = hashlib.sha256()
    for pth in sorted(paths):
        try:
            with open(pth, "rb") as f:
                h.update(os.path.relpath(pth, REPO).encode())
                h.update(f.read())
        except OSError:
            return None
    return h.hexdigest()


def provenance(torch, kvq):
    """Where and from what this line was measured (as the reference's scan
    harness records, benchmarks/selective_scan/run.py:91-116)."""
    import glob
    import subprocess

    def cmd(*argv):
        try:
            r = subprocess.run(list(argv), capture_output=True, text=True, timeout=20)
            return r.stdout.strip() if r.returncode == 0 else None
        except (OSError, subprocess.SubprocessError):
            return None

    pkg = os.path.join(REPO, "cuda-operators_amd")
    srcs = glob.glob(os.path.join(pkg, "csrc", "*")) + glob.glob(os.path.join(REPO, "include", "*.h"))
    build_info = None
    try:
        with open(os.path.join(pkg, "build_info.json")) as f:
            build_info = json.load(f)
    except (OSError, ValueError):
        pass
    rocm = None
    try:
        with open("/opt/rocm/.info/version") as f:
            rocm = f.read().strip()
    except OSError:
        pass
    # The compiler version comes from the build record: running hipcc here
    # would start further programs under a profiler's preload.
    hipcc = (build_info or {}).get("hipcc")
    props = torch.cuda.get_device_properties(0)
    return {
        "git_sha": cmd("git", "-C", REPO, "rev-parse", "HEAD"),
        "build": build_info,
        "sources_sha256": _sha256_files(srcs),
        "libkvq_sha256": _sha256_files([kvq.LIB_PATH]),
        "bench_sha256": _sha256_files([os.path.abspath(__file__)]),
        "library": kvq.version(),
        "rocm": rocm,
        "hipcc": hipcc,
        "torch": torch.__version__,
        "gpu": props.name,
        "gpu_arch": getattr(props, "gcnArchName", None),
        "gpu_cus": props.multi_processor_count,
        **host_info(),
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


def kernel_name(kvq, dec):
    """The kernel (and split plan) the library planned for decoder `dec`,
    from its host-only plan query (paged problems: the contiguous plan's
    kernel family)."""
    names = {kvq.KERNEL_DECODE_GENERIC: "decode_generic", kvq.KERNEL_DECODE_VALU: "decode_fast",
             kvq.KERNEL_DECODE_MFMA: "decode_mfma"}
    if not isinstance(dec.params, kvq.DecodeParams):
        return "paged"
    info = kvq.decode_plan(dec.params)
    name = f"{names[info.kernel]}<{dec.params.head_dim},{info.heads_per_group}>"
    if info.split_plan == kvq.SPLITS_TILES:
        return f"decode_mfma_flat<{dec.params.head_dim},{info.heads_per_group}> (tile-stream plan in-kernel)"
    if info.split_plan == kvq.SPLITS_IN_KERNEL:
        return name + " (split plan in-kernel)"
    if info.split_plan == kvq.SPLITS_SCHEDULE:
        return name + " (+ schedule_kernel per step)"
    return name + (f", {info.splits} splits" if info.splits > 1 else ", unsplit")


def time_config(args, torch, kvq, synth, name, steps, settle_ms, page_size=0):
    """Build config `name` (seeded, on the GPU), then W warm-up steps, settle,
    K timed steps over rotated replicas, a per-launch pass and a cache-warm
    pass.  Returns (result dict, the Problem, replica 0's output)."""
    stream = torch.cuda.current_stream()
    base = synth.make(name, seed=args.seed, device="cuda")
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
    if page_size > 0:
        decs = [paged_decoder(kvq, p, o, page_size, args.splits, args.seed + i, args.page_order)
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
    while (time.perf_counter() - t_warm) * 1e3 < settle_ms:
        for _ in range(50):
            decs[(args.warmup + settle) % R](sh)
            settle += 1
        torch.cuda.synchronize()

    # Pass 1: K steps between two events on the launch stream (the timed region).
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(steps):
        decs[i % R](sh)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / steps

    # Pass 2: every launch between its own events (kernel duration).
    n2 = min(steps, 100)
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

    gbps = kv_bytes / (ms_per_step * 1e-3) / 1e9
    res = {
        "workload": f"{name}: B{base.B} Hq{base.Hq} Hkv{base.Hkv} d{base.d} "
                    f"L{'U' if not base.uniform else ''}{base.max_len}"
                    f"{' +append' if base.k_new is not None else ''}",
        "kernel": kernel_name(kvq, decs[0]),
        "us_per_step": round(ms_per_step * 1e3, 3),
        "GB/s": round(gbps, 2),
        "frac": round(gbps / HBM_PEAK_GBPS, 4),
        "kv_bytes_per_step": kv_bytes,
        "steps": steps,
        "settle_steps": settle,
        "replicas": R,
        "kernel_us_isolated": round(kern_ms * 1e3, 3),
        "cache_warm_us_per_step": round(warm_ms * 1e3, 3),
        "splits": decs[0].params.num_splits or "auto",
    }
    out0 = outs[0]
    del decs, reps
    return res, base, out0


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

    head, base, out0 = time_config(args, torch, kvq, synth, args.config, args.steps, args.settle_ms,
                                   args.page_size)
    kv_bytes = head["kv_bytes_per_step"]
    ms_per_step = head["us_per_step"] * 1e-3
    head_check = None
    head_cpu = None
    if not args.no_cpu:
        head_cpu, ref = cpu_baseline(base, args.cpu_budget)
        head_check = check_step(out0.cpu().numpy(), ref)
    del base, out0
    torch.cuda.empty_cache()

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
    traffic_all = {}
    if os.path.exists(args.traffic):
        try:
            with open(args.traffic) as f:
                traffic_all = json.load(f).get("configs", {})
            entry = traffic_all.get(args.config)
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
        "settle_steps": head["settle_steps"],
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
            "workload": head["workload"],
            "kv_bytes_per_step": kv_bytes,
            "replicas": head["replicas"],
            "splits": head["splits"],
            "layout": (f"paged, {args.page_size} tokens per page, {args.page_order} pool" if args.page_size > 0
                       else "contiguous"),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": head["kernel"],
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel_us": round(ms_per_step * 1e3, 3),
            "kernel_us_isolated": head["kernel_us_isolated"],
            "bytes_per_launch": kv_bytes,
        },
        "cache_warm": {"us_per_step": head["cache_warm_us_per_step"],
                       "GB/s": round(kv_bytes / (head["cache_warm_us_per_step"] * 1e-6) / 1e9, 2),
                       "note": "single replica, Infinity-Cache resident; not the headline"},
    }
    if head_cpu is not None:
        line["cpu_baseline"] = head_cpu
        line["parity"] = head_check

    # Every other configuration under the same protocol.
    wanted = [] if args.configs.strip() in ("", "none") else [c.strip() for c in args.configs.split(",")]
    configs = {}
    for name in wanted:
        if name == args.config and args.page_size == 0:
            res = {k: head[k] for k in ("workload", "kernel", "us_per_step", "GB/s", "frac", "kv_bytes_per_step",
                                        "steps", "replicas", "kernel_us_isolated", "cache_warm_us_per_step")}
            if head_cpu is not None:
                res["cpu_baseline"] = head_cpu
                res.update(head_check)
        else:
            res, base, out0 = time_config(args, torch, kvq, synth, name, max(args.steps, args.config_steps),
                                          min(args.settle_ms, 200.0))
            if not args.no_cpu:
                res["cpu_baseline"], ref = cpu_baseline(base, args.config_cpu_budget, min_runs=3)
                res.update(check_step(out0.cpu().numpy(), ref))
            del base, out0
            torch.cuda.empty_cache()
        tr = traffic_all.get(name)
        res["traffic"] = tr.get("hbm_bytes_per_launch") if tr else None
        configs[name] = res
    if configs:
        line["configs"] = configs
    line["provenance"] = provenance(torch, kvq)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
