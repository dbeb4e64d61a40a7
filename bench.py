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
  * every configuration is set up first; then W untimed warm-up steps and
    untimed steps of each configuration until --settle-ms of wall time
    (sustained load first, so clocks and power state are at steady state);
  * --rounds rounds: round r visits the configurations in an order rotated by
    r, and times each for exactly its step count (K for the headline) between
    two HIP events on the launch stream, synchronised on both sides, after
    --round-settle-ms of its own untimed steps.  The median round gives
    ms_per_step and value; "rounds" lists every round with min and max;
  * every step is exactly one launch of the decode kernel, so the timed
    region / K is that kernel's average duration -> roofline.achieved; a
    further pass brackets every launch with its own events (reported as
    kernel_us_isolated: launches spaced by the event records);
  * cpu_baseline: the CPU oracle (same fp32 math as the reference's
    cpu_reference, OpenMP over heads) on the host copy of the same step;
    the checked step is also compared with the float64 oracle ("vs_f64":
    the GPU's error and the fp32 oracle's own, against the same yardstick);
  * verify_line() re-derives value, GB/s, fractions and the round summaries
    from the line's own fields before it is printed.

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
    ap.add_argument("--rounds", type=int, default=3,
                    help="timed rounds per configuration, in rotated order (the median round is reported)")
    ap.add_argument("--round-settle-ms", type=float, default=20.0,
                    help="untimed steps of a configuration right before each of its timed rounds")
    ap.add_argument("--config-cpu-budget", type=float, default=3.0,
                    help="max seconds for each extra configuration's CPU baseline")
    ap.add_argument("--calib", action="store_true",
                    help="also run a plain 1 GiB copy kernel (PMC byte-counter calibration)")
    ap.add_argument("--traffic", default=os.path.join(REPO, "profiles", "traffic.json"),
                    help="measured HBM traffic summary (from rocprofv3 --pmc), if present")
    ap.add_argument("--placement", type=int, default=0,
                    help="instead of the bench line: N separately allocated caches of --config, each timed "
                         "alone (contiguous layout), to show how the step time depends on where a cache sits")
    ap.add_argument("--placement-steps", type=int, default=200, help="timed steps per cache in --placement")
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
    ref64 = o.decode_f64(q, k, v, ks, vs, lengths=lengths)  # the same step in double precision
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
    return base, ref, ref64


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


def f64_errors(got, ref32, ref64):
    """Both the GPU's and the fp32 oracle's distance from the float64 oracle
    on the same step (as the reference's scan harness judges every
    implementation against an FP64 oracle, benchmarks/selective_scan/bench.cpp:85-99):
    which of the two carries the error the fp32 comparison reports."""
    import numpy as np
    r = np.asarray(ref64, np.float64)
    g = np.abs(np.asarray(got, np.float64) - r)
    c = np.abs(np.asarray(ref32, np.float64) - r)
    scale = 1e-4 + 1e-3 * np.abs(r)
    return {"gpu_max_abs": float(g.max()), "oracle_f32_max_abs": float(c.max()),
            "gpu_max_tol_frac": float((g / scale).max()), "oracle_f32_max_tol_frac": float((c / scale).max())}


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


class ConfigRun:
    """One configuration set up for timing: the seeded problem on the GPU,
    R cache replicas (R * KV bytes >= 512 MiB, R >= 3) so steps read HBM
    rather than the 256 MB Infinity Cache, one output per replica and one
    prepared launch per replica."""

    def __init__(self, args, torch, kvq, synth, name, steps, page_size=0):
        self.torch, self.name, self.steps = torch, name, steps
        base = synth.make(name, seed=args.seed, device="cuda")
        self.base = base
        self.kv_bytes = base.kv_bytes()
        alloc_bytes = base.B * base.Hkv * base.cap * (2 * base.d + 8)
        R = args.replicas or max(3, math.ceil(512 * 2**20 / alloc_bytes))
        reps = [base]
        for _ in range(R - 1):
            reps.append(synth.Problem(base.name, base.B, base.Hq, base.Hkv, base.d, base.cap, base.lengths_host,
                                      base.q.clone(), base.k.clone(), base.v.clone(), base.ks.clone(),
                                      base.vs.clone(), base.lengths, base.k_new, base.v_new))
        self.R = R
        self.outs = [torch.empty_like(base.q) for _ in reps]
        if page_size > 0:
            self.decs = [paged_decoder(kvq, p, o, page_size, args.splits, args.seed + i, args.page_order)
                         for i, (p, o) in enumerate(zip(reps, self.outs))]
        else:
            self.decs = [kvq.Decoder(p.q, p.k, p.v, p.ks, p.vs, o, lengths=p.lengths,
                                     max_seq_len=(0 if p.uniform else p.max_len) or p.cap,
                                     num_splits=args.splits, k_new=p.k_new, v_new=p.v_new)
                         for p, o in zip(reps, self.outs)]
        self.kernel = kernel_name(kvq, self.decs[0])
        self.splits = self.decs[0].params.num_splits or "auto"
        self.workload = (f"{name}: B{base.B} Hq{base.Hq} Hkv{base.Hkv} d{base.d} "
                         f"L{'U' if not base.uniform else ''}{base.max_len}"
                         f"{' +append' if base.k_new is not None else ''}")
        self.settle_steps = 0
        self.rounds_ms = []
        self.rounds_first = []  # this configuration's launch count at each timed round's start
        self.i = 0
        torch.cuda.synchronize()

    def launch(self, n, sh):
        # Launches go to the stream by its raw handle: one foreign call per
        # step, so host work between launches stays small (heavier per-launch
        # host work measurably slowed the running kernels on MI355X).
        for _ in range(n):
            self.decs[self.i % self.R](sh)
            self.i += 1

    def settle(self, sh, ms):
        """Untimed steps until `ms` of wall time has passed (sustained load)."""
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < ms:
            self.launch(50, sh)
            self.settle_steps += 50
            self.torch.cuda.synchronize()

    def timed(self, stream):
        """Exactly `steps` steps between two events on the launch stream,
        synchronised on both sides; ms per step."""
        torch = self.torch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        first = self.i
        e0.record(stream)
        self.launch(self.steps, stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / self.steps
        self.rounds_ms.append(ms)
        self.rounds_first.append(first)
        return ms

    def extras(self, stream):
        """Per-launch events (kernel duration) and a cache-warm pass over a
        single replica (labelled separately)."""
        torch = self.torch
        sh = stream.cuda_stream
        n2 = min(self.steps, 100)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n2)]
        for i, (a, b) in enumerate(ev):
            a.record(stream)
            self.decs[i % self.R](sh)
            b.record(stream)
        torch.cuda.synchronize()
        kern_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
        w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(5):
            self.decs[0](sh)
        w0.record(stream)
        for _ in range(n2):
            self.decs[0](sh)
        w1.record(stream)
        torch.cuda.synchronize()
        return kern_ms, w0.elapsed_time(w1) / n2

    def result(self, stream):
        """The configuration's line entry: the median round is the figure,
        min and max show the spread."""
        kern_ms, warm_ms = self.extras(stream)
        ms = statistics.median(self.rounds_ms)
        gbps = self.kv_bytes / (ms * 1e-3) / 1e9
        return {
            "workload": self.workload,
            "kernel": self.kernel,
            "us_per_step": round(ms * 1e3, 3),
            "GB/s": round(gbps, 2),
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "kv_bytes_per_step": self.kv_bytes,
            "steps": self.steps,
            "rounds": {"n": len(self.rounds_ms),
                       "us_per_step": [round(x * 1e3, 3) for x in self.rounds_ms],
                       "median": round(ms * 1e3, 3),
                       "min": round(min(self.rounds_ms) * 1e3, 3),
                       "max": round(max(self.rounds_ms) * 1e3, 3),
                       # Launch indices of this configuration's kernel (counting from its first
                       # warm-up launch) at which each timed round starts: a kernel trace of the
                       # same run selects the timed launches with them.
                       "first_launch": list(self.rounds_first)},
            "settle_steps": self.settle_steps,
            "replicas": self.R,
            "kernel_us_isolated": round(kern_ms * 1e3, 3),
            "cache_warm_us_per_step": round(warm_ms * 1e3, 3),
            "splits": self.splits,
        }

    def release(self):
        out0 = self.outs[0]
        base = self.base
        self.decs = self.outs = self.base = None
        return base, out0


def rotated(names, r):
    """Round r runs the configurations starting at the r-th, so no
    configuration always follows the same one (as the reference's harness
    shuffles its order per round, benchmarks/selective_scan/run.py:166-194)."""
    k = r % len(names)
    return names[k:] + names[:k]


def verify_line(line):
    """Problems with a bench line, re-derived from its own fields (as the
    reference's verify_results.py:21-72 recomputes its summaries from the raw
    rows): empty when the line is consistent."""
    bad = []

    def near(a, b, rel=2e-3, what="", digits=None):
        # digits: a is rounded to that many decimals, so half a unit of the
        # last place is allowed as well.
        tol = rel * max(abs(a or 0.0), abs(b or 0.0), 1e-12)
        if digits is not None:
            tol = max(tol, 0.5 * 10.0 ** -digits + 1e-12)
        if a is None or b is None or abs(a - b) > tol:
            bad.append(f"{what}: {a} vs {b}")

    kvb = line["config"]["kv_bytes_per_step"]
    near(line["value"], kvb / (line["ms_per_step"] * 1e-3) / 1e9, what="value = KV bytes / ms_per_step")
    near(line["us_per_step"], line["ms_per_step"] * 1e3, what="us_per_step")
    near(line["pct_hbm_peak"], 100.0 * line["value"] / HBM_PEAK_GBPS, what="pct_hbm_peak", digits=2)
    rf = line["roofline"]
    near(rf["frac"], rf["achieved"] / rf["peak"], what="roofline.frac", digits=4)
    near(rf["achieved"], line["value"], what="roofline.achieved")
    near(rf["peak"], HBM_PEAK_GBPS, what="roofline.peak")
    if rf["bytes_per_launch"] != kvb:
        bad.append("roofline.bytes_per_launch != config.kv_bytes_per_step")
    rounds = line.get("rounds")
    if rounds:
        us = rounds["us_per_step"]
        if len(us) != rounds["n"]:
            bad.append("rounds: n != len(us_per_step)")
        near(rounds["median"], statistics.median(us), what="rounds.median")
        near(rounds["min"], min(us), what="rounds.min")
        near(rounds["max"], max(us), what="rounds.max")
        near(line["us_per_step"], rounds["median"], what="us_per_step = median round")
    for name, c in (line.get("configs") or {}).items():
        near(c["GB/s"], c["kv_bytes_per_step"] / (c["us_per_step"] * 1e-6) / 1e9, what=f"{name} GB/s")
        near(c["frac"], c["GB/s"] / HBM_PEAK_GBPS, what=f"{name} frac", digits=4)
        r = c.get("rounds")
        if r:
            near(c["us_per_step"], statistics.median(r["us_per_step"]), what=f"{name} median round")
            if not r["min"] <= c["us_per_step"] <= r["max"]:
                bad.append(f"{name}: median outside [min, max]")
        if "within_tolerance" in c and c["max_tol_frac"] is not None:
            if c["within_tolerance"] != (c["max_tol_frac"] <= 1.0):
                bad.append(f"{name}: within_tolerance disagrees with max_tol_frac")
    return bad


def placement_sweep(args, torch, kvq, synth, stream):
    """--placement N: N caches of one configuration, allocated one after
    another; --warmup steps over all of them (steady clocks), then each cache
    launched 20 times untimed and --placement-steps times between two events,
    alone.  Prints one JSON line with each cache's K and V addresses and its
    us/step."""
    a = argparse.Namespace(**vars(args))
    a.replicas = args.placement
    run = ConfigRun(a, torch, kvq, synth, args.config, args.placement_steps)
    sh = stream.cuda_stream
    run.launch(args.warmup, sh)
    torch.cuda.synchronize()
    caches = []
    for r, dec in enumerate(run.decs):
        for _ in range(20):
            dec(sh)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.placement_steps):
            dec(sh)
        e1.record(stream)
        torch.cuda.synchronize()
        k, v = dec.keep[1], dec.keep[2]
        caches.append({"cache": r, "k": hex(k.data_ptr()), "v": hex(v.data_ptr()),
                       "us_per_step": round(e0.elapsed_time(e1) * 1e3 / args.placement_steps, 3)})
    print(json.dumps({"mode": "placement", "workload": run.workload, "kernel": run.kernel,
                      "steps_per_cache": args.placement_steps, "caches": caches}), flush=True)


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
    sh = stream.cuda_stream
    if args.placement > 0:
        placement_sweep(args, torch, kvq, synth, stream)
        return

    # Every configuration is set up first (seeded problems and replicas, about
    # 10 GB in all), then timed in rounds: round r runs them in rotated order,
    # each after a short settle on its own steps, each for exactly its step
    # count.  The headline's figure is its median round.
    wanted = [] if args.configs.strip() in ("", "none") else [c.strip() for c in args.configs.split(",")]
    head_key = "__head__"
    runs = {head_key: ConfigRun(args, torch, kvq, synth, args.config, args.steps, args.page_size)}
    for name in wanted:
        if name == args.config and args.page_size == 0:
            continue  # the headline is this configuration
        runs[name] = ConfigRun(args, torch, kvq, synth, name, max(args.steps, args.config_steps))
    # Sustained load first (clocks and power at steady state): W warm-up steps
    # of the headline, then --settle-ms of wall time across the configurations.
    runs[head_key].launch(args.warmup, sh)
    torch.cuda.synchronize()
    for key, r in runs.items():
        r.settle(sh, args.settle_ms if key == head_key else min(args.settle_ms, 100.0))
    order = list(runs)
    for rnd in range(args.rounds):
        for key in rotated(order, rnd):
            runs[key].settle(sh, args.round_settle_ms)
            runs[key].timed(stream)
    results = {key: r.result(stream) for key, r in runs.items()}

    head = results[head_key]
    kv_bytes = head["kv_bytes_per_step"]
    ms_per_step = head["us_per_step"] * 1e-3
    checks = {}
    cpus = {}
    for key, r in runs.items():
        base, out0 = r.release()
        if not args.no_cpu:
            budget = args.cpu_budget if key == head_key else args.config_cpu_budget
            cpus[key], ref, ref64 = cpu_baseline(base, budget, min_runs=5 if key == head_key else 3)
            got = out0.cpu().numpy()
            checks[key] = check_step(got, ref)
            checks[key]["vs_f64"] = f64_errors(got, ref, ref64)
        del base, out0
    runs.clear()
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
        "rounds": head["rounds"],
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
    if head_key in cpus:
        line["cpu_baseline"] = cpus[head_key]
        line["parity"] = checks[head_key]

    configs = {}
    for name in wanted:
        key = head_key if (name == args.config and args.page_size == 0) else name
        res = dict(results[key])
        res.pop("settle_steps", None)
        res.pop("splits", None) if key == head_key else None
        if key in cpus:
            res["cpu_baseline"] = cpus[key]
            res.update(checks[key])
        tr = traffic_all.get(name)
        res["traffic"] = tr.get("hbm_bytes_per_launch") if tr else None
        configs[name] = res
    if configs:
        line["configs"] = configs
    line["provenance"] = provenance(torch, kvq)
    problems = verify_line(line)
    if problems:  # a line that contradicts itself is a bench bug: say so, keep the line
        line["verify"] = problems
        print("bench.py: inconsistent line: " + "; ".join(problems), file=sys.stderr)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
