#!/usr/bin/env python3
"""Throughput of the operators beside the decode step, on one MI355X.

  --op attention   dense fp32 attention (attention_online_launch): one head,
                   Q[M,d], K/V[N,d]; algorithmic flops 4*M*N*d (QK^T and PV)
                   and bytes 4*(2*N*d + 2*M*d) (K and V read once, q read and
                   out written).  The roofline is the fp32 matrix-core peak
                   (157.3 TFLOP/s) when the flops per byte reach its ridge
                   (157.3 / 8 = 19.7), else HBM (8 TB/s): decode-shaped calls
                   (a few queries) are bandwidth-bound.
  --op prefill     prefill quantiser (kvq_prefill_quantize_launch): K and V
                   rows [B,Hkv,L,d] fp32 or bf16 into a contiguous int8 cache;
                   algorithmic bytes 2*rows*(d*in_bytes + d + 4) against HBM
                   peak (8 TB/s).

Inputs are resident in HBM; W untimed calls, then untimed calls for
--settle-ms of wall time, then K calls between two HIP events on the launch
stream.  Prints one JSON line.  The attention line also carries the CPU
oracle (test infrastructure, the checker) timed on a bounded sample of rows.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HBM_PEAK_GBPS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--op", choices=("attention", "prefill"), default="attention")
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=200.0)
    ap.add_argument("--M", type=int, default=4096)
    ap.add_argument("--N", type=int, default=4096)
    ap.add_argument("--d", type=int, default=128)
    ap.add_argument("--B", type=int, default=256)
    ap.add_argument("--Hkv", type=int, default=8)
    ap.add_argument("--L", type=int, default=1024)
    ap.add_argument("--dtype", choices=("f32", "bf16"), default="f32")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=64, help="query rows of the CPU oracle sample")
    ap.add_argument("--calib", action="store_true",
                    help="also run one plain 1 GiB copy (torch.mul) to calibrate rocprofv3 byte counters")
    return ap.parse_args()


def timed(torch, fn, steps, warmup, settle_ms):
    """Average microseconds per call of fn() over `steps` calls (HIP events)."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / steps


def bench_attention(torch, kvq, a):
    M, N, d = a.M, a.N, a.d
    gen = torch.Generator(device="cuda").manual_seed(1)
    q = torch.randn((M, d), generator=gen, device="cuda")
    k = torch.randn((N, d), generator=gen, device="cuda")
    v = torch.randn((N, d), generator=gen, device="cuda")
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    lib = kvq.lib()
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), M, N, d, stream)

    def call():
        code = lib.attention_online_launch(*args)
        if code:
            raise kvq.KvqError("attention_online_launch", code)

    us = timed(torch, call, a.steps, a.warmup, a.settle_ms)
    flops = 4.0 * M * N * d
    tflops = flops / (us * 1e-6) / 1e12
    p = kvq.attention_params(q, k, v, out)
    line = {
        "op": "attention", "metric": "dense fp32 attention TFLOP/s", "value": round(tflops, 2),
        "unit": "TFLOP/s", "us_per_call": round(us, 2), "steps": a.steps, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"attention M{M} N{N} d{d}", "M": M, "N": N, "d": d,
                   "workspace_bytes": kvq.attention_workspace_size(p)},
    }
    nbytes = 4.0 * (2 * N * d + 2 * M * d)
    if flops / nbytes >= FP32_MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBPS * 1e9):
        line["roofline"] = {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4),
                            "flops_per_call": flops}
    else:
        gbps = nbytes / (us * 1e-6) / 1e9
        line["roofline"] = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                            "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes_per_call": nbytes}
    if not a.no_cpu:
        from oracle import oracle as orc  # the checker, timed as the CPU baseline
        o = orc.get()
        rows = min(a.cpu_rows, M)
        qs, kc, vc = q[:rows].cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
        t0 = time.perf_counter()
        ref = o.attention_f32(qs, kc, vc)
        dt = time.perf_counter() - t0
        err = float(abs(out[:rows].cpu().numpy() - ref).max())
        line["cpu_baseline"] = {"value": round(4.0 * rows * N * d / dt / 1e12, 5), "unit": "TFLOP/s",
                                "cores": o.threads, "kind": "port",
                                "sample": f"{rows} query rows of the same problem ({dt:.2f} s)"}
        line["max_abs_err_vs_oracle"] = err
    return line


def bench_prefill(torch, kvq, a):
    B, H, L, d = a.B, a.Hkv, a.L, a.d
    dt = torch.float32 if a.dtype == "f32" else torch.bfloat16
    gen = torch.Generator(device="cuda").manual_seed(2)
    x = (torch.randn((B, H, L, d), generator=gen, device="cuda") * 3.0).to(dt)
    y = (torch.randn((B, H, L, d), generator=gen, device="cuda") * 3.0).to(dt)
    kc = torch.empty((B, H, L, d), dtype=torch.int8, device="cuda")
    vc = torch.empty_like(kc)
    ks = torch.empty((B, H, L), dtype=torch.float32, device="cuda")
    vs = torch.empty_like(ks)
    stream = torch.cuda.current_stream().cuda_stream
    us = timed(torch, lambda: kvq.prefill(x, y, kc, vc, ks, vs, uniform_start=0, stream=stream), a.steps,
               a.warmup, a.settle_ms)
    rows = B * H * L
    nbytes = 2.0 * rows * (d * x.element_size() + d + 4)
    gbps = nbytes / (us * 1e-6) / 1e9
    return {
        "op": "prefill", "metric": "prefill quantiser GB/s", "value": round(gbps, 1), "unit": "GB/s",
        "us_per_call": round(us, 2), "steps": a.steps, "dtype": a.dtype, "data": "synthetic",
        "config": {"workload": f"prefill B{B} Hkv{H} L{L} d{d} {a.dtype}", "B": B, "Hkv": H, "L": L, "d": d},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "bytes_per_call": nbytes},
    }


def main():
    a = parse()
    import torch
    if not torch.cuda.is_available():
        sys.exit("bench_ops.py needs a GPU")
    kvq = importlib.import_module("cuda-operators_amd").kvq
    line = bench_attention(torch, kvq, a) if a.op == "attention" else bench_prefill(torch, kvq, a)
    if a.calib:
        x = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
        y = torch.empty_like(x)
        torch.mul(x, 1.0, out=y)
        torch.cuda.synchronize()
        del x, y
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
