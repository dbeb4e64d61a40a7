"""Seeded synthetic decode problems for the five benchmark configurations.

Data is drawn on the GPU with torch generators (fp32), then quantised per token
into the int8 cache by the operator's own bulk quantiser
(kvq_quantize_rows_launch), exactly as a prefill would fill the cache.
Lengths are drawn on the host (numpy) so the algorithmic byte count of a step
is known without a device sync.

Configurations (task configs 0-4):
  cfg0  B1  Hq8  Hkv8 d64  L=1024                   N(0,1)
  cfg1  B8  Hq32 Hkv32 d128 L=4096, +append          N(0,1)
  cfg2  B16 Hq32 Hkv8 d128 L~U[1024,8192] ragged     N(0,1)
  cfg3  B1  Hq32 Hkv8 d128 L=131072                  K: N(0,1), 1% channels x20; V: N(0,1)
  cfg4  B256 Hq64 Hkv8 d128 L~U[512,4096] +append    Student-t(4)
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from . import kvq

CONFIGS = {
    "cfg0": dict(B=1, Hq=8, Hkv=8, d=64, lens=(1024, 1024), dist="normal", append=False),
    "cfg1": dict(B=8, Hq=32, Hkv=32, d=128, lens=(4096, 4096), dist="normal", append=True),
    "cfg2": dict(B=16, Hq=32, Hkv=8, d=128, lens=(1024, 8192), dist="normal", append=False),
    "cfg3": dict(B=1, Hq=32, Hkv=8, d=128, lens=(131072, 131072), dist="outlier", append=False),
    "cfg4": dict(B=256, Hq=64, Hkv=8, d=128, lens=(512, 4096), dist="student_t", append=True),
    # Not a BASELINE.json config: cfg2's ragged lengths with multi-head
    # attention (every query head its own kv head), the per-lane FMA kernel's
    # ragged path.
    "cfg2m": dict(B=16, Hq=32, Hkv=32, d=128, lens=(1024, 8192), dist="normal", append=False),
}


@dataclass
class Problem:
    name: str
    B: int
    Hq: int
    Hkv: int
    d: int
    cap: int
    lengths_host: np.ndarray          # int32 [B]
    q: torch.Tensor                   # [B, Hq, d] fp32
    k: torch.Tensor                   # [B, Hkv, cap, d] int8
    v: torch.Tensor
    ks: torch.Tensor                  # [B, Hkv, cap] fp32
    vs: torch.Tensor
    lengths: torch.Tensor | None      # [B] int32 on device, None when uniform
    k_new: torch.Tensor | None = None  # [B, Hkv, d] fp32 (append configs)
    v_new: torch.Tensor | None = None
    extra: dict = field(default_factory=dict)

    @property
    def uniform(self) -> bool:
        return self.lengths is None

    @property
    def max_len(self) -> int:
        return int(self.lengths_host.max())

    def kv_bytes(self) -> int:
        return kvq.kv_bytes(self.lengths_host, self.Hkv, self.d)


def _fill(gen, shape, dist, device, outlier_channels=None):
    if dist == "normal" or dist == "outlier":
        x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
        if dist == "outlier" and outlier_channels is not None:
            # outlier_channels: [B, H, n] channel ids per (b, kv head)
            B, H = shape[0], shape[1]
            for b in range(B):
                for h in range(H):
                    x[b, h, :, outlier_channels[b, h]] *= 20.0
        return x
    if dist == "student_t":
        z = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
        chi = torch.zeros(shape, device=device, dtype=torch.float32)
        for _ in range(4):
            chi.add_(torch.randn(shape, generator=gen, device=device, dtype=torch.float32).square_())
        return z.div_(chi.div_(4.0).sqrt_())
    raise ValueError(dist)


def _quantized_cache(gen, B, H, cap, d, dist, device, outlier_channels=None, chunk_rows=1 << 22):
    """int8 cache [B,H,cap,d] + scales [B,H,cap], generated in batch chunks."""
    q = torch.empty((B, H, cap, d), dtype=torch.int8, device=device)
    s = torch.empty((B, H, cap), dtype=torch.float32, device=device)
    per_b = H * cap
    bstep = max(1, chunk_rows // per_b)
    for b0 in range(0, B, bstep):
        b1 = min(B, b0 + bstep)
        oc = None if outlier_channels is None else outlier_channels[b0:b1]
        x = _fill(gen, (b1 - b0, H, cap, d), dist, device, oc)
        kvq.quantize_rows(x, q[b0:b1], s[b0:b1])
        del x
    return q, s


def make(name: str, seed: int = 17, device: str = "cuda", cap: int | None = None,
         scale_len: float = 1.0) -> Problem:
    """Build config `name` with `seed`.  scale_len < 1 shrinks the lengths
    (for fast parity runs of the same shape family)."""
    c = CONFIGS[name]
    B, Hq, Hkv, d = c["B"], c["Hq"], c["Hkv"], c["d"]
    lo, hi = c["lens"]
    lo = max(1, int(math.ceil(lo * scale_len)))
    hi = max(lo, int(math.ceil(hi * scale_len)))
    rng = np.random.default_rng(seed)
    if lo == hi:
        lengths_host = np.full(B, hi, np.int32)
    else:
        lengths_host = rng.integers(lo, hi + 1, B).astype(np.int32)
    cap = int(cap or hi)
    gen = torch.Generator(device=device)
    gen.manual_seed(int(seed))
    q = torch.randn((B, Hq, d), generator=gen, device=device, dtype=torch.float32)
    outl = None
    if c["dist"] == "outlier":
        n_out = max(1, int(math.ceil(0.01 * d)))
        outl = np.stack([np.stack([rng.choice(d, n_out, replace=False) for _ in range(Hkv)]) for _ in range(B)])
        outl = torch.as_tensor(outl, device=device, dtype=torch.long)
    k, ks = _quantized_cache(gen, B, Hkv, cap, d, c["dist"], device, outl)
    v, vs = _quantized_cache(gen, B, Hkv, cap, d, "normal" if c["dist"] == "outlier" else c["dist"], device)
    lengths = None if lo == hi else torch.as_tensor(lengths_host, device=device)
    p = Problem(name, B, Hq, Hkv, d, cap, lengths_host, q, k, v, ks, vs, lengths)
    if c["append"]:
        p.k_new = _fill(gen, (B, Hkv, d), "normal" if c["dist"] == "outlier" else c["dist"], device)
        p.v_new = _fill(gen, (B, Hkv, d), "normal" if c["dist"] == "outlier" else c["dist"], device)
    return p
