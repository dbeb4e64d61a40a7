"""PyTorch custom operators over libkvq.so (``torch.ops.kvq.*``).

The operators call the C ABI of include/kvq.h on the current torch stream.
They register fake (meta) implementations, so they trace under FakeTensor /
``torch.export`` and can be captured into CUDA (HIP) graphs: a decode launch
allocates nothing once its workspace exists.

  torch.ops.kvq.decode(q, k_cache, v_cache, k_scale, v_scale, lengths, max_seq_len,
                       softmax_scale, num_splits, k_new, v_new) -> out
      kvq_decode_launch; with k_new/v_new the token lengths[b]-1 (or
      max_seq_len-1) is first quantised into the caches (mutated in place).
  torch.ops.kvq.paged_decode(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table,
                             lengths, max_seq_len, softmax_scale, num_splits, k_new, v_new) -> out
      kvq_paged_decode_launch over a page pool.
  torch.ops.kvq.append(k_new, v_new, k_cache, v_cache, k_scale, v_scale, positions,
                       uniform_position) -> ()
      kvq_append_launch (mutates the caches).
  torch.ops.kvq.prefill(k_new, v_new, k_cache, v_cache, k_scale, v_scale, start,
                        uniform_start, block_table) -> ()
      kvq_prefill_quantize_launch (fp32 or bf16 rows; mutates the caches).
  torch.ops.kvq.attention(q, k, v, softmax_scale, num_splits) -> out
      kvq_attention_launch: dense fp32 softmax(q k^T * scale) v, q [M, d],
      k/v [N, d] (scale 0: 1/sqrt(d)).

Workspaces are cached per (operator, device, stream) and grown on demand:
launches on one stream are ordered, so they may share one; launches on
different streams get different ones.  A workspace is zero-filled by a kernel
(never a memset) when it is allocated.  A workspace that a later, larger call
supersedes is kept alive (never freed), because graphs captured before still
write to it on every replay.  A graph capture uses the stream's cached
workspace when it is large enough; otherwise the capture allocates one of its
own, whose zero-fill is recorded in the graph and runs only when the graph is
replayed, so that workspace belongs to that graph alone: it is never cached
for eager calls (which could run before the first replay) nor for other
captures.  Graphs captured on one stream that share its cached workspace must
not be replayed concurrently (on different streams), as for any two launches
that share a workspace.
"""
from __future__ import annotations

import ctypes
import threading
from typing import Optional

import torch
from torch import Tensor

from . import kvq

_ws_lock = threading.Lock()
_workspaces: dict = {}
# Superseded workspaces are kept, never freed: a graph captured from an earlier
# call still writes its split records and arrival counters there on every
# replay, and the caching allocator would otherwise hand that memory to other
# tensors.  Growth at least doubles, so these hold fewer bytes than the live ones.
_retired: list = []


def _workspace(key, nbytes: int, device) -> Tensor:
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is not None and ws.numel() >= nbytes:
            return ws
        size = max(nbytes, 2 * ws.numel() if ws is not None else 0, 1)
        new = torch.empty(size, dtype=torch.uint8, device=device)
        kvq.workspace_init(new, size)
        if torch.cuda.is_current_stream_capturing():
            # Allocated from the graph's private pool; the zero-fill kernel is
            # part of the graph and has not run yet.  Only this graph may use
            # it (kept alive for its replays).
            _retired.append(new)
            return new
        if ws is not None:
            _retired.append(ws)
        _workspaces[key] = new
        return new


def _opt(t: Optional[Tensor]):
    return None if t is None else t.data_ptr()


_MUTATED = ("k_cache", "v_cache", "k_scale", "v_scale")


@torch.library.custom_op("kvq::decode", mutates_args=_MUTATED)
def decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, k_scale: Tensor, v_scale: Tensor,
           lengths: Optional[Tensor], max_seq_len: int, softmax_scale: float, num_splits: int,
           k_new: Optional[Tensor], v_new: Optional[Tensor]) -> Tensor:
    _check_decode(q, k_cache, v_cache, k_scale, v_scale, lengths, k_new, v_new)
    out = torch.empty_like(q)
    p = kvq.decode_params(q, k_cache, v_cache, k_scale, v_scale, out, lengths, max_seq_len, softmax_scale,
                          num_splits, k_new, v_new)
    stream = torch.cuda.current_stream(q.device)
    nbytes = kvq.workspace_size(p)  # 0: one split, or arguments the launch will reject
    key = ("decode", q.device.index, stream.cuda_stream)
    ws = _workspace(key, nbytes, q.device) if nbytes else None
    code = kvq.lib().kvq_decode_launch(ctypes.byref(p), _opt(ws), nbytes, stream.cuda_stream)
    if code != kvq.HIP_SUCCESS:
        raise kvq.KvqError("kvq_decode_launch", code)
    return out


def _check_decode(q, k_cache, v_cache, k_scale, v_scale, lengths, k_new, v_new):
    B, Hq, d = q.shape
    _, Hkv, cap, _ = k_cache.shape
    kvq._need(q, torch.float32, (B, Hq, d), "q")
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        kvq._need(t, torch.int8, (B, Hkv, cap, d), n)
    for t, n in ((k_scale, "k_scale"), (v_scale, "v_scale")):
        kvq._need(t, torch.float32, (B, Hkv, cap), n)
    if lengths is not None:
        kvq._need(lengths, torch.int32, (B,), "lengths")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new must be given together")
    if k_new is not None:
        kvq._need(k_new, torch.float32, (B, Hkv, d), "k_new")
        kvq._need(v_new, torch.float32, (B, Hkv, d), "v_new")


@decode.register_fake
def _decode_fake(q, k_cache, v_cache, k_scale, v_scale, lengths, max_seq_len, softmax_scale, num_splits,
                 k_new, v_new):
    return torch.empty_like(q)


@torch.library.custom_op("kvq::paged_decode", mutates_args=("k_pages", "v_pages", "k_scale_pages",
                                                            "v_scale_pages"))
def paged_decode(q: Tensor, k_pages: Tensor, v_pages: Tensor, k_scale_pages: Tensor, v_scale_pages: Tensor,
                 block_table: Tensor, lengths: Optional[Tensor], max_seq_len: int, softmax_scale: float,
                 num_splits: int, k_new: Optional[Tensor], v_new: Optional[Tensor]) -> Tensor:
    out = torch.empty_like(q)
    kvq.check_paged(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, lengths, out, k_new, v_new)
    B, Hq, d = q.shape
    P_, Hkv, page, _ = k_pages.shape
    p = kvq.PagedDecodeParams(B, Hq, Hkv, d, page, P_, int(block_table.shape[1]), int(max_seq_len),
                              block_table.data_ptr(), _opt(lengths), q.data_ptr(), k_pages.data_ptr(),
                              v_pages.data_ptr(), k_scale_pages.data_ptr(), v_scale_pages.data_ptr(),
                              out.data_ptr(), float(softmax_scale), int(num_splits), _opt(k_new), _opt(v_new))
    L = kvq.lib()
    stream = torch.cuda.current_stream(q.device)
    nbytes = int(L.kvq_paged_decode_workspace_size(ctypes.byref(p)))
    key = ("paged", q.device.index, stream.cuda_stream)
    ws = _workspace(key, nbytes, q.device) if nbytes else None
    code = L.kvq_paged_decode_launch(ctypes.byref(p), _opt(ws), nbytes, stream.cuda_stream)
    if code != kvq.HIP_SUCCESS:
        raise kvq.KvqError("kvq_paged_decode_launch", code)
    return out


@paged_decode.register_fake
def _paged_decode_fake(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, lengths, max_seq_len,
                       softmax_scale, num_splits, k_new, v_new):
    return torch.empty_like(q)


@torch.library.custom_op("kvq::append", mutates_args=_MUTATED)
def append(k_new: Tensor, v_new: Tensor, k_cache: Tensor, v_cache: Tensor, k_scale: Tensor, v_scale: Tensor,
           positions: Optional[Tensor], uniform_position: int) -> None:
    kvq.append(k_new, v_new, k_cache, v_cache, k_scale, v_scale, positions=positions,
               uniform_position=uniform_position, stream=torch.cuda.current_stream(k_new.device).cuda_stream)


@append.register_fake
def _append_fake(k_new, v_new, k_cache, v_cache, k_scale, v_scale, positions, uniform_position):
    return None


@torch.library.custom_op("kvq::prefill", mutates_args=_MUTATED)
def prefill(k_new: Tensor, v_new: Tensor, k_cache: Tensor, v_cache: Tensor, k_scale: Tensor, v_scale: Tensor,
            start: Optional[Tensor], uniform_start: int, block_table: Optional[Tensor]) -> None:
    kvq.prefill(k_new, v_new, k_cache, v_cache, k_scale, v_scale, start=start, uniform_start=uniform_start,
                block_table=block_table, stream=torch.cuda.current_stream(k_new.device).cuda_stream)


@prefill.register_fake
def _prefill_fake(k_new, v_new, k_cache, v_cache, k_scale, v_scale, start, uniform_start, block_table):
    return None


@torch.library.custom_op("kvq::attention", mutates_args=())
def attention(q: Tensor, k: Tensor, v: Tensor, softmax_scale: float, num_splits: int) -> Tensor:
    out = torch.empty_like(q)
    p = kvq.attention_params(q, k, v, out, softmax_scale, num_splits)
    stream = torch.cuda.current_stream(q.device)
    nbytes = kvq.attention_workspace_size(p)  # 0: one split, or arguments the launch will reject
    ws = _workspace(("attention", q.device.index, stream.cuda_stream), nbytes, q.device) if nbytes else None
    code = kvq.lib().kvq_attention_launch(ctypes.byref(p), _opt(ws), nbytes, stream.cuda_stream)
    if code != kvq.HIP_SUCCESS:
        raise kvq.KvqError("kvq_attention_launch", code)
    return out


@attention.register_fake
def _attention_fake(q, k, v, softmax_scale, num_splits):
    return torch.empty_like(q)


__all__ = ["decode", "paged_decode", "append", "prefill", "attention"]
