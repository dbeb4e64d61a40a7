"""ctypes binding of libkvq.so (include/kvq.h) for torch device tensors.

The operator itself is the C ABI; this module only marshals torch tensors
(device memory) and torch streams into it.  There is no fallback: if
libkvq.so is missing or a call fails, an exception is raised.

Entry points mirror the reference's kv_cache/ interface:
  solve(...)                  -> kv_cache/KV_int8.cu:306 (legacy void ABI, null stream)
  kv_int8_split_launch(...)   -> kv_cache/KV_int8_split_optimized.cu:268
  kv_int8_simple_launch(...)  -> kv_cache/new_kvint8.cu:85
plus the batched / GQA / ragged / append extension (decode, append,
quantize_rows, workspace helpers).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkvq.so")
ATTN_LIB_PATH = os.path.join(HERE, "libkvq_attention.so")

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
MAX_HEAD_DIM = 4096
MAX_SEQ_LEN = 1 << 30  # KVQ_MAX_SEQ_LEN

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_attn_lib: ctypes.CDLL | None = None

_vp = ctypes.c_void_p
_int = ctypes.c_int


class DecodeParams(ctypes.Structure):
    """struct kvq_decode_params (include/kvq.h)."""
    _fields_ = [
        ("batch", _int), ("num_q_heads", _int), ("num_kv_heads", _int), ("head_dim", _int),
        ("capacity", _int), ("max_seq_len", _int),
        ("lengths", _vp), ("q", _vp), ("k_cache", _vp), ("v_cache", _vp),
        ("k_scale", _vp), ("v_scale", _vp), ("out", _vp),
        ("softmax_scale", ctypes.c_float), ("num_splits", _int),
        ("k_new", _vp), ("v_new", _vp),
    ]


class AppendParams(ctypes.Structure):
    """struct kvq_append_params (include/kvq.h)."""
    _fields_ = [
        ("batch", _int), ("num_kv_heads", _int), ("head_dim", _int), ("capacity", _int),
        ("positions", _vp), ("uniform_position", _int),
        ("k_new", _vp), ("v_new", _vp), ("k_cache", _vp), ("v_cache", _vp),
        ("k_scale", _vp), ("v_scale", _vp),
    ]


class PagedDecodeParams(ctypes.Structure):
    """struct kvq_paged_decode_params (include/kvq.h)."""
    _fields_ = [
        ("batch", _int), ("num_q_heads", _int), ("num_kv_heads", _int), ("head_dim", _int),
        ("page_size", _int), ("num_pages", _int), ("max_pages_per_seq", _int), ("max_seq_len", _int),
        ("block_table", _vp), ("lengths", _vp), ("q", _vp), ("k_pages", _vp), ("v_pages", _vp),
        ("k_scale_pages", _vp), ("v_scale_pages", _vp), ("out", _vp),
        ("softmax_scale", ctypes.c_float), ("num_splits", _int),
        ("k_new", _vp), ("v_new", _vp),
    ]


class PagedAppendParams(ctypes.Structure):
    """struct kvq_paged_append_params (include/kvq.h)."""
    _fields_ = [
        ("batch", _int), ("num_kv_heads", _int), ("head_dim", _int), ("page_size", _int),
        ("num_pages", _int), ("max_pages_per_seq", _int),
        ("block_table", _vp), ("positions", _vp), ("uniform_position", _int),
        ("k_new", _vp), ("v_new", _vp), ("k_pages", _vp), ("v_pages", _vp),
        ("k_scale_pages", _vp), ("v_scale_pages", _vp),
    ]


class PrefillParams(ctypes.Structure):
    """struct kvq_prefill_params (include/kvq.h)."""
    _fields_ = [
        ("batch", _int), ("num_kv_heads", _int), ("head_dim", _int), ("tokens", _int), ("dtype", _int),
        ("k_new", _vp), ("v_new", _vp), ("start", _vp), ("uniform_start", _int), ("capacity", _int),
        ("k_cache", _vp), ("v_cache", _vp), ("k_scale", _vp), ("v_scale", _vp),
        ("block_table", _vp), ("page_size", _int), ("num_pages", _int), ("max_pages_per_seq", _int),
    ]


DTYPE_F32 = 0
DTYPE_BF16 = 1


class AttentionParams(ctypes.Structure):
    """struct kvq_attention_params (include/kvq.h)."""
    _fields_ = [
        ("M", _int), ("N", _int), ("d", _int), ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp),
        ("softmax_scale", ctypes.c_float), ("num_splits", _int),
    ]


class PlanInfo(ctypes.Structure):
    """struct kvq_plan_info (include/kvq.h part 6)."""
    _fields_ = [
        ("kernel", _int), ("heads_per_group", _int), ("splits", _int), ("chunk", _int),
        ("split_plan", _int), ("query_block", _int), ("workspace_bytes", ctypes.c_size_t),
        ("tile_tokens", _int),
    ]


KERNEL_DECODE_GENERIC, KERNEL_DECODE_VALU, KERNEL_DECODE_MFMA = 0, 1, 2
KERNEL_ATTENTION_MFMA, KERNEL_ATTENTION_ROWS, KERNEL_ATTENTION_GENERIC, KERNEL_ATTENTION_DIRECT = 3, 4, 5, 6
SPLITS_STATIC, SPLITS_IN_KERNEL, SPLITS_SCHEDULE, SPLITS_TILES = 0, 1, 2, 3

EXPORTS = ("solve", "kv_int8_split_launch", "kv_int8_simple_launch", "kvq_decode_workspace_size",
           "kvq_workspace_init", "kvq_decode_launch", "kvq_append_launch", "kvq_quantize_rows_launch",
           "kvq_paged_decode_workspace_size", "kvq_paged_decode_launch", "kvq_paged_append_launch",
           "kvq_prefill_quantize_launch", "attention_online_launch", "kvq_attention_workspace_size",
           "kvq_attention_launch", "kvq_version", "kvq_reference_plan", "kvq_decode_plan", "kvq_attention_plan",
           "kvq_diagnostics", "kvq_decode_launch_noalloc", "kvq_paged_decode_plan")


class KvqError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} returned hipError {code}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load libkvq.so (built in-tree by __graft_entry__.build() / make)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libkvq.so is not built ({LIB_PATH}); run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        ref = [_vp] * 6 + [_int] * 3
        L.solve.argtypes = ref
        L.solve.restype = None
        for fn in ("kv_int8_split_launch", "kv_int8_simple_launch"):
            getattr(L, fn).argtypes = ref + [_vp, _vp]
            getattr(L, fn).restype = _int
        L.kvq_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeParams)]
        L.kvq_decode_workspace_size.restype = ctypes.c_size_t
        L.kvq_workspace_init.argtypes = [_vp, ctypes.c_size_t, _vp]
        L.kvq_workspace_init.restype = _int
        L.kvq_decode_launch.argtypes = [ctypes.POINTER(DecodeParams), _vp, ctypes.c_size_t, _vp]
        L.kvq_decode_launch.restype = _int
        L.kvq_decode_launch_noalloc.argtypes = [ctypes.POINTER(DecodeParams), _vp]
        L.kvq_decode_launch_noalloc.restype = _int
        L.kvq_append_launch.argtypes = [ctypes.POINTER(AppendParams), _vp]
        L.kvq_append_launch.restype = _int
        L.kvq_quantize_rows_launch.argtypes = [_vp, ctypes.c_int64, _int, _vp, _vp, _vp]
        L.kvq_quantize_rows_launch.restype = _int
        L.kvq_paged_decode_workspace_size.argtypes = [ctypes.POINTER(PagedDecodeParams)]
        L.kvq_paged_decode_workspace_size.restype = ctypes.c_size_t
        L.kvq_paged_decode_launch.argtypes = [ctypes.POINTER(PagedDecodeParams), _vp, ctypes.c_size_t, _vp]
        L.kvq_paged_decode_launch.restype = _int
        L.kvq_paged_append_launch.argtypes = [ctypes.POINTER(PagedAppendParams), _vp]
        L.kvq_paged_append_launch.restype = _int
        L.kvq_prefill_quantize_launch.argtypes = [ctypes.POINTER(PrefillParams), _vp]
        L.kvq_prefill_quantize_launch.restype = _int
        L.attention_online_launch.argtypes = [_vp, _vp, _vp, _vp, _int, _int, _int, _vp]
        L.attention_online_launch.restype = _int
        L.kvq_attention_workspace_size.argtypes = [ctypes.POINTER(AttentionParams)]
        L.kvq_attention_workspace_size.restype = ctypes.c_size_t
        L.kvq_attention_launch.argtypes = [ctypes.POINTER(AttentionParams), _vp, ctypes.c_size_t, _vp]
        L.kvq_attention_launch.restype = _int
        L.kvq_version.restype = ctypes.c_char_p
        L.kvq_reference_plan.argtypes = [_vp, _vp, _vp, _int, _int, _int, ctypes.POINTER(PlanInfo)]
        L.kvq_reference_plan.restype = _int
        L.kvq_decode_plan.argtypes = [ctypes.POINTER(DecodeParams), ctypes.POINTER(PlanInfo)]
        L.kvq_decode_plan.restype = _int
        L.kvq_paged_decode_plan.argtypes = [ctypes.POINTER(PagedDecodeParams), ctypes.POINTER(PlanInfo)]
        L.kvq_paged_decode_plan.restype = _int
        L.kvq_attention_plan.argtypes = [ctypes.POINTER(AttentionParams), ctypes.POINTER(PlanInfo)]
        L.kvq_attention_plan.restype = _int
        L.kvq_diagnostics.restype = _int
        _lib = L
        return L


def attention_lib() -> ctypes.CDLL:
    """Load libkvq_attention.so (include/kvq_attention.h): the dense-attention
    `solve` of attention/softmax_new.cu:283-287, whose symbol libkvq.so's
    decode `solve` already takes."""
    global _attn_lib
    lib()
    with _lock:
        if _attn_lib is not None:
            return _attn_lib
        if not os.path.exists(ATTN_LIB_PATH):
            raise RuntimeError(f"libkvq_attention.so is not built ({ATTN_LIB_PATH}); run __graft_entry__.build()")
        A = ctypes.CDLL(ATTN_LIB_PATH)
        A.solve.argtypes = [_vp] * 4 + [_int] * 3
        A.solve.restype = None
        _attn_lib = A
        return A


def version() -> str:
    return lib().kvq_version().decode()


def _ptr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _check(fn: str, code: int) -> None:
    if code != HIP_SUCCESS:
        raise KvqError(fn, code)


def _need(t, dtype, shape, name):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor")
    if t.dtype != dtype or tuple(t.shape) != tuple(shape) or not t.is_contiguous() or t.device.type != "cuda":
        raise ValueError(f"{name}: want contiguous cuda {dtype} {tuple(shape)}, got {t.dtype} "
                         f"{tuple(t.shape)} on {t.device}")


# ---------------------------------------------------------------------------
# reference ABI
# ---------------------------------------------------------------------------
def _check_reference(Q, K, V, k_scale, v_scale, out):
    """Dtypes, shapes and devices of a reference-ABI call (the C entry points
    see only pointers and (H, N, d)); returns (H, N, d)."""
    H, N, d = K.shape
    _need(Q, torch.float32, (H, d), "Q")
    _need(K, torch.int8, (H, N, d), "K")
    _need(V, torch.int8, (H, N, d), "V")
    _need(k_scale, torch.float32, (H, N), "k_scale")
    _need(v_scale, torch.float32, (H, N), "v_scale")
    _need(out, torch.float32, (H, d), "out")
    return H, N, d


def solve(Q, K, V, k_scale, v_scale, out) -> None:
    """Legacy `solve` on the null stream: Q[H,d], K/V[H,N,d] int8, scales[H,N], out[H,d]."""
    H, N, d = _check_reference(Q, K, V, k_scale, v_scale, out)
    lib().solve(_ptr(Q), _ptr(K), _ptr(V), _ptr(k_scale), _ptr(v_scale), _ptr(out), H, N, d)


def kv_int8_split_launch(Q, K, V, k_scale, v_scale, out, S, stream=None, simple=False) -> int:
    """Stream-aware reference launch; S is H*N floats of caller scratch. Returns the hipError code."""
    H, N, d = _check_reference(Q, K, V, k_scale, v_scale, out)
    if not (isinstance(S, torch.Tensor) and S.dtype == torch.float32 and S.is_contiguous()
            and S.device.type == "cuda" and S.numel() >= H * N):
        raise ValueError(f"S: want contiguous cuda float32 scratch of at least {H * N} elements")
    fn = lib().kv_int8_simple_launch if simple else lib().kv_int8_split_launch
    return int(fn(_ptr(Q), _ptr(K), _ptr(V), _ptr(k_scale), _ptr(v_scale), _ptr(out), H, N, d, _ptr(S),
                  _stream(stream)))


# ---------------------------------------------------------------------------
# extension
# ---------------------------------------------------------------------------
def decode_params(q, k_cache, v_cache, k_scale, v_scale, out, lengths=None, max_seq_len=0,
                  softmax_scale=0.0, num_splits=0, k_new=None, v_new=None) -> DecodeParams:
    B, Hq, d = q.shape
    _, Hkv, cap, _ = k_cache.shape
    return DecodeParams(B, Hq, Hkv, d, cap, int(max_seq_len), _ptr(lengths), _ptr(q), _ptr(k_cache),
                        _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), _ptr(out), float(softmax_scale),
                        int(num_splits), _ptr(k_new), _ptr(v_new))


def workspace_size(p: DecodeParams) -> int:
    return int(lib().kvq_decode_workspace_size(ctypes.byref(p)))


def workspace_init(ws, nbytes=None, stream=None) -> None:
    nbytes = ws.numel() * ws.element_size() if nbytes is None else nbytes
    _check("kvq_workspace_init", lib().kvq_workspace_init(_ptr(ws), nbytes, _stream(stream)))


def new_workspace(p: DecodeParams, device=None, stream=None) -> torch.Tensor:
    """Allocate and zero-fill a workspace for params p (an empty tensor when none is needed)."""
    n = workspace_size(p)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=device or "cuda")
    if n:
        workspace_init(ws, n, stream)
    return ws


def decode_launch(p: DecodeParams, ws, stream=None) -> None:
    nbytes = 0 if ws is None else ws.numel() * ws.element_size()
    _check("kvq_decode_launch", lib().kvq_decode_launch(ctypes.byref(p), _ptr(ws), nbytes, _stream(stream)))


NOALLOC_SCRATCH_BYTES = 16 << 20  # KVQ_NOALLOC_SCRATCH_BYTES


def decode_launch_noalloc(p: DecodeParams, stream=None) -> int:
    """kvq_decode_launch_noalloc: the library's fixed device scratch array in
    place of a workspace (allocates nothing).  Returns the hipError code."""
    return int(lib().kvq_decode_launch_noalloc(ctypes.byref(p), _stream(stream)))


class Decoder:
    """A decode problem with its own workspace: build once, launch many times."""

    def __init__(self, q, k_cache, v_cache, k_scale, v_scale, out, lengths=None, max_seq_len=0,
                 softmax_scale=0.0, num_splits=0, k_new=None, v_new=None, stream=None):
        B, Hq, d = q.shape
        _, Hkv, cap, d2 = k_cache.shape
        if d2 != d or Hq % Hkv:
            raise ValueError("shape mismatch")
        _need(q, torch.float32, (B, Hq, d), "q")
        for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
            _need(t, torch.int8, (B, Hkv, cap, d), n)
        for t, n in ((k_scale, "k_scale"), (v_scale, "v_scale")):
            _need(t, torch.float32, (B, Hkv, cap), n)
        _need(out, torch.float32, (B, Hq, d), "out")
        if lengths is not None:
            _need(lengths, torch.int32, (B,), "lengths")
        if k_new is not None:
            _need(k_new, torch.float32, (B, Hkv, d), "k_new")
            _need(v_new, torch.float32, (B, Hkv, d), "v_new")
        self.keep = (q, k_cache, v_cache, k_scale, v_scale, out, lengths, k_new, v_new)
        self.params = decode_params(q, k_cache, v_cache, k_scale, v_scale, out, lengths, max_seq_len,
                                    softmax_scale, num_splits, k_new, v_new)
        self.ws = new_workspace(self.params, q.device, stream)
        self.ws_bytes = workspace_size(self.params)
        # Launch arguments resolved once: a step costs one foreign call.
        self._launch = lib().kvq_decode_launch
        self._args = (ctypes.byref(self.params), _ptr(self.ws), self.ws_bytes)

    def __call__(self, stream=None) -> None:
        """Launch on `stream` (a torch stream or a raw hipStream_t handle;
        default: torch's current stream)."""
        code = self._launch(*self._args, stream if isinstance(stream, int) else _stream(stream))
        if code != HIP_SUCCESS:
            raise KvqError("kvq_decode_launch", code)


def decode(q, k_cache, v_cache, k_scale, v_scale, lengths=None, max_seq_len=0, softmax_scale=0.0,
           num_splits=0, k_new=None, v_new=None, out=None, stream=None) -> torch.Tensor:
    """One-shot batched decode attention; returns out[B, Hq, d]."""
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    Decoder(q, k_cache, v_cache, k_scale, v_scale, out, lengths, max_seq_len, softmax_scale, num_splits,
            k_new, v_new, stream)(stream)
    return out


def _check_cache(k_cache, v_cache, k_scale, v_scale, what="cache"):
    """An int8 K/V pair [X, Hkv, T, d] with fp32 scales [X, Hkv, T] (X: batch
    or pages, T: capacity or page size); returns (X, Hkv, T, d)."""
    X, Hkv, T, d = k_cache.shape
    for t, n in ((k_cache, f"k_{what}"), (v_cache, f"v_{what}")):
        _need(t, torch.int8, (X, Hkv, T, d), n)
    for t, n in ((k_scale, "k_scale"), (v_scale, "v_scale")):
        _need(t, torch.float32, (X, Hkv, T), n)
    return X, Hkv, T, d


def _check_new_rows(k_new, v_new, B, Hkv, d):
    for t, n in ((k_new, "k_new"), (v_new, "v_new")):
        _need(t, torch.float32, (B, Hkv, d), n)


def append(k_new, v_new, k_cache, v_cache, k_scale, v_scale, positions=None, uniform_position=0,
           stream=None) -> None:
    """One new K/V token per (b, kv head) into the contiguous cache (kvq_append_launch)."""
    B, Hkv, cap, d = _check_cache(k_cache, v_cache, k_scale, v_scale)
    _check_new_rows(k_new, v_new, B, Hkv, d)
    if positions is not None:
        _need(positions, torch.int32, (B,), "positions")
    p = AppendParams(B, Hkv, d, cap, _ptr(positions), int(uniform_position), _ptr(k_new), _ptr(v_new),
                     _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale))
    _check("kvq_append_launch", lib().kvq_append_launch(ctypes.byref(p), _stream(stream)))


def quantize_rows(x, q=None, scale=None, stream=None):
    """x[..., d] fp32 cuda -> (q int8 [..., d], scale fp32 [...])."""
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    _need(x, torch.float32, tuple(x.shape), "x")
    if q is None:
        q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    if scale is None:
        scale = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    _need(q, torch.int8, tuple(x.shape), "q")
    _need(scale, torch.float32, tuple(x.shape[:-1]), "scale")
    _check("kvq_quantize_rows_launch",
           lib().kvq_quantize_rows_launch(_ptr(x), rows, d, _ptr(q), _ptr(scale), _stream(stream)))
    return q, scale


# ---------------------------------------------------------------------------
# paged cache
# ---------------------------------------------------------------------------
def check_paged(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, lengths, out, k_new=None,
                v_new=None) -> None:
    """Dtype, shape, layout and device checks of a paged decode's tensors (the
    C ABI sees only pointers and sizes, so a wrong dtype would read out of bounds)."""
    B, Hq, d = q.shape
    P_, Hkv, page, d2 = k_pages.shape
    if d2 != d or Hq % Hkv:
        raise ValueError("shape mismatch")
    _need(q, torch.float32, (B, Hq, d), "q")
    for t, n in ((k_pages, "k_pages"), (v_pages, "v_pages")):
        _need(t, torch.int8, (P_, Hkv, page, d), n)
    for t, n in ((k_scale_pages, "k_scale_pages"), (v_scale_pages, "v_scale_pages")):
        _need(t, torch.float32, (P_, Hkv, page), n)
    if block_table.dim() != 2 or block_table.shape[0] != B:
        raise ValueError("block_table: want [B, max_pages_per_seq]")
    _need(block_table, torch.int32, tuple(block_table.shape), "block_table")
    if lengths is not None:
        _need(lengths, torch.int32, (B,), "lengths")
    _need(out, torch.float32, (B, Hq, d), "out")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new must be given together")
    if k_new is not None:
        _need(k_new, torch.float32, (B, Hkv, d), "k_new")
        _need(v_new, torch.float32, (B, Hkv, d), "v_new")


class PagedDecoder:
    """Decode over a paged cache (include/kvq.h part 3) with its own workspace.

    k/v_pages [num_pages, Hkv, page_size, d] int8, k/v_scale_pages
    [num_pages, Hkv, page_size] fp32, block_table [B, max_pages_per_seq]
    int32, lengths [B] int32 (or None with a uniform max_seq_len)."""

    def __init__(self, q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, lengths, out,
                 max_seq_len=0, softmax_scale=0.0, num_splits=0, k_new=None, v_new=None, stream=None):
        check_paged(q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, lengths, out, k_new, v_new)
        B, Hq, d = q.shape
        P_, Hkv, page, _ = k_pages.shape
        self.keep = (q, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, lengths, out, k_new, v_new)
        self.params = PagedDecodeParams(B, Hq, Hkv, d, page, P_, int(block_table.shape[1]), int(max_seq_len),
                                        _ptr(block_table), _ptr(lengths), _ptr(q), _ptr(k_pages), _ptr(v_pages),
                                        _ptr(k_scale_pages), _ptr(v_scale_pages), _ptr(out),
                                        float(softmax_scale), int(num_splits), _ptr(k_new), _ptr(v_new))
        self.ws_bytes = int(lib().kvq_paged_decode_workspace_size(ctypes.byref(self.params)))
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=q.device)
        if self.ws_bytes:
            workspace_init(self.ws, self.ws_bytes, stream)
        self._launch = lib().kvq_paged_decode_launch
        self._args = (ctypes.byref(self.params), _ptr(self.ws), self.ws_bytes)

    def __call__(self, stream=None) -> None:
        code = self._launch(*self._args, stream if isinstance(stream, int) else _stream(stream))
        if code != HIP_SUCCESS:
            raise KvqError("kvq_paged_decode_launch", code)


def paged_append(k_new, v_new, k_pages, v_pages, k_scale_pages, v_scale_pages, block_table, positions=None,
                 uniform_position=0, stream=None) -> None:
    """One new K/V token per (b, kv head) into its page slot (kvq_paged_append_launch)."""
    P_, Hkv, page, d = _check_cache(k_pages, v_pages, k_scale_pages, v_scale_pages, "pages")
    if block_table.dim() != 2:
        raise ValueError("block_table: want [B, max_pages_per_seq]")
    B = block_table.shape[0]
    _need(block_table, torch.int32, tuple(block_table.shape), "block_table")
    _check_new_rows(k_new, v_new, B, Hkv, d)
    if positions is not None:
        _need(positions, torch.int32, (B,), "positions")
    p = PagedAppendParams(B, Hkv, d, page, P_, int(block_table.shape[1]), _ptr(block_table), _ptr(positions),
                          int(uniform_position), _ptr(k_new), _ptr(v_new), _ptr(k_pages), _ptr(v_pages),
                          _ptr(k_scale_pages), _ptr(v_scale_pages))
    _check("kvq_paged_append_launch", lib().kvq_paged_append_launch(ctypes.byref(p), _stream(stream)))


def prefill(k_new, v_new, k_cache, v_cache, k_scale, v_scale, start=None, uniform_start=0, block_table=None,
            stream=None) -> None:
    """Quantise L new tokens per (b, kv head) into the cache (kvq_prefill_quantize_launch).

    k_new/v_new [B, Hkv, L, d] fp32 or bf16; the cache is contiguous
    ([B, Hkv, cap, d]) or, with block_table [B, max_pages], a page pool
    ([num_pages, Hkv, page_size, d]); start [B] int32 or uniform_start."""
    B, Hkv, L, d = k_new.shape
    if k_new.dtype == torch.bfloat16:
        dt = DTYPE_BF16
    elif k_new.dtype == torch.float32:
        dt = DTYPE_F32
    else:
        raise TypeError("k_new must be float32 or bfloat16")
    for t, n in ((k_new, "k_new"), (v_new, "v_new")):
        _need(t, k_new.dtype, (B, Hkv, L, d), n)
    X, Hkv2, T, d2 = _check_cache(k_cache, v_cache, k_scale, v_scale)
    if (Hkv2, d2) != (Hkv, d):
        raise ValueError("shape mismatch")
    if start is not None:
        _need(start, torch.int32, (B,), "start")
    if block_table is None:
        if X != B:
            raise ValueError("shape mismatch")
        cap = T
        pg = (0, 0, 0)
    else:
        if block_table.dim() != 2 or block_table.shape[0] != B:
            raise ValueError("block_table: want [B, max_pages_per_seq]")
        _need(block_table, torch.int32, tuple(block_table.shape), "block_table")
        cap = 0
        pg = (T, X, int(block_table.shape[1]))
    p = PrefillParams(B, Hkv, d, L, dt, _ptr(k_new), _ptr(v_new), _ptr(start), int(uniform_start), cap,
                      _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_table), *pg)
    _check("kvq_prefill_quantize_launch", lib().kvq_prefill_quantize_launch(ctypes.byref(p), _stream(stream)))


def _attention_shapes(q, k, v, out):
    M, d = q.shape
    N = k.shape[0]
    _need(q, torch.float32, (M, d), "q")
    _need(k, torch.float32, (N, d), "k")
    _need(v, torch.float32, (N, d), "v")
    if out is None:
        out = torch.empty_like(q)
    _need(out, torch.float32, (M, d), "out")
    return M, N, d, out


def attention_online(q, k, v, out=None, stream=None) -> torch.Tensor:
    """softmax(q k^T / sqrt(d)) v through the reference ABI (attention_online_launch):
    q [M, d], k/v [N, d] fp32; split workspaces are owned by the library."""
    M, N, d, out = _attention_shapes(q, k, v, out)
    _check("attention_online_launch",
           lib().attention_online_launch(_ptr(q), _ptr(k), _ptr(v), _ptr(out), M, N, d, _stream(stream)))
    return out


def attention_solve(q, k, v, out=None) -> torch.Tensor:
    """The reference's compatibility `solve(Q, K, V, output, M, N, d)` of
    attention/softmax_new.cu:283-287 (libkvq_attention.so): asynchronous on the
    null stream, errors not reported."""
    M, N, d, out = _attention_shapes(q, k, v, out)
    attention_lib().solve(_ptr(q), _ptr(k), _ptr(v), _ptr(out), M, N, d)
    return out


def attention_params(q, k, v, out, softmax_scale: float = 0.0, num_splits: int = 0) -> AttentionParams:
    M, N, d, out = _attention_shapes(q, k, v, out)
    return AttentionParams(M, N, d, _ptr(q), _ptr(k), _ptr(v), _ptr(out), float(softmax_scale), int(num_splits))


def attention_workspace_size(p: AttentionParams) -> int:
    return int(lib().kvq_attention_workspace_size(ctypes.byref(p)))


def attention(q, k, v, out=None, softmax_scale: float = 0.0, num_splits: int = 0, workspace=None,
              stream=None) -> torch.Tensor:
    """softmax(q k^T * scale) v (kvq_attention_launch) with a caller-owned
    workspace (allocated here when none is given)."""
    if out is None:
        out = torch.empty_like(q)
    p = attention_params(q, k, v, out, softmax_scale, num_splits)
    n = attention_workspace_size(p)
    if n and workspace is None:
        workspace = torch.empty(n, dtype=torch.uint8, device=q.device)
    nb = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check("kvq_attention_launch", lib().kvq_attention_launch(ctypes.byref(p), _ptr(workspace), nb,
                                                              _stream(stream)))
    return out


def reference_plan(H: int, N: int, d: int, q_ptr: int = 256, k_ptr: int = 4096, v_ptr: int = 8192) -> PlanInfo:
    """Plan of kv_int8_split_launch for [H, N, d] (host-only; the pointers only
    set the alignment)."""
    info = PlanInfo()
    _check("kvq_reference_plan", lib().kvq_reference_plan(q_ptr, k_ptr, v_ptr, H, N, d, ctypes.byref(info)))
    return info


def decode_plan(p: DecodeParams) -> PlanInfo:
    """Plan of kvq_decode_launch for p (host-only)."""
    info = PlanInfo()
    _check("kvq_decode_plan", lib().kvq_decode_plan(ctypes.byref(p), ctypes.byref(info)))
    return info


def paged_decode_plan(p: PagedDecodeParams) -> PlanInfo:
    """Plan of kvq_paged_decode_launch for p (host-only)."""
    info = PlanInfo()
    _check("kvq_paged_decode_plan", lib().kvq_paged_decode_plan(ctypes.byref(p), ctypes.byref(info)))
    return info


def attention_plan(p: AttentionParams) -> PlanInfo:
    """Plan of kvq_attention_launch for p (host-only)."""
    info = PlanInfo()
    _check("kvq_attention_plan", lib().kvq_attention_plan(ctypes.byref(p), ctypes.byref(info)))
    return info


def diagnostics() -> int:
    """kvq_diagnostics(): bit 0 KVQ_DEBUG_SYNC, bits 4-7 KVQ_FORCE_KERNEL."""
    return int(lib().kvq_diagnostics())


def default_softmax_scale(d: int) -> float:
    """1/sqrtf(d) in fp32, as kv_cache/KV_int8_split_optimized.cu:335."""
    import numpy as np
    return float(np.float32(1.0) / np.sqrt(np.float32(d)))


def kv_bytes(lengths, num_kv_heads: int, head_dim: int) -> int:
    """Algorithmic KV-cache bytes one decode step reads: sum_b len_b * Hkv * (2*d + 8)."""
    total = int(sum(int(x) for x in lengths))
    return total * num_kv_heads * (2 * head_dim + 8)


__all__ = ["lib", "version", "solve", "kv_int8_split_launch", "DecodeParams", "AppendParams", "Decoder",
           "decode", "decode_params", "decode_launch", "workspace_size", "workspace_init", "new_workspace",
           "append", "quantize_rows", "kv_bytes", "KvqError", "EXPORTS", "PagedDecodeParams",
           "PagedAppendParams", "PagedDecoder", "paged_append", "PrefillParams", "prefill", "DTYPE_F32",
           "DTYPE_BF16", "AttentionParams", "attention_online", "attention_params", "attention_workspace_size",
           "attention", "PlanInfo", "reference_plan", "decode_plan", "paged_decode_plan", "attention_plan", "diagnostics",
           "attention_lib", "attention_solve", "decode_launch_noalloc", "NOALLOC_SCRATCH_BYTES"]
