"""numpy front end for the CPU oracle (liboracle.so built from kvq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg.  The product (libkvq.so and the
cuda-operators_amd package) never imports this module.

Every function takes/returns C-contiguous numpy arrays in the layouts of the
reference ABI (kv_cache/KV_int8_split_optimized.cu:294-304):
  Q[H,d] fp32, K/V[H,N,d] int8, k_scale/v_scale[H,N] fp32, out[H,d] fp32
and of the batched extension:
  q[B,Hq,d], k/v[B,Hkv,cap,d], scales[B,Hkv,cap], lengths[B] int32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# KVQ_ORACLE_SANITIZED=1 selects the AddressSanitizer + UBSan builds
# (oracle/_asan, make target `sanitize`); the process must then run with the
# ASan runtime preloaded (tests/test_sanitizers_cpu.py does this).
SANITIZED = os.environ.get("KVQ_ORACLE_SANITIZED", "") == "1"
LIB_DIR = os.path.join(HERE, "_asan") if SANITIZED else HERE
LIB_PATH = os.path.join(LIB_DIR, "liboracle.so")

_c_f32p = ctypes.POINTER(ctypes.c_float)
_c_f64p = ctypes.POINTER(ctypes.c_double)
_c_i8p = ctypes.POINTER(ctypes.c_int8)
_c_i32p = ctypes.POINTER(ctypes.c_int32)

_lock = threading.Lock()
_libs: dict[str, ctypes.CDLL] = {}


def build(plants: bool = False) -> None:
    """Compile the oracle (and optionally the planted-mistake variants) with make."""
    targets = ["sanitize"] if SANITIZED else ["all"] + (["plants"] if plants else [])
    subprocess.run(["make", "-s", "-C", HERE] + targets, check=True)


def plant_path(plant: int) -> str:
    return os.path.join(LIB_DIR, "_plant", f"liboracle_plant{plant}.so")


def _load(path: str) -> ctypes.CDLL:
    with _lock:
        lib = _libs.get(path)
        if lib is not None:
            return lib
        if not os.path.exists(path):
            raise FileNotFoundError(f"oracle library not built: {path} (run make -C oracle)")
        lib = ctypes.CDLL(path)
        lib.kvq_ref_head_f32.argtypes = [_c_f32p, _c_i8p, _c_i8p, _c_f32p, _c_f32p, _c_f32p,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.kvq_ref_head_f32.restype = None
        dec = [_c_f32p, _c_i8p, _c_i8p, _c_f32p, _c_f32p, _c_i32p,
               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.kvq_ref_decode_f32.argtypes = dec + [_c_f32p]
        lib.kvq_ref_decode_f32.restype = None
        lib.kvq_ref_decode_f64.argtypes = dec + [_c_f64p]
        lib.kvq_ref_decode_f64.restype = None
        lib.kvq_ref_quantize_rows.argtypes = [_c_f32p, ctypes.c_int64, ctypes.c_int, _c_i8p, _c_f32p]
        lib.kvq_ref_quantize_rows.restype = None
        lib.kvq_ref_append.argtypes = [_c_f32p, _c_f32p, _c_i8p, _c_i8p, _c_f32p, _c_f32p, _c_i32p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int]
        lib.kvq_ref_append.restype = None
        lib.kvq_ref_attention_f32.argtypes = [_c_f32p, _c_f32p, _c_f32p, _c_f32p, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int]
        lib.kvq_ref_attention_f32.restype = None
        lib.kvq_ref_plant_id.restype = ctypes.c_int
        lib.kvq_ref_max_threads.restype = ctypes.c_int
        _libs[path] = lib
        return lib


def _p(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctype)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


class Oracle:
    """Bound view of one oracle build (the real one, or a planted variant)."""

    def __init__(self, path: str = LIB_PATH):
        self.path = path
        self.lib = _load(path)

    @property
    def plant(self) -> int:
        return int(self.lib.kvq_ref_plant_id())

    @property
    def threads(self) -> int:
        return int(self.lib.kvq_ref_max_threads())

    # -- reference ABI shape -------------------------------------------------
    def head_f32(self, Q, K, V, ks, vs) -> np.ndarray:
        """cpu_reference restated: Q[H,d], K/V[H,N,d], ks/vs[H,N] -> out[H,d] fp32."""
        Q, K, V = _c(Q, np.float32), _c(K, np.int8), _c(V, np.int8)
        ks, vs = _c(ks, np.float32), _c(vs, np.float32)
        H, N, d = K.shape
        assert Q.shape == (H, d) and V.shape == (H, N, d) and ks.shape == (H, N) == vs.shape
        out = np.empty((H, d), np.float32)
        self.lib.kvq_ref_head_f32(_p(Q, _c_f32p), _p(K, _c_i8p), _p(V, _c_i8p), _p(ks, _c_f32p),
                                  _p(vs, _c_f32p), _p(out, _c_f32p), H, N, d)
        return out

    # -- batched / GQA / ragged --------------------------------------------
    def _decode(self, fn, out_dtype, q, k, v, ks, vs, lengths, uniform_len):
        q, k, v = _c(q, np.float32), _c(k, np.int8), _c(v, np.int8)
        ks, vs = _c(ks, np.float32), _c(vs, np.float32)
        B, Hq, d = q.shape
        Bk, Hkv, cap, dk = k.shape
        assert Bk == B and dk == d and v.shape == k.shape and ks.shape == (B, Hkv, cap) == vs.shape
        assert Hq % Hkv == 0
        lp = None
        if lengths is not None:
            lengths = _c(lengths, np.int32)
            assert lengths.shape == (B,)
            lp = _p(lengths, _c_i32p)
        out = np.empty((B, Hq, d), out_dtype)
        fn(_p(q, _c_f32p), _p(k, _c_i8p), _p(v, _c_i8p), _p(ks, _c_f32p), _p(vs, _c_f32p), lp,
           B, Hq, Hkv, cap, d, int(uniform_len if uniform_len is not None else cap),
           _p(out, _c_f32p if out_dtype == np.float32 else _c_f64p))
        return out

    def decode_f32(self, q, k, v, ks, vs, lengths=None, uniform_len=None) -> np.ndarray:
        return self._decode(self.lib.kvq_ref_decode_f32, np.float32, q, k, v, ks, vs, lengths,
                            uniform_len)

    def decode_f64(self, q, k, v, ks, vs, lengths=None, uniform_len=None) -> np.ndarray:
        return self._decode(self.lib.kvq_ref_decode_f64, np.float64, q, k, v, ks, vs, lengths,
                            uniform_len)

    # -- dense attention -------------------------------------------------------
    def attention_f32(self, Q, K, V) -> np.ndarray:
        """softmax(Q K^T / sqrt(d)) V for Q[M,d], K/V[N,d] fp32 (attention/softmax_new.cu)."""
        Q, K, V = _c(Q, np.float32), _c(K, np.float32), _c(V, np.float32)
        M, d = Q.shape
        N = K.shape[0]
        assert K.shape == (N, d) == V.shape
        out = np.empty((M, d), np.float32)
        self.lib.kvq_ref_attention_f32(_p(Q, _c_f32p), _p(K, _c_f32p), _p(V, _c_f32p), _p(out, _c_f32p),
                                       M, N, d)
        return out

    # -- quantiser -----------------------------------------------------------
    def quantize_rows(self, x):
        """x[..., d] fp32 -> (int8[..., d], scale[...] fp32), one scale per row."""
        x = _c(x, np.float32)
        d = x.shape[-1]
        rows = x.size // d if d else 0
        q = np.empty(x.shape, np.int8)
        s = np.empty(x.shape[:-1], np.float32)
        self.lib.kvq_ref_quantize_rows(_p(x, _c_f32p), rows, d, _p(q, _c_i8p), _p(s, _c_f32p))
        return q, s

    def append(self, k_new, v_new, k, v, ks, vs, positions=None, uniform_pos=0):
        """In-place append of one token per (b, kv_head) into numpy caches."""
        k_new, v_new = _c(k_new, np.float32), _c(v_new, np.float32)
        for a, dt in ((k, np.int8), (v, np.int8), (ks, np.float32), (vs, np.float32)):
            assert a.dtype == dt and a.flags.c_contiguous
        B, Hkv, cap, d = k.shape
        assert k_new.shape == (B, Hkv, d) == v_new.shape
        pp = None
        if positions is not None:
            positions = _c(positions, np.int32)
            pp = _p(positions, _c_i32p)
        self.lib.kvq_ref_append(_p(k_new, _c_f32p), _p(v_new, _c_f32p), _p(k, _c_i8p), _p(v, _c_i8p),
                                _p(ks, _c_f32p), _p(vs, _c_f32p), pp, int(uniform_pos), B, Hkv, cap, d)


_default: Oracle | None = None


def get() -> Oracle:
    global _default
    if _default is None:
        _default = Oracle(LIB_PATH)
    return _default
