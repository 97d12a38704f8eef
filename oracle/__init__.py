"""CPU checker for the paged KV-cache path.  TEST INFRASTRUCTURE ONLY.

numpy front end to ``oracle/libffkv_oracle.so`` (the C restatement in ``ffkv_oracle.c``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this package, and only as the
checker or the timed CPU baseline; the product library never loads it.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
LIB_PATH = _DIR / "libffkv_oracle.so"
REF_SCHED_PATH = _DIR / "_ref" / "libref_sched.so"

DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_I8, DTYPE_FP8 = 0, 1, 2, 3, 8
_NP_STORAGE = {DTYPE_F32: np.float32, DTYPE_F16: np.uint16, DTYPE_BF16: np.uint16, DTYPE_I8: np.int8,
               DTYPE_FP8: np.uint8}


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run `make -C oracle`")
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    lib.ffo_append.restype = i32
    lib.ffo_append.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32]
    lib.ffo_paged_decode.restype = i32
    lib.ffo_paged_decode.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                     i32, f32, vp, i32]
    lib.ffo_paged_decode_f64.restype = i32
    lib.ffo_paged_decode_f64.argtypes = [vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                         i32, f32, vp]
    lib.ffo_paged_prefill_f64.restype = i32
    lib.ffo_paged_prefill_f64.argtypes = [vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                          i32, f32, vp]
    lib.ffo_rope.restype = i32
    lib.ffo_rope.argtypes = [vp, i32, vp, i32, i32, i32, i32, f32]
    lib.ffo_quant_i8_row.restype = f32
    lib.ffo_quant_i8_row.argtypes = [vp, i32, vp]
    for name, src, dst in [("f32_to_bf16", vp, vp), ("f32_to_f16", vp, vp), ("f32_to_e4m3", vp, vp),
                           ("e4m3_to_f32", vp, vp), ("bf16_to_f32", vp, vp), ("f16_to_f32", vp, vp)]:
        fn = getattr(lib, "ffo_cvt_" + name)
        fn.restype = None
        fn.argtypes = [src, dst, ctypes.c_size_t]
    lib.ffo_default_threads.restype = i32
    return lib


lib = _load()


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype=None):
    if a is None:
        return None
    return np.ascontiguousarray(a if dtype is None else a.astype(dtype, copy=False))


def default_threads() -> int:
    return int(lib.ffo_default_threads())


# ---- conversions -------------------------------------------------------------------------------------------

def _cvt(name, x, out_dtype):
    x = np.ascontiguousarray(x)
    y = np.empty(x.shape, dtype=out_dtype)
    getattr(lib, "ffo_cvt_" + name)(_p(x), _p(y), x.size)
    return y


def f32_to_bf16(x):
    return _cvt("f32_to_bf16", np.asarray(x, np.float32), np.uint16)


def f32_to_f16(x):
    return _cvt("f32_to_f16", np.asarray(x, np.float32), np.uint16)


def f32_to_e4m3(x):
    return _cvt("f32_to_e4m3", np.asarray(x, np.float32), np.uint8)


def e4m3_to_f32(q):
    return _cvt("e4m3_to_f32", np.asarray(q, np.uint8), np.float32)


def bf16_to_f32(h):
    return _cvt("bf16_to_f32", np.asarray(h, np.uint16), np.float32)


def f16_to_f32(h):
    return _cvt("f16_to_f32", np.asarray(h, np.uint16), np.float32)


def quant_i8_row(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.int8)
    s = lib.ffo_quant_i8_row(_p(x), x.size, _p(q))
    return q, np.float32(s)


# ---- path functions ----------------------------------------------------------------------------------------

def append(k_src, v_src, src_dtype, k_cache, v_cache, cache_dtype, block_table, context_lens, k_scale=None,
           v_scale=None, num_blocks=None):
    """In-place append into numpy page pools (storage arrays as produced by ``_NP_STORAGE``)."""
    B, S, Hkv, D = k_src.shape
    bt = _c(block_table, np.int32)
    ctx = _c(context_lens, np.int32)
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    for a in (k_cache, v_cache, k_scale, v_scale):
        assert a is None or a.flags.c_contiguous
    rc = lib.ffo_append(_p(_c(k_src)), _p(_c(v_src)), src_dtype, _p(k_cache), _p(v_cache), cache_dtype,
                        _p(k_scale), _p(v_scale), _p(bt), _p(ctx), B, S, Hkv, D, 16, bt.shape[-1], N)
    if rc != 0:
        raise ValueError(f"ffo_append returned {rc}")


def rope(x, dtype, context_lens, theta):
    """Rotated copy of x [B, S, H, D] (storage array of `dtype`)."""
    y = np.array(x, copy=True, order="C")
    B, S, H, D = y.shape
    ctx = _c(context_lens, np.int32)
    rc = lib.ffo_rope(_p(y), dtype, _p(ctx), B, S, H, D, theta)
    if rc != 0:
        raise ValueError(f"ffo_rope returned {rc}")
    return y


def paged_decode(q, qo_dtype, k_cache, v_cache, cache_dtype, block_table, context_lens, k_scale=None,
                 v_scale=None, max_context_len=0, scale=0.0, num_blocks=None, threads=0):
    """Returns (out in qo storage dtype [B, Hq*D], out_f32 [B, Hq, D])."""
    q = _c(q)
    B = q.shape[0]
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_cache.shape[2]
    bt = _c(block_table, np.int32)
    ctx = _c(context_lens, np.int32)
    out = np.zeros((B, Hq * D), dtype=_NP_STORAGE[qo_dtype])
    out32 = np.zeros((B, Hq, D), dtype=np.float32)
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    rc = lib.ffo_paged_decode(_p(q), _p(out), qo_dtype, _p(_c(k_cache)), _p(_c(v_cache)), cache_dtype,
                              _p(_c(k_scale, np.float32)), _p(_c(v_scale, np.float32)), _p(bt), _p(ctx), B, Hq, Hkv,
                              D, 16, bt.shape[-1], N, max_context_len, scale, _p(out32), threads)
    if rc != 0:
        raise ValueError(f"ffo_paged_decode returned {rc}")
    return out, out32


def paged_decode_f64(q, qo_dtype, k_cache, v_cache, cache_dtype, block_table, context_lens, k_scale=None,
                     v_scale=None, max_context_len=0, scale=0.0, num_blocks=None):
    q = _c(q)
    B = q.shape[0]
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_cache.shape[2]
    bt = _c(block_table, np.int32)
    ctx = _c(context_lens, np.int32)
    out = np.zeros((B, Hq, D), dtype=np.float64)
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    rc = lib.ffo_paged_decode_f64(_p(q), qo_dtype, _p(_c(k_cache)), _p(_c(v_cache)), cache_dtype,
                                  _p(_c(k_scale, np.float32)), _p(_c(v_scale, np.float32)), _p(bt), _p(ctx), B, Hq,
                                  Hkv, D, 16, bt.shape[-1], N, max_context_len, scale, _p(out))
    if rc != 0:
        raise ValueError(f"ffo_paged_decode_f64 returned {rc}")
    return out


def paged_prefill_f64(q, qo_dtype, k_cache, v_cache, cache_dtype, block_table, context_lens, k_scale=None,
                      v_scale=None, max_context_len=0, scale=0.0, num_blocks=None):
    """q [B, S, Hq, D] storage array; block_table None means contiguous K/V [B, S, Hkv, D].
    Returns float64 [B, S, Hq, D]."""
    q = _c(q)
    B, S, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    bt = None if block_table is None else _c(block_table, np.int32)
    ctx = None if context_lens is None else _c(context_lens, np.int32)
    out = np.zeros((B, S, Hq, D), dtype=np.float64)
    mb = 0 if bt is None else bt.shape[-1]
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    rc = lib.ffo_paged_prefill_f64(_p(q), qo_dtype, _p(_c(k_cache)), _p(_c(v_cache)), cache_dtype,
                                   _p(_c(k_scale, np.float32)), _p(_c(v_scale, np.float32)), _p(bt), _p(ctx), B, S,
                                   Hq, Hkv, D, mb, N, max_context_len, scale, _p(out))
    if rc != 0:
        raise ValueError(f"ffo_paged_prefill_f64 returned {rc}")
    return out
