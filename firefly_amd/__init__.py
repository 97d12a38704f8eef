"""firefly_amd - MI355X (gfx950) paged KV-cache path for Firefly.

The product is the shared library ``firefly_amd/libffkv.so`` (C ABI in ``include/ffkv.h``; C++ API in
``include/firefly/``).  This module loads it with ctypes and offers thin wrappers that take torch tensors, so
tests and benchmarks can drive the C ABI with device memory torch allocated.  There is no CPU fallback: if the
library is missing or fails to load, importing this package raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libffkv.so"

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_I8 = 3
DTYPE_FP8_E4M3 = 8

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED = -2
ERR_WORKSPACE = -3
ERR_HIP = -4

BLOCK_SIZE = 16
NOALLOC_SCRATCH_BYTES = 32 << 20  # FFKV_NOALLOC_SCRATCH_BYTES (include/ffkv.h)


class FFKVError(RuntimeError):
    """A C ABI call returned a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"ffkv error {code}: {message}")
        self.code = code


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run `python firefly_amd/build.py` (no CPU fallback exists)")
    # torch wheels bundle their own HIP runtime under the same soname (libamdhip64.so.7).  Loading torch first
    # makes libffkv.so bind to that already-loaded runtime, so there is one runtime per process and torch's
    # device pointers and streams are valid here; loading ours first would put two runtimes in the process.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | ctypes.RTLD_LOCAL)
    vp, i32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.ffkv_append.restype = i32
    lib.ffkv_append.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp]
    lib.ffkv_kv_block_bytes.restype = sz
    lib.ffkv_kv_block_bytes.argtypes = [i32, i32, i32]
    lib.ffkv_decode_workspace_bytes.restype = sz
    lib.ffkv_decode_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
    lib.ffkv_paged_decode.restype = i32
    lib.ffkv_paged_decode.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                      i32, f32, vp, sz, vp]
    lib.ffkv_paged_decode_noalloc.restype = i32
    lib.ffkv_paged_decode_noalloc.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32,
                                              i32, i32, f32, vp]
    lib.ffkv_decode_shared_prefix_workspace_bytes.restype = sz
    lib.ffkv_decode_shared_prefix_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32, i32]
    lib.ffkv_paged_decode_shared_prefix.restype = i32
    lib.ffkv_paged_decode_shared_prefix.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32,
                                                    i32, i32, i32, i32, f32, i32, vp, sz, vp]
    lib.ffkv_append_paged_decode.restype = i32
    lib.ffkv_append_paged_decode.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32,
                                             i32, i32, i32, i32, i32, f32, vp, sz, vp]
    lib.ffkv_paged_prefill.restype = i32
    lib.ffkv_paged_prefill.argtypes = [vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                       i32, i32, ctypes.c_float, vp]
    lib.ffkv_rope.restype = i32
    lib.ffkv_rope.argtypes = [vp, vp, i32, vp, i32, i32, i32, i32, i32, ctypes.c_float, vp]
    lib.ffkv_rope_append.restype = i32
    lib.ffkv_rope_append.argtypes = [vp, vp, vp, i32, vp, vp, i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                     i32, ctypes.c_float, vp]
    lib.ffkv_last_error.restype = ctypes.c_char_p
    lib.ffkv_last_error.argtypes = []
    lib.ffkv_version.restype = ctypes.c_char_p
    lib.ffkv_version.argtypes = []
    return lib


lib = _load()


def version() -> str:
    return lib.ffkv_version().decode()


def check(code: int) -> None:
    if code != OK:
        raise FFKVError(code, lib.ffkv_last_error().decode())


def torch_dtype_code(t) -> int:
    """ffkv dtype code of a torch tensor (uint8 storage is read as OCP fp8 e4m3)."""
    import torch

    table = {
        torch.float32: DTYPE_F32,
        torch.float16: DTYPE_F16,
        torch.bfloat16: DTYPE_BF16,
        torch.int8: DTYPE_I8,
        torch.uint8: DTYPE_FP8_E4M3,
    }
    fp8 = getattr(torch, "float8_e4m3fn", None)
    if fp8 is not None:
        table[fp8] = DTYPE_FP8_E4M3
    try:
        return table[t.dtype]
    except KeyError as e:
        raise TypeError(f"unsupported dtype {t.dtype}") from e


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def append_kv_cache(k, v, k_cache, v_cache, block_table, context_lens=None, k_scale=None, v_scale=None,
                    num_blocks: int | None = None, stream=None) -> None:
    """Append ``k``/``v`` ``[B, S, Hkv, D]`` into pages ``[N, 16, Hkv, D]`` (``ffkv_append``)."""
    B, S, Hkv, D = k.shape
    max_blocks = block_table.shape[-1]
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    check(lib.ffkv_append(_ptr(k), _ptr(v), torch_dtype_code(k), _ptr(k_cache), _ptr(v_cache),
                          torch_dtype_code(k_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_table),
                          _ptr(context_lens), B, S, Hkv, D, BLOCK_SIZE, max_blocks, N, _stream(stream)))


def paged_prefill(q, k_cache, v_cache, block_table, context_lens, out=None, k_scale=None, v_scale=None,
                  max_context_len: int = 0, scale: float = 0.0, num_blocks: int | None = None, stream=None):
    """Causal prefill attention (``ffkv_paged_prefill``): ``q`` ``[B, S, Hq, D]`` over the paged cache (queries at
    ``context_lens[b] + t``), or, with ``block_table=None``, over contiguous ``k_cache``/``v_cache``
    ``[B, S, Hkv, D]``.  Returns ``out`` ``[B, S, Hq * D]``."""
    import torch

    B, S, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    if out is None:
        out = torch.empty((B, S, Hq * D), dtype=q.dtype, device=q.device)
    max_blocks = 0 if block_table is None else block_table.shape[-1]
    N = (k_cache.shape[0] if num_blocks is None else num_blocks) if block_table is not None else 0
    check(lib.ffkv_paged_prefill(_ptr(q), _ptr(out), torch_dtype_code(q), _ptr(k_cache), _ptr(v_cache),
                                 torch_dtype_code(k_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_table),
                                 _ptr(context_lens), B, S, Hq, Hkv, D, BLOCK_SIZE, max_blocks, N, max_context_len,
                                 float(scale), _stream(stream)))
    return out


def apply_rope(q, k, context_lens=None, theta: float = 1e6, stream=None) -> None:
    """Rotary embedding of ``q`` ``[B, S, Hq, D]`` (or None) and ``k`` ``[B, S, Hkv, D]`` in place
    (``ffkv_rope``; the reference's ``kernels::apply_rope``)."""
    B, S, Hkv, D = k.shape
    Hq = 0 if q is None else q.shape[2]
    check(lib.ffkv_rope(_ptr(q), _ptr(k), torch_dtype_code(k), _ptr(context_lens), B, S, Hq, Hkv, D, float(theta),
                        _stream(stream)))


def rope_append_kv_cache(q, k, v, k_cache, v_cache, block_table, context_lens=None, theta: float = 1e6,
                         k_scale=None, v_scale=None, num_blocks: int | None = None, stream=None) -> None:
    """``apply_rope(q, k)`` then ``append_kv_cache(k, v, ...)`` in one kernel (``ffkv_rope_append``)."""
    B, S, Hkv, D = k.shape
    Hq = 0 if q is None else q.shape[2]
    max_blocks = block_table.shape[-1]
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    check(lib.ffkv_rope_append(_ptr(q), _ptr(k), _ptr(v), torch_dtype_code(k), _ptr(k_cache), _ptr(v_cache),
                               torch_dtype_code(k_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_table),
                               _ptr(context_lens), B, S, Hq, Hkv, D, BLOCK_SIZE, max_blocks, N, float(theta),
                               _stream(stream)))


def kv_block_bytes(cache_dtype: int, num_kv_heads: int, head_dim: int) -> int:
    """Bytes of one pool block (16 tokens of one layer, K and V, scales included) for a cache dtype."""
    return int(lib.ffkv_kv_block_bytes(cache_dtype, num_kv_heads, head_dim))


def decode_workspace_bytes(batch: int, num_heads: int, head_dim: int, max_blocks: int,
                           max_context_len: int = 0) -> int:
    return int(lib.ffkv_decode_workspace_bytes(batch, num_heads, head_dim, max_blocks, max_context_len))


def decode_workspace(batch: int, num_heads: int, head_dim: int, max_blocks: int, max_context_len: int = 0,
                     device=None, stream=None):
    """A decode workspace (uint8 tensor, contents irrelevant) sized by ``ffkv_decode_workspace_bytes``."""
    import torch

    n = max(decode_workspace_bytes(batch, num_heads, head_dim, max_blocks, max_context_len), 256)
    return torch.empty(n, dtype=torch.uint8, device=device if device is not None else "cuda")


def shared_prefix_workspace(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, max_blocks: int,
                            shared_blocks: int, max_context_len: int = 0, device=None):
    """A workspace for ``paged_attention_shared_prefix`` (``ffkv_decode_shared_prefix_workspace_bytes``)."""
    import torch

    n = max(int(lib.ffkv_decode_shared_prefix_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, max_blocks,
                                                              max_context_len, shared_blocks)), 256)
    return torch.empty(n, dtype=torch.uint8, device=device if device is not None else "cuda")


def paged_attention_shared_prefix(q, k_cache, v_cache, block_table, context_lens, shared_blocks: int, out=None,
                                  k_scale=None, v_scale=None, max_context_len: int = 0, scale: float = 0.0,
                                  workspace=None, num_blocks: int | None = None, stream=None):
    """Decode over rows whose first ``shared_blocks`` block-table entries are the same pages
    (``ffkv_paged_decode_shared_prefix``): the shared pages are attended once for all rows."""
    import torch

    B = q.shape[0]
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_cache.shape[2]
    if out is None:
        out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=q.device)
    max_blocks = block_table.shape[-1]
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.ffkv_paged_decode_shared_prefix(_ptr(q), _ptr(out), torch_dtype_code(q), _ptr(k_cache), _ptr(v_cache),
                                              torch_dtype_code(k_cache), _ptr(k_scale), _ptr(v_scale),
                                              _ptr(block_table), _ptr(context_lens), B, Hq, Hkv, D, BLOCK_SIZE,
                                              max_blocks, N, max_context_len, float(scale), int(shared_blocks),
                                              _ptr(workspace), ws_bytes, _stream(stream)))
    return out


def append_paged_attention(k_new, v_new, q, k_cache, v_cache, block_table, context_lens, out=None, k_scale=None,
                           v_scale=None, max_context_len: int = 0, scale: float = 0.0, workspace=None,
                           num_blocks: int | None = None, stream=None):
    """``append_kv_cache(k_new, v_new, ...)`` (one token per row) then ``paged_attention``, as one call
    (``ffkv_append_paged_decode``; a single launch for 16-bit caches fed in their own dtype)."""
    import torch

    B = q.shape[0]
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_cache.shape[2]
    if out is None:
        out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=q.device)
    max_blocks = block_table.shape[-1]
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.ffkv_append_paged_decode(_ptr(k_new), _ptr(v_new), torch_dtype_code(k_new), _ptr(q), _ptr(out),
                                       torch_dtype_code(q), _ptr(k_cache), _ptr(v_cache), torch_dtype_code(k_cache),
                                       _ptr(k_scale), _ptr(v_scale), _ptr(block_table), _ptr(context_lens), B, Hq,
                                       Hkv, D, BLOCK_SIZE, max_blocks, N, max_context_len, float(scale),
                                       _ptr(workspace), ws_bytes, _stream(stream)))
    return out


def paged_attention_noalloc(q, k_cache, v_cache, block_table, context_lens, out, k_scale=None, v_scale=None,
                            max_context_len: int = 0, scale: float = 0.0, num_blocks: int | None = None, stream=None):
    """PagedAttention decode that allocates no device memory (``ffkv_paged_decode_noalloc``): the split-K partials
    use the library's static per-GPU scratch.  ``out`` ``[B, 1, Hq * D]`` is the caller's."""
    B = q.shape[0]
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_cache.shape[2]
    max_blocks = block_table.shape[-1]
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    check(lib.ffkv_paged_decode_noalloc(_ptr(q), _ptr(out), torch_dtype_code(q), _ptr(k_cache), _ptr(v_cache),
                                        torch_dtype_code(k_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_table),
                                        _ptr(context_lens), B, Hq, Hkv, D, BLOCK_SIZE, max_blocks, N,
                                        max_context_len, float(scale), _stream(stream)))
    return out


def paged_attention(q, k_cache, v_cache, block_table, context_lens, out=None, k_scale=None, v_scale=None,
                    max_context_len: int = 0, scale: float = 0.0, workspace=None, num_blocks: int | None = None,
                    stream=None):
    """PagedAttention decode (``ffkv_paged_decode``).  ``q`` is ``[B, 1, Hq, D]`` (or ``[B, Hq, D]``)."""
    import torch

    B = q.shape[0]
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_cache.shape[2]
    if out is None:
        out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=q.device)
    max_blocks = block_table.shape[-1]
    N = k_cache.shape[0] if num_blocks is None else num_blocks
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib.ffkv_paged_decode(_ptr(q), _ptr(out), torch_dtype_code(q), _ptr(k_cache), _ptr(v_cache),
                                torch_dtype_code(k_cache), _ptr(k_scale), _ptr(v_scale), _ptr(block_table),
                                _ptr(context_lens), B, Hq, Hkv, D, BLOCK_SIZE, max_blocks, N, max_context_len,
                                float(scale), _ptr(workspace), ws_bytes, _stream(stream)))
    return out
