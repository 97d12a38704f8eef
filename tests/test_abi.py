"""The C ABI without a GPU: the library loads, exports every function include/ffkv.h declares, and rejects
invalid arguments with the documented status codes before it touches a device."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared_functions() -> list[str]:
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"\b(ffkv_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_exports_every_declared_symbol(ff):
    names = declared_functions()
    assert "ffkv_append" in names and "ffkv_paged_decode" in names
    for n in names:
        assert hasattr(ff.lib, n), f"{n} is declared in include/ but not exported by {ff.LIB_PATH}"


def test_version(ff):
    assert "gfx950" in ff.version()


def _append(ff, **kw):
    a = dict(k_src=16, v_src=16, src_dtype=ff.DTYPE_BF16, k_cache=16, v_cache=16, cache_dtype=ff.DTYPE_BF16,
             k_scale=None, v_scale=None, block_table=16, context_lens=None, batch=1, seq_len=1, num_kv_heads=8,
             head_dim=128, block_size=16, max_blocks=4, num_blocks=4, stream=None)
    a.update(kw)
    return ff.lib.ffkv_append(*a.values())


def _decode(ff, **kw):
    a = dict(q=16, out=16, qo_dtype=ff.DTYPE_BF16, k_cache=16, v_cache=16, cache_dtype=ff.DTYPE_BF16,
             k_scale=None, v_scale=None, block_table=16, context_lens=16, batch=1, num_heads=32, num_kv_heads=8,
             head_dim=128, block_size=16, max_blocks=4, num_blocks=4, max_context_len=0, scale=0.0,
             workspace=None, workspace_bytes=0, stream=None)
    a.update(kw)
    return ff.lib.ffkv_paged_decode(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(block_size=32), -2),
    (dict(head_dim=100), -2),         # not a multiple of 8
    (dict(head_dim=136), -2),         # over 128 and not 256
    (dict(head_dim=0), -2),
    (dict(src_dtype=3), -2),          # int8 is not an activation dtype
    (dict(cache_dtype=7), -2),        # the reference's UNKNOWN
    (dict(batch=-1), -1),
    (dict(num_kv_heads=0), -1),
    (dict(k_cache=None), -1),
    (dict(block_table=None), -1),
    (dict(cache_dtype=3), -1),        # int8 cache without scales
    (dict(cache_dtype=8), -1),        # fp8 cache without scales
    (dict(k_src=18), -1),             # misaligned
])
def test_append_rejects(ff, kw, code):
    assert _append(ff, **kw) == code
    assert ff.lib.ffkv_last_error().decode() != ""


def test_append_empty_is_ok(ff):
    assert _append(ff, batch=0, k_src=None, v_src=None) == 0
    assert _append(ff, seq_len=0) == 0
    assert ff.lib.ffkv_last_error().decode() == ""


@pytest.mark.parametrize("kw,code", [
    (dict(block_size=8), -2),
    (dict(head_dim=84), -2),          # not a multiple of 8
    (dict(head_dim=144), -2),         # over 128 and not 256
    (dict(qo_dtype=3), -2),
    (dict(num_heads=30), -1),         # not a multiple of num_kv_heads
    (dict(num_heads=8 * 17, cache_dtype=0), -2),  # GQA group above 16 on an fp32 cache (the generic kernel)
    (dict(num_heads=70000 * 2, num_kv_heads=70000), -2),  # more than 65535 query heads
    (dict(context_lens=None), -1),
    (dict(q=None), -1),
    (dict(cache_dtype=3), -1),
    (dict(q=20), -1),
    (dict(batch=70000), -2),
])
def test_decode_rejects(ff, kw, code):
    assert _decode(ff, **kw) == code
    assert ff.lib.ffkv_last_error().decode() != ""


def test_decode_workspace_too_small(ff):
    need = ff.decode_workspace_bytes(4, 32, 128, 600, 0)
    assert need > 0
    assert _decode(ff, batch=4, max_blocks=600, workspace=256, workspace_bytes=4096) == ff.ERR_WORKSPACE


def test_workspace_bytes_monotone(ff):
    a = ff.decode_workspace_bytes(8, 28, 128, 2049, 0)
    b = ff.decode_workspace_bytes(8, 28, 128, 2049, 8192)
    assert a >= b > 0
    # the matrix-core kernel splits any row over work items, so even one-chunk rows need partial slots
    assert ff.decode_workspace_bytes(8, 28, 128, 16, 0) > 0
    assert ff.decode_workspace_bytes(0, 28, 128, 2049, 0) == 0



def _decode_shared(ff, **kw):
    a = dict(q=16, out=16, qo_dtype=ff.DTYPE_BF16, k_cache=16, v_cache=16, cache_dtype=ff.DTYPE_BF16,
             k_scale=None, v_scale=None, block_table=16, context_lens=16, batch=1, num_heads=32, num_kv_heads=8,
             head_dim=128, block_size=16, max_blocks=4, num_blocks=4, max_context_len=0, scale=0.0,
             shared_blocks=2, workspace=None, workspace_bytes=0, stream=None)
    a.update(kw)
    return ff.lib.ffkv_paged_decode_shared_prefix(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(shared_blocks=-1), -1),
    (dict(shared_blocks=5), -1),      # beyond max_blocks
    (dict(block_size=8), -2),
    (dict(num_heads=30), -1),
    (dict(q=None), -1),
    (dict(cache_dtype=3), -1),        # int8 without scales: the plain decode's checks apply
])
def test_decode_shared_prefix_rejects(ff, kw, code):
    assert _decode_shared(ff, **kw) == code
    assert ff.lib.ffkv_last_error().decode() != ""


def test_decode_shared_prefix_workspace(ff):
    plain = ff.decode_workspace_bytes(120, 32, 128, 200, 0)
    shared = ff.lib.ffkv_decode_shared_prefix_workspace_bytes(120, 32, 8, 128, 200, 0, 128)
    # room for the prefix partials (chunks x rows x heads x (head_dim + 2) floats) on top of the plain decode's
    assert shared > plain + 120 * 32 * 130 * 4
    assert ff.lib.ffkv_decode_shared_prefix_workspace_bytes(120, 32, 8, 128, 200, 0, 0) == plain
    need = ff.lib.ffkv_decode_shared_prefix_workspace_bytes(4, 32, 8, 128, 600, 0, 100)
    assert need > ff.decode_workspace_bytes(4, 32, 128, 600, 0)
    assert _decode_shared(ff, batch=4, max_blocks=600, shared_blocks=100, workspace=256,
                          workspace_bytes=4096) == ff.ERR_WORKSPACE


def _rope_append(ff, **kw):
    a = dict(q=16, k=16, v=16, src_dtype=ff.DTYPE_BF16, k_cache=16, v_cache=16, cache_dtype=ff.DTYPE_BF16,
             k_scale=None, v_scale=None, block_table=16, context_lens=None, batch=1, seq_len=1, num_heads=32,
             num_kv_heads=8, head_dim=128, block_size=16, max_blocks=4, num_blocks=4, theta=1e6, stream=None)
    a.update(kw)
    return ff.lib.ffkv_rope_append(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(block_size=32), -2),
    (dict(head_dim=96), -2),
    (dict(src_dtype=3), -2),
    (dict(cache_dtype=7), -2),
    (dict(batch=-1), -1),
    (dict(num_kv_heads=0), -1),
    (dict(theta=0.0), -1),
    (dict(theta=float("nan")), -1),
    (dict(theta=float("inf")), -1),
    (dict(k=None), -1),
    (dict(v=None), -1),
    (dict(block_table=None), -1),
    (dict(cache_dtype=3), -1),        # int8 cache without scales
    (dict(q=18), -1),                 # misaligned
])
def test_rope_append_rejects(ff, kw, code):
    assert _rope_append(ff, **kw) == code
    assert ff.lib.ffkv_last_error().decode() != ""


def test_rope_rejects_and_empty(ff):
    assert ff.lib.ffkv_rope(16, 16, ff.DTYPE_BF16, None, 1, 1, 32, 8, 96, 1e6, None) == -2
    assert ff.lib.ffkv_rope(16, None, ff.DTYPE_BF16, None, 1, 1, 32, 8, 128, 1e6, None) == -1
    assert ff.lib.ffkv_rope(16, 16, ff.DTYPE_BF16, None, 0, 1, 32, 8, 128, 1e6, None) == 0
    assert ff.lib.ffkv_rope(None, 16, ff.DTYPE_BF16, None, 1, 0, 0, 8, 128, 1e6, None) == 0
    assert _rope_append(ff, batch=0, k=None, v=None, q=None) == 0


def _prefill(ff, **kw):
    a = dict(q=16, out=16, qo_dtype=ff.DTYPE_BF16, k_cache=16, v_cache=16, cache_dtype=ff.DTYPE_BF16,
             k_scale=None, v_scale=None, block_table=16, context_lens=16, batch=1, seq_len=8, num_heads=32,
             num_kv_heads=8, head_dim=128, block_size=16, max_blocks=4, num_blocks=4, max_context_len=0, scale=0.0,
             stream=None)
    a.update(kw)
    return ff.lib.ffkv_paged_prefill(*a.values())


@pytest.mark.parametrize("kw,code", [
    (dict(block_size=8), -2),
    (dict(head_dim=80), -2),
    (dict(qo_dtype=3), -2),
    (dict(cache_dtype=0), -2),                     # fp32 caches: decode only
    (dict(num_heads=30), -1),
    (dict(batch=-1), -1),
    (dict(q=None), -1),
    (dict(context_lens=None), -1),                 # paged mode needs context_lens
    (dict(cache_dtype=3), -1),                     # int8 without scales
    (dict(cache_dtype=3, block_table=None, k_scale=16, v_scale=16), -2),  # int8 needs pages
    (dict(out=24), -1),                            # misaligned
])
def test_prefill_rejects(ff, kw, code):
    assert _prefill(ff, **kw) == code
    assert ff.lib.ffkv_last_error().decode() != ""


def test_prefill_empty_and_contiguous_args_ok(ff):
    assert _prefill(ff, batch=0, q=None) == 0
    assert _prefill(ff, seq_len=0) == 0
    assert ff.lib.ffkv_last_error().decode() == ""


@pytest.mark.parametrize("Hkv,D", [(8, 128), (4, 128), (8, 64), (2, 256), (8, 96)])
def test_kv_block_bytes_matches_the_pool_tensors(ff, Hkv, D):
    """ffkv_kv_block_bytes x num_blocks = the bytes of the tensors kernels::append_kv_cache takes for a pool of
    that many blocks: K and V pages [N, 16, Hkv, D] of the cache type, plus int8's per-token-per-head fp32 scales
    [N, 16, Hkv] for K and V (fp8's per-head scales [Hkv] do not grow with N).  16-bit caches give the reference's
    divisor 16 * Hkv * D * 2 * 2 (src/engine.cc:90-96)."""
    import numpy as np

    N = 7
    elem = {ff.DTYPE_F32: 4, ff.DTYPE_F16: 2, ff.DTYPE_BF16: 2, ff.DTYPE_I8: 1, ff.DTYPE_FP8_E4M3: 1}
    for dt, es in elem.items():
        pages = 2 * np.empty((N, 16, Hkv, D), dtype=f"u{es}").nbytes
        scales = 2 * np.empty((N, 16, Hkv), dtype=np.float32).nbytes if dt == ff.DTYPE_I8 else 0
        assert ff.kv_block_bytes(dt, Hkv, D) * N == pages + scales, dt
    assert ff.kv_block_bytes(ff.DTYPE_BF16, Hkv, D) == 16 * Hkv * D * 2 * 2
    # an 8-bit pool holds about twice the blocks of a 16-bit one in the same memory
    assert ff.kv_block_bytes(ff.DTYPE_FP8_E4M3, Hkv, D) * 2 == ff.kv_block_bytes(ff.DTYPE_BF16, Hkv, D)
    assert ff.kv_block_bytes(ff.DTYPE_I8, Hkv, D) < ff.kv_block_bytes(ff.DTYPE_BF16, Hkv, D)


def test_kv_block_bytes_rejects(ff):
    assert ff.kv_block_bytes(7, 8, 128) == 0  # UNKNOWN
    assert ff.kv_block_bytes(ff.DTYPE_BF16, 0, 128) == 0
    assert ff.kv_block_bytes(ff.DTYPE_BF16, 8, -1) == 0
