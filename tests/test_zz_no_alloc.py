"""ffkv_paged_decode_noalloc, the decode entry point that allocates no device memory (its split-K partials live in
the library's static per-GPU scratch), against ffkv_paged_decode with a caller workspace: same kernels and split,
so outputs are bit-identical, and both are within tolerance of the CPU checker.  Two calls in a row, the second on
smaller inputs and another cache type, so the second finds the first's partials in the shared scratch.  Sizes
whose partials exceed the scratch are rejected before anything runs."""

import ctypes

import numpy as np
import pytest

import cases
import gpu_util as gu
import oracle as O
from test_gpu_parity import half_ulp

FFKV_ERR_WORKSPACE = -3


def _call(ff, **kw):
    a = dict(q=16, out=16, qo_dtype=ff.DTYPE_BF16, k_cache=16, v_cache=16, cache_dtype=ff.DTYPE_BF16,
             k_scale=None, v_scale=None, block_table=16, context_lens=16, batch=1, num_heads=32, num_kv_heads=8,
             head_dim=128, block_size=16, max_blocks=4, num_blocks=4, max_context_len=0, scale=0.0, stream=None)
    a.update(kw)
    return ff.lib.ffkv_paged_decode_noalloc(*a.values())


def test_noalloc_rejects_sizes_beyond_scratch(ff):
    """8192 rows x 32 heads of partials do not fit 32 MiB: FFKV_ERR_WORKSPACE with a message, nothing launched
    (fake pointers are never dereferenced).  Argument checks come first, as in ffkv_paged_decode."""
    assert _call(ff, batch=8192) == FFKV_ERR_WORKSPACE
    assert "noalloc" in ff.lib.ffkv_last_error().decode()
    assert _call(ff, head_dim=84) == -2
    assert _call(ff, batch=0) == 0


def _run(ff, dev, c, noalloc: bool):
    import torch

    kp = gu.to_dev(c.k_pool, c.kv, dev)
    vp = gu.to_dev(c.v_pool, c.kv, dev)
    ks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(dev)
    vs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(dev)
    bt = torch.from_numpy(c.block_table).to(dev)
    ctx = torch.from_numpy(c.ctx).to(dev)
    ff.append_kv_cache(gu.to_dev(c.k_new, c.act, dev), gu.to_dev(c.v_new, c.act, dev), kp, vp, bt, ctx, ks, vs)
    q = gu.to_dev(c.q, c.act, dev)
    out = torch.full((c.B, 1, c.Hq * c.D), float("nan"), dtype=q.dtype, device=dev)
    if noalloc:
        ff.paged_attention_noalloc(q, kp, vp, bt, ctx, out, k_scale=ks, v_scale=vs)
    else:
        ws = ff.decode_workspace(c.B, c.Hq, c.D, c.max_blocks, device=dev)
        ff.paged_attention(q, kp, vp, bt, ctx, out=out, k_scale=ks, v_scale=vs, workspace=ws)
    torch.cuda.synchronize()
    return gu.to_host(out, np.uint16).reshape(c.B, -1)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(ff, gpu):
    rng = np.random.default_rng(77)
    big = cases.make_case(77, 64, 32, 8, 128, rng.integers(512, 4097, size=64), act="bf16")
    small = cases.make_case(78, 5, 28, 4, 128, rng.integers(1, 3000, size=5), act="bf16", kv="fp8")
    for c, tol in ((big, 2e-3), (small, 2e-2)):
        print(f"case noalloc B={c.B} Hq={c.Hq} Hkv={c.Hkv} kv={c.kv}", flush=True)
        ref = _run(ff, gpu, c, noalloc=False)
        got = _run(ff, gpu, c, noalloc=True)
        assert np.array_equal(got, ref), "noalloc output differs from ffkv_paged_decode's"
        _, _, _, _, _, out32 = cases.oracle_step(c)
        g = O.bf16_to_f32(got).reshape(out32.shape)
        diff = np.abs(g.astype(np.float64) - out32)
        assert float((diff - half_ulp(np.maximum(np.abs(g), np.abs(out32)), O.DTYPE_BF16)).max()) <= tol
