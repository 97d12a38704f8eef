"""Parity at the full BASELINE workloads the bench reports: config 3 (long-context split-K), config 4's 512-token
chunk append, and config 5 (quantized caches filled by quantize-on-append), against the CPU checker.

Bar (as tests/test_gpu_parity.py): pages, int8/fp8 codes and int8 scales bit-exact over the whole pool
(sentinel-filled, so stray writes show); outputs within max-abs 2e-3 (bf16 caches) or 2e-2 (quantized) of the
checker's fp32 value, plus half an output ulp for the rounding to bf16.

Config 5 fills its pools the way a serving engine does: every row's cached tokens go through ffkv_append in one
bulk call (int8: per-token absmax/127 scales written by the append; fp8: per-head scales from the data's absmax,
read by the append), then the decode step appends one token per row and runs the decode.  The K/V data, N(0,1)
with 1% of the elements x8, is drawn on the GPU (seeded torch generator) and copied to the host for the checker,
which applies the same appends to its own sentinel-filled pools.
"""

import math

import numpy as np
import pytest

import cases
import gpu_util as gu
import oracle as O
from test_gpu_parity import _check, half_ulp

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A


def test_config3_full(ff, gpu):
    """Qwen2.5-7B layer (Hq28/Hkv4/D128, G = 7), B = 8, 32768-token contexts, blocks scattered
    by a seeded permutation of the pool; split-K over many work items per row and the merge."""
    c = cases.make_case(3, 8, 28, 4, 128, [32768] * 8, act="bf16")
    _check(ff, gpu, c, 2e-3, workspace=True)


def test_config4_chunk_append(ff, gpu):
    """Config 4's chunked-prefill append: 8 rows of a 512-token chunk each, after a shared 2048-token prefix and a
    private suffix (the prefix's 128 blocks in every table); the pool is compared byte for byte, then each row
    decodes over its context."""
    rng = np.random.default_rng(4)
    ctx = 2048 + rng.integers(64, 1025, size=8)
    c = cases.make_case(4, 8, 32, 8, 128, ctx, act="bf16", S=512, shared_prefix_blocks=128)
    _check(ff, gpu, c, 2e-3, workspace=True)


def _c5_tables(rng, B, ctx):
    """Block tables for ctx + 1 tokens per row over a seeded permutation of a pool 10% larger than needed."""
    need = [(int(x) + 1 + 15) // 16 for x in ctx]
    N = math.ceil(sum(need) * 1.1)
    perm = rng.permutation(N).astype(np.int32)
    table = np.full((B, max(need)), -1, dtype=np.int32)
    pos = 0
    for b in range(B):
        table[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    return table, N


def _gauss_outliers(torch, gen, shape, dev):
    x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)
    x = torch.where(torch.rand(shape, generator=gen, device=dev) < 0.01, x * 8.0, x)
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("kv", ["i8", "fp8"])
def test_config5_full_quantize_on_append(ff, gpu, kv):
    """Qwen3-8B layer (Hq32/Hkv8/D128), B = 256, contexts U[1024, 8192], K/V N(0,1) with 1%
    outliers x8, int8 with per-token-per-head scales or fp8 e4m3 with per-head scales."""
    import torch

    B, Hq, Hkv, D = 256, 32, 8, 128
    kv_dt = cases.NAMES[kv]
    rng = np.random.default_rng(5)
    ctx = rng.integers(1024, 8193, size=B).astype(np.int32)
    table, N = _c5_tables(rng, B, ctx)
    S = int(ctx.max())
    print(f"case config5 kv={kv} B={B} S={S} N={N} tokens={int(ctx.sum()) + B}", flush=True)

    gen = torch.Generator(device=gpu).manual_seed(55)
    k_src = _gauss_outliers(torch, gen, (B, S, Hkv, D), gpu)   # every row's cached tokens (positions 0 .. S-1)
    v_src = _gauss_outliers(torch, gen, (B, S, Hkv, D), gpu)
    k_new = _gauss_outliers(torch, gen, (B, 1, Hkv, D), gpu)   # the decode step's token (position ctx[b])
    v_new = _gauss_outliers(torch, gen, (B, 1, Hkv, D), gpu)
    q = _gauss_outliers(torch, gen, (B, 1, Hq, D), gpu)

    store = torch.int8 if kv == "i8" else torch.uint8
    kp = torch.full((N, 16, Hkv, D), SENTINEL, dtype=torch.uint8, device=gpu).view(store)
    vp = torch.full((N, 16, Hkv, D), SENTINEL, dtype=torch.uint8, device=gpu).view(store)
    if kv == "i8":
        ks = torch.full((N, 16, Hkv), -3.0, dtype=torch.float32, device=gpu)
        vs = torch.full((N, 16, Hkv), -3.0, dtype=torch.float32, device=gpu)
    else:  # per-head scales from the absmax of everything the cache will hold
        ks = (torch.maximum(k_src.float().abs().amax(dim=(0, 1, 3)), k_new.float().abs().amax(dim=(0, 1, 3)))
              / 448.0).contiguous()
        vs = (torch.maximum(v_src.float().abs().amax(dim=(0, 1, 3)), v_new.float().abs().amax(dim=(0, 1, 3)))
              / 448.0).contiguous()
    bt = torch.from_numpy(table).to(gpu)
    ctx_d = torch.from_numpy(ctx).to(gpu)

    # GPU: bulk quantize-on-append of the cached tokens (positions from 0), then the decode step
    ff.append_kv_cache(k_src, v_src, kp, vp, bt, None, ks, vs)
    ff.append_kv_cache(k_new, v_new, kp, vp, bt, ctx_d, ks, vs)
    ws = ff.decode_workspace(B, Hq, D, table.shape[1], device=gpu)
    out = ff.paged_attention(q, kp, vp, bt, ctx_d, k_scale=ks, v_scale=vs, workspace=ws)
    torch.cuda.synchronize()

    # CPU checker: the same appends into its own sentinel-filled pools, then its decode
    host = lambda t: gu.to_host(t, np.uint16)  # noqa: E731
    np_store = np.int8 if kv == "i8" else np.uint8
    hk = np.full((N, 16, Hkv, D), SENTINEL, dtype=np.uint8).view(np_store)
    hv = np.full((N, 16, Hkv, D), SENTINEL, dtype=np.uint8).view(np_store)
    if kv == "i8":
        hks = np.full((N, 16, Hkv), -3.0, dtype=np.float32)
        hvs = np.full((N, 16, Hkv), -3.0, dtype=np.float32)
    else:
        hks, hvs = ks.cpu().numpy(), vs.cpu().numpy()
    O.append(host(k_src), host(v_src), O.DTYPE_BF16, hk, hv, kv_dt, table, None, hks, hvs)
    del k_src, v_src
    O.append(host(k_new), host(v_new), O.DTYPE_BF16, hk, hv, kv_dt, table, ctx, hks, hvs)
    assert np.array_equal(kp.cpu().numpy().view(np.uint8), hk.view(np.uint8)), "K pages differ"
    assert np.array_equal(vp.cpu().numpy().view(np.uint8), hv.view(np.uint8)), "V pages differ"
    if kv == "i8":
        assert np.array_equal(ks.cpu().numpy().view(np.uint32), hks.view(np.uint32)), "K scales differ"
        assert np.array_equal(vs.cpu().numpy().view(np.uint32), hvs.view(np.uint32)), "V scales differ"
    _, out32 = O.paged_decode(host(q), O.DTYPE_BF16, hk, hv, kv_dt, table, ctx, hks, hvs)
    got = O.bf16_to_f32(host(out)).reshape(out32.shape)
    diff = np.abs(got.astype(np.float64) - out32)
    excess = float((diff - half_ulp(np.maximum(np.abs(got), np.abs(out32)), O.DTYPE_BF16)).max())
    print(f"  max-abs err {float(diff.max()):.3e}, beyond output rounding {excess:.3e} (tol 2e-2)", flush=True)
    assert excess <= 2e-2
