"""Pins of the CPU closed form for chunked / paged prefill attention (oracle ffo_paged_prefill_f64).

Query t of row b sits at position ctx[b] + t and attends keys 0 .. ctx[b] + t over the paged cache (the cached
prefix and the chunk itself).  Checks: seq_len = 1 is exactly the pinned decode closed form; torch SDPA (float64)
with an explicit causal mask over the gathered keys; the contiguous mode is torch SDPA is_causal (the reference's
prefill branch); sharing prefix pages between rows changes nothing.
"""

import math

import numpy as np
import pytest
import torch

import cases
import oracle as O


def _case(seed, B, Hq, Hkv, D, ctx, S, kv="bf16", shared=0):
    c = cases.make_case(seed, B, Hq, Hkv, D, ctx, act="bf16", kv=kv, S=S, input_scale=1 / math.sqrt(D),
                        shared_prefix_blocks=shared)
    rng = np.random.default_rng(seed + 99)
    q = cases.encode(rng.standard_normal((B, S, Hq, D), dtype=np.float32) / np.float32(math.sqrt(D)), c.act)
    kp, vp = c.k_pool.copy(), c.v_pool.copy()
    ks = None if c.k_scale is None else c.k_scale.copy()
    vs = None if c.v_scale is None else c.v_scale.copy()
    O.append(c.k_new, c.v_new, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    return c, q, kp, vp, ks, vs


def _dequant(pool, kv, scale):
    """Dequantized cache as the closed form defines it: code * scale as one fp32 product."""
    if kv == O.DTYPE_I8:
        return (pool.astype(np.float32) * scale[..., None]).astype(np.float64)
    if kv == O.DTYPE_FP8:
        return (O.e4m3_to_f32(pool) * scale[None, None, :, None]).astype(np.float64)
    return cases.decode(pool, kv).astype(np.float64)


def test_single_token_equals_decode_closed_form():
    c, q, kp, vp, ks, vs = _case(1, 5, 8, 2, 128, [0, 15, 16, 100, 333], S=1)
    pre = O.paged_prefill_f64(q, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    dec = O.paged_decode_f64(q[:, 0], c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    np.testing.assert_array_equal(pre[:, 0], dec)


@pytest.mark.parametrize("kv", ["bf16", "i8", "fp8"])
def test_matches_torch_sdpa_with_causal_mask_over_prefix(kv):
    c, q, kp, vp, ks, vs = _case(2, 3, 8, 2, 64, [0, 21, 70], S=9, kv=kv)
    got = O.paged_prefill_f64(q, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    K = _dequant(kp, c.kv, ks)
    V = _dequant(vp, c.kv, vs)
    G = c.Hq // c.Hkv
    qf = cases.decode(q, c.act).astype(np.float64)
    for b in range(c.B):
        L = int(c.ctx[b]) + c.S
        phys = c.block_table[b, np.arange(L) // 16]
        kb = torch.from_numpy(K[phys, np.arange(L) % 16]).permute(1, 0, 2).repeat_interleave(G, 0)  # [Hq, L, D]
        vb = torch.from_numpy(V[phys, np.arange(L) % 16]).permute(1, 0, 2).repeat_interleave(G, 0)
        qb = torch.from_numpy(qf[b]).permute(1, 0, 2)                                               # [Hq, S, D]
        mask = torch.from_numpy(np.arange(L)[None, :] <= (int(c.ctx[b]) + np.arange(c.S))[:, None])
        want = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask)
        np.testing.assert_allclose(got[b], want.permute(1, 0, 2).numpy(), rtol=0, atol=1e-10)


def test_contiguous_mode_is_causal_attention():
    """block_table = None: K/V contiguous [B, S, Hkv, D] and positions 0..S-1 (the reference's prefill branch)."""
    rng = np.random.default_rng(3)
    B, S, Hq, Hkv, D = 2, 37, 4, 2, 64
    q = cases.encode(rng.standard_normal((B, S, Hq, D), dtype=np.float32) * 0.2, O.DTYPE_BF16)
    k = cases.encode(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), O.DTYPE_BF16)
    v = cases.encode(rng.standard_normal((B, S, Hkv, D), dtype=np.float32), O.DTYPE_BF16)
    got = O.paged_prefill_f64(q, O.DTYPE_BF16, k, v, O.DTYPE_BF16, None, None)
    f = lambda a: torch.from_numpy(cases.decode(a, O.DTYPE_BF16).astype(np.float64)).permute(0, 2, 1, 3)  # noqa
    kk, vv = f(k).repeat_interleave(2, 1), f(v).repeat_interleave(2, 1)
    want = torch.nn.functional.scaled_dot_product_attention(f(q), kk, vv, is_causal=True)
    np.testing.assert_allclose(got, want.permute(0, 2, 1, 3).numpy(), rtol=0, atol=1e-10)


def test_shared_prefix_equals_private_copy():
    c, q, kp, vp, ks, vs = _case(4, 4, 8, 2, 128, [40, 40, 55, 64], S=6, shared=2)
    got = O.paged_prefill_f64(q, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    # duplicate the shared physical blocks so every row owns private copies
    tbl = c.block_table.copy()
    extra_k, extra_v = [kp], [vp]
    n = kp.shape[0]
    for b in range(1, c.B):
        for j in range(2):
            extra_k.append(kp[tbl[b, j]][None])
            extra_v.append(vp[tbl[b, j]][None])
            tbl[b, j] = n
            n += 1
    kp2, vp2 = np.concatenate(extra_k), np.concatenate(extra_v)
    assert len(set(tbl[:, 0])) == c.B
    again = O.paged_prefill_f64(q, c.act, kp2, vp2, c.kv, tbl, c.ctx, ks, vs)
    np.testing.assert_array_equal(got, again)


def test_rows_without_keys_are_zero_and_invalid_pages_skipped():
    c, q, kp, vp, ks, vs = _case(5, 3, 4, 1, 64, [0, 30, 5], S=3)
    tbl = c.block_table.copy()
    tbl[1, 0] = -1                    # first page of row 1 missing: its first 16 keys are skipped
    ctx = c.ctx.copy()
    ctx[2] = -10                      # positions -10..-8: no key is visible
    got = O.paged_prefill_f64(q, c.act, kp, vp, c.kv, tbl, ctx, ks, vs)
    assert not got[2].any()
    full = O.paged_prefill_f64(q, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    assert np.abs(got[1] - full[1]).max() > 0  # the masked page mattered
