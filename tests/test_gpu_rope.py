"""Fused rotary embedding + KV append on the GPU against the CPU checker.

Bar: the rotated q and k are bit-identical to the checker's (ffo_rope: inv_freq, cos, sin in double rounded to
float, fp32 angle and rotation, no fused multiply-add), and the pages (int8 scales included) are bit-identical
to the checker's append of that rotated k and the untouched v.
"""

import numpy as np
import pytest

import cases
import gpu_util as gu
import oracle as O

pytestmark = pytest.mark.gpu

THETA = 1e6


def _setup(ff, dev, seed, B, Hq, Hkv, D, ctx, act, kv, S):
    c = cases.make_case(seed, B, Hq, Hkv, D, ctx, act=act, kv=kv, S=S, input_scale=1.0)
    rng = np.random.default_rng(seed + 1)
    qn = cases.encode(rng.standard_normal((B, S, Hq, D), dtype=np.float32), c.act)
    return c, qn


def _pools(c, dev):
    import torch

    kp = gu.to_dev(c.k_pool, c.kv, dev)
    vp = gu.to_dev(c.v_pool, c.kv, dev)
    ks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(dev)
    vs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(dev)
    return kp, vp, ks, vs


def _host(t, c_dt):
    import torch

    if t.dtype in (torch.float16, torch.bfloat16):
        return gu.to_host(t, np.uint16)
    return t.cpu().numpy()


def _check_pages(c, k_rot, kp, vp, ks, vs):
    rk, rv = c.k_pool.copy(), c.v_pool.copy()
    rks = None if c.k_scale is None else c.k_scale.copy()
    rvs = None if c.v_scale is None else c.v_scale.copy()
    O.append(k_rot, c.v_new, c.act, rk, rv, c.kv, c.block_table, c.ctx, rks, rvs)
    assert np.array_equal(_host(kp, c.kv).view(np.uint8), rk.view(np.uint8)), "K pages differ"
    assert np.array_equal(_host(vp, c.kv).view(np.uint8), rv.view(np.uint8)), "V pages differ"
    if c.kv == O.DTYPE_I8:
        assert np.array_equal(ks.cpu().numpy().view(np.uint32), rks.view(np.uint32)), "K scales differ"
        assert np.array_equal(vs.cpu().numpy().view(np.uint32), rvs.view(np.uint32)), "V scales differ"


@pytest.mark.parametrize("act,kv", [("bf16", "bf16"), ("f16", "f16"), ("f32", "f32"), ("bf16", "i8"),
                                    ("bf16", "fp8"), ("f16", "i8"), ("f32", "bf16"), ("f32", "fp8")])
@pytest.mark.parametrize("S", [1, 7])
def test_rope_append_bit_exact(ff, gpu, act, kv, S):
    c, qn = _setup(ff, gpu, 40 + S, 4, 16, 4, 128, [0, 17, 300, 4000], act, kv, S)
    print(f"case rope_append act={act} kv={kv} S={S}", flush=True)
    q = gu.to_dev(qn, c.act, gpu)
    k = gu.to_dev(c.k_new, c.act, gpu)
    v = gu.to_dev(c.v_new, c.act, gpu)
    kp, vp, ks, vs = _pools(c, gpu)
    import torch

    bt = torch.from_numpy(c.block_table).to(gpu)
    ctx = torch.from_numpy(c.ctx).to(gpu)
    ff.rope_append_kv_cache(q, k, v, kp, vp, bt, ctx, THETA, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    q_ref = O.rope(qn, c.act, c.ctx, THETA)
    k_ref = O.rope(c.k_new, c.act, c.ctx, THETA)
    assert np.array_equal(_host(q, c.act), q_ref), "rotated q differs"
    assert np.array_equal(_host(k, c.act), k_ref), "rotated k differs"
    assert np.array_equal(_host(v, c.act), c.v_new), "v was modified"
    _check_pages(c, k_ref, kp, vp, ks, vs)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("kv", ["bf16", "i8", "fp8"])
def test_rope_append_head_dims(ff, gpu, D, kv):
    """Other head dims (4 and 16 lanes per head row: the int8 row maximum over one quad, and over a full 16-lane
    row with its mirrors)."""
    c, qn = _setup(ff, gpu, 50 + D + len(kv), 3, 8, 2, D, [5, 31, 1000], "bf16", kv, 3)
    print(f"case rope_append D={D} kv={kv}", flush=True)
    import torch

    q, k, v = gu.to_dev(qn, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
    kp, vp, ks, vs = _pools(c, gpu)
    ff.rope_append_kv_cache(q, k, v, kp, vp, torch.from_numpy(c.block_table).to(gpu),
                            torch.from_numpy(c.ctx).to(gpu), THETA, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    k_ref = O.rope(c.k_new, c.act, c.ctx, THETA)
    assert np.array_equal(_host(q, c.act), O.rope(qn, c.act, c.ctx, THETA))
    assert np.array_equal(_host(k, c.act), k_ref)
    _check_pages(c, k_ref, kp, vp, ks, vs)


def test_rope_alone_long_positions_and_null_ctx(ff, gpu):
    """ffkv_rope without the append: positions up to ~1M, q absent, context_lens NULL (positions = t)."""
    import torch

    rng = np.random.default_rng(60)
    for act in ("bf16", "f32"):
        dt = cases.NAMES[act]
        qn = cases.encode(rng.standard_normal((3, 5, 8, 128), dtype=np.float32), dt)
        kn = cases.encode(rng.standard_normal((3, 5, 2, 128), dtype=np.float32), dt)
        ctx = np.array([0, 32763, 1_000_000], np.int32)
        print(f"case rope act={act}", flush=True)
        q, k = gu.to_dev(qn, dt, gpu), gu.to_dev(kn, dt, gpu)
        ff.apply_rope(q, k, torch.from_numpy(ctx).to(gpu), THETA)
        k2 = gu.to_dev(kn, dt, gpu)
        ff.apply_rope(None, k2, None, 10000.0)
        torch.cuda.synchronize()
        assert np.array_equal(_host(q, dt), O.rope(qn, dt, ctx, THETA))
        assert np.array_equal(_host(k, dt), O.rope(kn, dt, ctx, THETA))
        assert np.array_equal(_host(k2, dt), O.rope(kn, dt, None, 10000.0))


def test_fused_equals_rope_then_append(ff, gpu):
    """ffkv_rope_append leaves exactly what ffkv_rope followed by ffkv_append leaves (int8 cache, S = 16)."""
    import torch

    c, qn = _setup(ff, gpu, 70, 5, 16, 4, 128, [3, 16, 64, 250, 1023], "bf16", "i8", 16)
    print("case fused vs separate", flush=True)
    bt = torch.from_numpy(c.block_table).to(gpu)
    ctx = torch.from_numpy(c.ctx).to(gpu)
    q1, k1, v1 = gu.to_dev(qn, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
    kp1, vp1, ks1, vs1 = _pools(c, gpu)
    ff.rope_append_kv_cache(q1, k1, v1, kp1, vp1, bt, ctx, THETA, k_scale=ks1, v_scale=vs1)
    q2, k2, v2 = gu.to_dev(qn, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
    kp2, vp2, ks2, vs2 = _pools(c, gpu)
    ff.apply_rope(q2, k2, ctx, THETA)
    ff.append_kv_cache(k2, v2, kp2, vp2, bt, ctx, ks2, vs2)
    torch.cuda.synchronize()
    for a, b in [(q1, q2), (k1, k2), (kp1, kp2), (vp1, vp2), (ks1, ks2), (vs1, vs2)]:
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.int8 else a, b.view(torch.uint8)
                           if b.dtype == torch.int8 else b)
