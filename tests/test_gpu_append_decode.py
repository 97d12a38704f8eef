"""The decode step as one call (ffkv_append_paged_decode): one token appended per row, then decode attention.
Same bar as the separate calls (tests/test_gpu_parity.py): every page byte and int8 scale bit-exact against the
CPU checker's append, outputs within max-abs 2e-3 (16-bit KV) / 2e-2 (quantized KV) of its decode.  The single-
launch form (16-bit cache fed in its own dtype, no truncation) is exercised over the cases that move the new
token around: first slot of a fresh page, last slot of a page, one-token rows, rows on several windows of 64,
invalid pages under the new token, head shapes, rows cut short by max_context_len; the two-launch fallback over
mixed dtypes and quantized caches."""

import numpy as np
import pytest

import cases
import oracle as O
from test_gpu_parity import TOL, half_ulp

pytestmark = pytest.mark.gpu

NAME = {O.DTYPE_F32: "f32", O.DTYPE_F16: "f16", O.DTYPE_BF16: "bf16", O.DTYPE_I8: "i8", O.DTYPE_FP8: "fp8"}


def _run(ff, dev, c, max_context_len=0, table=None, workspace=False):
    import torch

    import gpu_util as gu

    tbl = c.block_table if table is None else table
    print(f"case append+decode seed={c.seed} B={c.B} Hq={c.Hq} Hkv={c.Hkv} D={c.D} act={c.act} kv={c.kv} "
          f"ctx_max={int(c.ctx.max())} cap={max_context_len}", flush=True)
    kp, vp = c.k_pool.copy(), c.v_pool.copy()
    ks = None if c.k_scale is None else c.k_scale.copy()
    vs = None if c.v_scale is None else c.v_scale.copy()
    O.append(c.k_new, c.v_new, c.act, kp, vp, c.kv, tbl, c.ctx, ks, vs)
    _, ref = O.paged_decode(c.q, c.act, kp, vp, c.kv, tbl, c.ctx, ks, vs, max_context_len=max_context_len)
    dk, dv = gu.to_dev(c.k_pool, c.kv, dev), gu.to_dev(c.v_pool, c.kv, dev)
    dks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(dev)
    dvs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(dev)
    bt = torch.from_numpy(np.ascontiguousarray(tbl)).to(dev)
    cx = torch.from_numpy(c.ctx).to(dev)
    q, kn, vn = gu.to_dev(c.q, c.act, dev), gu.to_dev(c.k_new, c.act, dev), gu.to_dev(c.v_new, c.act, dev)
    ws = ff.decode_workspace(c.B, c.Hq, c.D, c.max_blocks, max_context_len, device=dev) if workspace else None
    out = ff.append_paged_attention(kn, vn, q, dk, dv, bt, cx, k_scale=dks, v_scale=dvs,
                                    max_context_len=max_context_len, workspace=ws, num_blocks=c.num_blocks)
    torch.cuda.synchronize()
    conv = (lambda t: gu.to_host(t, np.uint16)) if dk.dtype in (torch.float16, torch.bfloat16) else \
        (lambda t: t.cpu().numpy())
    assert np.array_equal(conv(dk).view(np.uint8), kp.view(np.uint8)), "K pages differ"
    assert np.array_equal(conv(dv).view(np.uint8), vp.view(np.uint8)), "V pages differ"
    if c.kv == O.DTYPE_I8:
        assert np.array_equal(dks.cpu().numpy().view(np.uint32), ks.view(np.uint32)), "K scales differ"
        assert np.array_equal(dvs.cpu().numpy().view(np.uint32), vs.view(np.uint32)), "V scales differ"
    got = (gu.out_to_f32(gu.to_host(out, np.uint16), c.act) if c.act != O.DTYPE_F32 else
           out.cpu().numpy()).reshape(ref.shape)
    tol = TOL[(NAME[c.act], NAME[c.kv])]
    diff = np.abs(got.astype(np.float64) - ref)
    excess = float((diff - half_ulp(np.maximum(np.abs(got), np.abs(ref)), c.act)).max())
    print(f"  max-abs err {diff.max():.3e}, beyond output rounding {excess:.3e} (tol {tol})", flush=True)
    assert excess <= tol


def test_config1_bf16(ff, gpu):
    _run(ff, gpu, cases.config1(act="bf16"))


def test_config2_shape(ff, gpu):
    rng = np.random.default_rng(70)
    c = cases.make_case(70, 64, 32, 8, 128, rng.integers(512, 4097, size=64), act="bf16")
    _run(ff, gpu, c, workspace=True)


def test_new_token_positions(ff, gpu):
    """The new token at slot 0 of a fresh page (ctx % 16 == 0), at slot 15, one-token rows (ctx 0) and a
    row of exactly one full page."""
    ctx = [0, 15, 16, 31, 32, 47, 1, 255, 256, 1000, 1023, 1024]
    c = cases.make_case(71, len(ctx), 32, 8, 128, ctx, act="bf16")
    _run(ff, gpu, c)


def test_many_windows_of_rows(ff, gpu):
    rng = np.random.default_rng(72)
    c = cases.make_case(72, 150, 16, 8, 128, rng.integers(0, 300, size=150), act="f16")
    _run(ff, gpu, c)


def test_invalid_page_under_new_token(ff, gpu):
    """Rows whose new token's page is -1 or out of the pool: the token is neither written nor attended."""
    ctx = [40, 95, 200, 16]
    c = cases.make_case(73, 4, 16, 4, 128, ctx, act="bf16")
    tbl = c.block_table.copy()
    tbl[0, 40 // 16] = -1
    tbl[2, 200 // 16] = c.num_blocks + 2
    _run(ff, gpu, c, table=tbl)


@pytest.mark.parametrize("D,G", [(64, 1), (64, 8), (256, 4), (128, 16), (128, 7), (128, 32), (64, 20), (96, 4),
                                 (40, 8), (80, 4), (112, 7), (112, 20)])
def test_head_shapes(ff, gpu, D, G):
    rng = np.random.default_rng(74 + D + G)
    c = cases.make_case(74 + D + G, 9, 2 * G, 2, D, rng.integers(0, 700, size=9), act="bf16")
    _run(ff, gpu, c)


@pytest.mark.parametrize("act,kv", [("f32", "bf16"), ("bf16", "i8"), ("bf16", "fp8"), ("f32", "f32"),
                                    ("f16", "f16")])
def test_two_launch_forms(ff, gpu, act, kv):
    """Source dtype other than the cache's, quantized and fp32 caches: append kernel then decode."""
    rng = np.random.default_rng(75)
    c = cases.make_case(75, 7, 32, 8, 128, rng.integers(0, 900, size=7), act=act, kv=kv)
    _run(ff, gpu, c)


@pytest.mark.parametrize("cap", [500, 1000, 16])
def test_truncated_rows(ff, gpu, cap):
    """max_context_len cutting some rows (their new token is written but not attended), none, or all."""
    rng = np.random.default_rng(76)
    c = cases.make_case(76, 70, 32, 8, 128, rng.integers(200, 900, size=70), act="bf16")
    _run(ff, gpu, c, max_context_len=cap)
