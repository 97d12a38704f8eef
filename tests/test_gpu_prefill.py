"""Chunked / paged prefill attention on the GPU against the CPU closed form (oracle ffo_paged_prefill_f64).

Bar (as for decode): outputs within max-abs 2e-3 for 16-bit caches and 2e-2 for int8/fp8 caches of the float64
closed form, beyond the output format's own rounding (half an ulp at the value).  Cases: chunks with and without
a cached prefix (context_lens > 0 is the prefix-reuse step the reference's model skips), GQA groups 1..16, head
dims 64/128/256, quantized caches, invalid pages and rows without keys, shared prefix pages, the contiguous
(block-table-free) mode of the reference's prefill branch, and seq_len = 1 against the decode kernel.
"""

import math

import numpy as np
import pytest

import cases
import gpu_util as gu
import oracle as O

pytestmark = pytest.mark.gpu


def half_ulp(x, act):
    if act == O.DTYPE_F32:
        return np.zeros_like(x)
    mant, emin = (7, -126) if act == O.DTYPE_BF16 else (10, -14)
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** emin)))
    return 2.0 ** (e - mant - 1)


def _run(ff, dev, c, qn, tbl=None, ctx=None, contiguous=False, scale=0.0):
    """Append the case's chunk (k_new/v_new) to its pools, then prefill; returns (out f32 [B,S,Hq,D], ref f64)."""
    import torch

    tbl = c.block_table if tbl is None else tbl
    ctx = c.ctx if ctx is None else ctx
    if contiguous:
        k = gu.to_dev(c.k_new, c.act, dev)
        v = gu.to_dev(c.v_new, c.act, dev)
        q = gu.to_dev(qn, c.act, dev)
        out = ff.paged_prefill(q, k, v, None, None)
        torch.cuda.synchronize()
        ref = O.paged_prefill_f64(qn, c.act, c.k_new, c.v_new, c.act, None, None)
    else:
        kp = gu.to_dev(c.k_pool, c.kv, dev)
        vp = gu.to_dev(c.v_pool, c.kv, dev)
        ks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(dev)
        vs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(dev)
        bt = torch.from_numpy(np.ascontiguousarray(tbl)).to(dev)
        cx = torch.from_numpy(np.ascontiguousarray(ctx)).to(dev)
        ff.append_kv_cache(gu.to_dev(c.k_new, c.act, dev), gu.to_dev(c.v_new, c.act, dev), kp, vp, bt, cx, ks, vs)
        q = gu.to_dev(qn, c.act, dev)
        out = ff.paged_prefill(q, kp, vp, bt, cx, k_scale=ks, v_scale=vs, scale=scale)
        torch.cuda.synchronize()
        rk, rv = c.k_pool.copy(), c.v_pool.copy()
        rks = None if c.k_scale is None else c.k_scale.copy()
        rvs = None if c.v_scale is None else c.v_scale.copy()
        O.append(c.k_new, c.v_new, c.act, rk, rv, c.kv, tbl, ctx, rks, rvs)
        ref = O.paged_prefill_f64(qn, c.act, rk, rv, c.kv, tbl, ctx, rks, rvs, scale=scale)
    got = out.float().cpu().numpy().reshape(ref.shape)
    return got, ref


def _check(got, ref, act, tol):
    diff = np.abs(got.astype(np.float64) - ref)
    excess = float((diff - half_ulp(np.maximum(np.abs(got), np.abs(ref)), act)).max())
    print(f"  max-abs err {diff.max():.3e}, beyond output rounding {excess:.3e} (tol {tol})", flush=True)
    assert excess <= tol


def _case(seed, B, Hq, Hkv, D, ctx, S, act="bf16", kv=None, shared=0):
    c = cases.make_case(seed, B, Hq, Hkv, D, ctx, act=act, kv=kv, S=S, input_scale=1.0,
                        shared_prefix_blocks=shared)
    rng = np.random.default_rng(seed + 1000)
    qn = cases.encode(rng.standard_normal((B, S, Hq, D), dtype=np.float32), c.act)
    print(f"case prefill seed={seed} B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} act={act} kv={kv or act} "
          f"ctx={list(np.asarray(ctx))}", flush=True)
    return c, qn


@pytest.mark.parametrize("S", [1, 16, 37, 130])
@pytest.mark.parametrize("ctx", [[0, 0, 0], [17, 300, 5]])
def test_prefill_bf16(ff, gpu, S, ctx):
    c, qn = _case(100 + S, 3, 32, 8, 128, ctx, S)
    _check(*_run(ff, gpu, c, qn), c.act, 2e-3)


@pytest.mark.parametrize("act,kv,tol", [("f16", "f16", 2e-3), ("bf16", "i8", 2e-2), ("bf16", "fp8", 2e-2),
                                        ("f16", "i8", 2e-2), ("f32", "bf16", 2e-3), ("f32", "fp8", 2e-2)])
def test_prefill_dtypes(ff, gpu, act, kv, tol):
    c, qn = _case(200, 3, 16, 4, 128, [0, 33, 250], 24, act=act, kv=kv)
    _check(*_run(ff, gpu, c, qn), c.act, tol)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("G", [1, 7, 16])
def test_prefill_head_shapes(ff, gpu, D, G):
    c, qn = _case(300 + D + G, 2, 2 * G, 2, D, [9, 70], 19)
    _check(*_run(ff, gpu, c, qn), c.act, 2e-3)


@pytest.mark.parametrize("kv", ["i8", "fp8"])
@pytest.mark.parametrize("D,G", [(64, 4), (128, 7), (256, 2)])
def test_prefill_quantized_head_shapes(ff, gpu, kv, D, G):
    c, qn = _case(320 + D + G, 3, 2 * G, 2, D, [5, 90, 200], 40, kv=kv)
    _check(*_run(ff, gpu, c, qn), c.act, 2e-2)


@pytest.mark.parametrize("kv", ["i8", "fp8"])
def test_prefill_quantized_long_chunk(ff, gpu, kv):
    """A 512-token chunk over a 1500-token prefix on an 8-bit cache (many steps, partial last pages)."""
    c, qn = _case(410, 2, 32, 8, 128, [1500, 64], 512, kv=kv)
    _check(*_run(ff, gpu, c, qn), c.act, 2e-2)


def test_prefill_long_chunk_over_long_prefix(ff, gpu):
    """A 512-token chunk after a 1500-token prefix (many workgroups per row, the causal limit varying)."""
    c, qn = _case(400, 2, 32, 8, 128, [1500, 64], 512)
    _check(*_run(ff, gpu, c, qn), c.act, 2e-3)


# both load-issue forms of the kernel: per run (bf16 q over a bf16 cache, head_dim 128) and per page (the others)
@pytest.mark.parametrize("act,kv,D,tol", [("bf16", "bf16", 128, 2e-3), ("f16", "f16", 128, 2e-3),
                                          ("bf16", "bf16", 64, 2e-3), ("bf16", "bf16", 256, 2e-3),
                                          ("bf16", "i8", 128, 2e-2), ("f32", "bf16", 128, 2e-3),
                                          ("bf16", "i8", 64, 2e-2), ("f16", "i8", 128, 2e-2),
                                          ("bf16", "i8", 256, 2e-2), ("bf16", "fp8", 64, 2e-2)])
def test_prefill_invalid_pages_and_rows_without_keys(ff, gpu, act, kv, D, tol):
    c, qn = _case(500, 4, 8, 2, D, [40, 0, 64, 20], 9, act=act, kv=kv)
    tbl = c.block_table.copy()
    tbl[0, 1] = -1                    # a hole in row 0's prefix
    tbl[2, 0] = c.num_blocks + 5      # out of the pool
    ctx = c.ctx.copy()
    ctx[3] = -30                      # positions -30..-22: no key; the append skips them too
    _check(*_run(ff, gpu, c, qn, tbl=tbl, ctx=ctx), c.act, tol)


@pytest.mark.parametrize("B,Hkv", [(40, 2), (130, 4)])
def test_prefill_many_rows_ordered_by_length(ff, gpu, B, Hkv):
    """Many (row, kv head) groups with repeated and negative cached lengths: each XCD takes its groups longest
    first (ties by index), or in index order past 64 groups per XCD (B = 130, Hkv = 4)."""
    rng = np.random.default_rng(950 + B)
    ctx = rng.choice([0, 17, 17, 64, 90, 90, 150], size=B).astype(np.int32)
    c, qn = _case(950 + B, B, 2 * Hkv, Hkv, 128, ctx, 5)
    ctx2 = c.ctx.copy()
    ctx2[1] = -7  # no key for the first positions of row 1
    _check(*_run(ff, gpu, c, qn, ctx=ctx2), c.act, 2e-3)


def test_prefill_shared_prefix_pages(ff, gpu):
    c, qn = _case(600, 4, 32, 8, 128, [64, 64, 80, 100], 12, shared=4)
    _check(*_run(ff, gpu, c, qn), c.act, 2e-3)


@pytest.mark.parametrize("S", [5, 64, 200])
def test_prefill_contiguous_mode_is_reference_causal_prefill(ff, gpu, S):
    c, qn = _case(700 + S, 2, 28, 4, 128, [0, 0], S)
    _check(*_run(ff, gpu, c, qn, contiguous=True), c.act, 2e-3)


@pytest.mark.parametrize("act,D", [("f16", 128), ("bf16", 64), ("bf16", 256), ("f16", 64)])
def test_prefill_contiguous_mode_head_dims(ff, gpu, act, D):
    """The contiguous mode (row offsets instead of a block table) through the per-page load issue."""
    c, qn = _case(760 + D, 3, 8, 2, D, [0, 0, 0], 83, act=act)
    _check(*_run(ff, gpu, c, qn, contiguous=True), c.act, 2e-3)


def test_prefill_single_token_agrees_with_decode(ff, gpu):
    import torch

    c, qn = _case(800, 6, 32, 8, 128, [0, 15, 16, 200, 1023, 4000], 1)
    got, ref = _run(ff, gpu, c, qn)
    # decode kernel on the same appended cache
    kp = gu.to_dev(c.k_pool, c.kv, gpu)
    vp = gu.to_dev(c.v_pool, c.kv, gpu)
    bt = torch.from_numpy(c.block_table).to(gpu)
    cx = torch.from_numpy(c.ctx).to(gpu)
    ff.append_kv_cache(gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu), kp, vp, bt, cx)
    dec = ff.paged_attention(gu.to_dev(qn, c.act, gpu), kp, vp, bt, cx)
    torch.cuda.synchronize()
    d = dec.float().cpu().numpy().reshape(got.shape)
    _check(got, ref, c.act, 2e-3)
    assert np.abs(d - got).max() <= 2 * 2e-3


@pytest.mark.parametrize("k_scale_kind", ["zero", "negative"])
def test_fp8_degenerate_k_scales(ff, gpu, k_scale_kind):
    """fp8 per-head K scales of 0 (every score 0: uniform weights) and below 0 (the softmax of the negated scores)
    give the checker's result in the prefill, the shared-prefix decode (whose prefix partials run the prefill
    kernel) and the plain decode alike, instead of NaN."""
    import torch

    c, qn = _case(61, 3, 8, 2, 128, [40, 300, 17], 37, kv="fp8")
    c.k_scale = c.k_scale.copy()
    if k_scale_kind == "zero":
        c.k_scale[:] = 0.0
    else:
        c.k_scale[0] = -c.k_scale[0]
    # a scale of 0 stores zero codes on append; keep the pool's codes for the negative-scale case only
    got, ref = _run(ff, gpu, c, qn)
    assert np.isfinite(got).all()
    _check(got, ref, c.act, 2e-2)

    # decode over a 1-page shared prefix and the plain decode on the same pools
    d = cases.make_case(62, 4, 8, 2, 128, [40, 90, 33, 70], act="bf16", kv="fp8", shared_prefix_blocks=1)
    d.k_scale = d.k_scale.copy()
    if k_scale_kind == "zero":
        d.k_scale[:] = 0.0
    else:
        d.k_scale[1] = -d.k_scale[1]
    kp, vp, ks, vs, _, out32 = cases.oracle_step(d)
    dev = gpu
    args = (gu.to_dev(d.q, d.act, dev), gu.to_dev(kp, d.kv, dev), gu.to_dev(vp, d.kv, dev),
            torch.from_numpy(d.block_table).to(dev), torch.from_numpy(d.ctx).to(dev))
    for shared in (0, 1):
        out = (ff.paged_attention_shared_prefix(*args, shared, k_scale=torch.from_numpy(ks).to(dev),
                                                v_scale=torch.from_numpy(vs).to(dev)) if shared else
               ff.paged_attention(*args, k_scale=torch.from_numpy(ks).to(dev), v_scale=torch.from_numpy(vs).to(dev)))
        torch.cuda.synchronize()
        g = out.float().cpu().numpy().reshape(out32.shape)
        assert np.isfinite(g).all(), f"shared={shared}"
        _check(g, out32.astype(np.float64), d.act, 2e-2)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_prefill_int8_large_q(ff, gpu, D):
    """bf16 queries beyond f16's range over an int8 cache: the f16 score products take q scaled into range by a
    power of two (exact) and the softmax scale compensates.  q is N(0,1) * 2^17 and the score scale 2^-17 /
    sqrt(D), so the softmax is the ordinary one; outputs within the quantized bar of the float64 closed form."""
    c, qn = _case(170 + D, 3, 16, 4, D, [17, 300, 5], 37, kv="i8")
    qf = cases.decode(qn, c.act) * np.float32(2.0 ** 17)
    qn = cases.encode(qf, c.act)
    _check(*_run(ff, gpu, c, qn, scale=2.0 ** -17 / math.sqrt(D)), c.act, 2e-2)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_prefill_bf16_small_v(ff, gpu, D):
    """V values of order 2^-16, below f16's normal range: where the PV products take V in f16, each value rounds
    to an f16 subnormal (an absolute error of at most 2^-25), so the outputs stay within 2^-23 of the float64
    closed form beyond their own rounding (values flushed to zero would miss by about 2^-18)."""
    c, qn = _case(160 + D, 3, 16, 4, D, [17, 300, 5], 37)
    s = np.float32(2.0 ** -16)
    c.v_pool = cases.encode(cases.decode(c.v_pool, c.kv) * s, c.kv)
    c.v_new = cases.encode(cases.decode(c.v_new, c.act) * s, c.act)
    got, ref = _run(ff, gpu, c, qn)
    assert float(np.abs(ref).max()) > 2.0 ** -19
    _check(got, ref, c.act, 2.0 ** -23)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_prefill_int8_large_v(ff, gpu, D):
    """int8 pages whose dequantized V reaches 3e4 (per-token scales of 3e4 / 127): P carries the keys' V scales
    into the f16 PV products, p < 2^8, so p times a scale stays within f16's range up to |V| of about 32,500, the
    documented limit.  Row 1, kv head 3 gets such tokens in its cached pages and in its chunk; its outputs match
    the float64 closed form relative to the largest |v|, and rows 0 and 2 keep the quantized bar."""
    big = 3.0e4
    c, qn = _case(190 + D, 3, 16, 4, D, [17, 300, 5], 37, kv="i8")
    rng = np.random.default_rng(191)
    for t in rng.choice(300, size=6, replace=False):
        page, slot = c.block_table[1, t // 16], t % 16
        c.v_scale[page, slot, 3] = np.float32(big / 127.0)
    c.v_new[1, 5, 3, 7] = cases.encode(np.array([big], np.float32), c.act)[0]
    got, ref = _run(ff, gpu, c, qn)
    for b in (0, 2):
        _check(got[b:b + 1], ref[b:b + 1], c.act, 2e-2)
    err = float(np.abs(got[1].astype(np.float64) - ref[1]).max())
    print(f"  row 1 max-abs err {err:.3e} against |v| up to {big:.1e}", flush=True)
    assert np.isfinite(got[1]).all() and err <= 2e-2 * big


@pytest.mark.parametrize("D,big", [(128, 6.0e4), (128, 7.0e4), (128, 3.0e5), (128, float("inf")), (64, 7.0e4),
                                   (256, 7.0e4), (256, float("inf"))])
def test_prefill_bf16_large_v(ff, gpu, D, big):
    """V values far beyond the N(0,1) data: row 1, kv head 3 gets them in its cached pages and in its chunk.
    6e4 still fits f16 (the PV products may take V in f16); the others do not, and the workgroups that meet them
    must fall back to products that keep V in bf16 (every head_dim: its own load layout and stage count).  Row
    1's outputs must match the float64 closed form relative to its largest |v|, and rows 0 and 2 keep the
    ordinary bar.  Infinite V: non-finite wherever the closed form is; a query for which the infinite value's key
    is masked (causal limit) may get NaN in that dim too, as the masked key still meets it in the step's products
    with p = 0 (0 * inf), but only in kv head 3's heads; the other heads keep the ordinary bar.  The reference's
    prefill does the same: its P.V tile product (src/kernels/attention.cu:232-243) takes every key of the 16-key
    tile, the causally masked ones with p = 0 (:173-174)."""
    Hq, Hkv = (16, 4) if D == 256 else (32, 8)
    c, qn = _case(150 + D, 3, Hq, Hkv, D, [17, 300, 5], 37)
    rng = np.random.default_rng(151)
    vals = np.array([big, -big, big / 3], np.float32)
    enc = cases.encode(vals, O.DTYPE_BF16)
    # cached tokens of row 1 (pages of its block table), kv head 3
    for t in rng.choice(300, size=6, replace=False):
        page, slot = c.block_table[1, t // 16], t % 16
        c.v_pool[page, slot, 3, rng.integers(0, D)] = enc[rng.integers(0, 3)]
    c.v_new[1, 5, 3, 7] = enc[0]
    got, ref = _run(ff, gpu, c, qn)
    for b in (0, 2):
        _check(got[b:b + 1], ref[b:b + 1], c.act, 2e-3)
    g1, r1 = got[1].astype(np.float64), ref[1]
    gf, rf = np.isfinite(g1), np.isfinite(r1)
    bad = np.argwhere(gf != rf)
    if len(bad):
        print(f"  {len(bad)} positions (token, head, dim) differ in finiteness, e.g. "
              + ", ".join(f"{tuple(int(x) for x in i)}: got {g1[tuple(i)]} ref {r1[tuple(i)]}" for i in bad[:6]),
              flush=True)
    assert not (gf & ~rf).any(), "an output the closed form makes non-finite came out finite"
    if np.isfinite(big):
        assert not len(bad), "non-finite outputs where the closed form has none"
        scale = max(1.0, big)
        err = float(np.abs(g1 - r1).max())
        print(f"  row 1 max-abs err {err:.3e} against |v| up to {scale:.1e}", flush=True)
        assert err <= 2e-3 * scale
    else:
        # kv head 3's heads (12..15) hold the infinities; the other heads keep the ordinary bar
        assert gf[:, :12].all() and rf[:, :12].all()
        _check(got[1][:, :12], ref[1][:, :12], c.act, 2e-3)


def _jump_scores(c, qn, D, b, kvh, positions, v_big, cached_len):
    """Arrange int8 pools so that the keys at `positions` of row b, kv head kvh score far above the keys before
    them, and carry V scales of v_big / 127: every K code is 1, q is 1, K scales are 0 except at those keys, whose
    scale puts the score at 7.9 / (scale * log2 e) above the others.  The online softmax's reference maximum is set
    by the first step's keys (score 0) and only moves when a score passes it by 8 in log2 units, so those keys
    enter the PV products with p = 2^7.9 and p times the V scale exceeds f16's range once v_big / 127 > 65504 /
    2^7.9 (v_big above about 3.1e4).  The chunk's own keys score 0 (zero K)."""
    c.k_pool[...] = 1
    c.k_scale[...] = 0.0
    kscale = np.float32(7.9 * math.log(2.0) / math.sqrt(D))  # s * scale = 7.9 ln 2 with s = D * kscale
    for t in positions:
        assert t >= 64 and t < cached_len  # after the first step of 64 keys, inside the cached part
        page, slot = c.block_table[b, t // 16], t % 16
        c.k_scale[page, slot, kvh] = kscale
        c.v_scale[page, slot, kvh] = np.float32(v_big / 127.0)
    c.k_new[...] = cases.encode(np.zeros(c.k_new.shape, np.float32), c.act)
    return cases.encode(np.ones(qn.shape, np.float32), c.act)


@pytest.mark.parametrize("big", [4.0e4, 1.0e6])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_prefill_int8_v_scale_overflow(ff, gpu, D, big):
    """int8 pages whose P times V scale overflows f16 in the PV products (keys that enter with p = 2^7.9 and V
    scales of big / 127): the workgroup must run again with p scaled down.  Row 0, kv head 1 holds the keys; its
    heads match the float64 closed form relative to the largest |v|, and every other (row, head) keeps the
    quantized bar."""
    c, qn = _case(180 + D, 2, 8, 2, D, [300, 300], 37, kv="i8")
    qn = _jump_scores(c, qn, D, 0, 1, [100, 130, 131, 200, 250], big, 300)
    got, ref = _run(ff, gpu, c, qn)
    _check(got[1:], ref[1:], c.act, 2e-2)
    _check(got[0][:, :4], ref[0][:, :4], c.act, 2e-2)
    g, r = got[0][:, 4:].astype(np.float64), ref[0][:, 4:]
    err = float(np.abs(g - r).max())
    print(f"  row 0 kv head 1: max |out| {float(np.abs(r).max()):.3e}, max-abs err {err:.3e}", flush=True)
    assert float(np.abs(r).max()) > 0.1 * big  # the jump keys dominate these outputs
    assert np.isfinite(g).all() and err <= 2e-2 * big
