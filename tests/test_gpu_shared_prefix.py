"""Decode over rows that share a prefix of pages (ffkv_paged_decode_shared_prefix) against the CPU checker's
decode on the same appended cache, to the same bar as the plain decode (tests/test_gpu_parity.py): outputs within
max-abs 2e-3 (16-bit KV) or 2e-2 (quantized KV) of the fp32 checker, beyond the output format's rounding.  The
shared pages are attended once for all rows by a separate matrix-product kernel and merged with each row's own
pages, so these cases cover the split itself: prefixes of 1 .. 128 pages, rows shorter than the prefix, rows
ending exactly at its end, truncation by max_context_len, holes in the prefix, every head_dim and group size, and
a workspace full of garbage reused across calls, and 8-bit caches (int8 per-token scales travel with the
prefix pages, fp8 per-head scales fold into the score scale and the output)."""

import numpy as np
import pytest

import cases
import oracle as O
from test_gpu_parity import half_ulp

pytestmark = pytest.mark.gpu


def _run(ff, dev, c, shared, max_context_len=0, workspace=None, table=None):
    import torch

    import gpu_util as gu

    tbl = c.block_table if table is None else table
    print(f"case shared-prefix seed={c.seed} B={c.B} Hq={c.Hq} Hkv={c.Hkv} D={c.D} act={c.act} kv={c.kv} "
          f"shared={shared} ctx_max={int(c.ctx.max())} cap={max_context_len}", flush=True)
    kp, vp = c.k_pool.copy(), c.v_pool.copy()
    ks = None if c.k_scale is None else c.k_scale.copy()
    vs = None if c.v_scale is None else c.v_scale.copy()
    O.append(c.k_new, c.v_new, c.act, kp, vp, c.kv, tbl, c.ctx, ks, vs)
    _, ref = O.paged_decode(c.q, c.act, kp, vp, c.kv, tbl, c.ctx, ks, vs, max_context_len=max_context_len)
    kd, vd = gu.to_dev(kp, c.kv, dev), gu.to_dev(vp, c.kv, dev)
    ksd = None if ks is None else torch.from_numpy(ks).to(dev)
    vsd = None if vs is None else torch.from_numpy(vs).to(dev)
    bt = torch.from_numpy(np.ascontiguousarray(tbl)).to(dev)
    cx = torch.from_numpy(c.ctx).to(dev)
    q = gu.to_dev(c.q, c.act, dev)
    out = ff.paged_attention_shared_prefix(q, kd, vd, bt, cx, shared, k_scale=ksd, v_scale=vsd,
                                           max_context_len=max_context_len, workspace=workspace,
                                           num_blocks=c.num_blocks)
    plain = ff.paged_attention(q, kd, vd, bt, cx, k_scale=ksd, v_scale=vsd, max_context_len=max_context_len,
                               num_blocks=c.num_blocks)
    torch.cuda.synchronize()
    conv = (lambda t: gu.out_to_f32(gu.to_host(t, np.uint16), c.act)) if c.act != O.DTYPE_F32 else \
        (lambda t: t.cpu().numpy())
    return conv(out).reshape(ref.shape), conv(plain).reshape(ref.shape), ref


def _check(got, ref, act, tol, what):
    diff = np.abs(got.astype(np.float64) - ref)
    excess = float((diff - half_ulp(np.maximum(np.abs(got), np.abs(ref)), act)).max())
    print(f"  {what}: max-abs err {diff.max():.3e}, beyond output rounding {excess:.3e} (tol {tol})", flush=True)
    assert excess <= tol


def _both(ff, dev, c, shared, tol=2e-3, **kw):
    got, plain, ref = _run(ff, dev, c, shared, **kw)
    _check(got, ref, c.act, tol, "shared-prefix decode")
    _check(plain, ref, c.act, tol, "plain decode")


@pytest.mark.parametrize("shared,suffix", [(1, (1, 40)), (8, (1, 200)), (32, (16, 600)), (128, (64, 1024))])
def test_shared_prefix_bf16(ff, gpu, shared, suffix):
    rng = np.random.default_rng(40 + shared)
    B = 24
    ctx = shared * 16 + rng.integers(suffix[0], suffix[1] + 1, size=B) - 1  # ctx + 1 tokens after the append
    c = cases.make_case(40 + shared, B, 32, 8, 128, ctx, act="bf16", shared_prefix_blocks=shared)
    _both(ff, gpu, c, shared)


@pytest.mark.parametrize("big", [4.0e4, 1.0e6])
def test_shared_prefix_int8_v_scale_overflow(ff, gpu, big):
    """int8 prefix pages whose keys enter the prefix kernel's f16 PV products with p = 2^7.9 and V scales of
    big / 127 (p times the scale beyond f16's range): its workgroups run again with p scaled down, and the
    partials they leave carry that scale in their maxima, so the merge with the rows' own pages is unchanged.
    Every K code is 1 and q is 1; K scales are 0 except at the jump keys (positions 200-203 and 230, in the
    second step of the second 8-page chunk of the 16-page prefix), of kv head 1.  Outputs match the checker
    relative to the largest |v| in kv head 1's heads, the quantized bar elsewhere; the plain decode (p <= 1,
    no overflow) too."""
    import math

    rng = np.random.default_rng(48)
    shared, B = 16, 12
    ctx = shared * 16 + rng.integers(1, 100, size=B) - 1
    c = cases.make_case(48, B, 8, 2, 128, ctx, act="bf16", kv="i8", shared_prefix_blocks=shared)
    c.k_pool[...] = 1
    c.k_scale[...] = 0.0
    for t in (200, 201, 202, 203, 230):
        page, slot = c.block_table[0, t // 16], t % 16
        c.k_scale[page, slot, 1] = np.float32(7.9 * math.log(2.0) / math.sqrt(128))
        c.v_scale[page, slot, 1] = np.float32(big / 127.0)
    c.k_new[...] = cases.encode(np.zeros(c.k_new.shape, np.float32), c.act)
    c.q = cases.encode(np.ones(c.q.shape, np.float32), c.act)
    got, plain, ref = _run(ff, gpu, c, shared)
    for out, what in ((got, "shared-prefix decode"), (plain, "plain decode")):
        _check(out[:, :4], ref[:, :4], c.act, 2e-2, what + ", kv head 0")
        err = float(np.abs(out[:, 4:].astype(np.float64) - ref[:, 4:]).max())
        print(f"  {what}, kv head 1: max |out| {float(np.abs(ref[:, 4:]).max()):.3e}, max-abs err {err:.3e}",
              flush=True)
        assert np.isfinite(out).all() and err <= 2e-2 * big
    assert float(np.abs(ref[:, 4:]).max()) > 0.1 * big


@pytest.mark.parametrize("big", [7.0e4, float("inf")])
def test_shared_prefix_large_v(ff, gpu, big):
    """bf16 V values beyond f16's range in the shared pages: the prefix kernel's f16 PV products overflow, and
    its workgroups that meet them must redo their pages with bf16 products.  Outputs match the checker relative
    to the largest |v| (infinite V: the same non-finite outputs)."""
    rng = np.random.default_rng(47)
    shared, B = 16, 24
    ctx = shared * 16 + rng.integers(1, 200, size=B) - 1
    c = cases.make_case(47, B, 32, 8, 128, ctx, act="bf16", shared_prefix_blocks=shared)
    enc = cases.encode(np.array([big, -big], np.float32), O.DTYPE_BF16)
    for t in rng.choice(shared * 16, size=5, replace=False):
        c.v_pool[c.block_table[0, t // 16], t % 16, 3, rng.integers(0, 128)] = enc[rng.integers(0, 2)]
    got, plain, ref = _run(ff, gpu, c, shared)
    for g, what in ((got, "shared-prefix decode"), (plain, "plain decode")):
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(g), fin), f"{what}: non-finite outputs differ from the checker"
        if np.isfinite(big):
            err = float(np.abs(g.astype(np.float64) - ref).max())
            print(f"  {what}: max-abs err {err:.3e} against |v| up to {big:.1e}", flush=True)
            assert err <= 2e-3 * big
        else:  # kv head 3's heads (12..15) hold the infinities; the others keep the ordinary bar
            _check(g[:, :12], ref[:, :12], c.act, 2e-3, what)


def test_c4_shape(ff, gpu):
    """BASELINE config 4's decode: 120 rows over one 2048-token prefix, private suffixes U[64, 1024]."""
    rng = np.random.default_rng(44)
    ctx = 2048 + rng.integers(64, 1025, size=120) - 1
    c = cases.make_case(44, 120, 32, 8, 128, ctx, act="bf16", shared_prefix_blocks=128)
    _both(ff, gpu, c, 128)


def test_rows_shorter_than_or_ending_at_the_prefix(ff, gpu):
    """Rows that end inside the prefix (they attend only their own tokens), exactly at its end (no private page),
    one token past it, and a one-token row."""
    ctx = [10, 127, 128, 200, 0, 300, 143, 160]
    c = cases.make_case(45, len(ctx), 16, 4, 128, ctx, act="bf16", shared_prefix_blocks=9, max_blocks=20)
    # the entry point's precondition: entries 0 .. shared_blocks - 1 hold the prefix pages in every row's table
    # (make_case fills a row's table only as far as its own tokens reach)
    c.block_table[:, :9] = c.block_table[int(np.argmax(c.ctx)), :9]
    _both(ff, gpu, c, 9)


@pytest.mark.parametrize("D,G", [(64, 1), (64, 8), (128, 16), (256, 4), (256, 7), (128, 32), (64, 40)])
def test_head_shapes(ff, gpu, D, G):
    rng = np.random.default_rng(46 + D + G)
    ctx = 160 + rng.integers(0, 300, size=10)
    c = cases.make_case(46 + D + G, 10, 2 * G, 2, D, ctx, act="bf16", shared_prefix_blocks=10)
    _both(ff, gpu, c, 10)


@pytest.mark.parametrize("act,kv,tol", [("f16", "f16", 2e-3), ("f32", "bf16", 2e-3), ("bf16", "i8", 2e-2),
                                        ("bf16", "fp8", 2e-2), ("f16", "i8", 2e-2), ("f32", "fp8", 2e-2)])
def test_dtypes(ff, gpu, act, kv, tol):
    rng = np.random.default_rng(47)
    ctx = 256 + rng.integers(0, 400, size=12)
    c = cases.make_case(47, 12, 32, 8, 128, ctx, act=act, kv=kv, shared_prefix_blocks=16)
    _both(ff, gpu, c, 16, tol=tol)


@pytest.mark.parametrize("kv,D,G", [("i8", 64, 4), ("i8", 256, 2), ("fp8", 64, 4), ("bf16", 64, 4)])
def test_quantized_head_shapes(ff, gpu, kv, D, G):
    """The prefix kernel's other load layouts: int8 pages at head_dim 64 (codes converted to f16 tiles in LDS,
    one run per wave) and 256 (8-bit tiles), fp8 at 64, bf16 at 64 (f16 V tiles)."""
    rng = np.random.default_rng(49 + D + G)
    ctx = 176 + rng.integers(0, 300, size=10)
    c = cases.make_case(49 + D + G, 10, 2 * G, 2, D, ctx, act="bf16", kv=kv, shared_prefix_blocks=11)
    _both(ff, gpu, c, 11, tol=2e-3 if kv == "bf16" else 2e-2)


def test_truncated_context(ff, gpu):
    """max_context_len below some rows' lengths, and below the prefix itself."""
    rng = np.random.default_rng(48)
    ctx = 320 + rng.integers(0, 500, size=9)
    c = cases.make_case(48, 9, 32, 8, 128, ctx, act="bf16", shared_prefix_blocks=20)
    _both(ff, gpu, c, 20, max_context_len=500)
    _both(ff, gpu, c, 20, max_context_len=200)


@pytest.mark.parametrize("kv,tol", [("bf16", 2e-3), ("i8", 2e-2), ("fp8", 2e-2)])
def test_hole_in_the_prefix(ff, gpu, kv, tol):
    """An invalid entry inside the shared prefix (every row holds it) is skipped like in the plain decode (for
    int8 its per-token scales are not read either)."""
    rng = np.random.default_rng(49)
    ctx = 200 + rng.integers(0, 300, size=8)
    c = cases.make_case(49, 8, 16, 4, 128, ctx, act="bf16", kv=kv, shared_prefix_blocks=12)
    tbl = c.block_table.copy()
    tbl[:, 3] = -1
    tbl[:, 7] = c.num_blocks + 3
    _both(ff, gpu, c, 12, tol=tol, table=tbl)


def test_zero_shared_blocks_is_the_plain_decode(ff, gpu):
    rng = np.random.default_rng(50)
    c = cases.make_case(50, 6, 32, 8, 128, rng.integers(1, 700, size=6), act="bf16")
    got, plain, ref = _run(ff, gpu, c, 0)
    assert np.array_equal(got, plain)
    _check(got, ref, c.act, 2e-3, "shared_blocks = 0")


def test_workspace_with_garbage_reused(ff, gpu):
    """One explicit workspace, filled with garbage, serves calls of different batch sizes and prefixes."""
    import torch

    ws = ff.shared_prefix_workspace(64, 32, 8, 128, 200, 64, device=gpu)
    ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, device=gpu))
    rng = np.random.default_rng(51)
    for i, (B, shared) in enumerate([(64, 64), (5, 3), (40, 64), (5, 3)]):
        ctx = shared * 16 + rng.integers(0, 900, size=B)
        c = cases.make_case(51 + i, B, 32, 8, 128, ctx, act="bf16", shared_prefix_blocks=shared, max_blocks=200)
        got, _, ref = _run(ff, gpu, c, shared, workspace=ws)
        _check(got, ref, c.act, 2e-3, f"call {i}")


@pytest.mark.parametrize("D", [80, 96, 112])
def test_head_dims_without_prefix_kernel_take_the_plain_decode(ff, gpu, D):
    """head_dim 80, 96 and 112 have no prefix-partial (prefill) kernel: the shared-prefix entry point runs the
    plain decode, same results."""
    rng = np.random.default_rng(D)
    ctx = 8 * 16 + rng.integers(1, 200, size=10) - 1
    c = cases.make_case(D, 10, 16, 4, D, ctx, act="bf16", shared_prefix_blocks=8)
    _both(ff, gpu, c, 8)



def test_decode_and_prefill_on_two_streams(ff, gpu):
    """A C4-style step with the decode rows (append + shared-prefix decode) on a second stream beside the chunk
    rows (append + prefill) on the first, forked and joined with events: the halves touch disjoint rows (shared
    prefix pages are only read), so outputs and pages equal the one-stream step's bit for bit."""
    import torch

    import gpu_util as gu

    rng = np.random.default_rng(97)
    Bd, Bc, S, shared = 12, 2, 40, 8
    ctx = shared * 16 + rng.integers(1, 300, size=Bd + Bc) - 1
    c = cases.make_case(97, Bd + Bc, 32, 8, 128, ctx, act="bf16", S=S, shared_prefix_blocks=shared)
    print(f"case two-stream step Bd={Bd} Bc={Bc} S={S} shared={shared}", flush=True)
    tbl = torch.from_numpy(c.block_table).to(gpu)
    cx = torch.from_numpy(c.ctx).to(gpu)
    kn, vn, q = gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu), gu.to_dev(c.q, c.act, gpu)
    qc = gu.to_dev(cases.encode(rng.standard_normal((Bc, S, 32, 128), dtype=np.float32), c.act), c.act, gpu)

    def run(two):
        kp, vp = gu.to_dev(c.k_pool, c.kv, gpu), gu.to_dev(c.v_pool, c.kv, gpu)
        s1 = torch.cuda.current_stream()
        s2 = torch.cuda.Stream(device=gpu) if two else s1
        fork, join = torch.cuda.Event(), torch.cuda.Event()
        fork.record(s1)
        s2.wait_event(fork)
        ff.append_kv_cache(kn[:Bd, :1].contiguous(), vn[:Bd, :1].contiguous(), kp, vp, tbl[:Bd], cx[:Bd], stream=s2)
        od = ff.paged_attention_shared_prefix(q[:Bd], kp, vp, tbl[:Bd], cx[:Bd], shared, stream=s2)
        ff.append_kv_cache(kn[Bd:].contiguous(), vn[Bd:].contiguous(), kp, vp, tbl[Bd:], cx[Bd:], stream=s1)
        oc = ff.paged_prefill(qc, kp, vp, tbl[Bd:], cx[Bd:], stream=s1)
        join.record(s2)
        s1.wait_event(join)
        torch.cuda.synchronize()
        return [gu.to_host(t, np.uint16) for t in (od, oc, kp, vp)]

    one, two = run(False), run(True)
    for what, a, b in zip(("decode out", "prefill out", "K pages", "V pages"), one, two):
        assert np.array_equal(a, b), what
