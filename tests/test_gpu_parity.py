"""Parity of the HIP path against the CPU checker on identical seeded inputs.

Bar: KV page bytes and int8/fp8 codes and scales bit-exact over the whole pool; decode outputs within max-abs
2e-3 for 16-bit KV (bf16/fp16 in, fp32 accumulate), 2e-2 for quantized KV, 1e-4 for fp32 everything.  The
GPU output (rounded to the activation dtype) is compared with the checker's fp32 value before rounding; the
rounding to the output format itself (half a bf16/fp16 ulp at the value's magnitude, which exceeds 2e-2 once
|O| >= 8 as with config 5's x8 outliers) is allowed on top of the tolerance.  fp32-output cases carry no
rounding allowance.
"""

import math

import numpy as np
import pytest

import cases
import oracle as O

pytestmark = pytest.mark.gpu

TOL = {("f32", "f32"): 1e-4, ("bf16", "bf16"): 2e-3, ("f16", "f16"): 2e-3, ("bf16", "i8"): 2e-2,
       ("bf16", "fp8"): 2e-2, ("f16", "i8"): 2e-2, ("f16", "fp8"): 2e-2, ("f32", "i8"): 2e-2,
       ("f32", "fp8"): 2e-2, ("bf16", "f32"): 2e-3, ("f32", "bf16"): 1e-4, ("f32", "f16"): 1e-4}


def half_ulp(x: np.ndarray, act: int) -> np.ndarray:
    """Half the spacing of the output format at |x| (0 for fp32)."""
    if act == O.DTYPE_F32:
        return np.zeros_like(x)
    mant, emin = (7, -126) if act == O.DTYPE_BF16 else (10, -14)
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** emin)))
    return 2.0 ** (e - mant - 1)


def _check(ff, dev, c, tol, max_context_len=0, workspace=False):
    import gpu_util as gu

    print(f"case seed={c.seed} B={c.B} Hq={c.Hq} Hkv={c.Hkv} D={c.D} act={c.act} kv={c.kv} "
          f"ctx_max={int(c.ctx.max())}", flush=True)
    kp, vp, ks, vs, out, out32 = cases.oracle_step(c, max_context_len=max_context_len)
    gk, gv, gks, gvs, gout = gu.run_step(ff, c, dev, max_context_len=max_context_len, workspace=workspace)
    assert np.array_equal(gk.view(np.uint8), kp.view(np.uint8)), "K pages differ"
    assert np.array_equal(gv.view(np.uint8), vp.view(np.uint8)), "V pages differ"
    if ks is not None and c.kv == O.DTYPE_I8:
        assert np.array_equal(gks.view(np.uint32), ks.view(np.uint32)), "K scales differ"
        assert np.array_equal(gvs.view(np.uint32), vs.view(np.uint32)), "V scales differ"
    got = gu.out_to_f32(gout, c.act).reshape(out32.shape)
    diff = np.abs(got.astype(np.float64) - out32)
    err = float(diff.max())
    excess = float((diff - half_ulp(np.maximum(np.abs(got), np.abs(out32)), c.act)).max())
    print(f"  max-abs err {err:.3e}, beyond output rounding {excess:.3e} (tol {tol})", flush=True)
    assert excess <= tol


@pytest.mark.parametrize("act,kv", [("bf16", "bf16"), ("f16", "f16"), ("f32", "f32"), ("bf16", "i8"),
                                    ("bf16", "fp8"), ("f32", "bf16"), ("f16", "i8"), ("f32", "fp8")])
def test_config1(ff, gpu, act, kv):
    _check(ff, gpu, cases.config1(act=act, kv=kv), TOL[(act, kv)])


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("G", [1, 2, 7, 16])
def test_head_shapes(ff, gpu, D, G):
    Hkv = 2
    rng = np.random.default_rng(D * 100 + G)
    ctx = rng.integers(0, 700, size=5)
    c = cases.make_case(11 + G, 5, Hkv * G, Hkv, D, ctx, act="bf16", input_scale=1 / math.sqrt(D))
    _check(ff, gpu, c, 2e-3)


@pytest.mark.parametrize("D,act,kv", [(128, "bf16", "bf16"), (96, "bf16", "bf16"), (128, "f32", "f32"),
                                      (128, "bf16", "i8"), (40, "f16", "f16"), (112, "bf16", "bf16")])
def test_peaked_softmax(ff, gpu, D, act, kv):
    """Inputs at 3x the usual scale: scores spread over tens of log2 units, so the running maximum jumps often and
    far, and the lazily rescaled softmax state (rescaled only when a score passes the reference by 2^8) is
    rescaled many times per row, on the matrix-core kernel (D 128 and 96) and the vector kernel (D 112 / 40,
    fp32 pages)."""
    rng = np.random.default_rng(300 + D + len(act) + len(kv))
    ctx = rng.integers(0, 2500, size=6)
    c = cases.make_case(3000 + D, 6, 16, 4, D, ctx, act=act, kv=kv, input_scale=3.0)
    _check(ff, gpu, c, TOL[(act, kv)])


@pytest.mark.parametrize("kv", ["i8", "fp8"])
def test_head_dim_64_quantized(ff, gpu, kv):
    """Quantize-on-append with 8 lanes per row (head_dim 64: the int8 row maximum over two quads and their
    mirror), pages and scales bit-exact, then the decode."""
    rng = np.random.default_rng(64 + len(kv))
    ctx = rng.integers(0, 500, size=6)
    c = cases.make_case(640 + len(kv), 6, 8, 2, 64, ctx, act="bf16", kv=kv, S=3, input_scale=1 / 8)
    _check(ff, gpu, c, 2e-2)


@pytest.mark.parametrize("act,kv", [("f16", "f16"), ("f32", "bf16"), ("bf16", "f16"), ("bf16", "i8"), ("f16", "i8"),
                                    ("bf16", "fp8"), ("f32", "fp8")])
def test_head_dim_256_dtypes(ff, gpu, act, kv):
    """head_dim 256 keeps one page in flight per wave (two would not fit the registers), for every q / cache
    type pair, including the ones whose q is split into two MFMA parts."""
    rng = np.random.default_rng(256)
    ctx = rng.integers(0, 900, size=7)
    c = cases.make_case(256, 7, 16, 4, 256, ctx, act=act, kv=kv, input_scale=1 / math.sqrt(256))
    _check(ff, gpu, c, 2e-3 if kv in ("f16", "bf16") else 2e-2)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("G", [1, 7, 16])
@pytest.mark.parametrize("kv", ["i8", "fp8"])
def test_quantized_head_shapes(ff, gpu, D, G, kv):
    """8-bit pages at head_dim 64 and 256 on the matrix cores: each lane stages its 16 codes of a V row as two
    converted 16-byte chunks in the wave's LDS tile, whose chunk order differs by lane group (the pair of a
    16-dim tile swapped for lanes 4..7 of every 8); outputs within the 8-bit bar."""
    Hkv = 2
    rng = np.random.default_rng(D * 1000 + G * 10 + len(kv))
    ctx = rng.integers(0, 700, size=5)
    c = cases.make_case(31 + G + D, 5, Hkv * G, Hkv, D, ctx, act="bf16", kv=kv, input_scale=1 / math.sqrt(D))
    _check(ff, gpu, c, TOL[("bf16", kv)])


@pytest.mark.parametrize("D", [8, 40, 80, 96, 112])
@pytest.mark.parametrize("act,kv", [("bf16", "bf16"), ("f16", "f16"), ("f32", "f32"), ("bf16", "i8"),
                                    ("bf16", "fp8"), ("f32", "fp8"), ("f16", "i8"), ("f16", "fp8")])
def test_head_dims_multiple_of_8(ff, gpu, D, act, kv):
    """Any head_dim that is a multiple of 8 up to 128, as the reference's decode takes (one 8-element vector per
    lane of a 16-lane group, src/kernels/attention.cu:307-316) and its append (any head_dim up to 128,
    src/model/qwen_model.cu:21-47): pages and int8 scales bit-exact, outputs within the bar.  head_dim 96 runs on
    the matrix cores (three k-steps of 32 dims; 8-bit codes read the odd last k-step's 8 codes alone), and so do
    80 and 112 (k-steps of 32 dims and a last one of 16, 4 dims per lane), the others on the vector kernel with 16
    lanes per token, those past head_dim / 8 idle."""
    rng = np.random.default_rng(D * 7 + len(act) + len(kv))
    ctx = rng.integers(0, 600, size=5)
    c = cases.make_case(80 + D, 5, 16, 4, D, ctx, act=act, kv=kv, input_scale=1 / math.sqrt(D))
    _check(ff, gpu, c, TOL[(act, kv)])


@pytest.mark.parametrize("kv", ["bf16", "i8"])
def test_head_dim_96_multi_token_append(ff, gpu, kv):
    """A 37-token chunk appended per row at head_dim 96 (12 of 16 lanes per row active), then decode."""
    c = cases.make_case(96, 3, 16, 4, 96, [0, 45, 300], act="bf16", kv=kv, S=37)
    _check(ff, gpu, c, 2e-3 if kv == "bf16" else 2e-2)


@pytest.mark.parametrize("G,Hkv,D,act,kv", [(17, 2, 128, "bf16", "bf16"), (32, 1, 128, "bf16", "bf16"),
                                             (48, 2, 128, "f16", "f16"), (24, 2, 64, "bf16", "fp8"),
                                             (32, 2, 128, "bf16", "i8"), (20, 1, 256, "f32", "bf16"),
                                             (20, 2, 96, "bf16", "bf16"), (40, 1, 96, "f16", "f16"),
                                             (20, 2, 96, "bf16", "i8"), (20, 2, 96, "bf16", "fp8"),
                                             (24, 1, 96, "f16", "i8"), (20, 2, 112, "bf16", "bf16"),
                                             (24, 1, 80, "f16", "i8"), (18, 2, 112, "f32", "fp8")])
def test_groups_over_16(ff, gpu, G, Hkv, D, act, kv):
    """GQA groups above 16 query heads per KV head (MQA-style): one wave per block of 16 heads of the group."""
    rng = np.random.default_rng(G * 10 + Hkv)
    ctx = rng.integers(0, 800, size=6)
    c = cases.make_case(70 + G, 6, G * Hkv, Hkv, D, ctx, act=act, kv=kv, input_scale=1 / math.sqrt(D))
    _check(ff, gpu, c, 2e-3 if kv in ("f16", "bf16") else 2e-2)


def test_config2_full(ff, gpu):
    """BASELINE config 2 at full size: Qwen3-8B layer, B=64, contexts U[512, 4096]."""
    rng = np.random.default_rng(2)
    ctx = rng.integers(512, 4097, size=64)
    c = cases.make_case(2, 64, 32, 8, 128, ctx, act="bf16")
    _check(ff, gpu, c, 2e-3, max_context_len=4097, workspace=True)


def test_split_k_long_context(ff, gpu):
    """Config-3 shape (Hq28/Hkv4, G = 7) with 8k contexts so that rows span many split-K chunks."""
    c = cases.make_case(3, 4, 28, 4, 128, [8191, 8000, 4100, 300], act="bf16")
    _check(ff, gpu, c, 2e-3)


def test_quantized_outliers(ff, gpu):
    """Config-5 style inputs: N(0,1) with 1% outliers at x8, int8 and fp8 caches."""
    rng = np.random.default_rng(5)
    ctx = rng.integers(1024, 2048, size=8)
    for act in ("bf16", "f32"):
        for kv in ("i8", "fp8"):
            c = cases.make_case(5, 8, 32, 8, 128, ctx, act=act, kv=kv, outlier_frac=0.01)
            _check(ff, gpu, c, 2e-2)


def test_invalid_pages_and_empty_rows(ff, gpu):
    """Negative / out-of-pool block ids are skipped by append and masked by decode; a row with no valid token
    gives zeros (the reference reads and writes block -1 here)."""
    c = cases.make_case(9, 6, 8, 4, 128, [40, 0, 100, 31, 15, 64], act="bf16")
    c.block_table[0, 1] = -1                 # hole in the middle of row 0
    c.block_table[2, :] = -1                 # row 2 fully padded
    c.block_table[3, 0] = c.num_blocks + 3   # out of the pool
    c.ctx[4] = -1                            # no tokens at all: appends at position -1 is skipped
    _check(ff, gpu, c, 2e-3)


def test_multi_token_append_chunk(ff, gpu):
    """Chunked-prefill style append of S=64 tokens per row, then decode."""
    c = cases.make_case(4, 3, 32, 8, 128, [0, 37, 200], act="bf16", S=64)
    _check(ff, gpu, c, 2e-3)


def test_many_short_rows(ff, gpu):
    """700 rows (more rows than scan threads per workgroup), contexts 0..40, some rows without tokens."""
    rng = np.random.default_rng(21)
    ctx = rng.integers(0, 41, size=700)
    ctx[::97] = -1                           # rows with no token at all: zeros
    c = cases.make_case(21, 700, 8, 2, 128, ctx, act="bf16", input_scale=1 / math.sqrt(128))
    _check(ff, gpu, c, 2e-3)


@pytest.mark.parametrize("Hq,Hkv", [(16, 1), (12, 6), (40, 5)])
def test_kv_head_groupings(ff, gpu, Hq, Hkv):
    """One KV head (64-thread workgroups), and KV-head counts that leave idle waves in the last group."""
    rng = np.random.default_rng(Hq * 10 + Hkv)
    ctx = rng.integers(100, 1500, size=6)
    c = cases.make_case(30 + Hkv, 6, Hq, Hkv, 128, ctx, act="bf16")
    _check(ff, gpu, c, 2e-3)


def test_truncated_context(ff, gpu):
    """max_context_len below context_lens + 1 clamps the attended tokens on both sides."""
    c = cases.make_case(22, 3, 32, 8, 128, [700, 100, 1000], act="bf16")
    _check(ff, gpu, c, 2e-3, max_context_len=513)


@pytest.mark.parametrize("act,kv", [("f16", "fp8"), ("bf16", "f16"), ("f16", "bf16")])
def test_mixed_dtypes(ff, gpu, act, kv):
    """q/out in another type than the cache (q is split into hi + lo MFMA parts)."""
    rng = np.random.default_rng(23)
    ctx = rng.integers(10, 900, size=5)
    c = cases.make_case(23, 5, 16, 4, 128, ctx, act=act, kv=kv)
    _check(ff, gpu, c, 2e-2 if kv in ("i8", "fp8") else 2e-3)


def test_generic_and_mfma_kernels_agree(ff, gpu):
    """The generic fp32-cache kernel and the matrix-core kernel on the same bf16 data (cache widened to fp32
    for the generic one) agree within the bf16 tolerance."""
    import torch

    import gpu_util as gu

    c = cases.make_case(24, 4, 32, 8, 128, [300, 1200, 47, 2050], act="f32", kv="bf16")
    kp, vp, _, _, _, out32 = cases.oracle_step(c)
    _, _, _, _, gout = gu.run_step(ff, c, gpu)
    kf = torch.from_numpy(O.bf16_to_f32(kp)).to(gpu)
    vf = torch.from_numpy(O.bf16_to_f32(vp)).to(gpu)
    q = torch.from_numpy(c.q).to(gpu)
    bt = torch.from_numpy(c.block_table).to(gpu)
    ctx = torch.from_numpy(c.ctx).to(gpu)
    gen = ff.paged_attention(q, kf, vf, bt, ctx).cpu().numpy().reshape(out32.shape)
    mf = gout.reshape(out32.shape)
    assert np.abs(gen - out32).max() <= 1e-4
    assert np.abs(mf - out32).max() <= 2e-3


def test_workspace_reused_across_calls(ff, gpu):
    """One workspace, filled with garbage first, serves consecutive calls of different shapes: B=64 (split-K
    partials folded by the per-row merge) and B=5 (folded by the per-(row, head) merge) alternating, so each call
    finds the other layout's partials and metadata in its slots and must overwrite every entry it reads."""
    import torch

    import gpu_util as gu

    rng = np.random.default_rng(25)
    big = cases.make_case(25, 64, 32, 8, 128, rng.integers(512, 4097, size=64), act="bf16")
    small = cases.make_case(26, 5, 32, 8, 128, rng.integers(1, 900, size=5), act="bf16")
    ws = ff.decode_workspace(64, 32, 128, max(big.max_blocks, small.max_blocks), device=gpu)
    ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, device=gpu))
    for c in (big, small, big, small, big):
        kp, vp, _, _, _, out32 = cases.oracle_step(c)
        kd, vd = gu.to_dev(kp, c.kv, gpu), gu.to_dev(vp, c.kv, gpu)
        out = ff.paged_attention(gu.to_dev(c.q, c.act, gpu), kd, vd, torch.from_numpy(c.block_table).to(gpu),
                                 torch.from_numpy(c.ctx).to(gpu), workspace=ws)
        torch.cuda.synchronize()
        got = gu.out_to_f32(gu.to_host(out, np.uint16), c.act).reshape(out32.shape)
        assert np.abs(got - out32).max() <= 2e-3 + 2 ** -8


def test_graph_capture_replays(ff, gpu):
    """Append + decode captured in a hipGraph (through torch.cuda.graph) and replayed several times, with eager
    work and host synchronization between replays; every replay matches the eager result."""
    import torch

    import gpu_util as gu

    rng = np.random.default_rng(27)
    c = cases.make_case(27, 16, 32, 8, 128, rng.integers(100, 2000, size=16), act="bf16")
    kp0, vp0 = gu.to_dev(c.k_pool, c.kv, gpu), gu.to_dev(c.v_pool, c.kv, gpu)
    bt = torch.from_numpy(c.block_table).to(gpu)
    ctx = torch.from_numpy(c.ctx).to(gpu)
    kn, vn, q = gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu), gu.to_dev(c.q, c.act, gpu)
    ws = ff.decode_workspace(c.B, c.Hq, c.D, c.max_blocks, device=gpu)
    out = torch.empty((c.B, 1, c.Hq * c.D), dtype=torch.bfloat16, device=gpu)
    kp, vp = kp0.clone(), vp0.clone()

    def step():
        ff.append_kv_cache(kn, vn, kp, vp, bt, ctx)
        ff.paged_attention(q, kp, vp, bt, ctx, out=out, workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()                                   # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(4):
        kp.copy_(kp0)
        vp.copy_(vp0)
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
