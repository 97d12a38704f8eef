"""Pins for the CPU checker under oracle/ (CPU only).

The reference ships no tests, fixtures or CPU implementation of this path, so the checker is pinned by:
  * the golden fixtures under tests/golden/ (written by make_golden.py from torch-CPU and numpy only),
  * library routines: numpy/torch round-to-nearest-even casts, torch.float8_e4m3fn, torch.round,
    torch scaled_dot_product_attention,
  * closed forms and invariants of attention (one token, constant keys, a dominant logit, GQA symmetry,
    shared-prefix tables, permuted physical pages),
  * mutation checks: a plausible mistake (dropped +1 token, wrong GQA map, swapped K/V, wrong scale, wrong
    page) planted in the checker's inputs must make the golden comparison fail.
"""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import cases
import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- conversions -------------------------------------------------------------------------------------------

def test_bf16_all_codes_round_trip():
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = O.bf16_to_f32(codes)
    back = O.f32_to_bf16(vals)
    nan = np.isnan(vals)
    assert np.array_equal(back[~nan], codes[~nan])
    assert np.all((back[nan] & 0x7fc0) == 0x7fc0)
    ref = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(vals[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 200000),
                        # exact ties: bf16 value + half an ulp, both parities
                        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
                        np.array([np.inf, -np.inf, 0.0, -0.0, 3.3895314e38, 1e-45], np.float32)]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), ref)


def test_f16_matches_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 200000),
                        (np.arange(1, 4000, dtype=np.uint32) << 13 | 0x1000).view(np.float32),  # ties
                        np.array([65504.0, 65519.99, 65520.0, 1e9, np.inf, -np.inf, 5.96e-8, 2.98e-8, 0.0],
                                 np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16(x), ref)
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    v = O.f16_to_f32(codes)
    nan = np.isnan(v)
    assert np.array_equal(v[~nan], codes.view(np.float16)[~nan].astype(np.float32))


def test_e4m3_codes_and_rounding():
    codes = np.arange(256, dtype=np.uint8)
    v = O.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(v), nan) and nan.sum() == 2
    assert np.array_equal(v[~nan], ref[~nan])
    assert v[0x7e] == 448.0 and v[0x01] == 2.0 ** -9 and v[0x08] == 2.0 ** -6
    back = O.f32_to_e4m3(v[~nan])
    assert np.array_equal(back, codes[~nan])
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-448, 448, 100000), rng.standard_normal(100000) * 2.0 ** -7,
                        (v[1:0x7e].astype(np.float64) + v[2:0x7f].astype(np.float64)) / 2]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.f32_to_e4m3(x), ref)
    # saturation edge (OCP OFP8: satfinite) where torch's non-saturating cast differs
    edge = O.f32_to_e4m3(np.array([448.0, 464.0, 465.0, 1e6, np.inf, -np.inf, np.nan, -500.0], np.float32))
    assert list(edge) == [0x7e, 0x7e, 0x7e, 0x7e, 0x7e, 0xfe, 0x7f, 0xfe]


def test_int8_row_quant_matches_torch_round():
    rng = np.random.default_rng(3)
    for n in (64, 128, 256):
        for _ in range(200):
            x = rng.standard_normal(n).astype(np.float32) * np.float32(rng.uniform(1e-3, 50))
            x[rng.integers(0, n)] *= 8
            q, s = O.quant_i8_row(x)
            xt = torch.from_numpy(x)
            st = xt.abs().max() / torch.tensor(127.0)
            assert np.float32(s) == st.item()
            qt = torch.clamp(torch.round(xt / st), -127, 127).to(torch.int8).numpy()
            assert np.array_equal(q, qt)
    q, s = O.quant_i8_row(np.zeros(128, np.float32))
    assert s == 0.0 and not q.any()
    # half-even: values landing exactly on .5 after the divide
    x = np.array([127.0, 0.5, 1.5, 2.5, -2.5, 126.5], np.float32)
    q, s = O.quant_i8_row(x)
    assert s == 1.0 and list(q) == [127, 0, 2, 2, -2, 126]


# ---- golden fixtures ---------------------------------------------------------------------------------------

def _golden(kv):
    return dict(np.load(GOLDEN / f"golden_{kv}.npz"))


KV_CODE = {"bf16": O.DTYPE_BF16, "i8": O.DTYPE_I8, "fp8": O.DTYPE_FP8}
GOLDEN_TOL = {"bf16": 2e-6, "i8": 2e-6, "fp8": 2e-6}


def _golden_decode(g, kv, **over):
    kvd = KV_CODE[kv]
    ks = vs = None
    if kv == "i8":
        ks, vs = g["k_scale_after"], g["v_scale_after"]
    elif kv == "fp8":
        ks, vs = g["k_head_scale"], g["v_head_scale"]
    args = dict(q=g["q_bf16"], k=g["k_pool_after"], v=g["v_pool_after"], table=g["block_table"], ctx=g["ctx"],
                scale=0.0)
    args.update(over)
    _, out32 = O.paged_decode(args["q"], O.DTYPE_BF16, args["k"], args["v"], kvd, args["table"], args["ctx"], ks,
                              vs, scale=args["scale"], threads=2)
    return out32


@pytest.mark.parametrize("kv", ["bf16", "i8", "fp8"])
def test_golden_append_bit_exact(kv):
    g = _golden(kv)
    kp, vp = g["k_pool_before"].copy(), g["v_pool_before"].copy()
    ks = vs = None
    if kv == "i8":
        ks, vs = g["k_scale_before"].copy(), g["v_scale_before"].copy()
    elif kv == "fp8":
        ks, vs = g["k_head_scale"].copy(), g["v_head_scale"].copy()
    O.append(g["k_new_bf16"], g["v_new_bf16"], O.DTYPE_BF16, kp, vp, KV_CODE[kv], g["block_table"], g["ctx"], ks, vs,
             num_blocks=int(g["num_blocks"]))
    assert np.array_equal(kp.view(np.uint8), g["k_pool_after"].view(np.uint8))
    assert np.array_equal(vp.view(np.uint8), g["v_pool_after"].view(np.uint8))
    if kv == "i8":
        assert np.array_equal(ks.view(np.uint32), g["k_scale_after"].view(np.uint32))
        assert np.array_equal(vs.view(np.uint32), g["v_scale_after"].view(np.uint32))


@pytest.mark.parametrize("kv", ["bf16", "i8", "fp8"])
def test_golden_decode(kv):
    g = _golden(kv)
    out32 = _golden_decode(g, kv)
    err = np.abs(out32 - g["out_f64"]).max()
    assert err <= GOLDEN_TOL[kv], err


def test_golden_detects_planted_mistakes():
    """Each plausible mistake, planted in the checker's inputs, moves the output far outside the tolerance."""
    g = _golden("bf16")
    tol = GOLDEN_TOL["bf16"]
    ref = g["out_f64"]
    mistakes = {
        "dropped +1 token (attend context_lens only)": dict(ctx=g["ctx"] - 1),
        "one extra token": dict(ctx=g["ctx"] + 1),
        "GQA map h % Hkv instead of h / G": dict(q=g["q_bf16"][:, :, [0, 2, 1, 3]]),
        "K and V swapped": dict(k=g["v_pool_after"], v=g["k_pool_after"]),
        "scale 1/D instead of 1/sqrt(D)": dict(scale=1.0 / 128),
        "block table row off by one": dict(table=np.roll(g["block_table"], 1, axis=0)),
        "pages of a row reversed": dict(table=np.where(g["block_table"] >= 0,
                                                       g["block_table"][:, ::-1], -1).astype(np.int32)),
    }
    for name, over in mistakes.items():
        if "ctx" in over:
            over["ctx"] = over["ctx"].astype(np.int32)
        err = np.abs(_golden_decode(g, "bf16", **over) - ref).max()
        assert err > 50 * tol, f"golden check misses: {name} (err {err})"


# ---- decode closed forms and invariants -------------------------------------------------------------------

def _sdpa_ref(c: cases.Case, kp, vp, ks=None, vs=None):
    """torch SDPA in float64 on the gathered, dequantized tokens of each row."""
    out = np.zeros((c.B, c.Hq, c.D))
    for b in range(c.B):
        L = int(c.ctx[b]) + 1
        tok = np.arange(L)
        pg, sl = c.block_table[b, tok // 16], tok % 16

        def deq(pool, sc):
            if c.kv == O.DTYPE_I8:
                return pool[pg, sl].astype(np.float64) * sc[pg, sl][..., None]
            if c.kv == O.DTYPE_FP8:
                return O.e4m3_to_f32(pool[pg, sl]).astype(np.float64) * sc[None, :, None]
            return cases.decode(pool[pg, sl], c.kv).astype(np.float64)

        K = torch.from_numpy(deq(kp, ks)).permute(1, 0, 2).repeat_interleave(c.Hq // c.Hkv, 0).contiguous()
        V = torch.from_numpy(deq(vp, vs)).permute(1, 0, 2).repeat_interleave(c.Hq // c.Hkv, 0).contiguous()
        q = torch.from_numpy(cases.decode(c.q[b, 0], c.act).astype(np.float64))[:, None, :]
        out[b] = torch.nn.functional.scaled_dot_product_attention(q, K, V, scale=1 / math.sqrt(c.D))[:, 0].numpy()
    return out


@pytest.mark.parametrize("act,kv,G,D", [("bf16", "bf16", 4, 128), ("f32", "f32", 7, 128), ("f16", "f16", 1, 64),
                                        ("bf16", "i8", 4, 128), ("f32", "fp8", 2, 256), ("bf16", "bf16", 16, 64)])
def test_decode_matches_sdpa(act, kv, G, D):
    rng = np.random.default_rng(G * 1000 + D)
    ctx = rng.integers(0, 300, size=5)
    ctx[0] = 15                      # L' = 16: the tail block is full
    ctx[1] = 16                      # L' = 17: one token in the tail block
    c = cases.make_case(40 + G, 5, 2 * G, 2, D, ctx, act=act, kv=kv, input_scale=1 / math.sqrt(D))
    kp, vp, ks, vs, _, out32 = cases.oracle_step(c, threads=2)
    ref = _sdpa_ref(c, kp, vp, ks, vs)
    assert np.abs(out32 - ref).max() < 5e-6


def test_decode_single_token_returns_v():
    c = cases.make_case(7, 3, 8, 2, 128, [0, 0, 0], act="f32")
    kp, vp, _, _, _, out32 = cases.oracle_step(c, threads=1)
    for b in range(3):
        page = c.block_table[b, 0]
        for h in range(8):
            assert np.array_equal(out32[b, h], vp[page, 0, h // 4])


def test_decode_constant_keys_gives_mean_v():
    c = cases.make_case(8, 2, 4, 1, 64, [37, 130], act="f32")
    c.k_pool[:] = 0.25
    c.k_new[:] = 0.25
    kp, vp, _, _, _, out32 = cases.oracle_step(c, threads=1)
    for b in range(2):
        L = int(c.ctx[b]) + 1
        tok = np.arange(L)
        mean = vp[c.block_table[b, tok // 16], tok % 16, 0].astype(np.float64).mean(0)
        assert np.abs(out32[b] - mean[None]).max() < 2e-6


def test_decode_dominant_logit_selects_token():
    c = cases.make_case(9, 1, 2, 1, 128, [90], act="f32", input_scale=0.01)
    j = 53
    page, slot = c.block_table[0, j // 16], j % 16
    c.q[0, 0, :, :] = 1.0
    c.k_pool[page, slot, 0, :] = 5.0              # logit 5*128/sqrt(128) ~ 56.6 above the rest
    kp, vp, _, _, _, out32 = cases.oracle_step(c, threads=1)
    assert np.abs(out32[0, 0] - vp[page, slot, 0]).max() < 1e-6


def test_decode_gqa_group_symmetry():
    c = cases.make_case(10, 3, 12, 3, 128, [50, 200, 17], act="bf16")
    c.q[:, :, 4:8, :] = c.q[:, :, 4:5, :]         # all heads of group 1 share one query
    *_, out32 = cases.oracle_step(c, threads=2)
    for h in range(5, 8):
        assert np.array_equal(out32[:, h], out32[:, 4])
    assert not np.array_equal(out32[:, 3], out32[:, 4])


def test_decode_shared_prefix_equals_private_copy():
    """Radix-tree sharing: rows whose tables point at the same prefix pages give the same result as rows that
    own private copies of those pages."""
    c = cases.make_case(11, 4, 8, 2, 128, [40, 90, 33, 64], act="bf16", shared_prefix_blocks=2)
    assert (c.block_table[:, :2] == c.block_table[0, :2]).all()
    *_, shared = cases.oracle_step(c, threads=2)
    # give every row its own copy of the two shared pages
    N0 = c.num_blocks
    extra = 2 * c.B
    grow = lambda p: np.concatenate([p, np.zeros((extra,) + p.shape[1:], p.dtype)])  # noqa: E731
    c.k_pool, c.v_pool = grow(c.k_pool), grow(c.v_pool)
    for b in range(c.B):
        for i in range(2):
            new = N0 + 2 * b + i
            c.k_pool[new] = c.k_pool[c.block_table[b, i]]
            c.v_pool[new] = c.v_pool[c.block_table[b, i]]
            c.block_table[b, i] = new
    c.num_blocks += extra
    *_, private = cases.oracle_step(c, threads=2)
    assert np.array_equal(shared, private)


def test_decode_page_permutation_invariance():
    c = cases.make_case(12, 3, 8, 4, 64, [100, 31, 250], act="bf16")
    *_, a = cases.oracle_step(c, threads=2)
    perm = np.random.default_rng(0).permutation(c.num_blocks)
    inv = np.argsort(perm)
    c.k_pool, c.v_pool = c.k_pool[perm], c.v_pool[perm]
    c.block_table = np.where(c.block_table >= 0, inv[np.maximum(c.block_table, 0)], -1).astype(np.int32)
    *_, b = cases.oracle_step(c, threads=2)
    assert np.array_equal(a, b)


def test_decode_f64_closed_form_agrees():
    c = cases.make_case(13, 4, 14, 2, 128, [1000, 5, 77, 160], act="bf16", kv="i8")
    kp, vp, ks, vs, _, out32 = cases.oracle_step(c, threads=2)
    o64 = O.paged_decode_f64(c.q, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    assert np.abs(out32 - o64).max() < 5e-6
    # the checker dequantizes in fp32 (code * scale rounded to float), the library routine in float64
    assert np.abs(o64 - _sdpa_ref(c, kp, vp, ks, vs)).max() < 1e-6


def test_decode_invalid_pages_masked_and_empty_rows_zero():
    c = cases.make_case(14, 3, 4, 2, 64, [40, 20, 5], act="f32")
    c.block_table[0, 1] = -1
    c.block_table[1, :] = -1
    *_, out32 = cases.oracle_step(c, threads=1)
    assert not out32[1].any()
    # row 0 equals attention over the tokens of its valid pages only
    c2 = cases.make_case(14, 3, 4, 2, 64, [40, 20, 5], act="f32")
    kp, vp, *_ = cases.oracle_step(c2, threads=1)
    toks = [t for t in range(41) if t // 16 != 1]
    pg, sl = c2.block_table[0, np.array(toks) // 16], np.array(toks) % 16
    K = torch.from_numpy(kp[pg, sl].astype(np.float64)).permute(1, 0, 2).repeat_interleave(2, 0).contiguous()
    V = torch.from_numpy(vp[pg, sl].astype(np.float64)).permute(1, 0, 2).repeat_interleave(2, 0).contiguous()
    q = torch.from_numpy(c2.q[0, 0].astype(np.float64))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(q, K, V, scale=1 / 8)[:, 0].numpy()
    assert np.abs(out32[0] - ref).max() < 5e-6


# ---- append ------------------------------------------------------------------------------------------------

def _numpy_append(c: cases.Case, kp, vp):
    """The address formula of src/model/qwen_model.cu:32-42 applied with numpy indexing (16-bit/f32 copy)."""
    for b in range(c.B):
        for t in range(c.S):
            pos = int(c.ctx[b]) + t
            if pos < 0 or pos // 16 >= c.max_blocks:
                continue
            page = c.block_table[b, pos // 16]
            if page < 0 or page >= c.num_blocks:
                continue
            kp[page, pos % 16] = c.k_new[b, t]
            vp[page, pos % 16] = c.v_new[b, t]


@pytest.mark.parametrize("S", [1, 5, 64])
def test_append_matches_address_formula(S):
    c = cases.make_case(20 + S, 4, 8, 4, 128, [0, 15, 16, 200], act="bf16", S=S)
    c.k_pool[:] = 0xA5A5
    c.v_pool[:] = 0xA5A5
    c.block_table[3, 2] = -1                      # a hole: its tokens are skipped
    ek, ev = c.k_pool.copy(), c.v_pool.copy()
    _numpy_append(c, ek, ev)
    kp, vp = c.k_pool.copy(), c.v_pool.copy()
    O.append(c.k_new, c.v_new, c.act, kp, vp, c.kv, c.block_table, c.ctx)
    assert np.array_equal(kp, ek) and np.array_equal(vp, ev)


def test_append_gather_round_trip_and_sentinel():
    c = cases.make_case(30, 3, 8, 2, 64, [3, 40, 17], act="f16", S=33)
    c.k_pool[:] = 0xA5A5
    kp, vp = c.k_pool.copy(), c.v_pool.copy()
    O.append(c.k_new, c.v_new, c.act, kp, vp, c.kv, c.block_table, c.ctx)
    touched = np.zeros(kp.shape[:2], bool)
    for b in range(c.B):
        for t in range(c.S):
            pos = int(c.ctx[b]) + t
            page = c.block_table[b, pos // 16]
            assert np.array_equal(kp[page, pos % 16], c.k_new[b, t])
            touched[page, pos % 16] = True
    assert (kp[~touched] == 0xA5A5).all()


def test_append_context_lens_null_means_zero():
    c = cases.make_case(31, 2, 4, 2, 64, [0, 0], act="f32", S=20)
    a_k, a_v = c.k_pool.copy(), c.v_pool.copy()
    O.append(c.k_new, c.v_new, c.act, a_k, a_v, c.kv, c.block_table, None)
    b_k, b_v = c.k_pool.copy(), c.v_pool.copy()
    O.append(c.k_new, c.v_new, c.act, b_k, b_v, c.kv, c.block_table, np.zeros(2, np.int32))
    assert np.array_equal(a_k, b_k) and np.array_equal(a_v, b_v)


def test_append_narrowing_rounds_like_torch():
    c = cases.make_case(32, 2, 4, 2, 128, [10, 70], act="f32", kv="bf16", S=3)
    kp, vp = c.k_pool.copy(), c.v_pool.copy()
    O.append(c.k_new, c.v_new, c.act, kp, vp, c.kv, c.block_table, c.ctx)
    for b in range(2):
        for t in range(3):
            pos = int(c.ctx[b]) + t
            page = c.block_table[b, pos // 16]
            ref = torch.from_numpy(c.k_new[b, t]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(kp[page, pos % 16], ref)
