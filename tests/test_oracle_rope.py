"""Pins of the CPU restatement of the rotary embedding (oracle ffo_rope, restating src/kernels/rope.cu:22-137).

Each check can fail for a plausible mistake: torch's rotate_half formulation (q*cos + rotate_half(q)*sin,
evaluated with torch's own fp32 ops) catches swapped halves, a wrong sign or a wrong frequency exponent; the
unit-vector case pins which output dim receives cos and which sin; position 0 must be the identity; the pair
norm must be preserved; and q.k after rotation must depend only on the position offset.
"""

import numpy as np
import pytest
import torch

import oracle as O

THETA = 1e6


def torch_rope_f32(x: np.ndarray, pos: np.ndarray, theta: float) -> np.ndarray:
    """HF-style rotate_half RoPE on [B, S, H, D] float32, with the inv_freq / cos / sin precision include/ffkv.h
    specifies (double, rounded once to float) and torch fp32 ops for the angle and the rotation."""
    B, S, H, D = x.shape
    i = np.arange(D // 2, dtype=np.float64)
    inv_freq = torch.from_numpy((theta ** (-2.0 * i / D)).astype(np.float32))        # float(theta^(-2i/D))
    p = torch.from_numpy(pos.astype(np.float32))                                      # [B, S]
    ang = p[..., None] * inv_freq                                                     # fp32 product
    cos = torch.cos(ang.double()).float()
    sin = torch.sin(ang.double()).float()
    emb_c = torch.cat([cos, cos], dim=-1)[:, :, None, :]
    emb_s = torch.cat([sin, sin], dim=-1)[:, :, None, :]
    t = torch.from_numpy(x)
    x1, x2 = t[..., : D // 2], t[..., D // 2:]
    rot = torch.cat([-x2, x1], dim=-1)
    return (t * emb_c + rot * emb_s).numpy()


def positions(ctx, B, S):
    base = np.zeros(B, np.int64) if ctx is None else ctx.astype(np.int64)
    return base[:, None] + np.arange(S)[None, :]


@pytest.mark.parametrize("D", [64, 128, 256])
def test_rope_matches_torch_rotate_half_bit_exact(D):
    rng = np.random.default_rng(D)
    x = rng.standard_normal((3, 5, 4, D)).astype(np.float32)
    ctx = np.array([0, 17, 32000], np.int32)
    got = O.rope(x, O.DTYPE_F32, ctx, THETA)
    want = torch_rope_f32(x, positions(ctx, 3, 5), THETA)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_rope_16bit_is_the_rounded_fp32_result(dt):
    rng = np.random.default_rng(3)
    x32 = rng.standard_normal((2, 4, 3, 128)).astype(np.float32)
    if dt == "bf16":
        code, enc, dec = O.DTYPE_BF16, O.f32_to_bf16, O.bf16_to_f32
    else:
        code, enc, dec = O.DTYPE_F16, O.f32_to_f16, O.f16_to_f32
    xs = enc(x32)
    ctx = np.array([5, 4095], np.int32)
    got = O.rope(xs, code, ctx, THETA)
    want = enc(torch_rope_f32(dec(xs), positions(ctx, 2, 4), THETA))
    np.testing.assert_array_equal(got, want)


def test_rope_position_zero_is_identity_and_null_ctx_means_zero():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 1, 3, 128)).astype(np.float32)
    np.testing.assert_array_equal(O.rope(x, O.DTYPE_F32, np.zeros(2, np.int32), THETA), x)
    np.testing.assert_array_equal(O.rope(x, O.DTYPE_F32, None, THETA), x)


def test_rope_unit_vectors_give_cos_and_sin():
    D, p = 128, 1234
    x = np.zeros((1, 1, D // 2, D), np.float32)
    for i in range(D // 2):
        x[0, 0, i, i] = 1.0                      # head i holds e_i
    y = O.rope(x, O.DTYPE_F32, np.array([p], np.int32), THETA)[0, 0]
    for i in range(D // 2):
        ang = np.float32(p) * np.float32(THETA ** (-2.0 * i / D))
        assert y[i, i] == np.float32(np.cos(np.float64(ang)))
        assert y[i, i + D // 2] == np.float32(np.sin(np.float64(ang)))
        others = np.delete(y[i], [i, i + D // 2])
        assert not others.any()


def test_rope_preserves_pair_norms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 6, 4, 128)).astype(np.float32)
    y = O.rope(x, O.DTYPE_F32, np.array([100, 20000], np.int32), THETA)
    n0 = x[..., :64].astype(np.float64) ** 2 + x[..., 64:].astype(np.float64) ** 2
    n1 = y[..., :64].astype(np.float64) ** 2 + y[..., 64:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-6, atol=1e-9)


def test_rope_scores_depend_only_on_offset():
    rng = np.random.default_rng(6)
    D = 128
    q = rng.standard_normal((1, 1, 1, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, 1, D)).astype(np.float32)

    def score(m, n):
        qm = O.rope(q, O.DTYPE_F32, np.array([m], np.int32), 10000.0)
        kn = O.rope(k, O.DTYPE_F32, np.array([n], np.int32), 10000.0)
        return float(np.dot(qm.ravel().astype(np.float64), kn.ravel().astype(np.float64)))

    for m, n, d in [(7, 3, 100), (50, 60, 900), (0, 5, 2000)]:
        assert abs(score(m, n) - score(m + d, n + d)) < 2e-3 * (1 + abs(score(m, n)))
    # ... and the offset does matter
    assert abs(score(7, 3) - score(7, 4)) > 1e-3


def test_rope_detects_planted_mistakes():
    """The torch formulation above distinguishes the oracle from plausible wrong variants."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, 3, 2, 64)).astype(np.float32)
    ctx = np.array([9], np.int32)
    want = torch_rope_f32(x, positions(ctx, 1, 3), THETA)
    # interleaved pairs (2i, 2i+1) instead of (i, i + D/2)
    xi = x.reshape(1, 3, 2, 32, 2).transpose(0, 1, 2, 4, 3).reshape(1, 3, 2, 64)
    inter = O.rope(xi, O.DTYPE_F32, ctx, THETA).reshape(1, 3, 2, 2, 32).transpose(0, 1, 2, 4, 3).reshape(1, 3, 2, 64)
    assert not np.allclose(inter, want, atol=1e-3)
    # opposite rotation direction (negated positions)
    assert not np.allclose(O.rope(x, O.DTYPE_F32, -ctx - 0, THETA)[:, 1:], want[:, 1:], atol=1e-3)
    # wrong base
    assert not np.allclose(O.rope(x, O.DTYPE_F32, ctx, 10000.0), want, atol=1e-3)
