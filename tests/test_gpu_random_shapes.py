"""Seeded random shapes for the decode (with its append), the decode over a shared prefix and the chunked prefill,
against the CPU checker, to the same bar as the fixed-shape parity tests: pages bit-exact, outputs within 2e-3
(16-bit caches) / 2e-2 (8-bit caches) / 1e-4 (fp32 decode) of the checker beyond the output's own rounding.  Each case
draws the batch, the GQA group (1 .. 40 query heads per KV head), the KV heads, head_dim, the row lengths (empty
rows included), the chunk length and the dtype pair from a fixed seed, so a failure names a reproducible case."""

import math

import numpy as np
import pytest

import cases
from test_gpu_parity import TOL, _check as _decode_check
from test_gpu_prefill import _case as _prefill_case, _check as _prefill_check, _run as _prefill_run

pytestmark = pytest.mark.gpu

DECODE_PAIRS = [("bf16", "bf16"), ("f16", "f16"), ("f32", "f32"), ("bf16", "i8"), ("bf16", "fp8"), ("f32", "bf16"),
                ("f16", "i8"), ("f32", "fp8")]
PREFILL_PAIRS = [("bf16", "bf16"), ("f16", "f16"), ("bf16", "i8"), ("bf16", "fp8"), ("f32", "bf16")]
GROUPS = [1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 24, 40]


@pytest.mark.parametrize("seed", range(12))
def test_random_decode(ff, gpu, seed):
    rng = np.random.default_rng(9000 + seed)
    act, kv = DECODE_PAIRS[seed % len(DECODE_PAIRS)]
    G = int(rng.choice(GROUPS if kv != "f32" else [g for g in GROUPS if g <= 16]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 128, 256]))
    B = int(rng.integers(1, 41))
    ctx = rng.integers(0, 2000, size=B)
    ctx[rng.random(B) < 0.1] = 0  # some rows hold only the new token
    c = cases.make_case(9000 + seed, B, G * Hkv, Hkv, D, ctx, act=act, kv=kv, input_scale=1 / math.sqrt(D))
    cap = int(rng.integers(64, 2000)) if seed % 4 == 3 else 0  # max_context_len cuts some rows
    _decode_check(ff, gpu, c, TOL[(act, kv)], max_context_len=cap)


@pytest.mark.parametrize("seed", range(10))
def test_random_prefill(ff, gpu, seed):
    rng = np.random.default_rng(9500 + seed)
    act, kv = PREFILL_PAIRS[seed % len(PREFILL_PAIRS)]
    G = int(rng.choice(GROUPS))
    Hkv = int(rng.choice([h for h in (1, 2, 4) if G * h <= 48]))
    D = int(rng.choice([64, 128, 256]))
    B = int(rng.integers(1, 4))
    S = int(rng.integers(1, 300))
    ctx = rng.integers(0, 1500, size=B)
    # keep the single-threaded float64 checker to the size of the fixed long-chunk case (about 1.5e10 flops)
    while S > 1 and B * S * G * Hkv * (int(ctx.max()) + S) * D * 4 > 1.5e10:
        S //= 2
    c, qn = _prefill_case(9500 + seed, B, G * Hkv, Hkv, D, ctx, S, act=act, kv=kv)
    _prefill_check(*_prefill_run(ff, gpu, c, qn), c.act, 2e-3 if kv in ("bf16", "f16") else 2e-2)


@pytest.mark.parametrize("seed", range(6))
def test_random_decode_head_dims(ff, gpu, seed):
    """head_dim drawn from the multiples of 8 up to 128 (the vector decode's range besides 64 and 128), groups up
    to 16 query heads per KV head."""
    rng = np.random.default_rng(9800 + seed)
    act, kv = DECODE_PAIRS[(seed * 3) % len(DECODE_PAIRS)]
    D = 8 * int(rng.integers(1, 17))
    G = int(rng.choice([g for g in GROUPS if g <= 16]))
    Hkv = int(rng.choice([1, 2, 4]))
    B = int(rng.integers(1, 25))
    ctx = rng.integers(0, 1200, size=B)
    ctx[rng.random(B) < 0.1] = 0
    c = cases.make_case(9800 + seed, B, G * Hkv, Hkv, D, ctx, act=act, kv=kv, input_scale=1 / math.sqrt(D))
    _decode_check(ff, gpu, c, TOL[(act, kv)])


SHARED_PAIRS = [("bf16", "bf16"), ("f16", "f16"), ("f32", "bf16"), ("bf16", "bf16"), ("bf16", "i8"), ("f16", "fp8")]


@pytest.mark.parametrize("seed", range(8))
def test_random_shared_prefix(ff, gpu, seed):
    """ffkv_paged_decode_shared_prefix on seeded shapes, against the checker and the plain decode: mostly 16-bit
    pages at head_dim 128 with KV-head counts that are multiples of 4 (the prefix partials inside the decode's
    grid; enough private pages for its weighted page split in most cases), the 8-bit pairs on the two-launch path.
    Some rows end exactly at the prefix."""
    from test_gpu_shared_prefix import _both

    rng = np.random.default_rng(9900 + seed)
    act, kv = SHARED_PAIRS[seed % len(SHARED_PAIRS)]
    G = int(rng.choice([g for g in GROUPS if g <= 16]))
    Hkv = int(rng.choice([4, 8, 12]))
    B = int(rng.integers(4, 49))
    shared = int(rng.integers(1, 161))
    ctx = shared * 16 + rng.integers(0, 601, size=B) - 1  # ctx + 1 tokens after the step's append
    ctx[rng.random(B) < 0.1] = shared * 16 - 1  # the row ends at the prefix's end
    c = cases.make_case(9900 + seed, B, G * Hkv, Hkv, 128, ctx, act=act, kv=kv, shared_prefix_blocks=shared,
                        input_scale=1 / math.sqrt(128))
    _both(ff, gpu, c, shared, tol=2e-3 if kv in ("bf16", "f16") else 2e-2)
