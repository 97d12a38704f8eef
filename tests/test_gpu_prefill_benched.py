"""Chunked prefill parity at the shapes the bench times (its C4 prefill and every `prefill_variants` entry).

Each case is 8 rows whose cached contexts are 2048 + U[64, 1024] tokens, a 512-token chunk per row appended by
ffkv_append and then attended by ffkv_paged_prefill (query t of row b sees keys 0 .. ctx[b] + t), over pools
whose first 128 blocks are shared by every row's table (a radix-cache prefix):

- head_dim 128, Hq32/Hkv8, bf16 / f16 / fp8 / int8 caches (q bf16 for the 8-bit caches, as the bench);
- bf16 at head_dim 64 (Hq32/Hkv8) and 256 (Hq16/Hkv4).

8-bit pools hold the append's own quantization of N(0,1) data with 1% of the elements x8 (int8: per-token-per-
head absmax/127 scales; fp8: per-head absmax/448 scales), and the chunk goes through the quantizing append on the
GPU and on the CPU checker alike.  Bar: the pools after the chunk's append are byte-identical over the whole pool,
and the outputs are within max-abs 2e-3 (16-bit caches) or 2e-2 (8-bit) of the float64 closed form
(oracle ffo_paged_prefill_f64), beyond half an output ulp.  At these sizes the launch deals 64 (row, kv head)
groups over the XCDs longest first and each query walks up to about 3.6k keys under the causal limit.
"""

import numpy as np
import pytest

import cases
import gpu_util as gu
import oracle as O
from test_gpu_prefill import _check

pytestmark = pytest.mark.gpu

SHAPES = [  # (name, cache, q, head_dim, Hq, Hkv)
    ("bf16_d128", "bf16", "bf16", 128, 32, 8),
    ("f16_d128", "f16", "f16", 128, 32, 8),
    ("fp8_d128", "fp8", "bf16", 128, 32, 8),
    ("i8_d128", "i8", "bf16", 128, 32, 8),
    ("bf16_d64", "bf16", "bf16", 64, 32, 8),
    ("bf16_d256", "bf16", "bf16", 256, 16, 4),
]


@pytest.mark.parametrize("name,kv,act,D,Hq,Hkv", SHAPES, ids=[s[0] for s in SHAPES])
def test_prefill_at_benched_shape(ff, gpu, name, kv, act, D, Hq, Hkv):
    import torch

    B, S, PRE = 8, 512, 2048
    rng = np.random.default_rng(4)
    ctx = (PRE + rng.integers(64, 1025, size=B)).astype(np.int32)
    eight_bit = kv in ("i8", "fp8")
    c = cases.make_case(4400 + D, B, Hq, Hkv, D, ctx, act=act, kv=kv, S=S, shared_prefix_blocks=PRE // 16,
                        outlier_frac=0.01 if eight_bit else 0.0)
    qn = cases.encode(np.random.default_rng(4401 + D).standard_normal((B, S, Hq, D), dtype=np.float32), c.act)
    print(f"case prefill-benched {name} B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} kv={kv} q={act} N={c.num_blocks} "
          f"ctx={list(ctx)}", flush=True)

    dev = gpu
    kp = gu.to_dev(c.k_pool, c.kv, dev)
    vp = gu.to_dev(c.v_pool, c.kv, dev)
    ks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(dev)
    vs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(dev)
    bt = torch.from_numpy(c.block_table).to(dev)
    cx = torch.from_numpy(c.ctx).to(dev)
    ff.append_kv_cache(gu.to_dev(c.k_new, c.act, dev), gu.to_dev(c.v_new, c.act, dev), kp, vp, bt, cx, ks, vs)
    out = ff.paged_prefill(gu.to_dev(qn, c.act, dev), kp, vp, bt, cx, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()

    rk, rv = c.k_pool.copy(), c.v_pool.copy()
    rks = None if c.k_scale is None else c.k_scale.copy()
    rvs = None if c.v_scale is None else c.v_scale.copy()
    O.append(c.k_new, c.v_new, c.act, rk, rv, c.kv, c.block_table, c.ctx, rks, rvs)
    as_bytes = lambda t: t.view(torch.uint8).cpu().numpy()  # noqa: E731
    assert np.array_equal(as_bytes(kp), rk.view(np.uint8)), "K pages differ after the chunk append"
    assert np.array_equal(as_bytes(vp), rv.view(np.uint8)), "V pages differ after the chunk append"
    if kv == "i8":
        assert np.array_equal(ks.cpu().numpy().view(np.uint32), rks.view(np.uint32)), "K scales differ"
        assert np.array_equal(vs.cpu().numpy().view(np.uint32), rvs.view(np.uint32)), "V scales differ"

    ref = O.paged_prefill_f64(qn, c.act, rk, rv, c.kv, c.block_table, c.ctx, rks, rvs)
    got = out.float().cpu().numpy().reshape(ref.shape)
    _check(got, ref, c.act, 2e-2 if eight_bit else 2e-3)
