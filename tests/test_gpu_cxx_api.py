"""The firefly:: C++ drop-in API (include/firefly/kernels.h, tensor.h) on the GPU, called the way the
reference's model calls its operators: Tensor::from_external views over device buffers, kernels::append_kv_cache
then kernels::attention with the block table and context_lens device pointers (tests/cpp/kernels_api_shim.cpp).
Same bar as the C-ABI parity tests: pages bit-exact, outputs within tolerance of the CPU checker."""

import ctypes
import math
import os
from pathlib import Path

import numpy as np
import pytest

import cases
import oracle as O

SHIM = Path(__file__).resolve().parent / "cpp" / "libkernels_api_shim.so"


def _excess_bf16(got, ref):
    """Max-abs error beyond half a bf16 ulp at the value (the output's own rounding)."""
    m = np.maximum(np.abs(got), np.abs(ref))
    half = 2.0 ** (np.floor(np.log2(np.maximum(m, 2.0 ** -126))) - 8)
    return float((np.abs(got.astype(np.float64) - ref) - half).max())


@pytest.fixture(scope="module")
def shim(ff):
    if not SHIM.exists():
        pytest.skip("tests/cpp/libkernels_api_shim.so not built")
    lib = ctypes.CDLL(str(SHIM), mode=os.RTLD_NOW)
    vp, i = ctypes.c_void_p, ctypes.c_int
    lib.kas_append_then_decode.restype = i
    lib.kas_append_then_decode.argtypes = [vp] * 7 + [i, vp, vp, vp] + [i] * 9 + [vp]
    lib.kas_rope_append.restype = i
    lib.kas_rope_append.argtypes = [vp] * 7 + [vp, vp] + [i] * 9 + [ctypes.c_float, i, vp]
    lib.kas_last_error.restype = ctypes.c_char_p
    lib.kas_contiguous_prefill.restype = i
    lib.kas_contiguous_prefill.argtypes = [vp] * 4 + [i] * 6 + [vp]
    lib.kas_paged_prefill.restype = i
    lib.kas_paged_prefill.argtypes = [vp] * 8 + [i] * 9 + [vp]
    lib.kas_decode_shared_prefix.restype = i
    lib.kas_decode_shared_prefix.argtypes = [vp] * 6 + [i] * 9 + [vp]
    lib.kas_append_attention.restype = i
    lib.kas_append_attention.argtypes = [vp, vp, i] + [vp] * 6 + [i] * 8 + [vp]
    lib.kas_release_workspace.restype = i
    lib.kas_release_workspace.argtypes = [vp]
    return lib


def test_shim_links_against_exported_cxx_api(shim):
    """Loading with RTLD_NOW resolves every firefly:: symbol the shim uses from libffkv.so."""
    assert shim.kas_last_error() == b""


@pytest.mark.gpu
@pytest.mark.parametrize("act,kv,tol", [("bf16", "bf16", 2e-3), ("f16", "f16", 2e-3), ("bf16", "i8", 2e-2),
                                        ("f32", "fp8", 2e-2), ("f32", "f32", 1e-4)])
def test_cxx_api_append_then_decode(shim, gpu, act, kv, tol):
    import torch

    import gpu_util as gu

    c = cases.config1(act=act, kv=kv)
    kp, vp, ks, vs, _, out32 = cases.oracle_step(c)
    dk, dv = gu.to_dev(c.k_pool, c.kv, gpu), gu.to_dev(c.v_pool, c.kv, gpu)
    dks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(gpu)
    dvs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(gpu)
    q, kn, vn = gu.to_dev(c.q, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
    bt, ctx = torch.from_numpy(c.block_table).to(gpu), torch.from_numpy(c.ctx).to(gpu)
    out = torch.empty((c.B, 1, c.Hq * c.D), dtype=q.dtype, device=gpu)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = shim.kas_append_then_decode(p(q), p(kn), p(vn), p(dk), p(dv), p(dks), p(dvs), 0, p(out), p(bt), p(ctx),
                                     c.B, c.S, c.Hq, c.Hkv, c.D, c.num_blocks, c.max_blocks, c.act, c.kv,
                                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, shim.kas_last_error()
    conv = (lambda t: gu.to_host(t, np.uint16)) if dk.dtype in (torch.float16, torch.bfloat16) else \
        (lambda t: t.cpu().numpy())
    assert np.array_equal(conv(dk).view(np.uint8), kp.view(np.uint8))
    assert np.array_equal(conv(dv).view(np.uint8), vp.view(np.uint8))
    if c.kv == O.DTYPE_I8:
        assert np.array_equal(dks.cpu().numpy().view(np.uint32), ks.view(np.uint32))
    got = out.float().cpu().numpy().reshape(out32.shape)
    assert np.abs(got - out32).max() <= tol + (0 if c.act == O.DTYPE_F32 else 2.0 ** -9)


@pytest.mark.gpu
def test_cxx_api_release_workspace_between_calls(shim, gpu):
    """kernels::release_workspace frees a stream's decode workspace: decodes on a fresh stream before and after a
    release (which allocates a new one) and on a stream never used (a no-op release) give the same bytes."""
    import torch

    import gpu_util as gu

    c = cases.make_case(33, 8, 32, 8, 128, [900, 20, 4000, 1, 77, 300, 2500, 64])
    outs = []
    side = torch.cuda.Stream(device=gpu)
    for release in (False, True, True):
        dk, dv = gu.to_dev(c.k_pool, c.kv, gpu), gu.to_dev(c.v_pool, c.kv, gpu)
        q, kn, vn = gu.to_dev(c.q, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
        bt, ctx = torch.from_numpy(c.block_table).to(gpu), torch.from_numpy(c.ctx).to(gpu)
        out = torch.empty((c.B, 1, c.Hq * c.D), dtype=q.dtype, device=gpu)
        torch.cuda.synchronize()
        rc = shim.kas_append_then_decode(q.data_ptr(), kn.data_ptr(), vn.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                         None, None, 0, out.data_ptr(), bt.data_ptr(), ctx.data_ptr(), c.B, c.S,
                                         c.Hq, c.Hkv, c.D, c.num_blocks, c.max_blocks, c.act, c.kv, side.cuda_stream)
        assert rc == 0, shim.kas_last_error()
        if release:
            assert shim.kas_release_workspace(side.cuda_stream) == 0, shim.kas_last_error()
            assert shim.kas_release_workspace(side.cuda_stream) == 0  # nothing left to release
        torch.cuda.synchronize()
        outs.append(gu.to_host(out, np.uint16))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    _, _, _, _, _, out32 = cases.oracle_step(c)
    got = gu.out_to_f32(outs[0], c.act).reshape(out32.shape)
    assert _excess_bf16(got, out32) <= 2e-3


@pytest.mark.gpu
def test_cxx_api_contiguous_prefill_branch(shim, gpu):
    """kernels::attention with a null block table: the reference's causal prefill over the chunk's K/V."""
    import torch

    import gpu_util as gu

    rng = np.random.default_rng(90)
    B, S, Hq, Hkv, D = 2, 45, 16, 4, 128
    q, k, v = (cases.encode(rng.standard_normal(s, dtype=np.float32), O.DTYPE_BF16)
               for s in [(B, S, Hq, D), (B, S, Hkv, D), (B, S, Hkv, D)])
    dq, dk, dv = (gu.to_dev(a, O.DTYPE_BF16, gpu) for a in (q, k, v))
    out = torch.empty((B, S, Hq * D), dtype=torch.bfloat16, device=gpu)
    rc = shim.kas_contiguous_prefill(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), B, S, Hq, Hkv, D,
                                     O.DTYPE_BF16, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, shim.kas_last_error()
    ref = O.paged_prefill_f64(q, O.DTYPE_BF16, k, v, O.DTYPE_BF16, None, None)
    got = out.float().cpu().numpy().reshape(ref.shape)
    assert _excess_bf16(got, ref) <= 2e-3


@pytest.mark.gpu
def test_cxx_api_chunked_prefill_over_cached_prefix(shim, gpu):
    """kernels::append_kv_cache then kernels::attention with a block table and a multi-token q."""
    import torch

    import gpu_util as gu

    c = cases.make_case(91, 3, 16, 4, 128, [0, 40, 130], act="bf16", S=20)
    rng = np.random.default_rng(92)
    qn = cases.encode(rng.standard_normal((c.B, c.S, c.Hq, c.D), dtype=np.float32), c.act)
    dq, kn, vn = gu.to_dev(qn, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
    dk, dv = gu.to_dev(c.k_pool, c.kv, gpu), gu.to_dev(c.v_pool, c.kv, gpu)
    bt, ctx = torch.from_numpy(c.block_table).to(gpu), torch.from_numpy(c.ctx).to(gpu)
    out = torch.empty((c.B, c.S, c.Hq * c.D), dtype=dq.dtype, device=gpu)
    rc = shim.kas_paged_prefill(dq.data_ptr(), kn.data_ptr(), vn.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                out.data_ptr(), bt.data_ptr(), ctx.data_ptr(), c.B, c.S, c.Hq, c.Hkv, c.D,
                                c.num_blocks, c.max_blocks, c.act, c.kv, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, shim.kas_last_error()
    rk, rv = c.k_pool.copy(), c.v_pool.copy()
    O.append(c.k_new, c.v_new, c.act, rk, rv, c.kv, c.block_table, c.ctx)
    ref = O.paged_prefill_f64(qn, c.act, rk, rv, c.kv, c.block_table, c.ctx)
    got = out.float().cpu().numpy().reshape(ref.shape)
    assert _excess_bf16(got, ref) <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("act,kv", [("bf16", "bf16"), ("f16", "i8"), ("bf16", "fp8")])
@pytest.mark.parametrize("fused", [1, 0])
def test_cxx_api_rope_then_append(shim, gpu, act, kv, fused):
    """kernels::rope_append_kv_cache and kernels::apply_rope + kernels::append_kv_cache: rotated q/k and pages
    bit-identical to the checker (rope, then append of the rotated k)."""
    import torch

    import gpu_util as gu

    theta = 1e6
    c = cases.make_case(80, 3, 8, 2, 128, [0, 40, 777], act=act, kv=kv, S=5)
    rng = np.random.default_rng(81)
    qn = cases.encode(rng.standard_normal((c.B, c.S, c.Hq, c.D), dtype=np.float32), c.act)
    q, kn, vn = gu.to_dev(qn, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
    dk, dv = gu.to_dev(c.k_pool, c.kv, gpu), gu.to_dev(c.v_pool, c.kv, gpu)
    dks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(gpu)
    dvs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(gpu)
    bt, ctx = torch.from_numpy(c.block_table).to(gpu), torch.from_numpy(c.ctx).to(gpu)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = shim.kas_rope_append(p(q), p(kn), p(vn), p(dk), p(dv), p(dks), p(dvs), p(bt), p(ctx), c.B, c.S, c.Hq,
                              c.Hkv, c.D, c.num_blocks, c.max_blocks, c.act, c.kv, theta, fused,
                              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, shim.kas_last_error()
    q_ref, k_ref = O.rope(qn, c.act, c.ctx, theta), O.rope(c.k_new, c.act, c.ctx, theta)
    host = (lambda t: gu.to_host(t, np.uint16)) if q.dtype in (torch.float16, torch.bfloat16) else \
        (lambda t: t.cpu().numpy())
    assert np.array_equal(host(q), q_ref) and np.array_equal(host(kn), k_ref)
    rk, rv = c.k_pool.copy(), c.v_pool.copy()
    rks = None if c.k_scale is None else c.k_scale.copy()
    rvs = None if c.v_scale is None else c.v_scale.copy()
    O.append(k_ref, c.v_new, c.act, rk, rv, c.kv, c.block_table, c.ctx, rks, rvs)
    conv = (lambda t: gu.to_host(t, np.uint16)) if dk.dtype in (torch.float16, torch.bfloat16) else \
        (lambda t: t.cpu().numpy())
    assert np.array_equal(conv(dk).view(np.uint8), rk.view(np.uint8))
    assert np.array_equal(conv(dv).view(np.uint8), rv.view(np.uint8))
    if c.kv == O.DTYPE_I8:
        assert np.array_equal(dks.cpu().numpy().view(np.uint32), rks.view(np.uint32))


@pytest.mark.gpu
def test_cxx_api_decode_shared_prefix(shim, gpu):
    """kernels::attention_shared_prefix on 24 rows over a 32-page shared prefix, against the CPU checker."""
    import torch

    import gpu_util as gu

    rng = np.random.default_rng(60)
    ctx = 512 + rng.integers(0, 400, size=24)
    c = cases.make_case(60, 24, 32, 8, 128, ctx, act="bf16", shared_prefix_blocks=32)
    kp, vp, _, _, _, out32 = cases.oracle_step(c)
    dk, dv = gu.to_dev(kp, c.kv, gpu), gu.to_dev(vp, c.kv, gpu)
    q = gu.to_dev(c.q, c.act, gpu)
    bt, cx = torch.from_numpy(c.block_table).to(gpu), torch.from_numpy(c.ctx).to(gpu)
    out = torch.empty((c.B, 1, c.Hq * c.D), dtype=q.dtype, device=gpu)
    rc = shim.kas_decode_shared_prefix(q.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), bt.data_ptr(),
                                       cx.data_ptr(), c.B, c.Hq, c.Hkv, c.D, c.num_blocks, c.max_blocks, c.act, c.kv,
                                       32, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, shim.kas_last_error()
    got = out.float().cpu().numpy().reshape(out32.shape)
    assert _excess_bf16(got, out32) <= 2e-3


@pytest.mark.gpu
@pytest.mark.parametrize("act,kv", [("bf16", "bf16"), ("f16", "f16"), ("f32", "bf16")])
def test_cxx_api_append_kv_cache_attention(shim, gpu, act, kv):
    """kernels::append_kv_cache_attention (the decode step in one call; one launch when k / v have the cache's
    dtype, append then decode otherwise): pages bit-exact with the CPU checker's append, output within 2e-3."""
    import torch

    import gpu_util as gu

    rng = np.random.default_rng(61)
    ctx = rng.integers(0, 900, size=20)
    c = cases.make_case(61, 20, 32, 8, 128, ctx, act=act, kv=kv)
    kp, vp, _, _, _, out32 = cases.oracle_step(c)
    dk, dv = gu.to_dev(c.k_pool, c.kv, gpu), gu.to_dev(c.v_pool, c.kv, gpu)
    q, kn, vn = gu.to_dev(c.q, c.act, gpu), gu.to_dev(c.k_new, c.act, gpu), gu.to_dev(c.v_new, c.act, gpu)
    bt, cx = torch.from_numpy(c.block_table).to(gpu), torch.from_numpy(c.ctx).to(gpu)
    out = torch.empty((c.B, 1, c.Hq * c.D), dtype=q.dtype, device=gpu)
    rc = shim.kas_append_attention(kn.data_ptr(), vn.data_ptr(), c.act, q.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                   out.data_ptr(), bt.data_ptr(), cx.data_ptr(), c.B, c.Hq, c.Hkv, c.D, c.num_blocks,
                                   c.max_blocks, c.act, c.kv, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, shim.kas_last_error()
    assert np.array_equal(gu.to_host(dk, np.uint16).view(np.uint8), kp.view(np.uint8))
    assert np.array_equal(gu.to_host(dv, np.uint16).view(np.uint8), vp.view(np.uint8))
    from test_gpu_parity import half_ulp

    got = out.float().cpu().numpy().reshape(out32.shape)
    diff = np.abs(got.astype(np.float64) - out32)
    assert float((diff - half_ulp(np.maximum(np.abs(got), np.abs(out32)), c.act)).max()) <= 2e-3
