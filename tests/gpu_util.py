"""Helpers that run a Case through the HIP library (torch only allocates device memory and copies)."""

from __future__ import annotations

import numpy as np
import torch

import oracle as O

_TORCH_STORAGE = {O.DTYPE_F32: torch.float32, O.DTYPE_F16: torch.float16, O.DTYPE_BF16: torch.bfloat16,
                  O.DTYPE_I8: torch.int8, O.DTYPE_FP8: torch.uint8}


def to_dev(a: np.ndarray | None, dt: int | None, dev):
    """Upload a storage array; 16-bit payloads are reinterpreted as the torch float type of `dt`."""
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    if dt in (O.DTYPE_F16, O.DTYPE_BF16):
        t = t.view(_TORCH_STORAGE[dt])
    return t


def to_host(t: torch.Tensor, storage_dtype) -> np.ndarray:
    if t.dtype in (torch.float16, torch.bfloat16):
        t = t.view(torch.int16)
    return t.cpu().numpy().view(storage_dtype)


def run_step(ff, c, dev, max_context_len: int = 0, workspace=False):
    """Append c's new tokens then decode, on the GPU.  Returns host arrays like cases.oracle_step."""
    kp = to_dev(c.k_pool, c.kv, dev)
    vp = to_dev(c.v_pool, c.kv, dev)
    ks = None if c.k_scale is None else torch.from_numpy(c.k_scale.copy()).to(dev)
    vs = None if c.v_scale is None else torch.from_numpy(c.v_scale.copy()).to(dev)
    bt = torch.from_numpy(c.block_table).to(dev)
    ctx = torch.from_numpy(c.ctx).to(dev)
    kn = to_dev(c.k_new, c.act, dev)
    vn = to_dev(c.v_new, c.act, dev)
    q = to_dev(c.q, c.act, dev)
    ff.append_kv_cache(kn, vn, kp, vp, bt, ctx, ks, vs)
    ws = None
    if workspace:
        ws = ff.decode_workspace(c.B, c.Hq, c.D, c.max_blocks, max_context_len, device=dev)
    out = ff.paged_attention(q, kp, vp, bt, ctx, k_scale=ks, v_scale=vs, max_context_len=max_context_len,
                             workspace=ws)
    torch.cuda.synchronize()
    st = kp.dtype
    pool_np = np.int16 if st in (torch.float16, torch.bfloat16) else None
    conv = (lambda t: to_host(t, np.uint16)) if pool_np else (lambda t: t.cpu().numpy())
    out_np = to_host(out, np.uint16) if out.dtype in (torch.float16, torch.bfloat16) else out.cpu().numpy()
    return (conv(kp), conv(vp), None if ks is None else ks.cpu().numpy(), None if vs is None else vs.cpu().numpy(),
            out_np.reshape(c.B, -1))


def out_to_f32(out_storage: np.ndarray, act: int) -> np.ndarray:
    if act == O.DTYPE_F32:
        return out_storage.astype(np.float32)
    return O.bf16_to_f32(out_storage) if act == O.DTYPE_BF16 else O.f16_to_f32(out_storage)
