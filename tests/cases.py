"""Deterministic synthetic inputs for the paged KV-cache path (numpy, seeded).

A Case holds a page pool [N, 16, Hkv, D] in its storage dtype, per-sequence block tables drawn from a seeded
permutation of the pool, pre-append context lengths, the new K/V tokens to append and the decode queries -
the shapes of the benchmark configurations (block size 16, ``context_lens`` = tokens cached before the append).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

import oracle as O

BLOCK = 16
STORAGE = {O.DTYPE_F32: np.float32, O.DTYPE_F16: np.uint16, O.DTYPE_BF16: np.uint16, O.DTYPE_I8: np.int8,
           O.DTYPE_FP8: np.uint8}
NAMES = {"f32": O.DTYPE_F32, "f16": O.DTYPE_F16, "bf16": O.DTYPE_BF16, "i8": O.DTYPE_I8, "fp8": O.DTYPE_FP8}


def encode(x: np.ndarray, dt: int) -> np.ndarray:
    """float32 -> storage of an activation dtype (round to nearest even)."""
    x = np.ascontiguousarray(x, np.float32)
    if dt == O.DTYPE_F32:
        return x
    if dt == O.DTYPE_F16:
        return O.f32_to_f16(x)
    if dt == O.DTYPE_BF16:
        return O.f32_to_bf16(x)
    raise ValueError(dt)


def decode(a: np.ndarray, dt: int) -> np.ndarray:
    if dt == O.DTYPE_F32:
        return a.astype(np.float32)
    if dt == O.DTYPE_F16:
        return O.f16_to_f32(a)
    if dt == O.DTYPE_BF16:
        return O.bf16_to_f32(a)
    raise ValueError(dt)


@dataclass
class Case:
    B: int
    Hq: int
    Hkv: int
    D: int
    ctx: np.ndarray            # int32 [B], tokens cached before the append
    block_table: np.ndarray    # int32 [B, max_blocks], -1 padded
    num_blocks: int
    act: int                   # dtype code of q / out / new k,v
    kv: int                    # dtype code of the pool
    k_pool: np.ndarray
    v_pool: np.ndarray
    k_scale: np.ndarray | None
    v_scale: np.ndarray | None
    k_new: np.ndarray          # storage [B, S, Hkv, D]
    v_new: np.ndarray
    q: np.ndarray              # storage [B, 1, Hq, D]
    seed: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def max_blocks(self) -> int:
        return self.block_table.shape[1]

    @property
    def S(self) -> int:
        return self.k_new.shape[1]


def _quantize_pool(xf: np.ndarray, kv: int, head_scale: np.ndarray | None):
    """Quantize a float32 pool [N,16,Hkv,D] the way append would."""
    N, _, Hkv, D = xf.shape
    if kv == O.DTYPE_I8:
        rows = xf.reshape(-1, D)
        amax = np.max(np.abs(rows), axis=1).astype(np.float32)
        s = (amax / np.float32(127.0)).astype(np.float32)
        safe = np.where(s == 0, np.float32(1), s)
        q = np.clip(np.rint(rows / safe[:, None]), -127, 127).astype(np.int8)
        q[s == 0] = 0
        return q.reshape(xf.shape), s.reshape(N, BLOCK, Hkv)
    if kv == O.DTYPE_FP8:
        return O.f32_to_e4m3(xf / head_scale[None, None, :, None]), head_scale
    return encode(xf, kv), None


def make_case(seed: int, B: int, Hq: int, Hkv: int, D: int, ctx, act="bf16", kv=None, S: int = 1,
              input_scale: float = 1.0, pool_extra: float = 0.1, max_blocks: int | None = None,
              outlier_frac: float = 0.0, outlier_mul: float = 8.0, shared_prefix_blocks: int = 0,
              fp8_scale_margin: float = 1.0) -> Case:
    """Build a case.  ``ctx`` are pre-append context lengths; each row gets blocks for ctx + S tokens.

    shared_prefix_blocks > 0 makes the first that many logical blocks of every row map to the same physical
    blocks (radix-tree prefix sharing)."""
    rng = np.random.default_rng(seed)
    act_dt = NAMES[act]
    kv_dt = NAMES[kv or act]
    ctx = np.asarray(ctx, dtype=np.int32)
    need = [math.ceil((int(c) + S) / BLOCK) for c in ctx]
    shared = shared_prefix_blocks
    private = [max(0, n - shared) for n in need]
    total = shared + sum(private)
    N = max(1, math.ceil(total * (1.0 + pool_extra)))
    perm = rng.permutation(N).astype(np.int32)
    mb = max(need) if max_blocks is None else max_blocks
    table = np.full((B, mb), -1, dtype=np.int32)
    pos = shared
    for b in range(B):
        table[b, :min(shared, need[b])] = perm[:min(shared, need[b])]
        table[b, shared:need[b]] = perm[pos:pos + private[b]]
        pos += private[b]

    def gauss(shape):
        x = rng.standard_normal(shape, dtype=np.float32) * np.float32(input_scale)
        if outlier_frac > 0:
            m = rng.random(shape) < outlier_frac
            x[m] *= np.float32(outlier_mul)
        return x

    kf = gauss((N, BLOCK, Hkv, D))
    vf = gauss((N, BLOCK, Hkv, D))
    k_new = gauss((B, S, Hkv, D))
    v_new = gauss((B, S, Hkv, D))
    qf = gauss((B, 1, Hq, D))

    hk = hv = None
    if kv_dt == O.DTYPE_FP8:
        # per-head scale from the absmax of everything that will live in the cache
        hk = (np.maximum(np.abs(kf).max(axis=(0, 1, 3)), np.abs(k_new).max(axis=(0, 1, 3))) / 448.0
              * fp8_scale_margin).astype(np.float32)
        hv = (np.maximum(np.abs(vf).max(axis=(0, 1, 3)), np.abs(v_new).max(axis=(0, 1, 3))) / 448.0
              * fp8_scale_margin).astype(np.float32)
    k_pool, k_scale = _quantize_pool(kf, kv_dt, hk)
    v_pool, v_scale = _quantize_pool(vf, kv_dt, hv)
    if k_scale is not None:
        k_scale = np.ascontiguousarray(k_scale, np.float32)
        v_scale = np.ascontiguousarray(v_scale, np.float32)

    return Case(B=B, Hq=Hq, Hkv=Hkv, D=D, ctx=ctx, block_table=table, num_blocks=N, act=act_dt, kv=kv_dt,
                k_pool=np.ascontiguousarray(k_pool), v_pool=np.ascontiguousarray(v_pool), k_scale=k_scale,
                v_scale=v_scale, k_new=encode(k_new, act_dt), v_new=encode(v_new, act_dt), q=encode(qf, act_dt),
                seed=seed)


def config1(act="bf16", kv=None, seed=0) -> Case:
    """Qwen3-0.6B layer, Hq16/Hkv8/D128, contexts {17,64,100,255}, 128-block pool,
    inputs N(0,1)/sqrt(128)."""
    c = make_case(seed, 4, 16, 8, 128, [17, 64, 100, 255], act=act, kv=kv, input_scale=1 / math.sqrt(128),
                  pool_extra=0.0)
    return _resize_pool(c, 128, seed)


def _resize_pool(c: Case, N: int, seed: int) -> Case:
    """Re-map the case's tables onto a seeded permutation of an N-block pool (config 1 fixes N = 128)."""
    if c.num_blocks == N:
        return c
    rng = np.random.default_rng(seed + 7919)
    assert N >= c.num_blocks
    perm = rng.permutation(N).astype(np.int32)
    remap = perm[:c.num_blocks]
    table = np.where(c.block_table >= 0, remap[np.maximum(c.block_table, 0)], -1).astype(np.int32)

    def grow(pool):
        out = np.zeros((N,) + pool.shape[1:], dtype=pool.dtype)
        out[remap] = pool
        return out

    c.k_pool, c.v_pool = grow(c.k_pool), grow(c.v_pool)
    if c.kv == O.DTYPE_I8:
        c.k_scale, c.v_scale = grow(c.k_scale), grow(c.v_scale)
    c.block_table, c.num_blocks = table, N
    return c


def oracle_step(c: Case, threads: int = 0, max_context_len: int = 0):
    """Append the case's new tokens into copies of its pools and decode, on the CPU checker.
    Returns (k_pool, v_pool, k_scale, v_scale, out_storage, out_f32)."""
    kp, vp = c.k_pool.copy(), c.v_pool.copy()
    ks = None if c.k_scale is None else c.k_scale.copy()
    vs = None if c.v_scale is None else c.v_scale.copy()
    O.append(c.k_new, c.v_new, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs)
    out, out32 = O.paged_decode(c.q, c.act, kp, vp, c.kv, c.block_table, c.ctx, ks, vs,
                                max_context_len=max_context_len, threads=threads)
    return kp, vp, ks, vs, out, out32
