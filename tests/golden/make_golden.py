"""Write the golden fixtures under tests/golden/ from library routines only (torch-CPU and numpy).

The reference has no CPU implementation, tests or fixtures for its paged KV-cache path, so these vectors are
the independent pin for the CPU checker (oracle/) and the HIP library.  Nothing here calls either of them:

  * inputs        numpy ``default_rng(seed)``; float tensors rounded to bf16 by torch ``.to(torch.bfloat16)``
  * append        the reference's address formula (src/model/qwen_model.cu:32-42) applied with numpy fancy
                  indexing: pos = ctx[b] + t, page = table[b, pos // 16], slot = pos % 16
  * int8 append   scale = absmax / 127 in float32, codes = clamp(torch.round(x / scale), -127, 127)
                  (torch.round is round-half-even)
  * fp8 append    codes = torch ``(x / head_scale).to(torch.float8_e4m3fn)`` (RNE; |x / scale| <= 448 by the
                  choice of head_scale, where the saturating and non-saturating conventions agree)
  * decode        torch ``scaled_dot_product_attention`` in float64 over the gathered context_lens + 1 tokens
                  of each row, K/V heads repeated Hq/Hkv times (the GQA map of src/kernels/attention.cu:304)

Geometry: BASELINE config 1 (contexts {17, 64, 100, 255}, block size 16, head_dim 128, inputs N(0,1)/sqrt(128))
with the head counts cut to Hq = 4, Hkv = 2 to keep the files small, a 40-block pool of which 30 blocks are
used (the rest hold a 0xA5 sentinel so stray writes show), one new token appended per sequence.

Run: ``python tests/golden/make_golden.py`` (writes golden_<kv>.npz next to this file).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
B, HQ, HKV, D, BLOCK = 4, 4, 2, 128, 16
CTX = [17, 64, 100, 255]
N = 40
SEED = 1234


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def bf16_val(bits: np.ndarray) -> np.ndarray:
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(torch.float32).numpy()


def make(kv: str) -> dict:
    rng = np.random.default_rng(SEED + {"bf16": 0, "i8": 1, "fp8": 2}[kv])
    ctx = np.array(CTX, np.int32)
    need = [math.ceil((c + 1) / BLOCK) for c in CTX]
    perm = rng.permutation(N).astype(np.int32)
    table = np.full((B, max(need)), -1, np.int32)
    pos = 0
    for b in range(B):
        table[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    used = perm[:pos]
    s = np.float32(1 / math.sqrt(D))
    kf = rng.standard_normal((N, BLOCK, HKV, D), dtype=np.float32) * s
    vf = rng.standard_normal((N, BLOCK, HKV, D), dtype=np.float32) * s
    k_new = bf16_val(bf16_bits(rng.standard_normal((B, 1, HKV, D), dtype=np.float32) * s))
    v_new = bf16_val(bf16_bits(rng.standard_normal((B, 1, HKV, D), dtype=np.float32) * s))
    q = bf16_val(bf16_bits(rng.standard_normal((B, 1, HQ, D), dtype=np.float32) * s))
    unused = np.setdiff1d(np.arange(N), used)

    def store(xf, new, head_scale=None):
        """Quantize/round a float pool and the appended tokens the way append specifies; returns the pool
        after the append, the pool before it, and the scale array (or None)."""
        pool = xf.copy()
        b_idx = np.arange(B)
        p = ctx                                    # position of the one appended token (t = 0)
        pages = table[b_idx, p // BLOCK]
        slots = p % BLOCK
        if kv == "bf16":
            before = bf16_bits(pool)
            before[unused] = 0xA5A5
            after = before.copy()
            after[pages, slots] = bf16_bits(new[:, 0])
            return after, before, None
        if kv == "i8":
            def q8(rows):
                rows_t = torch.from_numpy(np.ascontiguousarray(rows, np.float32))
                amax = rows_t.abs().amax(dim=-1)
                sc = amax / torch.tensor(127.0, dtype=torch.float32)
                safe = torch.where(sc == 0, torch.ones_like(sc), sc)
                codes = torch.clamp(torch.round(rows_t / safe[..., None]), -127, 127).to(torch.int8)
                codes[sc == 0] = 0
                return codes.numpy(), sc.numpy().astype(np.float32)
            before, sc = q8(pool)
            before[unused] = np.int8(-91)          # 0xA5
            sc[unused] = 0.0
            after, sc_after = before.copy(), sc.copy()
            c, s_new = q8(new[:, 0])
            after[pages, slots] = c
            sc_after[pages, slots] = s_new
            return after, before, (sc, sc_after)
        # fp8 e4m3 with per-head scales
        t = torch.from_numpy(np.ascontiguousarray(pool / head_scale[None, None, :, None], np.float32))
        before = t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        before[unused] = 0xA5
        after = before.copy()
        tn = torch.from_numpy(np.ascontiguousarray(new[:, 0] / head_scale[None, :, None], np.float32))
        after[pages, slots] = tn.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        return after, before, (head_scale, head_scale)

    hk = hv = None
    if kv == "fp8":
        hk = (np.maximum(np.abs(kf).max(axis=(0, 1, 3)), np.abs(k_new).max(axis=(0, 1, 3))) / 448.0) \
            .astype(np.float32)
        hv = (np.maximum(np.abs(vf).max(axis=(0, 1, 3)), np.abs(v_new).max(axis=(0, 1, 3))) / 448.0) \
            .astype(np.float32)
    k_after, k_before, k_sc = store(kf, k_new, hk)
    v_after, v_before, v_sc = store(vf, v_new, hv)

    def deq(pool, sc, which):
        if kv == "bf16":
            return bf16_val(pool).astype(np.float64)
        if kv == "i8":
            return pool.astype(np.float64) * sc[which].astype(np.float64)[..., None]
        vals = torch.from_numpy(pool).view(torch.float8_e4m3fn).to(torch.float64).numpy()
        return vals * sc[which].astype(np.float64)[None, None, :, None]

    kd = deq(k_after, k_sc, 1)
    vd = deq(v_after, v_sc, 1)
    out = np.zeros((B, HQ, D), np.float64)
    for b in range(B):
        L = CTX[b] + 1
        tok = np.arange(L)
        pg, sl = table[b, tok // BLOCK], tok % BLOCK
        Kb = torch.from_numpy(kd[pg, sl]).permute(1, 0, 2)            # [Hkv, L, D]
        Vb = torch.from_numpy(vd[pg, sl]).permute(1, 0, 2)
        Kb = Kb.repeat_interleave(HQ // HKV, dim=0).contiguous()
        Vb = Vb.repeat_interleave(HQ // HKV, dim=0).contiguous()
        qb = torch.from_numpy(q[b, 0].astype(np.float64))[:, None, :]   # [Hq, 1, D]
        o = torch.nn.functional.scaled_dot_product_attention(qb, Kb, Vb, scale=1.0 / math.sqrt(D))
        out[b] = o[:, 0].numpy()

    rec = dict(ctx=ctx, block_table=table, num_blocks=np.int32(N), q_bf16=bf16_bits(q),
               k_new_bf16=bf16_bits(k_new), v_new_bf16=bf16_bits(v_new), k_pool_before=k_before,
               v_pool_before=v_before, k_pool_after=k_after, v_pool_after=v_after, out_f64=out)
    if kv == "i8":
        rec.update(k_scale_before=k_sc[0], v_scale_before=v_sc[0], k_scale_after=k_sc[1], v_scale_after=v_sc[1])
    if kv == "fp8":
        rec.update(k_head_scale=hk, v_head_scale=hv)
    return rec


def main() -> None:
    for kv in ("bf16", "i8", "fp8"):
        rec = make(kv)
        path = HERE / f"golden_{kv}.npz"
        np.savez_compressed(path, **rec)
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
