"""Benchmark of the paged KV-cache hot path on one MI355X.

Workload: Qwen3-8B layer shape, bf16 KV, 32 query heads, 8 KV heads (GQA 4),
head_dim 128, block size 16, batch 64, pre-append context lengths uniform in [512, 4096], block tables a
seeded permutation of a pool sized to total blocks + 10 %, Q/K/V ~ N(0,1).  One step = append one new K/V
token per sequence and run decode attention over context_lens + 1 tokens, on one layer's pool, issued as one
call (ffkv_append_paged_decode: the decode kernel writes each row's new token into its page and attends it);
`step_ms_two_calls` times the same steps as ffkv_append then ffkv_paged_decode.  Steps rotate over `--layers` independent pools (as a model's layers do), so the
working set (~2.7 GB at 4 layers) is far beyond the 256 MB Infinity Cache and every step streams its KV from
HBM.

Printed JSON line (rank 0, N = 1):
  value          algorithmic HBM bytes of (append + decode) per step / wall time per step, in TB/s
  roofline       the decode call (split-K pass + merge pass) timed with HIP events on the launch stream;
                 achieved = algorithmic decode bytes / mean call duration, peak 8 TB/s
  cpu_baseline   the C restatement under oracle/ (the checker) timed on the host cores on the same layer-0
                 inputs, same algorithmic-bytes formula, threaded over every core this process may run on
  parity         max-abs error of the layer-0 GPU output against that CPU result (fp32, before rounding)
  device_copy    a 1 GiB torch device copy timed the same way: the streaming rate a plain kernel reaches here
  read_stream    a read-only 2 GiB stream (firefly_amd/libffkv_bench.so) over a few launch shapes: the practical
                 read ceiling for the read-dominated decode; decode_call_vs_read_stream = roofline.achieved over it;
                 at_call_size: the best shape over buffers of one decode call's bytes (start and tail included),
                 decode_call_vs_read_at_call_size = roofline.achieved over that
  other_configs  C3, C4 and C5 (int8 and fp8 pools filled by the quantizing append, whose bulk throughput is
                 reported as quantized_append), the C4 prefill on every cache type and head_dim, decodes at head_dim
                 256, 96, 112 and 80 and over fp32 pages (the vector kernel), the fused rope + append, and the decode
                 step's host upload

Algorithmic bytes per decode call (L'_b = context_lens[b] + 1):
  sum_b L'_b*Hkv*D*2*2 (K and V) + B*Hq*D*2*2 (q in, out) + sum_b ceil(L'_b/16)*4 (block table) + 4*B
Algorithmic bytes per append call: T*Hkv*D*2*2 (read k, v) + T*Hkv*D*2*2 (write pages) + 4*B (context_lens)
  + 4*T (one block-table entry per token).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_TBS = 8.0
B, HQ, HKV, D, BLOCK = 64, 32, 8, 128, 16
CTX_LO, CTX_HI = 512, 4096
SEED = 0


def workload(seed: int = SEED):
    """Context lengths and block tables of config 2 (numpy, seeded)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    ctx = rng.integers(CTX_LO, CTX_HI + 1, size=B).astype(np.int32)
    need = [math.ceil((int(c) + 1) / BLOCK) for c in ctx]
    total = sum(need)
    N = math.ceil(total * 1.1)
    perm = rng.permutation(N).astype(np.int32)
    mb = max(need)
    table = np.full((B, mb), -1, dtype=np.int32)
    pos = 0
    for b in range(B):
        table[b, :need[b]] = perm[pos:pos + need[b]]
        pos += need[b]
    return ctx, table, N


def decode_bytes(ctx) -> int:
    Lp = [int(c) + 1 for c in ctx]
    return (sum(Lp) * HKV * D * 2 * 2 + len(ctx) * HQ * D * 2 * 2 + sum(math.ceil(x / BLOCK) for x in Lp) * 4
            + 4 * len(ctx))


def append_bytes(T: int, batch: int) -> int:
    return T * HKV * D * 2 * 2 * 2 + 4 * batch + 4 * T


def measured_traffic():
    """(HBM bytes per decode call, commit it was measured at) from the rocprofv3 counter passes recorded in
    profiles/decode_c2_traffic.json (FETCH_SIZE and WRITE_SIZE of the decode and merge kernels, scaled by the same
    counters' reading for a copy of known size); (None, None) when that record is absent."""
    path = ROOT / "profiles" / "decode_c2_traffic.json"
    if not path.exists():
        return None, None
    rec = json.loads(path.read_text())
    return rec.get("bytes_per_call"), rec.get("measured_at_commit")


def device_copy_rate(torch, dev, stream, nbytes: int = 1 << 30) -> dict:
    """A 1 GiB device-to-device copy (torch), timed with HIP events: the streaming rate a plain kernel reaches on
    this GPU, reported beside the roofline's 8 TB/s peak (read + write bytes over time)."""
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    us = _events_us(lambda i: dst.copy_(src), 20, stream)
    del src, dst
    torch.cuda.empty_cache()
    return {"bytes_moved": 2 * nbytes, "us_per_copy": us, "TB_per_s": 2 * nbytes / (us * 1e-6) / 1e12,
            "pct_of_peak": 2 * nbytes / (us * 1e-6) / 1e12 / HBM_PEAK_TBS * 100}


def read_stream_rate(torch, dev, stream, nbytes: int = 2 << 30, call_bytes: int | None = None) -> dict | None:
    """A read-only stream over 2 GiB (firefly_amd/libffkv_bench.so: 16-byte loads, 4 or 8 in flight per lane, one
    word written per workgroup), timed with HIP events for a few launch shapes: the practical read ceiling of this
    GPU for a read-dominated kernel such as the decode.  The best shape is `TB_per_s`; every shape is listed.
    With call_bytes, the best shape also reads buffers of that size (four, in turn, so that the 256 MB on-chip
    cache cannot hold them, as the decode rotates its layer pools): `at_call_size`, the ceiling for a launch that
    reads as much as one decode call, start and tail included."""
    import ctypes

    path = ROOT / "firefly_amd" / "libffkv_bench.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    lib.ffkv_bench_stream_read.restype = ctypes.c_int
    lib.ffkv_bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p]
    src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)
    shapes = {}
    for blocks in (2048, 4096, 8192, 16384):  # powers of two: 2 GiB splits evenly over every lane
        for unroll in (4, 8):
            def call(i, b=blocks, u=unroll):
                rc = lib.ffkv_bench_stream_read(src.data_ptr(), nbytes, sink.data_ptr(), b, u, stream.cuda_stream)
                assert rc == 0
            us = _events_us(call, 20, stream)
            shapes[f"{blocks}x256_unroll{unroll}"] = {"us": us, "TB_per_s": nbytes / (us * 1e-6) / 1e12}
    del src
    torch.cuda.empty_cache()
    best = max(shapes, key=lambda k: shapes[k]["TB_per_s"])
    at_call = None
    if call_bytes is not None and call_bytes >= 16:
        nb = call_bytes // 16 * 16
        blocks = int(best.split("x")[0])
        unroll = int(best.rsplit("unroll", 1)[1])
        bufs = [torch.ones(nb, dtype=torch.uint8, device=dev) for _ in range(4)]

        def call(i):
            rc = lib.ffkv_bench_stream_read(bufs[i % 4].data_ptr(), nb, sink.data_ptr(), blocks, unroll,
                                            stream.cuda_stream)
            assert rc == 0
        us = _events_us(call, 20, stream)
        at_call = {"bytes_read": nb, "buffers": 4, "shape": best, "us": us, "TB_per_s": nb / (us * 1e-6) / 1e12}
        del bufs
    del sink
    torch.cuda.empty_cache()
    return {"bytes_read": nbytes, "best_shape": best, "TB_per_s": shapes[best]["TB_per_s"],
            "pct_of_peak": shapes[best]["TB_per_s"] / HBM_PEAK_TBS * 100, "shapes": shapes,
            "at_call_size": at_call}


BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def _events_us(fn, n: int, stream, warm_ms: float = 50.0) -> float:
    """Mean duration in us of fn(i) over n back-to-back calls, HIP events on the launch stream, after at least
    warm_ms of untimed calls (a GPU that has been idle runs its first tens of milliseconds of work up to 15 % slow,
    which would otherwise bias whichever configuration is measured first)."""
    import time

    import torch

    t0 = time.perf_counter()
    i = 0
    while True:
        fn(i)
        i += 1
        if i >= 3 and i % 4 == 0:
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= warm_ms or i >= 400:
                break
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n * 1e3


def _tables(rng, need, shared_blocks=0):
    """Block tables for rows needing `need` blocks each; the first `shared_blocks` logical blocks of every row map
    to the same physical blocks (a radix-cache prefix).  Returns (table int32 [B, max], pool blocks)."""
    import numpy as np

    private = [max(0, n - shared_blocks) for n in need]
    total = shared_blocks + sum(private)
    N = math.ceil(total * 1.1)
    perm = rng.permutation(N).astype(np.int32)
    table = np.full((len(need), max(need)), -1, dtype=np.int32)
    pos = shared_blocks
    for b, n in enumerate(need):
        k = min(shared_blocks, n)
        table[b, :k] = perm[:k]
        table[b, k:n] = perm[pos:pos + private[b]]
        pos += private[b]
    return table, N


def _pools(torch, gen, dev, N, Hkv, D, kv, layers):
    """Random bf16 or fp32 pools (quantized pools come from _appended_pools)."""
    assert kv in ("bf16", "f32")
    shape = (N, BLOCK, Hkv, D)
    dt = torch.bfloat16 if kv == "bf16" else torch.float32
    return [(torch.randn(shape, generator=gen, device=dev, dtype=dt),
             torch.randn(shape, generator=gen, device=dev, dtype=dt), None, None) for _ in range(layers)]


def _appended_pools(ff, torch, gen, dev, stream, N, Hkv, D, kv, layers, table, ctx, chunk=1024):
    """Quantized pools filled the way an engine fills them: bf16 K/V ~ N(0,1) with 1% of the elements x8 go
    through the quantizing append (int8: per-token absmax/127 scales written by the append; fp8: per-head scales
    absmax/448 read by it) in chunks of `chunk` tokens per row at positions 0, chunk, 2*chunk, ... (one chunk of
    source data, appended at every offset).  Returns (pools, quantized-append figure of the first chunk)."""
    import numpy as np

    B = table.shape[0]

    def src():
        x = torch.randn((B, chunk, Hkv, D), generator=gen, device=dev, dtype=torch.float32)
        x = torch.where(torch.rand(x.shape, generator=gen, device=dev) < 0.01, x * 8.0, x)
        return x.to(torch.bfloat16)

    ks_src, vs_src = src(), src()
    offsets = range(0, int(max(ctx)) + 1, chunk)
    cx = [torch.full((B,), o, dtype=torch.int32, device=dev) for o in offsets]
    pools, fig = [], None
    for layer in range(layers):
        store = torch.int8 if kv == "i8" else torch.uint8
        kp = torch.empty((N, BLOCK, Hkv, D), dtype=store, device=dev)
        vp = torch.empty_like(kp)
        if kv == "i8":
            ks = torch.empty((N, BLOCK, Hkv), device=dev)
            vs = torch.empty_like(ks)
        else:
            ks = (ks_src.float().abs().amax(dim=(0, 1, 3)) / 448.0).contiguous()
            vs = (vs_src.float().abs().amax(dim=(0, 1, 3)) / 448.0).contiguous()
        if layer == 0:  # time the first chunk's append: every row has >= 1024 cached tokens (C5 contexts)
            us = _events_us(lambda i: ff.append_kv_cache(ks_src, vs_src, kp, vp, table, cx[0], ks, vs, stream=stream),
                            10, stream)
            T = B * chunk
            nbytes = T * Hkv * D * (2 + 1) * 2 + (T * Hkv * 4 * 2 if kv == "i8" else Hkv * 4 * 2) + 4 * B + 4 * T
            fig = {"kv": kv, "tokens": T, "bytes": nbytes, "us_per_call": us, "GB_per_s": nbytes / (us * 1e-6) / 1e9,
                   "pct_of_peak": nbytes / (us * 1e-6) / 1e12 / HBM_PEAK_TBS * 100}
        for c in cx:
            ff.append_kv_cache(ks_src, vs_src, kp, vp, table, c, ks, vs, stream=stream)
        pools.append((kp, vp, ks, vs))
    torch.cuda.synchronize()
    del ks_src, vs_src
    return pools, fig


def decode_config(ff, torch, dev, stream, name, B, Hq, Hkv, D, ctx, kv="bf16", layers=2, shared_blocks=0,
                  calls=50, seed=0):
    """Decode attention alone on one configuration (layers rotated to defeat the 256 MB Infinity Cache).  bf16
    pools are random; int8 / fp8 pools are filled by the quantizing append (whose throughput is reported)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    Lp = [int(c) + 1 for c in ctx]
    need = [math.ceil(x / BLOCK) for x in Lp]
    table_np, N = _tables(rng, need, shared_blocks)
    bt = torch.from_numpy(table_np).to(dev)
    append_fig = None
    if kv in ("bf16", "f32"):
        pools = _pools(torch, gen, dev, N, Hkv, D, kv, layers)
    else:
        pools, append_fig = _appended_pools(ff, torch, gen, dev, stream, N, Hkv, D, kv, layers, bt, Lp)
    q = torch.randn((B, 1, Hq, D), generator=gen, device=dev, dtype=torch.bfloat16)
    out = torch.empty((B, 1, Hq * D), device=dev, dtype=torch.bfloat16)
    cx = torch.from_numpy(np.asarray(ctx, np.int32)).to(dev)
    ws = ff.decode_workspace(B, Hq, D, table_np.shape[1], max(Lp), device=dev)

    def call(i):
        kp, vp, ks, vs = pools[i % layers]
        ff.paged_attention(q, kp, vp, bt, cx, out=out, k_scale=ks, v_scale=vs, max_context_len=max(Lp),
                           workspace=ws, stream=stream)

    us = _events_us(call, calls, stream)
    es = {"bf16": 2, "f32": 4}.get(kv, 1)
    tok = sum(Lp)
    kv_bytes = tok * Hkv * D * es * 2 + (tok * Hkv * 4 * 2 if kv == "i8" else 0)
    other = B * Hq * D * 2 * 2 + sum(need) * 4 + 4 * B
    logical = kv_bytes + other
    rec = {"workload": name, "kv": kv, "batch": B, "heads": f"{Hq}/{Hkv}", "head_dim": D,
           "context_tokens": tok, "us_per_call": us, "algorithmic_bytes": logical,
           "TB_per_s": logical / (us * 1e-6) / 1e12, "pct_of_peak": logical / (us * 1e-6) / 1e12 / HBM_PEAK_TBS * 100,
           "tokens_per_s": B / (us * 1e-6)}
    if append_fig is not None:
        rec["quantized_append"] = append_fig
    if shared_blocks:
        ushared = shared_blocks * BLOCK
        utok = ushared + sum(x - min(ushared, x) for x in Lp)
        unique = utok * Hkv * D * es * 2 + other
        rec.update({"unique_bytes": unique, "unique_TB_per_s": unique / (us * 1e-6) / 1e12,
                    "unique_pct_of_peak": unique / (us * 1e-6) / 1e12 / HBM_PEAK_TBS * 100,
                    "effective_TB_per_s_logical": rec["TB_per_s"]})
    del pools
    torch.cuda.empty_cache()
    return rec


def c4_config(ff, torch, dev, stream, layers=2, calls=30, seed=4):
    """128 sequences sharing a 2048-token prefix (128 physical blocks in every table), private
    suffixes U[64, 1024]; per step 120 rows decode (append 1 token + attention) and 8 rows run a 512-token chunked
    prefill (append 512 tokens + causal attention over their cached prefix and the chunk)."""
    import numpy as np

    Bt, Bd, Hq, Hkv, D, PRE, CH = 128, 120, 32, 8, 128, 2048, 512
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    suffix = rng.integers(64, 1025, size=Bt)
    ctx = (PRE + suffix).astype(np.int32)                     # cached before this step
    new = np.array([1] * Bd + [CH] * (Bt - Bd))
    need = [math.ceil((int(c) + int(n)) / BLOCK) for c, n in zip(ctx, new)]
    table_np, N = _tables(rng, need, PRE // BLOCK)
    pools = _pools(torch, gen, dev, N, Hkv, D, "bf16", layers)
    bt_d = torch.from_numpy(table_np[:Bd].copy()).to(dev)
    bt_c = torch.from_numpy(table_np[Bd:].copy()).to(dev)
    cx_d = torch.from_numpy(ctx[:Bd].copy()).to(dev)
    cx_c = torch.from_numpy(ctx[Bd:].copy()).to(dev)
    Bc = Bt - Bd
    qd = torch.randn((Bd, 1, Hq, D), generator=gen, device=dev, dtype=torch.bfloat16)
    kd = torch.randn((Bd, 1, Hkv, D), generator=gen, device=dev, dtype=torch.bfloat16)
    vd = torch.randn((Bd, 1, Hkv, D), generator=gen, device=dev, dtype=torch.bfloat16)
    qc = torch.randn((Bc, CH, Hq, D), generator=gen, device=dev, dtype=torch.bfloat16)
    kc = torch.randn((Bc, CH, Hkv, D), generator=gen, device=dev, dtype=torch.bfloat16)
    vc = torch.randn((Bc, CH, Hkv, D), generator=gen, device=dev, dtype=torch.bfloat16)
    od = torch.empty((Bd, 1, Hq * D), device=dev, dtype=torch.bfloat16)
    oc = torch.empty((Bc, CH, Hq * D), device=dev, dtype=torch.bfloat16)
    ws = ff.decode_workspace(Bd, Hq, D, table_np.shape[1], device=dev)
    SB = PRE // BLOCK  # pages every table shares
    ws_sp = ff.shared_prefix_workspace(Bd, Hq, Hkv, D, table_np.shape[1], SB, device=dev)

    def dec(i):
        kp, vp, _, _ = pools[i % layers]
        ff.paged_attention(qd, kp, vp, bt_d, cx_d, out=od, workspace=ws, stream=stream)

    def dec_sp(i):
        kp, vp, _, _ = pools[i % layers]
        ff.paged_attention_shared_prefix(qd, kp, vp, bt_d, cx_d, SB, out=od, workspace=ws_sp, stream=stream)

    def chunk_append(i):
        kp, vp, _, _ = pools[i % layers]
        ff.append_kv_cache(kc, vc, kp, vp, bt_c, cx_c, stream=stream)

    def pre(i):
        kp, vp, _, _ = pools[i % layers]
        ff.paged_prefill(qc, kp, vp, bt_c, cx_c, out=oc, stream=stream)

    def step(i):
        kp, vp, _, _ = pools[i % layers]
        ff.append_kv_cache(kd, vd, kp, vp, bt_d, cx_d, stream=stream)
        ff.paged_attention_shared_prefix(qd, kp, vp, bt_d, cx_d, SB, out=od, workspace=ws_sp, stream=stream)
        ff.append_kv_cache(kc, vc, kp, vp, bt_c, cx_c, stream=stream)
        ff.paged_prefill(qc, kp, vp, bt_c, cx_c, out=oc, stream=stream)

    # The same step with the decode rows' half on a second stream (default priority), forked from and joined back
    # to the launch stream: the HBM-bound decode runs beside the matrix-bound prefill.  The two halves touch
    # disjoint rows (the shared prefix pages are only read), so the results are the same.
    side = torch.cuda.Stream(device=dev)
    forks = [torch.cuda.Event() for _ in range(layers)]
    joins = [torch.cuda.Event() for _ in range(layers)]

    def step_two_streams(i):
        kp, vp, _, _ = pools[i % layers]
        forks[i % layers].record(stream)
        side.wait_event(forks[i % layers])
        ff.append_kv_cache(kd, vd, kp, vp, bt_d, cx_d, stream=side)
        ff.paged_attention_shared_prefix(qd, kp, vp, bt_d, cx_d, SB, out=od, workspace=ws_sp, stream=side)
        ff.append_kv_cache(kc, vc, kp, vp, bt_c, cx_c, stream=stream)
        ff.paged_prefill(qc, kp, vp, bt_c, cx_c, out=oc, stream=stream)
        joins[i % layers].record(side)
        stream.wait_event(joins[i % layers])

    for i in range(layers):
        chunk_append(i)  # the chunks' K/V are in the pages before any prefill reads them
    torch.cuda.synchronize()
    us_dec = _events_us(dec, calls, stream)
    us_dsp = _events_us(dec_sp, calls, stream)
    us_app = _events_us(chunk_append, calls, stream)
    us_pre = _events_us(pre, calls, stream)
    us_step = _events_us(step, calls, stream)
    us_step2 = _events_us(step_two_streams, calls, stream)
    Lp = [int(c) + 1 for c in ctx[:Bd]]
    tok = sum(Lp)
    other = Bd * Hq * D * 2 * 2 + sum(math.ceil(x / BLOCK) for x in Lp) * 4 + 4 * Bd
    logical = tok * Hkv * D * 2 * 2 + other
    unique = (PRE + sum(x - PRE for x in Lp)) * Hkv * D * 2 * 2 + other
    flops = sum((int(c) + t + 1) * Hq * D * 4 for c in ctx[Bd:] for t in range(CH))
    app_bytes = append_bytes(Bc * CH, Bc)
    del pools
    torch.cuda.empty_cache()
    return {
        "workload": "C4 prefix-shared: 128 rows, 2048-token shared prefix (128 shared blocks), suffix U[64,1024]; "
                    "120 decode rows + 8 rows chunk-prefilling 512 tokens",
        "step_us": us_step,
        "step_us_two_streams": us_step2,
        "decode": {"rows": Bd, "us_per_call": us_dec, "logical_bytes": logical, "unique_bytes": unique,
                   "unique_TB_per_s": unique / (us_dec * 1e-6) / 1e12,
                   "unique_pct_of_peak": unique / (us_dec * 1e-6) / 1e12 / HBM_PEAK_TBS * 100,
                   "effective_TB_per_s_logical": logical / (us_dec * 1e-6) / 1e12},
        # the same decode with the shared pages attended once for all rows (ffkv_paged_decode_shared_prefix)
        "decode_shared_prefix": {"rows": Bd, "shared_blocks": SB, "us_per_call": us_dsp,
                                 "unique_TB_per_s": unique / (us_dsp * 1e-6) / 1e12,
                                 "unique_pct_of_peak": unique / (us_dsp * 1e-6) / 1e12 / HBM_PEAK_TBS * 100,
                                 "speedup_vs_plain": us_dec / us_dsp},
        "chunk_append": {"tokens": Bc * CH, "us_per_call": us_app, "bytes": app_bytes,
                         "GB_per_s": app_bytes / (us_app * 1e-6) / 1e9},
        "prefill": {"rows": Bc, "chunk": CH, "us_per_call": us_pre, "causal_flops": flops,
                    "TFLOP_per_s": flops / (us_pre * 1e-6) / 1e12,
                    "pct_of_bf16_mfma_peak": flops / (us_pre * 1e-6) / 1e12 / BF16_MFMA_PEAK_TFLOPS * 100},
    }


def prefill_variants_config(ff, torch, dev, stream, layers=2, calls=30, seed=7):
    """The C4 chunked prefill (8 rows x 512 new tokens over 2048 + U[64, 1024] cached tokens) on every cache type
    and head_dim the prefill serves: bf16 / f16 / fp8 / int8 caches at head_dim 128 (Hq32/Hkv8; q in the cache's
    16-bit type, bf16 for the 8-bit caches), and bf16 at head_dim 64 (Hq32/Hkv8) and 256 (Hq16/Hkv4).  16-bit pools
    are random; 8-bit pools are filled by the quantizing append."""
    import numpy as np

    Bc, CH, PRE = 8, 512, 2048
    out = {}
    for name, kv, D, Hq, Hkv in (("bf16_d128", "bf16", 128, 32, 8), ("f16_d128", "f16", 128, 32, 8),
                                 ("fp8_d128", "fp8", 128, 32, 8), ("i8_d128", "i8", 128, 32, 8),
                                 ("bf16_d64", "bf16", 64, 32, 8), ("bf16_d256", "bf16", 256, 16, 4)):
        rng = np.random.default_rng(seed)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        ctx = (PRE + rng.integers(64, 1025, size=Bc)).astype(np.int32)
        need = [math.ceil((int(c) + CH) / BLOCK) for c in ctx]
        table_np, N = _tables(rng, need)
        bt = torch.from_numpy(table_np).to(dev)
        cx = torch.from_numpy(ctx).to(dev)
        qt = torch.float16 if kv == "f16" else torch.bfloat16
        if kv in ("bf16", "f16"):
            shape = (N, BLOCK, Hkv, D)
            pools = [(torch.randn(shape, generator=gen, device=dev).to(qt),
                      torch.randn(shape, generator=gen, device=dev).to(qt), None, None) for _ in range(layers)]
        else:
            pools, _ = _appended_pools(ff, torch, gen, dev, stream, N, Hkv, D, kv, layers, bt,
                                       [int(c) + CH for c in ctx])
        q = torch.randn((Bc, CH, Hq, D), generator=gen, device=dev).to(qt)
        o = torch.empty((Bc, CH, Hq * D), device=dev, dtype=qt)

        def pre(i):
            kp, vp, ks, vs = pools[i % layers]
            ff.paged_prefill(q, kp, vp, bt, cx, out=o, k_scale=ks, v_scale=vs, stream=stream)

        us = _events_us(pre, calls, stream)
        flops = sum((int(c) + t + 1) * Hq * D * 4 for c in ctx for t in range(CH))
        out[name] = {"kv": kv, "q": "f16" if kv == "f16" else "bf16", "heads": f"{Hq}/{Hkv}", "head_dim": D,
                     "us_per_call": us, "causal_flops": flops, "TFLOP_per_s": flops / (us * 1e-6) / 1e12,
                     "pct_of_16bit_mfma_peak": flops / (us * 1e-6) / 1e12 / BF16_MFMA_PEAK_TFLOPS * 100}
        del pools, q, o
        torch.cuda.empty_cache()
    return {"workload": "chunked prefill, 8 rows x 512 tokens over 2048 + U[64,1024] cached tokens, per cache "
                        "type and head_dim", **out}


def rope_append_config(ff, torch, dev, stream, calls=50, seed=5):
    """Fused rotary embedding + KV append: the C2 decode-step shape (64 tokens) and a bulk 64 x 2048 prefill."""
    import numpy as np

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    rng = np.random.default_rng(seed)
    res = {}
    for label, S in (("decode_step", 1), ("bulk", 2048)):
        nb = math.ceil(S / BLOCK) + 1
        bt = torch.from_numpy(rng.permutation(B * nb).astype(np.int32).reshape(B, nb)).to(dev)
        ctx = torch.from_numpy(rng.integers(0, BLOCK, size=B).astype(np.int32)).to(dev)
        q = torch.randn((B, S, HQ, D), generator=gen, device=dev, dtype=torch.bfloat16)
        k = torch.randn((B, S, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        v = torch.randn((B, S, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        kc = torch.empty((B * nb, BLOCK, HKV, D), device=dev, dtype=torch.bfloat16)
        vc = torch.empty_like(kc)
        us = _events_us(lambda i: ff.rope_append_kv_cache(q, k, v, kc, vc, bt, ctx, 1e6, stream=stream),
                        calls if S == 1 else 10, stream)
        T = B * S
        # read q, k, v; write q, k back; write the K/V pages; the rows' context_lens and block-table entries
        nbytes = T * (HQ + 2 * HKV) * D * 2 + T * (HQ + HKV) * D * 2 + T * HKV * D * 2 * 2 + 4 * B + 4 * T
        res[label] = {"tokens": T, "us_per_call": us, "bytes": nbytes, "GB_per_s": nbytes / (us * 1e-6) / 1e9}
        del q, k, v, kc, vc
    torch.cuda.empty_cache()
    return res


def decode_batch_upload(torch, stream, ctx_np, table_np, calls=50) -> dict | None:
    """firefly::DecodeBatch::upload itself (through tests/cpp/libdecode_step_shim.so, the C++ API's test shim):
    the C2 rows packed with DecodeBatch::pack, then one upload per step on the launch stream (a kernel that reads
    the pinned staging through its device mapping), timed with HIP events (best of three runs)."""
    import ctypes

    import numpy as np

    path = ROOT / "tests" / "cpp" / "libdecode_step_shim.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    vp, i, ip = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)
    for name, res, args in [("dss_create", vp, [i, i]), ("dss_destroy", None, [vp]),
                            ("dss_pack", i, [vp, i, ip, ip, ip]), ("dss_upload", i, [vp, vp]),
                            ("dss_last_upload_bytes", ctypes.c_longlong, [vp])]:
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    Bn, stride = len(ctx_np), table_np.shape[1]
    nblk = [int((table_np[b] >= 0).sum()) for b in range(Bn)]
    blocks = [int(x) for b in range(Bn) for x in table_np[b, :nblk[b]]]
    arr = lambda xs: (ctypes.c_int * max(1, len(xs)))(*xs)  # noqa: E731
    h = lib.dss_create(Bn, stride)
    assert h
    try:
        width = lib.dss_pack(h, Bn, arr([int(c) for c in ctx_np]), arr(nblk), arr(blocks))
        assert width > 0

        def up(k):
            assert lib.dss_upload(h, stream.cuda_stream) == 0

        us = min(_events_us(up, calls, stream) for _ in range(3))
        nbytes = int(lib.dss_last_upload_bytes(h))
    finally:
        lib.dss_destroy(h)
    return {"row_stride_blocks": stride, "live_width": width, "bytes": nbytes, "copies": 1,
            "how": "one kernel reading the pinned staging through its device mapping", "us_per_step": us}


def decode_step_config(ff, torch, dev, stream, ctx_np, table_np, N, pools, q, k_new, v_new, out, ws, max_ctx,
                       calls=50):
    """The engine's per-step host -> device upload of context lengths and block tables (src/engine.cc:296-322):
    the reference's layout (row stride = pool blocks, the whole table every step) against the live width only
    (what firefly::DecodeBatch uploads), from pinned memory; and the C2 append + decode step replayed from one
    captured hipGraph against eager launches."""
    import numpy as np

    Bn = len(ctx_np)
    res = {}
    for label, stride in (("reference_layout", N), ("live_width", table_np.shape[1])):
        h = torch.full((Bn, stride), -1, dtype=torch.int32).pin_memory()
        h[:, :table_np.shape[1]] = torch.from_numpy(table_np)
        hc = torch.from_numpy(ctx_np.astype(np.int32)).pin_memory()
        d = torch.empty((Bn, stride), dtype=torch.int32, device=dev)
        dc = torch.empty(Bn, dtype=torch.int32, device=dev)

        def up(i):
            dc.copy_(hc, non_blocking=True)
            d.copy_(h, non_blocking=True)

        # best of three runs: a small pinned upload's time varies with the host-side copy path from run to run
        us = min(_events_us(up, calls, stream) for _ in range(3))
        res[label] = {"row_stride_blocks": stride, "bytes": Bn * stride * 4 + Bn * 4, "copies": 2, "us_per_step": us}
        del h, d
    res["decode_batch"] = decode_batch_upload(torch, stream, ctx_np, table_np, calls)
    table = torch.from_numpy(table_np).to(dev)
    cx = torch.from_numpy(ctx_np.astype(np.int32)).to(dev)
    L = len(pools)

    def step(i, s=stream):
        kp, vp = pools[i % L]
        ff.append_kv_cache(k_new, v_new, kp, vp, table, cx, stream=s)
        ff.paged_attention(q, kp, vp, table, cx, out=out, max_context_len=max_ctx, workspace=ws, stream=s)

    eager = _events_us(step, calls, stream)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for i in range(L):
                step(i, torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = _events_us(lambda i: g.replay(), max(1, calls // L), stream) / L
    res["step_us_eager"] = eager
    res["step_us_graph"] = graph
    return res


def decode_timeline(ff, torch, np, stream, call, calls: int = 5, warm: int = 20, out_path=None) -> dict:
    """Per-wave start and end times of the split-K decode kernel (a timeline build of the library records them on
    the GPU's 100 MHz clock), over `calls` decode calls after `warm` untimed ones: when the waves start, when they
    end (relative to the first start), and how far the last end trails the median one."""
    import ctypes

    fn = getattr(ff.lib, "ffkv_decode_timeline", None)
    if fn is None:
        raise SystemExit("--timeline needs --lib pointing at a timeline build: python -m firefly_amd.build "
                         "--define FFKV_DECODE_TIMELINE=1 --out PATH")
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    fn.restype = ctypes.c_int
    max_waves = 1 << 16
    buf = np.zeros(2 * max_waves, dtype=np.uint64)
    for i in range(warm):
        call(i)
    torch.cuda.synchronize()
    per_call, raw = [], []
    for i in range(calls):
        torch.cuda.synchronize()
        assert fn(None, max_waves, 1) == 0
        call(i)
        torch.cuda.synchronize()
        assert fn(buf.ctypes.data, max_waves, 0) == 0
        st, en = buf[0::2].copy(), buf[1::2].copy()
        raw.append((st, en))
        rec = st > 0
        t0 = int(st[rec].min())
        s_us = (st[rec] - t0) / 100.0  # 100 MHz ticks -> us
        e_us = (en[rec] - t0) / 100.0
        q = lambda x, p: float(np.percentile(x, p))
        per_call.append({
            "waves": int(rec.sum()),
            "start_us": {"p50": q(s_us, 50), "p90": q(s_us, 90), "max": float(s_us.max())},
            "end_us": {"p10": q(e_us, 10), "p50": q(e_us, 50), "p90": q(e_us, 90), "p99": q(e_us, 99),
                       "max": float(e_us.max())},
            "wave_us": {"p50": q(e_us - s_us, 50), "p90": q(e_us - s_us, 90)},
            "tail_after_median_end_us": float(e_us.max()) - q(e_us, 50),
        })
    if out_path is not None:  # wave w = (blockIdx.y * gridDim.x + blockIdx.x) * waves per workgroup + wave
        np.savez(out_path, start=np.stack([r[0] for r in raw]), end=np.stack([r[1] for r in raw]))
    med = lambda key, sub: float(np.median([c[key][sub] for c in per_call]))
    return {
        "timeline": "paged_decode_mfma, C2 decode call (bench.py workload), wave start/end on the 100 MHz clock",
        "calls": calls,
        "waves": per_call[0]["waves"],
        "median_over_calls": {
            "start_us": {k: med("start_us", k) for k in ("p50", "p90", "max")},
            "end_us": {k: med("end_us", k) for k in ("p10", "p50", "p90", "p99", "max")},
            "wave_us": {k: med("wave_us", k) for k in ("p50", "p90")},
            "tail_after_median_end_us": float(np.median([c["tail_after_median_end_us"] for c in per_call])),
        },
        "per_call": per_call,
    }


def cpu_baseline(ctx, table, N, k_pool, v_pool, q, gpu_out, seconds: float = 10.0):
    """Time the CPU restatement (oracle/) of the decode call on the host cores, on the same inputs as layer 0,
    and return (baseline dict, max-abs error of the GPU output against it)."""
    import numpy as np
    import torch

    import oracle as O

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    kp = k_pool.view(torch.int16).cpu().numpy().view(np.uint16)
    vp = v_pool.view(torch.int16).cpu().numpy().view(np.uint16)
    qn = q.view(torch.int16).cpu().numpy().view(np.uint16)
    runs, t0 = [], time.perf_counter()
    out32 = None
    while True:
        s = time.perf_counter()
        _, out32 = O.paged_decode(qn, O.DTYPE_BF16, kp, vp, O.DTYPE_BF16, table, ctx, threads=threads)
        runs.append(time.perf_counter() - s)
        if time.perf_counter() - t0 > seconds and len(runs) >= 3:
            break
    t = float(np.median(runs))
    # the same call on one core (two runs, after the threaded ones)
    one = []
    for _ in range(2):
        s = time.perf_counter()
        O.paged_decode(qn, O.DTYPE_BF16, kp, vp, O.DTYPE_BF16, table, ctx, threads=1)
        one.append(time.perf_counter() - s)
    t1 = float(min(one))
    got = gpu_out.float().cpu().numpy().reshape(out32.shape)
    err = float(np.abs(got - out32).max())
    tbs = decode_bytes(ctx) / t / 1e12
    return ({"value": tbs, "unit": "TB/s", "cores": threads, "kind": "port",
             "tokens_per_s": len(ctx) / t, "ms_per_call": t * 1e3,
             "single_core": {"value": decode_bytes(ctx) / t1 / 1e12, "ms_per_call": t1 * 1e3},
             "sample": f"full layer-0 decode call of the workload (B={len(ctx)}, {int(sum(ctx)) + len(ctx)} "
                       f"context tokens), median of {len(runs)} runs on {threads} threads; single_core: best of "
                       f"2 runs on 1 thread"}, err)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=4, help="independent KV pools rotated over the steps")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget (0 = skip)")
    ap.add_argument("--no-bulk", action="store_true", help="skip the bulk-append measurement")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other BASELINE configurations (C3, C4, C5 int8/fp8) and the rope+append figures")
    ap.add_argument("--configs", default="all",
                    help="comma-separated subset of C3,C5_int8,C5_fp8,C4,prefill_variants,decode_d256,decode_d96,"
                         "decode_d112,decode_d80,decode_f32,rope_append,C2_decode_step_host (default all)")
    ap.add_argument("--skip-c2", action="store_true",
                    help="skip the C2 steps, the device copy and the CPU baseline (profiling other configurations "
                         "alone); the headline fields are then null")
    ap.add_argument("--lib", default=None,
                    help="time another build of libffkv.so (for example one made from an earlier commit in a git "
                         "worktree) instead of firefly_amd/libffkv.so")
    ap.add_argument("--timeline", action="store_true",
                    help="with --lib pointing at a timeline build (python -m firefly_amd.build --define "
                         "FFKV_DECODE_TIMELINE=1 --out PATH): report when the split-K decode kernel's waves start and "
                         "end over a few C2 decode calls, then exit")
    ap.add_argument("--timeline-out", default=None,
                    help="with --timeline: also save every call's per-wave start and end ticks to this .npz file")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 1 GiB device-to-device copy (a kernel of known read/write bytes, used to "
                         "scale rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the paged KV-cache path shards by sequence or KV head with no "
              "exchange, and every box in this build has one GPU; run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import firefly_amd as ff

    if args.lib is not None:
        from pathlib import Path

        ff.LIB_PATH = Path(args.lib).resolve()
        ff.lib = ff._load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    ctx_np, table_np, N = workload()
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    ctx = torch.from_numpy(ctx_np).to(dev)
    table = torch.from_numpy(table_np).to(dev)
    shape = (N, BLOCK, HKV, D)
    pools = [(torch.randn(shape, generator=gen, device=dev, dtype=torch.bfloat16),
              torch.randn(shape, generator=gen, device=dev, dtype=torch.bfloat16)) for _ in range(args.layers)]
    q = torch.randn((B, 1, HQ, D), generator=gen, device=dev, dtype=torch.bfloat16)
    k_new = torch.randn((B, 1, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
    v_new = torch.randn((B, 1, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
    out = torch.empty((B, 1, HQ * D), device=dev, dtype=torch.bfloat16)
    max_ctx = int(ctx_np.max()) + 1
    ws = ff.decode_workspace(B, HQ, D, table_np.shape[1], max_ctx, device=dev)

    def step(i):
        kp, vp = pools[i % args.layers]
        # the decode step as one call: append 1 token per row, then decode (ffkv_append_paged_decode)
        ff.append_paged_attention(k_new, v_new, q, kp, vp, table, ctx, out=out, max_context_len=max_ctx,
                                  workspace=ws, stream=stream)

    def step_separate(i):
        kp, vp = pools[i % args.layers]
        ff.append_kv_cache(k_new, v_new, kp, vp, table, ctx, stream=stream)
        ff.paged_attention(q, kp, vp, table, ctx, out=out, max_context_len=max_ctx, workspace=ws, stream=stream)

    if args.timeline:
        print(json.dumps(decode_timeline(ff, torch, np, stream, lambda i: ff.paged_attention(
            q, pools[i % args.layers][0], pools[i % args.layers][1], table, ctx, out=out, max_context_len=max_ctx,
            workspace=ws, stream=stream), out_path=args.timeline_out)))
        return 0

    if args.calibrate_copy:
        src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    ms_per_step = ms_per_step_separate = app_ms = dec_ms = achieved = None
    dbytes = decode_bytes(ctx_np)
    abytes = append_bytes(B, B)
    if not args.skip_c2:
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()

        # Timed region: K steps, wall clock, synchronized on both sides.
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(i)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_per_step = wall / args.steps * 1e3

        # The same steps as two calls (ffkv_append, then ffkv_paged_decode), as the reference's model issues them.
        for i in range(args.warmup):
            step_separate(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            step_separate(i)
        torch.cuda.synchronize()
        ms_per_step_separate = (time.perf_counter() - t0) / args.steps * 1e3

        # Per-call durations with HIP events on the launch stream (same loop, events around each call).
        n_ev = args.steps
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n_ev)]
        for i in range(n_ev):
            kp, vp = pools[i % args.layers]
            ev[i][0].record(stream)
            ff.append_kv_cache(k_new, v_new, kp, vp, table, ctx, stream=stream)
            ev[i][1].record(stream)
            ff.paged_attention(q, kp, vp, table, ctx, out=out, max_context_len=max_ctx, workspace=ws, stream=stream)
            ev[i][2].record(stream)
        torch.cuda.synchronize()
        app_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in ev]))
        dec_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in ev]))

        achieved = dbytes / (dec_ms * 1e-3) / 1e12

    # Bulk append: 64 sequences x 2048 new tokens into fresh pages (the KV-append GB/s figure).
    bulk = None
    if not args.no_bulk:
        S = 2048
        nb = S // BLOCK
        rng = np.random.default_rng(SEED + 1)
        bt = torch.from_numpy(rng.permutation(B * nb).astype(np.int32).reshape(B, nb)).to(dev)
        ks = torch.randn((B, S, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        vs = torch.randn((B, S, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        kc = torch.empty((B * nb, BLOCK, HKV, D), device=dev, dtype=torch.bfloat16)
        vc = torch.empty_like(kc)
        zero = torch.zeros(B, dtype=torch.int32, device=dev)
        for _ in range(3):
            ff.append_kv_cache(ks, vs, kc, vc, bt, zero, stream=stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        e0.record(stream)
        for _ in range(reps):
            ff.append_kv_cache(ks, vs, kc, vc, bt, zero, stream=stream)
        e1.record(stream)
        torch.cuda.synchronize()
        bms = e0.elapsed_time(e1) / reps
        bulk = {"tokens": B * S, "bytes": append_bytes(B * S, B), "ms": bms,
                "GB_per_s": append_bytes(B * S, B) / (bms * 1e-3) / 1e9}
        del ks, vs, kc, vc

    # The other BASELINE configurations (decode attention alone unless stated), measured the same way.
    configs = None
    if not args.no_configs:
        rng = np.random.default_rng(SEED + 3)
        makers = {
            "C3": lambda: decode_config(ff, torch, dev, stream, "C3 Qwen2.5-7B layer: Hq28/Hkv4/D128 bf16, B=8, "
                                        "ctx 32768", 8, 28, 4, 128, [32768] * 8, seed=3),
            "C5_int8": lambda: decode_config(ff, torch, dev, stream, "C5 int8 KV (per-token scales): Hq32/Hkv8/D128, "
                                             "B=256, ctx U[1024,8192]", 256, 32, 8, 128, c5_ctx[0], kv="i8", seed=5),
            "C5_fp8": lambda: decode_config(ff, torch, dev, stream, "C5 fp8 e4m3 KV (per-head scales): Hq32/Hkv8/D128, "
                                            "B=256, ctx U[1024,8192]", 256, 32, 8, 128, c5_ctx[1], kv="fp8", seed=6),
            "C4": lambda: c4_config(ff, torch, dev, stream),
            "prefill_variants": lambda: prefill_variants_config(ff, torch, dev, stream),
            "decode_d256": lambda: decode_config(ff, torch, dev, stream, "head_dim 256 decode: Hq16/Hkv4/D256 bf16, "
                                                 "B=64, ctx U[512,4096]", 64, 16, 4, 256, d256_ctx, seed=8),
            "decode_d96": lambda: decode_config(ff, torch, dev, stream, "head_dim 96 decode (matrix cores): "
                                                "Hq32/Hkv8/D96 bf16, B=64, ctx U[512,4096]", 64, 32, 8, 96, d96_ctx,
                                                seed=9),
            "decode_d112": lambda: decode_config(ff, torch, dev, stream, "head_dim 112 decode (matrix cores, a last "
                                                 "k-step of 16 dims): Hq32/Hkv8/D112 bf16, B=64, ctx U[512,4096]",
                                                 64, 32, 8, 112, d112_ctx, seed=10),
            "decode_d80": lambda: decode_config(ff, torch, dev, stream, "head_dim 80 decode (matrix cores, a last "
                                                "k-step of 16 dims): Hq32/Hkv8/D80 bf16, B=64, ctx U[512,4096]",
                                                64, 32, 8, 80, d80_ctx, seed=11),
            "decode_f32": lambda: decode_config(ff, torch, dev, stream, "fp32 pages (the vector kernel): "
                                                "Hq32/Hkv8/D128, q bf16, B=64, ctx U[512,4096]",
                                                64, 32, 8, 128, f32_ctx, kv="f32", seed=12),
            "rope_append": lambda: rope_append_config(ff, torch, dev, stream),
            "C2_decode_step_host": lambda: decode_step_config(ff, torch, dev, stream, ctx_np, table_np, N, pools, q,
                                                              k_new, v_new, out, ws, max_ctx),
        }
        c5_ctx = [rng.integers(1024, 8193, size=256), rng.integers(1024, 8193, size=256)]
        d256_ctx = rng.integers(512, 4097, size=64)
        d96_ctx = rng.integers(512, 4097, size=64)
        d112_ctx = rng.integers(512, 4097, size=64)
        d80_ctx = rng.integers(512, 4097, size=64)
        f32_ctx = rng.integers(512, 4097, size=64)
        want = list(makers) if args.configs == "all" else [x for x in args.configs.split(",") if x]
        unknown = [x for x in want if x not in makers]
        if unknown:
            print(f"unknown --configs entries {unknown}; choose from {list(makers)}", file=sys.stderr)
            return 2
        configs = {name: makers[name]() for name in want}

    copy_rate = None if args.skip_c2 else device_copy_rate(torch, dev, stream)
    read_rate = None if args.skip_c2 else read_stream_rate(torch, dev, stream, call_bytes=dbytes)

    # Layer-0 output for the parity figure and the CPU baseline on the same inputs.
    kp0, vp0 = pools[0]
    ff.paged_attention(q, kp0, vp0, table, ctx, out=out, max_context_len=max_ctx, workspace=ws, stream=stream)
    torch.cuda.synchronize()
    cpu = None
    err = None
    if args.cpu_seconds > 0 and not args.skip_c2:
        cpu, err = cpu_baseline(ctx_np, table_np, N, kp0, vp0, q, out, args.cpu_seconds)

    traffic, traffic_commit = measured_traffic()

    def per_s(amount, ms, unit):  # amount per second of a duration in ms, in `unit`s (None without the duration)
        return None if ms is None else amount / (ms * 1e-3) / unit

    line = {
        "metric": "paged decode-attn HBM TB/s (% of peak) + tokens/s; KV-append GB/s, 1 GPU",
        "value": per_s(dbytes + abytes, ms_per_step, 1e12),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/Q, seeded block-table permutation)",
        "config": {"workload": "C2 Qwen3-8B layer: Hq32/Hkv8/D128 bf16, B=64, ctx U[512,4096], block 16, "
                               "append 1 token + decode per step",
                   "batch": B, "context_tokens": int(ctx_np.sum()) + B, "pool_blocks": N, "layers": args.layers},
        "pct_of_peak": per_s(dbytes + abytes, ms_per_step, HBM_PEAK_TBS * 1e10),
        "decode_tokens_per_s": per_s(B, ms_per_step, 1),
        "decode_tokens_per_s_qwen3_8b_36_layers": per_s(B, ms_per_step, 36),
        "decode_call_ms": dec_ms,
        "step_ms_two_calls": ms_per_step_separate,
        "append_call_us": None if app_ms is None else app_ms * 1e3,
        "append_bulk": bulk,
        "roofline": {"kernel": "ffkv_paged_decode (paged_decode_mfma + paged_decode_mfma_merge)", "bound": "hbm",
                     "achieved": None if achieved is None else achieved * 1e3, "peak": HBM_PEAK_TBS * 1e3,
                     "unit": "GB/s", "frac": None if achieved is None else achieved / HBM_PEAK_TBS,
                     "traffic": traffic, "traffic_measured_at_commit": traffic_commit,
                     "algorithmic_bytes": dbytes},
        "device_copy": copy_rate,
        "read_stream": read_rate,
        "decode_call_vs_read_stream": (None if read_rate is None or achieved is None else
                                         achieved / read_rate["TB_per_s"]),
        "decode_call_vs_read_at_call_size": (None if read_rate is None or achieved is None
                                             or read_rate["at_call_size"] is None else
                                             achieved / read_rate["at_call_size"]["TB_per_s"]),
        "other_configs": configs,
        "cpu_baseline": cpu,
        "parity_max_abs_err_vs_cpu": err,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
