"""The engine's decode step with this library (src/engine.cc:279-351): DecodeBatch packs the scheduled requests'
context lengths and block tables into pinned staging and uploads them, the table at its live width only, in one
copy; one hal::Graph,
captured once, replays append + PagedAttention for every layer on those device buffers while the batch changes
(contexts grow, rows cross into new blocks, a request leaves, another joins).  Every step's pages are compared
bit-exact and its outputs within tolerance with the CPU checker run on the same tables
(tests/cpp/decode_step_shim.cpp)."""

import ctypes
import os
from pathlib import Path

import numpy as np
import pytest

import cases
import gpu_util as gu
import oracle as O

pytestmark = pytest.mark.gpu

SHIM = Path(__file__).resolve().parent / "cpp" / "libdecode_step_shim.so"


@pytest.fixture(scope="module")
def shim(ff):
    if not SHIM.exists():
        pytest.skip("tests/cpp/libdecode_step_shim.so not built")
    lib = ctypes.CDLL(str(SHIM), mode=os.RTLD_NOW)
    vp, i, ip = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)
    pp = ctypes.POINTER(ctypes.c_void_p)
    for name, res, args in [("dss_create", vp, [i, i]), ("dss_destroy", None, [vp]),
                            ("dss_error", ctypes.c_char_p, [vp]), ("dss_pack", i, [vp, i, ip, ip, ip]),
                            ("dss_upload", i, [vp, vp]), ("dss_last_upload_bytes", ctypes.c_longlong, [vp]),
                            ("dss_host_table", ip, [vp]), ("dss_host_ctx", ip, [vp]),
                            ("dss_step", i, [vp, i, i, pp, pp, pp, pp, pp, pp, i, i, i, i, i, vp]),
                            ("dss_launch", i, [vp, vp])]:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _arr(xs):
    return (ctypes.c_int * max(1, len(xs)))(*[int(x) for x in xs])


def test_graph_replayed_decode_steps_match_checker(shim, gpu):
    import torch

    L, CAP, STRIDE, Hq, Hkv, D, N = 2, 8, 64, 16, 4, 128, 600
    rng = np.random.default_rng(11)
    free = list(rng.permutation(N))
    reqs = []  # [context_len, block list]

    def new_req(ctx):
        nb = (ctx + 16) // 16  # blocks for ctx cached tokens plus this step's token
        reqs.append([ctx, [int(free.pop()) for _ in range(nb)]])

    for c in rng.integers(10, 300, size=6):
        new_req(int(c))
    # pools per layer, the CPU copies follow every step
    pools = []
    for _ in range(L):
        kf = rng.standard_normal((N, 16, Hkv, D), dtype=np.float32) * np.float32(0.3)
        vf = rng.standard_normal((N, 16, Hkv, D), dtype=np.float32)
        pools.append([cases.encode(kf, O.DTYPE_BF16), cases.encode(vf, O.DTYPE_BF16)])
    dk = [gu.to_dev(p[0], O.DTYPE_BF16, gpu) for p in pools]
    dv = [gu.to_dev(p[1], O.DTYPE_BF16, gpu) for p in pools]
    dq = [torch.empty((CAP, 1, Hq, D), dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    dkn = [torch.empty((CAP, 1, Hkv, D), dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    dvn = [torch.empty((CAP, 1, Hkv, D), dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    dout = [torch.empty((CAP, 1, Hq * D), dtype=torch.bfloat16, device=gpu) for _ in range(L)]
    P = lambda ts: (ctypes.c_void_p * L)(*[t.data_ptr() for t in ts])  # noqa: E731
    side = torch.cuda.Stream()  # capture needs a stream other than the legacy default one
    stream = side.cuda_stream

    h = shim.dss_create(CAP, STRIDE)
    assert h
    try:
        for step in range(5):
            if step == 2:
                new_req(int(rng.integers(20, 200)))          # a request joins
            if step == 3:
                reqs.pop(1)                                  # a request finishes
            ctx = [r[0] for r in reqs]
            nblk = [len(r[1]) for r in reqs]
            blocks = [b for r in reqs for b in r[1]]
            width = shim.dss_pack(h, len(reqs), _arr(ctx), _arr(nblk), _arr(blocks))
            assert width == max(nblk)
            table = np.ctypeslib.as_array(shim.dss_host_table(h), shape=(CAP * STRIDE,)).reshape(CAP, STRIDE).copy()
            ctxs = np.ctypeslib.as_array(shim.dss_host_ctx(h), shape=(CAP,)).copy()
            assert list(ctxs[:len(reqs)]) == ctx and not ctxs[len(reqs):].any()
            assert (table[len(reqs):, :width] == -1).all()
            assert shim.dss_upload(h, stream) == 0
            # one copy: the context lengths' row and the table rows, each as wide as the live width (at least the
            # CAP lengths), against the lengths plus the whole stride in the reference's two copies
            assert shim.dss_last_upload_bytes(h) == (1 + CAP) * max(width, CAP) * 4 < CAP * 4 + CAP * STRIDE * 4
            # this step's inputs
            qs, kns, vns = [], [], []
            for l in range(L):
                qs.append(cases.encode(rng.standard_normal((CAP, 1, Hq, D), dtype=np.float32), O.DTYPE_BF16))
                kns.append(cases.encode(rng.standard_normal((CAP, 1, Hkv, D), dtype=np.float32) * np.float32(0.3),
                                        O.DTYPE_BF16))
                vns.append(cases.encode(rng.standard_normal((CAP, 1, Hkv, D), dtype=np.float32), O.DTYPE_BF16))
                dq[l].copy_(gu.to_dev(qs[l], O.DTYPE_BF16, gpu))
                dkn[l].copy_(gu.to_dev(kns[l], O.DTYPE_BF16, gpu))
                dvn[l].copy_(gu.to_dev(vns[l], O.DTYPE_BF16, gpu))
            torch.cuda.synchronize()  # inputs copied (current stream) before the step runs on `side`
            print(f"case decode step {step} rows={len(reqs)} width={width}", flush=True)
            if step == 0:
                rc = shim.dss_step(h, 1, L, P(dq), P(dkn), P(dvn), P(dk), P(dv), P(dout), Hq, Hkv, D, N,
                                   O.DTYPE_BF16, stream)
                assert rc == 0, shim.dss_error(h)
                rc = shim.dss_step(h, 0, L, P(dq), P(dkn), P(dvn), P(dk), P(dv), P(dout), Hq, Hkv, D, N,
                                   O.DTYPE_BF16, stream)  # capture only
                assert rc == 0, shim.dss_error(h)
            else:
                assert shim.dss_launch(h, stream) == 0, shim.dss_error(h)
            torch.cuda.synchronize()
            for l in range(L):
                O.append(kns[l], vns[l], O.DTYPE_BF16, pools[l][0], pools[l][1], O.DTYPE_BF16, table, ctxs)
                _, ref32 = O.paged_decode(qs[l], O.DTYPE_BF16, pools[l][0], pools[l][1], O.DTYPE_BF16, table, ctxs)
                assert np.array_equal(gu.to_host(dk[l], np.uint16), pools[l][0]), f"layer {l} K pages differ"
                assert np.array_equal(gu.to_host(dv[l], np.uint16), pools[l][1]), f"layer {l} V pages differ"
                got = dout[l].float().cpu().numpy().reshape(ref32.shape)
                m = np.maximum(np.abs(got), np.abs(ref32))
                half = 2.0 ** (np.floor(np.log2(np.maximum(m, 2.0 ** -126))) - 8)
                assert float((np.abs(got - ref32) - half).max()) <= 2e-3, f"layer {l} output"
                assert not got[len(reqs):].any()  # padded slots give zeros
            # the engine's bookkeeping: one more cached token, a new block when the next token crosses into it
            for r in reqs:
                r[0] += 1
                if (r[0] + 1 + 15) // 16 > len(r[1]):
                    r[1].append(int(free.pop()))
    finally:
        shim.dss_destroy(h)


def test_graph_survives_workspace_growth(shim, gpu):
    """A graph captured with the thread's cached decode workspace stays valid after a later eager call on the same
    stream needs a larger one: the old buffer is retired, not freed, so the replay neither writes freed memory
    nor disturbs a tensor allocated after the growth (firefly_amd/csrc/host/kernels.cpp)."""
    import torch

    Hq, Hkv, D, N, STRIDE = 32, 8, 128, 6000, 64
    rng = np.random.default_rng(31)
    kf = rng.standard_normal((N, 16, Hkv, D), dtype=np.float32) * np.float32(0.3)
    vf = rng.standard_normal((N, 16, Hkv, D), dtype=np.float32)
    pool_k, pool_v = cases.encode(kf, O.DTYPE_BF16), cases.encode(vf, O.DTYPE_BF16)
    side = torch.cuda.Stream()
    stream = side.cuda_stream
    free = list(rng.permutation(N))
    steps = {}
    try:
        for cap in (2, 64):  # the second step's workspace (more rows) outgrows the first's
            ctx = [int(c) for c in rng.integers(100, 900, size=cap)]
            blocks = [[int(free.pop()) for _ in range((c + 16) // 16)] for c in ctx]
            h = shim.dss_create(cap, STRIDE)
            assert h
            shim.dss_pack(h, cap, _arr(ctx), _arr([len(b) for b in blocks]), _arr([x for b in blocks for x in b]))
            assert shim.dss_upload(h, stream) == 0
            table = np.ctypeslib.as_array(shim.dss_host_table(h), shape=(cap * STRIDE,)).reshape(cap, STRIDE).copy()
            t = dict(h=h, cap=cap, table=table, ctx=np.array(ctx, np.int32),
                     q=cases.encode(rng.standard_normal((cap, 1, Hq, D), dtype=np.float32), O.DTYPE_BF16),
                     kn=cases.encode(rng.standard_normal((cap, 1, Hkv, D), dtype=np.float32), O.DTYPE_BF16),
                     vn=cases.encode(rng.standard_normal((cap, 1, Hkv, D), dtype=np.float32), O.DTYPE_BF16),
                     dk=gu.to_dev(pool_k, O.DTYPE_BF16, gpu), dv=gu.to_dev(pool_v, O.DTYPE_BF16, gpu))
            t["dq"] = gu.to_dev(t["q"], O.DTYPE_BF16, gpu)
            t["dkn"] = gu.to_dev(t["kn"], O.DTYPE_BF16, gpu)
            t["dvn"] = gu.to_dev(t["vn"], O.DTYPE_BF16, gpu)
            t["dout"] = torch.zeros((cap, 1, Hq * D), dtype=torch.bfloat16, device=gpu)
            steps[cap] = t
        torch.cuda.synchronize()

        def args(t):
            one = lambda x: (ctypes.c_void_p * 1)(x.data_ptr())  # noqa: E731
            return (one(t["dq"]), one(t["dkn"]), one(t["dvn"]), one(t["dk"]), one(t["dv"]), one(t["dout"]), Hq,
                    Hkv, D, N, O.DTYPE_BF16, stream)

        small, big = steps[2], steps[64]
        print("case workspace growth: eager + capture at B=2", flush=True)
        assert shim.dss_step(small["h"], 1, 1, *args(small)) == 0, shim.dss_error(small["h"])
        assert shim.dss_step(small["h"], 0, 1, *args(small)) == 0, shim.dss_error(small["h"])
        print("case workspace growth: eager at B=64 on the same stream", flush=True)
        assert shim.dss_step(big["h"], 1, 1, *args(big)) == 0, shim.dss_error(big["h"])
        torch.cuda.synchronize()
        canary = torch.full((64 << 20,), 7, dtype=torch.uint8, device=gpu)  # allocated after the growth
        small["dk"].copy_(gu.to_dev(pool_k, O.DTYPE_BF16, gpu))
        small["dv"].copy_(gu.to_dev(pool_v, O.DTYPE_BF16, gpu))
        small["dout"].zero_()
        torch.cuda.synchronize()
        print("case workspace growth: replay the B=2 graph", flush=True)
        assert shim.dss_launch(small["h"], stream) == 0, shim.dss_error(small["h"])
        torch.cuda.synchronize()
        assert bool((canary == 7).all()), "the replay wrote into memory allocated after the workspace grew"
        for t in (small,):
            hk, hv = pool_k.copy(), pool_v.copy()
            O.append(t["kn"], t["vn"], O.DTYPE_BF16, hk, hv, O.DTYPE_BF16, t["table"], t["ctx"])
            _, ref32 = O.paged_decode(t["q"], O.DTYPE_BF16, hk, hv, O.DTYPE_BF16, t["table"], t["ctx"])
            got = t["dout"].float().cpu().numpy().reshape(ref32.shape)
            m = np.maximum(np.abs(got), np.abs(ref32))
            half = 2.0 ** (np.floor(np.log2(np.maximum(m, 2.0 ** -126))) - 8)
            assert float((np.abs(got - ref32) - half).max()) <= 2e-3
    finally:
        for t in steps.values():
            shim.dss_destroy(t["h"])
