"""ctypes front end to oracle/sched_driver.cpp, built over this repository's scheduler (libsched_driver_ffkv.so)
or over the reference's own sources (oracle/_ref/libref_sched.so, only where /root/reference was mounted at build
time).  Scenario runners return plain Python data so two builds can be compared with ==."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

ORACLE = Path(__file__).resolve().parent.parent / "oracle"
MINE = ORACLE / "libsched_driver_ffkv.so"
REF = ORACLE / "_ref" / "libref_sched.so"

_I = ctypes.c_int
_P = ctypes.c_void_p
_IP = ctypes.POINTER(ctypes.c_int)


def load(path: Path):
    lib = ctypes.CDLL(str(path))
    sig = {
        "sd_create": (_P, [_I, _I, _I]), "sd_create_policy": (_P, [_I, _I, _I, _I]), "sd_destroy": (None, [_P]),
        "sd_add": (None, [_P, _I, _IP, _I, _I]),
        "sd_request": (_I, [_P, _I, _IP, _I]), "sd_engine_step": (_I, [_P, _IP, _I]), "sd_unfinished": (_I, [_P]),
        "sd_pool_create": (_P, [_I]), "sd_pool_destroy": (None, [_P]), "sd_alloc": (_I, [_P, _I, _IP]),
        "sd_free": (None, [_P, _IP, _I]), "sd_free_count": (_I, [_P]),
        "sd_match": (_I, [_P, _IP, _I, _IP, _I, _IP, _IP]), "sd_release": (None, [_P, _I]),
        "sd_insert": (None, [_P, _IP, _I, _IP, _I]), "sd_evict": (_I, [_P, _I]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _arr(xs):
    a = (ctypes.c_int * max(1, len(xs)))(*xs)
    return a


class Pool:
    """BlockAllocator + RadixTree without a scheduler."""

    def __init__(self, lib, total_blocks: int):
        self.lib = lib
        self.h = lib.sd_pool_create(total_blocks)

    def close(self):
        self.lib.sd_pool_destroy(self.h)

    def alloc(self, n: int):
        out = (ctypes.c_int * max(1, n))()
        ok = self.lib.sd_alloc(self.h, n, out)
        return list(out[:n]) if ok else None

    def free(self, blocks):
        self.lib.sd_free(self.h, _arr(blocks), len(blocks))

    def free_count(self) -> int:
        return self.lib.sd_free_count(self.h)

    def match(self, tokens):
        cap = len(tokens) // 16 + 2
        out = (ctypes.c_int * cap)()
        mt, nb = ctypes.c_int(0), ctypes.c_int(0)
        handle = self.lib.sd_match(self.h, _arr(tokens), len(tokens), out, cap, ctypes.byref(mt), ctypes.byref(nb))
        assert handle >= 0
        return handle, list(out[:nb.value]), mt.value

    def release(self, handle: int):
        self.lib.sd_release(self.h, handle)

    def insert(self, tokens, blocks):
        self.lib.sd_insert(self.h, _arr(tokens), len(tokens), _arr(blocks), len(blocks))

    def evict(self, n: int) -> int:
        return self.lib.sd_evict(self.h, n)


def run_pool_script(lib, total_blocks: int, ops):
    """Run [(op, args...)] on a fresh pool; returns the list of every op's result."""
    p = Pool(lib, total_blocks)
    res = []
    try:
        for op, *args in ops:
            if op == "alloc":
                res.append(p.alloc(*args))
            elif op == "free":
                p.free(*args)
                res.append(p.free_count())
            elif op == "match":
                h, blocks, mt = p.match(*args)
                res.append([h, blocks, mt])
            elif op == "release":
                p.release(*args)
                res.append(None)
            elif op == "insert":
                p.insert(*args)
                res.append(p.free_count())
            elif op == "evict":
                res.append([p.evict(*args), p.free_count()])
            else:
                raise ValueError(op)
    finally:
        p.close()
    return res


def parse_batch(v):
    n, i, reqs = v[0], 1, []
    for _ in range(n):
        rid, ctx, gen, nb = v[i:i + 4]
        reqs.append((rid, ctx, gen, list(v[i + 4:i + 4 + nb])))
        i += 4 + nb
    return reqs


def run_serving(lib, total_blocks: int, max_batch: int, chunk: int, arrivals, max_steps: int = 2000,
                per_chunk: bool = False):
    """arrivals: {step: [(id, tokens, max_tokens), ...]}.  Emulated engine loop; returns the scheduled batches
    (request id, context_len, generated count, block table) of every step.  per_chunk selects
    PrefillBlocks::PerChunk (this repository's build only); otherwise the reference's rule."""
    h = lib.sd_create_policy(total_blocks, max_batch, chunk, 1 if per_chunk else 0)
    assert h, "this build has no PerChunk policy"
    buf = (ctypes.c_int * (1 << 20))()
    trace = []
    try:
        for step in range(max_steps):
            for rid, tokens, max_tokens in arrivals.get(step, []):
                lib.sd_add(h, rid, _arr(tokens), len(tokens), max_tokens)
            n = lib.sd_engine_step(h, buf, len(buf))
            assert n >= 0
            trace.append(parse_batch(list(buf[:n])))
            if step > max(arrivals) and not lib.sd_unfinished(h):
                break
    finally:
        lib.sd_destroy(h)
    return trace


def shared_prefix_workload(seed: int, n_req: int, prefix_len: int, suffix_lo: int, suffix_hi: int,
                           gen_lo: int, gen_hi: int, n_prefixes: int = 2, spread: int = 3):
    """Requests sharing one of a few prompt prefixes (radix-cache hits), arriving over the first steps."""
    rng = np.random.default_rng(seed)
    prefixes = [list(rng.integers(1, 50000, size=prefix_len)) for _ in range(n_prefixes)]
    arrivals = {}
    for rid in range(n_req):
        pre = prefixes[int(rng.integers(0, n_prefixes))]
        cut = int(rng.integers(prefix_len // 2, prefix_len + 1))
        suffix = list(rng.integers(1, 50000, size=int(rng.integers(suffix_lo, suffix_hi + 1))))
        tokens = [int(t) for t in pre[:cut] + suffix]
        arrivals.setdefault(int(rng.integers(0, spread * n_req)), []).append(
            (rid, tokens, int(rng.integers(gen_lo, gen_hi + 1))))
    return arrivals
