"""Block-table producers (BlockAllocator, RadixTree, Scheduler) against the reference's own implementation.

This repository's C++ (include/firefly, firefly_amd/csrc/host) and the reference's sources (src/scheduler.cc,
src/radix_tree.cc) are driven through the same oracle/sched_driver.cpp.  Pins:
  * golden results recorded from the reference build (tests/golden/sched_golden.json: pool scripts in full,
    serving traces as digests of every scheduled block table / context length / generated count),
  * the live reference build when it exists (oracle/_ref, only where /root/reference is mounted) on further
    seeded workloads,
  * closed forms: LIFO allocation order and block-aligned prefix matches.
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import sched_util as su

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "sched_golden.json").read_text())


@pytest.fixture(scope="module")
def mine():
    if not su.MINE.exists():
        pytest.skip(f"{su.MINE} not built (python __graft_entry__.py)")
    return su.load(su.MINE)


@pytest.fixture(scope="module")
def ref():
    if not su.REF.exists():
        pytest.skip("reference scheduler build absent (oracle/_ref needs /root/reference at build time)")
    return su.load(su.REF)


def _digest(obj):
    return hashlib.sha256(json.dumps(obj, separators=(",", ":")).encode()).hexdigest()


def _jsonable(x):
    return json.loads(json.dumps(x))


@pytest.mark.parametrize("name", sorted(GOLDEN["pool"]))
def test_pool_scripts_match_reference_golden(mine, name):
    g = GOLDEN["pool"][name]
    ops = [tuple(op) for op in g["ops"]]
    assert _jsonable(su.run_pool_script(mine, g["total_blocks"], ops)) == g["results"]


@pytest.mark.parametrize("name", sorted(GOLDEN["serving"]))
def test_serving_trace_matches_reference_golden(mine, name):
    g = GOLDEN["serving"][name]
    arrivals = {int(k): [tuple(r) for r in v] for k, v in g["arrivals"].items()}
    trace = su.run_serving(mine, g["total_blocks"], g["max_batch"], g["chunk"], arrivals)
    assert len(trace) == g["steps"]
    assert sum(len(s) for s in trace) == g["scheduled_requests"]
    assert _digest(_jsonable(trace)) == g["trace_sha256"]


@pytest.mark.parametrize("seed", range(6))
def test_serving_matches_live_reference(mine, ref, seed):
    rng = np.random.default_rng(100 + seed)
    total = int(rng.integers(48, 400))
    arrivals = su.shared_prefix_workload(200 + seed, int(rng.integers(6, 24)), int(rng.integers(16, 200)),
                                         1, int(rng.integers(8, 120)), 1, int(rng.integers(2, 20)),
                                         n_prefixes=int(rng.integers(1, 4)))
    args = (total, int(rng.integers(2, 12)), int(rng.choice([16, 32, 48, 256])), arrivals)
    assert su.run_serving(mine, *args, max_steps=600) == su.run_serving(ref, *args, max_steps=600)


@pytest.mark.parametrize("seed", range(6))
def test_random_pool_ops_match_live_reference(mine, ref, seed):
    """Random inserts / matches / releases / evictions / allocations, including eviction-order ties."""
    rng = np.random.default_rng(seed)
    base = [list(rng.integers(0, 4, size=int(rng.integers(8, 90)))) for _ in range(6)]
    ops, live, next_block = [], [], 0
    for _ in range(80):
        r = rng.random()
        seq = [int(t) for t in base[int(rng.integers(0, len(base)))][:int(rng.integers(1, 90))]]
        if r < 0.3:
            nb = (len(seq) + 15) // 16
            ops.append(("insert", seq, list(range(next_block, next_block + nb))))
            next_block += nb
        elif r < 0.6:
            ops.append(("match", seq))
            live.append(len([o for o in ops if o[0] == "match"]) - 1)
        elif r < 0.75 and live:
            ops.append(("release", live.pop(int(rng.integers(0, len(live))))))
        elif r < 0.9:
            ops.append(("evict", int(rng.integers(1, 6))))
        else:
            ops.append(("alloc", int(rng.integers(1, 8))))
    assert su.run_pool_script(mine, 64, ops) == su.run_pool_script(ref, 64, ops)


def test_lifo_closed_form(mine):
    p = su.Pool(mine, 100)
    try:
        assert p.alloc(5) == [99, 98, 97, 96, 95]
        p.free([97, 42])
        assert p.alloc(3) == [42, 97, 94]
        assert p.alloc(100) is None and p.free_count() == 94
    finally:
        p.close()


def test_prefix_matches_are_block_aligned(mine):
    rng = np.random.default_rng(7)
    p = su.Pool(mine, 1000)
    try:
        seqs = []
        for i in range(20):
            s = [int(t) for t in rng.integers(0, 3, size=int(rng.integers(1, 120)))]
            p.insert(s, list(range(i * 10, i * 10 + (len(s) + 15) // 16)))
            seqs.append(s)
        for s in seqs:
            _, blocks, mt = p.match(s + [7, 7])
            assert mt % 16 == 0 and mt <= len(s)
            assert len(blocks) == mt // 16
    finally:
        p.close()


def _positions_covered(trace, prompts, chunk):
    """For every scheduled entry, (KV positions its step writes, positions its block table covers)."""
    rows = []
    for batch in trace:
        for rid, ctx, gen, blocks in batch:
            if gen == 0:  # prefill: the next chunk of the prompt
                end = ctx + min(len(prompts[rid]) - ctx, chunk)
            else:         # decode: the newest token goes to position ctx
                end = ctx + 1
            rows.append((rid, gen, end, 16 * len(blocks)))
    return rows


def test_long_prompt_chunks_hold_their_blocks_per_chunk(mine):
    """A 600-token prompt prefilled in chunks of 256: under PrefillBlocks::PerChunk every chunk's positions have
    blocks before it runs.  Under the reference's rule the second chunk (positions 256..511) runs with 17 blocks,
    as src/scheduler.cc:88-99 gives a running request one block per step; the reference build does the same."""
    prompt = list(range(1, 601))
    arrivals = {0: [(0, prompt, 4)]}
    fixed = su.run_serving(mine, 200, 4, 256, arrivals, per_chunk=True)
    rows = _positions_covered(fixed, {0: prompt}, 256)
    assert [r[2] for r in rows if r[1] == 0] == [256, 512, 600]
    assert all(end <= have for _, _, end, have in rows)
    assert [have for _, gen, _, have in rows if gen == 0] == [256, 512, 608]

    compat = su.run_serving(mine, 200, 4, 256, arrivals)
    short = [(end, have) for _, gen, end, have in _positions_covered(compat, {0: prompt}, 256) if end > have]
    assert short and short[0] == (512, 17 * 16)


def test_long_prompt_reference_rule_matches_reference(mine, ref):
    prompt = list(range(1, 601))
    arrivals = {0: [(0, prompt, 4)], 1: [(1, prompt[:300] + [7] * 50, 3)]}
    assert su.run_serving(mine, 200, 4, 256, arrivals) == su.run_serving(ref, 200, 4, 256, arrivals)


@pytest.mark.parametrize("seed", range(4))
def test_per_chunk_policy_equals_reference_when_prompts_fit_one_chunk(mine, seed):
    """The policies differ only for requests that need more than one prefill chunk."""
    rng = np.random.default_rng(300 + seed)
    arrivals = su.shared_prefix_workload(400 + seed, 12, int(rng.integers(16, 120)), 1, 60, 1, 12,
                                         n_prefixes=2)
    args = (int(rng.integers(40, 200)), int(rng.integers(2, 8)), 256, arrivals)
    assert su.run_serving(mine, *args, per_chunk=True) == su.run_serving(mine, *args)


@pytest.mark.parametrize("seed", range(4))
def test_per_chunk_policy_covers_every_step(mine, seed):
    """Random serving workloads with long prompts and small chunks: with PerChunk every scheduled step has blocks
    for every position it writes, and the allocator never hands out a block twice."""
    rng = np.random.default_rng(500 + seed)
    chunk = int(rng.choice([16, 32, 48, 64]))
    arrivals = su.shared_prefix_workload(600 + seed, 10, int(rng.integers(40, 160)), 10, 200, 1, 10,
                                         n_prefixes=2)
    prompts = {rid: toks for reqs in arrivals.values() for rid, toks, _ in reqs}
    trace = su.run_serving(mine, 2000, 6, chunk, arrivals, max_steps=3000, per_chunk=True)
    rows = _positions_covered(trace, prompts, chunk)
    assert rows and all(end <= have for _, _, end, have in rows)
    for batch in trace:
        # prefix blocks are shared between requests; a request's own blocks never repeat within its table
        for _, _, _, blocks in batch:
            assert len(set(blocks)) == len(blocks)


def test_per_chunk_long_prompts_do_not_wait_on_each_other(mine):
    """Two 600-token prompts (38 blocks each) over a 40-block pool with chunks of 256 tokens.  If both were
    admitted on their first chunk (16 blocks each), each would then wait forever for the 16 blocks of its second
    chunk (8 free, nothing to evict).  Under PerChunk a prompt is admitted only when the free and evictable
    blocks cover all of it beside what the running prompts still need: the second waits until the first has
    finished and its blocks can be evicted, and both complete, every step holding blocks for what it writes."""
    rng = np.random.default_rng(11)
    prompts = {rid: [int(t) for t in rng.integers(1, 50000, size=600)] for rid in (0, 1)}
    arrivals = {0: [(0, prompts[0], 4), (1, prompts[1], 4)]}
    trace = su.run_serving(mine, 40, 4, 256, arrivals, max_steps=100, per_chunk=True)
    assert len(trace) < 100, "the scheduler stopped making progress"
    done = {rid: max(gen for batch in trace for r, _, gen, _ in batch if r == rid) for rid in (0, 1)}
    assert done == {0: 3, 1: 3}  # the last scheduled step of each decodes its 4th token
    rows = _positions_covered(trace, prompts, 256)
    assert all(end <= have for _, _, end, have in rows)
    first_of_1 = next(i for i, batch in enumerate(trace) if any(r == 1 for r, *_ in batch))
    last_of_0 = max(i for i, batch in enumerate(trace) if any(r == 0 for r, *_ in batch))
    assert first_of_1 > last_of_0


def test_per_chunk_admits_beside_a_running_long_prompt(mine):
    """The reservation counts what a running prompt still needs, not more: a short prompt that fits beside it is
    admitted while the long one is still prefilling."""
    rng = np.random.default_rng(12)
    prompts = {0: [int(t) for t in rng.integers(1, 50000, size=600)],
               1: [int(t) for t in rng.integers(1, 50000, size=40)]}
    arrivals = {0: [(0, prompts[0], 2)], 1: [(1, prompts[1], 2)]}
    trace = su.run_serving(mine, 44, 4, 256, arrivals, max_steps=100, per_chunk=True)
    assert len(trace) < 100
    # step 1: request 0 runs its second chunk and request 1 (3 blocks) is admitted beside it (38 + 3 <= 44)
    assert sorted(r for r, *_ in trace[1]) == [0, 1]
