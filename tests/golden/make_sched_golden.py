"""Write tests/golden/sched_golden.json from the reference's own BlockAllocator / RadixTree / Scheduler.

Runs the scenarios of tests/test_sched.py through oracle/sched_driver.cpp compiled over the reference sources
(oracle/_ref/libref_sched.so, built by `make -C oracle ref` where /root/reference is mounted) and records, per
scenario, its inputs and the results: pool scripts in full, serving traces (the scheduled block tables, context
lengths and generated counts of every step) as a SHA-256 digest of their JSON plus a few summary counts.

Run: ``python tests/golden/make_sched_golden.py``.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

import sched_util as su  # noqa: E402


def digest(obj) -> str:
    return hashlib.sha256(json.dumps(obj, separators=(",", ":")).encode()).hexdigest()


def pool_scripts():
    a = list(range(1000, 1040))        # 40 tokens = 2 full blocks + 8
    b = a[:20] + list(range(2000, 2030))
    c = a[:32] + list(range(3000, 3016))
    return {
        "lifo": (10, [("alloc", 3), ("alloc", 2), ("free", [8]), ("alloc", 2), ("free", [1, 2]), ("alloc", 10),
                      ("alloc", 5), ("free", [0]), ("alloc", 1)]),
        "radix_split_and_evict": (12, [
            ("alloc", 3), ("insert", a, [11, 10, 9]),
            ("match", a), ("match", b), ("match", a[:10]), ("match", c),
            ("alloc", 9), ("alloc", 1), ("release", 0), ("release", 1), ("alloc", 1), ("evict", 5),
            ("release", 3), ("evict", 5), ("alloc", 2),
            ("insert", b, [4, 5, 6, 7]), ("match", b + [7, 7, 7]), ("evict", 100)]),
        "radix_unaligned_insert": (16, [
            ("insert", list(range(50)), [0, 1, 2, 3]), ("insert", list(range(37)) + [99] * 20, [0, 1, 2, 4, 5]),
            ("match", list(range(60))), ("match", list(range(37)) + [99] * 20), ("release", 0), ("release", 1),
            ("evict", 1), ("evict", 1), ("evict", 1), ("match", list(range(60)))]),
    }


def serving_scenarios():
    return {
        "small_shared_prefix": dict(total_blocks=64, max_batch=4, chunk=32,
                                    arrivals=su.shared_prefix_workload(1, 10, 48, 4, 40, 1, 12, spread=2)),
        "pool_pressure_evictions": dict(total_blocks=40, max_batch=8, chunk=64,
                                        arrivals=su.shared_prefix_workload(2, 16, 64, 8, 96, 2, 24, spread=2)),
        "prefix_heavy_c4_like": dict(total_blocks=420, max_batch=16, chunk=64,
                                     arrivals=su.shared_prefix_workload(3, 32, 256, 16, 128, 1, 8, n_prefixes=1,
                                                                        spread=4)),
    }


def run_all(lib):
    out = {"pool": {}, "serving": {}}
    for name, (n, ops) in pool_scripts().items():
        out["pool"][name] = {"total_blocks": n, "ops": ops, "results": su.run_pool_script(lib, n, ops)}
    for name, sc in serving_scenarios().items():
        trace = su.run_serving(lib, sc["total_blocks"], sc["max_batch"], sc["chunk"], sc["arrivals"])
        out["serving"][name] = {
            "total_blocks": sc["total_blocks"], "max_batch": sc["max_batch"], "chunk": sc["chunk"],
            "arrivals": {str(k): v for k, v in sc["arrivals"].items()},
            "trace_sha256": digest(trace), "steps": len(trace),
            "scheduled_requests": sum(len(s) for s in trace)}
    return out


def main() -> None:
    if not su.REF.exists():
        raise SystemExit(f"{su.REF} is not built (make -C oracle ref, needs the reference sources)")
    rec = run_all(su.load(su.REF))
    path = HERE / "sched_golden.json"
    path.write_text(json.dumps(rec, separators=(",", ":")) + "\n")
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
