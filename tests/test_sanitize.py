"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

- tests/cpp/sched_sanitize.cpp drives BlockAllocator / RadixTree / Scheduler (firefly_amd/csrc/host/) through seeded
  serving workloads with both PrefillBlocks policies and through random allocator / prefix-cache operations, built
  here with g++ -fsanitize=address,undefined (no GPU code is involved).
- tests/cpp/abi_sanitize.cpp runs the C ABI's argument validation (invalid sizes, dtypes, pointers, workspaces):
  firefly_amd/csrc/capi.cpp is compiled with host-side sanitizers only (-Xarch_host) and linked with the library's
  kernel objects from firefly_amd/_build; every call returns before any device work.
Any sanitizer report aborts the run."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _build(tmp_path, name, sources):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / name
    cmd = [gxx, "-std=c++20", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           f"-I{ROOT / 'include'}", *map(str, sources), "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return exe


def test_scheduler_radix_allocator_under_asan_ubsan(tmp_path):
    exe = _build(tmp_path, "sched_sanitize", [ROOT / "tests" / "cpp" / "sched_sanitize.cpp",
                                               ROOT / "firefly_amd" / "csrc" / "host" / "scheduler.cpp",
                                               ROOT / "firefly_amd" / "csrc" / "host" / "radix_tree.cpp"])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().endswith("OK")


def test_c_abi_validation_under_asan_ubsan(tmp_path):
    gxx, hipcc = shutil.which("g++"), "/opt/rocm/bin/hipcc"
    build = ROOT / "firefly_amd" / "_build"
    kernels = [build / f"{n}.hip.o" for n in ("kv_append", "paged_decode", "paged_decode_mfma", "paged_decode_pfx",
                                               "paged_prefill_dma", "rope_append")]
    if gxx is None or not Path(hipcc).exists() or not all(k.exists() for k in kernels):
        pytest.skip("needs g++, hipcc and the library's objects (python firefly_amd/build.py)")
    inc = [f"-I{ROOT / 'include'}", f"-I{ROOT / 'firefly_amd' / 'csrc'}"]
    capi = tmp_path / "capi_san.o"
    main = tmp_path / "abi_main.o"
    exe = tmp_path / "abi_sanitize"
    steps = [
        [hipcc, "-x", "hip", "--offload-arch=gfx950", "-std=c++20", "-O1", "-g", "-Xarch_host", "-fsanitize=address",
         "-Xarch_host", "-fsanitize=undefined", *inc, "-c", str(ROOT / "firefly_amd" / "csrc" / "capi.cpp"), "-o",
         str(capi)],
        [gxx, "-std=c++20", "-O1", "-g", "-fsanitize=address,undefined", *inc, "-c",
         str(ROOT / "tests" / "cpp" / "abi_sanitize.cpp"), "-o", str(main)],
        # link: host sanitizer runtimes only (-fno-gpu-sanitize on the same line)
        [hipcc, "--offload-arch=gfx950", "-fno-gpu-sanitize", "-fsanitize=address,undefined", str(main), str(capi),
         *map(str, kernels), "-o", str(exe)],
    ]
    for cmd in steps:
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, " ".join(cmd) + "\n" + res.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().endswith("OK")
