"""Build the gfx950 shared library ``firefly_amd/libffkv.so`` (and the CPU checker under ``oracle/``).

Every HIP and C++ source under ``firefly_amd/csrc`` is compiled with hipcc for gfx950 only and linked into one
shared library whose exported C ABI is declared in ``include/ffkv.h``.  Objects go to ``firefly_amd/_build``;
the library is written in-tree so it travels with the repository snapshot.

Usage: ``python firefly_amd/build.py [--jobs N] [--no-oracle]`` (run as a script: importing the package needs
the library this builds).
"""

from __future__ import annotations

import argparse
import hashlib
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libffkv.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]
# Device code: gfx950 only; packed fp32 math stays off (hipcc's host pass warns that it does not know it).
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")) + list((CSRC / "host").glob("*.cpp")))


def _compile(src: Path, build_dir: Path = BUILD, defines: tuple[str, ...] = ()) -> Path:
    obj = build_dir / (src.name + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE, *(f"-D{d}" for d in defines), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
    else:
        # host C++: only the C ABI (ffkv.h) and the firefly:: API (include/firefly) are exported
        cmd[1:1] = ["-fvisibility=hidden", "-fvisibility-inlines-hidden"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build_library(jobs: int = 8, defines: tuple[str, ...] = (), out: Path | None = None) -> Path:
    """Compile every source and link ``libffkv.so``.  Always rebuilds.

    ``defines`` (``NAME=VALUE`` strings) set the kernels' compile-time switches (``FFKV_*`` macros) for a variant
    build, which is linked to ``out`` (its objects under ``_build/variant-<hash of the switches>``) and leaves
    ``libffkv.so`` alone;
    ``bench.py --lib`` measures such a build beside the shipped one."""
    if defines and out is None:
        raise ValueError("a variant build (defines) needs its own output path")
    # each set of switches compiles into a folder of its own, so variant builds can run side by side
    tag = hashlib.sha1(" ".join(sorted(defines)).encode()).hexdigest()[:12]
    build_dir = BUILD / f"variant-{tag}" if defines else BUILD
    build_dir.mkdir(parents=True, exist_ok=True)
    target = Path(out) if out is not None else LIB
    target.parent.mkdir(parents=True, exist_ok=True)
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda src: _compile(src, build_dir, tuple(defines)), srcs))
    tmp = target.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, target)
    return target


def build_test_shims() -> None:
    """Test-only helpers linked against libffkv.so: the C++-API shims under tests/cpp/ (kernels_api_shim.cpp for
    tests/test_gpu_cxx_api.py, decode_step_shim.cpp for tests/test_gpu_decode_step.py) and engine_calls.bin
    (tests/test_hal.py)."""
    for name in ("kernels_api_shim", "decode_step_shim"):
        src = ROOT / "tests" / "cpp" / f"{name}.cpp"
        if not src.exists():
            continue
        out = ROOT / "tests" / "cpp" / f"lib{name}.so"
        cmd = [HIPCC, "-O2", "-std=c++20", "-fPIC", "-shared", f"-I{ROOT / 'include'}", str(src), "-o", str(out),
               f"-L{PKG}", "-lffkv", "-Wl,-rpath,$ORIGIN/../../firefly_amd"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"test shim build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # the reference engine's hal::Graph / hal::Result call shapes as an executable (tests/test_hal.py)
    src = ROOT / "tests" / "cpp" / "engine_calls.cpp"
    out = ROOT / "tests" / "cpp" / "engine_calls.bin"
    cmd = [HIPCC, "-O1", "-std=c++20", f"-I{ROOT / 'include'}", str(src), "-o", str(out), f"-L{PKG}", "-lffkv",
           "-Wl,-rpath,$ORIGIN/../../firefly_amd"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"test executable build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build_bench_helpers() -> Path:
    """bench.py's measurement helpers (csrc/bench/*.hip, e.g. the read-only stream) into libffkv_bench.so, apart
    from the product library."""
    out = PKG / "libffkv_bench.so"
    srcs = sorted((CSRC / "bench").glob("*.hip"))
    cmd = [HIPCC, "-x", "hip", *COMMON, *DEVICE, "-shared", *map(str, srcs), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"bench helper build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return out


def build_oracle() -> None:
    """Build the CPU checker (and, where the reference sources exist, the compiled reference host code)."""
    make = shutil.which("make") or "make"
    subprocess.run([make, "-C", str(ROOT / "oracle"), "-j4"], check=True, capture_output=True, text=True)
    if Path("/root/reference/src/scheduler.cc").exists():
        subprocess.run([make, "-C", str(ROOT / "oracle"), "ref"], check=True, capture_output=True, text=True)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--no-oracle", action="store_true")
    ap.add_argument("--define", action="append", default=[], metavar="NAME=VALUE",
                    help="compile-time switch for a variant build (repeatable; needs --out)")
    ap.add_argument("--out", default=None, help="output path of a variant build")
    args = ap.parse_args(argv)
    if args.define:
        lib = build_library(args.jobs, tuple(args.define), Path(args.out) if args.out else None)
        print(f"built {lib}")
        return 0
    lib = build_library(args.jobs)
    build_test_shims()
    build_bench_helpers()
    print(f"built {lib}")
    if not args.no_oracle:
        build_oracle()
        print("built oracle")
    return 0


if __name__ == "__main__":
    sys.exit(main())
