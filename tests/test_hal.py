"""hal::Result / hal::Status / hal::Graph against the reference engine's call shapes.

tests/cpp/engine_calls.cpp copies the shapes of the engine's decode-graph capture and replay (src/engine.cc:137-166,
:329-333: `auto result = graph.capture(stream, lambda)`, `if (!result) ... result.error().description()`,
`[[maybe_unused]] auto _ = graph.launch(stream)`, graphs moved into a map) and checks Result<T>, Status and
FIREFLY_TRY.  It is compiled here against include/firefly and linked with the library; without a GPU the capture
fails inside the HIP runtime and the error must arrive described, with a GPU (the gpu-marked run) the capture and
replay must succeed.  The executable is built with the library (firefly_amd/build.py); the CPU test rebuilds it
to prove the headers compile."""

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "cpp" / "engine_calls.cpp"
LIB_DIR = ROOT / "firefly_amd"


PREBUILT = ROOT / "tests" / "cpp" / "engine_calls.bin"


@pytest.fixture(scope="module")
def engine_calls(tmp_path_factory):
    if not (LIB_DIR / "libffkv.so").exists():
        pytest.skip("firefly_amd/libffkv.so not built")
    exe = tmp_path_factory.mktemp("hal") / "engine_calls"
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++20", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(SRC), "-o",
           str(exe), f"-L{LIB_DIR}", "-lffkv", f"-Wl,-rpath,{LIB_DIR}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, f"engine call shapes do not compile against include/firefly:\n{res.stderr}"
    return exe


def test_engine_call_shapes_compile_and_report_errors(engine_calls):
    res = subprocess.run([str(engine_calls)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().startswith("OK")
    if "(no gpu)" in res.stdout:
        assert "Failed to capture graph for batch size 8: " in res.stderr
        assert "Graph Launch failed: Graph: nothing captured to launch" in res.stderr


@pytest.mark.gpu
def test_engine_call_shapes_capture_and_replay_on_gpu(gpu):
    if not PREBUILT.exists():
        pytest.skip("tests/cpp/engine_calls.bin not built (python firefly_amd/build.py)")
    print("case engine_calls.bin capture + replay", flush=True)
    res = subprocess.run([str(PREBUILT)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "OK (gpu)" in res.stdout


def test_model_and_engine_kernel_call_shapes_compile():
    """Every firefly::kernels call of the reference's QwenModel::forward (src/model/qwen_model.cu:98-191) and
    engine (src/engine.cc:136-148, :267), the off-path operators included, compiles against include/firefly
    (tests/cpp/model_calls.cpp: compiled, not linked; those operators are defined by the caller's kernel files)."""
    src = ROOT / "tests" / "cpp" / "model_calls.cpp"
    cmd = ["/opt/rocm/bin/hipcc", "-std=c++20", "-Wall", "-Werror", "-Wno-unused-command-line-argument",
           "-fsyntax-only", f"-I{ROOT / 'include'}", str(src)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, f"model / engine call shapes do not compile against include/firefly:\n{res.stderr}"
