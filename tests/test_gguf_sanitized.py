"""The GGUF reader under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only): tests/fuzz/gguf_fuzz.cpp is built with g++ -fsanitize against
vx_gguf.cpp and vx_layout.cpp and runs thousands of mutations of two seed
files (the hand-assembled fixture and a writer-made file with every
metadata type, strings and arrays, and three tensors). Any sanitizer report
or a query failing on a file that opened ends the run non-zero."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from tests import gguf_writer as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _tiny() -> bytes:
    out = bytearray()
    with open(os.path.join(ROOT, "tests", "golden", "gguf_tiny.hex")) as f:
        for line in f:
            out += bytes(int(b, 16) for b in line.split("#", 1)[0].split())
    return bytes(out)


def _rich() -> bytes:
    rng = np.random.default_rng(1)
    kv = [("general.architecture", W.STRING, "llama"), ("x.f", W.FLOAT32, 1.5), ("x.b", W.BOOL, True),
          ("x.i64", W.INT64, -7), ("x.arr", W.ARRAY, (W.STRING, ["a", "bc", ""])),
          ("x.nums", W.ARRAY, (W.INT32, [1, -2, 3])), ("x.nest", W.ARRAY, (W.ARRAY, [(W.INT8, [1]), (W.STRING, ["q"])]))]
    tensors = [("w.q4", [64, 3], 2, rng.integers(0, 256, 3 * 2 * 18, dtype=np.uint8).tobytes()),
               ("w.q8", [32, 2], 8, rng.integers(0, 256, 2 * 34, dtype=np.uint8).tobytes()),
               ("w.f32", [8, 2], 0, rng.standard_normal(16).astype(np.float32).tobytes())]
    return W.build(kv, tensors, alignment=64)


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx or not os.path.exists(os.path.join(ROCM, "lib", "libamdhip64.so")):
        pytest.skip("needs g++ and the HIP runtime library")
    d = tmp_path_factory.mktemp("fuzz")
    exe = str(d / "gguf_fuzz")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           f"-I{ROOT}/include", f"-I{ROOT}/vortx_amd/csrc", f"-I{ROCM}/include",
           f"{ROOT}/tests/fuzz/gguf_fuzz.cpp", f"{ROOT}/vortx_amd/csrc/vx_gguf.cpp",
           f"{ROOT}/vortx_amd/csrc/vx_layout.cpp", f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib",
           "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "sanitize" in r.stderr and "cannot find" in r.stderr:
        pytest.skip("sanitizer runtime not installed")
    assert r.returncode == 0, r.stderr[-3000:]
    return exe, d


@pytest.mark.parametrize("seed_name,iters", [("tiny", 4000), ("rich", 4000)])
def test_gguf_mutations_under_asan_ubsan(fuzzer, seed_name, iters):
    exe, d = fuzzer
    seed = d / f"{seed_name}.gguf"
    seed.write_bytes(_tiny() if seed_name == "tiny" else _rich())
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, str(seed), str(iters), "12345", str(d / f"{seed_name}.scratch")],
                       capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "iterations" in r.stdout
