"""The NFW parser under AddressSanitizer and UndefinedBehaviorSanitizer (host
code only, on the CPU): tests/fuzz/nfw_fuzz.cpp opens every truncation and
thousands of random byte mutations of valid version 1, 2 and 3 files and
reads every tensor it accepts, in full and into too-small buffers.  Any
out-of-bounds access, leak or undefined arithmetic (a size product of a
hostile header, say) fails the run."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from vlrf_amd import formats as F
from vlrf_amd import nfw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _seeds(d):
    rng = np.random.default_rng(3)
    paths = [os.path.join(d, f"s{i}.nfw") for i in range(4)]
    nfw.write_nfw(paths[0], {"a": rng.standard_normal((3, 5)).astype(np.float32),
                             "b.bias": np.zeros(7, np.float32)}, version=1)
    nfw.write_nfw(paths[1], {"w": rng.standard_normal((4, 8)).astype(np.float16),
                             "n": rng.standard_normal(9).astype(np.float32)}, version=2)
    nfw.write_nfw(paths[2], {
        "q": nfw.Blocks(nfw.Q8_0, (2, 64), F.quantize(rng.standard_normal(128).astype(np.float32), F.DT_Q8_0)),
        "p": nfw.Blocks(nfw.Q4_0, (3, 32), F.quantize(rng.standard_normal(96).astype(np.float32), F.DT_Q4_0)),
        "h": rng.standard_normal((2, 3)).astype(np.float16), "f": np.ones(4, np.float32)})
    t = {}
    for i in range(4):
        t[f"layers.{i}.attn.q_proj.weight"] = nfw.Blocks(
            nfw.Q8_0, (4, 64), F.quantize(rng.standard_normal(256).astype(np.float32), F.DT_Q8_0))
        t[f"layers.{i}.ln1.weight"] = rng.standard_normal(64).astype(np.float16 if i % 2 else np.float32)
    nfw.write_nfw(paths[3], t)
    return paths


def test_nfw_parser_fuzz_under_sanitizers(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path / "nfw_fuzz")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
    cmd = [gxx, "-std=c++17", "-O1", "-g", *san, "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "fuzz", "nfw_fuzz.cpp"),
           os.path.join(ROOT, "vlrf_amd", "csrc", "host", "nfw.cpp"),
           os.path.join(ROOT, "vlrf_amd", "csrc", "host", "format.cpp"), "-o", exe, "-pthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "asan" in r.stderr.lower():
        pytest.skip("sanitizer runtime not available: " + r.stderr[-300:])
    assert r.returncode == 0, r.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([exe, str(tmp_path / "fuzz.nfw"), "4000", *_seeds(str(tmp_path))],
                       capture_output=True, text=True, env=env, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-3000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-3000:]
    assert "opened" in out
