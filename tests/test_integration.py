"""The engine-side adapters (vlrf_amd/integration/: HipBackend : IBackend and
HipDecoder) compiled against the reference engine's own headers, as a
maintainer would include them, into oracle/_ref/hip_integration (built by
oracle/Makefile where the reference tree is present; the prebuilt binary
travels with the tree).  The driver compares HipBackend's attention and gemm
with float64 / CpuBackend results and HipDecoder::generate with the
reference TransformerModel::generate on a tiny Q8_0 model."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "oracle", "_ref", "hip_integration")


def run(args, timeout):
    if not os.path.exists(DRIVER):
        pytest.skip("oracle/_ref/hip_integration not built (needs the reference tree)")
    p = subprocess.run([DRIVER] + args, capture_output=True, text=True, timeout=timeout)
    print(p.stdout, p.stderr, flush=True)
    return p


def test_adapter_cpu_fallbacks_against_reference_types():
    """No device used: HipBackend's CPU paths, including attention with
    T != ctx where the reference's default sdp_attention is wrong."""
    p = run(["--cpu"], 120)
    assert p.returncode == 0, p.stdout
    assert "SKIP decode" in p.stdout and "FAIL" not in p.stdout


@pytest.mark.gpu
def test_adapter_on_device_matches_reference_engine():
    print("[case] hip_integration driver on device", flush=True)
    p = run([], 300)
    assert p.returncode == 0, p.stdout
    for kv in ("f32", "f16", "q8_0"):
        assert f"PASS decode: HipDecoder::generate == TransformerModel::generate (64 greedy steps, KV {kv})" \
            in p.stdout, p.stdout
