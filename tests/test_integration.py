"""The engine-side adapters (vlrf_amd/integration/: HipBackend : IBackend and
HipDecoder) compiled against the reference engine's own headers, as a
maintainer would include them, into oracle/_ref/hip_integration (built by
oracle/Makefile where the reference tree is present; the prebuilt binary
travels with the tree).  The driver compares HipBackend's attention and gemm
with float64 / CpuBackend results and HipDecoder::generate with the
reference TransformerModel::generate on a tiny model: per KV cache dtype, per
weight origin (Q8_0 / Q4_0 blocks or plain f32, which picks the device
dtype), and at each way generation stops (EOS, max_seq_len, on_token, empty
prompt): token ids, tokens_generated and hit_eos."""
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
    want = [f"64 greedy steps, KV {kv}" for kv in ("f32", "f16", "q8_0")]
    want += ["48 greedy steps, Q4_0 weights", "48 greedy steps, F32 weights", "reached",
             "max_new_tokens 500 > max_seq_len 160 - 40", "empty prompt (from bos_token_id)",
             "on_token stops after 7"]
    passed = [ln for ln in p.stdout.splitlines()
              if ln.startswith("PASS decode: HipDecoder::generate == TransformerModel::generate, ")]
    for w in want:
        assert any(w in ln for ln in passed), (w, p.stdout)
    for w in ("Q8_0-derived weights kept as Q8_0 blocks", "Q4_0-derived weights uploaded as Q4_0 / LM head Q4_0",
              "F32-derived weights uploaded as F32 / LM head F32", "forcing Q8_0 on f32 weights is refused"):
        assert "PASS decode: " + w in p.stdout, (w, p.stdout)
    assert "FAIL" not in p.stdout
