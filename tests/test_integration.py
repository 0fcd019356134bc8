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
    # The opt-in matrix-core prompt pass (bf16 parity class) and the device
    # cache brought back into the engine's KVCache storage.
    for w in ("prefill: the matrix-core pass applies from 64 prompt tokens",
              "prefill: logits after a 100-token prompt on the matrix cores within 1e-2 of the reference",
              "prefill: first generated id == the reference's", "prefill: generation continues",
              "cache: CPU forward over the device's cache rows == the reference's, KV f32",
              "cache: CPU forward over the device's cache rows == the reference's, KV f16",
              "cache: CPU forward over the device's cache rows == the reference's, KV q8_0"):
        assert "PASS " + w in p.stdout, (w, p.stdout)
    assert "FAIL" not in p.stdout


ENGINE = os.path.join(ROOT, "oracle", "_ref", "engine_hip")


def _engine_model(tmp_path):
    """A tiny Llama-style checkpoint as the engine loads it: an NFW v2 file
    (the engine's WeightMap reads versions 1-2: f32 tensors, the projections
    the decoded values of Q8_0 blocks, as the converter leaves them; zero
    attention biases as converted checkpoints carry) with config.json beside
    it."""
    import json
    import numpy as np
    from vlrf_amd import formats as F
    from vlrf_amd import nfw
    cfg = F.tiny(F.DT_Q8_0, n_layers=2, max_seq_len=160)
    tensors = {}
    for name, rows, cols, kind in F.tensor_specs(cfg):
        payload, dec = F.make_tensor(71, name, rows, cols, kind, F.DT_Q8_0, 0.1)
        tensors[name] = dec.reshape(rows, cols) if rows > 1 else dec
    tensors["layers.0.attn.q_proj.bias"] = np.zeros(cfg["d_model"], np.float32)
    path = tmp_path / "model.nfw"
    nfw.write_nfw(path, tensors, version=2)
    conf = {k: cfg[k] for k in ("vocab_size", "d_model", "d_ff", "n_heads", "n_kv_heads", "n_layers", "max_seq_len")}
    conf.update(layer_norm_eps=cfg["norm_eps"], rope_theta=cfg["rope_theta"], pre_norm=True, use_rms_norm=True,
                tie_embeddings=False, pos_embedding="rotary", activation="silu", bos_token_id=1, eos_token_id=2)
    (tmp_path / "config.json").write_text(json.dumps(conf))
    return path


@pytest.mark.gpu
def test_engine_c_api_selects_the_hip_backend(tmp_path):
    """The engine's own C API with the integration patch applied
    (oracle/_ref/engine_hip, built by oracle/Makefile `engine` from the
    reference's src/api/vlrf_api.cpp): vlrf_set_backend(VLRF_BACKEND_HIP) +
    vlrf_generate_ids return the CPU backend's ids (F32 and Q8_0 KV caches,
    and a request past max_seq_len)."""
    if not os.path.exists(ENGINE):
        pytest.skip("oracle/_ref/engine_hip not built (needs the reference tree)")
    print("[case] engine C API with the HIP backend", flush=True)
    p = subprocess.run([ENGINE, str(_engine_model(tmp_path))], capture_output=True, text=True, timeout=300)
    print(p.stdout, p.stderr, flush=True)
    assert p.returncode == 0, p.stdout + p.stderr
    assert p.stdout.count("PASS engine vlrf_generate_ids, HIP backend == CPU backend") == 3, p.stdout
    assert p.stdout.count("PASS engine vlrf_context_length after generate, HIP == CPU") == 3, p.stdout
