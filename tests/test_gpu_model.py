"""GPU parity of the whole decode step (TransformerModel::forward/generate,
transformer.hpp:335-547) on a small Llama-style model with the same structure
as the 1.1B benchmark model (RMSNorm, RoPE, GQA, SwiGLU, Q8_0 KV cache).

The oracle runs the reference algorithm on the decoded f32 weights and does a
real prefill (M = prompt length GEMMs, causal attention), as
TransformerModel::generate does; the GPU feeds the prompt one token at a time
through the decode step.  Both then decode greedily starting from the last
prompt id (the reference feeds it twice, transformer.hpp:448-482)."""
import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu


def _models(ctx, orc, cfg, seed):
    m = V.Model(ctx, cfg)
    w = F.load_model(m, seed, want_f32=True, norm_std=0.1)
    om = orc.Model(cfg, w, n_threads=4)
    return m, om, w


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
def test_tiny_greedy_stream(ctx, orc, dtype):
    cfg = F.tiny(dtype, n_layers=3, max_seq_len=128)
    m, om, _ = _models(ctx, orc, cfg, 21)
    prompt = F.tokens(21, "prompt", 40, cfg["vocab_size"])
    gpu = m.generate(prompt, 64)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(64):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref
    assert m.used == om.used == 40 + 64


def test_tiny_logits_teacher_forced(ctx, orc):
    """Per-step logits against the oracle on the same token feed."""
    cfg = F.tiny(V.DT_Q8_0, n_layers=2, max_seq_len=96)
    m, om, _ = _models(ctx, orc, cfg, 22)
    ids = F.tokens(22, "feed", 70, cfg["vocab_size"])
    m.reset()
    om.reset()
    worst = 0.0
    for t in ids:
        g_next, g_logits = m.step(int(t), want_logits=True)
        o_next, o_logits = om.forward([int(t)], want_logits=True)
        worst = max(worst, rel_err(g_logits, o_logits))
        assert g_next == int(np.argmax(g_logits))
    assert worst <= 1e-3, worst
    # KV caches: same codes up to rare +/-1 flips where a K/V value sits on a
    # rounding boundary (f32 GEMV order differs from the AVX2 reference order).
    kv_gpu = V.KVCache  # noqa: F841  (the model's cache is internal; compare via logits)


def test_generate_matches_step_loop(ctx, orc):
    """Device token feedback (replayed graph) == host-driven step loop."""
    cfg = F.tiny(V.DT_Q8_0, n_layers=2, max_seq_len=80)
    m, _, _ = _models(ctx, orc, cfg, 23)
    prompt = F.tokens(23, "p", 10, cfg["vocab_size"])
    a = m.generate(prompt, 50)
    m.reset()
    m.prefill(prompt)
    last, b = int(prompt[-1]), []
    for _ in range(50):
        last = m.step(last)
        b.append(last)
    assert list(a) == b


def test_model_capacity_and_errors(ctx, orc):
    cfg = F.tiny(V.DT_Q8_0, n_layers=1, max_seq_len=8)
    m, _, _ = _models(ctx, orc, cfg, 24)
    m.reset()
    m.prefill(np.arange(6, dtype=np.int32))
    with pytest.raises(V.HipError) as e:
        m.generate_ids(1, 3)             # 6 + 3 > 8
    assert e.value.rc == -4
    with pytest.raises(V.HipError):
        m.step(cfg["vocab_size"])        # token id out of range
    m.generate_ids(1, 2)
    assert m.used == 8


def test_unset_weights_rejected(ctx):
    m = V.Model(ctx, F.tiny(V.DT_Q8_0, n_layers=1))
    with pytest.raises(V.HipError):
        m.step(0)


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
def test_argmax_ties_take_the_lowest_index(ctx, dtype):
    """sampler::argmax (transformer.hpp:43-47) returns the first index of the
    maximum.  An LM head whose rows repeat with period 37 over a 32000-token
    vocabulary gives every logit 864-865 bit-identical copies spread over all
    the LM head's workgroups and waves (whose per-workgroup maxima the step's
    argmax reduces); each step's token must be the lowest index of the
    maximum."""
    cfg = dict(F.tiny(dtype, n_layers=1, max_seq_len=64), vocab_size=32000)
    m = V.Model(ctx, cfg)
    F.load_model(m, 31, norm_std=0.1)
    D, nv, P = cfg["d_model"], cfg["vocab_size"], 37
    rows = np.random.default_rng(31).normal(0.0, 0.5, (P, D)).astype(np.float32)
    w = np.tile(rows, (nv // P + 1, 1))[:nv]
    m.set_weight("lm_head.weight", F.quantize(w.reshape(-1), dtype), dtype, nv, D)
    m.reset()
    for t in F.tokens(31, "tie", 12, nv):
        print(f"[case] argmax ties, token {int(t)}", flush=True)
        g_next, gl = m.step(int(t), want_logits=True)
        k = int(np.argmax(gl))
        assert k < P and gl[k + P] == gl[k] and gl[nv - P + (k - nv % P) % P] == gl[k]
        assert g_next == k


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
def test_llama8b_layer_decode(ctx, orc, dtype):
    """The decode step at the 8B shape (hidden 4096, 32/8 heads, d_head 128,
    FFN 14336: the down projection's 14336-wide rows take the wide M = 1
    GEMV), one layer, vocabulary 256: greedy stream identical to the
    oracle's and teacher-forced logits within 1e-3."""
    cfg = F.llama8b_layer(dtype, max_seq_len=96, n_layers=1, vocab_size=256)
    print(f"[case] 8B-shape layer decode dtype={dtype}", flush=True)
    m, om, _ = _models(ctx, orc, cfg, 23)
    prompt = F.tokens(23, "prompt", 24, cfg["vocab_size"])
    gpu = m.generate(prompt, 16)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(16):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref
    m.reset()
    om.reset()
    worst = 0.0
    for t in F.tokens(23, "feed", 12, cfg["vocab_size"]):
        _, gl = m.step(int(t), want_logits=True)
        _, ol = om.forward([int(t)], want_logits=True)
        worst = max(worst, rel_err(gl, ol))
    print(f"  teacher-forced logits: worst rel err {worst:.2e}", flush=True)
    assert worst <= 1e-3, worst


@pytest.mark.parametrize("n_heads,n_kv,dtype", [(8, 2, V.DT_Q8_0), (8, 8, V.DT_Q8_0), (8, 2, V.DT_Q4_0)])
def test_head_dim_128_chunked_cache(ctx, orc, n_heads, n_kv, dtype):
    """d_head 128 over a cache of three 512-row chunks (the chunked decode
    attention with the token's key as its own partial, merged by the O
    projection): a 1100-token prompt fed through the decode step, then a
    greedy stream identical to the oracle's and teacher-forced logits within
    1e-3 at contexts past the second chunk boundary."""
    cfg = dict(vocab_size=256, d_model=128 * n_heads, d_ff=2048, n_heads=n_heads, n_kv_heads=n_kv, n_layers=2,
               max_seq_len=1400, norm_eps=1e-5, rope_theta=10000.0, weight_dtype=dtype)
    print(f"[case] d_head 128 chunked cache heads={n_heads}/{n_kv} dtype={dtype}", flush=True)
    m, om, _ = _models(ctx, orc, cfg, 29)
    prompt = F.tokens(29, "prompt", 1100, cfg["vocab_size"])
    gpu = m.generate(prompt, 24)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(24):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref
    worst = 0.0
    for t in F.tokens(29, "feed", 8, cfg["vocab_size"]):
        _, gl = m.step(int(t), want_logits=True)
        _, ol = om.forward([int(t)], want_logits=True)
        worst = max(worst, rel_err(gl, ol))
    print(f"  teacher-forced logits at ctx {m.used}: worst rel err {worst:.2e}", flush=True)
    assert worst <= 1e-3, worst


def test_time_launches_runs_the_same_steps(ctx, orc):
    """vlrf_hip_model_time_launches (each launch timed by its own events)
    decodes the same greedy stream as generate and labels every launch: one
    QKV (+ attention) launch, O, gate/up and down per layer, one LM head and
    one argmax per step, all with positive durations."""
    cfg = F.tiny(V.DT_Q8_0, n_layers=3, max_seq_len=96)
    m, _, _ = _models(ctx, orc, cfg, 25)
    prompt = F.tokens(25, "p", 12, cfg["vocab_size"])
    ref = m.generate(prompt, 20)
    m.reset()
    m.prefill(prompt)
    steps = 20
    kinds = m.time_launches(int(prompt[-1]), steps)
    got = m.read_generated(steps)
    assert list(got) == list(ref)
    assert m.used == 12 + steps
    L = cfg["n_layers"]
    for k in ("o_proj", "gate_up", "down"):
        assert kinds[k][1] == L * steps, (k, kinds[k])
    assert kinds["qkv_attn"][1] == L * steps
    assert kinds["lm_head"][1] == steps and kinds["argmax"][1] == steps
    assert all(us > 0 for us, _ in kinds.values())
    with pytest.raises(V.HipError):
        m.time_launches(int(prompt[-1]), 96)      # past the cache
