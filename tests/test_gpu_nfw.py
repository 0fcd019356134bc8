"""A GGUF model converted with its Q8_0/Q4_0 blocks passed through
(vlrf_amd.convert_gguf -> NFW v3) and loaded with vlrf_hip_model_load_nfw runs
the same device model as the weights set one by one: identical logits step by
step, and the oracle's greedy stream on the decoded weights (what the
reference runs after its converter decodes the same file,
convert_gguf.py:175-263)."""
import numpy as np
import pytest

import vlrf_amd as V
from vlrf_amd import convert_gguf as CG
from vlrf_amd import formats as F

import gguf_fixture as G

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("wdt", [V.DT_Q8_0, V.DT_Q4_0])
def test_loaded_nfw_model_matches_set_weights_and_oracle(ctx, orc, tmp_path, wdt):
    print(f"[case] load_nfw dtype={wdt}", flush=True)
    cfg = F.tiny(wdt, n_layers=2, max_seq_len=96)
    src = tmp_path / "m.gguf"
    made = G.llama_gguf(str(src), cfg, seed=31, embed_q8=True, fused_qkv=True, f16_norms=True)
    path, _ = CG.convert(src, tmp_path / "out", log=lambda *a: None)

    a = V.Model(ctx, cfg)
    n = a.load_nfw(path)
    assert n == len(made)                      # every weight set, the zero biases dropped
    b = V.Model(ctx, cfg)
    specs = {name: (rows, cols, kind) for name, rows, cols, kind in F.tensor_specs(cfg)}
    for name, (raw, dec) in made.items():
        rows, cols, kind = specs[name]
        if kind == "proj":
            b.set_weight(name, np.frombuffer(raw, np.uint8), wdt, rows, cols)
        else:
            b.set_weight(name, dec, V.DT_F32, rows, cols)

    ids = F.tokens(31, "nfw.feed", 24, cfg["vocab_size"])
    for t in ids:
        na, la = a.step(int(t), want_logits=True)
        nb, lb = b.step(int(t), want_logits=True)
        assert na == nb and np.array_equal(la, lb)

    w = {name: dec for name, (_, dec) in made.items()}
    om = orc.Model(cfg, w, n_threads=4)
    prompt = F.tokens(31, "nfw.prompt", 30, cfg["vocab_size"])
    gpu = a.generate(prompt, 32)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(32):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref


def test_load_nfw_rejects_f32_projection_for_block_model(ctx, tmp_path):
    from vlrf_amd import nfw
    cfg = F.tiny(V.DT_Q8_0, n_layers=1, max_seq_len=32)
    p = tmp_path / "f.nfw"
    nfw.write_nfw(p, {"layers.0.attn.q_proj.weight": np.zeros((cfg["d_model"], cfg["d_model"]), np.float32)})
    m = V.Model(ctx, cfg)
    with pytest.raises(V.HipError, match="block type"):
        m.load_nfw(p)
    nfw.write_nfw(p, {"layers.0.attn.q_proj.bias": np.ones(cfg["d_model"], np.float32)})
    with pytest.raises(V.HipError, match="non-zero bias"):
        m.load_nfw(p)
