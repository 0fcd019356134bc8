"""Writes the golden fixtures of tests/golden/ by running the REFERENCE
implementation, compiled from its own sources by oracle/Makefile into
oracle/_ref/libvlrf_ref.so (this container only; the GPU box never runs it).

Inputs are this repo's seeded synthetic data (vlrf_amd.formats): projection
weights N(0, 0.02) quantized to Q8_0 and decoded back to f32 -- exactly what
the reference runs after its GGUF converter dequantizes (convert_gguf.py:
233-263) -- norm weights 1, seeded prompt ids.  The reference's own
TransformerModel (Q8_0 KV cache, RMSNorm, RoPE, SwiGLU, GQA) then does what
TransformerModel::generate does (transformer.hpp:439-547): one prefill
forward over the prompt, then greedy decode steps that start from the last
prompt id.

    python tests/golden/gen_golden.py [--only tiny|llama1b]

Fixtures (JSON): config, seed, prompt recipe, generated ids, and per-step
top-2 logit margins (how close each greedy choice was to a tie).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from vlrf_amd import formats as F  # noqa: E402


def run_reference(cfg, seed, n_prompt, n_steps, norm_std=0.0, log=print):
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libvlrf_ref.so is missing: run `make -C oracle` with the "
                         "reference tree present")
    t0 = time.time()
    w = F.make_f32_weights(cfg, seed, norm_std=norm_std)
    log(f"  weights generated in {time.time() - t0:.1f}s")
    h = R.ref_model_create(cfg["vocab_size"], cfg["d_model"], cfg["d_ff"], cfg["n_heads"],
                           cfg["n_kv_heads"], cfg["n_layers"], cfg["max_seq_len"], cfg["norm_eps"],
                           cfg["rope_theta"])
    try:
        for k, v in w.items():
            R.ref_model_set_tensor(h, k.encode(), v, v.shape[0] if v.ndim == 2 else 0, v.shape[-1])
        R.ref_model_bind(h)
        prompt = F.tokens(seed, "golden.prompt", n_prompt, cfg["vocab_size"])
        logits = np.zeros(cfg["vocab_size"], np.float32)
        t0 = time.time()
        R.ref_model_forward(h, prompt, n_prompt, logits.ctypes.data)
        log(f"  prefill of {n_prompt} tokens: {time.time() - t0:.1f}s")
        ids, margins = [], []
        last = int(prompt[-1])
        t0 = time.time()
        for step in range(n_steps):
            last = R.ref_model_forward(h, np.array([last], np.int32), 1, logits.ctypes.data)
            top2 = np.sort(logits)[-2:]
            ids.append(int(last))
            margins.append(float(top2[1] - top2[0]))
            if step % 16 == 15:
                log(f"  step {step + 1}/{n_steps} ({time.time() - t0:.1f}s)")
        return prompt, ids, margins
    finally:
        R.ref_model_destroy(h)


def write(name, cfg, seed, n_prompt, n_steps, norm_std, prompt, ids, margins):
    out = {
        "source": "reference TransformerModel compiled from /root/reference (oracle/_ref)",
        "config": {k: v for k, v in cfg.items()},
        "seed": seed,
        "norm_std": norm_std,
        "prompt": {"recipe": "vlrf_amd.formats.tokens(seed, 'golden.prompt', n, vocab)",
                   "n": n_prompt, "first": [int(t) for t in prompt[:8]]},
        "generated_ids": ids,
        "top2_margins": margins,
    }
    path = os.path.join(HERE, name)
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=["tiny", "llama1b"], default=None)
    a = ap.parse_args()
    if a.only in (None, "tiny"):
        cfg = F.tiny(F.DT_Q8_0, n_layers=3, max_seq_len=200)
        p, ids, m = run_reference(cfg, 41, 60, 128, norm_std=0.1)
        write("tiny_q8_stream.json", cfg, 41, 60, 128, 0.1, p, ids, m)
    if a.only in (None, "llama1b"):
        cfg = F.llama_1b(max_seq_len=2048 + 128)
        p, ids, m = run_reference(cfg, 1234, 2048, 128)
        write("llama1b_q8_stream.json", cfg, 1234, 2048, 128, 0.0, p, ids, m)


if __name__ == "__main__":
    main()
