"""Greedy token streams against fixtures written by the reference itself
(tests/golden/gen_golden.py runs the reference TransformerModel compiled from
its own sources).  The CPU oracle must reproduce them exactly; the GPU decode
path must produce the identical stream, feeding the prompt one token at a
time through the decode step where the reference runs one prefill forward."""
import json
import os

import numpy as np
import pytest

import oracle
from vlrf_amd import formats as F

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    path = os.path.join(HERE, name)
    if not os.path.exists(path):
        pytest.skip(f"{name} not generated")
    with open(path) as f:
        return json.load(f)


def prompt_of(fx):
    c = fx["config"]
    p = F.tokens(fx["seed"], "golden.prompt", fx["prompt"]["n"], c["vocab_size"])
    assert [int(t) for t in p[:8]] == fx["prompt"]["first"]
    return p


def test_oracle_reproduces_reference_tiny_stream():
    fx = load("tiny_q8_stream.json")
    cfg = fx["config"]
    w = F.make_f32_weights(cfg, fx["seed"], norm_std=fx["norm_std"])
    om = oracle.Model(cfg, w, n_threads=4)
    p = prompt_of(fx)
    om.forward(p)
    last, ids = int(p[-1]), []
    for _ in range(len(fx["generated_ids"])):
        last = om.forward([last])
        ids.append(last)
    assert ids == fx["generated_ids"]


def _gpu_stream(ctx, fx):
    import vlrf_amd as V
    cfg = dict(fx["config"])
    m = V.Model(ctx, cfg)
    F.load_model(m, fx["seed"], norm_std=fx["norm_std"])
    return list(m.generate(prompt_of(fx), len(fx["generated_ids"])))


def _first_divergence(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return i
    return None


@pytest.mark.gpu
def test_gpu_tiny_stream_matches_reference(ctx):
    fx = load("tiny_q8_stream.json")
    assert _gpu_stream(ctx, fx) == fx["generated_ids"]


@pytest.mark.gpu
def test_gpu_llama1b_128_step_stream_matches_reference(ctx):
    """The 1.1B shape with Q8_0 weights and KV cache, a 2048-token prompt and
    128 greedy steps, against the reference's own stream: identical token for
    token, free-running (the fixture's closest call, step 38, has a reference
    top-2 logit gap of 1.4e-3; the GPU logits agree with the oracle's to
    ~1e-4 there).  Teacher-forced with the reference's ids, every step's
    argmax must match as well, so a divergence would name its step."""
    fx = load("llama1b_q8_stream.json")
    ref, margins = fx["generated_ids"], fx["top2_margins"]
    print("[case] llama1b q8 2048+128 golden stream", flush=True)
    import vlrf_amd as V
    m = V.Model(ctx, dict(fx["config"]))
    F.load_model(m, fx["seed"], norm_std=fx["norm_std"])
    prompt = prompt_of(fx)
    got = list(m.generate(prompt, len(ref)))
    i = _first_divergence(got, ref)
    print(f"  free-running: first divergence {i}", flush=True)
    m.reset()
    m.prefill(prompt)
    feed, bad = int(prompt[-1]), []
    for j, want in enumerate(ref):
        nxt = m.step(feed)
        if nxt != want:
            bad.append((j, nxt, want, margins[j]))
        feed = want
    assert i is None, (f"stream diverges at step {i}: gpu {got[i]} vs reference {ref[i]} "
                       f"(reference top-2 margin there {margins[i]:.3g})")
    assert not bad, f"teacher-forced argmax mismatches (step, gpu, ref, margin): {bad[:8]}"
