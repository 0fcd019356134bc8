"""The one-launch decode step (VLRF_HIP_FLOW=1, kernels/flow.hip): every
phase of every layer in one grid whose workgroups wait for each other's
tagged outputs.  Parity as for the per-kernel step (TransformerModel::forward/
generate, transformer.hpp:335-547): greedy streams identical to the oracle's
and teacher-forced logits within 1e-3 of them, for Q8_0/Q4_0 weights and
Q8_0/F16/F32 caches, with one and several 512-row attention chunks; the two
steps agree with each other to 1e-5; a wait that runs out is reported as an
error and leaves the model usable."""
import os

import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import formats as F
from vlrf_amd._lib import ERR_RUNTIME

pytestmark = pytest.mark.gpu


def _model(ctx, cfg, seed, flow, wait_us=None):
    old = {k: os.environ.get(k) for k in ("VLRF_HIP_FLOW", "VLRF_HIP_WAIT_US")}
    os.environ["VLRF_HIP_FLOW"] = "1" if flow else "0"
    if wait_us is not None:
        os.environ["VLRF_HIP_WAIT_US"] = str(wait_us)
    try:
        m = V.Model(ctx, cfg)             # the switches are read when the model is created
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    w = F.load_model(m, seed, want_f32=True, norm_std=0.1)
    return m, w


CASES = [  # (weights, cache, max_seq_len): 1, 2 and 3 attention chunks
    (V.DT_Q8_0, V.KV_Q8_0, 128),
    (V.DT_Q4_0, V.KV_Q8_0, 128),
    (V.DT_Q8_0, V.KV_F16, 700),
    (V.DT_Q8_0, V.KV_F32, 1100),
    (V.DT_Q4_0, V.KV_Q8_0, 1100),
]


@pytest.mark.parametrize("wdt,kdt,cap", CASES)
def test_flow_stream_and_logits_match_oracle(ctx, orc, wdt, kdt, cap):
    print(f"[case] flow stream weights {wdt} kv {kdt} cap {cap}", flush=True)
    cfg = dict(F.tiny(wdt, n_layers=3, max_seq_len=cap), kv_dtype=kdt)
    m, w = _model(ctx, cfg, 41, True)
    om = orc.Model(cfg, w, n_threads=4)
    prompt = F.tokens(41, "prompt", 40, cfg["vocab_size"])
    gpu = m.generate(prompt, 48)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(48):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref
    assert m.used == om.used == 40 + 48
    # teacher-forced logits on a fresh feed
    m.reset()
    om.reset()
    worst = 0.0
    for t in F.tokens(41, "feed", 24, cfg["vocab_size"]):
        g_next, gl = m.step(int(t), want_logits=True)
        o_next, ol = om.forward([int(t)], want_logits=True)
        worst = max(worst, rel_err(gl, ol))
        assert g_next == int(np.argmax(gl))
    assert worst <= 1e-3, worst


def test_flow_agrees_with_the_per_kernel_step(ctx):
    """Same weights through both steps: logits within 1e-5, same tokens."""
    cfg = F.tiny(V.DT_Q8_0, n_layers=2, max_seq_len=600)
    a, _ = _model(ctx, cfg, 42, True)
    b, _ = _model(ctx, cfg, 42, False)
    worst = 0.0
    for t in F.tokens(42, "feed", 30, cfg["vocab_size"]):
        na, la = a.step(int(t), want_logits=True)
        nb, lb = b.step(int(t), want_logits=True)
        worst = max(worst, rel_err(la, lb))
        assert na == nb
    assert worst <= 1e-5, worst
    assert list(a.generate_ids(na, 40)) == list(b.generate_ids(nb, 40))


def test_flow_wait_timeout_is_reported(ctx, orc):
    """A 1 us limit on every wait: a step whose workgroups must wait reports
    VLRF_HIP_ERR_RUNTIME (the grid drains: every wait is bounded and leaves on
    the failure flag); the model stays usable and a model with the normal limit
    still matches the oracle."""
    cfg = F.tiny(V.DT_Q8_0, n_layers=3, max_seq_len=128)
    m, _ = _model(ctx, cfg, 43, True, wait_us=1)
    failed = 0
    for t in F.tokens(43, "feed", 8, cfg["vocab_size"]):
        try:
            m.step(int(t))
        except V.HipError as e:
            assert e.rc == ERR_RUNTIME and "ran out" in str(e), str(e)
            failed += 1
    print(f"[case] 1 us waits: {failed} of 8 steps reported a timeout", flush=True)
    m2, w = _model(ctx, cfg, 43, True)
    om = orc.Model(cfg, w, n_threads=4)
    prompt = F.tokens(43, "prompt", 20, cfg["vocab_size"])
    gpu = m2.generate(prompt, 16)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(16):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref
