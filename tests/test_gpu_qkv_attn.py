"""The fused QKV + attention launch of the decode step (kernels/qkv_attn.hip):
the projection's workgroups publish their rows as tagged words and the
attention's workgroups, in the same grid, wait for the 64 q words of their
head and the token's K/V row.  Parity as for the two kernels it replaces
(TransformerModel::forward/generate, transformer.hpp:335-547;
AttentionBlock::forward, attention.hpp:89-186): greedy streams identical to
the oracle's and teacher-forced logits within 1e-3 of them, for Q8_0/Q4_0
weights, Q8_0/F16 caches, GQA groups 1-8 and one to three 512-row chunks; the
fused step is as close to the oracle as the unfused one over 560 steps; a wait
that runs out is reported and leaves the model usable."""
import os

import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import formats as F
from vlrf_amd._lib import ERR_RUNTIME

pytestmark = pytest.mark.gpu


def _model(ctx, cfg, seed, fused=True, wait_us=None):
    old = {k: os.environ.get(k) for k in ("VLRF_HIP_QKV_ATTN", "VLRF_HIP_WAIT_US")}
    os.environ["VLRF_HIP_QKV_ATTN"] = "1" if fused else "0"
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


def _cfg(wdt, kdt, cap, heads=4, kv=1, d_model=256):
    return dict(F.tiny(wdt, n_layers=3, max_seq_len=cap), kv_dtype=kdt, n_heads=heads, n_kv_heads=kv,
                d_model=d_model)


CASES = [  # (weights, cache, max_seq_len, heads, kv heads, d_model)
    (V.DT_Q8_0, V.KV_Q8_0, 128, 4, 1, 256),
    (V.DT_Q4_0, V.KV_Q8_0, 128, 4, 1, 256),
    (V.DT_Q8_0, V.KV_F16, 700, 4, 1, 256),
    (V.DT_Q4_0, V.KV_Q8_0, 1100, 4, 1, 256),
    (V.DT_Q8_0, V.KV_Q8_0, 600, 8, 1, 512),    # GQA 8
    (V.DT_Q8_0, V.KV_Q8_0, 600, 8, 4, 512),    # GQA 2
    (V.DT_Q4_0, V.KV_F16, 300, 8, 8, 512),     # no grouping, 8 KV heads
    (V.DT_Q4_0, V.KV_Q8_0, 1100, 16, 2, 1024),  # 16 heads, three chunks
    (V.DT_Q8_0, V.KV_Q8_0, 600, 32, 4, 2048),   # the 1.1B attention shape
]


@pytest.mark.parametrize("wdt,kdt,cap,heads,kv,dm", CASES)
def test_fused_stream_and_logits_match_oracle(ctx, orc, wdt, kdt, cap, heads, kv, dm):
    print(f"[case] qkv_attn stream weights {wdt} kv {kdt} cap {cap} heads {heads}/{kv} d_model {dm}", flush=True)
    cfg = _cfg(wdt, kdt, cap, heads, kv, dm)
    m, w = _model(ctx, cfg, 61)
    om = orc.Model(cfg, w, n_threads=4)
    prompt = F.tokens(61, "prompt", 40, cfg["vocab_size"])
    gpu = m.generate(prompt, 48)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(48):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref
    assert m.used == om.used == 40 + 48
    m.reset()
    om.reset()
    worst = 0.0
    for t in F.tokens(61, "feed", 24, cfg["vocab_size"]):
        g_next, gl = m.step(int(t), want_logits=True)
        o_next, ol = om.forward([int(t)], want_logits=True)
        worst = max(worst, rel_err(gl, ol))
        assert g_next == int(np.argmax(gl))
    assert worst <= 1e-3, worst


def test_fused_as_accurate_as_the_two_kernels(ctx, orc):
    """Same weights with and without the fusion, fed the same 560 tokens (the
    cache crosses a 512-row chunk boundary), each against the oracle at every
    step.  The fused attention exponentiates against the chunk's maximum and
    merges the token's key as its own partial, so the two paths agree to
    rounding, not bit for bit, and a rounding difference can flip a Q8_0 code
    of a cached row; each path's distance from the oracle is what is bounded:
    within the parity tolerance, and the fused path no further than twice the
    unfused one's."""
    cfg = _cfg(V.DT_Q8_0, V.KV_Q8_0, 1100)
    a, w = _model(ctx, cfg, 62, fused=True)
    b, _ = _model(ctx, cfg, 62, fused=False)
    om = orc.Model(cfg, w, n_threads=4)
    ea = eb = eab = 0.0
    for t in F.tokens(62, "feed", 560, cfg["vocab_size"]):
        _, la = a.step(int(t), want_logits=True)
        _, lb = b.step(int(t), want_logits=True)
        _, lo = om.forward([int(t)], want_logits=True)
        ea, eb, eab = max(ea, rel_err(la, lo)), max(eb, rel_err(lb, lo)), max(eab, rel_err(la, lb))
    print(f"  560 steps vs oracle: fused {ea:.2e}, two kernels {eb:.2e}; between them {eab:.2e}", flush=True)
    assert ea <= 1e-3 and eb <= 1e-3, (ea, eb)
    assert ea <= max(2 * eb, 1e-4), (ea, eb)


def test_fused_wait_timeout_is_reported(ctx, orc):
    """A zero limit on the attention's wait: a step reports
    VLRF_HIP_ERR_RUNTIME naming the attention phase (every wait is bounded, so
    the grid drains); the model stays usable and one with the normal limit
    still matches the oracle."""
    cfg = _cfg(V.DT_Q8_0, V.KV_Q8_0, 128)
    m, _ = _model(ctx, cfg, 63, wait_us=0)
    failed = 0
    for t in F.tokens(63, "feed", 8, cfg["vocab_size"]):
        try:
            m.step(int(t))
        except V.HipError as e:
            assert e.rc == ERR_RUNTIME and "ran out" in str(e) and "phase 2" in str(e), str(e)
            failed += 1
    print(f"[case] zero-length waits: {failed} of 8 steps reported a timeout", flush=True)
    assert failed > 0
    m2, w = _model(ctx, cfg, 63)
    om = orc.Model(cfg, w, n_threads=4)
    prompt = F.tokens(63, "prompt", 20, cfg["vocab_size"])
    gpu = m2.generate(prompt, 16)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(16):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref


