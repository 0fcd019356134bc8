"""GPU parity of the decode step's long-cache attention (caches of more than
512 rows; smaller caches take the single-pass kernel): AttentionBlock::forward
with the cache (attention.hpp:89-186), the append (kv_cache.hpp:215-251) and
flash_attn_head's online softmax (attention.hpp:207-309), with RoPE and the
new row's quantization fused into the chunk that holds the new token.  The
step runs the chunked form (512 cached rows per workgroup and query head,
merged by the O projection's GEMV) where it applies, else split-K + combine.
Every GQA group size and both head sizes, all three cache dtypes, decode
positions on both sides of the chunk boundaries (the new token as the first,
a middle and the last row of a chunk), and generations after resets.  Bars:
greedy streams identical to the oracle's; logits within 1e-3 (f32 paths)."""
import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu

CAP = 1100  # > 512 rows: the chunked path, 3 chunks of 512 (and 18 split-K chunks of 64)


def _cfg(n_heads, n_kv, d_model, kv_dtype=V.KV_Q8_0, n_layers=2, weight_dtype=V.DT_Q8_0):
    cfg = dict(F.tiny(weight_dtype, n_layers=n_layers, max_seq_len=CAP), n_heads=n_heads, n_kv_heads=n_kv,
               d_model=d_model, d_ff=2 * d_model)
    cfg["kv_dtype"] = kv_dtype
    return cfg


def _models(ctx, orc, cfg, seed):
    m = V.Model(ctx, cfg)
    w = F.load_model(m, seed, want_f32=True, norm_std=0.1)
    return m, orc.Model(cfg, w, n_threads=8)


def _oracle_stream(om, prompt, n):
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(n):
        last = om.forward([last])
        ref.append(last)
    return ref


@pytest.mark.parametrize("n_heads,n_kv,d_model", [(4, 4, 256), (8, 4, 512), (4, 1, 256), (8, 2, 512),
                                                  (8, 1, 512), (8, 8, 512), (8, 8, 1024), (8, 1, 1024)])
def test_greedy_stream_gqa_shapes(ctx, orc, n_heads, n_kv, d_model):
    """GQA groups 1, 2, 4 and 8 at d_head 64 (up to 8 KV heads: a 512-element
    new row) and 128: a 520-token prompt through
    the decode step, then 30 greedy steps (positions 520..549, past the first
    512-row chunk)."""
    print(f"[case] split-K decode heads={n_heads}/{n_kv} d_model={d_model}", flush=True)
    cfg = _cfg(n_heads, n_kv, d_model)
    m, om = _models(ctx, orc, cfg, 61)
    prompt = F.tokens(61, "skp", 520, cfg["vocab_size"])
    assert list(m.generate(prompt, 30)) == _oracle_stream(om, prompt, 30)
    assert m.used == om.used == 550


@pytest.mark.parametrize("kv_dtype", [V.KV_Q8_0, V.KV_F16, V.KV_F32])
def test_logits_across_chunk_boundaries(ctx, orc, kv_dtype):
    """Teacher-forced logits at every position 0..539 (chunk boundaries at 64
    and 512, so the new token is the first, a middle and the last row of a
    chunk) for each cache dtype."""
    print(f"[case] split-K logits kv_dtype={kv_dtype}", flush=True)
    cfg = _cfg(8, 2, 512, kv_dtype)
    m, om = _models(ctx, orc, cfg, 62)
    m.reset()
    om.reset()
    worst = 0.0
    for t in F.tokens(62, "skf", 540, cfg["vocab_size"]):
        g_next, gl = m.step(int(t), want_logits=True)
        _, ol = om.forward([int(t)], want_logits=True)
        worst = max(worst, rel_err(gl, ol))
        assert g_next == int(np.argmax(gl))
    assert worst <= 1e-3, worst


def test_generations_after_resets(ctx, orc):
    """Three generations on one model with resets between them (prompt lengths
    that end just before, on and just after a chunk boundary): each stream
    equals the oracle's."""
    cfg = _cfg(4, 1, 256, n_layers=1)
    m, om = _models(ctx, orc, cfg, 63)
    for i, n in enumerate((511, 512, 513)):
        print(f"[case] split-K generation {i}: prompt {n}", flush=True)
        prompt = F.tokens(63, f"skr{i}", n, cfg["vocab_size"])
        m.reset()
        assert list(m.generate(prompt, 20)) == _oracle_stream(om, prompt, 20), i


def test_greedy_stream_q4_weights(ctx, orc):
    """Q4_0 weights: the O projection's chunk merge on the Q4_0 GEMV."""
    print("[case] long-cache decode, Q4_0 weights", flush=True)
    cfg = _cfg(8, 2, 512, weight_dtype=V.DT_Q4_0)
    m, om = _models(ctx, orc, cfg, 64)
    prompt = F.tokens(64, "skq4", 520, cfg["vocab_size"])
    assert list(m.generate(prompt, 30)) == _oracle_stream(om, prompt, 30)


def test_greedy_stream_wide_model(ctx, orc):
    """d_model 4096 at d_head 64 (64 query heads, 8 KV heads): the O
    projection's chunk merge with three float4 of x per thread (a 4096-wide
    GEMV row), which holds up to 5 chunks in registers."""
    print("[case] long-cache decode, d_model 4096 d_head 64", flush=True)
    cfg = _cfg(64, 8, 4096, n_layers=1)
    m, om = _models(ctx, orc, cfg, 65)
    prompt = F.tokens(65, "skw", 520, cfg["vocab_size"])
    assert list(m.generate(prompt, 12)) == _oracle_stream(om, prompt, 12)


def test_last_row_and_overflow(ctx, orc):
    """The cache filled to its last row (the third chunk partly past the
    capacity): the logits of the final position match the oracle's, and one
    more step is refused (KVCache::append's capacity error, kv_cache.hpp:215-251)."""
    print("[case] long-cache decode to the last cache row", flush=True)
    cfg = _cfg(4, 1, 256, n_layers=1)
    m, om = _models(ctx, orc, cfg, 66)
    ids = F.tokens(66, "skl", CAP, cfg["vocab_size"])
    m.reset()
    om.reset()
    m.prefill(ids[:-1])
    om.forward(ids[:-1])
    _, gl = m.step(int(ids[-1]), want_logits=True)
    _, ol = om.forward([int(ids[-1])], want_logits=True)
    assert m.used == om.used == CAP
    assert rel_err(gl, ol) <= 1e-3
    with pytest.raises(V.HipError) as e:
        m.step(int(ids[0]))
    assert e.value.rc == -4
