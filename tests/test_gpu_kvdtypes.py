"""GPU parity of the F32 and F16 KV caches (KVCacheDType, kv_cache.hpp:37-41;
the reference's default is F32).  F16 appends must equal the reference's own
f32_to_f16 (kv_cache.hpp:68-97: half-up rounding, flush below 2^-14, overflow
to inf), restated in the oracle and pinned against the reference build in
tests/test_oracle.py; F32 appends are copies.  Attention over either cache,
the decode step and the batched MFMA prefill are checked against the oracle
running the same cache dtype."""
import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu

DTYPES = [V.KV_F32, V.KV_F16]


def _special_rows(row):
    base = F.normal(41, "kvspecial", 4 * row).reshape(4, row)
    base[0, :12] = [1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65520.0, 1e9, 2.0 ** -14,
                    2.0 ** -15, -1e-6, 0.0, -0.0, 6.1e-5, -65519.0]
    base[1] *= 1e-6                      # mostly below the f16 normal range: flushed
    base[2] *= 3e4
    return base.astype(np.float32)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n_kv,d,T", [(4, 64, 200), (8, 128, 9), (1, 64, 1)])
def test_append_matches_reference_conversion(ctx, orc, dtype, n_kv, d, T):
    print(f"[case] kv append dtype={dtype} n_kv={n_kv} d={d} T={T}", flush=True)
    row = n_kv * d
    kv = V.KVCache(ctx, 2, 256, n_kv, d, dtype)
    K = (F.normal(42, f"K{row}", T * row) * 3).reshape(T, row)
    Vv = (F.normal(42, f"V{row}", T * row) * 0.3).reshape(T, row)
    if T >= 4:
        K[:4] = _special_rows(row)
    kv.append(1, ctx.to_device(K), ctx.to_device(Vv), T)
    k, v, ks, vs = kv.read(1, 0, T)
    assert ks is None and vs is None and kv.used(1) == T
    if dtype == V.KV_F32:
        assert np.array_equal(k.view(np.uint32), K.view(np.uint32))
        assert np.array_equal(v.view(np.uint32), Vv.view(np.uint32))
    else:
        assert np.array_equal(k.ravel(), orc.f32_to_f16_kv(K))
        assert np.array_equal(v.ravel(), orc.f32_to_f16_kv(Vv))
    # dequant_into: f16 widened exactly, f32 as stored
    Ko, Vo = ctx.alloc(K.nbytes), ctx.alloc(Vv.nbytes)
    kv.dequant_into(1, T, Ko, Vo)
    want_k = K if dtype == V.KV_F32 else k.view(np.float16).astype(np.float32)
    assert np.array_equal(Ko.download(K.shape).view(np.uint32), want_k.view(np.uint32))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n_heads,n_kv,d,ctx_len", [(32, 4, 64, 2048), (16, 2, 128, 777), (8, 1, 64, 1),
                                                    (16, 4, 64, 500)])
def test_decode_attention(ctx, orc, dtype, n_heads, n_kv, d, ctx_len):
    """Split-K (2048 and 777 tokens) and the single-pass kernel (caches of <= 512
    rows: 1 and 500 tokens) over the F32 / F16 cache."""
    print(f"[case] decode attention dtype={dtype} heads={n_heads}/{n_kv} d={d} ctx={ctx_len}", flush=True)
    row = n_kv * d
    kv = V.KVCache(ctx, 1, ctx_len + 3, n_kv, d, dtype)
    K = F.normal(43, "Kd", ctx_len * row)
    Vv = F.normal(43, "Vd", ctx_len * row)
    kv.append(0, ctx.to_device(K), ctx.to_device(Vv), ctx_len)
    k, v, _, _ = kv.read(0, 0, ctx_len)
    Kd = k if dtype == V.KV_F32 else k.view(np.float16).astype(np.float32)
    Vd = v if dtype == V.KV_F32 else v.view(np.float16).astype(np.float32)
    q = F.normal(43, "qd", n_heads * d)
    dq, dout = ctx.to_device(q), ctx.alloc(q.nbytes)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    kv.attention_decode(0, dq, dout, n_heads, ctx_len, scale)
    out = dout.download(q.shape)
    ref = np.zeros_like(q)
    rep = n_heads // n_kv
    for h in range(n_heads):
        g = h // rep
        ref[h * d:(h + 1) * d] = orc.flash_attn_head(q[h * d:(h + 1) * d][None, :], Kd[:, g * d:(g + 1) * d],
                                                     Vd[:, g * d:(g + 1) * d], scale, False)[0]
    assert rel_err(out, ref) <= 1e-3
    assert np.max(np.abs(out - ref)) <= 1e-4


def _models(ctx, orc, cfg, seed):
    m = V.Model(ctx, cfg)
    w = F.load_model(m, seed, want_f32=True, norm_std=0.1)
    return m, orc.Model(cfg, w, n_threads=4)


@pytest.mark.parametrize("dtype", DTYPES)
def test_model_greedy_stream_and_cache(ctx, orc, dtype):
    """The decode step (fused RoPE + append + split-K attention) with an F32 /
    F16 cache: the greedy stream equals the oracle's, teacher-forced logits
    within 1e-3, and the cache rows agree: F32 to f32 rounding of the
    projections; F16 to one f16 step (2^-10) of the largest element, since a
    value within f32 rounding of a conversion boundary lands on the
    neighbouring half, for a few percent of the elements (the differences grow
    through the layers, as the Q8_0 tests' one-code flips do)."""
    print(f"[case] model kv dtype={dtype}", flush=True)
    cfg = F.tiny(V.DT_Q8_0, n_layers=3, max_seq_len=128)
    cfg["kv_dtype"] = dtype
    m, om = _models(ctx, orc, cfg, 44)
    prompt = F.tokens(44, "kvp", 40, cfg["vocab_size"])
    gpu = m.generate(prompt, 48)
    om.reset()
    om.forward(prompt)
    last, ref = int(prompt[-1]), []
    for _ in range(48):
        last = om.forward([last])
        ref.append(last)
    assert list(gpu) == ref
    n = 40 + 48
    for layer in range(cfg["n_layers"]):
        gk, gv, _, _ = m.kv_rows(layer, 0, n)
        ok, ov = om.kv_raw(layer)
        for g, o in ((gk, ok[:n]), (gv, ov[:n])):
            if dtype == V.KV_F32:
                assert rel_err(g, o) <= 1e-5
            else:
                gf, of = g.view(np.float16).astype(np.float32), o.view(np.float16).astype(np.float32)
                assert rel_err(gf, of) <= 2.0 ** -10, layer
                assert np.mean(g != o) < 0.05
    m.reset()
    om.reset()
    worst = 0.0
    for t in F.tokens(44, "kvf", 30, cfg["vocab_size"]):
        _, gl = m.step(int(t), want_logits=True)
        _, ol = om.forward([int(t)], want_logits=True)
        worst = max(worst, rel_err(gl, ol))
    assert worst <= 1e-3, worst


@pytest.mark.parametrize("dtype", DTYPES)
def test_prefill_mfma_then_decode(ctx, orc, dtype):
    """Batched MFMA prefill into an F32 / F16 cache, then decode steps: logits
    in the bf16 class (1e-2 normwise) of the oracle's."""
    cfg = F.tiny(V.DT_Q8_0, n_layers=2, max_seq_len=160)
    cfg["kv_dtype"] = dtype
    m, om = _models(ctx, orc, cfg, 45)
    prompt = F.tokens(45, "kvpf", 90, cfg["vocab_size"])
    m.reset()
    om.reset()
    m.prefill_mfma(prompt)
    om.forward(prompt)
    assert m.used == 90
    tok = int(prompt[-1])
    for _ in range(4):
        _, gl = m.step(tok, want_logits=True)
        tok, ol = om.forward([tok], want_logits=True)
        assert rel_err(gl, ol) <= 1e-2


@pytest.mark.parametrize("kv_dtype", [V.KV_Q8_0, V.KV_F16, V.KV_F32])
@pytest.mark.parametrize("n_heads,n_kv,d_model", [(8, 4, 1024), (8, 8, 1024), (4, 4, 256)])
def test_prefill_append_vector_path_equals_element_path(ctx, monkeypatch, kv_dtype, n_heads, n_kv, d_model):
    """The prefill's K/V append reads its runs as float4 and writes them as whole
    words where rows and tables are aligned (4 and 8 RoPE pairs a lane: 512 and
    1024 K elements a row); VLRF_HIP_KV_VEC=0 keeps the element-wise loads and
    stores.  The same prefill either way leaves the same cache bit for bit, for
    every cache type (the 2-pair shape takes the element path both times)."""
    cfg = dict(F.tiny(V.DT_Q8_0, n_layers=1, max_seq_len=96), n_heads=n_heads, n_kv_heads=n_kv,
               d_model=d_model, d_ff=2 * d_model, kv_dtype=kv_dtype)
    print(f"[case] prefill append vec/element heads={n_heads}/{n_kv} d={d_model} kv={kv_dtype}", flush=True)
    m = V.Model(ctx, cfg)
    F.load_model(m, 53)
    T = 70
    x = ctx.to_device(F.normal(53, "kvvec", T * d_model))
    caches = []
    for flag in ("1", "0"):
        monkeypatch.setenv("VLRF_HIP_KV_VEC", flag)
        m.reset()
        m.forward_hidden(x)
        caches.append(m.kv_rows(0, 0, T))
    for a, b in zip(*caches):
        if a is None:
            assert b is None
        else:
            assert np.array_equal(a, b)
    kq = caches[0][0]
    assert np.any(kq != 0)
