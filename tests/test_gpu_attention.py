"""GPU parity: f32 flash attention (IBackend::sdp_attention) and the Q8_0-KV
GQA decode attention, against the oracle's restatement of
AttentionBlock::flash_attn_head (attention.hpp:207-309).

Inputs are seeded N(0,1) from vlrf_amd.formats.normal (the reference test's
mt19937 stream is not reproducible outside libstdc++; shapes, masks and
tolerances follow tests/test_flash_attention.cpp:77-121)."""
import numpy as np
import pytest

from conftest import rel_err
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu

# (T, ctx, d_h, causal, seed): tests/test_flash_attention.cpp:96-121
REF_SHAPES = [(64, 64, 32, False, 1), (128, 128, 32, True, 2), (37, 37, 8, True, 5),
              (130, 130, 64, True, 6), (1, 1, 16, False, 3), (1, 200, 16, False, 4),
              (1, 1, 4, True, 8), (200, 500, 64, True, 7), (300, 300, 128, False, 9)]


def _qkv(seed, n_h, T, ctx_len, d):
    Q = F.normal(seed, "Q", n_h * T * d).reshape(n_h, T, d)
    K = F.normal(seed, "K", n_h * ctx_len * d).reshape(n_h, ctx_len, d)
    V = F.normal(seed, "V", n_h * ctx_len * d).reshape(n_h, ctx_len, d)
    return Q, K, V


def _run_gpu(ctx, Q, K, V, scale, causal):
    n_h, T, d = Q.shape
    ctx_len = K.shape[1]
    dq, dk, dv = ctx.to_device(Q), ctx.to_device(K), ctx.to_device(V)
    do = ctx.alloc(Q.nbytes)
    ctx.sdp_attention(dq, dk, dv, do, n_h, T, ctx_len, d, scale, causal)
    return do.download(Q.shape)


@pytest.mark.parametrize("T,ctx_len,d,causal,seed", REF_SHAPES)
def test_sdp_attention_reference_shapes(ctx, orc, T, ctx_len, d, causal, seed):
    print(f"[case] sdp T={T} ctx={ctx_len} d={d} causal={causal}", flush=True)
    n_h = 2
    Q, K, V = _qkv(seed, n_h, T, ctx_len, d)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    out = _run_gpu(ctx, Q, K, V, scale, causal)
    ref = orc.sdp_attention(Q, K, V, scale, causal)
    assert np.max(np.abs(out - ref)) <= 1e-4          # the reference test's own bound
    assert rel_err(out, ref) <= 1e-3


def test_config1_decode_f32(ctx, orc):
    """Benchmark config 1: 1 query, 8 heads, d 64, KV 512, non-causal, scale 1/8."""
    Q, K, V = _qkv(11, 8, 1, 512, 64)
    out = _run_gpu(ctx, Q, K, V, np.float32(0.125), False)
    ref = orc.sdp_attention(Q, K, V, np.float32(0.125), False)
    assert np.max(np.abs(out - ref)) <= 1e-4
    assert rel_err(out, ref) <= 1e-3


@pytest.mark.parametrize("ctx_len", [1, 255, 256, 257, 1000])
def test_decode_f32_split_boundaries(ctx, orc, ctx_len):
    """Split-K chunk boundaries (256 tokens) and a single-token context."""
    Q, K, V = _qkv(ctx_len, 4, 1, ctx_len, 128)
    s = np.float32(1.0) / np.sqrt(np.float32(128))
    out = _run_gpu(ctx, Q, K, V, s, False)
    ref = orc.sdp_attention(Q, K, V, s, False)
    assert rel_err(out, ref) <= 1e-3


def _gqa_reference(orc, q, kq, vq, ks, vs, n_heads, n_kv, d, ctx_len, scale):
    """Reference decode attention: dequant_into (kv_cache.hpp:259-286), GQA head
    h -> kv head h/(n_heads/n_kv) (attention.hpp:328-342), non-causal
    flash_attn_head per head."""
    row = n_kv * d
    Kd = kq[:ctx_len].astype(np.float32) * ks[:ctx_len, None]
    Vd = vq[:ctx_len].astype(np.float32) * vs[:ctx_len, None]
    out = np.zeros(n_heads * d, np.float32)
    rep = n_heads // n_kv
    for h in range(n_heads):
        g = h // rep
        out[h * d:(h + 1) * d] = orc.flash_attn_head(q[h * d:(h + 1) * d][None, :],
                                                     Kd[:, g * d:(g + 1) * d],
                                                     Vd[:, g * d:(g + 1) * d], scale, False)[0]
    assert Kd.shape[1] == row
    return out


@pytest.mark.parametrize("n_heads,n_kv,d,ctx_len", [(32, 4, 64, 4096), (32, 4, 64, 2048),
                                                    (8, 8, 64, 300), (16, 2, 128, 777),
                                                    (8, 1, 64, 1), (16, 8, 64, 509),
                                                    (32, 8, 64, 65), (32, 4, 64, 510),
                                                    (8, 2, 64, 4600)])
def test_q8_decode_attention(ctx, orc, n_heads, n_kv, d, ctx_len):
    """Benchmark config 2 (32q/4kv, d 64, ctx 4096) and other GQA groupings.
    d_head 64 takes the one-launch chunked kernel (64-row chunks up to 1024
    tokens; 509 + 3 rows fill a chunk's round), d_head 128 the split-K
    kernel and its combine."""
    import vlrf_amd as V_
    print(f"[case] q8 decode heads={n_heads}/{n_kv} d={d} ctx={ctx_len}", flush=True)
    row = n_kv * d
    kv = V_.KVCache(ctx, 1, ctx_len + 3, n_kv, d)
    K = F.normal(5, "Kc", ctx_len * row)
    Vv = F.normal(5, "Vc", ctx_len * row)
    kv.append(0, ctx.to_device(K), ctx.to_device(Vv), ctx_len)
    kq, vq, ks, vs = kv.read(0, 0, ctx_len)
    q = F.normal(5, "q", n_heads * d)
    dq = ctx.to_device(q)
    dout = ctx.alloc(q.nbytes)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    kv.attention_decode(0, dq, dout, n_heads, ctx_len, scale)
    out = dout.download(q.shape)
    ref = _gqa_reference(orc, q, kq, vq, ks, vs, n_heads, n_kv, d, ctx_len, scale)
    assert rel_err(out, ref) <= 1e-3
    assert np.max(np.abs(out - ref)) <= 1e-4


def _dequant_rows(kv, ctx_len):
    import vlrf_amd as V_
    kq, vq, ks, vs = kv.read(0, 0, ctx_len)
    if kv.dtype == V_.KV_Q8_0:
        return kq.astype(np.float32) * ks[:, None], vq.astype(np.float32) * vs[:, None]
    if kv.dtype == V_.KV_F16:
        return kq.view(np.float16).astype(np.float32), vq.view(np.float16).astype(np.float32)
    return kq, vq


@pytest.mark.parametrize("kv_name", ["Q8_0", "F16", "F32"])
@pytest.mark.parametrize("n_heads,n_kv,ctx_len", [(32, 4, 1024), (32, 4, 1025), (8, 2, 2049),
                                                  (16, 16, 4097), (32, 4, 8192), (8, 8, 8193)])
def test_decode_attention_chunk_sizes(ctx, orc, kv_name, n_heads, n_kv, ctx_len):
    """d_head 64 decode attention in one launch: contexts at the chunk-size
    steps (64 rows up to 1024 tokens, then 128/256/512 so that at most 16
    chunks cover the context) and past 8192 (the split-K pair of launches).
    Two calls in a row, the second over a shorter context: the per-head
    counters left by the first must read zero again."""
    import vlrf_amd as V_
    dt = {"Q8_0": V_.KV_Q8_0, "F16": V_.KV_F16, "F32": V_.KV_F32}[kv_name]
    print(f"[case] decode chunks kv={kv_name} heads={n_heads}/{n_kv} ctx={ctx_len}", flush=True)
    d, row = 64, n_kv * 64
    kv = V_.KVCache(ctx, 1, ctx_len + 5, n_kv, d, dt)
    K = F.normal(9, "Kc", ctx_len * row)
    Vv = F.normal(9, "Vc", ctx_len * row)
    kv.append(0, ctx.to_device(K), ctx.to_device(Vv), ctx_len)
    Kd, Vd = _dequant_rows(kv, ctx_len)
    scale = np.float32(0.125)
    rep = n_heads // n_kv
    for call, n in enumerate((ctx_len, max(1, ctx_len // 3))):
        q = F.normal(call, "q", n_heads * d)
        dout = ctx.alloc(q.nbytes)
        kv.attention_decode(0, ctx.to_device(q), dout, n_heads, n, scale)
        out = dout.download(q.shape)
        ref = np.concatenate([orc.flash_attn_head(q[h * d:(h + 1) * d][None, :],
                                                  Kd[:n, (h // rep) * d:(h // rep + 1) * d],
                                                  Vd[:n, (h // rep) * d:(h // rep + 1) * d], scale, False)[0]
                              for h in range(n_heads)])
        assert rel_err(out, ref) <= 1e-3, (call, n)
        assert np.max(np.abs(out - ref)) <= 1e-4, (call, n)
