"""Pins the CPU oracle (oracle/vlrf_oracle.c) before it is trusted as the
checker: against the reference compiled from its own sources (oracle/_ref,
bit for bit, when present), the reference's own test shapes and tolerances
(tests/test_flash_attention.cpp, test_kv_cache_quant.cpp, test_ops.cpp), and
closed forms / brute force in float64 chosen so that a dropped term, a wrong
sign or index, or a transposed operand fails."""
import numpy as np
import pytest

import oracle
from vlrf_amd import formats as F

R = oracle.ref()
needs_ref = pytest.mark.skipif(R is None, reason="oracle/_ref not built (reference tree absent)")

REF_SHAPES = [(64, 64, 32, False, 1), (128, 128, 32, True, 2), (37, 37, 8, True, 5),
              (130, 130, 64, True, 6), (1, 1, 16, False, 3), (1, 200, 16, False, 4),
              (1, 1, 4, True, 8), (200, 500, 64, True, 7), (300, 300, 128, False, 9)]


def dense_attention(Q, K, V, scale, causal):
    """Textbook softmax(QK^T*scale + mask) V in float64 (the independent dense
    reference of test_flash_attention.cpp:48-75)."""
    Q, K, V = (np.asarray(a, np.float64) for a in (Q, K, V))
    T, ctx = Q.shape[0], K.shape[0]
    s = (Q @ K.T) * float(scale)
    if causal:
        past = ctx - T
        mask = np.arange(ctx)[None, :] > (np.arange(T)[:, None] + past)
        s[mask] = -np.inf
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p @ V) / p.sum(axis=1, keepdims=True)


def qkv(seed, T, ctx, d):
    return (F.normal(seed, "Q", T * d).reshape(T, d), F.normal(seed, "K", ctx * d).reshape(ctx, d),
            F.normal(seed, "V", ctx * d).reshape(ctx, d))


# ---- flash attention ----------------------------------------------------------------
@pytest.mark.parametrize("T,ctx,d,causal,seed", REF_SHAPES)
def test_flash_attn_vs_dense(T, ctx, d, causal, seed):
    Q, K, V = qkv(seed, T, ctx, d)
    s = np.float32(1) / np.sqrt(np.float32(d))
    out = oracle.flash_attn_head(Q, K, V, s, causal)
    assert np.max(np.abs(out - dense_attention(Q, K, V, s, causal))) <= 1e-4


def test_flash_attn_decode_is_noncausal_and_uses_all_keys():
    """A decode query (T=1) sees every key; the last key alone decides the
    output when it dominates the scores (catches an off-by-one on ctx)."""
    d, ctx = 16, 70
    K = np.zeros((ctx, d), np.float32)
    V = np.tile(np.arange(ctx, dtype=np.float32)[:, None], (1, d))
    Q = np.zeros((1, d), np.float32)
    Q[0, 0] = 1.0
    K[-1, 0] = 100.0
    out = oracle.flash_attn_head(Q, K, V, 1.0, False)
    assert np.allclose(out, ctx - 1)


@needs_ref
@pytest.mark.parametrize("T,ctx,d,causal,seed", REF_SHAPES + [(1, 512, 64, False, 11)])
def test_flash_attn_bit_exact_vs_reference(T, ctx, d, causal, seed):
    Q, K, V = qkv(seed, T, ctx, d)
    s = np.float32(1) / np.sqrt(np.float32(d))
    a = oracle.flash_attn_head(Q, K, V, s, causal)
    b = np.zeros_like(a)
    R.ref_flash_attn_head(Q, K, V, b, T, ctx, d, s, int(causal))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- Q8_0 KV quantization ------------------------------------------------------------
def test_quantize_zero_row():
    q, s = oracle.quantize_row_q8_0(np.zeros(32, np.float32))
    assert s == 0.0 and not q.any()


def test_quantize_ties_and_extremes():
    x = np.zeros(16, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, -127.0, 126.5]
    q, s = oracle.quantize_row_q8_0(x)
    assert s == 1.0
    assert list(q[:9]) == [127, 1, -1, 2, -2, 3, -3, -127, 127]


def test_quantize_roundtrip_bound():
    """test_kv_cache_quant.cpp:39-60: n=64, U(-5,5), error <= 1.5*amax/127."""
    rng = np.random.default_rng(123)
    x = rng.uniform(-5, 5, 64).astype(np.float32)
    q, s = oracle.quantize_row_q8_0(x)
    back = np.zeros(64, np.float32)
    oracle.lib().orc_dequantize_row_q8_0(q, s, back, 64)
    assert s > 0
    assert np.abs(back - x).max() <= np.abs(x).max() / 127 * 1.5
    assert np.array_equal(back, q.astype(np.float32) * s)


@needs_ref
def test_quantize_bit_exact_vs_reference():
    for n, seed in [(256, 1), (1024, 2), (64, 3), (17, 4)]:
        x = F.normal(seed, "row", n) * (10.0 ** (seed - 2))
        a, sa = oracle.quantize_row_q8_0(x)
        b = np.zeros(n, np.int8)
        sb = R.ref_quantize_row_q8_0(x, b, n)
        assert sa == sb and np.array_equal(a, b)


# ---- linear --------------------------------------------------------------------------
def test_linear_known_answers():
    """test_ops.cpp:85-99 as x.W^T: [[1,2,3],[4,5,6]] . [[1,2],[3,4],[5,6]]."""
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    W = np.array([[1, 3, 5], [2, 4, 6]], np.float32)      # B^T
    assert np.array_equal(oracle.linear(x, W), [[22, 28], [49, 64]])
    eye = np.eye(2, dtype=np.float32)
    B = np.array([[2, 3], [4, 5]], np.float32)
    assert np.array_equal(oracle.linear(eye, B.T.copy()), B)


@pytest.mark.parametrize("M,K,N", [(1, 2048, 2560), (1, 5632, 300), (4, 512, 77), (2, 96, 40),
                                   (16, 256, 264)])
def test_linear_vs_float64(M, K, N):
    x = F.normal(1, "x", M * K).reshape(M, K)
    W = F.normal(1, "W", N * K, 0.02).reshape(N, K)
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    out = oracle.linear(x, W)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))


@needs_ref
@pytest.mark.parametrize("M,K,N", [(1, 2048, 2560), (1, 5632, 2048), (1, 2048, 100), (1, 40, 257),
                                   (1, 2048, 259), (2, 64, 100), (4, 2048, 300), (16, 64, 37)])
def test_linear_bit_exact_vs_reference(M, K, N):
    x = F.normal(2, "x", M * K).reshape(M, K)
    W = F.normal(2, "W", N * K, 0.02).reshape(N, K)
    a = oracle.linear(x, W, n_threads=R.ref_hw_threads())
    b = np.zeros((M, N), np.float32)
    R.ref_linear(x, W, b, M, K, N)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- RMSNorm / RoPE / SwiGLU / argmax ---------------------------------------------------
def test_rms_norm_closed_form():
    x = F.normal(3, "x", 3 * 2048).reshape(3, 2048) * 4
    w = 1 + F.normal(3, "w", 2048, 0.3)
    out = oracle.rms_norm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * w
    assert np.max(np.abs(out - ref) / np.abs(ref).max()) <= 1e-6


def test_rope_closed_form():
    d, H, T, pos0, theta = 64, 3, 4, 9, 10000.0
    tabs = oracle.rope_tables(32, d, theta)
    x = F.normal(4, "x", T * H * d)
    out = oracle.rope_apply(x, H, d, pos0, tabs, 32).reshape(T, H, d).astype(np.float64)
    xr = x.reshape(T, H, d).astype(np.float64)
    half = d // 2
    i = np.arange(half)
    for t in range(T):
        ang = (pos0 + t) * theta ** (-2.0 * i / d)
        c, s = np.cos(ang), np.sin(ang)
        a, b = xr[t, :, :half], xr[t, :, half:]
        np.testing.assert_allclose(out[t, :, :half], a * c - b * s, atol=2e-5)
        np.testing.assert_allclose(out[t, :, half:], b * c + a * s, atol=2e-5)
    ident = oracle.rope_apply(x[:H * d], H, d, 0, tabs, 32)      # position 0 is the identity
    assert np.array_equal(ident, x[:H * d])


def test_silu_mul_and_argmax():
    h = F.normal(5, "h", 100)
    g = F.normal(5, "g", 100) * 3
    ref = h.astype(np.float64) * g / (1 + np.exp(-g.astype(np.float64)))
    assert np.max(np.abs(oracle.silu_mul(h, g) - ref)) <= 1e-6
    p = np.array([1, 3, 3, 2, -1], np.float32)
    assert oracle.lib().orc_argmax(p, 5) == 1


@needs_ref
def test_edge_ops_bit_exact_vs_reference():
    x = F.normal(6, "x", 3 * 2048).reshape(3, 2048)
    w = 1 + F.normal(6, "w", 2048, 0.1)
    b = np.zeros_like(x)
    R.ref_rms_norm(x, w, b, 3, 2048, 1e-5)
    assert np.array_equal(oracle.rms_norm(x, w, 1e-5), b)
    tabs = oracle.rope_tables(64, 64, 10000.0)
    y = F.normal(6, "y", 3 * 32 * 64)
    r = y.copy()
    R.ref_rope(r, 3, 32, 64, 61, 64, 10000.0)          # crosses max_seq
    assert np.array_equal(oracle.rope_apply(y, 32, 64, 61, tabs, 64), r)
    h, g = F.normal(6, "h", 5000), F.normal(6, "g", 5000)
    h2, g2 = h.copy(), g.copy()
    R.ref_silu_mul(h2, g2, 5000)
    assert np.array_equal(oracle.silu_mul(h, g), h2)


# ---- GGUF block decode (convert_gguf.py:233-263) -----------------------------------------
def test_dequant_q8_0_gguf_fixture_recipe():
    """The synthetic Q8_0 tensor of tools/converter/test_converters.py:327-343:
    numel 256, default_rng(42), scale U(0.01,0.1) stored as f16, qs in [-127,127)."""
    rng = np.random.default_rng(42)
    blocks, expected = bytearray(), np.zeros(256, np.float32)
    for b in range(8):
        scale = np.float32(rng.uniform(0.01, 0.1))
        qs = rng.integers(-127, 127, size=32, dtype=np.int8)
        d16 = np.float16(scale)
        blocks += d16.tobytes() + qs.tobytes()
        expected[b * 32:(b + 1) * 32] = qs.astype(np.float32) * float(d16)
    out = oracle.dequant_q8_0(np.frombuffer(bytes(blocks), np.uint8), 256)
    assert np.array_equal(out, expected)


def test_dequant_q4_0_nibble_order():
    """Low nibble -> even element, high nibble -> odd element, value (n-8)*d."""
    d16 = np.float16(0.5)
    qs = np.array([(j & 0xF) | ((15 - j) << 4) for j in range(16)], np.uint8)
    block = np.frombuffer(d16.tobytes() + qs.tobytes(), np.uint8)
    out = oracle.dequant_q4_0(block, 32)
    exp = np.empty(32, np.float32)
    exp[0::2] = (np.arange(16) - 8) * 0.5
    exp[1::2] = (15 - np.arange(16) - 8) * 0.5
    assert np.array_equal(out, exp)


# ---- whole model ------------------------------------------------------------------------
def _tiny(seed=31):
    cfg = F.tiny(F.DT_Q8_0, n_layers=2, max_seq_len=64)
    return cfg, F.make_f32_weights(cfg, seed, norm_std=0.1)


@needs_ref
def test_model_bit_exact_vs_reference():
    """Prefill (M=20 GEMMs, causal attention) then 24 decode steps: logits and
    the Q8_0 KV caches equal the reference TransformerModel's bit for bit."""
    import ctypes as C
    cfg, w = _tiny()
    nt = R.ref_hw_threads()
    om = oracle.Model(cfg, w, n_threads=nt)
    h = R.ref_model_create(cfg["vocab_size"], cfg["d_model"], cfg["d_ff"], cfg["n_heads"],
                           cfg["n_kv_heads"], cfg["n_layers"], cfg["max_seq_len"],
                           cfg["norm_eps"], cfg["rope_theta"])
    try:
        for k, v in w.items():
            R.ref_model_set_tensor(h, k.encode(), v, v.shape[0] if v.ndim == 2 else 0, v.shape[-1])
        R.ref_model_bind(h)
        prompt = F.tokens(31, "prompt", 20, cfg["vocab_size"])
        lg = np.zeros(cfg["vocab_size"], np.float32)
        t1, l1 = om.forward(prompt, True)
        t2 = R.ref_model_forward(h, prompt, 20, lg.ctypes.data)
        assert t1 == t2 and np.array_equal(l1, lg)
        for _ in range(24):
            t1, l1 = om.forward([t1], True)
            t2 = R.ref_model_forward(h, np.array([t2], np.int32), 1, lg.ctypes.data)
            assert t1 == t2 and np.array_equal(l1, lg)
        for layer in range(cfg["n_layers"]):
            kq, vq, ks, vs = om.kv(layer)
            p = [C.c_void_p() for _ in range(4)]
            R.ref_model_kv(h, layer, *[C.byref(x) for x in p])
            rk = np.ctypeslib.as_array(C.cast(p[0], C.POINTER(C.c_int8)), kq.shape)
            rs = np.ctypeslib.as_array(C.cast(p[3], C.POINTER(C.c_float)), vs.shape)
            assert np.array_equal(rk, kq) and np.array_equal(rs, vs)
    finally:
        R.ref_model_destroy(h)


@needs_ref
def test_filled_cache_decode_bit_exact_vs_reference():
    """The CPU baseline's set-up: both models' caches filled with the same
    seeded Q8_0 rows (no prefill), then decode steps from there give the same
    logits bit for bit, and the fill length is what was asked."""
    cfg, w = _tiny(33)
    om = oracle.Model(cfg, w, n_threads=R.ref_hw_threads())
    rm = oracle.RefModel(cfg, w)
    om.fill_kv(40, seed=7)
    rm.fill_kv(40, seed=7)
    assert om.used == rm.used == 40
    t1 = t2 = 5
    for _ in range(6):
        t1, l1 = om.forward([t1], True)
        t2, l2 = rm.forward([t2], True)
        assert t1 == t2 and np.array_equal(l1, l2)
    assert om.used == rm.used == 46
    rm.fill_kv(40, seed=8)                    # another seed: other codes, other logits
    _, l3 = rm.forward([5], True)
    om.fill_kv(40, seed=7)
    _, l4 = om.forward([5], True)
    assert not np.array_equal(l3, l4)


def test_model_prefill_matches_incremental():
    """The invariant of test_flash_attention.cpp:131-182 at model level: a
    one-shot prefill and token-by-token decode give the same next-token logits."""
    cfg, w = _tiny(32)
    prompt = F.tokens(32, "p", 30, cfg["vocab_size"])
    a = oracle.Model(cfg, w, n_threads=4)
    ta, la = a.forward(prompt, True)
    b = oracle.Model(cfg, w, n_threads=4)
    for t in prompt:
        tb, lb = b.forward([int(t)], True)
    assert ta == tb
    assert np.max(np.abs(la - lb)) <= 1e-3 * np.max(np.abs(la))


# ---- F32 / F16 KV caches (kv_cache.hpp:37-41, 68-97, 152-286) --------------------
def test_f32_to_f16_kv_known_answers():
    """Closed-form answers of the reference's conversion, chosen where it
    differs from IEEE round-to-nearest-even: exact halfway cases round up in
    magnitude, values below 2^-14 flush to signed zero, 65520 overflows."""
    cases = {1.0: 0x3C00, -2.0: 0xC000, 65504.0: 0x7BFF, 65520.0: 0x7C00, 1e9: 0x7C00,
             2.0 ** -14: 0x0400, 2.0 ** -15: 0x0000, -1e-6: 0x8000, 0.0: 0x0000,
             1.0 + 2.0 ** -11: 0x3C01,            # tie: RNE would give 0x3C00
             1.0 + 3 * 2.0 ** -11: 0x3C02,        # tie between 0x3C01 and 0x3C02
             float("inf"): 0x7C00, float("-inf"): 0xFC00}
    for x, want in cases.items():
        assert oracle.lib().orc_f32_to_f16_kv(x) == want, (x, hex(oracle.lib().orc_f32_to_f16_kv(x)))
    nan = oracle.lib().orc_f32_to_f16_kv(float("nan"))
    assert nan & 0x7C00 == 0x7C00 and nan & 0x3FF == 0x200


@needs_ref
def test_f32_to_f16_kv_bit_exact_vs_reference():
    rng = np.random.default_rng(5)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32),
                           np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0x00000001,
                                     0x387FFFFF, 0x38800000, 0x477FEFFF, 0x477FF000, 0x33800000], np.uint32)])
    xs = bits.view(np.float32)
    # inputs around every rounding boundary of the 10-bit mantissa
    base = (rng.integers(0x38800000, 0x47800000, 2000).astype(np.uint32) & ~np.uint32(0x1FFF)) | np.uint32(0x1000)
    xs = np.concatenate([xs, base.view(np.float32), (base - 1).view(np.float32), (base + 1).view(np.float32)])
    f_orc, f_ref = oracle.lib().orc_f32_to_f16_kv, R.ref_f32_to_f16
    for x in xs:
        assert f_orc(float(x)) == f_ref(float(x)), hex(np.float32(x).view(np.uint32))


@needs_ref
@pytest.mark.parametrize("kv_dtype", [oracle.KV_F32, oracle.KV_F16])
def test_model_f32_f16_kv_bit_exact_vs_reference(kv_dtype):
    """Prefill then 24 decode steps with the reference's F32 / F16 caches:
    logits and the caches' raw contents equal the reference's bit for bit."""
    import ctypes as C
    cfg, w = _tiny(33)
    cfg["kv_dtype"] = kv_dtype
    nt = R.ref_hw_threads()
    om = oracle.Model(cfg, w, n_threads=nt)
    h = R.ref_model_create_kv(cfg["vocab_size"], cfg["d_model"], cfg["d_ff"], cfg["n_heads"],
                              cfg["n_kv_heads"], cfg["n_layers"], cfg["max_seq_len"],
                              cfg["norm_eps"], cfg["rope_theta"], kv_dtype)
    try:
        for k, v in w.items():
            R.ref_model_set_tensor(h, k.encode(), v, v.shape[0] if v.ndim == 2 else 0, v.shape[-1])
        R.ref_model_bind(h)
        prompt = F.tokens(33, "prompt", 20, cfg["vocab_size"])
        lg = np.zeros(cfg["vocab_size"], np.float32)
        t1, l1 = om.forward(prompt, True)
        t2 = R.ref_model_forward(h, prompt, 20, lg.ctypes.data)
        assert t1 == t2 and np.array_equal(l1, lg)
        for _ in range(24):
            t1, l1 = om.forward([t1], True)
            t2 = R.ref_model_forward(h, np.array([t2], np.int32), 1, lg.ctypes.data)
            assert t1 == t2 and np.array_equal(l1, lg)
        ct = C.c_float if kv_dtype == oracle.KV_F32 else C.c_uint16
        for layer in range(cfg["n_layers"]):
            ok, ov = om.kv_raw(layer)
            rk, rv = C.c_void_p(), C.c_void_p()
            R.ref_model_kv_raw(h, layer, C.byref(rk), C.byref(rv))
            assert np.array_equal(np.ctypeslib.as_array(C.cast(rk, C.POINTER(ct)), ok.shape), ok)
            assert np.array_equal(np.ctypeslib.as_array(C.cast(rv, C.POINTER(ct)), ov.shape), ov)
            assert ok[:44].any() and not ok[44:].any()       # 20 + 24 rows written
    finally:
        R.ref_model_destroy(h)


# ---- the engine's remaining per-op calls (ops.hpp) -------------------------------
def test_per_op_closed_forms():
    x = F.normal(50, "lnx", 6 * 333).reshape(6, 333) * 3 + 1
    y = oracle.layer_norm(x, np.ones(333), np.zeros(333), 1e-5).astype(np.float64)
    assert np.allclose(y.mean(axis=1), 0, atol=1e-5) and np.allclose(y.var(axis=1), 1, atol=1e-3)
    w, b = F.normal(50, "lnw", 333), F.normal(50, "lnb", 333)
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5) * w + b
    assert np.max(np.abs(oracle.layer_norm(x, w, b, 1e-5) - want)) <= 1e-5 * np.max(np.abs(want))
    s = oracle.softmax(x)
    assert np.allclose(s.sum(axis=1), 1, atol=1e-6)
    assert np.allclose(oracle.softmax(x + 7.5), s, atol=1e-6)          # shift invariance
    g = F.normal(51, "gx", 5000) * 4
    assert np.allclose(oracle.gelu(g) - oracle.gelu(-g), g, atol=1e-5 * 16)   # gelu(x) - gelu(-x) = x
    assert oracle.gelu(np.zeros(3)).tolist() == [0.0, 0.0, 0.0]
    A, B = F.normal(52, "gA", 7 * 13).reshape(7, 13), F.normal(52, "gB", 13 * 5).reshape(13, 5)
    C0 = F.normal(52, "gC", 35).reshape(7, 5)
    for ta in (False, True):
        for tb in (False, True):
            Ai = A.T.copy() if ta else A
            Bi = B.T.copy() if tb else B
            got = oracle.gemm(Ai, Bi, C0, 1.5, 0.5, ta, tb)
            want = 0.5 * C0.astype(np.float64) + 1.5 * (A.astype(np.float64) @ B.astype(np.float64))
            assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want)), (ta, tb)


@needs_ref
def test_per_op_vs_reference():
    x = F.normal(53, "rx", 5 * 300).reshape(5, 300) * 2
    w, b = F.normal(53, "rw", 300), F.normal(53, "rb", 300)
    o1, o2 = np.zeros_like(x), np.zeros_like(x)
    oracle.lib().orc_layer_norm(x, w, b, o1, 5, 300, 1e-5)
    R.ref_layer_norm(x, w, b, o2, 5, 300, 1e-5)
    assert np.array_equal(o1, o2)
    s1, s2 = (F.normal(53, "rs", 4 * 1000).reshape(4, 1000) * 5 for _ in range(2))
    oracle.lib().orc_softmax(s1, 4, 1000)
    R.ref_softmax(s2, 4, 1000)
    assert np.array_equal(s1, s2)
    g1, g2 = (F.normal(53, "rg", 9000) * 6 for _ in range(2))
    oracle.lib().orc_gelu(g1, g1.size)
    R.ref_gelu(g2, g2.size)
    assert np.array_equal(g1, g2)
    A, B = F.normal(53, "rA", 37 * 64).reshape(37, 64), F.normal(53, "rB", 64 * 29).reshape(64, 29)
    C0 = F.normal(53, "rC", 37 * 29).reshape(37, 29)
    for ta in (False, True):
        for tb in (False, True):
            for alpha, beta in ((1.0, 0.0), (0.7, 1.0), (-1.25, 0.5)):
                Ai = A.T.copy() if ta else A
                Bi = B.T.copy() if tb else B
                got = oracle.gemm(Ai, Bi, C0, alpha, beta, ta, tb)
                ref = C0.copy()
                R.ref_gemm(Ai, Ai.shape[0], Ai.shape[1], Bi, Bi.shape[0], Bi.shape[1], ref, 37, 29, alpha, beta,
                           int(ta), int(tb))
                assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref)), (ta, tb, alpha, beta)
