"""ctypes bindings for the test oracle (never imported by the product).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module as the checker for the HIP backend.

`lib()` loads the C restatement (oracle/liboracle.so, built by
oracle/Makefile); `ref()` loads the reference compiled from its own sources
(oracle/_ref/libvlrf_ref.so) and returns None when it was never built.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def build(with_ref=True):
    """Compile liboracle.so (and _ref when the reference tree is present)."""
    target = "all" if with_ref else os.path.join(HERE, "liboracle.so")
    subprocess.run(["make", "-s", "-C", HERE, target], check=True)


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab_size", "d_model", "d_ff", "n_heads",
                                       "n_kv_heads", "n_layers", "max_seq_len")] + \
               [("norm_eps", C.c_float), ("rope_theta", C.c_float), ("n_threads", C.c_int),
                ("kv_dtype", C.c_int)]


KV_F32, KV_F16, KV_Q8_0 = 0, 1, 2     # KVCacheDType (kv_cache.hpp:37-41)


def lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    path = os.path.join(HERE, "liboracle.so")
    if not os.path.exists(path):
        build(with_ref=False)
    L = C.CDLL(path)
    L.orc_quantize_row_q8_0.argtypes = [f32p, i8p, C.c_int]
    L.orc_quantize_row_q8_0.restype = C.c_float
    L.orc_dequantize_row_q8_0.argtypes = [i8p, C.c_float, f32p, C.c_int]
    L.orc_flash_attn_head.argtypes = [f32p, C.c_int, f32p, f32p, C.c_int, f32p, C.c_int,
                                      C.c_int, C.c_int, C.c_int, C.c_float, C.c_int]
    L.orc_sdp_attention.argtypes = [f32p, f32p, f32p, f32p] + [C.c_int] * 4 + [C.c_float, C.c_int]
    L.orc_rms_norm.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
    L.orc_rope_tables.argtypes = [C.c_int, C.c_int, C.c_float, f32p, f32p]
    L.orc_rope_apply.argtypes = [f32p, C.c_int, C.c_int, C.c_int, C.c_int, f32p, f32p, C.c_int]
    L.orc_silu_mul.argtypes = [f32p, f32p, C.c_int64]
    L.orc_argmax.argtypes = [f32p, C.c_int]
    L.orc_argmax.restype = C.c_int
    L.orc_linear.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]
    L.orc_dequant_q8_0.argtypes = [u8p, f32p, C.c_int64]
    L.orc_dequant_q4_0.argtypes = [u8p, f32p, C.c_int64]
    L.orc_f16_to_f32.argtypes = [C.c_uint16]
    L.orc_f16_to_f32.restype = C.c_float
    L.orc_f32_to_f16_kv.argtypes = [C.c_float]
    L.orc_f32_to_f16_kv.restype = C.c_uint16
    L.orc_model_kv_raw.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
    L.orc_layer_norm.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
    L.orc_softmax.argtypes = [f32p, C.c_int, C.c_int]
    L.orc_gelu.argtypes = [f32p, C.c_int64]
    L.orc_gemm.argtypes = [f32p, f32p, f32p] + [C.c_int] * 6 + [C.c_float, C.c_float, C.c_int, C.c_int]
    L.orc_model_create.argtypes = [C.POINTER(OrcConfig)]
    L.orc_model_create.restype = C.c_void_p
    L.orc_model_destroy.argtypes = [C.c_void_p]
    L.orc_model_set_globals.argtypes = [C.c_void_p, f32p, f32p, f32p]
    L.orc_model_set_layer.argtypes = [C.c_void_p, C.c_int] + [f32p] * 9
    L.orc_model_reset.argtypes = [C.c_void_p]
    L.orc_model_used.argtypes = [C.c_void_p]
    L.orc_model_used.restype = C.c_int
    L.orc_model_forward.argtypes = [C.c_void_p, i32p, C.c_int, C.c_void_p]
    L.orc_model_forward.restype = C.c_int
    L.orc_model_forward_hidden.argtypes = [C.c_void_p, f32p, C.c_int]
    L.orc_model_forward_hidden.restype = C.c_int
    L.orc_model_kv.argtypes = [C.c_void_p, C.c_int] + [C.c_void_p] * 4
    L.orc_model_fill_kv.argtypes = [C.c_void_p, C.c_int, C.c_uint64]
    _LIB = L
    return L


def ref():
    """The reference built from its own sources, or None if never built."""
    global _REF
    if _REF is not None:
        return _REF
    path = os.path.join(HERE, "_ref", "libvlrf_ref.so")
    if not os.path.exists(path):
        return None
    R = C.CDLL(path)
    R.ref_quantize_row_q8_0.argtypes = [f32p, i8p, C.c_int]
    R.ref_quantize_row_q8_0.restype = C.c_float
    R.ref_flash_attn_head.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int,
                                      C.c_float, C.c_int]
    R.ref_rms_norm.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
    R.ref_rope.argtypes = [f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
    R.ref_linear.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int]
    R.ref_silu_mul.argtypes = [f32p, f32p, C.c_int64]
    R.ref_hw_threads.restype = C.c_int
    R.ref_model_create.argtypes = [C.c_int] * 7 + [C.c_float, C.c_float]
    R.ref_model_create.restype = C.c_void_p
    R.ref_model_create_kv.argtypes = [C.c_int] * 7 + [C.c_float, C.c_float, C.c_int]
    R.ref_model_create_kv.restype = C.c_void_p
    R.ref_model_kv_raw.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
    R.ref_f32_to_f16.argtypes = [C.c_float]
    R.ref_f32_to_f16.restype = C.c_uint16
    R.ref_layer_norm.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
    R.ref_softmax.argtypes = [f32p, C.c_int, C.c_int]
    R.ref_gelu.argtypes = [f32p, C.c_int64]
    R.ref_gemm.argtypes = [f32p, C.c_int, C.c_int, f32p, C.c_int, C.c_int, f32p, C.c_int, C.c_int,
                           C.c_float, C.c_float, C.c_int, C.c_int]
    R.ref_model_set_tensor.argtypes = [C.c_void_p, C.c_char_p, f32p, C.c_int, C.c_int]
    R.ref_model_bind.argtypes = [C.c_void_p]
    R.ref_model_reset.argtypes = [C.c_void_p]
    R.ref_model_used.argtypes = [C.c_void_p]
    R.ref_model_used.restype = C.c_int
    R.ref_model_forward.argtypes = [C.c_void_p, i32p, C.c_int, C.c_void_p]
    R.ref_model_forward.restype = C.c_int
    R.ref_model_kv.argtypes = [C.c_void_p, C.c_int] + [C.c_void_p] * 4
    R.ref_model_fill_kv.argtypes = [C.c_void_p, C.c_int, C.c_uint64]
    R.ref_model_destroy.argtypes = [C.c_void_p]
    _REF = R
    return R


# ---- thin numpy helpers ----------------------------------------------------

def quantize_row_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, dtype=np.int8)
    s = lib().orc_quantize_row_q8_0(x, q, x.size)
    return q, np.float32(s)


def flash_attn_head(Q, K, V, scale, causal):
    """Q [T,d], K/V [ctx,d] -> O [T,d] (attention.hpp:207-309)."""
    Q = np.ascontiguousarray(Q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    T, d = Q.shape
    ctx = K.shape[0]
    O = np.zeros((T, d), np.float32)
    lib().orc_flash_attn_head(Q, d, K, V, d, O, d, T, ctx, d, float(scale), int(causal))
    return O


def sdp_attention(Q, K, V, scale, causal):
    """Batched [n_h,T,d] x [n_h,ctx,d] (IBackend::sdp_attention semantics)."""
    Q = np.ascontiguousarray(Q, np.float32)
    K = np.ascontiguousarray(K, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    n_h, T, d = Q.shape
    ctx = K.shape[1]
    O = np.zeros_like(Q)
    lib().orc_sdp_attention(Q, K, V, O, n_h, T, ctx, d, float(scale), int(causal))
    return O


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    rows, D = x.reshape(-1, x.shape[-1]).shape
    out = np.zeros_like(x)
    lib().orc_rms_norm(x, w, out, rows, D, float(eps))
    return out


def rope_tables(max_seq, d_head, theta):
    half = d_head // 2
    c = np.zeros(max_seq * half, np.float32)
    s = np.zeros(max_seq * half, np.float32)
    lib().orc_rope_tables(max_seq, d_head, float(theta), c, s)
    return c, s


def rope_apply(x, n_heads, d_head, pos_offset, tables, max_seq):
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    T = x.size // (n_heads * d_head)
    lib().orc_rope_apply(x, T, n_heads, d_head, pos_offset, tables[0], tables[1], max_seq)
    return x


def silu_mul(h, g):
    h = np.array(h, np.float32, copy=True)
    g = np.array(g, np.float32, copy=True)
    lib().orc_silu_mul(h, g, h.size)
    return h


def linear(x, W, n_threads=8):
    x = np.ascontiguousarray(x, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    M, K = x.reshape(-1, x.shape[-1]).shape
    N = W.shape[0]
    y = np.zeros((M, N), np.float32)
    lib().orc_linear(x, W, y, M, K, N, int(n_threads))
    return y


def dequant_q8_0(blocks, numel):
    out = np.zeros(numel, np.float32)
    lib().orc_dequant_q8_0(np.ascontiguousarray(blocks, np.uint8), out, numel)
    return out


def dequant_q4_0(blocks, numel):
    out = np.zeros(numel, np.float32)
    lib().orc_dequant_q4_0(np.ascontiguousarray(blocks, np.uint8), out, numel)
    return out


def layer_norm(x, w, b, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    rows, D = x.shape
    lib().orc_layer_norm(x, np.ascontiguousarray(w, np.float32), np.ascontiguousarray(b, np.float32), out, rows,
                         D, float(eps))
    return out


def softmax(x):
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_softmax(y, y.shape[0], y.shape[1])
    return y


def gelu(x):
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_gelu(y.ravel(), y.size)
    return y


def gemm(A, B, C, alpha, beta, trans_a, trans_b):
    """ops::gemm semantics on stored A [rA, cA], B [rB, cB]; returns the new C."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    C = np.ascontiguousarray(C, np.float32).copy()
    M, K = (A.shape[1], A.shape[0]) if trans_a else A.shape
    N = B.shape[0] if trans_b else B.shape[1]
    lib().orc_gemm(A, B, C, M, N, K, A.shape[1], B.shape[1], N, float(alpha), float(beta), int(trans_a),
                   int(trans_b))
    return C


def f32_to_f16_kv(x):
    """KVCache's f32 -> f16 element conversion (kv_cache.hpp:68-97), elementwise."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    f = lib().orc_f32_to_f16_kv
    return np.array([f(float(v)) for v in x], np.uint16)


class Model:
    """Llama-style decoder with an F32, F16 or Q8_0 KV cache (TransformerModel
    restatement; cfg["kv_dtype"], default Q8_0).

    `weights` is a dict of f32 numpy arrays keyed like the reference WeightMap
    (transformer.hpp:566-629 names plus `layers.{l}.ffn.gate.weight`)."""

    def __init__(self, cfg, weights, n_threads=8):
        self.cfg = cfg
        self.w = weights  # keep arrays alive
        c = OrcConfig(cfg["vocab_size"], cfg["d_model"], cfg["d_ff"], cfg["n_heads"],
                      cfg["n_kv_heads"], cfg["n_layers"], cfg["max_seq_len"],
                      cfg["norm_eps"], cfg["rope_theta"], n_threads, cfg.get("kv_dtype", KV_Q8_0))
        L = lib()
        self.h = L.orc_model_create(C.byref(c))
        L.orc_model_set_globals(self.h, weights["embed.weight"], weights["ln_final.weight"],
                                weights["lm_head.weight"])
        for l in range(cfg["n_layers"]):
            p = f"layers.{l}."
            L.orc_model_set_layer(self.h, l, weights[p + "ln1.weight"], weights[p + "ln2.weight"],
                                  weights[p + "attn.q_proj.weight"], weights[p + "attn.k_proj.weight"],
                                  weights[p + "attn.v_proj.weight"], weights[p + "attn.o_proj.weight"],
                                  weights[p + "ffn.gate.weight"], weights[p + "ffn.fc1.weight"],
                                  weights[p + "ffn.fc2.weight"])

    def reset(self):
        lib().orc_model_reset(self.h)

    @property
    def used(self):
        return lib().orc_model_used(self.h)

    def forward(self, ids, want_logits=False):
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.zeros(self.cfg["vocab_size"], np.float32) if want_logits else None
        tok = lib().orc_model_forward(self.h, ids, ids.size,
                                      logits.ctypes.data if want_logits else None)
        if tok < 0:
            raise RuntimeError("oracle forward failed (cache overflow or bad token id)")
        return (tok, logits) if want_logits else tok

    def forward_hidden(self, x):
        """The layers over embedded rows x [T, d_model]; returns the residual
        stream after the last layer (a new array) and appends T cache rows."""
        y = np.ascontiguousarray(x, np.float32).copy()
        if lib().orc_model_forward_hidden(self.h, y, y.shape[0]) != 0:
            raise RuntimeError("oracle forward_hidden failed (cache overflow)")
        return y

    def fill_kv(self, used, seed=1):
        lib().orc_model_fill_kv(self.h, int(used), int(seed))

    def kv(self, l):
        """(K int8 [max_seq,row], V int8, K scales [max_seq], V scales) views."""
        ptrs = [C.c_void_p() for _ in range(4)]
        lib().orc_model_kv(self.h, l, *[C.byref(p) for p in ptrs])
        c = self.cfg
        row = c["n_kv_heads"] * (c["d_model"] // c["n_heads"])
        n = c["max_seq_len"]
        kq = np.ctypeslib.as_array(C.cast(ptrs[0], C.POINTER(C.c_int8)), (n, row))
        vq = np.ctypeslib.as_array(C.cast(ptrs[1], C.POINTER(C.c_int8)), (n, row))
        ks = np.ctypeslib.as_array(C.cast(ptrs[2], C.POINTER(C.c_float)), (n,))
        vs = np.ctypeslib.as_array(C.cast(ptrs[3], C.POINTER(C.c_float)), (n,))
        return kq, vq, ks, vs

    def kv_raw(self, l):
        """Layer l's K and V storage [max_seq, row] in the cache's own element
        type: float32 (F32), uint16 f16 bits (F16) or int8 codes (Q8_0)."""
        k, v = C.c_void_p(), C.c_void_p()
        lib().orc_model_kv_raw(self.h, l, C.byref(k), C.byref(v))
        c = self.cfg
        row = c["n_kv_heads"] * (c["d_model"] // c["n_heads"])
        ct = {KV_F32: C.c_float, KV_F16: C.c_uint16}.get(c.get("kv_dtype", KV_Q8_0), C.c_int8)
        shape = (c["max_seq_len"], row)
        return (np.ctypeslib.as_array(C.cast(k, C.POINTER(ct)), shape),
                np.ctypeslib.as_array(C.cast(v, C.POINTER(ct)), shape))

    def __del__(self):
        try:
            lib().orc_model_destroy(self.h)
        except Exception:
            pass


class RefModel:
    """The reference TransformerModel itself (oracle/_ref, built from its own
    sources) behind the same calls as Model: Q8_0 KV cache, the reference's
    own thread pool (every hardware thread, ops.hpp:34-37).  Weights are
    borrowed, so this object keeps `weights` alive."""

    def __init__(self, cfg, weights):
        R = ref()
        if R is None:
            raise RuntimeError("oracle/_ref/libvlrf_ref.so was not built")
        self.cfg = cfg
        self.w = weights
        self.h = R.ref_model_create(cfg["vocab_size"], cfg["d_model"], cfg["d_ff"], cfg["n_heads"],
                                    cfg["n_kv_heads"], cfg["n_layers"], cfg["max_seq_len"],
                                    cfg["norm_eps"], cfg["rope_theta"])
        for k, v in weights.items():
            R.ref_model_set_tensor(self.h, k.encode(), v, v.shape[0] if v.ndim == 2 else 0, v.shape[-1])
        R.ref_model_bind(self.h)

    @staticmethod
    def threads():
        return ref().ref_hw_threads()

    def reset(self):
        ref().ref_model_reset(self.h)

    @property
    def used(self):
        return ref().ref_model_used(self.h)

    def fill_kv(self, used, seed=1):
        """Same seeded codes and scales as Model.fill_kv."""
        ref().ref_model_fill_kv(self.h, int(used), int(seed))

    def forward(self, ids, want_logits=False):
        ids = np.ascontiguousarray(ids, np.int32)
        logits = np.zeros(self.cfg["vocab_size"], np.float32) if want_logits else None
        tok = ref().ref_model_forward(self.h, ids, ids.size,
                                      logits.ctypes.data if want_logits else None)
        return (tok, logits) if want_logits else tok

    def __del__(self):
        try:
            ref().ref_model_destroy(self.h)
        except Exception:
            pass
