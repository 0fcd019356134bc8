"""Python objects over the C ABI handles (context, buffers, cache, weights,
model).  Names and argument meanings follow the reference interfaces the ABI
replaces: IBackend (include/backend/ibackend.hpp), KVCache
(include/model/kv_cache.hpp), compute::linear (include/model/compute.hpp) and
TransformerModel (include/model/transformer.hpp)."""
import ctypes as C

import numpy as np

from ._lib import lib, check, ModelConfig, DT_F32, KV_F16, KV_F32, KV_Q8_0


class DeviceBuffer:
    """A device allocation of the context (vlrf_hip_malloc)."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().vlrf_hip_malloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, ctx, a):
        a = np.ascontiguousarray(a)
        b = cls(ctx, max(a.nbytes, 1))
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes, "upload larger than the buffer"
        check(lib().vlrf_hip_h2d(self.ctx.h, self.ptr, a.ctypes.data, a.nbytes))

    def download(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes, "download larger than the buffer"
        check(lib().vlrf_hip_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def zero(self):
        check(lib().vlrf_hip_memset(self.ctx.h, self.ptr, 0, self.nbytes))

    def copy_from(self, src, nbytes=None):
        """Device-to-device copy from another DeviceBuffer (queued, no wait)."""
        n = src.nbytes if nbytes is None else nbytes
        assert n <= self.nbytes and n <= src.nbytes, "copy larger than a buffer"
        check(lib().vlrf_hip_d2d(self.ctx.h, self.ptr, src.ptr, n))

    def free(self):
        if self.ptr:
            check(lib().vlrf_hip_free(self.ctx.h, self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One device + one HIP stream (vlrf_hip_init).  The backend object of the
    reference's BackendRegistry (backend.hpp:544-578) maps to one Context."""

    def __init__(self, device=0):
        h = C.c_void_p()
        check(lib().vlrf_hip_init(device, C.byref(h)))
        self.h = h.value

    @staticmethod
    def device_count():
        return lib().vlrf_hip_device_count()

    def device_info(self):
        buf = C.create_string_buffer(256)
        check(lib().vlrf_hip_device_info(self.h, buf, 256))
        return buf.value.decode()

    def sync(self):
        check(lib().vlrf_hip_sync(self.h))

    def stream(self):
        return lib().vlrf_hip_stream(self.h)

    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def to_device(self, a):
        return DeviceBuffer.from_array(self, a)

    def timer_start(self):
        check(lib().vlrf_hip_timer_start(self.h))

    def timer_stop(self):
        ms = C.c_float()
        check(lib().vlrf_hip_timer_stop(self.h, C.byref(ms)))
        return ms.value

    # ---- ops on device buffers -------------------------------------------
    def sdp_attention(self, Q, K, V, O, n_h, T, ctx_len, d_h, scale, causal):
        """IBackend::sdp_attention (ibackend.hpp:79-82) on device buffers."""
        check(lib().vlrf_hip_attn_f32(self.h, Q.ptr, K.ptr, V.ptr, O.ptr, n_h, T, ctx_len, d_h,
                                      float(scale), int(bool(causal))))

    def qlinear(self, w, x, y, M, norm_w=None, eps=1e-5, residual=None):
        check(lib().vlrf_hip_qlinear(self.h, w.h, x.ptr, y.ptr, M, norm_w.ptr if norm_w else None,
                                     float(eps), residual.ptr if residual else None))

    def qlinear_swiglu(self, wg, wu, x, h, M, norm_w=None, eps=1e-5):
        check(lib().vlrf_hip_qlinear_swiglu(self.h, wg.h, wu.h, x.ptr, h.ptr, M,
                                            norm_w.ptr if norm_w else None, float(eps)))

    def gemm_f32(self, A, B, C, M, N, K, alpha=1.0, beta=0.0, trans_a=False, trans_b=False,
                 lda=None, ldb=None, ldc=None):
        """IBackend::gemm (ops.hpp:170-310) on device buffers: C = beta*C + alpha*op(A).op(B)."""
        lda = lda or (M if trans_a else K)
        ldb = ldb or (K if trans_b else N)
        ldc = ldc or N
        check(lib().vlrf_hip_gemm_f32(self.h, A.ptr, B.ptr, C.ptr, M, N, K, lda, ldb, ldc, float(alpha),
                                      float(beta), int(trans_a), int(trans_b)))

    def layer_norm(self, x, w, b, out, rows, D, eps):
        check(lib().vlrf_hip_layer_norm(self.h, x.ptr, w.ptr, b.ptr, out.ptr, rows, D, float(eps)))

    def softmax(self, x, rows, D):
        check(lib().vlrf_hip_softmax(self.h, x.ptr, rows, D))

    def gelu(self, x, n):
        check(lib().vlrf_hip_gelu(self.h, x.ptr, n))

    def add(self, dst, src, n):
        check(lib().vlrf_hip_add(self.h, dst.ptr, src.ptr, n))

    def rms_norm(self, x, w, out, rows, D, eps):
        check(lib().vlrf_hip_rmsnorm(self.h, x.ptr, w.ptr, out.ptr, rows, D, float(eps)))

    def rope(self, x, T, n_heads, d_head, pos_offset, max_seq, theta):
        check(lib().vlrf_hip_rope(self.h, x.ptr, T, n_heads, d_head, pos_offset, max_seq,
                                  float(theta)))

    def close(self):
        if self.h:
            lib().vlrf_hip_shutdown(self.h)
            self.h = None


class QuantWeight:
    """A resident weight [N, K] uploaded from GGUF-layout host blocks."""

    def __init__(self, ctx, blocks, dtype, N, K):
        self.ctx = ctx
        self.dtype, self.N, self.K = dtype, N, K
        blocks = np.ascontiguousarray(blocks)
        h = C.c_void_p()
        check(lib().vlrf_hip_weight_upload(ctx.h, blocks.ctypes.data, dtype, N, K, C.byref(h)))
        self.h = h.value

    @property
    def device_bytes(self):
        return lib().vlrf_hip_weight_bytes(self.h)

    def __del__(self):
        try:
            if self.h:
                lib().vlrf_hip_weight_free(self.h)
                self.h = None
        except Exception:
            pass


class KVCache:
    """Device Q8_0 KV cache for n_layers (KVCache, kv_cache.hpp:132-293)."""

    def __init__(self, ctx, n_layers, max_seq_len, n_kv_heads, d_head, dtype=KV_Q8_0):
        self.ctx = ctx
        self.n_layers, self.max_seq_len, self.n_kv_heads, self.d_head = (n_layers, max_seq_len,
                                                                         n_kv_heads, d_head)
        self.row_dim = n_kv_heads * d_head
        self.dtype = dtype
        h = C.c_void_p()
        check(lib().vlrf_hip_kv_create(ctx.h, n_layers, max_seq_len, n_kv_heads, d_head, dtype,
                                       C.byref(h)))
        self.h = h.value

    def used(self, layer=0):
        return lib().vlrf_hip_kv_used(self.h, layer)

    def reset(self):
        check(lib().vlrf_hip_kv_reset(self.h))

    def append(self, layer, k, v, T):
        check(lib().vlrf_hip_kv_append(self.h, layer, k.ptr, v.ptr, T))

    def read(self, layer, row0, n):
        """(K [n,row], V [n,row], K scales [n], V scales [n]) in the reference's
        token-major layout: int8 codes with f32 scales (Q8_0), or uint16 f16
        bits / float32 elements with the scales None."""
        et = {KV_F32: np.float32, KV_F16: np.uint16}.get(self.dtype, np.int8)
        kq = np.zeros((n, self.row_dim), et)
        vq = np.zeros((n, self.row_dim), et)
        q8 = self.dtype == KV_Q8_0
        ks = np.zeros(n, np.float32) if q8 else None
        vs = np.zeros(n, np.float32) if q8 else None
        check(lib().vlrf_hip_kv_read(self.h, layer, row0, n, kq.ctypes.data, vq.ctypes.data,
                                     ks.ctypes.data if q8 else None, vs.ctypes.data if q8 else None))
        return kq, vq, ks, vs

    def dequant_into(self, layer, ctx_len, K_out, V_out):
        check(lib().vlrf_hip_kv_dequant(self.h, layer, ctx_len, K_out.ptr, V_out.ptr))

    def attention_decode(self, layer, q, out, n_heads, ctx_len, scale):
        check(lib().vlrf_hip_attn_decode(self.h, layer, q.ptr, out.ptr, n_heads, ctx_len,
                                         float(scale)))

    def __del__(self):
        try:
            if self.h:
                lib().vlrf_hip_kv_destroy(self.h)
                self.h = None
        except Exception:
            pass


class Model:
    """Device-resident Llama-style decoder (TransformerModel decode path)."""

    def __init__(self, ctx, cfg):
        self.ctx = ctx
        self.cfg = dict(cfg)
        c = ModelConfig(cfg["vocab_size"], cfg["d_model"], cfg["d_ff"], cfg["n_heads"],
                        cfg["n_kv_heads"], cfg["n_layers"], cfg["max_seq_len"], cfg["norm_eps"],
                        cfg["rope_theta"], cfg["weight_dtype"], cfg.get("kv_dtype", KV_Q8_0))
        h = C.c_void_p()
        check(lib().vlrf_hip_model_create(ctx.h, C.byref(c), C.byref(h)))
        self.h = h.value

    def set_weight(self, name, host, dtype, rows, cols):
        host = np.ascontiguousarray(host)
        check(lib().vlrf_hip_model_set_weight(self.h, name.encode(), host.ctypes.data, dtype,
                                              rows, cols))

    def load_nfw(self, path):
        """Sets the model's tensors from an NFW v1/v2/v3 file (vlrf_hip_model_load_nfw);
        returns how many were set."""
        n = C.c_int()
        check(lib().vlrf_hip_model_load_nfw(self.h, str(path).encode(), C.byref(n)))
        return n.value

    def reset(self):
        check(lib().vlrf_hip_model_reset(self.h))

    @property
    def used(self):
        return lib().vlrf_hip_model_used(self.h)

    def step(self, token, want_logits=False):
        nxt = C.c_int32()
        logits = np.zeros(self.cfg["vocab_size"], np.float32) if want_logits else None
        check(lib().vlrf_hip_model_step(self.h, int(token), C.byref(nxt),
                                        logits.ctypes.data if want_logits else None))
        return (nxt.value, logits) if want_logits else nxt.value

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        nxt = C.c_int32()
        check(lib().vlrf_hip_model_prefill(self.h, ids.ctypes.data, ids.size, C.byref(nxt)))
        return nxt.value

    def prefill_mfma(self, ids):
        """Batched prefill on the matrix cores (bf16 GEMMs and attention)."""
        ids = np.ascontiguousarray(ids, np.int32)
        nxt = C.c_int32()
        check(lib().vlrf_hip_model_prefill_mfma(self.h, ids.ctypes.data, ids.size, C.byref(nxt)))
        return nxt.value

    def forward_hidden(self, x, out=None):
        """All layers over embedded rows x (DeviceBuffer [T][d_model]); returns
        the output DeviceBuffer (out, or a new one)."""
        T = x.nbytes // (4 * self.cfg["d_model"])
        out = out if out is not None else self.ctx.alloc(x.nbytes)
        check(lib().vlrf_hip_model_forward_hidden(self.h, x.ptr, T, out.ptr))
        return out

    def kv_rows(self, layer, row0, n):
        """(K [n,row], V, K scales [n], V scales) of the model's cache: int8 codes
        and f32 scales (Q8_0), or uint16 f16 bits / float32 with scales None."""
        c = self.cfg
        row = c["n_kv_heads"] * (c["d_model"] // c["n_heads"])
        dt = c.get("kv_dtype", KV_Q8_0)
        et = {KV_F32: np.float32, KV_F16: np.uint16}.get(dt, np.int8)
        kq, vq = np.zeros((n, row), et), np.zeros((n, row), et)
        q8 = dt == KV_Q8_0
        ks = np.zeros(n, np.float32) if q8 else None
        vs = np.zeros(n, np.float32) if q8 else None
        check(lib().vlrf_hip_model_kv_read(self.h, layer, row0, n, kq.ctypes.data, vq.ctypes.data,
                                           ks.ctypes.data if q8 else None, vs.ctypes.data if q8 else None))
        return kq, vq, ks, vs

    def generate_ids(self, first, n_steps):
        out = np.zeros(n_steps, np.int32)
        check(lib().vlrf_hip_model_generate(self.h, int(first), n_steps, out.ctypes.data))
        return out

    def generate_async(self, first, n_steps):
        check(lib().vlrf_hip_model_generate_async(self.h, int(first), n_steps))

    def read_generated(self, n):
        out = np.zeros(n, np.int32)
        check(lib().vlrf_hip_model_read_generated(self.h, out.ctypes.data, n))
        return out

    def generate(self, prompt_ids, max_new_tokens):
        """Greedy TransformerModel::generate (transformer.hpp:439-547) with default
        penalties: reset, prefill the prompt, then decode starting from the last
        prompt id (which the reference feeds again as the first decode input)."""
        prompt_ids = np.ascontiguousarray(prompt_ids, np.int32)
        self.reset()
        self.prefill(prompt_ids)
        return self.generate_ids(int(prompt_ids[-1]), max_new_tokens)

    LAUNCH_KINDS = ("qkv_attn", "attn", "o_proj", "gate_up", "down", "lm_head", "argmax", "other")

    def time_launches(self, first, n_steps):
        """n_steps greedy steps from `first` with every launch timed by its own
        events: {kind: (summed kernel us, launches)} for the kinds launched."""
        us = (C.c_double * 8)()
        calls = (C.c_int * 8)()
        check(lib().vlrf_hip_model_time_launches(self.h, int(first), n_steps, us, calls))
        return {k: (us[i], calls[i]) for i, k in enumerate(self.LAUNCH_KINDS) if calls[i]}

    def step_bytes(self, ctx_len):
        out = (C.c_double * 3)()
        check(lib().vlrf_hip_model_step_bytes(self.h, ctx_len, out))
        return list(out)

    def __del__(self):
        try:
            if self.h:
                lib().vlrf_hip_model_destroy(self.h)
                self.h = None
        except Exception:
            pass
