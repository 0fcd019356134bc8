"""ctypes declarations for libvlrf_hip.so (include/vlrf_hip.h)."""
import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libvlrf_hip.so")

DT_F32, DT_Q4_0, DT_Q8_0 = 0, 2, 8
KV_F32, KV_F16, KV_Q8_0 = 0, 1, 2     # KVCacheDType (kv_cache.hpp:37-41)

OK, ERR_ARG, ERR_RUNTIME, ERR_NOMEM, ERR_OVERFLOW, ERR_NODEV = 0, -1, -2, -3, -4, -5


class HipError(RuntimeError):
    def __init__(self, rc, msg):
        super().__init__(f"vlrf_hip error {rc}: {msg}")
        self.rc = rc


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab_size", "d_model", "d_ff", "n_heads", "n_kv_heads",
                                         "n_layers", "max_seq_len")] + \
               [("norm_eps", C.c_float), ("rope_theta", C.c_float), ("weight_dtype", C.c_int32),
                ("kv_dtype", C.c_int32)]


vp, i32, i64, u64, f32, sz = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_size_t

# name: (restype, argtypes)
_SIGS = {
    "vlrf_hip_last_error": (C.c_char_p, []),
    "vlrf_hip_device_count": (i32, []),
    "vlrf_hip_init": (i32, [i32, C.POINTER(vp)]),
    "vlrf_hip_shutdown": (None, [vp]),
    "vlrf_hip_device_info": (i32, [vp, C.c_char_p, sz]),
    "vlrf_hip_sync": (i32, [vp]),
    "vlrf_hip_stream": (vp, [vp]),
    "vlrf_hip_malloc": (i32, [vp, sz, C.POINTER(vp)]),
    "vlrf_hip_free": (i32, [vp, vp]),
    "vlrf_hip_h2d": (i32, [vp, vp, vp, sz]),
    "vlrf_hip_d2h": (i32, [vp, vp, vp, sz]),
    "vlrf_hip_memset": (i32, [vp, vp, i32, sz]),
    "vlrf_hip_d2d": (i32, [vp, vp, vp, sz]),
    "vlrf_hip_timer_start": (i32, [vp]),
    "vlrf_hip_timer_stop": (i32, [vp, C.POINTER(f32)]),
    "vlrf_hip_attn_f32": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, f32, i32]),
    "vlrf_hip_kv_create": (i32, [vp, i32, i32, i32, i32, i32, C.POINTER(vp)]),
    "vlrf_hip_kv_destroy": (None, [vp]),
    "vlrf_hip_kv_reset": (i32, [vp]),
    "vlrf_hip_kv_used": (i32, [vp, i32]),
    "vlrf_hip_kv_append": (i32, [vp, i32, vp, vp, i32]),
    "vlrf_hip_kv_read": (i32, [vp, i32, i32, i32, vp, vp, vp, vp]),
    "vlrf_hip_kv_dequant": (i32, [vp, i32, i32, vp, vp]),
    "vlrf_hip_attn_decode": (i32, [vp, i32, vp, vp, i32, i32, f32]),
    "vlrf_hip_attn_decode_noalloc": (i32, [vp, i32, vp, vp, i32, i32, f32]),
    "vlrf_hip_weight_upload": (i32, [vp, vp, i32, i32, i32, C.POINTER(vp)]),
    "vlrf_hip_weight_free": (None, [vp]),
    "vlrf_hip_weight_bytes": (sz, [vp]),
    "vlrf_hip_qlinear": (i32, [vp, vp, vp, vp, i32, vp, f32, vp]),
    "vlrf_hip_qlinear_swiglu": (i32, [vp, vp, vp, vp, vp, i32, vp, f32]),
    "vlrf_hip_rmsnorm": (i32, [vp, vp, vp, vp, i32, i32, f32]),
    "vlrf_hip_rope": (i32, [vp, vp, i32, i32, i32, i32, i32, f32]),
    "vlrf_quantize_q8_0": (i32, [vp, vp, i64]),
    "vlrf_quantize_q4_0": (i32, [vp, vp, i64]),
    "vlrf_dequantize": (i32, [vp, i32, vp, i64]),
    "vlrf_synth_normal": (i32, [u64, u64, f32, vp, i64]),
    "vlrf_synth_tokens": (i32, [u64, u64, i32, vp, i64]),
    "vlrf_hip_model_create": (i32, [vp, C.POINTER(ModelConfig), C.POINTER(vp)]),
    "vlrf_hip_model_destroy": (None, [vp]),
    "vlrf_hip_model_set_weight": (i32, [vp, C.c_char_p, vp, i32, i32, i32]),
    "vlrf_hip_model_get_config": (i32, [vp, C.POINTER(ModelConfig)]),
    "vlrf_hip_gemm_f32": (i32, [vp, vp, vp, vp] + [i32] * 6 + [f32, f32, i32, i32]),
    "vlrf_hip_layer_norm": (i32, [vp, vp, vp, vp, vp, i32, i32, f32]),
    "vlrf_hip_softmax": (i32, [vp, vp, i32, i32]),
    "vlrf_hip_gelu": (i32, [vp, vp, i64]),
    "vlrf_hip_add": (i32, [vp, vp, vp, i64]),
    "vlrf_hip_model_load_nfw": (i32, [vp, C.c_char_p, C.POINTER(C.c_int)]),
    "vlrf_nfw_open": (i32, [C.c_char_p, C.POINTER(vp)]),
    "vlrf_nfw_close": (None, [vp]),
    "vlrf_nfw_version": (i32, [vp]),
    "vlrf_nfw_count": (i32, [vp]),
    "vlrf_nfw_find": (i32, [vp, C.c_char_p]),
    "vlrf_nfw_tensor_info": (i32, [vp, i32, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(C.c_int),
                                   C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "vlrf_nfw_read": (i32, [vp, i32, vp, i64]),
    "vlrf_nfw_read_f32": (i32, [vp, i32, vp, i64]),
    "vlrf_hip_model_reset": (i32, [vp]),
    "vlrf_hip_model_used": (i32, [vp]),
    "vlrf_hip_model_step": (i32, [vp, i32, C.POINTER(C.c_int32), vp]),
    "vlrf_hip_model_prefill": (i32, [vp, vp, i32, C.POINTER(C.c_int32)]),
    "vlrf_hip_model_prefill_mfma": (i32, [vp, vp, i32, C.POINTER(C.c_int32)]),
    "vlrf_hip_model_forward_hidden": (i32, [vp, vp, i32, vp]),
    "vlrf_hip_model_kv_read": (i32, [vp, i32, i32, i32, vp, vp, vp, vp]),
    "vlrf_hip_model_generate": (i32, [vp, i32, i32, vp]),
    "vlrf_hip_model_generate_async": (i32, [vp, i32, i32]),
    "vlrf_hip_model_read_generated": (i32, [vp, vp, i32]),
    "vlrf_hip_model_step_bytes": (i32, [vp, i32, C.POINTER(C.c_double)]),
    "vlrf_hip_model_time_launches": (i32, [vp, i32, i32, C.POINTER(C.c_double), C.POINTER(C.c_int)]),
}

_LIB = None


def lib():
    """Loads libvlrf_hip.so; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m vlrf_amd.csrc.build` "
                          "(there is no CPU fallback)")
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def last_error():
    return lib().vlrf_hip_last_error().decode(errors="replace")


def check(rc):
    if rc != OK:
        raise HipError(rc, last_error())
    return rc
