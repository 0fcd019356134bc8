"""vlrf_hip_attn_decode_noalloc (no reference counterpart: the decode attention
entry point for callers that cannot allocate) against vlrf_hip_attn_decode
through the C ABI: the same kernels, so the outputs are bit-identical; two
calls in a row, the second with a smaller shape (fewer heads, a shorter
context, a different cache dtype), and the size limit of its fixed scratch."""
import ctypes as C

import numpy as np
import pytest

import vlrf_amd as V
from vlrf_amd import formats as F
from vlrf_amd._lib import ERR_ARG

pytestmark = pytest.mark.gpu


def _cache(ctx, kv_dtype, n_kv, cap, seed):
    kv = V.KVCache(ctx, 2, cap, n_kv, 64, dtype=kv_dtype)
    k = ctx.to_device(F.normal(seed, "na.k", cap * n_kv * 64))
    v = ctx.to_device(F.normal(seed, "na.v", cap * n_kv * 64))
    kv.append(1, k, v, cap)
    return kv


def _both(ctx, kv, n_heads, ctx_len, seed):
    q = ctx.to_device(F.normal(seed, "na.q", n_heads * 64))
    a, b = ctx.alloc(n_heads * 64 * 4), ctx.alloc(n_heads * 64 * 4)
    V.check(V.lib().vlrf_hip_attn_decode(kv.h, 1, q.ptr, a.ptr, n_heads, ctx_len, C.c_float(0.125)))
    V.check(V.lib().vlrf_hip_attn_decode_noalloc(kv.h, 1, q.ptr, b.ptr, n_heads, ctx_len, C.c_float(0.125)))
    ctx.sync()
    return a.download((n_heads * 64,)), b.download((n_heads * 64,))


def test_noalloc_equals_attn_decode_twice(ctx):
    print("[case] noalloc decode attention: 32 q / 4 kv heads, Q8_0 cache, ctx 4096", flush=True)
    kv = _cache(ctx, V.KV_Q8_0, 4, 4096, 71)
    a, b = _both(ctx, kv, 32, 4096, 71)
    assert np.array_equal(a, b) and np.all(np.isfinite(a))
    print("[case] noalloc decode attention: 8 q / 2 kv heads, F16 cache, ctx 700", flush=True)
    kv2 = _cache(ctx, V.KV_F16, 2, 1024, 72)
    a, b = _both(ctx, kv2, 8, 700, 72)
    assert np.array_equal(a, b) and np.all(np.isfinite(a))


def test_noalloc_rejects_shapes_beyond_its_scratch(ctx):
    print("[case] noalloc decode attention: 64 heads x 128 splits exceeds the fixed scratch", flush=True)
    kv = _cache(ctx, V.KV_Q8_0, 8, 8192, 73)
    q = ctx.to_device(F.normal(73, "na.q", 64 * 64))
    o = ctx.alloc(64 * 64 * 4)
    rc = V.lib().vlrf_hip_attn_decode_noalloc(kv.h, 1, q.ptr, o.ptr, 64, 8192, C.c_float(0.125))
    assert rc == ERR_ARG and b"exceed the fixed scratch" in V.lib().vlrf_hip_last_error()
    # the same cache at a context that fits: still usable
    rc = V.lib().vlrf_hip_attn_decode_noalloc(kv.h, 1, q.ptr, o.ptr, 64, 4096, C.c_float(0.125))
    assert rc == 0
