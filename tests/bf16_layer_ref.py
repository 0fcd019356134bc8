"""A float64 model of the prefill path's own precision scheme, for checking
that the matrix-core kernels compute exactly the intended mixed-precision
arithmetic.  It rounds to bf16 where the GPU path does (normalised activations,
decoded weights, q, dequantized K/V, softmax numerators P, the attention
output, the SwiGLU output) and keeps f32/f64 elsewhere (norms, RoPE, the Q8_0
KV quantizer, accumulations, residual stream).  The parity claim itself is
against the f32 oracle; this reference only separates implementation error
from the rounding the bf16 operands imply."""
import numpy as np


def bf16(a):
    """Round to bfloat16 (nearest even) and return as float64."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def rms_norm(x, w, eps):
    x32 = x.astype(np.float32)
    ss = (x32.astype(np.float64) ** 2).sum(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(ss / x.shape[1] + eps)
    return x32 * inv.astype(np.float32) * w.astype(np.float32)


def rope(x, T, n_heads, dh, pos0, theta):
    half = dh // 2
    i = np.arange(half, dtype=np.float32)
    freq = (1.0 / np.power(np.float32(theta), (2.0 * i / dh).astype(np.float32))).astype(np.float32)
    pos = (pos0 + np.arange(T)).astype(np.float32)[:, None]
    ang = (pos * freq[None, :]).astype(np.float32)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x = x.reshape(T, n_heads, dh).astype(np.float32)
    a, b = x[..., :half].copy(), x[..., half:].copy()
    out = np.empty_like(x)
    out[..., :half] = a * c[:, None, :] - b * s[:, None, :]
    out[..., half:] = b * c[:, None, :] + a * s[:, None, :]
    return out.reshape(T, n_heads * dh)


def quant_rows(r):
    """quantize_row_q8_0 per row (kv_cache.hpp:102-117), returns dequantized f32."""
    r = r.astype(np.float32)
    amax = np.abs(r).max(axis=1).astype(np.float32)
    scale = np.where(amax != 0, amax / np.float32(127), 0).astype(np.float32)
    inv = np.where(amax != 0, np.float32(1) / np.where(scale != 0, scale, 1), 0).astype(np.float32)
    v = (r * inv[:, None]).astype(np.float32)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127)
    return (q.astype(np.float32) * scale[:, None]).astype(np.float32)


def layer(x, w, cfg, pos0=0, kcache=None, vcache=None):
    """One pre-norm block over T rows of x (f32), weights `w` (decoded f32)
    keyed like the WeightMap for layer 0.  Returns (x_out, K, V) with the
    dequantized cache rows [0, pos0+T)."""
    T, D = x.shape
    H, G = cfg["n_heads"], cfg["n_kv_heads"]
    dh = D // H
    dkv = G * dh
    eps = cfg["norm_eps"]
    p = "layers.0."
    a = bf16(rms_norm(x, w[p + "ln1.weight"], eps))
    q = (a @ bf16(w[p + "attn.q_proj.weight"]).T).astype(np.float32)
    k = (a @ bf16(w[p + "attn.k_proj.weight"]).T).astype(np.float32)
    v = (a @ bf16(w[p + "attn.v_proj.weight"]).T).astype(np.float32)
    q = rope(q, T, H, dh, pos0, cfg["rope_theta"])
    k = rope(k, T, G, dh, pos0, cfg["rope_theta"])
    K = quant_rows(k) if kcache is None else np.concatenate([kcache, quant_rows(k)])
    Vv = quant_rows(v) if vcache is None else np.concatenate([vcache, quant_rows(v)])
    Kb, Vb = bf16(K), bf16(Vv)
    scale = 1.0 / np.sqrt(np.float32(dh))
    att = np.zeros((T, D))
    ctx = pos0 + T
    mask = np.arange(ctx)[None, :] <= (pos0 + np.arange(T))[:, None]
    for h in range(H):
        g = h // (H // G)
        qh = bf16(q[:, h * dh:(h + 1) * dh])
        s = (qh @ Kb[:, g * dh:(g + 1) * dh].T) * scale
        s = np.where(mask, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        e = np.exp(s - m)
        l = e.sum(axis=1, keepdims=True)
        att[:, h * dh:(h + 1) * dh] = (bf16(e) @ Vb[:, g * dh:(g + 1) * dh]) / l
    x1 = x.astype(np.float64) + bf16(att) @ bf16(w[p + "attn.o_proj.weight"]).T
    a2 = bf16(rms_norm(x1.astype(np.float32), w[p + "ln2.weight"], eps))
    gg = a2 @ bf16(w[p + "ffn.gate.weight"]).T
    uu = a2 @ bf16(w[p + "ffn.fc1.weight"]).T
    hh = bf16(uu * (gg / (1.0 + np.exp(-gg))))
    x2 = x1 + hh @ bf16(w[p + "ffn.fc2.weight"]).T
    return x2.astype(np.float32), K, Vv
