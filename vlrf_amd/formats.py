"""Host-side block formats, seeded synthetic data and the benchmark model
shapes (host functions of libvlrf_hip.so; no device needed)."""
import zlib

import numpy as np

from ._lib import lib, check, DT_F32, DT_Q4_0, DT_Q8_0

BLOCK_BYTES = {DT_Q8_0: 34, DT_Q4_0: 18}


def quantize(x, dtype):
    """f32 -> GGUF blocks (uint8, rows of K/32 blocks); F32 passes through."""
    x = np.ascontiguousarray(x, np.float32)
    if dtype == DT_F32:
        return x
    n = x.size
    out = np.zeros(n // 32 * BLOCK_BYTES[dtype], np.uint8)
    fn = lib().vlrf_quantize_q8_0 if dtype == DT_Q8_0 else lib().vlrf_quantize_q4_0
    check(fn(x.ctypes.data, out.ctypes.data, n))
    return out


def dequantize(blocks, dtype, n):
    out = np.zeros(n, np.float32)
    blocks = np.ascontiguousarray(blocks)
    check(lib().vlrf_dequantize(blocks.ctypes.data, dtype, out.ctypes.data, n))
    return out


def stream_id(name):
    return zlib.crc32(name.encode())


def normal(seed, name, n, std=1.0):
    """std * N(0,1), counter-based: identical on every host for (seed, name)."""
    out = np.empty(n, np.float32)
    check(lib().vlrf_synth_normal(seed, stream_id(name), float(std), out.ctypes.data, n))
    return out


def tokens(seed, name, n, vocab):
    out = np.empty(n, np.int32)
    check(lib().vlrf_synth_tokens(seed, stream_id(name), vocab, out.ctypes.data, n))
    return out


# ---- model shapes ------------------------------------------------------------
def llama_1b(max_seq_len=2048 + 128, weight_dtype=DT_Q8_0):
    """The 1.1B Llama-style decode configuration of the benchmark."""
    return dict(vocab_size=32000, d_model=2048, d_ff=5632, n_heads=32, n_kv_heads=4,
                n_layers=22, max_seq_len=max_seq_len, norm_eps=1e-5, rope_theta=10000.0,
                weight_dtype=weight_dtype)


def llama8b_layer(weight_dtype=DT_Q8_0, max_seq_len=2048, n_layers=1, vocab_size=256):
    """One Llama-8B-shape decoder layer (the prefill benchmark configuration:
    hidden 4096, 32/8 heads, head_dim 128, FFN 14336 SwiGLU).  The vocabulary
    is small: the layer's input is given as embedded rows."""
    return dict(vocab_size=vocab_size, d_model=4096, d_ff=14336, n_heads=32, n_kv_heads=8,
                n_layers=n_layers, max_seq_len=max_seq_len, norm_eps=1e-5, rope_theta=10000.0,
                weight_dtype=weight_dtype)


def tiny(weight_dtype=DT_Q8_0, n_layers=2, max_seq_len=160):
    """A small configuration with the same structure (GQA 4:1, d_head 64)."""
    return dict(vocab_size=512, d_model=256, d_ff=704, n_heads=4, n_kv_heads=1,
                n_layers=n_layers, max_seq_len=max_seq_len, norm_eps=1e-5, rope_theta=10000.0,
                weight_dtype=weight_dtype)


def tensor_specs(cfg):
    """(name, rows, cols, kind) in the reference WeightMap naming
    (transformer.hpp:566-629) plus the SwiGLU gate (feedforward.hpp:39-46).
    kind: 'proj' (quantized), 'norm' (f32), 'embed' (f32)."""
    D, F = cfg["d_model"], cfg["d_ff"]
    dkv = cfg["n_kv_heads"] * (D // cfg["n_heads"])
    specs = [("embed.weight", cfg["vocab_size"], D, "embed")]
    for l in range(cfg["n_layers"]):
        p = f"layers.{l}."
        specs += [(p + "ln1.weight", 1, D, "norm"), (p + "ln2.weight", 1, D, "norm"),
                  (p + "attn.q_proj.weight", D, D, "proj"),
                  (p + "attn.k_proj.weight", dkv, D, "proj"),
                  (p + "attn.v_proj.weight", dkv, D, "proj"),
                  (p + "attn.o_proj.weight", D, D, "proj"),
                  (p + "ffn.gate.weight", F, D, "proj"),
                  (p + "ffn.fc1.weight", F, D, "proj"),
                  (p + "ffn.fc2.weight", D, F, "proj")]
    specs += [("ln_final.weight", 1, D, "norm"), ("lm_head.weight", cfg["vocab_size"], D, "proj")]
    return specs


def make_tensor(seed, name, rows, cols, kind, dtype, norm_std=0.0):
    """Returns (host payload for the device, decoded f32 the reference would run).

    Projections: N(0, 0.02) then quantized to `dtype`; the f32 copy is the
    block-decoded weight (what the reference runs after the converter
    dequantizes, convert_gguf.py:233-263).  Norm weights are 1 (random_init,
    transformer.hpp:595-598) plus an optional N(0, norm_std) perturbation;
    the embedding is N(0, 0.02) f32."""
    n = rows * cols
    if kind == "norm":
        w = np.ones(n, np.float32)
        if norm_std:
            w += normal(seed, name, n, norm_std)
        return w, w
    w = normal(seed, name, n, 0.02)
    if kind == "embed" or dtype == DT_F32:
        return w, w
    blocks = quantize(w, dtype)
    return blocks, dequantize(blocks, dtype, n)


def load_model(model, seed, want_f32=False, norm_std=0.0):
    """Generates every tensor, uploads it to `model` (a runtime.Model) and
    optionally returns the decoded f32 weights keyed by name (for the oracle)."""
    cfg = model.cfg
    f32 = {}
    for name, rows, cols, kind in tensor_specs(cfg):
        payload, dec = make_tensor(seed, name, rows, cols, kind, cfg["weight_dtype"], norm_std)
        dt = cfg["weight_dtype"] if kind == "proj" else DT_F32
        model.set_weight(name, payload, dt, rows, cols)
        if want_f32:
            f32[name] = dec.reshape(rows, cols) if rows > 1 else dec
    return f32


def make_f32_weights(cfg, seed, norm_std=0.0):
    """Decoded f32 weights only (no device), for the CPU oracle / reference."""
    out = {}
    for name, rows, cols, kind in tensor_specs(cfg):
        _, dec = make_tensor(seed, name, rows, cols, kind, cfg["weight_dtype"], norm_std)
        out[name] = dec.reshape(rows, cols) if rows > 1 else dec
    return out
