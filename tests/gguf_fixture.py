"""Synthetic GGUF files for the converter and loader tests (test
infrastructure).  The byte layout is GGUF v3 as the reference's reader parses
it (tools/converter/convert_gguf.py:133-171): magic, version, tensor and
metadata counts, metadata key/values, tensor descriptors (dims innermost
first), data section aligned to 32 bytes, each tensor's offset aligned to 32.
"""
import struct

import numpy as np

from vlrf_amd import formats as F

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q6_K = 0, 1, 2, 8, 14
T_U32, T_F32, T_STRING = 4, 6, 8


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, meta, tensors, align=32):
    """meta: [(key, vtype, value)] with vtype u32/f32/string; tensors:
    [(name, ggml_type, shape outermost-first, payload bytes)]."""
    kv = b""
    for key, vt, val in meta:
        kv += _s(key) + struct.pack("<I", vt)
        kv += _s(val) if vt == T_STRING else struct.pack("<I" if vt == T_U32 else "<f", val)
    desc, data = b"", b""
    for name, gt, shape, payload in tensors:
        off = len(data)
        desc += _s(name) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            desc += struct.pack("<Q", d)
        desc += struct.pack("<I", gt) + struct.pack("<Q", off)
        data += payload + b"\0" * ((-len(payload)) % align)
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(meta)) + kv + desc
    with open(path, "wb") as f:
        f.write(head + b"\0" * ((-len(head)) % align) + data)


def reference_recipe_q8_0(path, numel=256):
    """One Q8_0 tensor 'token_embd.weight' of `numel` elements, built by the
    recipe of the reference's make_fake_gguf_q8_0 (test_converters.py:327-379):
    rng = default_rng(42); per block scale uniform(0.01, 0.1) stored as f16,
    32 codes integers(-127, 127) int8; expected value code * f32(f16 scale).
    Returns the expected f32 values."""
    rng = np.random.default_rng(42)
    blocks, expected = b"", np.zeros(numel, np.float32)
    for b in range(numel // 32):
        scale = np.float16(np.float32(rng.uniform(0.01, 0.1)))
        qs = rng.integers(-127, 127, size=32, dtype=np.int8)
        blocks += scale.tobytes() + qs.tobytes()
        expected[b * 32:(b + 1) * 32] = qs.astype(np.float32) * float(scale)
    write_gguf(path, [("general.architecture", T_STRING, "llama")],
               [("token_embd.weight", GGML_Q8_0, (numel,), blocks)])
    return expected


GGUF_NAME = {"embed.weight": "token_embd.weight", "ln_final.weight": "output_norm.weight",
             "lm_head.weight": "output.weight"}
LAYER_NAME = {"ln1.weight": "attn_norm.weight", "ln2.weight": "ffn_norm.weight",
              "attn.q_proj.weight": "attn_q.weight", "attn.k_proj.weight": "attn_k.weight",
              "attn.v_proj.weight": "attn_v.weight", "attn.o_proj.weight": "attn_output.weight",
              "ffn.gate.weight": "ffn_gate.weight", "ffn.fc1.weight": "ffn_up.weight",
              "ffn.fc2.weight": "ffn_down.weight"}


def gguf_name(engine_name):
    if engine_name in GGUF_NAME:
        return GGUF_NAME[engine_name]
    _, l, rest = engine_name.split(".", 2)
    return f"blk.{l}.{LAYER_NAME[rest]}"


def llama_gguf(path, cfg, seed, embed_q8=False, fused_qkv=False, f16_norms=False, extra=()):
    """A Llama-style GGUF of the synthetic model `cfg` (formats.tensor_specs):
    projections as cfg['weight_dtype'] blocks, norms F32 (or F16), the
    embedding F32 (or Q8_0 blocks).  Returns {engine name: (gguf payload,
    decoded f32 [rows, cols] or [n])}."""
    wdt = cfg["weight_dtype"]
    out, tensors = {}, []
    for name, rows, cols, kind in F.tensor_specs(cfg):
        payload, dec = F.make_tensor(seed, name, rows, cols, kind, wdt)
        shape = (rows, cols) if rows > 1 else (cols,)
        if kind == "proj":
            gt, raw = wdt, payload.tobytes()
        elif kind == "embed" and embed_q8:
            blocks = F.quantize(payload, GGML_Q8_0)
            gt, raw, dec = GGML_Q8_0, blocks.tobytes(), F.dequantize(blocks, GGML_Q8_0, payload.size)
        elif kind == "norm" and f16_norms:
            h = payload.astype(np.float16)
            gt, raw, dec = GGML_F16, h.tobytes(), h.astype(np.float32)
        else:
            gt, raw = GGML_F32, np.asarray(payload, np.float32).tobytes()
        out[name] = (raw, np.asarray(dec, np.float32).reshape(shape))
        tensors.append((gguf_name(name), gt, shape, raw))
    if fused_qkv:
        D = cfg["d_model"]
        for l in range(cfg["n_layers"]):
            names = [f"blk.{l}.attn_{k}.weight" for k in "qkv"]
            parts = [t for t in tensors if t[0] in names]
            tensors = [t for t in tensors if t[0] not in names]
            rows = sum(p[2][0] for p in parts)
            tensors.append((f"blk.{l}.attn_qkv.weight", wdt, (rows, D), b"".join(p[3] for p in parts)))
    tensors += list(extra)
    meta = [("general.architecture", T_STRING, "llama"), ("general.name", T_STRING, "synthetic"),
            ("llama.embedding_length", T_U32, cfg["d_model"]),
            ("llama.attention.head_count", T_U32, cfg["n_heads"]),
            ("llama.attention.head_count_kv", T_U32, cfg["n_kv_heads"]),
            ("llama.block_count", T_U32, cfg["n_layers"]),
            ("llama.feed_forward_length", T_U32, cfg["d_ff"]),
            ("llama.context_length", T_U32, cfg["max_seq_len"]),
            ("llama.attention.layer_norm_rms_epsilon", T_F32, cfg["norm_eps"])]
    write_gguf(path, meta, tensors)
    return out
