"""GGUF -> NFW v3 converter that keeps Q8_0/Q4_0 tensors as GGUF blocks.

The reference converter (tools/converter/convert_gguf.py) decodes every GGUF
tensor to f32 (load_tensor_f32 / _dequantise, :175-263) and writes NFW
version 1.  This one reads the same GGUF v2/v3 layout (header :133-171),
builds the same config.json (build_vlrf_config_from_gguf, :479-526) and maps
tensor names the same way (remap_key, :530-642, including the zero biases it
adds), but stores Q8_0 and Q4_0 tensors as their GGUF blocks in an NFW
version-3 file, byte for byte, so the device kernels run the file's weights.
F32 and F16 tensors are written as f32, as the reference does.  Other GGML
types (K-quants, Q4_1, Q5_x, BF16) have no kernel here and are refused.

    python -m vlrf_amd.convert_gguf --model model.gguf --out outdir [--verify]

Tokenizer extraction (the reference's extract_tokenizer) is out of scope.
"""
import argparse
import json
import struct
import sys
from pathlib import Path

import numpy as np

from . import nfw

GGUF_MAGIC = 0x46554747
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8
# elements per block, bytes per block (convert_gguf.py:58-72)
GGML_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
              10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 30: (1, 2)}


class GGUFReader:
    """GGUF v2/v3 reader returning raw blocks or f32 arrays."""

    _SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q",
               11: "<q", 12: "<d"}

    def __init__(self, path):
        self.path = str(path)
        self.f = open(self.path, "rb")
        self.meta, self.tensors = {}, []
        self._parse_header()

    def close(self):
        self.f.close()

    def _u(self, fmt):
        return struct.unpack(fmt, self.f.read(struct.calcsize(fmt)))[0]

    def _str(self):
        return self.f.read(self._u("<Q")).decode("utf-8", errors="replace")

    def _value(self, vtype):
        if vtype == 8:
            return self._str()
        if vtype == 9:
            et, n = self._u("<I"), self._u("<Q")
            return [self._value(et) for _ in range(n)]
        if vtype not in self._SCALAR:
            raise ValueError(f"unknown GGUF value type {vtype}")
        v = self._u(self._SCALAR[vtype])
        return bool(v) if vtype == 7 else v

    def _parse_header(self):
        if self._u("<I") != GGUF_MAGIC:
            raise ValueError(f"{self.path}: not a GGUF file")
        self.version = self._u("<I")
        if not 2 <= self.version <= 3:
            raise ValueError(f"{self.path}: unsupported GGUF version {self.version}")
        n_tensors, n_kv = self._u("<Q"), self._u("<Q")
        for _ in range(n_kv):
            key = self._str()
            self.meta[key] = self._value(self._u("<I"))
        for _ in range(n_tensors):
            name = self._str()
            dims = [self._u("<Q") for _ in range(self._u("<I"))]
            self.tensors.append({"name": name, "dims": dims, "dtype": self._u("<I"), "offset": self._u("<Q")})
        align = int(self.meta.get("general.alignment", 32))
        pos = self.f.tell()
        self.data_offset = (pos + align - 1) // align * align

    def raw(self, desc):
        """(dtype, shape outermost-first, payload bytes) of one tensor."""
        numel = int(np.prod(desc["dims"])) if desc["dims"] else 1
        if desc["dtype"] not in GGML_BLOCK:
            raise ValueError(f"{desc['name']}: unknown GGML type {desc['dtype']}")
        epb, bpb = GGML_BLOCK[desc["dtype"]]
        self.f.seek(self.data_offset + desc["offset"])
        data = self.f.read(numel // epb * bpb)
        return desc["dtype"], tuple(reversed(desc["dims"])), data

    def load_tensor(self, desc):
        """np.float32 array for F32/F16, nfw.Blocks for Q8_0/Q4_0."""
        dtype, shape, data = self.raw(desc)
        if dtype == GGML_F32:
            return np.frombuffer(data, np.float32).reshape(shape).copy()
        if dtype == GGML_F16:
            return np.frombuffer(data, np.float16).astype(np.float32).reshape(shape)
        if dtype in (GGML_Q8_0, GGML_Q4_0):
            return nfw.Blocks(dtype, shape, data)
        raise ValueError(f"{desc['name']}: GGML type {dtype} is not passed through "
                         f"(only F32, F16, Q8_0, Q4_0 have kernels here)")


def build_config(meta):
    """Same fields and defaults as build_vlrf_config_from_gguf (:479-526)."""
    arch = meta.get("general.architecture", "llama")

    def m(key, default=None):
        return meta.get(f"{arch}.{key}", meta.get(key, default))

    d = int(m("embedding_length", 4096))
    n_heads = int(m("attention.head_count", 32))
    return {
        "model_name": meta.get("general.name", arch), "model_version": "1.0.0", "source_arch": arch,
        "vocab_size": len(meta["tokenizer.ggml.tokens"]) if "tokenizer.ggml.tokens" in meta else 32000,
        "d_model": d, "d_ff": int(m("feed_forward_length", 4 * d)), "n_heads": n_heads,
        "n_kv_heads": int(m("attention.head_count_kv", n_heads)), "n_layers": int(m("block_count", 32)),
        "max_seq_len": int(m("context_length", 4096)),
        "bos_token_id": int(meta.get("tokenizer.ggml.bos_token_id", 1)),
        "eos_token_id": int(meta.get("tokenizer.ggml.eos_token_id", 2)),
        "pad_token_id": int(meta.get("tokenizer.ggml.padding_token_id", 0)),
        "layer_norm_eps": float(m("attention.layer_norm_rms_epsilon", m("attention.layer_norm_epsilon", 1e-5))),
        "pre_norm": True, "use_rms_norm": "rms" in str(m("attention.layer_norm_type", "rms")).lower(),
        "tie_embeddings": False, "pos_embedding": "sinusoidal", "activation": "silu",
        "temperature": 0.8, "top_p": 0.9, "top_k": 50, "max_new_tokens": 256,
    }


def _rows_of(t):
    return t.shape[0]


def _zeros(n):
    return np.zeros(n, np.float32)


def remap(name, t, out, n_heads, kv_heads, d_model):
    """GGUF name -> engine names, as remap_key (:530-642): same targets, same
    zero biases, fused attn_qkv split by rows; t is an array or nfw.Blocks."""
    if name == "token_embd.weight":
        out["embed.weight"] = t
        return
    if name in ("output_norm.weight", "final_norm.weight"):
        out["ln_final.weight"] = t
        out["ln_final.bias"] = _zeros(_rows_of(t))
        return
    if name == "output.weight":
        out["lm_head.weight"] = t
        return
    if not name.startswith("blk."):
        return
    parts = name.split(".")
    pfx, rest = f"layers.{int(parts[1])}", ".".join(parts[2:])
    d_kv = kv_heads * (d_model // n_heads)
    simple = {
        "attn_norm.weight": ("ln1", True), "ffn_norm.weight": ("ln2", True),
        "attn_q.weight": ("attn.q_proj", True), "attn_k.weight": ("attn.k_proj", True),
        "attn_v.weight": ("attn.v_proj", True), "attn_output.weight": ("attn.o_proj", True),
        "ffn_gate.weight": ("ffn.gate", False), "ffn_up.weight": ("ffn.fc1", True),
        "ffn_down.weight": ("ffn.fc2", True), "ffn_gate_up.weight": ("ffn.fc1", True),
    }
    if rest in simple:
        target, bias = simple[rest]
        out[f"{pfx}.{target}.weight"] = t
        if bias:
            out[f"{pfx}.{target}.bias"] = _zeros(_rows_of(t))
        return
    if rest == "attn_qkv.weight":
        parts3 = ((0, d_model), (d_model, d_model + d_kv), (d_model + d_kv, d_model + 2 * d_kv))
        for key, (r0, r1) in zip(("q_proj", "k_proj", "v_proj"), parts3):
            out[f"{pfx}.attn.{key}.weight"] = t.rows(r0, r1) if isinstance(t, nfw.Blocks) else t[r0:r1]
            out[f"{pfx}.attn.{key}.bias"] = _zeros(r1 - r0)


def convert(model, out_dir, verify=False, log=print):
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    reader = GGUFReader(model)
    cfg = build_config(reader.meta)
    tensors = {}
    for desc in reader.tensors:
        remap(desc["name"], reader.load_tensor(desc), tensors, cfg["n_heads"], cfg["n_kv_heads"], cfg["d_model"])
    reader.close()
    path = out_dir / "model.nfw"
    nfw.write_nfw(path, tensors, version=3)
    (out_dir / "config.json").write_text(json.dumps(cfg, indent=2))
    n_blocks = sum(isinstance(t, nfw.Blocks) for t in tensors.values())
    log(f"{len(tensors)} tensors ({n_blocks} as GGUF blocks) -> {path}")
    if verify:
        verify_nfw(tensors, path)
        log("verified: every tensor reads back identical")
    return path, cfg


def verify_nfw(tensors, path):
    """Block payloads byte-identical, f32 tensors bit-identical after reading back."""
    with nfw.NfwFile(path) as f:
        for name, t in tensors.items():
            i = f.find(name)
            if i < 0:
                raise ValueError(f"verify: {name} missing")
            if isinstance(t, nfw.Blocks):
                if f.raw(i) != t.data:
                    raise ValueError(f"verify: {name} blocks differ")
            elif not np.array_equal(f.f32(i), np.asarray(t, np.float32)):
                raise ValueError(f"verify: {name} differs")


def main(argv=None):
    ap = argparse.ArgumentParser(description="Convert GGUF to NFW v3 keeping Q8_0/Q4_0 blocks")
    ap.add_argument("--model", required=True, help="input .gguf file")
    ap.add_argument("--out", required=True, help="output directory")
    ap.add_argument("--verify", action="store_true", help="read the written file back and compare")
    a = ap.parse_args(argv)
    if not Path(a.model).exists():
        sys.exit(f"Error: file not found: {a.model}")
    convert(a.model, a.out, a.verify)


if __name__ == "__main__":
    main()
