"""NFW files and the GGUF pass-through converter (host side, no device).

The reference's NFW layout (weights.hpp:58-62,289-339; nfw_writer.py:11-44) is
pinned by hand-packed bytes; its f16 widening (weights.hpp:76-96) by IEEE
half->float on special values; the GGUF reader by the reference test's own
Q8_0 recipe (test_converters.py:327-379); the name mapping by the reference
test's expectations (test_converters.py:412-444) and remap_key's rules
(convert_gguf.py:530-642); block pass-through by byte equality with the GGUF
payloads."""
import json
import struct

import numpy as np
import pytest

import vlrf_amd as V
from vlrf_amd import convert_gguf as CG
from vlrf_amd import formats as F
from vlrf_amd import nfw

import gguf_fixture as G


def test_gguf_reader_reference_recipe(tmp_path):
    p = tmp_path / "test.gguf"
    expected = G.reference_recipe_q8_0(str(p), numel=256)
    r = CG.GGUFReader(p)
    assert r.meta["general.architecture"] == "llama"
    assert [t["name"] for t in r.tensors] == ["token_embd.weight"]
    t = r.load_tensor(r.tensors[0])
    r.close()
    assert isinstance(t, nfw.Blocks) and t.shape == (256,)
    dec = F.dequantize(np.frombuffer(t.data, np.uint8), V.DT_Q8_0, 256)
    assert np.array_equal(dec, expected)            # the recipe's values, exactly


def test_nfw_v1_v2_layout_matches_reference_writer(tmp_path):
    a = np.arange(6, dtype=np.float32).reshape(2, 3) - 2.5
    p1, p2 = tmp_path / "v1.nfw", tmp_path / "v2.nfw"
    nfw.write_nfw(p1, {"w": a}, version=1)
    nfw.write_nfw(p2, {"w": a.astype(np.float16)}, version=2)
    # nfw_writer.py:18-26: <IIII> header, <H> name length, name, <B> ndim,
    # <i> dims, <q> numel, [v2: <B> dtype], payload
    v1 = struct.pack("<IIII", 0x4E465746, 1, 1, 0) + struct.pack("<H", 1) + b"w" + struct.pack("<B", 2) + \
        struct.pack("<ii", 2, 3) + struct.pack("<q", 6) + a.tobytes()
    v2 = struct.pack("<IIII", 0x4E465746, 2, 1, 0) + struct.pack("<H", 1) + b"w" + struct.pack("<B", 2) + \
        struct.pack("<ii", 2, 3) + struct.pack("<q", 6) + struct.pack("<B", 1) + a.astype(np.float16).tobytes()
    assert p1.read_bytes() == v1 and p2.read_bytes() == v2
    with nfw.NfwFile(p1) as f:
        assert f.version == 1 and f.info(0) == {"name": "w", "dtype": 0, "shape": (2, 3), "numel": 6, "bytes": 24}
        assert np.array_equal(f.f32(0), a)
    with nfw.NfwFile(p2) as f:
        assert f.version == 2 and f.info(0)["dtype"] == nfw.F16
        assert np.array_equal(f.f32(0), a)


def test_f16_widening_is_exact_on_special_values(tmp_path):
    bits = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF,
                     0x7C00, 0xFC00, 0x3555, 0x8001, 0x83FF], np.uint16)
    p = tmp_path / "h.nfw"
    nfw.write_nfw(p, {"h": bits.view(np.float16)}, version=2)
    with nfw.NfwFile(p) as f:
        got = f.f32(0)
    assert np.array_equal(got.view(np.uint32), bits.view(np.float16).astype(np.float32).view(np.uint32))
    nan = np.array([0x7E00, 0x7C01], np.uint16).view(np.float16)
    nfw.write_nfw(p, {"n": nan}, version=2)
    with nfw.NfwFile(p) as f:
        n = f.f32(0)
    # weights.hpp:92-93: exponent 31 keeps the mantissa shifted into place
    assert list(n.view(np.uint32)) == [0x7FC00000, 0x7F802000]


def test_v3_blocks_round_trip(tmp_path):
    for dt in (nfw.Q8_0, nfw.Q4_0):
        w = F.normal(3, f"blk{dt}", 6 * 64, 0.02)
        b = F.quantize(w, dt)
        p = tmp_path / f"b{dt}.nfw"
        nfw.write_nfw(p, {"x": nfw.Blocks(dt, (6, 64), b.tobytes())})
        with nfw.NfwFile(p) as f:
            inf = f.info(0)
            assert inf["dtype"] == dt and inf["shape"] == (6, 64) and inf["bytes"] == len(b.tobytes())
            assert f.raw(0) == b.tobytes()
            assert np.array_equal(f.f32(0).ravel(), F.dequantize(b, dt, w.size))


def test_nfw_rejects_bad_files(tmp_path):
    good = tmp_path / "g.nfw"
    nfw.write_nfw(good, {"x": nfw.Blocks(nfw.Q8_0, (2, 32), bytes(68))})
    raw = good.read_bytes()
    cases = {
        "magic": b"XXXX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 4) + raw[8:],
        "truncated": raw[:-1],
        "v2_blocks": raw[:4] + struct.pack("<I", 2) + raw[8:],
        "odd_cols": raw.replace(struct.pack("<ii", 2, 32), struct.pack("<ii", 4, 16)),
    }
    # Headers whose size products overflow int64 or ask for more than the
    # file holds: refused as bad files, never a wrapped size or an
    # allocation that escapes the C ABI.
    def one(dims, numel, dtype=0, payload=b""):
        name = b"w"
        body = struct.pack("<H", len(name)) + name + struct.pack("<B", len(dims))
        body += struct.pack(f"<{len(dims)}i", *dims) + struct.pack("<qB", numel, dtype)
        return raw[:8] + struct.pack("<I", 1) + raw[12:16] + body + payload
    cases.update({
        "wrapping_f32": one((1 << 30, 1 << 30, 4), 1 << 62),            # numel * 4 wraps to 0
        "negative_dim": one((-4, -8), 32, payload=bytes(128)),
        "dims_overflow": one((2**31 - 1,) * 3, 0),
        "numel_beyond_file": one((1 << 20,), 1 << 20, payload=bytes(64)),
        "negative_numel": one((), -(1 << 61)),                        # numel * 4 would overflow int64
        "negative_numel_f16": one((), -3, dtype=1, payload=bytes(8)),
    })
    for name, data in cases.items():
        p = tmp_path / f"{name}.nfw"
        p.write_bytes(data)
        with pytest.raises(V.HipError):
            nfw.NfwFile(p)


@pytest.mark.parametrize("wdt", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("fused", [False, True])
def test_convert_passes_blocks_through(tmp_path, wdt, fused):
    cfg = F.tiny(wdt, n_layers=2)
    src = tmp_path / "m.gguf"
    made = G.llama_gguf(str(src), cfg, seed=5, embed_q8=True, fused_qkv=fused, f16_norms=True)
    out = tmp_path / "out"
    path, conf = CG.convert(src, out, verify=True, log=lambda *a: None)
    assert json.loads((out / "config.json").read_text()) == conf
    assert (conf["d_model"], conf["n_heads"], conf["n_kv_heads"], conf["n_layers"], conf["d_ff"]) == \
        (cfg["d_model"], cfg["n_heads"], cfg["n_kv_heads"], cfg["n_layers"], cfg["d_ff"])
    assert conf["pos_embedding"] == "sinusoidal" and conf["vocab_size"] == 32000   # as the reference writes
    with nfw.NfwFile(path) as f:
        assert f.version == 3
        names = set(f.names())
        for name, (raw, dec) in made.items():
            i = f.find(name)
            assert i >= 0, name
            inf = f.info(i)
            assert inf["shape"] == dec.shape
            if inf["dtype"] in (nfw.Q8_0, nfw.Q4_0):
                assert f.raw(i) == raw, name                  # GGUF blocks, byte for byte
            assert np.array_equal(f.f32(i), dec), name
        # remap_key's zero biases (convert_gguf.py:562-612); no bias for ffn.gate
        D, dkv = cfg["d_model"], cfg["n_kv_heads"] * (cfg["d_model"] // cfg["n_heads"])
        for l in range(cfg["n_layers"]):
            for key, n in (("ln1", D), ("ln2", D), ("attn.q_proj", D), ("attn.k_proj", dkv), ("attn.v_proj", dkv),
                           ("attn.o_proj", D), ("ffn.fc1", cfg["d_ff"]), ("ffn.fc2", D)):
                b = f.f32(f.find(f"layers.{l}.{key}.bias"))
                assert b.shape == (n,) and not b.any()
            assert f"layers.{l}.ffn.gate.bias" not in names
        assert not f.f32(f.find("ln_final.bias")).any()


def test_remap_matches_reference_test_expectations():
    """test_converters.py:412-444: the same inputs map to the same names/shapes
    (plus a fused attn_qkv, split by rows as remap_key does, :614-623)."""
    d, n_heads, kv_heads = 64, 4, 2
    d_kv = kv_heads * d // n_heads
    out = {}
    r = np.random.default_rng(0)
    CG.remap("token_embd.weight", r.standard_normal((100, d)).astype(np.float32), out, n_heads, kv_heads, d)
    CG.remap("blk.0.attn_q.weight", r.standard_normal((d, d)).astype(np.float32), out, n_heads, kv_heads, d)
    CG.remap("blk.0.attn_k.weight", r.standard_normal((d_kv, d)).astype(np.float32), out, n_heads, kv_heads, d)
    CG.remap("blk.0.ffn_gate.weight", r.standard_normal((128, d)).astype(np.float32), out, n_heads, kv_heads, d)
    CG.remap("blk.1.attn_qkv.weight", r.standard_normal((d + 2 * d_kv, d)).astype(np.float32), out, n_heads,
             kv_heads, d)
    CG.remap("output_norm.weight", np.ones(d, np.float32), out, n_heads, kv_heads, d)
    CG.remap("blk.0.ffn_norm.weight", np.ones(d, np.float32), out, n_heads, kv_heads, d)
    assert out["embed.weight"].shape == (100, d)
    assert out["layers.0.attn.q_proj.weight"].shape == (d, d)
    assert out["layers.0.attn.k_proj.weight"].shape == (d_kv, d)
    assert out["layers.0.ffn.gate.weight"].shape == (128, d)
    assert out["layers.1.attn.v_proj.weight"].shape == (d_kv, d)
    assert out["ln_final.weight"].shape == (d,) and out["ln_final.bias"].shape == (d,)
    assert out["layers.0.ln2.weight"].shape == (d,)


def test_convert_refuses_types_without_kernels(tmp_path):
    cfg = F.tiny(V.DT_Q8_0, n_layers=1)
    src = tmp_path / "k.gguf"
    G.llama_gguf(str(src), cfg, seed=6, extra=[("blk.0.extra.weight", G.GGML_Q6_K, (1, 256), bytes(210))])
    with pytest.raises(ValueError, match="not passed through"):
        CG.convert(src, tmp_path / "o", log=lambda *a: None)
