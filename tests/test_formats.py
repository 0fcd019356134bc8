"""CPU tests of the product's host-side helpers in libvlrf_hip.so (no GPU
needed): the GGUF block encoders/decoders and the seeded synthetic data."""
import numpy as np
import pytest

import oracle
from vlrf_amd import formats as F


@pytest.mark.parametrize("dtype", [F.DT_Q8_0, F.DT_Q4_0])
def test_decoder_matches_oracle_on_arbitrary_blocks(dtype):
    """vlrf_dequantize == the convert_gguf.py decode (oracle) bit for bit, on
    random codes (including -128 / all nibbles) and random finite f16 scales."""
    rng = np.random.default_rng(5)
    nb, bsz = 257, F.BLOCK_BYTES[dtype]
    blocks = rng.integers(0, 256, size=(nb, bsz), dtype=np.uint8)
    d = (rng.standard_normal(nb) * 0.05).astype(np.float16)
    d[:3] = [0.0, -0.0, 6.1e-5]                      # zero, negative zero, subnormal-adjacent
    blocks[:, :2] = d.view(np.uint8).reshape(nb, 2)
    flat = blocks.reshape(-1)
    ours = F.dequantize(flat, dtype, nb * 32)
    ref = oracle.dequant_q8_0(flat, nb * 32) if dtype == F.DT_Q8_0 else oracle.dequant_q4_0(flat, nb * 32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_q8_0_encoder_closed_form():
    x = F.normal(1, "q8", 32 * 64, 0.7)
    x[:32] = 0.0                                     # an all-zero block
    blocks = F.quantize(x, F.DT_Q8_0).reshape(-1, 34)
    d16 = blocks[:, :2].copy().view(np.float16).reshape(-1)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert np.array_equal(d16, (amax / np.float32(127)).astype(np.float16))   # RNE to f16
    dec = F.dequantize(blocks.reshape(-1), F.DT_Q8_0, x.size).reshape(-1, 32)
    d = d16.astype(np.float32)[:, None]
    assert np.all(np.abs(dec - x.reshape(-1, 32)) <= d * 0.5000001 + 1e-12)
    assert not dec[0].any()
    q = blocks[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127


def test_q4_0_encoder_closed_form():
    x = F.normal(2, "q4", 32 * 64, 0.3)
    blocks = F.quantize(x, F.DT_Q4_0).reshape(-1, 18)
    xb = x.reshape(-1, 32)
    mx = xb[np.arange(xb.shape[0]), np.abs(xb).argmax(axis=1)]
    d16 = blocks[:, :2].copy().view(np.float16).reshape(-1)
    assert np.array_equal(d16, (mx / np.float32(-8)).astype(np.float16))
    dec = F.dequantize(blocks.reshape(-1), F.DT_Q4_0, x.size).reshape(-1, 32)
    d = np.abs(d16.astype(np.float32))[:, None]
    # every element within half a step, except values clamped at the top code
    err = np.abs(dec - xb)
    assert np.all((err <= d * 0.5000001 + 1e-9) | (np.abs(dec - 7 * d16.astype(np.float32)[:, None]) < 1e-9))
    # the signed max-magnitude element maps to code 0, i.e. exactly -8*d
    assert np.allclose(dec[np.arange(xb.shape[0]), np.abs(xb).argmax(axis=1)], -8 * d16.astype(np.float32))


def test_synth_is_deterministic_and_normal():
    a = F.normal(7, "w", 1 << 16, 0.02)
    b = F.normal(7, "w", 1 << 16, 0.02)
    c = F.normal(7, "w2", 1 << 16, 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 5e-4 and abs(a.std() - 0.02) < 5e-4
    assert np.array_equal(F.normal(7, "w", 1001)[:1000], F.normal(7, "w", 1000))   # prefix-stable
    t = F.tokens(7, "p", 10000, 32000)
    assert t.min() >= 0 and t.max() < 32000 and len(np.unique(t)) > 8000


def test_tensor_specs_cover_the_reference_weight_names():
    cfg = F.tiny(n_layers=2)
    names = {n for n, *_ in F.tensor_specs(cfg)}
    for l in range(2):
        for k in ("ln1.weight", "ln2.weight", "attn.q_proj.weight", "attn.k_proj.weight",
                  "attn.v_proj.weight", "attn.o_proj.weight", "ffn.gate.weight", "ffn.fc1.weight",
                  "ffn.fc2.weight"):
            assert f"layers.{l}.{k}" in names
    assert {"embed.weight", "ln_final.weight", "lm_head.weight"} <= names


@pytest.mark.parametrize("dtype", [F.DT_Q8_0, F.DT_Q4_0])
def test_reencoding_decoded_blocks_is_lossless(dtype):
    """Weights that reach the engine as f32 after the GGUF converter decoded
    them (convert_gguf.py:233-263) re-encode to the identical blocks, so the
    device model built from a WeightMap holds exactly the file's weights."""
    x = F.normal(9, "reenc", 32 * 512, 0.05)
    x[:32] = 0.0
    blocks = F.quantize(x, dtype)
    dec = F.dequantize(blocks, dtype, x.size)
    assert np.array_equal(F.quantize(dec, dtype), blocks)
