"""GPU parity: dequant-fused quantized linear (compute::linear on weights
decoded from GGUF Q8_0/Q4_0 blocks, convert_gguf.py:233-263), benchmark
config 3 shapes, plus the fused RMSNorm prologue, residual epilogue and the
SwiGLU gate/up variant.  Oracle: ops::gemm restated (oracle/vlrf_oracle.c)
on the decoded f32 weights.  Tolerance: 1e-3 relative (fp32 path)."""
import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu


def _weight(ctx, seed, name, N, K, dtype):
    w = F.normal(seed, name, N * K, 0.02)
    blocks = F.quantize(w, dtype)
    dec = F.dequantize(blocks, dtype, N * K).reshape(N, K) if dtype != V.DT_F32 else w.reshape(N, K)
    return V.QuantWeight(ctx, blocks, dtype, N, K), dec


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("N,K", [(5632, 2048), (2048, 5632)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_config3_qlinear(ctx, orc, dtype, N, K, M):
    print(f"[case] qlinear dtype={dtype} N={N} K={K} M={M}", flush=True)
    w, dec = _weight(ctx, 7, f"W{N}x{K}", N, K, dtype)
    x = F.normal(7, f"x{M}", M * K).reshape(M, K)
    dx, dy = ctx.to_device(x), ctx.alloc(M * N * 4)
    ctx.qlinear(w, dx, dy, M)
    y = dy.download((M, N))
    ref = orc.linear(x, dec)
    assert rel_err(y, ref) <= 1e-3
    np.testing.assert_allclose(y, ref, rtol=1e-3, atol=1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("N,K", [(4096, 14336), (300, 14336), (37, 6176)])
def test_m1_wide_rows(ctx, orc, dtype, N, K):
    """M = 1 over rows wider than the general staging (K > 6144, up to the
    8B shape's d_ff 14336): plain and with the residual added."""
    print(f"[case] wide M=1 dtype={dtype} N={N} K={K}", flush=True)
    w, dec = _weight(ctx, 11, f"W{N}x{K}", N, K, dtype)
    x = F.normal(11, "xw", K).reshape(1, K)
    res = F.normal(11, "rw", N).reshape(1, N)
    dx, dy = ctx.to_device(x), ctx.alloc(N * 4)
    ctx.qlinear(w, dx, dy, 1)
    ref = orc.linear(x, dec)
    assert rel_err(dy.download((1, N)), ref) <= 1e-3
    dr = ctx.to_device(res)
    ctx.qlinear(w, dx, dr, 1, residual=dr)
    assert rel_err(dr.download((1, N)), ref + res) <= 1e-3


@pytest.mark.parametrize("M", [1, 3, 9])
@pytest.mark.parametrize("N,K", [(37, 64), (300, 96), (8, 1056)])
def test_qlinear_ragged_shapes(ctx, orc, M, N, K):
    """Row counts not divisible by the 8-row workgroup tile; K not a multiple of
    the 1024 staging tile; M between the 1/4/16 instantiations."""
    for dtype in (V.DT_Q8_0, V.DT_Q4_0, V.DT_F32):
        w, dec = _weight(ctx, 8, f"R{N}x{K}", N, K, dtype)
        x = F.normal(8, f"xr{M}", M * K).reshape(M, K)
        dx, dy = ctx.to_device(x), ctx.alloc(M * N * 4)
        ctx.qlinear(w, dx, dy, M)
        assert rel_err(dy.download((M, N)), orc.linear(x, dec)) <= 1e-3


def test_qlinear_fused_norm_and_residual(ctx, orc):
    """y = residual + W . rms_norm(x; g) (ops.hpp:478-499 then the residual add)."""
    N, K, M = 2560, 2048, 1
    w, dec = _weight(ctx, 9, "Wqkv", N, K, V.DT_Q8_0)
    x = F.normal(9, "xn", M * K).reshape(M, K) * 0.05
    g = 1.0 + F.normal(9, "g", K, 0.1)
    res = F.normal(9, "res", M * N).reshape(M, N)
    dx, dg, dr = ctx.to_device(x), ctx.to_device(g), ctx.to_device(res)
    dy = ctx.alloc(M * N * 4)
    ctx.qlinear(w, dx, dy, M, norm_w=dg, eps=1e-5)
    ref = orc.linear(orc.rms_norm(x, g, 1e-5), dec)
    assert rel_err(dy.download((M, N)), ref) <= 1e-3
    ctx.qlinear(w, dx, dr, M, norm_w=dg, eps=1e-5, residual=dr)      # in place on the residual
    assert rel_err(dr.download((M, N)), ref + res) <= 1e-3


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("M", [1, 4])
def test_swiglu_gate_up(ctx, orc, dtype, M):
    """h = silu(x.Wg^T) * (x.Wu^T) (feedforward.hpp:54-62) with the fused norm."""
    Fd, K = 5632, 2048
    wg, gdec = _weight(ctx, 10, "Wg", Fd, K, dtype)
    wu, udec = _weight(ctx, 10, "Wu", Fd, K, dtype)
    x = F.normal(10, "xs", M * K).reshape(M, K)
    g = np.ones(K, np.float32)
    dx, dg, dh = ctx.to_device(x), ctx.to_device(g), ctx.alloc(M * Fd * 4)
    ctx.qlinear_swiglu(wg, wu, dx, dh, M, norm_w=dg, eps=1e-5)
    xn = orc.rms_norm(x, g, 1e-5)
    ref = orc.silu_mul(orc.linear(xn, udec), orc.linear(xn, gdec))
    assert rel_err(dh.download((M, Fd)), ref) <= 1e-3


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("M,N,K", [(2, 37, 256), (7, 300, 2304), (16, 1000, 4352), (5, 16, 512)])
def test_small_m_matrix_core_path(ctx, orc, dtype, M, N, K):
    """2 <= M <= 16 with K % 256 == 0 runs on the matrix cores (codes exact in
    bf16, activations split into bf16 hi + lo): row counts off the 16-row tile,
    one 256-column slice, 9 slices over 16 waves (7 idle), 17 slices (one wave
    takes two).  Fused norm, then the residual added in place.  The split keeps
    the f32 class: 1e-4, ten times tighter than the path's stated 1e-3."""
    print(f"[case] qlinear small-M dtype={dtype} M={M} N={N} K={K}", flush=True)
    w, dec = _weight(ctx, 12, f"S{N}x{K}", N, K, dtype)
    x = F.normal(12, f"xs{M}x{K}", M * K).reshape(M, K)
    g = 1.0 + F.normal(12, f"gs{K}", K, 0.1)
    res = F.normal(12, f"rs{M}x{N}", M * N).reshape(M, N)
    dx, dg, dr, dy = ctx.to_device(x), ctx.to_device(g), ctx.to_device(res), ctx.alloc(M * N * 4)
    ctx.qlinear(w, dx, dy, M)
    assert rel_err(dy.download((M, N)), orc.linear(x, dec)) <= 1e-4
    ref = orc.linear(orc.rms_norm(x, g, 1e-5), dec)
    ctx.qlinear(w, dx, dr, M, norm_w=dg, eps=1e-5, residual=dr)
    assert rel_err(dr.download((M, N)), ref + res) <= 1e-4


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
def test_small_m_swiglu_ragged(ctx, orc, dtype):
    """SwiGLU on the small-M matrix-core path: M = 13, F = 1000 (not a multiple
    of 16), K = 4352 (17 slices)."""
    M, Fd, K = 13, 1000, 4352
    wg, gdec = _weight(ctx, 13, "SWg", Fd, K, dtype)
    wu, udec = _weight(ctx, 13, "SWu", Fd, K, dtype)
    x = F.normal(13, "sxs", M * K).reshape(M, K)
    g = 1.0 + F.normal(13, "sgs", K, 0.1)
    dx, dg, dh = ctx.to_device(x), ctx.to_device(g), ctx.alloc(M * Fd * 4)
    ctx.qlinear_swiglu(wg, wu, dx, dh, M, norm_w=dg, eps=1e-5)
    xn = orc.rms_norm(x, g, 1e-5)
    ref = orc.silu_mul(orc.linear(xn, udec), orc.linear(xn, gdec))
    assert rel_err(dh.download((M, Fd)), ref) <= 1e-4


def test_small_m_one_launch_calls_in_a_row(ctx, orc):
    """The small-M path reduces each row tile's slice partials in the tile's
    last workgroup, found by a per-tile counter that the reduction resets:
    calls in a row on one context with different tile and slice counts (a
    grid of fewer columns than slices, so workgroups take two slices, then
    one slice, then 22 slices) each match the oracle, twice over."""
    cases = [(4, 20000, 2048), (2, 300, 256), (16, 2048, 5632), (9, 5632, 2048)]
    for rep in range(2):
        for i, (M, N, K) in enumerate(cases):
            print(f"[case] small-M calls in a row: M={M} N={N} K={K} (pass {rep})", flush=True)
            w, dec = _weight(ctx, 40 + i, f"R{N}x{K}", N, K, V.DT_Q8_0)
            x = F.normal(40 + i, f"rx{M}x{K}", M * K).reshape(M, K)
            dx, dy = ctx.to_device(x), ctx.alloc(M * N * 4)
            ctx.qlinear(w, dx, dy, M)
            assert rel_err(dy.download((M, N)), orc.linear(x, dec)) <= 1e-4, (M, N, K)


def test_qlinear_rejects_bad_shapes(ctx):
    w, _ = _weight(ctx, 11, "Wbad", 64, 96, V.DT_Q8_0)
    x = ctx.alloc(96 * 4 * 17)
    with pytest.raises(V.HipError):
        ctx.qlinear(w, x, ctx.alloc(64 * 4 * 17), 17)      # M > 16 (MFMA path) needs K % 64 == 0
    wf, _ = _weight(ctx, 11, "Wbadf", 64, 64, V.DT_F32)
    with pytest.raises(V.HipError):
        ctx.qlinear(wf, x, ctx.alloc(64 * 4 * 17), 17)     # and a block-quantized weight
    with pytest.raises(V.HipError):
        ctx.qlinear(w, x, x, 1)                             # x aliasing y
