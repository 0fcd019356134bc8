"""GPU parity of the prefill (M > 16) linear: the MFMA GEMM on bf16 operands
with f32 accumulation, against ops::gemm restated in f32 (oracle) on the
decoded weights (compute.hpp:58-68, ops.hpp:254-305, convert_gguf.py:233-263).
Tolerance: the 1e-2 class of bf16 paths (max |diff| / max |ref|); measured
errors are ~3e-3."""
import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import _lib
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _weight(ctx, seed, name, N, K, dtype):
    w = F.normal(seed, name, N * K, 0.02)
    blocks = F.quantize(w, dtype)
    dec = F.dequantize(blocks, dtype, N * K).reshape(N, K)
    return V.QuantWeight(ctx, blocks, dtype, N, K), dec


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
# Kernel selection: M <= 128 -> 128-row register-staged tiles; Q8_0 with M > 128 -> the
# direct-to-LDS kernel (256x128 tiles); Q4_0 with M > 128 -> the register-staged 256x128
# tiles (two per CU for 257..512 tiles, as 520 x 16600's 390).
# Wide 256x256 tiles (two 128-row halves of the one weight) where they give at
# least 192 workgroups: 520 x 16600 and 2048 x 6144 (the 8B layer's QKV at T = 2048).
@pytest.mark.parametrize("M,N,K", [(256, 6144, 4096), (128, 4096, 14336), (2048, 1024, 4096),
                                   (520, 16600, 64), (2048, 6144, 512)])
def test_prefill_gemm_config5_shapes(ctx, orc, dtype, M, N, K):
    """The 8B-layer projections (QKV 6144x4096, down 4096x14336) at prompt rows."""
    print(f"[case] qgemm dtype={dtype} M={M} N={N} K={K}", flush=True)
    w, dec = _weight(ctx, 21, f"P{N}x{K}", N, K, dtype)
    x = F.normal(21, f"px{M}x{K}", M * K).reshape(M, K)
    dx, dy = ctx.to_device(x), ctx.alloc(M * N * 4)
    ctx.qlinear(w, dx, dy, M)
    ref = x.astype(np.float64) @ dec.astype(np.float64).T
    assert rel_err(dy.download((M, N)), ref) <= TOL


@pytest.mark.parametrize("M,N,K", [(17, 37, 64), (200, 300, 128), (129, 130, 704), (300, 256, 2048),
                                   (1000, 8300, 192), (1500, 8300, 192), (300, 100, 256), (129, 37, 64)])
def test_prefill_gemm_ragged_with_norm_and_residual(ctx, orc, M, N, K):
    """Row/column counts off the 128x128 tile, with the fused RMSNorm prologue
    and the residual epilogue (in place on the residual)."""
    print(f"[case] qgemm ragged M={M} N={N} K={K}", flush=True)
    w, dec = _weight(ctx, 22, f"G{N}x{K}", N, K, V.DT_Q8_0)
    x = F.normal(22, f"gx{M}", M * K).reshape(M, K) * 3
    g = 1.0 + F.normal(22, f"gg{K}", K, 0.1)
    res = F.normal(22, f"gr{M}x{N}", M * N).reshape(M, N)
    dx, dg, dr = ctx.to_device(x), ctx.to_device(g), ctx.to_device(res)
    ctx.qlinear(w, dx, dr, M, norm_w=dg, eps=1e-5, residual=dr)
    ref = orc.linear(orc.rms_norm(x, g, 1e-5), dec) + res
    assert rel_err(dr.download((M, N)), ref) <= TOL


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("M", [100, 192])
def test_prefill_swiglu(ctx, orc, dtype, M):
    """h = silu(x.Wg^T) * (x.Wu^T) at M rows (feedforward.hpp:54-62); M = 100 takes
    the 128-row tiles, M = 192 the 256-row ones."""
    Fd, K = 1408, 1024
    wg, gdec = _weight(ctx, 23, "PWg", Fd, K, dtype)
    wu, udec = _weight(ctx, 23, "PWu", Fd, K, dtype)
    x = F.normal(23, "psx", M * K).reshape(M, K)
    g = np.ones(K, np.float32)
    dx, dg, dh = ctx.to_device(x), ctx.to_device(g), ctx.alloc(M * Fd * 4)
    ctx.qlinear_swiglu(wg, wu, dx, dh, M, norm_w=dg, eps=1e-5)
    xn = orc.rms_norm(x, g, 1e-5)
    ref = orc.silu_mul(orc.linear(xn, udec), orc.linear(xn, gdec))
    assert rel_err(dh.download((M, Fd)), ref) <= TOL


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("M,Fd,K", [(257, 1000, 192), (300, 100, 64)])
def test_prefill_swiglu_ragged(ctx, orc, dtype, M, Fd, K):
    """SwiGLU with the FFN width and the row count off the 256x128 tile (the
    gate and up tiles of the direct-to-LDS kernel share one workgroup)."""
    print(f"[case] swiglu ragged dtype={dtype} M={M} F={Fd} K={K}", flush=True)
    wg, gdec = _weight(ctx, 24, f"RWg{Fd}x{K}", Fd, K, dtype)
    wu, udec = _weight(ctx, 24, f"RWu{Fd}x{K}", Fd, K, dtype)
    x = F.normal(24, f"rsx{M}x{K}", M * K).reshape(M, K)
    g = 1.0 + F.normal(24, f"rsg{K}", K, 0.1)
    dx, dg, dh = ctx.to_device(x), ctx.to_device(g), ctx.alloc(M * Fd * 4)
    ctx.qlinear_swiglu(wg, wu, dx, dh, M, norm_w=dg, eps=1e-5)
    xn = orc.rms_norm(x, g, 1e-5)
    ref = orc.silu_mul(orc.linear(xn, udec), orc.linear(xn, gdec))
    assert rel_err(dh.download((M, Fd)), ref) <= TOL


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
# 17 <= M <= 128 over codes with K split into slices (64 x 256 tiles to M = 64,
# 128 x 128 above): the 1.1B up and down shapes, the 8B down shape (16 col
# tiles x 16 slices), ragged N, the residual form, and K = 128 (one slice).
@pytest.mark.parametrize("M,N,K,res", [(17, 5632, 2048, False), (64, 2048, 5632, True), (65, 300, 1024, False),
                                       (128, 4096, 14336, True), (100, 1000, 128, False), (33, 6144, 4096, False)])
def test_split_k_gemm_mid_m(ctx, orc, monkeypatch, dtype, M, N, K, res):
    """The K-split GEMM against the oracle, and against the unsplit
    register-staged kernel (VLRF_HIP_PREFILL_DQ=0): the same bf16 products,
    summed in another order (slices added last), so equal to f32 rounding."""
    print(f"[case] split-K qgemm dtype={dtype} M={M} N={N} K={K} res={res}", flush=True)
    w, dec = _weight(ctx, 26, f"S{N}x{K}", N, K, dtype)
    x = F.normal(26, f"sx{M}x{K}", M * K).reshape(M, K)
    r = F.normal(26, f"sr{M}x{N}", M * N).reshape(M, N)
    dx = ctx.to_device(x)

    def run():
        dy = ctx.to_device(r) if res else ctx.alloc(M * N * 4)
        ctx.qlinear(w, dx, dy, M, residual=dy if res else None)
        return dy.download((M, N))

    monkeypatch.delenv("VLRF_HIP_PREFILL_DQ", raising=False)
    got = run()
    monkeypatch.setenv("VLRF_HIP_PREFILL_DQ", "0")
    unsplit = run()
    monkeypatch.delenv("VLRF_HIP_PREFILL_DQ", raising=False)
    ref = x.astype(np.float64) @ dec.astype(np.float64).T + (r if res else 0)
    assert rel_err(got, ref) <= TOL
    assert rel_err(got, unsplit) <= 2e-5, rel_err(got, unsplit)


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("M,Fd,K", [(17, 5632, 2048), (100, 1408, 1024), (128, 14336, 4096), (70, 200, 384)])
def test_split_k_swiglu_mid_m(ctx, orc, monkeypatch, dtype, M, Fd, K):
    """SwiGLU at 17 <= M <= 128 with K split: gate and up partial sums reduced
    before silu(g) * u, against the oracle and the unsplit kernel."""
    print(f"[case] split-K swiglu dtype={dtype} M={M} F={Fd} K={K}", flush=True)
    wg, gdec = _weight(ctx, 27, f"SG{Fd}x{K}", Fd, K, dtype)
    wu, udec = _weight(ctx, 27, f"SU{Fd}x{K}", Fd, K, dtype)
    x = F.normal(27, f"ssx{M}x{K}", M * K).reshape(M, K)
    dx = ctx.to_device(x)

    def run():
        dh = ctx.alloc(M * Fd * 4)
        ctx.qlinear_swiglu(wg, wu, dx, dh, M)
        return dh.download((M, Fd))

    monkeypatch.delenv("VLRF_HIP_PREFILL_DQ", raising=False)
    got = run()
    monkeypatch.setenv("VLRF_HIP_PREFILL_DQ", "0")
    unsplit = run()
    monkeypatch.delenv("VLRF_HIP_PREFILL_DQ", raising=False)
    ref = orc.silu_mul(orc.linear(x, udec), orc.linear(x, gdec))
    assert rel_err(got, ref) <= TOL
    assert rel_err(got, unsplit) <= 2e-5, rel_err(got, unsplit)


def _check_forms(a, b, c):
    """Expansion and in-LDS forms identical bit for bit; the in-register form
    identical too, except where the GEMM's few tiles make the two others
    split K into slices (300 x 4096 x 2048), which it does not: there it
    differs by the f32 summation order only."""
    assert np.array_equal(a, b)
    assert np.array_equal(a, c) or rel_err(a, c) <= 2e-5, rel_err(a, c)


def _all_forms(monkeypatch, run):
    """run() with the weights' bf16 expansion (the default for M > 128), with
    VLRF_HIP_PREFILL_BF16=0 (Q8_0 with K % 128 == 0: codes decoded into LDS
    tiles, once per workgroup; otherwise in registers) and with
    VLRF_HIP_PREFILL_DQ=0 as well (codes decoded in registers)."""
    monkeypatch.delenv("VLRF_HIP_PREFILL_BF16", raising=False)
    monkeypatch.delenv("VLRF_HIP_PREFILL_DQ", raising=False)
    a = run()
    monkeypatch.setenv("VLRF_HIP_PREFILL_BF16", "0")
    b = run()
    monkeypatch.setenv("VLRF_HIP_PREFILL_DQ", "0")
    c = run()
    monkeypatch.delenv("VLRF_HIP_PREFILL_BF16", raising=False)
    monkeypatch.delenv("VLRF_HIP_PREFILL_DQ", raising=False)
    return a, b, c


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
# 256x128 tiles (1000 x 1024), wide 256x256 tiles (2048 x 6144), a ragged
# wide edge (520 x 16600), the residual form (300 x 4096 x 2048), ragged rows
# and columns on the LDS-decode tiles (257 x 1000 x 256, 129 x 130 x 128, 300 x 100 x 384)
@pytest.mark.parametrize("M,N,K,res", [(1000, 1024, 512, False), (2048, 6144, 256, False),
                                       (520, 16600, 64, False), (300, 4096, 2048, True),
                                       (257, 1000, 256, False), (129, 130, 128, True),
                                       (300, 100, 384, True)])
def test_bf16_expansion_equals_in_register_decode(ctx, monkeypatch, dtype, M, N, K, res):
    """The GEMM over the weights' bf16 expansion multiplies the operands the
    in-register and in-LDS decodes form, in the same MFMA order: bit-identical
    outputs."""
    print(f"[case] bf16 expansion dtype={dtype} M={M} N={N} K={K} res={res}", flush=True)
    x = F.normal(24, f"bx{M}x{K}", M * K).reshape(M, K)
    r = F.normal(24, f"br{M}x{N}", M * N).reshape(M, N)
    dx = ctx.to_device(x)

    def run():
        w, _ = _weight(ctx, 24, f"B{N}x{K}", N, K, dtype)   # a fresh weight: no expansion yet
        dy = ctx.to_device(r) if res else ctx.alloc(M * N * 4)
        ctx.qlinear(w, dx, dy, M, residual=dy if res else None)
        return dy.download((M, N))

    a, b, c = _all_forms(monkeypatch, run)
    _check_forms(a, b, c)


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
# 2048 x 14336: 112 x 8 tiles of 256 x 128, the last round (128 columns x 8)
# as 128-row tiles over columns 12288..14335 (two launches)
@pytest.mark.parametrize("M,Fd,K", [(2048, 14336, 128), (257, 1000, 192), (257, 1000, 256), (600, 136, 512)])
def test_bf16_expansion_swiglu_equals_in_register_decode(ctx, monkeypatch, dtype, M, Fd, K):
    print(f"[case] bf16 expansion swiglu dtype={dtype} M={M} F={Fd} K={K}", flush=True)
    x = F.normal(25, f"sx{M}x{K}", M * K).reshape(M, K)
    dx = ctx.to_device(x)

    def run():
        wg, _ = _weight(ctx, 25, f"SG{Fd}x{K}", Fd, K, dtype)
        wu, _ = _weight(ctx, 25, f"SU{Fd}x{K}", Fd, K, dtype)
        dh = ctx.alloc(M * Fd * 4)
        ctx.qlinear_swiglu(wg, wu, dx, dh, M)
        return dh.download((M, Fd))

    a, b, c = _all_forms(monkeypatch, run)
    _check_forms(a, b, c)


def test_bf16_expansion_is_counted_in_the_weight_bytes(ctx):
    """vlrf_hip_weight_bytes: the packed codes and scales, plus 2 bytes per
    weight once a GEMM of more than 128 rows has made the bf16 expansion."""
    N, K, M = 384, 512, 200
    w, _ = _weight(ctx, 26, "WB", N, K, V.DT_Q8_0)
    packed = N * K + N * (K // 32) * 2
    assert w.device_bytes == packed
    x = ctx.to_device(F.normal(26, "wbx", M * K).reshape(M, K))
    y = ctx.alloc(M * N * 4)
    ctx.qlinear(w, x, y, 8)                      # M <= 128: no expansion
    assert w.device_bytes == packed
    ctx.qlinear(w, x, y, M)
    ctx.sync()
    assert w.device_bytes == packed + 2 * N * K


def _hip():
    import ctypes as C
    h = C.CDLL("libamdhip64.so")
    h.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    h.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    h.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    h.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    h.hipGraphExecDestroy.argtypes = [C.c_void_p]
    h.hipGraphDestroy.argtypes = [C.c_void_p]
    return h


@pytest.mark.parametrize("dtype", [V.DT_Q8_0, V.DT_Q4_0])
@pytest.mark.parametrize("M", [160, 64])
def test_prefill_gemm_under_graph_capture(orc, dtype, M):
    """A stream under graph capture: the M > 128 GEMM records no allocation
    (the weight's bf16 expansion is not made, the tiles decode the blocks),
    the captured graph replays to the eager result (over the expansion) bit
    for bit, replay after replay with eager work between; a call that would
    grow the context scratch while capturing is refused with an error
    instead of being recorded.  M = 64 takes the K-split GEMM and its reduce
    launch (partial sums in the context scratch after the bf16 rows)."""
    import ctypes as C
    hip = _hip()
    ctx = V.Context(0)                  # its own scratch buffer, empty until the first call
    N, K = 512, 1024
    print(f"[case] qgemm under capture dtype={dtype} M={M} N={N} K={K}", flush=True)
    w1, dec = _weight(ctx, 31, "cap", N, K, dtype)
    w2, _ = _weight(ctx, 31, "cap", N, K, dtype)              # the same blocks, never expanded
    packed = w2.device_bytes
    x = F.normal(31, "capx", M * K).reshape(M, K)
    dx, y1, y2 = ctx.to_device(x), ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ctx.qlinear(w1, dx, y1, M)                                 # eager: grows the scratch, expands w1
    ctx.sync()
    eager = y1.download((M, N))
    ref = x.astype(np.float64) @ dec.astype(np.float64).T
    assert rel_err(eager, ref) <= TOL
    s = C.c_void_p(ctx.stream())
    assert hip.hipStreamBeginCapture(s, 2) == 0               # hipStreamCaptureModeRelaxed
    rc = V.lib().vlrf_hip_qlinear(ctx.h, w2.h, dx.ptr, y2.ptr, M, None, C.c_float(0.0), None)
    g = C.c_void_p()
    assert hip.hipStreamEndCapture(s, C.byref(g)) == 0
    assert rc == 0, V.lib().vlrf_hip_last_error()
    assert V.lib().vlrf_hip_weight_bytes(w2.h) == packed       # no expansion recorded
    ge = C.c_void_p()
    assert hip.hipGraphInstantiate(C.byref(ge), g, None, None, 0) == 0
    for i in range(3):
        y2.zero()
        ctx.qlinear(w1, dx, y1, M)                             # eager work between replays
        assert hip.hipGraphLaunch(ge, s) == 0
        ctx.sync()
        got = y2.download((M, N))
        assert rel_err(got, ref) <= TOL, i
        assert np.array_equal(got, eager), i
    hip.hipGraphExecDestroy(ge)
    hip.hipGraphDestroy(g)
    # Scratch growth while capturing: refused, the capture ends cleanly.
    M2 = 4 * M
    dx2, y3 = ctx.to_device(np.tile(x, (4, 1))), ctx.alloc(M2 * N * 4)
    assert hip.hipStreamBeginCapture(s, 2) == 0
    rc = V.lib().vlrf_hip_qlinear(ctx.h, w1.h, dx2.ptr, y3.ptr, M2, None, C.c_float(0.0), None)
    g = C.c_void_p()
    hip.hipStreamEndCapture(s, C.byref(g))
    if g.value:
        hip.hipGraphDestroy(g)
    assert rc == _lib.ERR_ARG and b"captured" in V.lib().vlrf_hip_last_error()
    ctx.qlinear(w1, dx2, y3, M2)                               # eagerly it runs
    ctx.sync()
    assert rel_err(y3.download((M2, N))[:M], ref) <= TOL
