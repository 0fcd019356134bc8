"""GPU parity of the engine's remaining per-op backend calls (IBackend::gemm,
layer_norm, softmax_inplace, gelu_inplace, add_inplace; ibackend.hpp:61-70)
against the oracle's restatements of ops.hpp (pinned against the reference
build in tests/test_oracle.py).  Tolerance 1e-3 relative (f32 paths); the
reductions run in a different order than the CPU's sequential loops."""
import numpy as np
import pytest

import vlrf_amd as V
from conftest import rel_err
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(1, 300, 64), (37, 29, 64), (130, 257, 515), (64, 64, 16), (200, 768, 3072)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_f32(ctx, orc, M, N, K, ta, tb):
    print(f"[case] gemm_f32 {M}x{N}x{K} ta={ta} tb={tb}", flush=True)
    A = F.normal(60, f"A{M}x{K}", M * K).reshape(M, K)
    B = F.normal(60, f"B{K}x{N}", K * N).reshape(K, N)
    Ai = A.T.copy() if ta else A
    Bi = B.T.copy() if tb else B
    for alpha, beta in ((1.0, 0.0), (0.7, 1.0), (-1.25, 0.5)):
        C0 = F.normal(60, f"C{M}x{N}", M * N).reshape(M, N)
        if beta == 0.0:
            C0[:] = np.nan                        # beta == 0 must not read C (ops.hpp:186-188)
        dA, dB, dC = ctx.to_device(Ai), ctx.to_device(Bi), ctx.to_device(C0)
        ctx.gemm_f32(dA, dB, dC, M, N, K, alpha, beta, ta, tb)
        got = dC.download((M, N))
        ref = orc.gemm(Ai, Bi, np.nan_to_num(C0) if beta == 0.0 else C0, alpha, beta, ta, tb)
        assert np.isfinite(got).all()
        assert rel_err(got, ref) <= 1e-3, (alpha, beta)


def test_gemm_f32_rejects_bad_shapes(ctx):
    a = ctx.alloc(64)
    with pytest.raises(V.HipError):
        ctx.gemm_f32(a, a, a, 0, 4, 4)
    with pytest.raises(V.HipError):
        ctx.gemm_f32(a, a, a, 4, 4, 4, lda=2)


@pytest.mark.parametrize("rows,D", [(1, 768), (7, 1000), (3, 5000), (2, 1)])
def test_layer_norm(ctx, orc, rows, D):
    x = F.normal(61, f"lx{D}", rows * D).reshape(rows, D) * 3 + 0.5
    w, b = 1 + F.normal(61, f"lw{D}", D, 0.1), F.normal(61, f"lb{D}", D, 0.1)
    dx, dw, db, do = ctx.to_device(x), ctx.to_device(w), ctx.to_device(b), ctx.alloc(x.nbytes)
    ctx.layer_norm(dx, dw, db, do, rows, D, 1e-5)
    assert rel_err(do.download(x.shape), orc.layer_norm(x, w, b, 1e-5)) <= 1e-3


@pytest.mark.parametrize("rows,D", [(1, 2048), (12, 77), (4, 5000), (3, 1)])
def test_softmax(ctx, orc, rows, D):
    x = F.normal(62, f"sx{D}", rows * D).reshape(rows, D) * 4
    if D > 2:
        x[0, 1] = -np.inf                         # a masked score: exp(-inf) = 0
    dx = ctx.to_device(x)
    ctx.softmax(dx, rows, D)
    got = dx.download(x.shape)
    ref = orc.softmax(x)        # the oracle sums sequentially for every D
    assert rel_err(got, ref) <= 1e-3
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-5)


@pytest.mark.parametrize("n", [1, 1000, 300001])
def test_gelu_and_add(ctx, orc, n):
    x = F.normal(63, f"gx{n}", n) * 5
    dx = ctx.to_device(x)
    ctx.gelu(dx, n)
    assert rel_err(dx.download(x.shape), orc.gelu(x)) <= 1e-5 * 10
    y = F.normal(63, f"gy{n}", n)
    a, b = ctx.to_device(x), ctx.to_device(y)
    ctx.add(a, b, n)
    assert np.array_equal(a.download(x.shape), x + y)       # one rounding per element, as the CPU
