"""GPU parity: RMSNorm (ops.hpp:478-499) and RoPE (rope.hpp:49-99).
RoPE is bit-exact: same host tables, each product rounded separately."""
import numpy as np
import pytest

from conftest import rel_err
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,D", [(1, 2048), (3, 4096), (7, 100)])
def test_rmsnorm(ctx, orc, rows, D):
    x = F.normal(1, "x", rows * D).reshape(rows, D) * 3
    w = 1.0 + F.normal(1, "w", D, 0.2)
    dx, dw, do = ctx.to_device(x), ctx.to_device(w), ctx.alloc(x.nbytes)
    ctx.rms_norm(dx, dw, do, rows, D, 1e-5)
    out = do.download(x.shape)
    ref = orc.rms_norm(x, w, 1e-5)
    assert rel_err(out, ref) <= 1e-5


@pytest.mark.parametrize("T,n_heads,d_head,pos,max_seq", [(1, 32, 64, 2047, 2176), (5, 4, 64, 0, 64),
                                                          (3, 8, 128, 60, 62), (2, 2, 16, 7, 9)])
def test_rope_bit_exact(ctx, orc, T, n_heads, d_head, pos, max_seq):
    """Includes positions at/after max_seq, which the reference leaves unrotated."""
    x = F.normal(2, "x", T * n_heads * d_head)
    dx = ctx.to_device(x)
    ctx.rope(dx, T, n_heads, d_head, pos, max_seq, 10000.0)
    out = dx.download(x.shape)
    tabs = orc.rope_tables(max_seq, d_head, 10000.0)
    ref = orc.rope_apply(x, n_heads, d_head, pos, tabs, max_seq)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_device_copy_roundtrip(ctx):
    """vlrf_hip_d2d: a device-to-device copy returns the bytes unchanged."""
    a = np.arange(1 << 20, dtype=np.int32) * 7 - 5
    src, dst = ctx.to_device(a), ctx.alloc(a.nbytes)
    dst.copy_from(src)
    ctx.sync()
    assert np.array_equal(dst.download(a.shape, np.int32), a)
