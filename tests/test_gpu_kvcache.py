"""GPU parity: the Q8_0 KV cache (kv_cache.hpp).  Quantize/pack must match
quantize_row_q8_0 (kv_cache.hpp:102-117) bit for bit on the same f32 rows;
edge cases follow tests/test_kv_cache_quant.cpp (zero row, round-trip bound,
reset, overflow)."""
import numpy as np
import pytest

import vlrf_amd as V
from vlrf_amd import formats as F

pytestmark = pytest.mark.gpu


def _oracle_rows(orc, rows):
    qs, ss = [], []
    for r in rows:
        q, s = orc.quantize_row_q8_0(r)
        qs.append(q)
        ss.append(s)
    return np.stack(qs), np.array(ss, np.float32)


def _append(ctx, kv, layer, K, Vv):
    T = K.shape[0]
    kv.append(layer, ctx.to_device(K), ctx.to_device(Vv), T)


@pytest.mark.parametrize("n_kv,d,T", [(4, 64, 300), (8, 128, 17), (1, 64, 1), (2, 16, 5)])
def test_append_bit_exact(ctx, orc, n_kv, d, T):
    row = n_kv * d
    kv = V.KVCache(ctx, 2, 512, n_kv, d)
    K = (F.normal(3, "K", T * row) * 2.5).reshape(T, row)
    Vv = (F.normal(3, "V", T * row) * 0.7).reshape(T, row)
    _append(ctx, kv, 1, K, Vv)
    assert kv.used(1) == T and kv.used(0) == 0
    kq, vq, ks, vs = kv.read(1, 0, T)
    ekq, eks = _oracle_rows(orc, K)
    evq, evs = _oracle_rows(orc, Vv)
    assert np.array_equal(kq, ekq) and np.array_equal(vq, evq)
    assert np.array_equal(ks.view(np.uint32), eks.view(np.uint32))
    assert np.array_equal(vs.view(np.uint32), evs.view(np.uint32))


def test_append_special_rows(ctx, orc):
    """All-zero row -> scale 0 and zero codes (test_kv_cache_quant.cpp:62-71);
    +/-amax -> +/-127; exact .5 ties round away from zero (std::lround)."""
    row = 64
    zero = np.zeros(row, np.float32)
    ties = np.zeros(row, np.float32)
    ties[0] = 127.0                      # amax 127 -> scale 1, inv 1
    ties[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
    tiny = np.full(row, 1e-30, np.float32)
    tiny[3] = -2e-30
    big = F.normal(9, "big", row) * 1e30
    rows = np.stack([zero, ties, tiny, big])
    kv = V.KVCache(ctx, 1, 8, 1, row)
    _append(ctx, kv, 0, rows, rows[::-1].copy())
    kq, vq, ks, vs = kv.read(0, 0, 4)
    eq, es = _oracle_rows(orc, rows)
    assert np.array_equal(kq, eq) and np.array_equal(ks.view(np.uint32), es.view(np.uint32))
    assert ks[0] == 0.0 and not kq[0].any()
    assert list(kq[1][:9]) == [127, 1, -1, 2, -2, 3, -3, 127, -127]
    evq, evs = _oracle_rows(orc, rows[::-1].copy())
    assert np.array_equal(vq, evq) and np.array_equal(vs.view(np.uint32), evs.view(np.uint32))


def test_roundtrip_bound_and_dequant(ctx, orc):
    """max error <= 1.5*amax/127 per row (test_kv_cache_quant.cpp:39-60) and the
    device dequant equals code * scale exactly (kv_cache.hpp:119-121)."""
    n_kv, d, T = 4, 64, 40
    row = n_kv * d
    kv = V.KVCache(ctx, 1, 64, n_kv, d)
    K = (F.normal(4, "K", T * row) * 5).reshape(T, row)
    Vv = (F.normal(4, "V", T * row) * 5).reshape(T, row)
    _append(ctx, kv, 0, K, Vv)
    Kd, Vd = ctx.alloc(K.nbytes), ctx.alloc(Vv.nbytes)
    kv.dequant_into(0, T, Kd, Vd)
    kd, vd = Kd.download((T, row)), Vd.download((T, row))
    kq, vq, ks, vs = kv.read(0, 0, T)
    assert np.array_equal(kd, kq.astype(np.float32) * ks[:, None])
    assert np.array_equal(vd, vq.astype(np.float32) * vs[:, None])
    for t in range(T):
        amax = np.abs(K[t]).max()
        assert np.abs(kd[t] - K[t]).max() <= 1.5 * amax / 127


def test_incremental_appends_and_reset(ctx, orc):
    n_kv, d = 2, 64
    row = n_kv * d
    kv = V.KVCache(ctx, 1, 16, n_kv, d)
    rows = F.normal(6, "K", 5 * row).reshape(5, row)
    for t in range(5):                   # token-by-token, as decode appends
        _append(ctx, kv, 0, rows[t:t + 1], rows[t:t + 1] * 2)
    assert kv.used(0) == 5
    kq, _, ks, _ = kv.read(0, 0, 5)
    eq, es = _oracle_rows(orc, rows)
    assert np.array_equal(kq, eq) and np.array_equal(ks, es)
    kv.reset()
    assert kv.used(0) == 0
    kq, vq, ks, vs = kv.read(0, 0, 16)
    assert not kq.any() and not vq.any() and not ks.any() and not vs.any()


def test_overflow_is_an_error(ctx):
    """KVCache::append throws past max_seq_len (test_kv_cache_quant.cpp:135-147)."""
    kv = V.KVCache(ctx, 1, 2, 1, 16)
    one = np.ones((1, 16), np.float32)
    _append(ctx, kv, 0, one, one)
    _append(ctx, kv, 0, one, one)
    with pytest.raises(V.HipError) as e:
        _append(ctx, kv, 0, one, one)
    assert e.value.rc == -4
    assert kv.used(0) == 2
