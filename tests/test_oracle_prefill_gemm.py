"""Pins the oracle's prefill GEMM path (per-(row, group) int8, src/q27_rb.cpp:43-55 and
src/q27_epi.hip:14-75, 189-243) against what the mathematics fixes, on the CPU:
- the int32 group slabs against numpy's exact int64 matrix product;
- the fp32 slab sum against a float64 evaluation of the same sum (a transposed or misindexed scale
  is off by far more than fp32 rounding);
- the group quantizers against their closed forms (identity and halving cases) and invariants
  (every code within half a step of its value, the group maximum at +-127)."""
import numpy as np


def rand_codes(rng, shape):
    return rng.integers(-127, 128, size=shape, dtype=np.int64).astype(np.int8)


def test_partials_are_exact_group_products(O):
    rng = np.random.default_rng(11)
    M, N, K, gs = 7, 48, 2048, 1024
    x, w = rand_codes(rng, (M, K)), rand_codes(rng, (N, K))
    x[0] = 127
    w[0] = -127                                   # extreme products in one slab
    part = np.empty((K // gs, M, N), np.int32)
    O.lib().q27o_gemm_i8g_partials(w.ctypes.data, N, K, gs, x.ctypes.data, M, part.ctypes.data)
    for g in range(K // gs):
        ref = x[:, g * gs:(g + 1) * gs].astype(np.int64) @ w[:, g * gs:(g + 1) * gs].astype(np.int64).T
        assert np.array_equal(part[g].astype(np.int64), ref)
    assert part[0, 0, 0] == -127 * 127 * gs


def gemm(O, w, sw, x, sx, gs, alpha, res=None, rs=0.0):
    N, K = w.shape
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    O.lib().q27o_gemm_i8g(w.ctypes.data, sw.ctypes.data, N, K, gs, alpha, x.ctypes.data, sx.ctypes.data, M,
                          y.ctypes.data, N, None if res is None else res.ctypes.data, N, rs)
    return y


def test_gemm_matches_float64_sum(O):
    rng = np.random.default_rng(12)
    M, N, K, gs = 9, 64, 5120, 1024
    ng = K // gs
    x, w = rand_codes(rng, (M, K)), rand_codes(rng, (N, K))
    sx = rng.uniform(0.001, 0.05, (M, ng)).astype(np.float32)
    sw = rng.uniform(1e-4, 2e-3, (N, ng)).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    y = gemm(O, w, sw, x, sx, gs, 0.75, res, 0.5)
    ref = np.zeros((M, N))
    for g in range(ng):
        acc = x[:, g * gs:(g + 1) * gs].astype(np.int64) @ w[:, g * gs:(g + 1) * gs].astype(np.int64).T
        ref += acc * (sx[:, g:g + 1].astype(np.float64) * sw[:, g].astype(np.float64)[None, :])
    ref = ref * 0.75 + 0.5 * res
    np.testing.assert_allclose(y, ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
    # one group over the whole K with unit scales is the exact integer product
    y1 = gemm(O, w, np.ones((N, 1), np.float32), x, np.ones((M, 1), np.float32), K, 1.0)
    exact = x.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(y1.astype(np.int64), exact)


def test_gemm_scale_indexing(O):
    # a scale that differs only for one (token, group) or one (row, group) changes only that output
    rng = np.random.default_rng(13)
    M, N, K, gs = 4, 8, 3072, 1024
    x, w = rand_codes(rng, (M, K)), rand_codes(rng, (N, K))
    sx = np.ones((M, 3), np.float32)
    sw = np.ones((N, 3), np.float32)
    base = gemm(O, w, sw, x, sx, gs, 1.0)
    sx2 = sx.copy()
    sx2[2, 1] = 2.0
    y = gemm(O, w, sw, x, sx2, gs, 1.0)
    g1 = x[2, gs:2 * gs].astype(np.int64) @ w[:, gs:2 * gs].astype(np.int64).T
    assert np.array_equal(np.delete(y, 2, axis=0), np.delete(base, 2, axis=0))
    np.testing.assert_allclose(y[2] - base[2], g1, rtol=0, atol=1e-3 * np.abs(g1).max() + 1)
    sw2 = sw.copy()
    sw2[5, 2] = 0.0
    y = gemm(O, w, sw2, x, sx, gs, 1.0)
    g2 = x[:, 2 * gs:].astype(np.int64) @ w[5, 2 * gs:].astype(np.int64)
    assert np.array_equal(np.delete(y, 5, axis=1), np.delete(base, 5, axis=1))
    np.testing.assert_allclose(base[:, 5] - y[:, 5], g2, rtol=0, atol=1e-3 * np.abs(g2).max() + 1)


def test_quant_tok_groups_invariants(O):
    rng = np.random.default_rng(14)
    M, K, gs = 5, 5120, 1024
    x = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
    x[1, 1024:2048] = 0.0                         # an all-zero group
    xq = np.empty((M, K), np.int8)
    xs = np.empty((M, K // gs), np.float32)
    O.lib().q27o_quant_tok_groups(x.ctypes.data, K, M, K, gs, xq.ctypes.data, xs.ctypes.data)
    assert xs[1, 1] == 0 and not xq[1, 1024:2048].any()
    for t in range(M):
        for g in range(K // gs):
            v = x[t, g * gs:(g + 1) * gs].astype(np.float64)
            s = float(xs[t, g])
            if s == 0:
                continue
            assert abs(s - np.abs(v).max() / 127) <= 1e-6 * s
            err = np.abs(xq[t, g * gs:(g + 1) * gs] * s - v)
            assert err.max() <= 0.5 * s * (1 + 1e-5)
            assert np.abs(xq[t, g * gs:(g + 1) * gs]).max() == 127


def test_i8g64_to_grp_closed_forms(O):
    rng = np.random.default_rng(15)
    rows, K, gs = 6, 2048, 1024
    w = rand_codes(rng, (rows, K))
    # powers of two, so the products are exact: equal sub-scales leave the codes unchanged, and a
    # block at half the group's scale halves its codes (rounded half to even)
    s64 = np.full((rows, K // 64), 2.0 ** -7, np.float32)
    s64[3, 20] = 2.0 ** -8                              # columns 1280..1343 of row 3
    wg = np.empty_like(w)
    sg = np.empty((rows, K // gs), np.float32)
    O.lib().q27o_i8g64_to_grp(w.ctypes.data, s64.ctypes.data, rows, K, gs, wg.ctypes.data, sg.ctypes.data)
    assert np.all(sg == np.float32(2.0 ** -7))
    expect = w.copy()
    half = w[3, 1280:1344].astype(np.float64) / 2
    expect[3, 1280:1344] = np.rint(half).astype(np.int8)   # round half to even
    assert np.array_equal(wg, expect)
    # the group scale is the largest sub-scale of its group, per row and group
    s64b = rng.uniform(0.001, 0.01, (rows, K // 64)).astype(np.float32)
    O.lib().q27o_i8g64_to_grp(w.ctypes.data, s64b.ctypes.data, rows, K, gs, wg.ctypes.data, sg.ctypes.data)
    assert np.array_equal(sg, s64b.reshape(rows, K // gs, gs // 64).max(axis=2))
    deq = wg.astype(np.float64) * np.repeat(sg, gs, axis=1)
    orig = w.astype(np.float64) * np.repeat(s64b, 64, axis=1)
    assert np.all(np.abs(deq - orig) <= 0.5 * np.repeat(sg, gs, axis=1) * (1 + 1e-5))
