"""Pins the oracle's quantizers and projections (oracle/q27o.c) against closed forms and float64:
  R5  activation quantizer  src/q27_fp8.hip:373-425
  R8  weight mirror rule    src/q27_nvfp4.hip:4259-4289
  R16 SwiGLU + quantize     src/q27_nvfp4.hip:3984-4031
  R7  W8A8 projection       src/q27_fp8.hip:3814-3871 (exact int32 per 16-slab, fp32 scaling)
  R9  bf16 GEMV             src/q27_util.hip:114-167
  R22 RMSNorm (1+w) + quantize  src/q27_elem.hip:453-613, 835-910
Each check is chosen so that a plausible slip (127 vs 128, a transposed operand, a scale taken
from the wrong group, a dropped residual term) fails it."""
import numpy as np
import pytest

import ref64


def quant_rows(O, x_bf16, n, nr, in_scale=1.0):
    xq = np.empty((nr, n), np.int8)
    xs = np.empty((nr, n // 16), np.float32)
    O.lib().q27o_quant_rows(x_bf16.ctypes.data, n, xq.ctypes.data, n, xs.ctypes.data, n // 16, n, in_scale, nr)
    return xq, xs


def test_r5_quantizer_invariants(O):
    rng = np.random.default_rng(10)
    nr, n = 3, 5120
    x = O.f2bf(rng.standard_normal((nr, n)).astype(np.float32))
    x[0, :16] = 0                                                     # all-zero group
    x[1, 16:32] = O.f2bf(np.full(16, -0.75, np.float32))              # constant group
    xq, xs = quant_rows(O, x, n, nr)
    v = ref64.bf2f(x).astype(np.float64)
    assert np.abs(xq.astype(int)).max() <= 127
    assert (xq[0, :16] == 0).all() and xs[0, 0] == 0.0
    assert (xq[1, 16:32] == -127).all()
    g = v.reshape(nr, -1, 16)
    imax = np.abs(g).argmax(axis=2)
    codes = xq.reshape(nr, -1, 16)
    top = np.take_along_axis(codes, imax[..., None], 2)[..., 0]
    nz = np.abs(g).max(axis=2) > 0
    assert (np.abs(top[nz]) == 127).all()                             # the group max maps to +-127
    assert (np.sign(top[nz]) == np.sign(np.take_along_axis(g, imax[..., None], 2)[..., 0][nz])).all()
    # scale = max|x| / 127 (to fp32 rounding), codes = float64 ideal except at exact half ties
    np.testing.assert_allclose(xs.astype(np.float64), np.abs(g).max(axis=2) / 127.0, rtol=2e-7)
    ref64.assert_codes_match_ideal(xq, v, 16)
    # dequantization error within half a step
    deq = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 16, axis=1)
    assert (np.abs(deq - v) <= np.repeat(xs.astype(np.float64), 16, axis=1) * (0.5 + 1e-5)).all()


def test_r5_half_even_ties_and_in_scale(O):
    """With max|x| = 127 the step is exactly 1, so x = k + 1/2 exercises rint's half-to-even:
    2.5 -> 2, 3.5 -> 4, -2.5 -> -2, -0.5 -> 0, 0.5 -> 0, 1.5 -> 2."""
    vals = np.array([127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, -1.5, 126.5, 5.5, 0, -127, 64, 4.5, -3.5, 7.5],
                    np.float32)
    x = O.f2bf(vals)[None, :]
    xq, xs = quant_rows(O, x, 16, 1)
    assert xs[0, 0] == np.float32(1.0)
    assert xq[0].tolist() == [127, 2, 4, -2, 0, 0, 2, -2, 126, 6, 0, -127, 64, 4, -4, 8]
    # in_scale cancels in the codes (g/s = 127/mx) and multiplies the stored scale by 1/in_scale
    rng = np.random.default_rng(3)
    y = O.f2bf(rng.standard_normal((2, 256)).astype(np.float32))
    q1, s1 = quant_rows(O, y, 256, 2, 1.0)
    q2, s2 = quant_rows(O, y, 256, 2, 0.25)
    assert np.array_equal(q1, q2)
    np.testing.assert_allclose(s2, s1 * 4, rtol=1e-6)


def test_r8_weight_quantizer(O):
    rng = np.random.default_rng(11)
    rows, K = 96, 1024
    w = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    w[5, 64:128] = 0
    wq = np.empty((rows, K), np.int8)
    ws = np.empty((rows, K // 64), np.float32)
    O.lib().q27o_quant_weights_i8g64(w.ctypes.data, rows, K, wq.ctypes.data, ws.ctypes.data)
    assert ws[5, 1] == 0 and (wq[5, 64:128] == 0).all()
    np.testing.assert_allclose(ws.astype(np.float64), np.abs(w.reshape(rows, -1, 64)).max(axis=2) / 127.0,
                               rtol=2e-7)
    ref64.assert_codes_match_ideal(wq, w, 64)
    g = np.abs(wq.reshape(rows, -1, 64).astype(int)).max(axis=2)
    assert ((g == 127) | (ws == 0)).all()                            # per-64 groups, not per-16 or per-row


def test_r16_swiglu_quant(O):
    rng = np.random.default_rng(12)
    nr, n = 3, 2048
    g = (rng.standard_normal((nr, n)) * 3).astype(np.float32)
    u = (rng.standard_normal((nr, n)) * 3).astype(np.float32)
    g[0, :4] = [-100.0, 100.0, 0.0, 88.0]
    xq = np.empty((nr, n), np.int8)
    xs = np.empty((nr, n // 16), np.float32)
    O.lib().q27o_swiglu_quant_rows(g.ctypes.data, u.ctypes.data, n, xq.ctypes.data, xs.ctypes.data, n, 1.0, nr)
    v = ref64.silu(g) * u
    np.testing.assert_allclose(xs.astype(np.float64), np.abs(v.reshape(nr, -1, 16)).max(axis=2) / 127.0, rtol=3e-6)
    ref64.assert_codes_match_ideal(xq, v, 16, tie_tol=2e-4)
    assert xq[0, 2] == 0                                              # silu(0) * u = 0


@pytest.mark.parametrize("rows,K,nr", [(257, 5120, 3), (64, 1024, 8), (33, 17408, 1)])
def test_r7_partials_exact_and_fp32_output(O, rows, K, nr):
    rng = np.random.default_rng(rows + K)
    w = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    wq = np.empty((rows, K), np.int8)
    ws = np.empty((rows, K // 64), np.float32)
    O.lib().q27o_quant_weights_i8g64(w.ctypes.data, rows, K, wq.ctypes.data, ws.ctypes.data)
    x = O.f2bf(rng.standard_normal((nr, K)).astype(np.float32))
    xq, xs = quant_rows(O, x, K, nr)
    part = np.empty((nr, rows, K // 16), np.int32)
    O.lib().q27o_proj_partials(wq.ctypes.data, rows, K, xq.ctypes.data, K, part.ctypes.data, nr)
    brute = np.einsum("rsk,nsk->nrs", wq.reshape(rows, -1, 16).astype(np.int64),
                      xq.reshape(nr, -1, 16).astype(np.int64))
    assert np.array_equal(part.astype(np.int64), brute)
    assert np.abs(part).max() <= 16 * 127 * 127
    y = np.empty((nr, rows), np.float32)
    alpha = 0.75
    O.lib().q27o_proj_rows(wq.ctypes.data, ws.ctypes.data, alpha, rows, K, xq.ctypes.data, K, xs.ctypes.data,
                           y.ctypes.data, rows, nr)
    ref = ref64.proj(wq, ws, xq, xs, alpha)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    assert err < 2e-6, err
    # sensitivity: the same comparison rejects a scale read from the neighbouring 64-group
    ref_bad = ref64.proj(wq, np.roll(ws, 1, axis=1), xq, xs, alpha)
    assert np.abs(y - ref_bad).max() / np.abs(ref).max() > 1e-2


def test_r7_epilogue_residual_and_bf16(O):
    rng = np.random.default_rng(13)
    rows, K, nr = 128, 2048, 3
    w = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    wq = np.empty((rows, K), np.int8)
    ws = np.empty((rows, K // 64), np.float32)
    O.lib().q27o_quant_weights_i8g64(w.ctypes.data, rows, K, wq.ctypes.data, ws.ctypes.data)
    xq, xs = quant_rows(O, O.f2bf(rng.standard_normal((nr, K)).astype(np.float32)), K, nr)
    res = O.f2bf(rng.standard_normal((nr, rows)).astype(np.float32))
    y = np.empty((nr, rows), np.uint16)
    O.lib().q27o_proj_rows_epi(wq.ctypes.data, ws.ctypes.data, 1.0, rows, K, xq.ctypes.data, K, xs.ctypes.data,
                               y.ctypes.data, rows, 1, res.ctypes.data, 1, rows, 0.5, nr)
    ref = ref64.proj(wq, ws, xq, xs, 1.0) + 0.5 * ref64.bf2f(res).astype(np.float64)
    got = ref64.bf2f(y).astype(np.float64)
    # bf16 output: within half a bf16 step (2^-9 relative) plus the fp32 accumulation error
    assert (np.abs(got - ref) <= np.abs(ref) * (2.0 ** -8) + 1e-6).all()
    fp = np.empty((nr, rows), np.float32)
    O.lib().q27o_proj_rows(wq.ctypes.data, ws.ctypes.data, 1.0, rows, K, xq.ctypes.data, K, xs.ctypes.data,
                           fp.ctypes.data, rows, nr)
    assert np.array_equal(y, ref64.bf16_rne(fp + np.float32(0.5) * ref64.bf2f(res)))


def test_r9_bf16_gemv(O):
    rng = np.random.default_rng(14)
    rows, K, nr = 300, 5120, 3
    W = O.f2bf((rng.standard_normal((rows, K)) * 0.02).astype(np.float32))
    x = O.f2bf(rng.standard_normal((nr, K)).astype(np.float32))
    y = np.empty((nr, rows), np.float32)
    O.lib().q27o_bf16_gemv_rows(W.ctypes.data, rows, K, x.ctypes.data, K, y.ctypes.data, rows, nr)
    ref = ref64.bf2f(x).astype(np.float64) @ ref64.bf2f(W).astype(np.float64).T
    assert np.abs(y - ref).max() / np.abs(ref).max() < 2e-6


@pytest.mark.parametrize("x_bf16,quant_bf16,plus", [(1, 1, 1.0), (0, 0, 1.0), (0, 1, 0.0)])
def test_r22_rmsnorm_quant(O, x_bf16, quant_bf16, plus):
    rng = np.random.default_rng(15 + x_bf16)
    nr, n = 3, 5120
    xf = (rng.standard_normal((nr, n)) * 3).astype(np.float32)
    x = O.f2bf(xf) if x_bf16 else xf
    xv = ref64.bf2f(x) if x_bf16 else xf
    w = O.f2bf((rng.standard_normal(n) * 0.1 + (1 - plus)).astype(np.float32))
    hc, y = np.empty((nr, n), np.uint16), np.empty((nr, n), np.uint16)
    xq, xs = np.empty((nr, n), np.int8), np.empty((nr, n // 16), np.float32)
    O.lib().q27o_rmsnorm_quant_rows(x.ctypes.data, x_bf16, n, w.ctypes.data, plus, 1e-6, n, hc.ctypes.data,
                                    y.ctypes.data, n, xq.ctypes.data, xs.ctypes.data, quant_bf16, 1.0, nr)
    ref = ref64.rmsnorm(xv, ref64.bf2f(w), plus, 1e-6)
    got = ref64.bf2f(y).astype(np.float64)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-7).all()
    assert np.array_equal(hc, ref64.bf16_rne(xv))
    src = ref64.bf2f(y) if quant_bf16 else ref
    ref64.assert_codes_match_ideal(xq, src, 16, tie_tol=1e-3)
