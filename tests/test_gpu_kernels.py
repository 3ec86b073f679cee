"""Kernel-tier parity: every gfx950 kernel against the CPU oracle on the same seeded inputs,
through the C ABI. Integer results and fp32/bf16 outputs are compared bit for bit (the kernels
and the oracle share one fixed reduction order); shapes are benchmark configs 0-2."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def same(name, got, ref):
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    g = got.view(np.uint8) if got.dtype.kind == "f" else got
    r = ref.view(np.uint8) if ref.dtype.kind == "f" else ref
    if not np.array_equal(g, r):
        bad = np.flatnonzero(got.ravel() != ref.ravel())
        pytest.fail(f"{name}: {bad.size} of {got.size} differ; first {bad[:5]}: "
                    f"got {got.ravel()[bad[:5]]} ref {ref.ravel()[bad[:5]]}")


def bf16_normal(rng, shape, std=1.0, O=None):
    return O.f2bf((rng.standard_normal(shape) * std).astype(np.float32))


def dev(X, a):
    return X.DevBuf(array=a)


def quant_weights(X, O, rng, rows, K, std=0.02):
    w = (rng.standard_normal((rows, K)) * std).astype(np.float32)
    wq_o = np.empty((rows, K), np.int8)
    ws_o = np.empty((rows, K // 64), np.float32)
    O.lib().q27o_quant_weights_i8g64(w.ctypes.data, rows, K, wq_o.ctypes.data, ws_o.ctypes.data)
    dw = dev(X, w)
    dq = X.DevBuf(rows * K)
    ds = X.DevBuf(rows * K // 16)
    X.call("q27x_quant_weights_i8g64", dw.ptr, rows, K, dq.ptr, ds.ptr, None)
    X.call("q27x_device_sync")
    same("R8 weight codes", dq.download(np.int8, (rows, K)), wq_o)
    same("R8 weight scales", ds.download(np.float32, (rows, K // 64)), ws_o)
    dw.free()
    return wq_o, ws_o, dq, ds


@pytest.mark.parametrize("nr", [1, 3, 8])
def test_quant_rows(gpu, O, nr):
    X = gpu
    rng = np.random.default_rng(0x51E70000 + nr)
    n = 5120
    x = bf16_normal(rng, (nr, n), O=O)
    x[0, :16] = 0                      # an all-zero group
    x[0, 16:32] = O.f2bf(np.float32(0.5) * np.arange(16, dtype=np.float32))   # exact ties
    xq_o = np.empty((nr, n), np.int8)
    xs_o = np.empty((nr, n // 16), np.float32)
    O.lib().q27o_quant_rows(x.ctypes.data, n, xq_o.ctypes.data, n, xs_o.ctypes.data, n // 16, n, 1.0, nr)
    dx, dq, ds = dev(X, x), X.DevBuf(nr * n), X.DevBuf(nr * n // 4)
    X.call("q27x_quant_rows", dx.ptr, n, dq.ptr, n, ds.ptr, n // 16, n, 1.0, nr, None)
    X.call("q27x_device_sync")
    same("R5 codes", dq.download(np.int8, (nr, n)), xq_o)
    same("R5 scales", ds.download(np.float32, (nr, n // 16)), xs_o)


@pytest.mark.parametrize("nr", [3])
def test_proj_config0(gpu, O, nr):
    """Benchmark config 0: 3 rows x [17408 x 5120] int8 W8A8, per-64 / per-16 scales."""
    X = gpu
    rng = np.random.default_rng(0x51E70000)
    rows, K = 17408, 5120
    x = bf16_normal(rng, (nr, K), O=O)
    xq = np.empty((nr, K), np.int8)
    xs = np.empty((nr, K // 16), np.float32)
    O.lib().q27o_quant_rows(x.ctypes.data, K, xq.ctypes.data, K, xs.ctypes.data, K // 16, K, 1.0, nr)
    wq, ws, dq, ds = quant_weights(X, O, rng, rows, K)
    h = X.I8G(dq.ptr, ds.ptr, 1.0, rows, K)
    dxq, dxs = dev(X, xq), dev(X, xs)
    # int32 slab partials: exact, against the oracle and an int64 numpy brute force
    part = X.DevBuf(nr * rows * (K // 16) * 4)
    X.call("q27x_proj_partials", ctypes.byref(h), dxq.ptr, K, part.ptr, nr, None)
    X.call("q27x_device_sync")
    got = part.download(np.int32, (nr, rows, K // 16))
    sub = slice(0, 257)
    brute = np.einsum("rsk,nsk->nrs", wq[sub].reshape(-1, K // 16, 16).astype(np.int64),
                      xq.reshape(nr, K // 16, 16).astype(np.int64))
    same("int32 partials vs int64 brute force", got[:, sub].astype(np.int64), brute)
    po = np.empty((nr, rows, K // 16), np.int32)
    O.lib().q27o_proj_partials(wq.ctypes.data, rows, K, xq.ctypes.data, K, po.ctypes.data, nr)
    same("int32 partials vs oracle", got, po)
    part.free()
    # fp32 output, bf16 output, fp32 + bf16 residual
    y_o = np.empty((nr, rows), np.float32)
    O.lib().q27o_proj_rows(wq.ctypes.data, ws.ctypes.data, 1.0, rows, K, xq.ctypes.data, K, xs.ctypes.data,
                           y_o.ctypes.data, rows, nr)
    dy = X.DevBuf(nr * rows * 4)
    X.call("q27x_proj_rows", ctypes.byref(h), dxq.ptr, K, dxs.ptr, dy.ptr, rows, 0, None, 0, 0, 0.0, nr, None)
    X.call("q27x_device_sync")
    y = dy.download(np.float32, (nr, rows))
    same("fp32 projection", y, y_o)
    ref64 = np.einsum("nrs,rs,ns->nr", po.astype(np.float64), ws.repeat(4, axis=1).astype(np.float64),
                      xs.astype(np.float64))
    rel = np.abs(y - ref64).max() / np.abs(ref64).max()
    assert rel < 1e-5, rel
    res = bf16_normal(rng, (nr, rows), O=O)
    dres = dev(X, res)
    X.call("q27x_proj_rows", ctypes.byref(h), dxq.ptr, K, dxs.ptr, dy.ptr, rows, 1, dres.ptr, 1, rows, 1.0, nr, None)
    X.call("q27x_device_sync")
    yb_o = np.empty((nr, rows), np.uint16)
    O.lib().q27o_proj_rows_epi(wq.ctypes.data, ws.ctypes.data, 1.0, rows, K, xq.ctypes.data, K, xs.ctypes.data,
                               yb_o.ctypes.data, rows, 1, res.ctypes.data, 1, rows, 1.0, nr)
    same("bf16 projection + bf16 residual", dy.download(np.uint16, (nr, rows)), yb_o)


@pytest.mark.parametrize("rows,K,nr", [(5120, 6144, 3), (5120, 17408, 3), (5120, 17408, 8), (5120, 17408, 5),
                                       (1000, 17408, 7), (5120, 17408, 4), (5120, 17408, 6), (10240, 5120, 8),
                                       (5120, 6144, 8), (5120, 4096, 7), (5120, 4096, 2), (1000, 1024, 5),
                                       (1000, 3136, 6)])
def test_proj_shapes(gpu, O, rows, K, nr):
    X = gpu
    rng = np.random.default_rng(rows * 7 + K + nr)
    x = bf16_normal(rng, (nr, K), O=O)
    xq = np.empty((nr, K), np.int8)
    xs = np.empty((nr, K // 16), np.float32)
    O.lib().q27o_quant_rows(x.ctypes.data, K, xq.ctypes.data, K, xs.ctypes.data, K // 16, K, 1.0, nr)
    wq, ws, dq, ds = quant_weights(X, O, rng, rows, K)
    h = X.I8G(dq.ptr, ds.ptr, 0.75, rows, K)
    res = rng.standard_normal((nr, rows)).astype(np.float32)
    y_o = np.empty((nr, rows), np.float32)
    O.lib().q27o_proj_rows_epi(wq.ctypes.data, ws.ctypes.data, 0.75, rows, K, xq.ctypes.data, K, xs.ctypes.data,
                               y_o.ctypes.data, rows, 0, res.ctypes.data, 0, rows, 1.0, nr)
    dxq, dxs, dres, dy = dev(X, xq), dev(X, xs), dev(X, res), X.DevBuf(nr * rows * 4)
    X.call("q27x_proj_rows", ctypes.byref(h), dxq.ptr, K, dxs.ptr, dy.ptr, rows, 0, dres.ptr, 0, rows, 1.0, nr, None)
    X.call("q27x_device_sync")
    same(f"proj {rows}x{K} nr={nr}", dy.download(np.float32, (nr, rows)), y_o)


@pytest.mark.parametrize("nr", [1, 3, 5, 8])
def test_bf16_gemv(gpu, O, nr):
    X = gpu
    rng = np.random.default_rng(11 + nr)
    rows, K = 62080, 5120
    w = bf16_normal(rng, (rows, K), 0.02, O=O)
    x = bf16_normal(rng, (nr, K), O=O)
    y_o = np.empty((nr, rows), np.float32)
    O.lib().q27o_bf16_gemv_rows(w.ctypes.data, rows, K, x.ctypes.data, K, y_o.ctypes.data, rows, nr)
    dw, dx, dy = dev(X, w), dev(X, x), X.DevBuf(nr * rows * 4)
    X.call("q27x_bf16_gemv_rows", dw.ptr, rows, K, dx.ptr, K, dy.ptr, rows, 0, nr, None)
    X.call("q27x_device_sync")
    y = dy.download(np.float32, (nr, rows))
    same("bf16 gemv", y, y_o)
    # argmax over these logits (ties -> lowest index; a planted tie and a NaN)
    y[0, 7] = np.float32(np.nan)
    y[0, 100] = np.nanmax(y[0]) + 1
    y[0, 50] = y[0, 100]
    dl = dev(X, y)
    di, dv = X.DevBuf(4 * nr), X.DevBuf(4 * nr)
    X.call("q27x_argmax_rows", dl.ptr, rows, rows, nr, di.ptr, dv.ptr, None)
    X.call("q27x_device_sync")
    idx = di.download(np.int32, (nr,))
    i_o = np.empty(nr, np.int32)
    v_o = np.empty(nr, np.float32)
    O.lib().q27o_argmax_rows(y.ctypes.data, rows, rows, nr, i_o.ctypes.data, v_o.ctypes.data)
    same("argmax", idx, i_o)
    assert idx[0] == 50
    yy = np.where(np.isfinite(y), y, -np.inf)
    assert (idx == np.argmax(yy, axis=1)).all()


@pytest.mark.parametrize("x_bf16,quant_bf16", [(1, 1), (0, 0), (0, 1)])
def test_rmsnorm_quant(gpu, O, x_bf16, quant_bf16):
    X = gpu
    rng = np.random.default_rng(5 + 2 * x_bf16 + quant_bf16)
    nr, n = 3, 5120
    if x_bf16:
        x = bf16_normal(rng, (nr, n), 3.0, O=O)
    else:
        x = (rng.standard_normal((nr, n)) * 3).astype(np.float32)
    w = bf16_normal(rng, (n,), 0.02, O=O)
    hc_o, y_o = np.empty((nr, n), np.uint16), np.empty((nr, n), np.uint16)
    xq_o, xs_o = np.empty((nr, n), np.int8), np.empty((nr, n // 16), np.float32)
    O.lib().q27o_rmsnorm_quant_rows(x.ctypes.data, x_bf16, n, w.ctypes.data, 1.0, 1e-6, n, hc_o.ctypes.data,
                                    y_o.ctypes.data, n, xq_o.ctypes.data, xs_o.ctypes.data, quant_bf16, 1.0, nr)
    dx, dw = dev(X, x), dev(X, w)
    dh, dy, dq, ds = X.DevBuf(nr * n * 2), X.DevBuf(nr * n * 2), X.DevBuf(nr * n), X.DevBuf(nr * n // 4)
    X.call("q27x_rmsnorm_quant_rows", dx.ptr, x_bf16, n, dw.ptr, 1.0, 1e-6, n, dh.ptr, dy.ptr, n, dq.ptr, ds.ptr,
           quant_bf16, 1.0, nr, None)
    X.call("q27x_device_sync")
    same("norm hcopy", dh.download(np.uint16, (nr, n)), hc_o)
    same("norm y", dy.download(np.uint16, (nr, n)), y_o)
    same("norm codes", dq.download(np.int8, (nr, n)), xq_o)
    same("norm scales", ds.download(np.float32, (nr, n // 16)), xs_o)


def test_swiglu_quant(gpu, O):
    X = gpu
    rng = np.random.default_rng(77)
    nr, n = 3, 17408
    g = (rng.standard_normal((nr, n)) * 2).astype(np.float32)
    u = (rng.standard_normal((nr, n)) * 2).astype(np.float32)
    g[0, :5] = [-100.0, 100.0, 0.0, -20.0, 88.0]
    xq_o, xs_o = np.empty((nr, n), np.int8), np.empty((nr, n // 16), np.float32)
    O.lib().q27o_swiglu_quant_rows(g.ctypes.data, u.ctypes.data, n, xq_o.ctypes.data, xs_o.ctypes.data, n, 1.0, nr)
    dg, du, dq, ds = dev(X, g), dev(X, u), X.DevBuf(nr * n), X.DevBuf(nr * n // 4)
    X.call("q27x_swiglu_quant_rows", dg.ptr, du.ptr, n, dq.ptr, ds.ptr, n, 1.0, nr, None)
    X.call("q27x_device_sync")
    same("swiglu codes", dq.download(np.int8, (nr, n)), xq_o)
    same("swiglu scales", ds.download(np.float32, (nr, n // 16)), xs_o)


@pytest.mark.parametrize("op,lo,hi", [(0, -110, 95), (1, -160, 130), (2, -0.99, 1e9), (3, -100, 100),
                                      (4, -100, 100), (5, -30, 30)])
def test_math_bit_exact(gpu, O, op, lo, hi):
    X = gpu
    rng = np.random.default_rng(op)
    x = rng.uniform(lo, hi, 1 << 16).astype(np.float32)
    if op == 2:
        x = np.concatenate([x, np.logspace(-12, 9, 4096).astype(np.float32)])
    x = np.concatenate([x, np.array([0.0, -0.0, 1e-30, -1e-30, 20.0, 20.000002], np.float32)])
    y_o = np.empty_like(x)
    O.lib().q27o_math_vec(x.ctypes.data, y_o.ctypes.data, x.size, op)
    dx, dy = dev(X, x), X.DevBuf(x.nbytes)
    X.call("q27x_math_test", dx.ptr, dy.ptr, x.size, op, None)
    X.call("q27x_device_sync")
    same(f"math op {op}", dy.download(np.float32, x.shape), y_o)


def gdn_inputs(rng, O, nr, kh=16, vh=48, d=128):
    nqkv = (2 * kh + vh) * d
    return dict(
        qkv=bf16_normal(rng, (nr, nqkv), 1.0, O=O),
        z=bf16_normal(rng, (nr, vh * d), 1.0, O=O),
        a=rng.uniform(-4, 0, (nr, vh)).astype(np.float32),
        b=rng.uniform(-4, 0, (nr, vh)).astype(np.float32))


@pytest.mark.parametrize("rollback", [0, 1, 2])
def test_gdn_verify_config1(gpu, O, rollback):
    """Benchmark config 1 GDN core: 3 verify rows, state ~N(0, 0.1), a/b ~U(-4, 0), then a second
    call that commits an accepted prefix of rollback + 1 rows (the rest rolled back), then the
    commit-only entry for that call's accepted prefix followed by a call with nothing pending --
    all compared bit for bit with the oracle."""
    X = gpu
    rng = np.random.default_rng(0x51E70001 + 17 * rollback)
    kh, vh, d, nr = 16, 48, 128, 3
    nqkv, nz = (2 * kh + vh) * d, vh * d
    S = (rng.standard_normal((vh, d, d)) * 0.1).astype(np.float32)
    hist = bf16_normal(rng, (nqkv, 3), O=O)
    conv_w = bf16_normal(rng, (nqkv, 4), 0.3, O=O)
    A_log = O.f2bf(rng.uniform(0, 2.7, vh).astype(np.float32))
    dt_bias = bf16_normal(rng, (vh,), 0.1, O=O)
    norm_w = O.f2bf((1 + rng.standard_normal(d) * 0.02).astype(np.float32))
    So, ho = S.copy(), hist.copy()
    pend_o = np.zeros(O.lib().q27o_gdn_pend_bytes(kh, vh, d, 8), np.uint8)
    dS, dh = dev(X, S), dev(X, hist)
    dpend = X.DevBuf(X.lib().q27x_gdn_pend_bytes(kh, vh, d, 8))
    dpend.zero()
    dconv, dA, ddt, dnw = dev(X, conv_w), dev(X, A_log), dev(X, dt_bias), dev(X, norm_w)
    for call_i, npend in enumerate([0, rollback + 1, 2 - rollback + 1]):
        if call_i == 2:
            # commit the previous call's accepted prefix on its own, then run with nothing pending;
            # the oracle gets the same prefix as npend of one call
            X.call("q27x_gdn_commit", dS.ptr, dh.ptr, dpend.ptr, npend, kh, vh, d, None)
        gpu_npend = 0 if call_i == 2 else npend
        inp = gdn_inputs(rng, O, nr, kh, vh, d)
        out_o = np.empty((nr, nz), np.uint16)
        xq_o, xs_o = np.empty((nr, nz), np.int8), np.empty((nr, nz // 16), np.float32)
        O.lib().q27o_gdn_verify(inp["qkv"].ctypes.data, nqkv, inp["z"].ctypes.data, nz, inp["a"].ctypes.data,
                                inp["b"].ctypes.data, vh, A_log.ctypes.data, dt_bias.ctypes.data, norm_w.ctypes.data,
                                conv_w.ctypes.data, So.ctypes.data, ho.ctypes.data, pend_o.ctypes.data, npend, kh, vh,
                                d, 1e-6, out_o.ctypes.data, nz, xq_o.ctypes.data, xs_o.ctypes.data, nr)
        dq, dzz, da, db = dev(X, inp["qkv"]), dev(X, inp["z"]), dev(X, inp["a"]), dev(X, inp["b"])
        dout, dxq, dxs = X.DevBuf(nr * nz * 2), X.DevBuf(nr * nz), X.DevBuf(nr * nz // 4)
        X.call("q27x_gdn_verify", dq.ptr, nqkv, dzz.ptr, nz, da.ptr, db.ptr, vh, dA.ptr, ddt.ptr, dnw.ptr, dconv.ptr,
               dS.ptr, dh.ptr, dpend.ptr, gpu_npend, kh, vh, d, dout.ptr, nz, dxq.ptr, dxs.ptr, nr, None)
        X.call("q27x_device_sync")
        same(f"gdn out (call {call_i})", dout.download(np.uint16, (nr, nz)), out_o)
        same(f"gdn codes (call {call_i})", dxq.download(np.int8, (nr, nz)), xq_o)
        same(f"gdn scales (call {call_i})", dxs.download(np.float32, (nr, nz // 16)), xs_o)
        same(f"gdn committed state (call {call_i})", dS.download(np.float32, S.shape), So)
        same(f"conv history (call {call_i})", dh.download(np.uint16, hist.shape), ho)


def fill_kv(rng, O, L, nkv, hd, group, ctx):
    kv = nkv * hd
    kc, vc = np.zeros((ctx, kv), np.int8), np.zeros((ctx, kv), np.int8)
    ks, vs = np.zeros((ctx, kv // group), np.float32), np.zeros((ctx, kv // group), np.float32)
    K = rng.standard_normal((L, kv)).astype(np.float32)
    V = rng.standard_normal((L, kv)).astype(np.float32)
    for arr, c, s in ((K, kc, ks), (V, vc, vs)):
        q = np.empty(L * kv, np.int8)
        sc = np.empty(L * kv // group, np.float32)
        O.lib().q27o_quant_f32(arr.ctypes.data, L * kv, group, q.ctypes.data, sc.ctypes.data)
        c[:L] = q.reshape(L, kv)
        s[:L] = sc.reshape(L, kv // group)
    return kc, ks, vc, vs


def attention_case(X, O, L0, nq, nkv, hd, rot, group, nr, seed):
    """Prep (norm, RoPE, K/V to the int8 cache) of nr rows at positions L0.. and their attention over
    the L0 cached positions before them plus their own, through the kernel tier, against the oracle
    bit for bit: q, the cache codes and scales, the output, its codes and scales."""
    rng = np.random.default_rng(seed)
    gate = 1
    ctx = L0 + nr
    qw = 2 * hd
    qkv_rows = nq * qw + 2 * nkv * hd
    kc, ks, vc, vs = fill_kv(rng, O, L0, nkv, hd, group, ctx)
    qkv = bf16_normal(rng, (nr, qkv_rows), 1.0, O=O)
    qn, kn = bf16_normal(rng, (hd,), 0.02, O=O), bf16_normal(rng, (hd,), 0.02, O=O)
    cs = np.empty(ctx * rot // 2, np.float32)
    sn = np.empty(ctx * rot // 2, np.float32)
    O.lib().q27o_rope_table(ctx, rot, 1e7, cs.ctypes.data, sn.ctypes.data)
    dk, dks, dv, dvs = dev(X, kc), dev(X, ks), dev(X, vc), dev(X, vs)
    dqkv, dqn, dkn, dcs, dsn = dev(X, qkv), dev(X, qn), dev(X, kn), dev(X, cs), dev(X, sn)
    dqh = X.DevBuf(nr * nq * hd * 2)
    qh_o = np.empty((nr, nq * hd), np.uint16)
    O.lib().q27o_attn_prep_rows(qkv.ctypes.data, qkv_rows, qn.ctypes.data, kn.ctypes.data, cs.ctypes.data,
                                sn.ctypes.data, rot, kc.ctypes.data, ks.ctypes.data, vc.ctypes.data, vs.ctypes.data,
                                group, qh_o.ctypes.data, nq, nkv, hd, gate, 1e-6, L0, nr)
    X.call("q27x_attn_prep_rows", dqkv.ptr, qkv_rows, dqn.ptr, dkn.ptr, dcs.ptr, dsn.ptr, rot, dk.ptr, dks.ptr,
           dv.ptr, dvs.ptr, group, dqh.ptr, nq, nkv, hd, gate, 1e-6, L0, nr, None)
    X.call("q27x_device_sync")
    same("q after norm+rope", dqh.download(np.uint16, (nr, nq * hd)), qh_o)
    same("K cache", dk.download(np.int8, kc.shape), kc)
    same("K scales", dks.download(np.float32, ks.shape), ks)
    same("V cache", dv.download(np.int8, vc.shape), vc)
    same("V scales", dvs.download(np.float32, vs.shape), vs)
    out_o = np.empty((nr, nq * hd), np.uint16)
    xq_o, xs_o = np.empty((nr, nq * hd), np.int8), np.empty((nr, nq * hd // 16), np.float32)
    O.lib().q27o_attn_rows(qh_o.ctypes.data, qkv.ctypes.data, qkv_rows, kc.ctypes.data, ks.ctypes.data,
                           vc.ctypes.data, vs.ctypes.data, group, nq, nkv, hd, gate, L0, nr, out_o.ctypes.data,
                           xq_o.ctypes.data, xs_o.ctypes.data)
    work = X.DevBuf(X.lib().q27x_attn_work_bytes(nq, hd, ctx, nr))
    dout, dxq, dxs = X.DevBuf(nr * nq * hd * 2), X.DevBuf(nr * nq * hd), X.DevBuf(nr * nq * hd // 4)
    X.call("q27x_attn_rows", dqh.ptr, dqkv.ptr, qkv_rows, dk.ptr, dks.ptr, dv.ptr, dvs.ptr, group, nq, nkv, hd, gate,
           L0, nr, work.ptr, dout.ptr, dxq.ptr, dxs.ptr, None)
    X.call("q27x_device_sync")
    same("attention out", dout.download(np.uint16, (nr, nq * hd)), out_o)
    same("attention codes", dxq.download(np.int8, (nr, nq * hd)), xq_o)
    same("attention scales", dxs.download(np.float32, (nr, nq * hd // 16)), xs_o)


@pytest.mark.parametrize("L0", [1024, 4096, 16384, 20000])
def test_attention_config2(gpu, O, L0):
    """Benchmark config 2: GQA 32q/8kv x 128, RoPE theta 1e7, int8 KV per 32, 3 causal verify rows.
    (20000 positions: 313 splits, past one LDS window of the combine, which then takes two.)"""
    attention_case(gpu, O, L0, 32, 8, 128, 32, 32, 3, 0x51E70002 + L0)


@pytest.mark.parametrize("L0,nr", [(0, 1), (5, 3), (61, 3), (1100, 3), (2100, 8), (9700, 1), (20000, 2)])
def test_attention_trunk_geometry(gpu, O, L0, nr):
    """The reference trunk's attention (include/q27.h:25-35): 24 q / 4 kv heads of 256 dims (GQA
    group 6), q_proj emitting q and the output gate per head, RoPE on the first 64 of 256 dims
    (src/q27_attn.hip:10-11), int8 KV per 32; rows straddling a 64-key split, one split to several
    per block (2100 and more positions: 33+ splits on 64 blocks per kv head), and a combine over
    two LDS windows (20000 positions: 313 splits against a window of 150)."""
    attention_case(gpu, O, L0, 24, 4, 256, 64, 32, nr, 0x51E70020 + L0)


def test_attention_group_6_at_128(gpu, O):
    """A GQA group that is not a power of two at 128-dim heads (the general kernel at 128)."""
    attention_case(gpu, O, 700, 24, 4, 128, 32, 32, 3, 0x51E70021)


def test_accept(gpu):
    X = gpu
    for nx, dt, exp in (([5, 6, 7], [5, 6], 2), ([5, 6, 7], [5, 9], 1), ([5, 6, 7], [4, 6], 0), ([1], [], 0)):
        k = len(dt)
        dnx = X.DevBuf(array=np.array(nx, np.int32))
        ddt = X.DevBuf(array=np.array(dt + [0], np.int32))
        dn, dc = X.DevBuf(8), X.DevBuf(32)
        X.call("q27x_accept", dnx.ptr, ddt.ptr, k, dn.ptr, dc.ptr, None)
        X.call("q27x_device_sync")
        nacc, ncommit = dn.download(np.int32, (2,))
        assert nacc == exp and ncommit == exp + 1
        assert dc.download(np.int32, (8,))[: ncommit].tolist() == nx[: ncommit]


def test_mtp_draft_entry_matches_oracle(gpu, O):
    """Kernel-tier MTP draft layer (q27x_mtp_draft) against the oracle's mtp_pass on the tiny
    geometry: a 3-row pass at positions 0..2 (head row 2), a 2-row pass at 3..4 that attends to
    the cache (head row 1), and a catch-up row that overwrites position 1 -- residual rows, the
    drafted tokens and the layer's whole KV cache bit for bit."""
    X = gpu
    cfg = X.tiny_config(spec_k=2, n_layers=4)
    eng = X.Engine(cfg, 0x51E70003)
    om = O.Model(cfg, 0x51E70003)
    rng = np.random.default_rng(0x51E7A010)
    H = cfg.hidden
    h = O.f2bf(rng.standard_normal((6, H)).astype(np.float32))
    t = rng.integers(0, cfg.vocab, 6).astype(np.int32)
    for rows, dpos0, head in ((slice(0, 3), 0, 2), (slice(3, 5), 3, 1), (slice(5, 6), 1, 0), (slice(0, 2), 4, -1)):
        tg, rg = eng.mtp_draft(h[rows], t[rows], dpos0, head)
        to, ro, _ = om.mtp_pass(h[rows], t[rows], dpos0, head)
        same(f"mtp residual rows at {dpos0}", rg, ro)
        if head >= 0:
            assert tg == to, (dpos0, tg, to)
    n = cfg.ctx * cfg.n_kv * cfg.head_dim
    for name, dt, cnt in (("kc", np.int8, n), ("vc", np.int8, n), ("ks", np.float32, n // cfg.kv_group),
                          ("vs", np.float32, n // cfg.kv_group)):
        same(f"mtp cache {name}", eng.read(name, -1, dt, cnt), om.tensor(name, -1, dt)[:cnt])
    eng.close()
    om.close()
