"""Prefill ingest on int8 MFMA: the per-(row, group) GEMM and its two quantizers (the reference's
layer-split prefill data path, src/q27_rb.cpp:43-55 and src/q27_epi.hip:14-75, 189-243) against
the CPU oracle, bit for bit, through the C ABI. The int32 group sums are exact whatever the MFMA
tiling, and the fp32 slab sum runs in the reference's group order, so outputs match exactly."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q27X_E_SHAPE = -2


def same(name, got, ref):
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    if not np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        bad = np.flatnonzero(got.ravel() != ref.ravel())
        pytest.fail(f"{name}: {bad.size} of {got.size} differ; first {bad[:5]}: "
                    f"got {got.ravel()[bad[:5]]} ref {ref.ravel()[bad[:5]]}")


def codes(rng, shape):
    return rng.integers(-127, 128, size=shape, dtype=np.int64).astype(np.int8)


def gpu_gemm(X, w, sw, x, sx, gs, alpha, res=None, rs=0.0):
    N, K = w.shape
    M = x.shape[0]
    bufs = [X.DevBuf(array=a) for a in (w, sw, x, sx)]
    dy = X.DevBuf(M * N * 4)
    dr = X.DevBuf(array=res) if res is not None else None
    X.call("q27x_gemm_i8g", bufs[0].ptr, bufs[1].ptr, N, K, gs, alpha, bufs[2].ptr, bufs[3].ptr, M, dy.ptr, N,
           dr.ptr if dr else None, N, rs, None)
    X.call("q27x_device_sync")
    y = dy.download(np.float32, (M, N))
    for b in bufs + [dy] + ([dr] if dr else []):
        b.free()
    return y


def oracle_gemm(O, w, sw, x, sx, gs, alpha, res=None, rs=0.0):
    N, K = w.shape
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    O.lib().q27o_gemm_i8g(w.ctypes.data, sw.ctypes.data, N, K, gs, alpha, x.ctypes.data, sx.ctypes.data, M,
                          y.ctypes.data, N, None if res is None else res.ctypes.data, N, rs)
    return y


@pytest.mark.parametrize("M,N,K,gs,with_res", [
    (1, 128, 1024, 1024, False),       # one token, one group
    (37, 256, 5120, 1024, True),       # ragged token tile, residual
    (128, 128, 2048, 1024, False),     # exactly one tile
    (300, 384, 5120, 5120, True),      # one group over the whole K (per-token scales)
    (130, 256, 17408, 1024, False),    # down's K: 17 groups
    (257, 128, 6144, 1024, True),      # out_proj's K
    (600, 256, 5120, 1024, True),      # 256-token tiles (register-staged), ragged last tile
    (1024, 384, 17408, 1024, False),   # 256-token tiles (register-staged), 17 groups
    (520, 128, 1152, 1152, True),      # 256-token tiles, K % 256 != 0: the LDS-DMA ring
    (777, 256, 3200, 640, False),      # 256-token tiles, K % 256 != 0, 5 groups of 640
    (600, 256, 5120, 5120, True),      # 256-token tiles, one group over the whole K (the default arm)
    (130, 256, 17408, 17408, False),   # down's K as one group
    (1024, 384, 17408, 17408, True),   # 256-token tiles, down's K as one group
])
def test_gemm_i8g(gpu, O, M, N, K, gs, with_res):
    rng = np.random.default_rng(0x51E70400 + M + N + K)
    ng = K // gs
    w, x = codes(rng, (N, K)), codes(rng, (M, K))
    w[0], x[0] = 127, -127                                    # extreme products
    sw = rng.uniform(1e-4, 2e-3, (N, ng)).astype(np.float32)
    sx = rng.uniform(1e-3, 5e-2, (M, ng)).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32) if with_res else None
    y = gpu_gemm(gpu, w, sw, x, sx, gs, 0.8125, res, 1.0)
    same(f"gemm {M}x{N}x{K}/{gs}", y, oracle_gemm(O, w, sw, x, sx, gs, 0.8125, res, 1.0))


@pytest.mark.parametrize("M,N,K,with_res", [
    (512, 256, 256, False),     # one tile, two K stages
    (600, 512, 5120, True),     # ragged last token tile, two weight tiles, residual
    (777, 768, 1152, True),     # an odd number of K stages
    (1024, 256, 17408, False),  # down's K as one group (136 stages)
])
def test_gemm_i8g_wide_tiles(gpu, O, monkeypatch, M, N, K, with_res):
    # the 256 x 256 tiles of the whole-K arm, taken at shapes where the launch would otherwise use
    # the 256 x 128 ones (Q27X_GEMM_W4 = 1), against the oracle bit for bit
    monkeypatch.setenv("Q27X_GEMM_W4", "1")
    rng = np.random.default_rng(0x51E70500 + M + N + K)
    w, x = codes(rng, (N, K)), codes(rng, (M, K))
    w[0], x[0] = 127, -127
    sw = rng.uniform(1e-4, 2e-3, (N, 1)).astype(np.float32)
    sx = rng.uniform(1e-3, 5e-2, (M, 1)).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32) if with_res else None
    y = gpu_gemm(gpu, w, sw, x, sx, K, 0.8125, res, 1.0)
    same(f"wide-tile gemm {M}x{N}x{K}", y, oracle_gemm(O, w, sw, x, sx, K, 0.8125, res, 1.0))


@pytest.mark.parametrize("gs", [5120, 1024])
def test_gemm_i8g_full_shape_sampled(gpu, O, gs):
    # the prefill shape of gate (M = 4096 tokens, N = 17408, K = 5120) with whole-K groups (the
    # default) and 1024-column groups: the whole product on the GPU, eight token rows (first, last,
    # and across the token tiles) recomputed by the oracle
    X = gpu
    rng = np.random.default_rng(0x51E70404)
    M, N, K = 4096, 17408, 5120
    w, x = codes(rng, (N, K)), codes(rng, (M, K))
    sw = rng.uniform(1e-4, 2e-3, (N, K // gs)).astype(np.float32)
    sx = rng.uniform(1e-3, 5e-2, (M, K // gs)).astype(np.float32)
    y = gpu_gemm(X, w, sw, x, sx, gs, 1.0)
    rows = np.array([0, 1, 127, 128, 1500, 2049, 4094, 4095])
    same("gemm 4096x17408x5120 sampled rows", y[rows],
         oracle_gemm(O, w, sw, np.ascontiguousarray(x[rows]), np.ascontiguousarray(sx[rows]), gs, 1.0))


def test_gemm_i8g_rejects_shapes(gpu):
    X = gpu
    L = X.lib()
    a = X.DevBuf(1 << 20)
    for N, K, gs in ((100, 1024, 1024), (128, 1000, 1000), (128, 2048, 192), (128, 43008, 1024)):
        rc = L.q27x_gemm_i8g(a.ptr, a.ptr, N, K, gs, 1.0, a.ptr, a.ptr, 4, a.ptr, N, None, N, 0.0, None)
        assert rc == Q27X_E_SHAPE, (N, K, gs, rc)
    a.free()


@pytest.mark.parametrize("K,gs", [(5120, 1024), (5120, 5120), (17408, 1024), (17408, 17408)])
def test_quant_tok_groups(gpu, O, K, gs):
    X = gpu
    rng = np.random.default_rng(0x51E70410 + K + gs)
    M = 7
    x = (rng.standard_normal((M, K)) * rng.uniform(0.05, 20, (M, 1))).astype(np.float32)
    x[1, :gs] = 0.0                                           # an all-zero group
    x[2, :16] = np.float32(0.5) * np.arange(16, dtype=np.float32)   # exact half ties after scaling
    xq_o = np.empty((M, K), np.int8)
    xs_o = np.empty((M, K // gs), np.float32)
    O.lib().q27o_quant_tok_groups(x.ctypes.data, K, M, K, gs, xq_o.ctypes.data, xs_o.ctypes.data)
    dx, dq, ds = X.DevBuf(array=x), X.DevBuf(M * K), X.DevBuf(M * (K // gs) * 4)
    X.call("q27x_quant_tok_groups", dx.ptr, K, M, K, gs, dq.ptr, ds.ptr, None)
    X.call("q27x_device_sync")
    same("token-group codes", dq.download(np.int8, (M, K)), xq_o)
    same("token-group scales", ds.download(np.float32, (M, K // gs)), xs_o)
    for b in (dx, dq, ds):
        b.free()


@pytest.mark.parametrize("rows,K,gs,in_place", [(300, 5120, 1024, False), (64, 17408, 1024, True),
                                                (128, 5120, 5120, False)])
def test_i8g64_to_grp(gpu, O, rows, K, gs, in_place):
    X = gpu
    rng = np.random.default_rng(0x51E70420 + rows + K)
    w = codes(rng, (rows, K))
    s64 = rng.uniform(1e-4, 3e-3, (rows, K // 64)).astype(np.float32)
    s64[0, :gs // 64] = 0.0                                   # an all-zero group scale
    wg_o = np.empty_like(w)
    sg_o = np.empty((rows, K // gs), np.float32)
    O.lib().q27o_i8g64_to_grp(w.ctypes.data, s64.ctypes.data, rows, K, gs, wg_o.ctypes.data, sg_o.ctypes.data)
    dw, ds64, dsg = X.DevBuf(array=w), X.DevBuf(array=s64), X.DevBuf(rows * (K // gs) * 4)
    dwg = dw if in_place else X.DevBuf(rows * K)
    X.call("q27x_i8g64_to_grp", dw.ptr, ds64.ptr, rows, K, gs, dwg.ptr, dsg.ptr, None)
    X.call("q27x_device_sync")
    same("group codes", dwg.download(np.int8, (rows, K)), wg_o)
    same("group scales", dsg.download(np.float32, (rows, K // gs)), sg_o)
    for b in {id(b): b for b in (dw, ds64, dsg, dwg)}.values():
        b.free()


def test_prefill_chain_quant_then_gemm(gpu, O):
    # weights from the per-64 mirror and activations from fp32 rows, both quantized on the GPU,
    # then the GEMM: the three steps chained as the prefill runs them
    X = gpu
    rng = np.random.default_rng(0x51E70430)
    M, N, K, gs = 200, 256, 5120, 1024
    w64 = codes(rng, (N, K))
    s64 = rng.uniform(1e-4, 3e-3, (N, K // 64)).astype(np.float32)
    xf = rng.standard_normal((M, K)).astype(np.float32)
    wg_o, sg_o = np.empty_like(w64), np.empty((N, K // gs), np.float32)
    O.lib().q27o_i8g64_to_grp(w64.ctypes.data, s64.ctypes.data, N, K, gs, wg_o.ctypes.data, sg_o.ctypes.data)
    xq_o, xs_o = np.empty((M, K), np.int8), np.empty((M, K // gs), np.float32)
    O.lib().q27o_quant_tok_groups(xf.ctypes.data, K, M, K, gs, xq_o.ctypes.data, xs_o.ctypes.data)
    y_o = oracle_gemm(O, wg_o, sg_o, xq_o, xs_o, gs, 1.0)
    dw, ds64, dsg = X.DevBuf(array=w64), X.DevBuf(array=s64), X.DevBuf(N * (K // gs) * 4)
    dx, dxq, dxs, dy = X.DevBuf(array=xf), X.DevBuf(M * K), X.DevBuf(M * (K // gs) * 4), X.DevBuf(M * N * 4)
    X.call("q27x_i8g64_to_grp", dw.ptr, ds64.ptr, N, K, gs, dw.ptr, dsg.ptr, None)
    X.call("q27x_quant_tok_groups", dx.ptr, K, M, K, gs, dxq.ptr, dxs.ptr, None)
    X.call("q27x_gemm_i8g", dw.ptr, dsg.ptr, N, K, gs, 1.0, dxq.ptr, dxs.ptr, M, dy.ptr, N, None, N, 0.0, None)
    X.call("q27x_device_sync")
    same("chained prefill GEMM", dy.download(np.float32, (M, N)), y_o)
    for b in (dw, ds64, dsg, dx, dxq, dxs, dy):
        b.free()
