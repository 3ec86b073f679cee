"""The committed golden fixtures (tests/golden/, written by make_golden.py) against the oracle
(CPU) and the HIP path (GPU): exact integer results, float64 textbook values within tolerance, and
the tiny model's greedy token streams."""
import json
import os

import numpy as np
import pytest

import ref64

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def F():
    return dict(np.load(os.path.join(GOLD, "kernels.npz")))


@pytest.fixture(scope="module")
def T():
    with open(os.path.join(GOLD, "tiny_tokens.json")) as fh:
        return json.load(fh)


def test_golden_r5(O, F):
    x = F["r5_x"]
    xq, xs = np.empty((3, 256), np.int8), np.empty((3, 16), np.float32)
    O.lib().q27o_quant_rows(x.ctypes.data, 256, xq.ctypes.data, 256, xs.ctypes.data, 16, 256, 1.0, 3)
    assert np.array_equal(xq, F["r5_xq"]) and np.array_equal(xs, F["r5_xs"])
    assert F["r5_xq"][1, :8].tolist() == [127, 2, 4, -2, 0, 0, 2, -2]          # half-even ties
    ref64.assert_codes_match_ideal(F["r5_xq"], ref64.bf2f(x), 16)


def test_golden_r7(O, F):
    wq, ws, xq, xs = F["r7_wq"], F["r7_ws"], F["r7_xq"], F["r7_xs"]
    part = np.empty((3, 64, 64), np.int32)
    O.lib().q27o_proj_partials(wq.ctypes.data, 64, 1024, xq.ctypes.data, 1024, part.ctypes.data, 3)
    assert np.array_equal(part, F["r7_part"])
    y = np.empty((3, 64), np.float32)
    O.lib().q27o_proj_rows(wq.ctypes.data, ws.ctypes.data, 1.0, 64, 1024, xq.ctypes.data, 1024, xs.ctypes.data,
                           y.ctypes.data, 64, 3)
    assert np.array_equal(y, F["r7_y"])
    assert np.abs(y - F["r7_y64"]).max() <= 2e-6 * np.abs(F["r7_y64"]).max()


def test_golden_gdn(O, F):
    kh, vh, d, nr = 1, 2, 128, 3
    nqkv, nz = (2 * kh + vh) * d, vh * d
    g = {k[4:]: F[k] for k in F if k.startswith("gdn_")}
    S, hist = g["S"].copy(), g["hist"].copy()
    pend = np.zeros(O.lib().q27o_gdn_pend_bytes(kh, vh, d, 8), np.uint8)
    out = np.empty((nr, nz), np.uint16)
    args = lambda q, z, a, b, o, npend, n: (q.ctypes.data, nqkv, z.ctypes.data, nz, a.ctypes.data, b.ctypes.data, vh,
                                            g["A_log"].ctypes.data, g["dt_bias"].ctypes.data, g["norm_w"].ctypes.data,
                                            g["conv_w"].ctypes.data, S.ctypes.data, hist.ctypes.data, pend.ctypes.data,
                                            npend, kh, vh, d, 1e-6, o.ctypes.data, nz, None, None, n)
    O.lib().q27o_gdn_verify(*args(g["qkv"], g["z"], g["a"], g["b"], out, 0, nr))
    assert np.array_equal(out, g["out"])
    got = ref64.bf2f(out).astype(np.float64)
    assert np.linalg.norm(got - g["y64"]) / np.linalg.norm(g["y64"]) < 4e-3
    one = {k: np.ascontiguousarray(g[k][:1]) for k in ("qkv", "z", "a", "b")}
    o1 = np.empty((1, nz), np.uint16)
    O.lib().q27o_gdn_verify(*args(one["qkv"], one["z"], one["a"], one["b"], o1, 2, 1))
    assert np.array_equal(S, g["S_commit2"])
    _, S64, _ = ref64.gdn_rows(g["qkv"][:2], g["z"][:2], g["a"][:2], g["b"][:2], g["A_log"], g["dt_bias"],
                               g["norm_w"], g["conv_w"], g["S"], g["hist"], kh, vh, d)
    assert np.abs(S - S64).max() <= 1e-5 * np.abs(S64).max()


def test_golden_tiny_tokens_oracle(O, T):
    m = O.Model(T["config"], T["seed"])
    p = np.array(T["prompt"], np.int32)
    first = m.prefill(p)
    plain = [first] + [m.decode_step() for _ in range(len(T["plain"]) - 1)]
    assert plain == T["plain"]
    m.prefill(p)
    for r, exp in enumerate(T["spec_rounds"]):
        assert m.spec_round() == exp, r
    m.close()


@pytest.mark.gpu
def test_golden_tiny_tokens_gpu(gpu, T):
    X = gpu
    c = X.tiny_config()
    for k, v in T["config"].items():
        setattr(c, k, v)
    eng = X.Engine(c, T["seed"])
    p = np.array(T["prompt"], np.int32)
    first = eng.prefill(p)
    plain = [first] + [eng.decode_step() for _ in range(len(T["plain"]) - 1)]
    assert plain == T["plain"]
    eng.prefill(p)
    for r, exp in enumerate(T["spec_rounds"]):
        assert eng.spec_round() == exp, r
    eng.close()


@pytest.mark.gpu
def test_golden_r7_gpu(gpu, F):
    X = gpu
    wq, ws, xq, xs = F["r7_wq"], F["r7_ws"], F["r7_xq"], F["r7_xs"]
    dq, ds, dxq, dxs = X.DevBuf(array=wq), X.DevBuf(array=ws), X.DevBuf(array=xq), X.DevBuf(array=xs)
    h = X.I8G(dq.ptr, ds.ptr, 1.0, 64, 1024)
    import ctypes
    part, dy = X.DevBuf(3 * 64 * 64 * 4), X.DevBuf(3 * 64 * 4)
    X.call("q27x_proj_partials", ctypes.byref(h), dxq.ptr, 1024, part.ptr, 3, None)
    X.call("q27x_proj_rows", ctypes.byref(h), dxq.ptr, 1024, dxs.ptr, dy.ptr, 64, 0, None, 0, 0, 0.0, 3, None)
    X.call("q27x_device_sync")
    assert np.array_equal(part.download(np.int32, (3, 64, 64)), F["r7_part"])
    assert np.array_equal(dy.download(np.float32, (3, 64)), F["r7_y"])
