#!/usr/bin/env python3
"""Writes the committed golden fixtures of the verify path (tests/golden/*.npz, *.json).

The reference ships no usable golden vectors for this path (its tests/reference_tokens.txt needs
the real checkpoint and four MI50s), so the fixtures are made here: seeded small inputs, the
float64 textbook results (tests/ref64.py, written from the mathematics) and the oracle's exact
outputs. tests/test_golden.py checks the oracle against both on every CPU run, and the GPU tests
check the HIP path against the oracle. Run from the repo root: python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import q27o  # noqa: E402
import ref64  # noqa: E402


def quant_rows(x, n, nr):
    xq, xs = np.empty((nr, n), np.int8), np.empty((nr, n // 16), np.float32)
    q27o.lib().q27o_quant_rows(x.ctypes.data, n, xq.ctypes.data, n, xs.ctypes.data, n // 16, n, 1.0, nr)
    return xq, xs


def kernels():
    L = q27o.lib()
    rng = np.random.default_rng(0x51E70000)
    f = {}
    # R5 activation quantizer: 3 rows x 256 with a zero group and exact half ties
    x = q27o.f2bf(rng.standard_normal((3, 256)).astype(np.float32))
    x[0, :16] = 0
    x[1, :16] = q27o.f2bf(np.array([127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, -1.5, 126.5, 5.5, 0, -127, 64, 4.5, -3.5, 7.5],
                                   np.float32))
    f["r5_x"] = x
    f["r5_xq"], f["r5_xs"] = quant_rows(x, 256, 3)
    # R7 projection: 64 x 1024 int8 per-64 weights, 3 rows
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    wq, ws = np.empty((64, 1024), np.int8), np.empty((64, 16), np.float32)
    L.q27o_quant_weights_i8g64(w.ctypes.data, 64, 1024, wq.ctypes.data, ws.ctypes.data)
    xq, xs = quant_rows(q27o.f2bf(rng.standard_normal((3, 1024)).astype(np.float32)), 1024, 3)
    f.update(r7_wq=wq, r7_ws=ws, r7_xq=xq, r7_xs=xs)
    f["r7_part"] = np.einsum("rsk,nsk->nrs", wq.reshape(64, -1, 16).astype(np.int64),
                             xq.reshape(3, -1, 16).astype(np.int64)).astype(np.int32)
    f["r7_y64"] = ref64.proj(wq, ws, xq, xs, 1.0)
    y = np.empty((3, 64), np.float32)
    L.q27o_proj_rows(wq.ctypes.data, ws.ctypes.data, 1.0, 64, 1024, xq.ctypes.data, 1024, xs.ctypes.data,
                     y.ctypes.data, 64, 3)
    f["r7_y"] = y
    # R10-R12 GDN: kh 1, vh 2, d 128, 3 rows from a random state, then commit 2 of them
    kh, vh, d, nr = 1, 2, 128, 3
    nqkv, nz = (2 * kh + vh) * d, vh * d
    g = dict(A_log=q27o.f2bf(rng.uniform(0, 2.7, vh).astype(np.float32)),
             dt_bias=q27o.f2bf((rng.standard_normal(vh) * 0.1).astype(np.float32)),
             norm_w=q27o.f2bf((1 + rng.standard_normal(d) * 0.02).astype(np.float32)),
             conv_w=q27o.f2bf((rng.standard_normal((nqkv, 4)) * 0.3).astype(np.float32)),
             S=(rng.standard_normal((vh, d, d)) * 0.1).astype(np.float32),
             hist=q27o.f2bf(rng.standard_normal((nqkv, 3)).astype(np.float32)),
             qkv=q27o.f2bf(rng.standard_normal((nr, nqkv)).astype(np.float32)),
             z=q27o.f2bf(rng.standard_normal((nr, nz)).astype(np.float32)),
             a=rng.uniform(-4, 0, (nr, vh)).astype(np.float32), b=rng.uniform(-4, 0, (nr, vh)).astype(np.float32))
    y64all, _, _ = ref64.gdn_rows(g["qkv"], g["z"], g["a"], g["b"], g["A_log"], g["dt_bias"], g["norm_w"],
                                  g["conv_w"], g["S"], g["hist"], kh, vh, d)
    S, hist = g["S"].copy(), g["hist"].copy()
    pend = np.zeros(L.q27o_gdn_pend_bytes(kh, vh, d, 8), np.uint8)
    out = np.empty((nr, nz), np.uint16)
    L.q27o_gdn_verify(g["qkv"].ctypes.data, nqkv, g["z"].ctypes.data, nz, g["a"].ctypes.data, g["b"].ctypes.data,
                      vh, g["A_log"].ctypes.data, g["dt_bias"].ctypes.data, g["norm_w"].ctypes.data,
                      g["conv_w"].ctypes.data, S.ctypes.data, hist.ctypes.data, pend.ctypes.data, 0, kh, vh, d, 1e-6,
                      out.ctypes.data, nz, None, None, nr)
    one = {k: g[k][:1].copy() for k in ("qkv", "z", "a", "b")}
    out2 = np.empty((1, nz), np.uint16)
    L.q27o_gdn_verify(one["qkv"].ctypes.data, nqkv, one["z"].ctypes.data, nz, one["a"].ctypes.data,
                      one["b"].ctypes.data, vh, g["A_log"].ctypes.data, g["dt_bias"].ctypes.data,
                      g["norm_w"].ctypes.data, g["conv_w"].ctypes.data, S.ctypes.data, hist.ctypes.data,
                      pend.ctypes.data, 2, kh, vh, d, 1e-6, out2.ctypes.data, nz, None, None, 1)
    for k, v in g.items():
        f["gdn_" + k] = v
    f.update(gdn_out=out, gdn_y64=y64all, gdn_S_commit2=S)
    return f


def tokens():
    cfg = q27o.Cfg(hidden=1024, inter=2048, vocab=4096, n_layers=4, attn_period=4, gdn_kh=2, gdn_vh=6, gdn_d=128,
                   n_q=4, n_kv=1, head_dim=128, attn_gate=1, rot_dims=32, rope_theta=1e7, kv_group=32,
                   rms_eps=1e-6, head_double_residual=1, mtp_swap=1, mtp_plus_one=1, spec_k=2, ctx=512)
    d = {f: getattr(cfg, f) for f, _ in q27o.Cfg._fields_}
    m = q27o.Model(d, 0x51E70003)
    prompt = np.random.default_rng(7).integers(0, 4096, 17).astype(np.int32)
    first = m.prefill(prompt)
    plain = [first] + [m.decode_step() for _ in range(23)]
    m.prefill(prompt)
    spec, rounds = [first], []
    while len(spec) < 24:
        got = m.spec_round()
        rounds.append(got)
        spec.extend(got)
    m.close()
    return {"config": d, "seed": 0x51E70003, "prompt": prompt.tolist(), "plain": plain, "spec_rounds": rounds}


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "kernels.npz"), **kernels())
    with open(os.path.join(HERE, "tiny_tokens.json"), "w") as fh:
        json.dump(tokens(), fh, indent=1)
    print("wrote", sorted(os.listdir(HERE)))
