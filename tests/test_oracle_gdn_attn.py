"""Pins the oracle's gated-delta-rule verify (R10-R12, src/q27_gdn.hip:206-372, 411-592) and its
attention prep / causal GQA attention (R14-R15, src/q27_attn.hip:156-463) against float64 textbook
forms, invariants and special cases:
  GDN: the single-pass state/output identity against the two-pass update-then-read form; the
       deferred-commit rollback equals running the accepted prefix from scratch (bitwise); with
       orthonormal keys, unit gate and beta, and zero state it is a linear-attention prefix sum.
  attention: float64 softmax over the dequantized cache; causality (later keys cannot move row
       r); RoPE depends only on relative position."""
import numpy as np
import pytest

import ref64


def gdn_call(O, inp, S, hist, pend, npend, params, kh, vh, d):
    nr = inp["qkv"].shape[0]
    nqkv, nz = (2 * kh + vh) * d, vh * d
    out = np.empty((nr, nz), np.uint16)
    xq, xs = np.empty((nr, nz), np.int8), np.empty((nr, nz // 16), np.float32)
    O.lib().q27o_gdn_verify(inp["qkv"].ctypes.data, nqkv, inp["z"].ctypes.data, nz, inp["a"].ctypes.data,
                            inp["b"].ctypes.data, vh, params["A_log"].ctypes.data, params["dt_bias"].ctypes.data,
                            params["norm_w"].ctypes.data, params["conv_w"].ctypes.data, S.ctypes.data,
                            hist.ctypes.data, pend.ctypes.data, npend, kh, vh, d, 1e-6, out.ctypes.data, nz,
                            xq.ctypes.data, xs.ctypes.data, nr)
    return out, xq, xs


def gdn_setup(O, rng, kh, vh, d):
    nqkv = (2 * kh + vh) * d
    params = dict(
        A_log=O.f2bf(rng.uniform(0, 2.7, vh).astype(np.float32)),
        dt_bias=O.f2bf((rng.standard_normal(vh) * 0.1).astype(np.float32)),
        norm_w=O.f2bf((1 + rng.standard_normal(d) * 0.02).astype(np.float32)),
        conv_w=O.f2bf((rng.standard_normal((nqkv, 4)) * 0.3).astype(np.float32)))
    S = (rng.standard_normal((vh, d, d)) * 0.1).astype(np.float32)
    hist = O.f2bf(rng.standard_normal((nqkv, 3)).astype(np.float32))
    pend = np.zeros(O.lib().q27o_gdn_pend_bytes(kh, vh, d, 8), np.uint8)
    return params, S, hist, pend


def gdn_rows(O, rng, nr, kh, vh, d):
    nqkv = (2 * kh + vh) * d
    return dict(qkv=O.f2bf(rng.standard_normal((nr, nqkv)).astype(np.float32)),
                z=O.f2bf(rng.standard_normal((nr, vh * d)).astype(np.float32)),
                a=rng.uniform(-4, 0, (nr, vh)).astype(np.float32),
                b=rng.uniform(-4, 0, (nr, vh)).astype(np.float32))


def test_gdn_against_two_pass_float64(O):
    kh, vh, d, nr = 2, 6, 128, 3
    rng = np.random.default_rng(20)
    params, S, hist, pend = gdn_setup(O, rng, kh, vh, d)
    inp = gdn_rows(O, rng, nr, kh, vh, d)
    y64, S64, _ = ref64.gdn_rows(inp["qkv"], inp["z"], inp["a"], inp["b"], params["A_log"], params["dt_bias"],
                                 params["norm_w"], params["conv_w"], S, hist, kh, vh, d)
    S0 = S.copy()
    out, xq, xs = gdn_call(O, inp, S, hist, pend, 0, params, kh, vh, d)
    got = ref64.bf2f(out).astype(np.float64)
    assert (np.abs(got - y64) <= np.abs(y64) * 2.0 ** -7 + 2e-3 * np.abs(y64).max()).all()
    rel = np.linalg.norm(got - y64) / np.linalg.norm(y64)
    assert rel < 4e-3, rel
    assert np.array_equal(S, S0)                 # nothing committed yet: rows are pending
    # commit all 3 rows: the committed state equals the float64 state after the 3 rows
    nxt = gdn_rows(O, rng, 1, kh, vh, d)
    gdn_call(O, nxt, S, hist, pend, 3, params, kh, vh, d)
    assert np.abs(S - S64).max() <= 1e-5 * np.abs(S64).max()
    # the quantized output is the per-16 quantization of the bf16 output
    ref64.assert_codes_match_ideal(xq, ref64.bf2f(out), 16, tie_tol=1e-3)


@pytest.mark.parametrize("accepted", [0, 1, 2, 3])
def test_gdn_rollback_equals_prefix_rerun(O, accepted):
    """Verify 3 rows, accept a prefix, then one more row: the committed state and conv history
    equal (bit for bit) running only the accepted rows, one call each, from the same start."""
    kh, vh, d = 1, 3, 128
    rng = np.random.default_rng(30 + accepted)
    params, S, hist, pend = gdn_setup(O, rng, kh, vh, d)
    rows = gdn_rows(O, rng, 3, kh, vh, d)
    nxt = gdn_rows(O, rng, 1, kh, vh, d)
    Sa, ha, pa = S.copy(), hist.copy(), pend.copy()
    gdn_call(O, rows, Sa, ha, pa, 0, params, kh, vh, d)
    out_a, _, _ = gdn_call(O, nxt, Sa, ha, pa, accepted, params, kh, vh, d)
    Sb, hb, pb = S.copy(), hist.copy(), pend.copy()
    npend = 0
    for i in range(accepted):
        one = {k: v[i:i + 1].copy() for k, v in rows.items()}
        gdn_call(O, one, Sb, hb, pb, npend, params, kh, vh, d)
        npend = 1
    out_b, _, _ = gdn_call(O, nxt, Sb, hb, pb, npend, params, kh, vh, d)
    assert np.array_equal(Sa.view(np.uint32), Sb.view(np.uint32))
    assert np.array_equal(ha, hb)
    assert np.array_equal(out_a, out_b)


def test_gdn_linear_attention_special_case(O):
    """decay = 1 (A_log = -inf), beta = 1 (b = +inf), S = 0, conv = identity tap, keys with
    disjoint supports (orthonormal after L2 norm): delta_t = v_t and the output is the linear
    attention prefix sum o_t = sum_{i<=t} (k_i . q_t) v_i, then the gated RMS norm."""
    kh, vh, d, nr = 1, 1, 128, 3
    nqkv = (2 * kh + vh) * d
    rng = np.random.default_rng(40)
    params = dict(A_log=O.f2bf(np.array([-np.inf], np.float32)), dt_bias=O.f2bf(np.zeros(1, np.float32)),
                  norm_w=O.f2bf(np.ones(d, np.float32)),
                  conv_w=O.f2bf(np.tile(np.array([0, 0, 0, 1], np.float32), (nqkv, 1))))
    S = np.zeros((vh, d, d), np.float32)
    hist = np.zeros((nqkv, 3), np.uint16)
    pend = np.zeros(O.lib().q27o_gdn_pend_bytes(kh, vh, d, 8), np.uint8)
    raw = np.zeros((nr, nqkv), np.float32)
    for t in range(nr):
        raw[t, :d] = rng.uniform(1, 3, d)                             # q
        raw[t, d + 32 * t: d + 32 * t + 32] = rng.uniform(1, 3, 32)   # k, disjoint support per row
        raw[t, 2 * d:] = rng.standard_normal(d)                       # v
    inp = dict(qkv=O.f2bf(raw), z=O.f2bf(np.full((nr, d), 30.0, np.float32)),   # silu(30) = 30
               a=np.zeros((nr, 1), np.float32), b=np.full((nr, 1), np.inf, np.float32))
    out, _, _ = gdn_call(O, inp, S, hist, pend, 0, params, kh, vh, d)
    cv = ref64.bf2f(O.f2bf(ref64.silu(ref64.bf2f(inp["qkv"])).astype(np.float32))).astype(np.float64)
    q = cv[:, :d] / np.linalg.norm(cv[:, :d], axis=1, keepdims=True) / np.sqrt(d)
    k = cv[:, d:2 * d]
    k = k / np.linalg.norm(k, axis=1, keepdims=True)
    v = cv[:, 2 * d:]
    for t in range(nr):
        o = sum((k[i] @ q[t]) * v[i] for i in range(t + 1))
        y = o / np.sqrt((o * o).mean() + 1e-6) * 30.0
        got = ref64.bf2f(out[t]).astype(np.float64)
        assert np.abs(got - y).max() <= 2.0 ** -7 * np.abs(y).max(), t


def attn_setup(O, rng, L0, nq, nkv, hd, rot, group, nr, gate=1):
    ctx = L0 + nr + 8
    kv = nkv * hd
    qw = 2 * hd if gate else hd
    qkv_rows = nq * qw + 2 * kv
    kc, vc = np.zeros((ctx, kv), np.int8), np.zeros((ctx, kv), np.int8)
    ks, vs = np.zeros((ctx, kv // group), np.float32), np.zeros((ctx, kv // group), np.float32)
    for arr, c, s in ((rng.standard_normal((L0, kv)).astype(np.float32), kc, ks),
                      (rng.standard_normal((L0, kv)).astype(np.float32), vc, vs)):
        q = np.empty(L0 * kv, np.int8)
        sc = np.empty(L0 * kv // group, np.float32)
        O.lib().q27o_quant_f32(arr.ctypes.data, L0 * kv, group, q.ctypes.data, sc.ctypes.data)
        c[:L0], s[:L0] = q.reshape(L0, kv), sc.reshape(L0, kv // group)
    qkv = O.f2bf(rng.standard_normal((nr, qkv_rows)).astype(np.float32))
    qn = O.f2bf((rng.standard_normal(hd) * 0.1).astype(np.float32))
    kn = O.f2bf((rng.standard_normal(hd) * 0.1).astype(np.float32))
    cs, sn = np.empty(ctx * rot // 2, np.float32), np.empty(ctx * rot // 2, np.float32)
    O.lib().q27o_rope_table(ctx, rot, 1e7, cs.ctypes.data, sn.ctypes.data)
    return dict(kc=kc, ks=ks, vc=vc, vs=vs, qkv=qkv, qn=qn, kn=kn, cs=cs, sn=sn, qkv_rows=qkv_rows, qw=qw)


def prep(O, A, rot, group, nq, nkv, hd, gate, L0, nr):
    qh = np.empty((nr, nq * hd), np.uint16)
    O.lib().q27o_attn_prep_rows(A["qkv"].ctypes.data, A["qkv_rows"], A["qn"].ctypes.data, A["kn"].ctypes.data,
                                A["cs"].ctypes.data, A["sn"].ctypes.data, rot, A["kc"].ctypes.data,
                                A["ks"].ctypes.data, A["vc"].ctypes.data, A["vs"].ctypes.data, group,
                                qh.ctypes.data, nq, nkv, hd, gate, 1e-6, L0, nr)
    return qh


def attend(O, A, qh, group, nq, nkv, hd, gate, L0, nr):
    out = np.empty((nr, nq * hd), np.uint16)
    O.lib().q27o_attn_rows(qh.ctypes.data, A["qkv"].ctypes.data, A["qkv_rows"], A["kc"].ctypes.data,
                           A["ks"].ctypes.data, A["vc"].ctypes.data, A["vs"].ctypes.data, group, nq, nkv, hd, gate,
                           L0, nr, out.ctypes.data, None, None)
    return out


# (nq, nkv, hd, rot): the benchmark attention's shape, and the reference trunk's (24q/4kv x 256 with 64
# rotary dims, include/q27.h:25-35, src/q27_attn.hip:10-11) at one kv head with its GQA group of 6
GEOMS = [(4, 2, 128, 32), (6, 1, 256, 64), (12, 2, 256, 64)]


@pytest.mark.parametrize("nq,nkv,hd,rot", GEOMS)
def test_attn_prep_against_float64(O, nq, nkv, hd, rot):
    group, nr, L0 = 32, 3, 100
    rng = np.random.default_rng(50 + hd + nq)
    A = attn_setup(O, rng, L0, nq, nkv, hd, rot, group, nr)
    qh = prep(O, A, rot, group, nq, nkv, hd, 1, L0, nr)
    raw = ref64.bf2f(A["qkv"]).astype(np.float64)
    for r in range(nr):
        for h in range(nq):
            x = raw[r, h * A["qw"]: h * A["qw"] + hd]
            y = ref64.rope_rotate(ref64.rmsnorm(x, ref64.bf2f(A["qn"]), 1.0, 1e-6), L0 + r, rot, 1e7)
            got = ref64.bf2f(qh[r, h * hd:(h + 1) * hd]).astype(np.float64)
            assert np.abs(got - y).max() <= 2.0 ** -8 * np.abs(y).max() + 1e-6
        for h in range(nkv):
            kx = raw[r, nq * A["qw"] + h * hd: nq * A["qw"] + (h + 1) * hd]
            ky = ref64.rope_rotate(ref64.rmsnorm(kx, ref64.bf2f(A["kn"]), 1.0, 1e-6), L0 + r, rot, 1e7)
            ref64.assert_codes_match_ideal(A["kc"][L0 + r, h * hd:(h + 1) * hd], ky, group, tie_tol=1e-3)
            vx = raw[r, nq * A["qw"] + nkv * hd + h * hd: nq * A["qw"] + nkv * hd + (h + 1) * hd]
            ref64.assert_codes_match_ideal(A["vc"][L0 + r, h * hd:(h + 1) * hd], vx, group, tie_tol=1e-3)
            np.testing.assert_allclose(A["vs"][L0 + r, h * hd // group:(h + 1) * hd // group],
                                       np.abs(vx.reshape(-1, group)).max(axis=1) / 127, rtol=2e-7)


def test_rope_relative_position(O):
    """<rot(q, p), rot(k, p')> depends only on p - p' (float tables at theta 1e7)."""
    ctx, rot = 4096, 32
    cs, sn = np.empty(ctx * rot // 2, np.float32), np.empty(ctx * rot // 2, np.float32)
    O.lib().q27o_rope_table(ctx, rot, 1e7, cs.ctypes.data, sn.ctypes.data)
    cs, sn = cs.reshape(ctx, -1).astype(np.float64), sn.reshape(ctx, -1).astype(np.float64)
    rng = np.random.default_rng(51)
    q, k = rng.standard_normal(rot), rng.standard_normal(rot)
    h = rot // 2

    def rotate(x, p):
        return np.concatenate([x[:h] * cs[p] - x[h:] * sn[p], x[h:] * cs[p] + x[:h] * sn[p]])
    for p, pk, shift in ((10, 3, 1000), (500, 499, 3000), (7, 7, 4000)):
        a = rotate(q, p) @ rotate(k, pk)
        b = rotate(q, p + shift - 1) @ rotate(k, pk + shift - 1)
        assert abs(a - b) <= 2e-4 * (np.abs(q).sum() * np.abs(k).max())
    assert np.allclose(cs[0], 1) and np.allclose(sn[0], 0)
    # the first frequency pair rotates by exactly the position (inv_freq = 1)
    np.testing.assert_allclose(np.arctan2(sn[1:50, 0], cs[1:50, 0]), np.angle(np.exp(1j * np.arange(1, 50))), atol=1e-6)


@pytest.mark.parametrize("L0,nq,nkv,hd,rot", [(5, 8, 2, 128, 32), (63, 8, 2, 128, 32), (64, 8, 2, 128, 32),
                                               (200, 8, 2, 128, 32), (63, 6, 1, 256, 64), (200, 12, 2, 256, 64)])
def test_attention_against_float64(O, L0, nq, nkv, hd, rot):
    group, nr = 32, 3
    rng = np.random.default_rng(60 + L0 + hd)
    A = attn_setup(O, rng, L0, nq, nkv, hd, rot, group, nr)
    qh = prep(O, A, rot, group, nq, nkv, hd, 1, L0, nr)
    out = attend(O, A, qh, group, nq, nkv, hd, 1, L0, nr)
    Kd = A["kc"].astype(np.float64) * np.repeat(A["ks"].astype(np.float64), group, axis=1)
    Vd = A["vc"].astype(np.float64) * np.repeat(A["vs"].astype(np.float64), group, axis=1)
    gates = np.stack([np.concatenate([ref64.bf2f(A["qkv"][r, h * A["qw"] + hd: (h + 1) * A["qw"]])
                                      for h in range(nq)]) for r in range(nr)])
    ref = ref64.attention_rows(ref64.bf2f(qh), gates, Kd, Vd, nq, nkv, hd, L0, nr)
    got = ref64.bf2f(out).astype(np.float64)
    assert (np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-5 * np.abs(ref).max()).all()


def test_attention_causality(O):
    """Row r reads keys 0..L0+r only: rewriting the cache rows after L0+r leaves row r's output
    bit for bit unchanged and changes the later rows."""
    nq, nkv, hd, rot, group, nr, L0 = 4, 1, 128, 32, 32, 3, 70
    rng = np.random.default_rng(70)
    A = attn_setup(O, rng, L0, nq, nkv, hd, rot, group, nr, gate=0)
    qh = prep(O, A, rot, group, nq, nkv, hd, 0, L0, nr)
    base = attend(O, A, qh, group, nq, nkv, hd, 0, L0, nr)
    A["kc"][L0 + 1:] = rng.integers(-127, 128, A["kc"][L0 + 1:].shape)
    A["vc"][L0 + 1:] = rng.integers(-127, 128, A["vc"][L0 + 1:].shape)
    pert = attend(O, A, qh, group, nq, nkv, hd, 0, L0, nr)
    assert np.array_equal(base[0], pert[0])
    assert not np.array_equal(base[1], pert[1]) and not np.array_equal(base[2], pert[2])
