"""Pins the oracle's MTP draft layer (oracle/q27o_model.c mtp_pass; reference mtp_pass_nr,
src/q27_main.cpp:2551-2618) without the reference: its composition against a float64 forward
written from the layer's definition (tests/ref64.py mtp_forward), with plausible composition
mistakes shown to fail the same comparison; its down projection against the exact chain of four
bf16-rounded K = inter/4 slices (src/q27_main.cpp:2605-2612), each slice computed by the pinned
kernel-tier projection; and the catch-up rows' KV overwrite."""
import numpy as np
import pytest

import ref64

SEED = 0x51E70003
WNAMES = ["pre_emb", "pre_hid", "mtp_norm", "fc0_w", "fc0_s", "fc1_w", "fc1_s", "in_norm", "post_norm",
          "qkv_w", "qkv_s", "q_norm", "k_norm", "o_w", "o_s", "gate_w", "gate_s", "up_w", "up_s",
          "down4_w0", "down4_s0", "down4_w1", "down4_s1", "down4_w2", "down4_s2", "down4_w3", "down4_s3"]


def weights(m, cfg):
    H, I = cfg.hidden, cfg.inter
    qrows = cfg.n_q * (2 if cfg.attn_gate else 1) * cfg.head_dim + 2 * cfg.n_kv * cfg.head_dim
    shapes = {"fc0_w": (H, H), "fc1_w": (H, H), "fc0_s": (H, H // 64), "fc1_s": (H, H // 64),
              "qkv_w": (qrows, H), "qkv_s": (qrows, H // 64),
              "o_w": (H, cfg.n_q * cfg.head_dim), "o_s": (H, cfg.n_q * cfg.head_dim // 64),
              "gate_w": (I, H), "gate_s": (I, H // 64), "up_w": (I, H), "up_s": (I, H // 64)}
    for j in range(4):
        shapes[f"down4_w{j}"] = (H, I // 4)
        shapes[f"down4_s{j}"] = (H, I // 256)
    W = {}
    for n in WNAMES:
        dt = np.int8 if n.endswith("_w") or n.startswith("down4_w") else (np.float32 if "_s" in n else np.uint16)
        a = m.tensor(n, -1, dt)
        W[n] = a.reshape(shapes[n]) if n in shapes else a
    W["emb"] = m.tensor("emb", -1, np.uint16)
    W["lm_head"] = m.tensor("lm_head", -1, np.uint16)
    return W


@pytest.fixture(scope="module")
def mtp_case(X, O):
    cfg = X.tiny_config(spec_k=2, n_layers=4)
    m = O.Model(cfg, SEED)
    W = weights(m, cfg)
    c = cfg.as_dict()
    rng = np.random.default_rng(0x51E7A002)
    H = cfg.hidden
    h = O.f2bf(rng.standard_normal((5, H)).astype(np.float32))
    toks = rng.integers(0, cfg.vocab, 5).astype(np.int32)
    # two calls: rows 0..2 at positions 0..2, then rows 3, 4 at positions 3, 4 attending to the cache
    t1, r1, l1 = m.mtp_pass(h[:3], toks[:3], 0, 2)
    t2, r2, l2 = m.mtp_pass(h[3:], toks[3:], 3, 1)
    yield dict(m=m, W=W, c=c, h=h, toks=toks, res=np.concatenate([r1, r2]), logits=(l1, l2), tok=(t1, t2))
    m.close()


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# measured: 0.7% for the oracle's pass (int8 activations, bf16 residual) against float64;
# the planted mistakes below are 9% (attention output dropped) to 5000% off
TOL_RES, TOL_LOGIT = 1.5e-2, 1.5e-2


def test_mtp_layer_matches_float64_forward(mtp_case, O):
    k = mtp_case
    res64, log64 = ref64.mtp_forward(k["W"], k["c"], k["h"], k["toks"], 0)
    res = O.bf2f(k["res"]).astype(np.float64)
    for r in range(5):
        assert rel(res[r], res64[r]) < TOL_RES, (r, rel(res[r], res64[r]))
    l1, l2 = k["logits"]
    assert rel(l1, log64[2]) < TOL_LOGIT, rel(l1, log64[2])
    assert rel(l2, log64[4]) < TOL_LOGIT, rel(l2, log64[4])
    # the drafted token is the float64 argmax unless the two best float64 logits are closer than
    # the comparison's own error
    for tok, lg in zip(k["tok"], (log64[2], log64[4])):
        top = np.argsort(lg)[::-1]
        assert tok == top[0] or (lg[top[0]] - lg[tok]) < TOL_LOGIT * np.abs(lg).max()


@pytest.mark.parametrize("mistake", ["swap_halves", "no_plus_one", "drop_o"])
def test_planted_composition_mistakes_fail(mtp_case, O, mistake):
    """The same comparison rejects a float64 forward with one composition mistake: the fc halves
    exchanged, the internal norms without +1, the attention output not added."""
    k = mtp_case
    kw = {"swap_halves": dict(swap_halves=True), "no_plus_one": dict(plus_one=0.0),
          "drop_o": dict(drop_o=True)}[mistake]
    res64, log64 = ref64.mtp_forward(k["W"], k["c"], k["h"], k["toks"], 0, **kw)
    res = O.bf2f(k["res"]).astype(np.float64)
    worst = max(rel(res[r], res64[r]) for r in range(5))
    assert worst > 5 * TOL_RES, (mistake, worst)


def test_down_is_four_bf16_rounded_slices(X, O):
    """The layer's residual after the MLP equals the exact chain
    res <- bf16(res + proj(slice j)), j = 0..3, of the kernel-tier projection (pinned on its own)
    over the four K = inter/4 slices -- not one K = inter projection with a single rounding."""
    cfg = X.tiny_config(spec_k=2, n_layers=4)
    m = O.Model(cfg, SEED)
    H, I = cfg.hidden, cfg.inter
    rng = np.random.default_rng(0x51E7A003)
    L = O.lib()
    res0 = O.f2bf(rng.standard_normal((2, H)).astype(np.float32))
    act = O.f2bf(rng.standard_normal((2, I)).astype(np.float32))
    xq, xs = np.empty((2, I), np.int8), np.empty((2, I // 16), np.float32)
    L.q27o_quant_rows(act.ctypes.data, I, xq.ctypes.data, I, xs.ctypes.data, I // 16, I, 1.0, 2)
    chain = res0.copy()
    I4 = I // 4
    for j in range(4):
        w = m.tensor(f"down4_w{j}", -1, np.int8).reshape(H, I4)
        s = m.tensor(f"down4_s{j}", -1, np.float32).reshape(H, I4 // 64)
        xqj = np.ascontiguousarray(xq[:, j * I4:(j + 1) * I4])
        xsj = np.ascontiguousarray(xs[:, j * I4 // 16:(j + 1) * I4 // 16])
        out = np.empty((2, H), np.uint16)
        L.q27o_proj_rows_epi(w.ctypes.data, s.ctypes.data, 1.0, H, I4, xqj.ctypes.data, I4, xsj.ctypes.data,
                             out.ctypes.data, H, 1, chain.ctypes.data, 1, H, 1.0, 2)
        chain = out
    # one projection over the whole K with one rounding differs in some bits
    wall = np.concatenate([m.tensor(f"down4_w{j}", -1, np.int8).reshape(H, I4) for j in range(4)], axis=1)
    sall = np.concatenate([m.tensor(f"down4_s{j}", -1, np.float32).reshape(H, I4 // 64) for j in range(4)], axis=1)
    one = np.empty((2, H), np.uint16)
    L.q27o_proj_rows_epi(np.ascontiguousarray(wall).ctypes.data, np.ascontiguousarray(sall).ctypes.data, 1.0, H, I,
                         xq.ctypes.data, I, xs.ctypes.data, one.ctypes.data, H, 1, res0.ctypes.data, 1, H, 1.0, 2)
    assert not np.array_equal(one, chain)
    # and the float64 sum agrees with the chain to bf16 accuracy
    f64 = O.bf2f(res0).astype(np.float64) + ref64.proj(wall, sall, xq, xs, 1.0)
    assert rel(O.bf2f(chain), f64) < 1e-2
    m.close()


def test_catch_up_rows_overwrite_draft_kv(X, O):
    """A catch-up pass over draft positions that an earlier draft already wrote replaces their K/V
    (src/q27_main.cpp:2942-2950: the next round's draft 0 re-runs the accepted rows): the cache
    after (draft at p, then catch-up at p) equals the cache of the catch-up alone."""
    cfg = X.tiny_config(spec_k=2, n_layers=4)
    a, b = O.Model(cfg, SEED), O.Model(cfg, SEED)
    H = cfg.hidden
    rng = np.random.default_rng(0x51E7A005)
    h = O.f2bf(rng.standard_normal((3, H)).astype(np.float32))
    t = rng.integers(0, cfg.vocab, 3).astype(np.int32)
    a.mtp_pass(h[:1], t[:1], 0, 0)                   # position 0
    a.mtp_pass(h[1:2], t[1:2], 1, 0)                 # a draft at position 1
    a.mtp_pass(h[2:3], t[2:3], 1, 0)                 # catch-up row at position 1 replaces it
    b.mtp_pass(h[:1], t[:1], 0, 0)
    b.mtp_pass(h[2:3], t[2:3], 1, 0)
    for n in ("kc", "ks", "vc", "vs"):
        assert np.array_equal(a.tensor(n, -1, np.uint8), b.tensor(n, -1, np.uint8)), n
    a.close()
    b.close()
