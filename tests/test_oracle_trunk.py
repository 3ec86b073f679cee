"""Pins the oracle's trunk composition (oracle/q27o_model.c verify(); reference run_layer_tp_nr,
src/q27_main.cpp:2271-2489, and its head 2457-2481) without the reference, against float64 forwards
of the layer stack written from its definition (tests/ref64.py trunk_forward):
  * the ideal forward (no rounding, no quantization) within the quantization error, with gross
    composition mistakes (a residual dropped, the head's double count missing, the GDN output gate
    applied before its norm, the attention gate dropped) shown to fail the same comparison;
  * the storage-faithful forward (bf16 and int8 exactly where the reference stores them, sums in
    float64) within the float32-summation error, with a storage-point mistake (the post norm
    reading bf16(r1) instead of the fp32 r1) shown to fail it.
Two GDN and two attention layers (attention period 2), eight rows over two verify calls (the second
commits the first's pending GDN rows and reads the first's KV)."""
import numpy as np
import pytest

import ref64

SEED = 0x51E70003


def trunk_weights(m, c):
    """The oracle's weights, per layer and global, as ref64.trunk_forward takes them."""
    H, I = c["hidden"], c["inter"]

    def layer(L):
        def t(name, dt, shape=None):
            a = m.tensor(name, L, dt)
            return a.reshape(shape) if shape else a
        d = {"in_norm": t("in_norm", np.uint16), "post_norm": t("post_norm", np.uint16),
             "gate_w": t("gate_w", np.int8, (I, H)), "gate_s": t("gate_s", np.float32, (I, H // 64)),
             "up_w": t("up_w", np.int8, (I, H)), "up_s": t("up_s", np.float32, (I, H // 64)),
             "down_w": t("down_w", np.int8, (H, I)), "down_s": t("down_s", np.float32, (H, I // 64))}
        if (L % c["attn_period"]) == c["attn_period"] - 1:
            w = t("qkv_w", np.int8)
            d["qkv_w"] = w.reshape(-1, H)
            d["qkv_s"] = t("qkv_s", np.float32, (d["qkv_w"].shape[0], H // 64))
            d["q_norm"], d["k_norm"] = t("q_norm", np.uint16), t("k_norm", np.uint16)
            att = c["n_q"] * c["head_dim"]
            d["o_w"], d["o_s"] = t("o_w", np.int8, (H, att)), t("o_s", np.float32, (H, att // 64))
        else:
            w = t("qkvz_w", np.int8)
            d["qkvz_w"] = w.reshape(-1, H)
            d["qkvz_s"] = t("qkvz_s", np.float32, (d["qkvz_w"].shape[0], H // 64))
            nz = c["gdn_vh"] * c["gdn_d"]
            d["out_w"], d["out_s"] = t("out_w", np.int8, (H, nz)), t("out_s", np.float32, (H, nz // 64))
            for n in ("in_a", "in_b", "A_log", "dt_bias", "gdn_norm", "conv_w"):
                d[n] = t(n, np.uint16)
        return d

    return {"layers": [layer(L) for L in range(c["n_layers"])], "emb": m.tensor("emb", -1, np.uint16),
            "final_norm": m.tensor("final_norm", -1, np.uint16), "lm_head": m.tensor("lm_head", -1, np.uint16)}


@pytest.fixture(scope="module")
def case(X, O):
    cfg = X.tiny_config(spec_k=2, n_layers=4, attn_period=2)    # GDN, attention, GDN, attention
    c = cfg.as_dict()
    m = O.Model(cfg, SEED)
    W = trunk_weights(m, c)
    toks = np.random.default_rng(0x51E7A010).integers(0, c["vocab"], 8).astype(np.int32)
    t1 = m.verify_trace(toks[:5])          # positions 0..4
    t2 = m.verify_trace(toks[5:])          # positions 5..7: commits the pending GDN rows, reads the KV
    cat = lambda k: np.concatenate([t1[k], t2[k]], axis=1 if t1[k].ndim == 3 else 0)
    tr = {k: cat(k) for k in ("r1", "r2", "pq", "ps", "logits")}
    tr["hfinal"] = O.bf2f(np.concatenate([t1["hfinal"], t2["hfinal"]])).astype(np.float64)
    tr["nx"] = t1["nx"] + t2["nx"]
    nl = c["n_layers"]
    force = {("head", "r2"): tr["r2"][nl - 1]}
    for L in range(nl):
        force[(L, "r1")] = tr["r1"][L]
        if L:
            force[(L, "x")] = tr["r2"][L - 1]
    yield dict(m=m, W=W, c=c, toks=toks, tr=tr, force=force)
    m.close()


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# Ideal forward: measured 0.67% (final residual) and 0.69% (logits) for the oracle's quantized
# path; the gross mistakes below measure 5.4% (gate before the GDN norm) to 465%.
TOL_IDEAL = 1.2e-2
# Faithful forward, each stage from the oracle's own inputs: measured r1 / r2 within 2e-5 (a rare
# bf16 flip of one mixer value), 0 differing post-norm codes, 0 differing final-residual bits,
# logits within 7e-8. A single int8 code flip of a projection input moves r1 by ~4e-4.
TOL_STAGE = 1e-3
MAX_CODE_FLIPS = 8          # of 8 x 1024 post-norm codes per layer
MAX_HFIN_FLIPS = 8          # of 8 x 1024 final-residual bf16 values
TOL_LOGITS = 1e-5


def ideal_errors(k, plant=None):
    hf, lg = ref64.trunk_forward(k["W"], k["c"], k["toks"], faithful=False, plant=plant)
    n = len(k["toks"])
    return (max(rel(k["tr"]["hfinal"][r], hf[r]) for r in range(n)),
            max(rel(k["tr"]["logits"][r], lg[r]) for r in range(n)), lg)


def stage_errors(k, plant=None):
    """Per stage, faithful forward under teacher forcing against the oracle's trace: the worst
    r1 and r2 relative errors over the layers, the most post-norm codes that differ in a layer,
    the final-residual values that differ, the logits' relative error."""
    tr, nl = k["tr"], k["c"]["n_layers"]
    t = {}
    hf, lg = ref64.trunk_forward(k["W"], k["c"], k["toks"], faithful=True, plant=plant, trace=t, force=k["force"])
    return dict(r1=max(rel(t[(L, "r1")], tr["r1"][L]) for L in range(nl)),
                r2=max(rel(t[(L, "r2")], tr["r2"][L]) for L in range(nl)),
                codes=max(int((t[(L, "a2")] != tr["pq"][L]).sum()) for L in range(nl)),
                hfin=int((hf != tr["hfinal"]).sum()),
                logits=rel(lg, tr["logits"]))


def test_trunk_matches_ideal_float64(case):
    eh, el, lg = ideal_errors(case)
    assert eh < TOL_IDEAL and el < TOL_IDEAL, (eh, el)
    # each row's greedy token is the float64 argmax unless the two best float64 logits are closer
    # than the comparison's own error
    for r, tok in enumerate(case["tr"]["nx"]):
        top = np.argsort(lg[r])[::-1]
        assert tok == top[0] or (lg[r][top[0]] - lg[r][tok]) < TOL_IDEAL * np.abs(lg[r]).max(), r


@pytest.mark.parametrize("plant", ["drop_out_residual", "single_head_residual", "zgate_before_norm",
                                   "attn_gate_dropped"])
def test_ideal_comparison_rejects_composition_mistakes(case, plant):
    eh, el, _ = ideal_errors(case, plant)
    assert max(eh, el) > 4 * TOL_IDEAL, (plant, eh, el)


def test_trunk_stages_match_faithful_float64(case):
    e = stage_errors(case)
    assert e["r1"] < TOL_STAGE and e["r2"] < TOL_STAGE, e
    assert e["codes"] <= MAX_CODE_FLIPS and e["hfin"] <= MAX_HFIN_FLIPS, e
    assert e["logits"] < TOL_LOGITS, e


@pytest.mark.parametrize("plant", ["drop_out_residual", "single_head_residual", "post_norm_bf16",
                                   "zgate_before_norm", "attn_gate_dropped"])
def test_faithful_stages_reject_mistakes(case, plant):
    """Every planted mistake, the storage-point one (post norm from bf16(r1)) included, misses at
    least one stage bound by a factor of five or more."""
    e = stage_errors(case, plant)
    worst = max(e["r1"] / TOL_STAGE, e["r2"] / TOL_STAGE, e["codes"] / MAX_CODE_FLIPS,
                e["hfin"] / MAX_HFIN_FLIPS, e["logits"] / TOL_LOGITS)
    assert worst > 5, (plant, e)
