"""Whole-path parity: the chained-MTP round on the GPU against the CPU oracle (tiny geometry,
identical tokens and identical final-residual bits), the reference's invariant "the spec run's
token stream must be IDENTICAL to plain greedy" (src/q27_main.cpp:2181-2182), forced acceptance,
and the full 27B geometry's self-consistency on one MI355X."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 0x51E70003


def tiny(X, **kw):
    return X.tiny_config(**kw)


@pytest.fixture(scope="module")
def tiny_pair(gpu, O):
    X = gpu
    cfg = tiny(X, spec_k=2)
    eng = X.Engine(cfg, SEED)
    om = O.Model(cfg, SEED)
    yield X, cfg, eng, om
    eng.close()
    om.close()


def prompt_of(cfg, n, seed=7):
    return np.random.default_rng(seed).integers(0, cfg.vocab, n).astype(np.int32)


def test_tiny_prefill_and_plain_greedy(tiny_pair):
    X, cfg, eng, om = tiny_pair
    p = prompt_of(cfg, 37)
    t_g, t_o = eng.prefill(p), om.prefill(p)
    assert t_g == t_o
    hg = eng.read("hprev", -1, np.uint16, cfg.hidden)
    ho = om.tensor("hprev", -1, np.uint16)
    assert np.array_equal(hg, ho), "final residual of the last prompt position differs"
    S_g = eng.read("S", 0, np.float32, cfg.gdn_vh * 128 * 128)
    S_o = om.tensor("S", 0, np.float32)
    assert np.array_equal(S_g.view(np.uint32), S_o.view(np.uint32)), "committed GDN state differs"
    g, o = [t_g], [t_o]
    for _ in range(20):
        g.append(eng.decode_step())
        o.append(om.decode_step())
    assert g == o


def test_tiny_spec_rounds_match_oracle(tiny_pair):
    X, cfg, eng, om = tiny_pair
    p = prompt_of(cfg, 29, seed=9)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(12):
        a = eng.spec_round()
        b = om.spec_round()
        assert a == b, f"round {r}: gpu {a} oracle {b}"


def test_tiny_k7_rounds_match_oracle(gpu, O):
    # the widest chain (K = 7: 8 verify rows through every layer, the 8-row projection and
    # attention forms), round by round against the oracle
    X = gpu
    cfg = tiny(X, spec_k=7)
    eng = X.Engine(cfg, SEED)
    om = O.Model(cfg, SEED)
    p = prompt_of(cfg, 33, seed=11)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(10):
        a = eng.spec_round()
        b = om.spec_round()
        assert a == b, f"round {r}: gpu {a} oracle {b}"
    eng.close()
    om.close()


@pytest.mark.parametrize("inter", [5120, 6144])
def test_tiny_split_swiglu_units_match_oracle(gpu, O, inter):
    """gate|up with more 32-row SwiGLU units than blocks (one block per CU): 320 units leave 64
    units split into quarters over the blocks (one quarter per block), 384 units leave 128 (two
    quarters on every block); the split units' codes must be the bits of the oracle's."""
    X = gpu
    cfg = tiny(X, spec_k=2, inter=inter)
    eng = X.Engine(cfg, SEED)
    om = O.Model(cfg, SEED)
    p = prompt_of(cfg, 19, seed=inter)
    assert eng.prefill(p) == om.prefill(p)
    hg = eng.read("hprev", -1, np.uint16, cfg.hidden)
    assert np.array_equal(hg, om.tensor("hprev", -1, np.uint16))
    for r in range(6):
        a, b = eng.spec_round(), om.spec_round()
        assert a == b, f"inter {inter} round {r}: gpu {a} oracle {b}"
    eng.close()
    om.close()


def test_tiny_rounds_across_a_key_split_match_oracle(tiny_pair):
    """Verify rows whose positions straddle a 64-key attention split (e.g. 62, 63 | 64): the split
    that holds the new positions computes their K/V itself, and the next split sees them in the
    cache; tokens and the final residual bits must be the oracle's."""
    X, cfg, eng, om = tiny_pair
    p = prompt_of(cfg, 60, seed=11)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(8):
        a, b = eng.spec_round(), om.spec_round()
        assert a == b, f"round {r}: gpu {a} oracle {b}"
    hg = eng.read("hprev", -1, np.uint16, cfg.hidden)
    assert np.array_equal(hg, om.tensor("hprev", -1, np.uint16))


def test_tiny_spec_equals_plain_and_forced(gpu, O):
    X = gpu
    for k in (1, 2, 3, 7):
        cfg = tiny(X, spec_k=k)
        eng = X.Engine(cfg, SEED)
        p = prompt_of(cfg, 21, seed=k)
        first = eng.prefill(p)
        plain, st0 = eng.generate(48, spec=False)
        assert plain[0] == first
        eng.prefill(p)
        spec, st = eng.generate(48, spec=True)
        assert spec == plain, f"K={k}: spec stream differs from plain greedy"
        assert st.rounds >= 1
        # forced acceptance: drafts = the trunk's own greedy continuation -> K+1 per round
        eng.prefill(p)
        eng.set_forced(np.array(plain, np.int32))
        forced, stf = eng.generate(48, spec=True)
        assert forced == plain
        full = stf.acc_hist[k]
        assert full >= stf.rounds - 1, (k, stf.rounds, list(stf.acc_hist))
        eng.set_forced([])
        eng.close()


def test_full_geometry_spec_equals_plain(gpu):
    """BASELINE config 3 geometry (64 layers, 48 GDN + 16 attention, hidden 5120): spec(K=2)
    committed stream == plain greedy; forced acceptance commits 3 tokens per round."""
    X = gpu
    cfg = X.default_config(spec_k=2, ctx=512)
    eng = X.Engine(cfg, SEED)
    assert eng.weight_bytes() > 25e9
    p = prompt_of(cfg, 64, seed=3)
    eng.prefill(p)
    plain, _ = eng.generate(32, spec=False)
    eng.prefill(p)
    spec, st = eng.generate(32, spec=True)
    assert spec == plain
    eng.prefill(p)
    eng.set_forced(np.array(plain, np.int32))
    forced, stf = eng.generate(32, spec=True)
    assert forced == plain
    assert stf.acc_hist[2] >= stf.rounds - 1
    eng.close()
