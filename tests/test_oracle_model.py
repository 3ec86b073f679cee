"""Pins the oracle's whole-round semantics (oracle/q27o_model.c) by the reference's own
invariants, on the tiny geometry (hidden 1024, 8 layers with attention every 4th, vocab 4096):
  - "the spec run's token stream must be IDENTICAL to plain greedy" (src/q27_main.cpp:2181-2182),
    for K = 1, 2, 3 and 7 (Q27_SPEC_K's range, src/q27_main.cpp:3361);
  - forced acceptance (drafts = the trunk's own greedy continuation) commits K+1 per round;
  - an NR-row verify computes each row exactly as the single-row step does
    (src/q27_main.cpp:2172-2182): same tokens, same final residual bits;
  - argmax ties go to the lowest index, non-finite values are skipped (src/q27_elem.hip:216-322);
  - acceptance is the longest matching draft prefix (src/q27_main.cpp:2811-2812, 2929-2932);
  - runs are deterministic in the seed."""
import numpy as np
import pytest

SEED = 0x51E70003


def tiny(X, **kw):
    return X.tiny_config(**kw)


def prompt(cfg, n, seed):
    return np.random.default_rng(seed).integers(0, cfg.vocab, n).astype(np.int32)


def spec_stream(m, first, n):
    out = [first]
    hist = []
    while len(out) < n:
        got = m.spec_round()
        hist.append(len(got))
        out.extend(got)
    return out[:n], hist


def plain_stream(m, first, n):
    out = [first]
    while len(out) < n:
        out.append(m.decode_step())
    return out


@pytest.fixture(scope="module")
def cfgs(X):
    return {k: tiny(X, spec_k=k, n_layers=4) for k in (1, 2, 3, 7)}


@pytest.mark.parametrize("k", [1, 2, 3, 7])
def test_spec_equals_plain_greedy(O, cfgs, k):
    cfg = cfgs[k]
    m = O.Model(cfg, SEED)
    p = prompt(cfg, 13, seed=k)
    first = m.prefill(p)
    plain = plain_stream(m, first, 24)
    assert m.prefill(p) == first
    spec, hist = spec_stream(m, first, 24)
    assert spec == plain
    assert all(1 <= h <= k + 1 for h in hist)
    m.close()


@pytest.mark.parametrize("k", [2, 3])
def test_forced_acceptance_commits_k_plus_one(O, cfgs, k):
    cfg = cfgs[k]
    m = O.Model(cfg, SEED)
    p = prompt(cfg, 11, seed=5)
    first = m.prefill(p)
    plain = plain_stream(m, first, 40)
    m.prefill(p)
    out = [first]
    while len(out) < 30:
        i = len(out)
        got = m.spec_round(forced=np.array(plain[i:i + k] + [0] * 8, np.int32))
        assert len(got) == k + 1
        out.extend(got)
    assert out[:30] == plain[:30]
    m.close()


def test_mismatching_drafts_roll_back(O, cfgs):
    """Drafts forced wrong at j: nacc = j, and the committed stream still equals plain greedy
    (the rejected rows' recurrent state updates are discarded)."""
    k = 3
    cfg = cfgs[k]
    m = O.Model(cfg, SEED)
    p = prompt(cfg, 9, seed=6)
    first = m.prefill(p)
    plain = plain_stream(m, first, 60)
    m.prefill(p)
    out = [first]
    j = 0
    while len(out) < 40:
        i = len(out)
        d = list(plain[i:i + k])
        bad = j % (k + 1)                           # draft index to corrupt (k = none)
        if bad < k:
            d[bad] = (d[bad] + 1) % cfg.vocab
        got = m.spec_round(forced=np.array(d + [0] * 8, np.int32))
        assert len(got) == (bad if bad < k else k) + 1
        out.extend(got)
        j += 1
    assert out[:40] == plain[:40]
    m.close()


def test_multirow_verify_equals_single_rows(O, X):
    """A 4-row verify of the greedy continuation [t0, t1, t2, t3] gives, row for row, the tokens
    and final-residual bits of four plain single-row steps."""
    cfg = tiny(X, spec_k=3, n_layers=4)
    a, b = O.Model(cfg, SEED), O.Model(cfg, SEED)
    p = prompt(cfg, 10, seed=8)
    first = a.prefill(p)
    assert b.prefill(p) == first
    toks, hs = [first], []
    for _ in range(4):
        toks.append(b.decode_step())
        hs.append(b.tensor("hprev", -1, np.uint16)[: cfg.hidden].copy())
    nx = np.zeros(8, np.int32)
    O.lib().q27o_model_verify_rows(a.m, 4, np.array(toks[:4], np.int32).ctypes.data, nx.ctypes.data)
    assert nx[:4].tolist() == toks[1:5]
    ha = a.tensor("hfinal", -1, np.uint16)[: 4 * cfg.hidden].reshape(4, -1)
    for r in range(4):
        assert np.array_equal(ha[r], hs[r]), r
    a.close()
    b.close()


def test_determinism(O, X):
    cfg = tiny(X, spec_k=2, n_layers=4)
    outs = []
    for _ in range(2):
        m = O.Model(cfg, SEED)
        first = m.prefill(prompt(cfg, 7, seed=1))
        outs.append(spec_stream(m, first, 16)[0])
        m.close()
    assert outs[0] == outs[1]
    m = O.Model(cfg, SEED + 1)
    other = spec_stream(m, m.prefill(prompt(cfg, 7, seed=1)), 16)[0]
    m.close()
    assert other != outs[0]


def test_argmax_semantics(O):
    L = O.lib()
    x = np.array([[1.0, 3.0, 3.0, -np.inf, 2.0],
                  [np.nan, np.inf, 0.5, 0.5, -1.0],
                  [np.nan, np.inf, -np.inf, np.nan, np.inf],
                  [-5.0, -4.0, -4.0, -7.0, -4.5]], np.float32)
    idx, val = np.empty(4, np.int32), np.empty(4, np.float32)
    L.q27o_argmax_rows(x.ctypes.data, 5, 5, 4, idx.ctypes.data, val.ctypes.data)
    assert idx.tolist() == [1, 2, 0, 1]
    assert val[0] == 3.0 and val[1] == 0.5 and val[2] == -np.inf and val[3] == -4.0
    rng = np.random.default_rng(3)
    y = rng.standard_normal((3, 62080)).astype(np.float32)
    L.q27o_argmax_rows(y.ctypes.data, 62080, 62080, 3, idx.ctypes.data, val.ctypes.data)
    assert idx[:3].tolist() == np.argmax(y, axis=1).tolist()


@pytest.mark.parametrize("nx,dt,nacc", [([5, 6, 7], [5, 6], 2), ([5, 6, 7], [5, 9], 1), ([5, 6, 7], [4, 6], 0),
                                        ([1], [], 0), ([1, 2, 3, 4, 5, 6, 7, 8], [1, 2, 3, 4, 5, 6, 7], 7),
                                        ([1, 2, 3, 4], [1, 2, 9], 2)])
def test_accept_definition(O, nx, dt, nacc):
    out = np.zeros(8, np.int32)
    a, d = np.array(nx, np.int32), np.array(dt + [0], np.int32)
    n = O.lib().q27o_accept(a.ctypes.data, d.ctypes.data, len(dt), out.ctypes.data)
    assert n == nacc
    assert out[: n + 1].tolist() == nx[: n + 1]
