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


@pytest.mark.parametrize("k", [1, 3, 4, 5, 6])
def test_tiny_rounds_every_k_match_oracle(gpu, O, k):
    """K = 1 and 3..6 (2 and 4..7 verify rows: the projection, norm-prologue, SwiGLU, conv and
    attention instances between the 3-row and 8-row ones), round by round with everything each
    round leaves behind compared with the oracle."""
    X = gpu
    cfg = tiny(X, spec_k=k)
    eng, om = X.Engine(cfg, SEED), O.Model(cfg, SEED)
    p = prompt_of(cfg, 29, seed=13 + k)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(4):
        a, b = eng.spec_round(), om.spec_round()
        assert a == b, (k, r, a, b)
        check_round_state(eng, om, cfg, f"K={k} round {r}")
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
    """Benchmark config 3 geometry (64 layers, 48 GDN + 16 attention, hidden 5120): spec(K=2)
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


@pytest.mark.parametrize("k", [2, 7])
def test_long_context_spec_equals_plain(gpu, k):
    """Past 2048 positions each attention block takes several 64-key splits in turn, so the step's
    new positions (normed, roped, written to the cache inside the split kernel) can fall in a later
    split of a block. After a 2400-token prompt: spec == plain greedy, and forced acceptance
    commits K + 1 tokens per round."""
    X = gpu
    cfg = X.default_config(spec_k=k, ctx=2560)
    eng = X.Engine(cfg, SEED)
    p = prompt_of(cfg, 2400, seed=5)
    eng.prefill_gemm(p)
    plain, _ = eng.generate(40, spec=False)
    eng.prefill_gemm(p)
    spec, _ = eng.generate(40, spec=True)
    assert spec == plain
    eng.prefill_gemm(p)
    eng.set_forced(np.array(plain, np.int32))
    forced, stf = eng.generate(40, spec=True)
    assert forced == plain
    assert stf.acc_hist[k] >= stf.rounds - 1, (stf.rounds, list(stf.acc_hist))
    eng.set_forced([])
    eng.close()


def test_config4_k7_ctx16k_forced_equals_plain(gpu):
    """Benchmark config 4 (64 layers, K = 7, ctx 16384): after a 16200-token prompt, forced
    acceptance (drafts = the trunk's own greedy continuation) commits K + 1 = 8 tokens per round
    and the stream equals plain greedy -- the 8-row verify forms (one weight pass for down and
    lm_head), attention over ~16K positions, and the K = 7 hand-off at full geometry."""
    X = gpu
    cfg = X.default_config(spec_k=7, ctx=16384)
    eng = X.Engine(cfg, SEED)
    p = prompt_of(cfg, 16200, seed=4)
    first = eng.prefill_gemm(p)
    print("config 4: prompt ingested", flush=True)
    plain, _ = eng.generate(48, spec=False)
    assert plain[0] == first
    print("config 4: plain stream done", flush=True)
    eng.prefill_gemm(p)
    print("config 4: prompt ingested again", flush=True)
    eng.set_forced(np.array(plain, np.int32))
    forced, stf = eng.generate(48, spec=True)
    print("config 4: forced rounds done", flush=True)
    assert forced == plain
    assert stf.acc_hist[7] >= stf.rounds - 1, (stf.rounds, list(stf.acc_hist))
    assert stf.committed >= 8 * (stf.rounds - 1)
    eng.set_forced([])
    eng.close()

# ---------------------------------------------------------------- drafts and hand-off
def kv_bytes(cfg):
    return cfg.ctx * cfg.n_kv * cfg.head_dim


def check_round_state(eng, om, cfg, tag, gdn_layer=0):
    """Everything a round leaves behind, GPU against oracle, bit for bit: the drafts (what the
    verify saw and the MTP argmax before any forcing), the verify argmaxes, the hand-off (catch-up
    rows and tokens, h_prev), the MTP chain residual, the MTP layer's KV cache, and one GDN layer's
    committed state."""
    H, K = cfg.hidden, cfg.spec_k
    g_dt, o_dt = eng.read("dt", -1, np.int32, 8)[:K], om.tensor("dt", -1, np.int32)[:K]
    assert g_dt.tolist() == o_dt.tolist(), (tag, "drafts", g_dt, o_dt)
    g_raw, o_raw = eng.read("dt_raw", -1, np.int32, 8)[:K], om.tensor("dt_raw", -1, np.int32)[:K]
    assert g_raw.tolist() == o_raw.tolist(), (tag, "MTP argmax", g_raw, o_raw)
    g_nx, o_nx = eng.read("nx", -1, np.int32, 8)[:K + 1], om.tensor("nx", -1, np.int32)[:K + 1]
    assert g_nx.tolist() == o_nx.tolist(), (tag, "verify argmax", g_nx, o_nx)
    nc = int(eng.read("ncatch", -1, np.int32, 1)[0])
    assert nc == int(om.tensor("ncatch", -1, np.int32)[0]), (tag, "ncatch")
    if nc:
        assert eng.read("catch_tok", -1, np.int32, 8)[:nc].tolist() == om.tensor("catch_tok", -1, np.int32)[:nc].tolist()
        hc_g = eng.read("hcatch", -1, np.uint16, 8 * H)[: nc * H]
        hc_o = om.tensor("hcatch", -1, np.uint16)[: nc * H]
        assert np.array_equal(hc_g, hc_o), (tag, "catch-up rows")
    assert np.array_equal(eng.read("hprev", -1, np.uint16, H), om.tensor("hprev", -1, np.uint16)), (tag, "h_prev")
    head = int(eng.read("mtp_head", -1, np.int32, 1)[0])
    chain = eng.read("mtp_res", -1, np.uint16, 8 * H)[head * H:(head + 1) * H]
    assert np.array_equal(chain, om.tensor("hchain", -1, np.uint16)), (tag, "MTP chain residual")
    n = kv_bytes(cfg)
    for name, dt, cnt in (("kc", np.int8, n), ("vc", np.int8, n), ("ks", np.float32, n // cfg.kv_group),
                          ("vs", np.float32, n // cfg.kv_group)):
        assert np.array_equal(eng.read(name, -1, dt, cnt).view(np.uint8), om.tensor(name, -1, dt)[:cnt].view(np.uint8)), \
            (tag, "MTP cache " + name)
    S_g = eng.read("S", gdn_layer, np.float32, cfg.gdn_vh * 128 * 128)
    assert np.array_equal(S_g.view(np.uint32), om.tensor("S", gdn_layer, np.float32).view(np.uint32)), (tag, "GDN S")
    nqkv = (2 * cfg.gdn_kh + cfg.gdn_vh) * 128
    hg = eng.read("conv_hist", gdn_layer, np.uint16, nqkv * 3)
    assert np.array_equal(hg, om.tensor("conv_hist", gdn_layer, np.uint16)), (tag, "committed conv history")


@pytest.mark.parametrize("k", [2, 7])
def test_tiny_drafts_and_handoff_match_oracle(gpu, O, k):
    """Natural acceptance, round by round: drafts, MTP argmax, MTP chain residual and KV cache,
    hand-off and GDN state are the oracle's bits (on random weights the MTP rarely matches the
    trunk, so this checks the draft layer itself)."""
    X = gpu
    cfg = tiny(X, spec_k=k)
    eng, om = X.Engine(cfg, SEED), O.Model(cfg, SEED)
    p = prompt_of(cfg, 23, seed=40 + k)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(6):
        a, b = eng.spec_round(), om.spec_round()
        assert a == b, (k, r, a, b)
        check_round_state(eng, om, cfg, f"K={k} round {r}")
    eng.close()
    om.close()


def corrupted_stream(plain, vocab, seed, density=0.3):
    rng = np.random.default_rng(seed)
    s = np.array(plain, np.int32)
    bad = rng.random(len(s)) < density
    bad[0] = False
    s[bad] = (s[bad] + 1 + rng.integers(0, 7, bad.sum())) % vocab
    return s


@pytest.mark.parametrize("k", [2, 7])
def test_tiny_partial_acceptance_matches_oracle(gpu, O, k):
    """Forced drafts from the trunk's own greedy stream with wrong tokens planted at seeded
    positions: every acceptance length 0..K occurs, so the rollback of 0 < nacc < K rows, the
    catch-up rows of the next draft and the deferred GDN commit all run on the GPU; each round's
    state is the oracle's, and the committed stream is plain greedy."""
    X = gpu
    cfg = tiny(X, spec_k=k)
    eng, om = X.Engine(cfg, SEED), O.Model(cfg, SEED)
    p = prompt_of(cfg, 19, seed=60 + k)
    n = len(p)
    first = om.prefill(p)
    plain = [first] + [om.decode_step() for _ in range(120)]
    forced = corrupted_stream(plain, cfg.vocab, seed=70 + k, density=0.12 if k == 7 else 0.3)
    assert eng.prefill(p) == om.prefill(p) == first
    eng.set_forced(forced)
    out, seen = [first], set()
    for r in range(14):
        b0 = int(om.tensor("pos", -1, np.int32)[0]) - n
        d = list(forced[b0 + 1:b0 + 1 + k])
        got_o = om.spec_round(forced=np.array(d + [0] * 8, np.int32))
        got_g = eng.spec_round()
        assert got_g == got_o, (k, r, got_g, got_o)
        seen.add(len(got_o) - 1)
        check_round_state(eng, om, cfg, f"K={k} forced round {r}")
        out.extend(got_o)
    assert out == plain[:len(out)]
    assert 0 in seen and any(0 < s < k for s in seen), (k, sorted(seen))
    eng.set_forced([])
    eng.close()
    om.close()


def test_generate_continues_after_its_budget(tiny_pair):
    """A generate call that reached max_new leaves the context ready: the next generate (larger
    budget), a plain step and a spec round continue the oracle's greedy stream."""
    X, cfg, eng, om = tiny_pair
    p = prompt_of(cfg, 17, seed=21)
    first = om.prefill(p)
    plain = [first] + [om.decode_step() for _ in range(40)]
    assert eng.prefill(p) == first
    a, _ = eng.generate(10, spec=True)
    assert a == plain[:10]
    b, st = eng.generate(20, spec=True)
    assert b == plain[:20] and st.committed >= 1
    eng.decode_step()
    eng.spec_round()
    c = int(eng.read("pos", -1, np.int32, 1)[0]) - len(p) + 1     # tokens committed so far
    stream, _ = eng.generate(c, spec=True)                         # budget already met: reads them
    assert len(stream) == c and stream == plain[:c], (stream, plain[:c])


def _first_occurrence_at(stream, lo, residue, mod):
    """An index j >= lo with j % mod == residue whose token does not occur before it."""
    for j in range(lo, len(stream)):
        if j % mod == residue and stream[j] not in stream[:j]:
            return j
    raise AssertionError("no token with a first occurrence at the wanted index")


def test_generate_stops_after_the_stop_token(gpu, O):
    """q27x_generate ends a request after the first committed stop token (src/q27_main.cpp:6680-6683):
    the output is the oracle's greedy stream through that token, also when it is the middle token
    of a forced round (the round still commits all of its tokens to the state); a later generate
    returns the same output, the single-step entries continue the stream, and a prompt whose first
    token is the stop token yields only that token."""
    X = gpu
    base = tiny(X, spec_k=2)
    om = O.Model(base, SEED)
    p = prompt_of(base, 17, seed=31)
    first = om.prefill(p)
    plain = [first] + [om.decode_step() for _ in range(48)]
    om.close()
    for spec, forced, field in ((True, False, "eos_id"), (False, False, "eos_id"), (True, True, "eos_id2")):
        # forced rounds commit indices 1 + 3r .. 3 + 3r: index 3r + 2 is a round's middle token
        j = _first_occurrence_at(plain, 6, 2, 3) if forced else _first_occurrence_at(plain, 6, 0, 1)
        cfg = tiny(X, spec_k=2, eos_id=-1, eos_id2=-1)
        setattr(cfg, field, plain[j])
        eng = X.Engine(cfg, SEED)
        assert eng.prefill(p) == first
        if forced:
            eng.set_forced(np.array(plain + [0] * 16, np.int32))
        out, st = eng.generate(40, spec=spec)
        assert out == plain[:j + 1], (spec, forced, j, out)
        committed = int(eng.read("pos", -1, np.int32, 1)[0]) - len(p) + 1
        if forced:
            assert committed == j + 2, committed          # the whole round
        elif not spec:
            assert committed == j + 1, committed
        else:
            assert j + 1 <= committed <= j + 3, committed  # natural rounds commit 1 + nacc
        again, _ = eng.generate(40, spec=spec)
        assert again == plain[:j + 1]
        eng.set_forced([])
        assert eng.decode_step() == plain[committed]
        eng.close()
    # the prompt's own first token is the stop token: the request is over at once
    cfg = tiny(X, spec_k=2, eos_id=first, eos_id2=-1)
    eng = X.Engine(cfg, SEED)
    assert eng.prefill(p) == first
    out, st = eng.generate(40, spec=True)
    assert out == [first] and st.rounds == 0
    eng.close()


def test_generate_runs_to_the_end_of_the_context(gpu, O):
    """max_new past the context: speculative rounds while pos + K < ctx, then plain steps, and the
    request ends with the context full (src/q27_main.cpp:6384, 6391) -- no error, and the tokens are
    the oracle's plain greedy stream to the last position."""
    X = gpu
    cfg = tiny(X, spec_k=3, ctx=64)
    eng, om = X.Engine(cfg, SEED), O.Model(cfg, SEED)
    p = prompt_of(cfg, 40, seed=5)
    first = om.prefill(p)
    plain = [first] + [om.decode_step() for _ in range(cfg.ctx - len(p))]
    assert eng.prefill(p) == first
    out, st = eng.generate(200, spec=True)
    assert out == plain, (len(out), len(plain))
    assert int(eng.read("pos", -1, np.int32, 1)[0]) == cfg.ctx
    # forced acceptance (K+1 per round) reaches the edge with larger steps
    eng.prefill(p)
    eng.set_forced(np.array(plain + [0] * 16, np.int32))
    out2, st2 = eng.generate(200, spec=True)
    assert out2 == plain
    eng.set_forced([])
    with pytest.raises(X.Q27XError):
        eng.spec_round()                     # pos == ctx: nothing left to run
    eng.close()
    om.close()


def test_round_phase_times_are_reported(tiny_pair):
    X, cfg, eng, om = tiny_pair
    eng.prefill(prompt_of(cfg, 12, seed=2))
    st = eng.run_rounds(5, spec=True)
    assert st.rounds == 5
    parts = [st.draft_ms, st.verify_ms, st.head_ms, st.tail_ms]
    assert all(v > 0 for v in parts), parts
    assert sum(parts) < st.decode_ms * 1.05, (parts, st.decode_ms)


def full_width_rounds(X, O, cfg, prompt, natural, forced_rounds, seed, prefill="decode", tag=""):
    """Natural rounds, then forced rounds with planted wrong drafts (partial acceptance), on the
    engine and the oracle side by side: every round's tokens and the whole round state
    (check_round_state) bit for bit."""
    K = cfg.spec_k
    eng, om = X.Engine(cfg, SEED), O.Model(cfg, SEED)
    ing_e = eng.prefill if prefill == "decode" else eng.prefill_gemm
    ing_o = om.prefill if prefill == "decode" else (lambda ids: om.prefill_gemm(ids, 0))
    first = ing_o(prompt)
    print(f"{tag}: oracle ingested {len(prompt)} tokens", flush=True)
    assert ing_e(prompt) == first
    assert np.array_equal(eng.read("hprev", -1, np.uint16, cfg.hidden), om.tensor("hprev", -1, np.uint16))
    for r in range(natural):
        a, b = eng.spec_round(), om.spec_round()
        assert a == b, (tag, r, a, b)
        check_round_state(eng, om, cfg, f"{tag} natural round {r}")
    print(f"{tag}: {natural} natural rounds match", flush=True)
    # plain greedy continuation (the oracle's), then drafts from it with wrong tokens planted
    ing_o(prompt)
    plain = [first] + [om.decode_step() for _ in range(forced_rounds * (K + 1) + 2)]
    forced = corrupted_stream(plain, cfg.vocab, seed=seed, density=0.12 if K >= 5 else 0.35)
    assert ing_e(prompt) == ing_o(prompt) == first
    eng.set_forced(forced)
    n, seen, out = len(prompt), set(), [first]
    for r in range(forced_rounds):
        b0 = int(om.tensor("pos", -1, np.int32)[0]) - n
        d = list(forced[b0 + 1:b0 + 1 + K])
        got_o = om.spec_round(forced=np.array(d + [0] * 8, np.int32))
        got_g = eng.spec_round()
        assert got_g == got_o, (tag, r, got_g, got_o)
        check_round_state(eng, om, cfg, f"{tag} forced round {r}")
        seen.add(len(got_o) - 1)
        out.extend(got_o)
    assert out == plain[:len(out)]
    print(f"{tag}: {forced_rounds} forced rounds match, acceptance lengths {sorted(seen)}", flush=True)
    eng.set_forced([])
    eng.close()
    om.close()
    return seen


@pytest.mark.parametrize("k", [1, 2, 3, 5, 7])
def test_full_width_rounds_match_oracle(gpu, O, k):
    """The model's widths (hidden 5120, inter 17408, vocab 62080, GDN 16/48 heads, attention 32q/8kv,
    kv_group 32, MTP layer on) at 4 layers (3 GDN + 1 attention), against the oracle at K = 1, 2,
    3, 5 and 7 (2, 3, 4, 6 and 8 verify rows): prefill of 64 tokens, 3 natural rounds and 4 forced rounds with
    planted wrong drafts (partial acceptance), each round's tokens, drafts, hand-off, MTP state and
    GDN state bit for bit. These are the engine's full-width kernel instantiations at every row
    count the benchmark configs use: the norm prologues at K = 5120 (two rows per 256-thread group
    past 4 rows), the split SwiGLU units, the conv epilogue and a/b rows, the 32q/8kv attention,
    the one-pass 8-row down, the MTP layer's down in one launch (1 to 4 rows) and in four slice
    launches (6 and 8 rows) and the 62080-row lm_head with argmax partials."""
    X = gpu
    cfg = X.default_config(spec_k=k, n_layers=4, ctx=256)
    p = prompt_of(cfg, 64, seed=31)
    seen = full_width_rounds(X, O, cfg, p, natural=3, forced_rounds=4, seed=30 + k, tag=f"full width K={k}")
    assert any(s < k for s in seen), (k, sorted(seen))


def test_full_width_long_context_rounds_match_oracle(gpu, O):
    """Past 2048 positions at 8 kv heads each attention block takes several 64-key splits in turn
    (the grid holds 32 blocks per kv head), and the step's new positions fall in a later split of a
    block. Full-width attention geometry (hidden 5120, 32q/8kv, GDN 16/48 heads, vocab 62080) with
    one GDN and one attention layer and a narrow MLP (inter 1024) so that the oracle ingests a
    2100-token prompt (GEMM prefill) in seconds; then K = 7 rounds, natural and forced, against the
    oracle round by round."""
    X = gpu
    cfg = X.default_config(spec_k=7, n_layers=2, attn_period=2, inter=1024, ctx=2304)
    p = prompt_of(cfg, 2100, seed=35)
    full_width_rounds(X, O, cfg, p, natural=3, forced_rounds=4, seed=37, prefill="gemm", tag="ctx 2.1K K=7")


# ---------------------------------------------------------------- the reference trunk's attention
# include/q27.h:25-35, src/q27_attn.hip:10-11: 24 q / 4 kv heads of 256 dims (GQA group 6), q_proj
# rows [q 256 | gate 256] per head, RoPE on the first 64 of 256 dims
TRUNK_ATTN = dict(head_dim=256, rot_dims=64)


@pytest.mark.parametrize("k", [2, 7])
def test_trunk_attention_geometry_rounds_match_oracle(gpu, O, k):
    """Tiny widths with the trunk's attention head shape (6 q / 1 kv heads of 256 dims, group 6,
    64 rotary dims): decode-path prefill, then rounds with the whole round state against the oracle,
    and forced rounds with wrong drafts planted (partial acceptance)."""
    X = gpu
    cfg = tiny(X, spec_k=k, n_q=6, n_kv=1, **TRUNK_ATTN)
    p = prompt_of(cfg, 70, seed=80 + k)
    seen = full_width_rounds(X, O, cfg, p, natural=4, forced_rounds=5, seed=81 + k, tag=f"hd256 tiny K={k}")
    assert any(s < k for s in seen), sorted(seen)


def test_trunk_attention_geometry_gemm_prefill_matches_oracle(gpu, O):
    """The same geometry through the GEMM-path prefill (several 128-row attention launches of
    8-row tiles on the general kernel), then rounds."""
    X = gpu
    cfg = tiny(X, spec_k=2, n_q=6, n_kv=1, **TRUNK_ATTN)
    p = prompt_of(cfg, 300, seed=84)
    full_width_rounds(X, O, cfg, p, natural=3, forced_rounds=3, seed=85, prefill="gemm", tag="hd256 tiny GEMM prefill")


def test_full_width_trunk_attention_geometry_rounds_match_oracle(gpu, O):
    """The model's widths with the trunk's attention (hidden 5120, 24 q / 4 kv x 256, group 6, 64 rotary
    dims; q|k|v 14336 rows, o_proj K = 6144) at 4 layers, K = 2: decode-path prefill and rounds,
    natural and forced, bit for bit against the oracle."""
    X = gpu
    cfg = X.default_config(spec_k=2, n_layers=4, ctx=256, n_q=24, n_kv=4, **TRUNK_ATTN)
    p = prompt_of(cfg, 64, seed=86)
    full_width_rounds(X, O, cfg, p, natural=3, forced_rounds=4, seed=87, tag="hd256 full width K=2")
