"""A checkpoint in the reference's naming and formats (fp8 / NVFP4 projections with per-tensor
weight and input scales, bf16 norms and MTP head, NVFP4 lm_head), loaded by the engine
(q27x_load_checkpoint) and, through the oracle's converter restatements, into the CPU oracle:
prefill on both paths and speculative rounds, tokens and the whole committed state bit for bit."""
import numpy as np
import pytest

import ckpt_synth as CS
from test_gpu_model import check_round_state, prompt_of
from test_gpu_prefill import check_prefill_state

pytestmark = pytest.mark.gpu

SEED = 0x51E70003


@pytest.fixture(scope="module")
def loaded(gpu, O, tmp_path_factory):
    X = gpu
    cfg = X.tiny_config(spec_k=2, n_layers=4)
    syn = CS.Synth(cfg, seed=11)
    d = tmp_path_factory.mktemp("ck")
    n, b = CS.write(syn.t, d)
    ck = X.Checkpoint(d, 3, n, b)
    eng = X.Engine(cfg, SEED)
    eng.load_checkpoint(ck)
    om = O.Model(cfg, SEED)
    CS.install_into_oracle(O, om, syn)
    yield X, cfg, eng, om
    eng.close()
    om.close()
    ck.close()


def test_checkpoint_decode_path_matches_oracle(loaded):
    X, cfg, eng, om = loaded
    p = prompt_of(cfg, 29, seed=12)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(3):
        a, b = eng.spec_round(), om.spec_round()
        assert a == b, (r, a, b)
        check_round_state(eng, om, cfg, f"checkpoint round {r}")


def test_checkpoint_gemm_prefill_matches_oracle(loaded):
    X, cfg, eng, om = loaded
    p = prompt_of(cfg, 75, seed=13)
    assert eng.prefill_gemm(p) == om.prefill_gemm(p, 0)
    check_prefill_state(eng, om, cfg, "checkpoint GEMM prefill")
    for r in range(2):
        a, b = eng.spec_round(), om.spec_round()
        assert a == b, (r, a, b)
        check_round_state(eng, om, cfg, f"checkpoint round {r} after the GEMM prefill")


def test_checkpoint_shape_mismatch_is_refused(gpu, tmp_path):
    """A checkpoint of another geometry: the upload checks the plan first and changes nothing."""
    X = gpu
    syn = CS.Synth(X.tiny_config(spec_k=2, n_layers=4), seed=2)
    CS.write(syn.t, tmp_path)
    ck = X.Checkpoint(tmp_path)
    eng = X.Engine(X.tiny_config(spec_k=2, n_layers=4, inter=1024), SEED)
    first = eng.prefill(prompt_of(eng.cfg, 9))
    with pytest.raises(X.Q27XError) as e:
        eng.load_checkpoint(ck)
    assert e.value.rc == -2 and "expected" in str(e.value)
    assert eng.prefill(prompt_of(eng.cfg, 9)) == first       # still the generated weights
    eng.close()
    ck.close()


def test_reload_after_rounds_matches_oracle(gpu, O, tmp_path):
    """New weights on a context that already ran with other ones: the captured round and plain-step
    graphs hold weight pointers, alphas and input scales, and the GEMM prefill holds its own copy of
    every matrix. After load_checkpoint (and back to generated weights with load_synthetic) the
    prefill, the rounds and the GEMM prefill follow the new weights, bit for bit against the oracle,
    and the old GEMM copies are released instead of piling up."""
    X = gpu
    cfg = X.tiny_config(spec_k=2, n_layers=4)
    eng = X.Engine(cfg, SEED)                         # generated weights
    p = prompt_of(cfg, 29, seed=12)
    eng.prefill_gemm(p)                               # GEMM copies of the generated weights
    eng.spec_round()                                  # round graph captured on them
    eng.decode_step()                                 # plain-step graph too
    held = int(eng.read("pf_allocs", -1, np.int32, 1)[0])
    assert held > 0
    syn = CS.Synth(cfg, seed=11)
    n, b = CS.write(syn.t, tmp_path)
    ck = X.Checkpoint(tmp_path, 3, n, b)
    eng.load_checkpoint(ck)
    assert int(eng.read("pf_allocs", -1, np.int32, 1)[0]) == 0
    om = O.Model(cfg, SEED)
    CS.install_into_oracle(O, om, syn)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(3):
        a, b_ = eng.spec_round(), om.spec_round()
        assert a == b_, (r, a, b_)
        check_round_state(eng, om, cfg, f"reloaded round {r}")
    assert eng.decode_step() == om.decode_step()
    assert eng.prefill_gemm(p) == om.prefill_gemm(p, 0)
    check_prefill_state(eng, om, cfg, "reloaded GEMM prefill")
    assert int(eng.read("pf_allocs", -1, np.int32, 1)[0]) == held
    a, b_ = eng.spec_round(), om.spec_round()
    assert a == b_
    om.close()
    # and back to generated weights
    eng.load_synthetic(SEED)
    assert int(eng.read("pf_allocs", -1, np.int32, 1)[0]) == 0
    om2 = O.Model(cfg, SEED)
    assert eng.prefill(p) == om2.prefill(p)
    for r in range(2):
        a, b_ = eng.spec_round(), om2.spec_round()
        assert a == b_, (r, a, b_)
        check_round_state(eng, om2, cfg, f"generated again, round {r}")
    assert eng.decode_step() == om2.decode_step()
    om2.close()
    eng.close()
    ck.close()


def test_checkpoint_with_trunk_attention_geometry(gpu, O, tmp_path):
    """A synthetic checkpoint whose attention has the reference trunk's head shape (256-dim heads,
    GQA group 6, q_proj emitting q and the gate per head, 64 rotary dims; include/q27.h:25-35) passes
    the plan check, loads, and matches the oracle through both prefills and rounds."""
    X = gpu
    cfg = X.tiny_config(spec_k=2, n_layers=4, n_q=6, n_kv=1, head_dim=256, rot_dims=64)
    syn = CS.Synth(cfg, seed=21)
    n, b = CS.write(syn.t, tmp_path)
    ck = X.Checkpoint(tmp_path, 3, n, b)
    assert ck.check(cfg) == (0, "")
    eng = X.Engine(cfg, SEED)
    eng.load_checkpoint(ck)
    om = O.Model(cfg, SEED)
    CS.install_into_oracle(O, om, syn)
    p = prompt_of(cfg, 37, seed=22)
    assert eng.prefill(p) == om.prefill(p)
    for r in range(3):
        a, b_ = eng.spec_round(), om.spec_round()
        assert a == b_, (r, a, b_)
        check_round_state(eng, om, cfg, f"hd256 checkpoint round {r}")
    assert eng.prefill_gemm(p) == om.prefill_gemm(p, 0)
    check_prefill_state(eng, om, cfg, "hd256 checkpoint GEMM prefill")
    for r in range(2):
        a, b_ = eng.spec_round(), om.spec_round()
        assert a == b_, (r, a, b_)
    eng.close()
    om.close()
    ck.close()
