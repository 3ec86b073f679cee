"""Seeded random cases of the whole round against the oracle: K in 1..7, tiny geometries with the
benchmark-shaped and the trunk-shaped attention (GQA groups 4, 6 and 8, 128- and 256-dim heads),
more SwiGLU units than blocks, two-layer attention periods, prompts of 1..259 tokens through
either prefill and either prefill group setting; each case runs natural rounds, then forced rounds
with planted wrong drafts, and compares every round's tokens and whole state bit for bit."""
import numpy as np
import pytest

from test_gpu_model import full_width_rounds

pytestmark = pytest.mark.gpu

GEOMS = [dict(), dict(inter=5120), dict(n_q=6, n_kv=1, head_dim=256, rot_dims=64), dict(n_q=8, n_kv=1),
         dict(n_layers=4, attn_period=2)]


def draw(case):
    rng = np.random.default_rng(0x5EED + case)
    k = int(rng.integers(1, 8))
    geom = GEOMS[case % len(GEOMS)]
    n = int(rng.integers(1, 260))
    prefill = "decode" if rng.random() < 0.5 else "gemm"
    gs = int(rng.choice([0, 1024]))
    return k, geom, n, prefill, gs, rng


@pytest.mark.parametrize("case", range(15))
def test_random_rounds_match_oracle(gpu, O, case):
    X = gpu
    k, geom, n, prefill, gs, rng = draw(case)
    cfg = X.tiny_config(spec_k=k, ctx=512, pf_gs=gs, **geom)
    prompt = rng.integers(0, cfg.vocab, n).astype(np.int32)
    tag = f"case {case}: K={k} geometry={geom} prompt={n} prefill={prefill} gs={gs}"
    print(tag, flush=True)
    full_width_rounds(X, O, cfg, prompt, natural=3, forced_rounds=5, seed=2000 + case, prefill=prefill, tag=tag)
