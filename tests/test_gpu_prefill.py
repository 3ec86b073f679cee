"""The layer-major prefill on the int8 MFMA GEMM path (q27x_prefill_gemm) against the oracle's
restatement (q27o_model_prefill_gemm): after the prompt, the first token and the whole committed
state bit for bit (h_prev, every GDN layer's state and conv history, every attention layer's and
the MTP layer's KV cache), then speculative rounds continuing from it, round by round with their
drafts and hand-off. Prompts span several chunks (Q27X_PF_CHUNK) and several attention launches
(128 query rows each); the the model's widths run at 4 layers; the full 64-layer model checks that
spec == plain greedy after a GEMM prefill."""
import os

import numpy as np
import pytest

from test_gpu_model import check_round_state, kv_bytes, prompt_of

pytestmark = pytest.mark.gpu

SEED = 0x51E70003


def check_prefill_state(eng, om, cfg, tag):
    H = cfg.hidden
    assert np.array_equal(eng.read("hprev", -1, np.uint16, H), om.tensor("hprev", -1, np.uint16)), (tag, "h_prev")
    n = kv_bytes(cfg)
    nqkv = (2 * cfg.gdn_kh + cfg.gdn_vh) * 128
    kv = (("kc", np.int8, n), ("vc", np.int8, n), ("ks", np.float32, n // cfg.kv_group),
          ("vs", np.float32, n // cfg.kv_group))
    for L in list(range(cfg.n_layers)) + [-1]:
        if L < 0 or (L + 1) % cfg.attn_period == 0:
            for name, dt, cnt in kv:
                g = eng.read(name, L, dt, cnt).view(np.uint8)
                o = om.tensor(name, L, dt)[:cnt].view(np.uint8)
                assert np.array_equal(g, o), (tag, L, name, int(np.argmax(g != o)))
        else:
            S = eng.read("S", L, np.float32, cfg.gdn_vh * 128 * 128)
            assert np.array_equal(S.view(np.uint32), om.tensor("S", L, np.float32).view(np.uint32)), (tag, L, "S")
            h = eng.read("conv_hist", L, np.uint16, nqkv * 3)
            assert np.array_equal(h, om.tensor("conv_hist", L, np.uint16)), (tag, L, "conv history")


def run_case(X, O, cfg, n, rounds, chunk=None, seed=3):
    p = prompt_of(cfg, n, seed=seed)
    eng, om = X.Engine(cfg, SEED), O.Model(cfg, SEED)
    old = os.environ.get("Q27X_PF_CHUNK")
    try:
        if chunk:
            os.environ["Q27X_PF_CHUNK"] = str(chunk)
        first_g = eng.prefill_gemm(p)
        first_o = om.prefill_gemm(p, 0)
        assert first_g == first_o, (n, first_g, first_o)
        check_prefill_state(eng, om, cfg, f"prefill n={n} chunk={chunk}")
        for r in range(rounds):
            a, b = eng.spec_round(), om.spec_round()
            assert a == b, (r, a, b)
            check_round_state(eng, om, cfg, f"round {r} after a GEMM prefill of {n}")
    finally:
        if chunk:
            if old is None:
                del os.environ["Q27X_PF_CHUNK"]
            else:
                os.environ["Q27X_PF_CHUNK"] = old
        eng.close()
        om.close()


@pytest.mark.parametrize("n,chunk,gs", [(1, None, 0), (9, None, 0), (300, None, 0), (150, 64, 0), (70, 8, 0),
                                        (300, None, 1024), (70, 8, 1024)])
def test_tiny_prefill_gemm_matches_oracle(gpu, O, n, chunk, gs):
    """gs: the K-group of the trunk's GEMMs (Q27_Q8_GS): 0 = the whole K (the reference default),
    1024 (at the tiny widths only the K = 2048 down has two groups)."""
    run_case(gpu, O, gpu.tiny_config(spec_k=2, pf_gs=gs), n, 3, chunk)


def test_tiny_wide_group_swiglu_prefill_matches_oracle(gpu, O):
    """inter 5120 with whole-K groups: the down projection's input is quantized per (token, 5120)
    by the wide-group SwiGLU kernel (values held in registers: 1280 quads on 1024 threads, the
    second chunk partly filled)."""
    run_case(gpu, O, gpu.tiny_config(spec_k=2, inter=5120, pf_gs=0), 40, 3, None)


def test_tiny_k7_prefill_gemm_matches_oracle(gpu, O):
    run_case(gpu, O, gpu.tiny_config(spec_k=7), 45, 2, 16)


@pytest.mark.parametrize("n,chunk,gs", [(64, None, 0), (96, 32, 0), (64, None, 1024)])
def test_full_width_prefill_gemm_matches_oracle(gpu, O, n, chunk, gs):
    """The model's widths at 4 layers (3 GDN + 1 attention): the 16384-row in_qkv|in_z, 34816-row
    gate|up and K = 17408 down GEMMs, 32q/8kv attention, the 62080-row head, with whole-K groups
    (the reference default) and with 1024-column groups (5, 6 and 17 of them). (96 tokens in 32-row
    chunks: three chunks on alternating streams, each layer behind the previous chunk's.)"""
    run_case(gpu, O, gpu.default_config(spec_k=2, n_layers=4, ctx=512, pf_gs=gs), n, 2, chunk)


def test_full_width_prefill_wide_gemm_tiles_match_oracle(gpu, O, monkeypatch):
    """The 256 x 256 GEMM tiles in every epilogue form the prefill uses (fp32 and bf16 outputs, the
    bf16 residual of down, out_proj and o_proj) at the model's widths: 520 tokens in a 512-row
    chunk (the tiles need 512 rows) and an 8-row one, with the tiles forced wherever the shape
    allows them (Q27X_GEMM_W4 = 1); state after the prompt and two rounds bit for bit."""
    monkeypatch.setenv("Q27X_GEMM_W4", "1")
    run_case(gpu, O, gpu.default_config(spec_k=2, n_layers=4, ctx=1024), 520, 2)


def test_full_model_spec_equals_plain_after_prefill_gemm(gpu):
    X = gpu
    cfg = X.default_config(spec_k=2, ctx=2048)
    eng = X.Engine(cfg, SEED)
    p = prompt_of(cfg, 1500, seed=6)
    first = eng.prefill_gemm(p)
    plain, _ = eng.generate(24, spec=False)
    assert plain[0] == first
    assert eng.prefill_gemm(p) == first
    spec, _ = eng.generate(24, spec=True)
    assert spec == plain
    eng.close()
