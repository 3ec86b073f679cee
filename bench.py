#!/usr/bin/env python3
"""Benchmark of the chained-MTP K=2 speculative decode of the random-init int8 27B model on one
MI355X (benchmark config 3): committed tok/s and verify-step HBM GB/s.

A step is one chained-MTP round (K=2 drafts through the MTP layer, a 3-row verify through all 64
layers, greedy acceptance, rollback and hand-off, all on the device, one HIP graph launch). The
timed region is exactly --steps rounds after --warmup rounds, with the prompt (1024 uniform-random
ids) already ingested and every input resident in HBM. Natural acceptance is the headline value;
the forced-acceptance mode (drafts = the trunk's own greedy continuation, same draft and verify
work) is reported beside it.
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qwen3.8-27b-mi50-cpp-engine_amd")
HBM_PEAK_GBS = 8000.0
SEED = 0x51E70003


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _load(name, path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def verify_bytes(c, ctx_len, nr):
    """Algorithmic HBM bytes of one nr-row verify at context ctx_len (weights once per verify,
    KV once per layer, recurrent state read once and written once)."""
    H, I, V, D = c.hidden, c.inter, c.vocab, c.gdn_d
    nqkv, nz = (2 * c.gdn_kh + c.gdn_vh) * D, c.gdn_vh * D
    qr = c.n_q * (2 * c.head_dim if c.attn_gate else c.head_dim)
    kvr, att = c.n_kv * c.head_dim, c.n_q * c.head_dim
    i8 = 1.0 + 4.0 / 64
    total = 0.0
    for L in range(c.n_layers):
        total += 3 * I * H * i8 + 2 * H * 2
        if L % c.attn_period == c.attn_period - 1:
            total += (qr + 2 * kvr) * H * i8 + H * att * i8 + 2 * 128 * 2
            total += 2 * ctx_len * kvr * (1 + 4.0 / c.kv_group) + 2 * nr * kvr * (1 + 4.0 / c.kv_group)
        else:
            total += (nqkv + nz) * H * i8 + H * nz * i8 + 2 * c.gdn_vh * H * 2 + nqkv * 4 * 2
            total += 2 * c.gdn_vh * D * D * 4 + 2 * nqkv * 3 * 2
    total += V * H * 2 + H * 2
    return total


def host_info():
    """CPU model, logical CPUs and the OpenMP thread count the oracle runs with."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    return {"cpu_model": model, "nproc": os.cpu_count(), "omp_threads": threads}


def best_of(fn, reps):
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return min(ts), float(np.median(ts))


def cpu_baseline(cfg_dict, q27o, k, pos):
    """The oracle's integer path (int8 x int8 -> int32 per 16, fp32 scaling; OpenMP over output rows,
    attention (row, head) pairs and GDN value heads) on a bounded sample of one round at the GPU
    line's context: the (k+1)-row verify of a 4-layer full-width slice (3 GDN + 1 attention) at
    positions pos.. with the lm_head, the lm_head alone, and one single-row MTP draft pass with its
    head at draft position pos - 1. The attention layer's and the MTP layer's KV caches hold pos
    positions of seeded random int8 codes and scales (the cost of a verify depends on the cache
    length, not on how the cache was filled). A round is 16 x (slice - lm_head) + lm_head + k drafts
    (one token per round at natural acceptance on random weights)."""
    d = dict(cfg_dict)
    d["n_layers"] = 4
    d["ctx"] = pos + 64
    t0 = time.time()
    m = q27o.Model(d, SEED)
    gen_s = time.time() - t0
    lib = q27o.lib()
    H, V = d["hidden"], d["vocab"]
    rng = np.random.default_rng(3)
    kvr = d["n_kv"] * d["head_dim"]
    for layer in (3, -1):
        for name in ("kc", "vc"):
            codes = np.zeros((d["ctx"], kvr), np.int8)
            codes[:pos] = rng.integers(-127, 128, (pos, kvr), dtype=np.int8)
            m.set_tensor(name, layer, codes)
        for name in ("ks", "vs"):
            sc = np.zeros((d["ctx"], kvr // d["kv_group"]), np.float32)
            sc[:pos] = rng.uniform(1e-3, 2e-2, (pos, kvr // d["kv_group"]))
            m.set_tensor(name, layer, sc)
    toks = np.arange(1, k + 2, dtype=np.int32)
    nx = np.zeros(8, np.int32)

    def slice_verify():
        lib.q27o_model_set_pos(m.m, pos)
        lib.q27o_model_verify_rows(m.m, k + 1, toks.ctypes.data, nx.ctypes.data)
    t_slice, _ = best_of(slice_verify, 3)
    lm = m.tensor("lm_head", -1, np.uint16)
    y = q27o.f2bf(np.random.default_rng(2).standard_normal((k + 1, H)).astype(np.float32))
    logits = np.empty((k + 1, V), np.float32)
    idx, val = np.empty(8, np.int32), np.empty(8, np.float32)

    def head():
        lib.q27o_bf16_gemv_rows(lm.ctypes.data, V, H, y.ctypes.data, H, logits.ctypes.data, V, k + 1)
        lib.q27o_argmax_rows(logits.ctypes.data, V, V, k + 1, idx.ctypes.data, val.ctypes.data)
    t_head, _ = best_of(head, 3)
    del lm
    hrow = y[:1].copy()
    t_draft, _ = best_of(lambda: m.mtp_pass(hrow, toks[:1], pos - 1, 0), 3)
    m.close()
    scale = cfg_dict["n_layers"] / 4.0
    round_s = scale * max(t_slice - t_head, 0.0) + t_head + k * t_draft
    info = host_info()
    return {"value": round(1.0 / round_s, 4), "unit": "committed tok/s", "cores": info["omp_threads"],
            "kind": "port", **info,
            "sample": f"best of 3 at context {pos}: {k + 1}-row verify of a 4-layer full-width slice (3 GDN + "
                      f"1 attention) + lm_head {t_slice:.3f} s, lm_head alone {t_head:.3f} s, one MTP draft pass "
                      f"{t_draft:.3f} s; round = {scale:.0f} x (slice - lm_head) + lm_head + {k} drafts = "
                      f"{round_s:.2f} s at one token per round; KV caches of {pos} positions filled with seeded "
                      f"random codes; weight generation {gen_s:.1f} s not timed"}


# ---------------------------------------------------------------- benchmark configs 0-2
CFG_SHAPES = dict(H=5120, I=17408, KH=16, VH=48, D=128, NQ=32, NKV=8, HD=128, GROUP=32, NR=3)


def cpu_configs(q27o, attn_ctx, reps=5):
    """Benchmark configs 0-2 on the host through the oracle's kernel-tier functions (OpenMP over
    output rows), on seeded synthetic inputs of the benchmark shapes; best and median of reps."""
    L = q27o.lib()
    c = CFG_SHAPES
    H, I, nr, D, VH, KH = c["H"], c["I"], c["NR"], c["D"], c["VH"], c["KH"]
    rng = np.random.default_rng(SEED)
    i8 = 1.0 + 4.0 / 64
    out = {}

    def i8w(rows, K):
        return (rng.integers(-127, 128, (rows, K), dtype=np.int8),
                rng.uniform(1e-4, 2e-3, (rows, K // 64)).astype(np.float32))

    def bf(shape, std=1.0, mean=0.0):
        return q27o.f2bf((mean + rng.standard_normal(shape) * std).astype(np.float32))

    # config 0: one 3-row W8A8 projection [17408 x 5120], fp32 out
    W, WS = i8w(I, H)
    xq = rng.integers(-127, 128, (nr, H), dtype=np.int8)
    xs = rng.uniform(1e-3, 5e-2, (nr, H // 16)).astype(np.float32)
    y = np.empty((nr, I), np.float32)
    tmin, tmed = best_of(lambda: L.q27o_proj_rows(W.ctypes.data, WS.ctypes.data, 1.0, I, H, xq.ctypes.data, H,
                                                  xs.ctypes.data, y.ctypes.data, I, nr), reps)
    b0 = I * H * i8 + nr * H * (1 + 4.0 / 16) + nr * I * 4
    threads = host_info()["omp_threads"]
    out["config0_projection"] = {"ms": round(tmin * 1e3, 3), "ms_median": round(tmed * 1e3, 3),
                                 "bytes": b0, "GB_s": round(b0 / tmin / 1e9, 2), "threads": threads}
    del W, WS
    # shared: the layer input (fp32 residual rows), its norm + quantize
    xres = rng.standard_normal((nr, H)).astype(np.float32)
    nw = bf((H,), 0.02)
    hq = np.empty((nr, H), np.int8)
    hs = np.empty((nr, H // 16), np.float32)
    hb = np.empty((nr, H), np.uint16)
    yn = np.empty((nr, H), np.uint16)

    def norm():
        L.q27o_rmsnorm_quant_rows(xres.ctypes.data, 0, H, nw.ctypes.data, 1.0, 1e-6, H, hb.ctypes.data, yn.ctypes.data,
                                  H, hq.ctypes.data, hs.ctypes.data, 0, 1.0, nr)
    # config 1: one GDN layer's mixer
    nqkv, nz = (2 * KH + VH) * D, VH * D
    Wz, Sz = i8w(nqkv + nz, H)
    Wo, So = i8w(H, nz)
    in_a, in_b = bf((VH, H), 0.02), bf((VH, H), 0.02)
    A_log = q27o.f2bf(rng.uniform(0, 2.7, VH).astype(np.float32))
    dtb = bf((VH,), 0.1)
    gnw = bf((D,), 0.02, 1.0)
    conv_w = bf((nqkv, 4), 0.3)
    S = (rng.standard_normal((VH, D, D)) * 0.1).astype(np.float32)
    hist = bf((nqkv, 3))
    pend = np.zeros(L.q27o_gdn_pend_bytes(KH, VH, D, 8), np.uint8)
    pb = np.empty((nr, nqkv + nz), np.uint16)
    ab = np.empty((2, nr, VH), np.float32)
    tmp = np.empty((nr, VH), np.float32)
    gout = np.empty((nr, nz), np.uint16)
    gq, gs = np.empty((nr, nz), np.int8), np.empty((nr, nz // 16), np.float32)
    r1 = np.empty((nr, H), np.float32)

    def gdn_layer():
        norm()
        L.q27o_proj_rows_epi(Wz.ctypes.data, Sz.ctypes.data, 1.0, nqkv + nz, H, hq.ctypes.data, H, hs.ctypes.data,
                             pb.ctypes.data, nqkv + nz, 1, None, 0, 0, 0.0, nr)
        for j, w in enumerate((in_a, in_b)):
            L.q27o_bf16_gemv_rows(w.ctypes.data, VH, H, yn.ctypes.data, H, tmp.ctypes.data, VH, nr)
            ab[j] = q27o.bf2f(q27o.f2bf(tmp))
        L.q27o_gdn_verify(pb.ctypes.data, nqkv + nz, pb.ctypes.data + nqkv * 2, nqkv + nz, ab[0].ctypes.data, ab[1].ctypes.data, VH, A_log.ctypes.data, dtb.ctypes.data,
                          gnw.ctypes.data, conv_w.ctypes.data, S.ctypes.data, hist.ctypes.data, pend.ctypes.data, 1,
                          KH, VH, D, 1e-6, gout.ctypes.data, nz, gq.ctypes.data, gs.ctypes.data, nr)
        L.q27o_proj_rows_epi(Wo.ctypes.data, So.ctypes.data, 1.0, H, nz, gq.ctypes.data, nz, gs.ctypes.data,
                             r1.ctypes.data, H, 0, hb.ctypes.data, 1, H, 1.0, nr)
    gdn_layer()
    tmin, tmed = best_of(gdn_layer, reps)
    b1 = ((nqkv + nz) * H * i8 + nr * H * 4 + nr * (nqkv + nz) * 2 + 2.0 * VH * H * 2 + nqkv * 4 * 2 +
          2.0 * VH * D * D * 4 + H * nz * i8 + nr * H * 6)
    out["config1_gdn_layer"] = {"ms": round(tmin * 1e3, 3), "ms_median": round(tmed * 1e3, 3), "bytes": b1,
                                "GB_s": round(b1 / tmin / 1e9, 2), "threads": threads}
    del Wz, Sz, Wo, So
    # config 2: one attention layer's mixer at contexts attn_ctx
    NQ, NKV, HD, G = c["NQ"], c["NKV"], c["HD"], c["GROUP"]
    qr, kvr, att = NQ * 2 * HD, NKV * HD, NQ * HD
    Wq, Sq = i8w(qr + 2 * kvr, H)
    Wo2, So2 = i8w(H, att)
    qn, kn = bf((HD,), 0.02), bf((HD,), 0.02)
    qkv = np.empty((nr, qr + 2 * kvr), np.uint16)
    qh = np.empty((nr, att), np.uint16)
    ao = np.empty((nr, att), np.uint16)
    aq, asc = np.empty((nr, att), np.int8), np.empty((nr, att // 16), np.float32)
    for L0 in attn_ctx:
        ctx = L0 + nr
        kc = rng.integers(-127, 128, (ctx, kvr), dtype=np.int8)
        vc = rng.integers(-127, 128, (ctx, kvr), dtype=np.int8)
        ks = rng.uniform(1e-3, 2e-2, (ctx, kvr // G)).astype(np.float32)
        vs = rng.uniform(1e-3, 2e-2, (ctx, kvr // G)).astype(np.float32)
        cs, sn = np.empty(ctx * 16, np.float32), np.empty(ctx * 16, np.float32)
        L.q27o_rope_table(ctx, 32, 1e7, cs.ctypes.data, sn.ctypes.data)

        def attn_layer():
            norm()
            L.q27o_proj_rows_epi(Wq.ctypes.data, Sq.ctypes.data, 1.0, qr + 2 * kvr, H, hq.ctypes.data, H,
                                 hs.ctypes.data, qkv.ctypes.data, qr + 2 * kvr, 1, None, 0, 0, 0.0, nr)
            L.q27o_attn_prep_rows(qkv.ctypes.data, qr + 2 * kvr, qn.ctypes.data, kn.ctypes.data, cs.ctypes.data,
                                  sn.ctypes.data, 32, kc.ctypes.data, ks.ctypes.data, vc.ctypes.data, vs.ctypes.data,
                                  G, qh.ctypes.data, NQ, NKV, HD, 1, 1e-6, L0, nr)
            L.q27o_attn_rows(qh.ctypes.data, qkv.ctypes.data, qr + 2 * kvr, kc.ctypes.data, ks.ctypes.data,
                             vc.ctypes.data, vs.ctypes.data, G, NQ, NKV, HD, 1, L0, nr, ao.ctypes.data, aq.ctypes.data,
                             asc.ctypes.data)
            L.q27o_proj_rows_epi(Wo2.ctypes.data, So2.ctypes.data, 1.0, H, att, aq.ctypes.data, att,
                                 asc.ctypes.data, r1.ctypes.data, H, 0, hb.ctypes.data, 1, H, 1.0, nr)
        tmin, tmed = best_of(attn_layer, reps)
        b2 = ((qr + 2 * kvr) * H * i8 + nr * H * 4 + nr * (qr + 2 * kvr) * 2 + 2.0 * ctx * kvr * (1 + 4.0 / G) +
              H * att * i8 + nr * H * 6)
        out[f"config2_attention_ctx{L0}"] = {"ms": round(tmin * 1e3, 3), "ms_median": round(tmed * 1e3, 3),
                                             "bytes": b2, "GB_s": round(b2 / tmin / 1e9, 2), "threads": threads}
    out["host"] = host_info()
    return out


def gpu_config0(q27x, iters=50, copies=6):
    """Benchmark config 0 on the GPU through the kernel tier (q27x_proj_rows, fp32 out): 3 rows x
    [17408 x 5120]; launches cycle through `copies` weight copies (570 MB) so none hits the
    Infinity Cache; device events around iters launches."""
    import ctypes
    c = CFG_SHAPES
    H, I, nr = c["H"], c["I"], c["NR"]
    rng = np.random.default_rng(SEED)
    W = rng.integers(-127, 128, (I, H), dtype=np.int8)
    WS = rng.uniform(1e-4, 2e-3, (I, H // 64)).astype(np.float32)
    ws = [(q27x.DevBuf(array=W), q27x.DevBuf(array=WS)) for _ in range(copies)]
    xq = q27x.DevBuf(array=rng.integers(-127, 128, (nr, H), dtype=np.int8))
    xs = q27x.DevBuf(array=rng.uniform(1e-3, 5e-2, (nr, H // 16)).astype(np.float32))
    y = q27x.DevBuf(nr * I * 4)
    hs = [q27x.I8G(w.ptr, s.ptr, 1.0, I, H) for w, s in ws]

    def launch(i):
        q27x.call("q27x_proj_rows", ctypes.byref(hs[i % copies]), xq.ptr, H, xs.ptr, y.ptr, I, 0, None, 0, 0, 0.0, nr,
                  None)
    e0, e1, ms = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_float()
    q27x.call("q27x_event_create", ctypes.byref(e0))
    q27x.call("q27x_event_create", ctypes.byref(e1))
    for i in range(3):
        launch(i)
    q27x.call("q27x_event_record", e0, None)
    for i in range(iters):
        launch(i + 3)
    q27x.call("q27x_event_record", e1, None)
    q27x.call("q27x_device_sync")
    q27x.call("q27x_event_elapsed_ms", e0, e1, ctypes.byref(ms))
    for e in (e0, e1):
        q27x.call("q27x_event_destroy", e)
    for w, s in ws:
        w.free()
        s.free()
    for b in (xq, xs, y):
        b.free()
    i8 = 1.0 + 4.0 / 64
    b0 = I * H * i8 + nr * H * (1 + 4.0 / 16) + nr * I * 4
    us = ms.value * 1e3 / iters
    return {"us": round(us, 2), "bytes": b0, "GB_s": round(b0 / (us * 1e-6) / 1e9, 1),
            "frac_of_hbm_peak": round(b0 / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


COPY_BYTES = 1 << 28       # calibration copy: 256 MiB read + 256 MiB written per launch
CFG4_PROMPT = 16320        # benchmark config 4: ctx 16384; the prompt leaves room for one 8-row verify


def config4(eng, cfg, prefill):
    """Benchmark config 4 (K = 7, ctx 16384) on the bench's own context: a CFG4_PROMPT-token prompt
    ingested on the GEMM path (wall clock), then the 8-row verify (K = 7: NR = 8) over all 64 layers
    at that context, timed with device events over 10 launches; its algorithmic bytes (weights once,
    the KV of CFG4_PROMPT positions per attention layer, the GDN state read and written) give GB/s.
    The 4096-token ingest rate comes from the prefill legs. Runs last on the context (it overwrites
    the prompt state)."""
    if cfg.ctx < CFG4_PROMPT + 8:
        return None
    p = np.random.default_rng(0x51E70004).integers(0, cfg.vocab, CFG4_PROMPT).astype(np.int32)
    t = time.time()
    eng.prefill_gemm(p)
    ingest_s = time.time() - t
    vms = eng.bench_verify(8, 10)
    vb = verify_bytes(cfg, CFG4_PROMPT, 8)
    gbs = vb / (vms / 1e3) / 1e9
    g4096 = prefill.get("gemm_path_4096", {})
    return {"verify_rows": 8, "ctx": CFG4_PROMPT, "verify_ms": round(vms, 4), "verify_bytes": vb,
            "verify_GB_s": round(gbs, 1), "verify_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "ingest_tokens": CFG4_PROMPT, "ingest_s": round(ingest_s, 3),
            "ingest_tok_s": round(CFG4_PROMPT / ingest_s, 1), "ingest_4096_tok_s": g4096.get("tok_s")}


def kernel_only(q27x, args):
    """The dominant kernel alone (gate|up with its norm prologue, 20 launches cycling the layers)
    and a plain copy of COPY_BYTES (10 launches), so that a rocprofv3 --pmc pass sees both."""
    import ctypes
    cfg = q27x.default_config(spec_k=args.k, ctx=args.prompt + 256)
    eng = q27x.Engine(cfg, SEED)
    eng.prefill(np.random.default_rng(SEED).integers(0, cfg.vocab, 64).astype(np.int32))
    ms, b = eng.bench_kernel(0, 1, args.k + 1, 20)
    eng.close()
    t = ctypes.c_float()
    q27x.call("q27x_bench_stream", 1, COPY_BYTES, 4, 4, 10, ctypes.byref(t))
    print(json.dumps({"kernel_us": round(ms * 1e3, 2), "kernel_bytes": b, "copy_bytes": COPY_BYTES,
                      "copy_us": round(t.value * 1e3, 2)}), flush=True)
    return 0


INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA, published


def prefill_gemm(q27x, reps=20, gs=5120):
    """The prefill ingest GEMM on int8 MFMA (q27x_gemm_i8g) at benchmark config 4's shape: M = 4096
    tokens x N = 17408 (gate) x K = 5120, groups of gs columns (the whole K by default, the
    reference's default Q27_Q8_GS arm; 1024 is the other), seeded codes and scales resident on the
    device; device events around `reps` back-to-back launches."""
    import ctypes
    M, N, K = 4096, 17408, 5120
    rng = np.random.default_rng(SEED)
    host = [rng.integers(-127, 127, (N, K), dtype=np.int8, endpoint=True),
            rng.uniform(1e-4, 2e-3, (N, K // gs)).astype(np.float32),
            rng.integers(-127, 127, (M, K), dtype=np.int8, endpoint=True),
            rng.uniform(1e-3, 5e-2, (M, K // gs)).astype(np.float32)]
    bufs = [q27x.DevBuf(array=h) for h in host]
    y = q27x.DevBuf(M * N * 4)
    args = (bufs[0].ptr, bufs[1].ptr, N, K, gs, 1.0, bufs[2].ptr, bufs[3].ptr, M, y.ptr, N, None, N, 0.0, None)
    e0, e1, ms = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_float()
    q27x.call("q27x_event_create", ctypes.byref(e0))
    q27x.call("q27x_event_create", ctypes.byref(e1))
    for _ in range(3):
        q27x.call("q27x_gemm_i8g", *args)
    q27x.call("q27x_event_record", e0, None)
    for _ in range(reps):
        q27x.call("q27x_gemm_i8g", *args)
    q27x.call("q27x_event_record", e1, None)
    q27x.call("q27x_device_sync")
    q27x.call("q27x_event_elapsed_ms", e0, e1, ctypes.byref(ms))
    for e in (e0, e1):
        q27x.call("q27x_event_destroy", e)
    for b in bufs + [y]:
        b.free()
    us = ms.value * 1e3 / reps
    tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
    kern = ("k_gemm_i8g_w4 (256 x 256 tiles, 8 waves of 128 x 64, two per SIMD, 128-byte LDS-DMA stages, one group over the whole K)"
            if gs == K else
            "k_gemm_i8g_rs (256-token x 128-row tiles, register-staged 128-byte stages, fp32 group-sum epilogue)")
    return {"kernel": kern,
            "shape": {"M": M, "N": N, "K": K, "gs": gs}, "us_per_launch": round(us, 1),
            "achieved": round(tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TOPS (int8, dense)",
            "frac": round(tops / INT8_PEAK_TOPS, 4)}


def traffic_from_profiles():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by the same counter's reading for the calibration copy)."""
    path = os.path.join(ROOT, "profiles", "gate_up_k2_pmc_traffic.json")
    try:
        with open(path) as fh:
            return json.load(fh).get("traffic_bytes")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=1024)
    ap.add_argument("--k", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-forced", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="eager launches (profilers that cannot follow graphs)")
    ap.add_argument("--prefill-gemm-only", action="store_true",
                    help="only the int8-MFMA prefill GEMM leg (for rocprofv3 passes on it)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the GEMM-path prompt ingest of --prompt tokens, twice (for kernel traces)")
    ap.add_argument("--rounds-only", action="store_true",
                    help="only the prompt ingest (GEMM path) and the natural-acceptance rounds (for kernel traces)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the dominant kernel (gate|up) and the calibration copy, for rocprofv3 --pmc passes")
    args = ap.parse_args()
    if args.no_graph:
        os.environ["Q27X_GRAPH"] = "0"
    if args.gpus != 1:
        print(f"bench.py: this build runs the hot path on one GPU; --gpus {args.gpus} is not supported "
              f"(nothing here is sharded across GPUs)", file=sys.stderr)
        return 2
    q27x = _load("q27x", os.path.join(PKG, "q27x.py"))
    if q27x.gpu_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    q27x.call("q27x_set_device", 0)
    if args.kernel_only:
        return kernel_only(q27x, args)
    if args.prefill_gemm_only:
        print(json.dumps({"prefill_gemm": prefill_gemm(q27x)}), flush=True)
        return 0
    K = args.k
    rounds_total = args.warmup + args.steps
    attn_ctx = [1024, 4096, 16384]
    ctx = max(args.prompt + rounds_total * (K + 1) + 128, max(attn_ctx) + 64)
    cfg = q27x.default_config(spec_k=K, ctx=ctx)
    t0 = time.time()
    eng = q27x.Engine(cfg, SEED)
    log(f"engine: {eng.weight_bytes() / 1e9:.2f} GB weights resident, {time.time() - t0:.1f} s")
    prompt = np.random.default_rng(0x51E70003).integers(0, cfg.vocab, args.prompt).astype(np.int32)
    if args.prefill_only:
        ts = []
        for _ in range(2):
            t = time.time()
            eng.prefill_gemm(prompt)
            ts.append(time.time() - t)
        print(json.dumps({"prefill_only": {"tokens": args.prompt, "s": [round(x, 4) for x in ts],
                                           "tok_s": round(args.prompt / ts[-1], 1)}}), flush=True)
        eng.close()
        return 0
    if args.rounds_only:
        eng.prefill_gemm(prompt)
        eng.run_rounds(args.warmup, spec=True)
        st = eng.run_rounds(args.steps, spec=True)
        print(json.dumps({"rounds_only": {"spec_k": K, "prompt": args.prompt, "rounds": st.rounds,
                                          "committed": st.committed,
                                          "ms_per_round": round(st.decode_ms / st.rounds, 4)}}), flush=True)
        eng.close()
        return 0

    # ---- natural acceptance
    # prompt ingest: the verify kernels over the prompt (q27x_prefill) and the layer-major int8-MFMA
    # GEMM path (q27x_prefill_gemm, benchmark config 4's prefill ingest), wall clock per call
    t = time.time()
    eng.prefill(prompt)
    prefill_s = time.time() - t
    prefill = {"verify_path": {"tokens": args.prompt, "s": round(prefill_s, 4),
                               "tok_s": round(args.prompt / prefill_s, 1)}}
    for n_pf in sorted({args.prompt, 1024, 4096}):
        p_pf = np.random.default_rng(0x51E70004 + n_pf).integers(0, cfg.vocab, n_pf).astype(np.int32)
        eng.prefill_gemm(p_pf)                      # first call allocates its buffers
        t = time.time()
        eng.prefill_gemm(p_pf)
        s_pf = time.time() - t
        prefill[f"gemm_path_{n_pf}"] = {"tokens": n_pf, "s": round(s_pf, 4), "tok_s": round(n_pf / s_pf, 1)}
    log(f"prefill: {prefill}")
    eng.prefill_gemm(prompt)
    eng.run_rounds(args.warmup, spec=True)
    st = eng.run_rounds(args.steps, spec=True)
    nat_tps = st.committed / (st.decode_ms / 1e3)
    ms_per_round = st.decode_ms / st.rounds
    phases = {n: round(getattr(st, n + "_ms") / st.rounds, 4) for n in ("draft", "verify", "head", "tail")}
    log(f"natural: {st.rounds} rounds, {st.committed} committed, {nat_tps:.1f} tok/s, {ms_per_round:.3f} ms/round; "
        f"phases {phases}")

    # ---- plain greedy (comparator, and the forced-acceptance draft stream)
    eng.prefill_gemm(prompt)
    n_plain = rounds_total * (K + 1) + 4
    t = time.time()
    plain, _ = eng.generate(n_plain, spec=False)
    plain_s = time.time() - t
    plain_tps = (len(plain) - 1) / plain_s
    log(f"plain: {len(plain)} tokens, {plain_tps:.1f} tok/s")

    forced = None
    if not args.no_forced:
        eng.prefill_gemm(prompt)
        eng.set_forced(np.array(plain, np.int32))
        eng.run_rounds(args.warmup, spec=True)
        sf = eng.run_rounds(args.steps, spec=True)
        forced = {"committed_tok_s": round(sf.committed / (sf.decode_ms / 1e3), 2),
                  "tokens_per_round": round(sf.committed / sf.rounds, 3),
                  "ms_per_round": round(sf.decode_ms / sf.rounds, 4)}
        eng.set_forced([])
        log(f"forced: {forced}")

    # ---- verify step and dominant kernel, timed with device events on the engine stream
    vms = eng.bench_verify(K + 1, 20)
    ctx_now = args.prompt + rounds_total
    vbytes = verify_bytes(cfg, ctx_now, K + 1)
    v_gbs = vbytes / (vms / 1e3) / 1e9
    kms, kbytes = eng.bench_kernel(0, 1, K + 1, 50)
    k_gbs = kbytes / (kms / 1e3) / 1e9
    log(f"verify: {vms:.3f} ms, {v_gbs:.0f} GB/s ({v_gbs / HBM_PEAK_GBS:.3f} of peak); "
        f"gate|up kernel {kms * 1e3:.1f} us {k_gbs:.0f} GB/s")
    kernels = {}
    for which, name in ((0, "in_qkv_z_conv"), (2, "down_residual"), (3, "out_proj_residual"), (4, "lm_head_argmax")):
        ms_, b_ = eng.bench_kernel(0, which, K + 1, 50)
        kernels[name] = {"us": round(ms_ * 1e3, 2), "GB_s": round(b_ / (ms_ / 1e3) / 1e9, 1)}
    log(f"kernels: {kernels}")

    # ---- benchmark configs 0-2 on the GPU (3 rows; config 0 through the kernel tier, 1 and 2 on the
    # engine's own kernels; these overwrite the context's state, so they run last)
    gpu_cfg = {"config0_projection": gpu_config0(q27x)}
    ms_, b_ = eng.bench_mixer(False, args.prompt, 3, 48)
    gpu_cfg["config1_gdn_layer"] = {"us": round(ms_ * 1e3, 2), "bytes": b_, "GB_s": round(b_ / (ms_ / 1e3) / 1e9, 1)}
    for L0 in attn_ctx:
        ms_, b_ = eng.bench_mixer(True, L0, 3, 48)
        gpu_cfg[f"config2_attention_ctx{L0}"] = {"us": round(ms_ * 1e3, 2), "bytes": b_,
                                                 "GB_s": round(b_ / (ms_ / 1e3) / 1e9, 1)}
    for v in gpu_cfg.values():
        v["frac_of_hbm_peak"] = round(v["GB_s"] / HBM_PEAK_GBS, 4)
    log(f"configs 0-2 (GPU): {gpu_cfg}")
    cfg4 = config4(eng, cfg, prefill)
    log(f"config 4: {cfg4}")
    eng.close()
    pg = prefill_gemm(q27x)
    pg["gs1024"] = {k_: v_ for k_, v_ in prefill_gemm(q27x, gs=1024).items() if k_ in ("us_per_launch", "achieved", "frac")}
    log(f"prefill GEMM: {pg}")
    cfg4["prefill_gemm_frac_of_int8_peak"] = pg["frac"]

    cpu = None
    cpu_cfg = None
    if not args.no_cpu:
        q27o = _load("q27o", os.path.join(ROOT, "oracle", "q27o.py"))
        log("cpu baseline (oracle) ...")
        cpu = cpu_baseline(cfg.as_dict(), q27o, K, args.prompt)
        log(f"cpu: {cpu}")
        cpu_cfg = cpu_configs(q27o, attn_ctx)
        log(f"configs 0-2 (CPU): {cpu_cfg}")

    workload = (f"BASELINE config {3 if (K == 2 and args.prompt == 1024) else 4 if K == 7 else 3}: random-init "
                f"int8 27B (64 layers: 48 GDN + 16 attention), chained MTP K={K}, {args.prompt}-token prompt, "
                f"natural acceptance")
    out = {
        "metric": "committed tok/s (MTP K=2, 27B int8, 1 GPU) + verify-step HBM GB/s",
        "value": round(nat_tps, 2),
        "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_round, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8",
        "data": f"synthetic: seeded random-init int8 weights, {args.prompt} uniform-random prompt ids",
        "config": {"workload": workload, "spec_k": K, "prompt": args.prompt, "hidden": cfg.hidden,
                   "layers": cfg.n_layers},
        "acceptance": {"tokens_per_round": round(st.committed / st.rounds, 3), "rounds": st.rounds,
                       "p_ge": [round(st.acc_hist[j] / st.rounds, 3) for j in range(1, K + 1)]},
        "round_phases_ms": phases,
        "forced_acceptance": forced,
        "plain_decode_tok_s": round(plain_tps, 2),
        "verify_step": {"ms": round(vms, 4), "bytes": vbytes, "GB_s": round(v_gbs, 1),
                        "frac_of_hbm_peak": round(v_gbs / HBM_PEAK_GBS, 4), "rows": K + 1},
        "roofline": {"bound": "hbm",
                     "kernel": f"k_proj<{K + 1}, 5, 1, 2, true, true, 16> (gate|up: post-norm prologue, W8A8, "
                               f"SwiGLU + quantize)",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                     "bytes_per_launch": kbytes, "us_per_launch": round(kms * 1e3, 2)},
        "kernels": kernels,
        "configs_gpu": gpu_cfg,
        "configs_cpu": cpu_cfg,
        "prefill_s": round(prefill_s, 3),
        "prefill": prefill,
        "prefill_gemm": pg,
        "config4": cfg4,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
