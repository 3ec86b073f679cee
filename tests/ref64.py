"""Float64 textbook forms of the verify-path operators, written from the mathematics (not from
the oracle's code): the independent side of the oracle-pinning tests and of the golden fixtures.
Nothing here mirrors a reduction order; agreement is asserted within stated tolerances."""
import numpy as np


def bf2f(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_rne(x):
    """Round float32 values to the nearest bf16 (ties to even mantissa), by comparing the two
    neighbouring bf16 values in float64 -- no bit trick."""
    x = np.asarray(x, np.float32)
    u = x.view(np.uint32)
    lo = (u >> 16).astype(np.uint32)                 # truncation (toward zero in magnitude)
    hi = lo + 1
    flo = (lo << 16).view(np.float32).astype(np.float64)
    fhi = (hi << 16).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    dlo, dhi = np.abs(xd - flo), np.abs(fhi - xd)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo & 1) == 1))
    return np.where(pick_hi, hi, lo).astype(np.uint16)


def quant_ideal(v, group):
    """Symmetric absmax int8 quantization in float64: s = max|v|/127, q = round-half-even(v/s)."""
    v = np.asarray(v, np.float64).reshape(-1, group)
    mx = np.abs(v).max(axis=1, keepdims=True)
    s = mx / 127.0
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(s > 0, np.rint(v / np.where(s > 0, s, 1)), 0)
    return np.clip(q, -127, 127).astype(np.int64).ravel(), s.ravel(), (v / np.where(s > 0, s, 1)).ravel()


def assert_codes_match_ideal(codes, v, group, tie_tol=1e-4):
    """int8 codes equal the float64 ideal except where v/s sits within tie_tol of a half-integer
    (there float32 rounding may legitimately go either way, by one code)."""
    q, s, t = quant_ideal(v, group)
    codes = np.asarray(codes).astype(np.int64).ravel()
    diff = codes != q
    if diff.any():
        near_tie = np.abs(np.abs(t - np.floor(t)) - 0.5) < tie_tol
        bad = diff & ~(near_tie & (np.abs(codes - q) == 1))
        assert not bad.any(), f"{bad.sum()} codes off the float64 ideal (first at {np.flatnonzero(bad)[:5]})"


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def softplus(x):
    x = np.asarray(x, np.float64)
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))


def rmsnorm(x, w, plus, eps):
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return x * inv * (plus + np.asarray(w, np.float64))


def proj(Wq, Ws, xq, xs, alpha):
    """y[n][r] = alpha * sum_k W[r][k] x[n][k] * ws[r][k/64] * xs[n][k/16] in float64."""
    rows, K = Wq.shape
    wd = Wq.astype(np.float64) * np.repeat(Ws.astype(np.float64), 64, axis=1)
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 16, axis=1)
    return alpha * (xd @ wd.T)


def gdn_rows(qkv_raw, z, a, b, A_log, dt_bias, norm_w, conv_w, S, hist, kh, vh, d, eps=1e-6):
    """Gated delta rule, two-pass textbook form in float64 over nr rows.
    Conv: causal depthwise over [h0, h1, h2, x] then SiLU (rounded to bf16, as the stored
    activations are). Per value head h with key head h // (vh/kh):
      q = q / ||q|| / sqrt(d), k = k / ||k||, beta = sigmoid(b), g = exp(-exp(A_log) softplus(a + dt))
      S <- g S + k (beta (v - g S^T k))^T ;  o = S^T q  (state updated first, then read)
      y = o / rms(o) * norm_w * silu(z).
    S is key-major [h][key j][value e]. Returns y [nr][vh*d], new S, new history."""
    S = np.array(S, np.float64, copy=True)
    hist = np.array(bf2f(hist), np.float64).reshape(-1, 3)
    cw = bf2f(conv_w).astype(np.float64).reshape(-1, 4)
    nr = qkv_raw.shape[0]
    ratio = vh // kh
    ys = np.zeros((nr, vh * d))
    for n in range(nr):
        x = bf2f(qkv_raw[n]).astype(np.float64)
        win = np.concatenate([hist, x[:, None]], axis=1)
        acc = (win * cw).sum(axis=1)
        cv = bf2f(bf16_rne(silu(acc).astype(np.float32))).astype(np.float64)
        hist = win[:, 1:]
        for h in range(vh):
            kk = h // ratio
            q = cv[kk * d:(kk + 1) * d]
            k = cv[kh * d + kk * d: kh * d + (kk + 1) * d]
            v = cv[2 * kh * d + h * d: 2 * kh * d + (h + 1) * d]
            qh = q / np.sqrt((q * q).sum() + 1e-6) / np.sqrt(d)
            khat = k / np.sqrt((k * k).sum() + 1e-6)
            beta = sigmoid(b[n, h])
            g = np.exp(-np.exp(float(bf2f(A_log)[h])) * softplus(a[n, h] + float(bf2f(dt_bias)[h])))
            Sh = S[h]
            delta = beta * (v - g * (Sh.T @ khat))
            Sh = g * Sh + np.outer(khat, delta)
            S[h] = Sh
            o = Sh.T @ qh
            zz = bf2f(z[n, h * d:(h + 1) * d]).astype(np.float64)
            y = o / np.sqrt((o * o).mean() + eps) * bf2f(norm_w).astype(np.float64) * silu(zz)
            ys[n, h * d:(h + 1) * d] = y
    return ys, S, hist


def rope_rotate(y, pos, rot, theta):
    """Rotate-half RoPE on the first `rot` dims of y at position pos, float64."""
    y = np.asarray(y, np.float64).copy()
    half = rot // 2
    f = np.arange(half)
    ang = pos * theta ** (-(2.0 * f) / rot)
    c, s = np.cos(ang), np.sin(ang)
    a, b = y[:half].copy(), y[half:rot].copy()
    y[:half] = a * c - b * s
    y[half:rot] = b * c + a * s
    return y


def attention_rows(qh, gate_vals, Kd, Vd, nq, nkv, hd, pos0, nr):
    """Causal GQA softmax attention in float64: row r attends keys 0..pos0+r; output times
    sigmoid(gate) when gate_vals is given. qh [nr][nq*hd]; Kd/Vd dequantized [ctx][nkv*hd]."""
    G = nq // nkv
    out = np.zeros((nr, nq * hd))
    for r in range(nr):
        L = pos0 + r + 1
        for h in range(nq):
            kv = h // G
            q = qh[r, h * hd:(h + 1) * hd].astype(np.float64)
            K = Kd[:L, kv * hd:(kv + 1) * hd].astype(np.float64)
            V = Vd[:L, kv * hd:(kv + 1) * hd].astype(np.float64)
            sc = K @ q / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            o = (p @ V) / p.sum()
            if gate_vals is not None:
                o = o * sigmoid(gate_vals[r, h * hd:(h + 1) * hd])
            out[r, h * hd:(h + 1) * hd] = o
    return out


def dequant_rows(wq, ws):
    """int8 weights [rows][K] with per-64 scales [rows][K/64] -> float64."""
    return wq.astype(np.float64) * np.repeat(ws.astype(np.float64), 64, axis=1)


def mtp_forward(W, c, hrows, toks, pos0, swap_halves=False, plus_one=None, drop_o=False):
    """The MTP draft layer in float64, from its definition: rows r = (hidden h_r, token t_r) at
    positions pos0 + r;
      x_r = [norm_e(emb[t_r]) | norm_h(h_r)]   (embedding half first when mtp_swap is set)
      res = fc x                                (fc = [fc0 | fc1] over the two halves)
      res += o_proj(attention(norm_in(res)))   (a full-attention decoder layer: per-head norms
                                                 (1 + w), rotate-half RoPE on the first rot dims,
                                                 causal GQA over the rows, output * sigmoid(gate))
      res += down(silu(gate(n)) * up(n)),  n = norm_post(res)
      logits_r = lm_head norm_mtp(res_r)
    W holds the oracle's weights (int8 + scales, bf16 vectors); c the config dict. The keyword
    arguments plant a mistake (for showing that the comparison detects it). Returns (res [nr][H],
    logits [nr][vocab]), float64; every activation stays unquantized."""
    H, hd, nq, nkv = c["hidden"], c["head_dim"], c["n_q"], c["n_kv"]
    po = float(c["mtp_plus_one"]) if plus_one is None else plus_one
    eps = c["rms_eps"]
    nr = len(toks)
    e = bf2f(W["emb"].reshape(-1, H)[np.asarray(toks)]).astype(np.float64)
    h = bf2f(hrows).reshape(nr, H).astype(np.float64)
    ne = rmsnorm(e, bf2f(W["pre_emb"]), po, eps)
    nh = rmsnorm(h, bf2f(W["pre_hid"]), po, eps)
    first, second = (ne, nh) if c["mtp_swap"] else (nh, ne)
    if swap_halves:
        first, second = second, first
    res = first @ dequant_rows(W["fc0_w"], W["fc0_s"]).T + second @ dequant_rows(W["fc1_w"], W["fc1_s"]).T
    # attention block
    x = rmsnorm(res, bf2f(W["in_norm"]), po, eps)
    qkv = x @ dequant_rows(W["qkv_w"], W["qkv_s"]).T
    qw = 2 * hd if c["attn_gate"] else hd
    qrows = nq * qw
    rot, theta = c["rot_dims"], c["rope_theta"]
    qn, kn = bf2f(W["q_norm"]).astype(np.float64), bf2f(W["k_norm"]).astype(np.float64)
    Q = np.zeros((nr, nq, hd))
    G = np.zeros((nr, nq, hd))
    Kh = np.zeros((nr, nkv, hd))
    Vh = np.zeros((nr, nkv, hd))
    for r in range(nr):
        for hh in range(nq):
            q = qkv[r, hh * qw: hh * qw + hd]
            q = q / np.sqrt((q * q).mean() + eps) * (1.0 + qn)
            Q[r, hh] = rope_rotate(q, pos0 + r, rot, theta)
            if c["attn_gate"]:
                G[r, hh] = qkv[r, hh * qw + hd: hh * qw + 2 * hd]
        for kv in range(nkv):
            k = qkv[r, qrows + kv * hd: qrows + (kv + 1) * hd]
            k = k / np.sqrt((k * k).mean() + eps) * (1.0 + kn)
            Kh[r, kv] = rope_rotate(k, pos0 + r, rot, theta)
            Vh[r, kv] = qkv[r, qrows + nkv * hd + kv * hd: qrows + nkv * hd + (kv + 1) * hd]
    att = np.zeros((nr, nq * hd))
    grp = nq // nkv
    for r in range(nr):
        for hh in range(nq):
            kv = hh // grp
            sc = Kh[: r + 1, kv] @ Q[r, hh] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            o = (p @ Vh[: r + 1, kv]) / p.sum()
            if c["attn_gate"]:
                o = o * sigmoid(G[r, hh])
            att[r, hh * hd:(hh + 1) * hd] = o
    if not drop_o:
        res = res + att @ dequant_rows(W["o_w"], W["o_s"]).T
    # MLP
    x = rmsnorm(res, bf2f(W["post_norm"]), po, eps)
    g = x @ dequant_rows(W["gate_w"], W["gate_s"]).T
    u = x @ dequant_rows(W["up_w"], W["up_s"]).T
    a = silu(g) * u
    Wd = np.concatenate([dequant_rows(W[f"down4_w{j}"], W[f"down4_s{j}"]) for j in range(4)], axis=1)
    res = res + a @ Wd.T
    xn = rmsnorm(res, bf2f(W["mtp_norm"]), 1.0, eps)
    logits = xn @ bf2f(W["lm_head"]).reshape(-1, H).astype(np.float64).T
    return res, logits


def absmax_codes(v, group):
    """int8 absmax codes per `group` of the last axis, decided in float32 as the reference's
    quantizer does (src/q27_fp8.hip:373-425 with in_scale 1: s = mx (1/127), inv = 1/s,
    q = clamp(rintf(v inv), -127, 127)). Returns (codes [..., n] int8, scales [..., n/group] float32)."""
    v = np.asarray(v, np.float64).astype(np.float32)
    g = v.reshape(v.shape[:-1] + (v.shape[-1] // group, group))
    s = (np.abs(g).max(axis=-1, keepdims=True) * np.float32(1.0 / 127.0)).astype(np.float32)
    inv = np.where(s > 0, np.float32(1.0) / np.where(s > 0, s, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint((g * inv).astype(np.float32)), -127, 127).astype(np.int8)
    return q.reshape(v.shape), s[..., 0]


def trunk_forward(W, c, toks, faithful=False, plant=None, trace=None, force=None):
    """The verify trunk (run_layer_tp_nr, src/q27_main.cpp:2271-2489, and its head 2457-2481) in
    float64, written from the layer definition, for tokens toks at positions 0..n-1 from an empty
    state. Per layer L (attention when L % attn_period == attn_period - 1, else Gated DeltaNet):
      n   = rmsnorm(x_L) (1 + w_in)                  x_0 = emb[tok]; x_L = r2 of layer L-1
      r1  = x_L + out_proj(mixer(n))                 (o_proj for attention)
      r2  = r1 + down(silu(gate(m)) * up(m)),  m = rmsnorm(r1) (1 + w_post)
    head: hfin = r1 + r2 of the last layer (the reference adds the residual twice, 2471), then
    logits = lm_head rmsnorm(hfin) (1 + w_final).
    GDN mixer: causal depthwise conv4 + SiLU over the q|k|v channels; per value head h (key head
    h // (vh/kh)) q^ = q/||q||/sqrt(d), k^ = k/||k||, beta = sigmoid(b), decay = exp(-exp(A_log)
    softplus(a + dt_bias)), S <- decay S + k^ (beta (v - decay S^T k^))^T, o = S^T q^,
    y = o / rms(o) * w_norm * silu(z); a, b = in_a n, in_b n.
    Attention mixer: per head RMSNorm (1 + w), rotate-half RoPE on the first rot dims, causal GQA
    softmax attention, output * sigmoid(gate) (gate rows follow each head's q rows in q_proj).

    faithful=False: every value float64, no rounding or quantization (the "ideal" model).
    faithful=True: the reference's storage points applied, every sum still float64: bf16 where it
    stores bf16 (the residual copy x_L and r1, projection outputs, the normed rows, conv and mixer
    outputs, the final residual and its norm), int8 absmax codes per 16 of every projection input
    (layer 0 codes the bf16 normed rows, later layers the unrounded ones), the fp32 residual r1 / r2
    unrounded, K and V as int8 per kv_group.
    plant names one composition mistake, to show that a comparison rejects it:
      "drop_out_residual"   r1 = out_proj(...) in the GDN layers (residual not added)
      "single_head_residual" hfin = r2 (no double count)
      "post_norm_bf16"      the post norm reads bf16(r1) instead of r1
      "zgate_before_norm"   y = rmsnorm(o * silu(z)) * w_norm (gate applied before the norm)
      "attn_gate_dropped"   attention output without the sigmoid gate
    W: {"layers": [per-layer dicts], "emb", "final_norm", "lm_head"} of the oracle's weights.
    trace: an optional dict that receives the intermediate values, keyed (layer, stage): "r1"
    (before any forcing), "a2" (the post norm's int8 codes, faithful mode), "r2".
    force: optional values that replace the forward's own at a stage boundary (teacher forcing,
    so that a comparison of one stage does not inherit rounding flips of earlier ones): (L, "x")
    the input rows of layer L >= 1 (r2 of layer L-1), (L, "r1") the residual after layer L's mixer,
    ("head", "r2") the last layer's r2.
    Returns (hfin [n][H], logits [n][vocab]) float64."""
    force = force or {}
    H, eps = c["hidden"], c["rms_eps"]
    D, kh, vh = c["gdn_d"], c["gdn_kh"], c["gdn_vh"]
    hd, nq, nkv = c["head_dim"], c["n_q"], c["n_kv"]
    toks = np.asarray(toks)
    n = len(toks)

    def R(v):
        v = np.asarray(v, np.float64)
        return bf2f(bf16_rne(v.astype(np.float32))).astype(np.float64).reshape(v.shape) if faithful else v

    def Q(v, group=16):
        v = np.asarray(v, np.float64)
        if not faithful:
            return v
        q, s = absmax_codes(v, group)
        return (q.astype(np.float64) * np.repeat(s.astype(np.float64), group, axis=-1)).reshape(v.shape)

    def wmat(Wl, name):
        return dequant_rows(Wl[name + "_w"], Wl[name + "_s"])

    def norm(x, w, plus=1.0):
        return rmsnorm(x, bf2f(w), plus, eps)

    emb = bf2f(W["emb"]).reshape(-1, H).astype(np.float64)
    x = emb[toks]
    h = x.copy()                 # the residual operand of the layer (bf16 copy of x_L)
    r1 = r2 = None
    for L, Wl in enumerate(W["layers"]):
        is_attn = (L % c["attn_period"]) == c["attn_period"] - 1
        if L == 0:
            nn_ = norm(x, Wl["in_norm"])
            y = R(nn_)
            a_in = Q(y)
        else:
            r2 = np.asarray(force.get((L, "x"), r2), np.float64)
            nn_ = norm(r2, Wl["in_norm"])
            h = R(r2)
            y = R(nn_)
            a_in = Q(nn_)
        if is_attn:
            qkv = R(a_in @ wmat(Wl, "qkv").T)
            if trace is not None:
                trace[(L, "a_in")], trace[(L, "qkv")] = a_in, qkv
            qw = 2 * hd if c["attn_gate"] else hd
            qrows = nq * qw
            qn, kn = bf2f(Wl["q_norm"]).astype(np.float64), bf2f(Wl["k_norm"]).astype(np.float64)
            Qh = np.zeros((n, nq, hd)); Gt = np.zeros((n, nq, hd))
            Kh = np.zeros((n, nkv, hd)); Vh = np.zeros((n, nkv, hd))
            for r in range(n):
                for hh in range(nq):
                    q = qkv[r, hh * qw: hh * qw + hd]
                    q = q / np.sqrt((q * q).mean() + eps) * (1.0 + qn)
                    Qh[r, hh] = R(rope_rotate(q, r, c["rot_dims"], c["rope_theta"]))
                    if c["attn_gate"]:
                        Gt[r, hh] = qkv[r, hh * qw + hd: hh * qw + 2 * hd]
                for kv in range(nkv):
                    k = qkv[r, qrows + kv * hd: qrows + (kv + 1) * hd]
                    k = k / np.sqrt((k * k).mean() + eps) * (1.0 + kn)
                    Kh[r, kv] = Q(rope_rotate(k, r, c["rot_dims"], c["rope_theta"]), c["kv_group"])
                    Vh[r, kv] = Q(qkv[r, qrows + nkv * hd + kv * hd: qrows + nkv * hd + (kv + 1) * hd], c["kv_group"])
            att = np.zeros((n, nq * hd))
            grp = nq // nkv
            for r in range(n):
                for hh in range(nq):
                    kv = hh // grp
                    sc = Kh[: r + 1, kv] @ Qh[r, hh] / np.sqrt(hd)
                    p = np.exp(sc - sc.max())
                    o = (p @ Vh[: r + 1, kv]) / p.sum()
                    if c["attn_gate"] and plant != "attn_gate_dropped":
                        o = o * sigmoid(Gt[r, hh])
                    att[r, hh * hd:(hh + 1) * hd] = R(o)
            if trace is not None:
                trace[(L, "q")], trace[(L, "k")], trace[(L, "v")], trace[(L, "att")] = Qh, Kh, Vh, att
            r1 = h + Q(att) @ wmat(Wl, "o").T
        else:
            nqkv = (2 * kh + vh) * D
            qkvz = R(a_in @ wmat(Wl, "qkvz").T)
            qkv_raw, z = qkvz[:, :nqkv], qkvz[:, nqkv:]
            ab_a = R(y @ bf2f(Wl["in_a"]).reshape(vh, H).astype(np.float64).T)
            ab_b = R(y @ bf2f(Wl["in_b"]).reshape(vh, H).astype(np.float64).T)
            cw = bf2f(Wl["conv_w"]).astype(np.float64).reshape(nqkv, 4)
            A_log = bf2f(Wl["A_log"]).astype(np.float64)
            dt_bias = bf2f(Wl["dt_bias"]).astype(np.float64)
            w_norm = bf2f(Wl["gdn_norm"]).astype(np.float64)
            hist = np.zeros((nqkv, 3))
            S = np.zeros((vh, D, D))
            ratio = vh // kh
            mix = np.zeros((n, vh * D))
            for t in range(n):
                win = np.concatenate([hist, qkv_raw[t][:, None]], axis=1)
                cv = R(silu((win * cw).sum(axis=1)))
                hist = win[:, 1:]
                for hh in range(vh):
                    kk = hh // ratio
                    q = cv[kk * D:(kk + 1) * D]
                    k = cv[kh * D + kk * D: kh * D + (kk + 1) * D]
                    v = cv[2 * kh * D + hh * D: 2 * kh * D + (hh + 1) * D]
                    qh_ = q / np.sqrt((q * q).sum() + 1e-6) / np.sqrt(D)
                    kh_ = k / np.sqrt((k * k).sum() + 1e-6)
                    beta = sigmoid(ab_b[t, hh])
                    decay = np.exp(-np.exp(A_log[hh]) * softplus(ab_a[t, hh] + dt_bias[hh]))
                    delta = beta * (v - decay * (S[hh].T @ kh_))
                    S[hh] = decay * S[hh] + np.outer(kh_, delta)
                    o = S[hh].T @ qh_
                    g = silu(z[t, hh * D:(hh + 1) * D])
                    if plant == "zgate_before_norm":
                        og = o * g
                        yv = og / np.sqrt((og * og).mean() + eps) * w_norm
                    else:
                        yv = o / np.sqrt((o * o).mean() + eps) * w_norm * g
                    mix[t, hh * D:(hh + 1) * D] = R(yv)
            if trace is not None:
                trace[(L, "qkvz")], trace[(L, "a")], trace[(L, "b")], trace[(L, "mix")] = qkvz, ab_a, ab_b, mix
            proj = Q(mix) @ wmat(Wl, "out").T
            r1 = proj if plant == "drop_out_residual" else h + proj
        if trace is not None:
            trace[(L, "r1")] = r1
        r1 = np.asarray(force.get((L, "r1"), r1), np.float64)
        m = norm(R(r1) if plant == "post_norm_bf16" else r1, Wl["post_norm"])
        h = R(r1)
        a2 = Q(m)
        g = a2 @ wmat(Wl, "gate").T
        u = a2 @ wmat(Wl, "up").T
        r2 = h + Q(silu(g) * u) @ wmat(Wl, "down").T
        if trace is not None:
            trace[(L, "a2")], trace[(L, "r2")] = absmax_codes(m, 16)[0] if faithful else None, r2
    r2 = np.asarray(force.get(("head", "r2"), r2), np.float64)
    if c["head_double_residual"] and plant != "single_head_residual":
        hfin = R(R(r1) + r2)
    else:
        hfin = R(r2)
    nf = R(norm(hfin, W["final_norm"]))
    logits = nf @ bf2f(W["lm_head"]).reshape(-1, H).astype(np.float64).T
    return hfin, logits
