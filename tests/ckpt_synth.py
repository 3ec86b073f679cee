"""Synthetic checkpoints in the reference's naming and storage formats (src/q27_load.cpp:690-815,
src/q27_main.cpp:7134-7152; include/q27.h:60-69), written as safetensors shards, and their
installation into the CPU oracle through the oracle's converter restatements. Test helper."""
import json
import os

import numpy as np
import torch

LP = "model.language_model.layers"


def e4m3_bytes(v):
    """float32 values -> E4M3 bytes (torch's float8_e4m3fn encoder, round to nearest)."""
    t = torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.float8_e4m3fn)
    return t.view(torch.uint8).numpy()


def bf16_bits(v):
    t = torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def geometry(cfg):
    hd = cfg.head_dim
    return dict(H=cfg.hidden, I=cfg.inter, V=cfg.vocab, hd=hd, D=cfg.gdn_d,
                qr=cfg.n_q * (2 * hd if cfg.attn_gate else hd), kvr=cfg.n_kv * hd, att=cfg.n_q * hd,
                nqkv=(2 * cfg.gdn_kh + cfg.gdn_vh) * cfg.gdn_d, nz=cfg.gdn_vh * cfg.gdn_d, vh=cfg.gdn_vh)


class Synth:
    """The tensors of one synthetic checkpoint: {name: (dtype string, numpy array)}."""

    def __init__(self, cfg, seed=7):
        self.cfg, self.g = cfg, geometry(cfg)
        self.rng = np.random.default_rng(seed)
        self.t = {}
        self.build()

    def scalar(self, name, lo, hi):
        self.t[name] = ("F32", np.array([self.rng.uniform(lo, hi)], np.float32).reshape(()))

    def bf16(self, name, shape, std, mean=0.0, uniform=None):
        v = self.rng.uniform(*uniform, size=shape) if uniform else mean + std * self.rng.standard_normal(shape)
        self.t[name] = ("BF16", bf16_bits(v).reshape(shape))

    def fp8(self, base, rows, K):
        ws = self.rng.uniform(0.004, 0.02)
        self.t[base + ".weight"] = ("F8_E4M3", e4m3_bytes(self.rng.standard_normal((rows, K)) * 0.02 / ws))
        self.t[base + ".weight_scale"] = ("F32", np.array(ws, np.float32).reshape(()))
        self.scalar(base + ".input_scale", 0.02, 0.2)

    def nvfp4(self, base, rows, K, in_scale=None):
        nib = self.rng.integers(0, 16, size=(rows, K), dtype=np.uint8)
        self.t[base + ".weight"] = ("U8", (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8))
        gs = np.exp2(self.rng.uniform(-3, 1, size=(rows, K // 16)))
        self.t[base + ".weight_scale"] = ("F8_E4M3", e4m3_bytes(gs))
        self.t[base + ".weight_scale_2"] = ("F32", np.array(self.rng.uniform(0.002, 0.01), np.float32).reshape(()))
        if in_scale is None:
            self.scalar(base + ".input_scale", 0.02, 0.2)
        else:
            self.t[base + ".input_scale"] = ("F32", np.array(in_scale, np.float32).reshape(()))

    def build(self):
        c, g = self.cfg, self.g
        H, I = g["H"], g["I"]
        for L in range(c.n_layers):
            b = f"{LP}.{L}"
            self.bf16(f"{b}.input_layernorm.weight", (H,), 0.02)
            self.bf16(f"{b}.post_attention_layernorm.weight", (H,), 0.02)
            s_gu = float(self.rng.uniform(0.02, 0.2))
            self.nvfp4(f"{b}.mlp.gate_proj", I, H, s_gu)
            self.nvfp4(f"{b}.mlp.up_proj", I, H, s_gu)
            self.nvfp4(f"{b}.mlp.down_proj", H, I)
            if (L + 1) % c.attn_period == 0:
                s_in = float(self.rng.uniform(0.02, 0.2))
                for n, r in (("q_proj", g["qr"]), ("k_proj", g["kvr"]), ("v_proj", g["kvr"])):
                    self.fp8(f"{b}.self_attn.{n}", r, H)
                    self.t[f"{b}.self_attn.{n}.input_scale"] = ("F32", np.array(s_in, np.float32).reshape(()))
                self.fp8(f"{b}.self_attn.o_proj", H, g["att"])
                self.bf16(f"{b}.self_attn.q_norm.weight", (g["hd"],), 0.02)
                self.bf16(f"{b}.self_attn.k_norm.weight", (g["hd"],), 0.02)
            else:
                self.fp8(f"{b}.linear_attn.in_proj_qkv", g["nqkv"], H)
                self.fp8(f"{b}.linear_attn.in_proj_z", g["nz"], H)
                self.fp8(f"{b}.linear_attn.out_proj", H, g["nz"])
                self.bf16(f"{b}.linear_attn.in_proj_a.weight", (g["vh"], H), 0.02)
                self.bf16(f"{b}.linear_attn.in_proj_b.weight", (g["vh"], H), 0.02)
                self.bf16(f"{b}.linear_attn.conv1d.weight", (g["nqkv"], 1, 4), 0.3)
                self.bf16(f"{b}.linear_attn.A_log", (g["vh"],), 0, uniform=(0.0, 2.7))
                self.bf16(f"{b}.linear_attn.dt_bias", (g["vh"],), 0.1)
                self.bf16(f"{b}.linear_attn.norm.weight", (g["D"],), 0.02, mean=1.0)
        self.bf16("model.language_model.embed_tokens.weight", (g["V"], H), 1.0)
        self.bf16("model.language_model.norm.weight", (H,), 0.02)
        self.nvfp4("lm_head", g["V"], H)
        del self.t["lm_head.input_scale"]
        m = "mtp.layers.0"
        for n, shape in (("self_attn.q_proj", (g["qr"], H)), ("self_attn.k_proj", (g["kvr"], H)),
                         ("self_attn.v_proj", (g["kvr"], H)), ("self_attn.o_proj", (H, g["att"])),
                         ("mlp.gate_proj", (I, H)), ("mlp.up_proj", (I, H)), ("mlp.down_proj", (H, I))):
            self.bf16(f"{m}.{n}.weight", shape, 0.02)
        self.bf16("mtp.fc.weight", (H, 2 * H), 0.02)
        for n in ("input_layernorm", "post_attention_layernorm"):
            self.bf16(f"{m}.{n}.weight", (H,), 0.02)
        self.bf16(f"{m}.self_attn.q_norm.weight", (g["hd"],), 0.02)
        self.bf16(f"{m}.self_attn.k_norm.weight", (g["hd"],), 0.02)
        for n in ("mtp.norm.weight", "mtp.pre_fc_norm_embedding.weight", "mtp.pre_fc_norm_hidden.weight"):
            self.bf16(n, (H,), 0.02)


def write(tensors, path, nshards=3, base=0, metadata=True):
    """safetensors shards model-XXXXX-of-NNNNN (tensors dealt round-robin); returns (count, payload bytes)."""
    os.makedirs(path, exist_ok=True)
    names = sorted(tensors)
    total = 0
    for s in range(nshards):
        mine = names[s::nshards]
        hdr, off, blobs = {}, 0, []
        for n in mine:
            dt, a = tensors[n]
            b = np.ascontiguousarray(a).tobytes()
            hdr[n] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
            off += len(b)
            blobs.append(b)
        if metadata:
            hdr["__metadata__"] = {"format": "pt"}
        h = json.dumps(hdr).encode()
        h += b" " * ((8 - len(h) % 8) % 8)
        with open(os.path.join(path, f"model-{s + base:05d}-of-{nshards:05d}.safetensors"), "wb") as f:
            f.write(len(h).to_bytes(8, "little"))
            f.write(h)
            for b in blobs:
                f.write(b)
        total += off
    return len(names), total


def install_into_oracle(O, m, synth):
    """The checkpoint's weights in the oracle model, converted by the oracle's restatements, and
    each layer's scales (alpha = input_scale x weight_scale per source tensor, input scales)."""
    L_ = O.lib()
    c, g, t = synth.cfg, synth.g, synth.t
    H, I = g["H"], g["I"]

    def arr(n):
        return np.ascontiguousarray(t[n][1])

    def sc(n):
        return float(t[n][1])

    def fp8(base, rows, K):
        w8, s64 = np.empty((rows, K), np.int8), np.empty((rows, K // 64), np.float32)
        L_.q27o_fp8_to_i8g64(arr(base + ".weight").ctypes.data, rows, K, K, w8.ctypes.data, s64.ctypes.data)
        return w8, s64, sc(base + ".input_scale") * sc(base + ".weight_scale")

    def nv(base, rows, K):
        w8, s64 = np.empty((rows, K), np.int8), np.empty((rows, K // 64), np.float32)
        L_.q27o_nvfp4_to_i8g64(arr(base + ".weight").ctypes.data, arr(base + ".weight_scale").ctypes.data, rows, K,
                               w8.ctypes.data, s64.ctypes.data)
        return w8, s64, sc(base + ".input_scale") * sc(base + ".weight_scale_2")

    def bfm(name, rows, K, ld, col0=0):
        src = arr(name).reshape(rows, ld)[:, col0:col0 + K].copy()
        w8, s64 = np.empty((rows, K), np.int8), np.empty((rows, K // 64), np.float32)
        L_.q27o_bf16_to_i8g64(src.ctypes.data, rows, K, K, w8.ctypes.data, s64.ctypes.data)
        return w8, s64

    for L in range(c.n_layers):
        b = f"{LP}.{L}"
        m.set_tensor("in_norm", L, arr(f"{b}.input_layernorm.weight"))
        m.set_tensor("post_norm", L, arr(f"{b}.post_attention_layernorm.weight"))
        gw, gsc, ag = nv(f"{b}.mlp.gate_proj", I, H)
        uw, usc, au = nv(f"{b}.mlp.up_proj", I, H)
        dw, dsc, ad = nv(f"{b}.mlp.down_proj", H, I)
        for n, a in (("gate_w", gw), ("gate_s", gsc), ("up_w", uw), ("up_s", usc), ("down_w", dw), ("down_s", dsc)):
            m.set_tensor(n, L, a)
        s_post, s_down = sc(f"{b}.mlp.gate_proj.input_scale"), sc(f"{b}.mlp.down_proj.input_scale")
        if (L + 1) % c.attn_period == 0:
            qw, qs, aq = fp8(f"{b}.self_attn.q_proj", g["qr"], H)
            kw, ks, ak = fp8(f"{b}.self_attn.k_proj", g["kvr"], H)
            vw, vs, av = fp8(f"{b}.self_attn.v_proj", g["kvr"], H)
            ow, os_, ao = fp8(f"{b}.self_attn.o_proj", H, g["att"])
            m.set_tensor("qkv_w", L, np.concatenate([qw, kw, vw]))
            m.set_tensor("qkv_s", L, np.concatenate([qs, ks, vs]))
            m.set_tensor("o_w", L, ow)
            m.set_tensor("o_s", L, os_)
            m.set_tensor("q_norm", L, arr(f"{b}.self_attn.q_norm.weight"))
            m.set_tensor("k_norm", L, arr(f"{b}.self_attn.k_norm.weight"))
            m.set_scales(L, [aq, ak, av, ao, ag, au, ad, sc(f"{b}.self_attn.q_proj.input_scale"), s_post, s_down,
                             sc(f"{b}.self_attn.o_proj.input_scale")])
        else:
            qw, qs, aq = fp8(f"{b}.linear_attn.in_proj_qkv", g["nqkv"], H)
            zw, zs, az = fp8(f"{b}.linear_attn.in_proj_z", g["nz"], H)
            ow, os_, ao = fp8(f"{b}.linear_attn.out_proj", H, g["nz"])
            m.set_tensor("qkvz_w", L, np.concatenate([qw, zw]))
            m.set_tensor("qkvz_s", L, np.concatenate([qs, zs]))
            m.set_tensor("out_w", L, ow)
            m.set_tensor("out_s", L, os_)
            for n, src in (("in_a", "in_proj_a.weight"), ("in_b", "in_proj_b.weight"), ("A_log", "A_log"),
                           ("dt_bias", "dt_bias"), ("gdn_norm", "norm.weight"), ("conv_w", "conv1d.weight")):
                m.set_tensor(n, L, arr(f"{b}.linear_attn.{src}"))
            m.set_scales(L, [aq, az, 1.0, ao, ag, au, ad, sc(f"{b}.linear_attn.in_proj_qkv.input_scale"), s_post,
                             s_down, sc(f"{b}.linear_attn.out_proj.input_scale")])
    m.set_tensor("emb", -1, arr("model.language_model.embed_tokens.weight"))
    m.set_tensor("final_norm", -1, arr("model.language_model.norm.weight"))
    lm = np.empty((g["V"], H), np.uint16)
    L_.q27o_nvfp4_to_bf16(arr("lm_head.weight").ctypes.data, arr("lm_head.weight_scale").ctypes.data,
                          sc("lm_head.weight_scale_2"), g["V"], H, lm.ctypes.data)
    m.set_tensor("lm_head", -1, lm)
    mb = "mtp.layers.0"
    qw, qs = bfm(f"{mb}.self_attn.q_proj.weight", g["qr"], H, H)
    kw, ks = bfm(f"{mb}.self_attn.k_proj.weight", g["kvr"], H, H)
    vw, vs = bfm(f"{mb}.self_attn.v_proj.weight", g["kvr"], H, H)
    m.set_tensor("qkv_w", -1, np.concatenate([qw, kw, vw]))
    m.set_tensor("qkv_s", -1, np.concatenate([qs, ks, vs]))
    ow, os_ = bfm(f"{mb}.self_attn.o_proj.weight", H, g["att"], g["att"])
    m.set_tensor("o_w", -1, ow)
    m.set_tensor("o_s", -1, os_)
    for n, name in (("gate", "gate_proj"), ("up", "up_proj")):
        w, s_ = bfm(f"{mb}.mlp.{name}.weight", I, H, H)
        m.set_tensor(f"{n}_w", -1, w)
        m.set_tensor(f"{n}_s", -1, s_)
    for j in range(4):
        w, s_ = bfm(f"{mb}.mlp.down_proj.weight", H, I // 4, I, j * (I // 4))
        m.set_tensor(f"down4_w{j}", -1, w)
        m.set_tensor(f"down4_s{j}", -1, s_)
    for j in range(2):
        w, s_ = bfm("mtp.fc.weight", H, H, 2 * H, j * H)
        m.set_tensor(f"fc{j}_w", -1, w)
        m.set_tensor(f"fc{j}_s", -1, s_)
    m.set_tensor("in_norm", -1, arr(f"{mb}.input_layernorm.weight"))
    m.set_tensor("post_norm", -1, arr(f"{mb}.post_attention_layernorm.weight"))
    m.set_tensor("q_norm", -1, arr(f"{mb}.self_attn.q_norm.weight"))
    m.set_tensor("k_norm", -1, arr(f"{mb}.self_attn.k_norm.weight"))
    m.set_tensor("mtp_norm", -1, arr("mtp.norm.weight"))
    m.set_tensor("pre_emb", -1, arr("mtp.pre_fc_norm_embedding.weight"))
    m.set_tensor("pre_hid", -1, arr("mtp.pre_fc_norm_hidden.weight"))
