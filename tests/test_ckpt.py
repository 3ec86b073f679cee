"""The checkpoint catalog, its fail-closed census and tensor plan (q27x_ckpt_*, reference
q27_open / tp_plan, src/q27_load.cpp:428-494, 690-815), and the oracle's restatements of the
load-time converters (src/q27_nvfp4.hip:4166-4311) pinned against independent decoders: torch's
float8_e4m3fn for E4M3 bytes, the E2M1 value from its bit fields (OCP MX definition), the
pinned per-64 weight rule for the int8 mirror, torch's bfloat16 rounding for the bf16 lm_head.
All host-side: no GPU."""
import json
import os

import numpy as np
import pytest
import torch

import ckpt_synth as CS

E_IO, E_FORMAT, E_MISSING, E_SHAPE = -8, -9, -10, -2


@pytest.fixture(scope="module")
def synth(X):
    return CS.Synth(X.tiny_config(spec_k=2, n_layers=4), seed=3)


@pytest.fixture(scope="module")
def ckdir(tmp_path_factory, synth):
    d = tmp_path_factory.mktemp("ck")
    n, b = CS.write(synth.t, d)
    return d, n, b


def open_ck(X, d, n=-1, b=-1, nshards=3):
    return X.Checkpoint(d, nshards, n, b)


def test_catalog_census_and_host_pointers(X, ckdir, synth):
    d, n, b = ckdir
    ck = open_ck(X, d, n, b)
    assert ck.tensor_count() == n and ck.payload_bytes() == b
    assert sorted(ck.names()) == sorted(synth.t)
    name = "model.language_model.layers.0.mlp.gate_proj.weight_scale_2"
    nb, dt, nd = X.ctypes.c_size_t(0), X.ctypes.c_int(0), X.ctypes.c_int(0)
    shape = (X.ctypes.c_longlong * 8)()
    p = X.lib().q27x_ckpt_host_ptr(ck.ck, name.encode(), X.ctypes.byref(nb), X.ctypes.byref(dt), X.ctypes.byref(nd), shape)
    assert p and nb.value == 4 and dt.value == 3 and nd.value == 0            # F32 scalar
    assert np.frombuffer((X.ctypes.c_char * 4).from_address(p), np.float32)[0] == synth.t[name][1]
    ck.close()


def test_census_fails_closed(X, ckdir):
    d, n, b = ckdir
    for kw, msg in (((n + 1, b), "tensors"), ((n, b - 1), "bytes of tensor data")):
        with pytest.raises(X.Q27XError) as e:
            open_ck(X, d, *kw)
        assert "census" in str(e.value) and msg in str(e.value)
    with pytest.raises(X.Q27XError) as e:
        open_ck(X, d, nshards=4)                                    # shard 3 of 4 does not exist
    assert "cannot open" in str(e.value)


def test_shards_numbered_from_one(X, tmp_path, synth):
    n, b = CS.write(synth.t, tmp_path, base=1)
    ck = open_ck(X, tmp_path, n, b)
    assert ck.tensor_count() == n
    ck.close()


def corrupt(tmp_path, header_edit=None, raw=None):
    t = {"a": ("F32", np.arange(4, dtype=np.float32)), "b": ("BF16", np.zeros((2, 3), np.uint16))}
    CS.write(t, tmp_path, nshards=1)
    p = os.path.join(tmp_path, "model-00000-of-00001.safetensors")
    data = open(p, "rb").read()
    hl = int.from_bytes(data[:8], "little")
    hdr = json.loads(data[8:8 + hl])
    if header_edit:
        header_edit(hdr)
        h = json.dumps(hdr).encode()
        data = len(h).to_bytes(8, "little") + h + data[8 + hl:]
    if raw:
        data = raw(data)
    open(p, "wb").write(data)
    return tmp_path


@pytest.mark.parametrize("case,want", [
    ("offsets_outside", "outside"), ("shape_bytes", "shape needs"), ("dtype", "unknown dtype"),
    ("no_offsets", "required"), ("header_len", "header length field"), ("not_json", "not a JSON object"),
    ("duplicate", "duplicate")])
def test_header_checks_fail_closed(X, tmp_path, case, want):
    edits = {
        "offsets_outside": dict(header_edit=lambda h: h["b"].__setitem__("data_offsets", [16, 4096])),
        "shape_bytes": dict(header_edit=lambda h: h["b"].__setitem__("shape", [3, 3])),
        "dtype": dict(header_edit=lambda h: h["a"].__setitem__("dtype", "F7")),
        "no_offsets": dict(header_edit=lambda h: h["a"].pop("data_offsets")),
        "header_len": dict(raw=lambda d: (10 ** 9).to_bytes(8, "little") + d[8:]),
        "not_json": dict(raw=lambda d: d[:8] + b"[" + d[9:]),
        "duplicate": dict(raw=lambda d: d.replace(b'"b"', b'"a"', 1)),
    }
    d = corrupt(tmp_path, **edits[case])
    with pytest.raises(X.Q27XError) as e:
        open_ck(X, d, nshards=1)
    assert want in str(e.value), str(e.value)


def test_plan_check(X, ckdir, synth, tmp_path):
    d, n, b = ckdir
    ck = open_ck(X, d, n, b)
    assert ck.check(synth.cfg) == (0, "")
    # another geometry: the shapes do not match
    rc, msg = ck.check(X.tiny_config(spec_k=2, n_layers=4, hidden=2048))
    assert rc == E_SHAPE and "expected" in msg
    ck.close()
    # a missing tensor, a wrong dtype, gate / up input scales that differ, a non-positive scale
    t = dict(synth.t)
    for mutate, want_rc, want in (
            (lambda t: t.pop("model.language_model.layers.1.linear_attn.A_log"), E_MISSING, "A_log"),
            (lambda t: t.__setitem__("model.language_model.norm.weight", ("F32", np.zeros(synth.g["H"], np.float32))),
             E_SHAPE, "norm.weight"),
            (lambda t: t.__setitem__("model.language_model.layers.2.mlp.up_proj.input_scale",
                                     ("F32", np.array(0.5, np.float32).reshape(()))), E_SHAPE, "gate input_scale"),
            (lambda t: t.__setitem__("lm_head.weight_scale_2", ("F32", np.array(-1.0, np.float32).reshape(()))),
             E_SHAPE, "positive")):
        tt = dict(t)
        mutate(tt)
        dd = tmp_path / f"m{want_rc}{len(want)}"
        CS.write(tt, dd)
        ck = open_ck(X, dd)
        rc, msg = ck.check(synth.cfg)
        ck.close()
        assert rc == want_rc and want in msg, (rc, msg)


# ---------------------------------------------------------------- converters
def test_e4m3_decoder_matches_torch(O):
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([O.lib().q27o_e4m3(int(c)) for c in codes], np.float32)
    nan = (codes & 0x7F) == 0x7F                      # OCP NaN; the reference decodes it as infinity
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.isinf(got[nan]).all() and (np.sign(got[nan]) == np.where(codes[nan] & 0x80, -1, 1)).all()
    assert got[0x38] == 1.0 and got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9


def e2m1_from_bits(nib):
    s, e, m = (nib >> 3) & 1, (nib >> 1) & 3, nib & 1
    mag = np.where(e == 0, m * 0.5, np.exp2(e.astype(np.float64) - 1) * (1 + m / 2))
    return np.where(s == 1, -mag, mag)


def pinned_i8g64(O, v):
    rows, K = v.shape
    w8, s64 = np.empty((rows, K), np.int8), np.empty((rows, K // 64), np.float32)
    O.lib().q27o_quant_weights_i8g64(np.ascontiguousarray(v, np.float32).ctypes.data, rows, K, w8.ctypes.data,
                                     s64.ctypes.data)
    return w8, s64


def test_fp8_and_nvfp4_converters(O):
    rng = np.random.default_rng(5)
    rows, K = 24, 256
    f8 = CS.e4m3_bytes(rng.standard_normal((rows, K)) * 3)
    w8, s64 = np.empty((rows, K), np.int8), np.empty((rows, K // 64), np.float32)
    O.lib().q27o_fp8_to_i8g64(f8.ctypes.data, rows, K, K, w8.ctypes.data, s64.ctypes.data)
    r8, rs = pinned_i8g64(O, torch.from_numpy(f8).view(torch.float8_e4m3fn).float().numpy())
    assert np.array_equal(w8, r8) and np.array_equal(s64.view(np.uint32), rs.view(np.uint32))
    nib = rng.integers(0, 16, (rows, K)).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    gsv = np.exp2(rng.uniform(-3, 1, (rows, K // 16)))
    gsb = CS.e4m3_bytes(gsv)
    O.lib().q27o_nvfp4_to_i8g64(packed.ctypes.data, gsb.ctypes.data, rows, K, w8.ctypes.data, s64.ctypes.data)
    gdec = torch.from_numpy(gsb).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    v = (e2m1_from_bits(nib) * np.repeat(gdec, 16, axis=1)).astype(np.float32)   # exact: <= 5 significant bits
    r8, rs = pinned_i8g64(O, v)
    assert np.array_equal(w8, r8) and np.array_equal(s64.view(np.uint32), rs.view(np.uint32))
    ws2 = np.float32(0.0037)
    out = np.empty((rows, K), np.uint16)
    O.lib().q27o_nvfp4_to_bf16(packed.ctypes.data, gsb.ctypes.data, float(ws2), rows, K, out.ctypes.data)
    ref = CS.bf16_bits(v.astype(np.float32) * ws2)
    assert np.array_equal(out, ref)


def test_bf16_converter(O):
    rng = np.random.default_rng(6)
    rows, ld, K = 8, 384, 256
    x = CS.bf16_bits(rng.standard_normal((rows, ld)) * 0.02)
    w8, s64 = np.empty((rows, K), np.int8), np.empty((rows, K // 64), np.float32)
    sub = np.ascontiguousarray(x[:, 64:64 + K])
    tail = x[:, 64:].copy()                              # columns 64.. with row stride ld - 64
    O.lib().q27o_bf16_to_i8g64(tail.ctypes.data, rows, K, ld - 64, w8.ctypes.data, s64.ctypes.data)
    r8, rs = pinned_i8g64(O, torch.from_numpy(sub.view(np.int16)).view(torch.bfloat16).float().numpy())
    assert np.array_equal(w8, r8) and np.array_equal(s64.view(np.uint32), rs.view(np.uint32))
