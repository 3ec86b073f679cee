"""ctypes binding of the CPU oracle (libq27o.so). TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the
product never loads it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq27o.so")
VP, I, F, SZ, U64, D = (ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t,
                        ctypes.c_uint64, ctypes.c_double)


class Cfg(ctypes.Structure):
    _fields_ = [
        ("hidden", I), ("inter", I), ("vocab", I), ("n_layers", I), ("attn_period", I),
        ("gdn_kh", I), ("gdn_vh", I), ("gdn_d", I),
        ("n_q", I), ("n_kv", I), ("head_dim", I), ("attn_gate", I), ("rot_dims", I),
        ("rope_theta", D), ("kv_group", I), ("rms_eps", F),
        ("head_double_residual", I), ("mtp_swap", I), ("mtp_plus_one", I),
        ("spec_k", I), ("ctx", I), ("pf_gs", I),
    ]


_SIGS = {
    "q27o_f2bf": ([F], ctypes.c_uint16), "q27o_bf2f": ([ctypes.c_uint16], F),
    "q27o_exp": ([F], F), "q27o_exp2": ([F], F), "q27o_log1p": ([F], F),
    "q27o_math_vec": ([VP, VP, I, I], None),
    "q27o_hash": ([U64, U64, U64], U64), "q27o_normal": ([U64, U64, U64], F),
    "q27o_uniform": ([U64, U64, U64], F),
    "q27o_quant_rows": ([VP, I, VP, I, VP, I, I, F, I], None),
    "q27o_quant_f32": ([VP, I, I, VP, VP], None),
    "q27o_quant_weights_i8g64": ([VP, I, I, VP, VP], None),
    "q27o_swiglu_quant_rows": ([VP, VP, I, VP, VP, I, F, I], None),
    "q27o_proj_rows": ([VP, VP, F, I, I, VP, I, VP, VP, I, I], None),
    "q27o_proj_partials": ([VP, I, I, VP, I, VP, I], None),
    "q27o_i8g64_to_grp": ([VP, VP, I, I, I, VP, VP], None),
    "q27o_quant_tok_groups": ([VP, I, I, I, I, VP, VP], None),
    "q27o_gemm_i8g_partials": ([VP, I, I, I, VP, I, VP], None),
    "q27o_gemm_i8g": ([VP, VP, I, I, I, F, VP, VP, I, VP, I, VP, I, F], None),
    "q27o_proj_rows_epi": ([VP, VP, F, I, I, VP, I, VP, VP, I, I, VP, I, I, F, I], None),
    "q27o_bf16_gemv_rows": ([VP, I, I, VP, I, VP, I, I], None),
    "q27o_rowsumsq": ([VP, I], F), "q27o_headsum": ([VP, VP, I], F),
    "q27o_rmsnorm_quant_rows": ([VP, I, I, VP, F, F, I, VP, VP, I, VP, VP, I, F, I], None),
    "q27o_gdn_pend_bytes": ([I, I, I, I], SZ),
    "q27o_gdn_verify": ([VP, I, VP, I, VP, VP, I, VP, VP, VP, VP, VP, VP, VP, I, I, I, I, F, VP,
                         I, VP, VP, I], None),
    "q27o_rope_table": ([I, I, D, VP, VP], None),
    "q27o_attn_prep_rows": ([VP, I, VP, VP, VP, VP, I, VP, VP, VP, VP, I, VP, I, I, I, I, F, I,
                             I], None),
    "q27o_attn_rows": ([VP, VP, I, VP, VP, VP, VP, I, I, I, I, I, I, I, VP, VP, VP], None),
    "q27o_argmax_rows": ([VP, I, I, I, VP, VP], None),
    "q27o_accept": ([VP, VP, I, VP], I),
    "q27o_model_create": ([VP, U64], VP), "q27o_model_destroy": ([VP], None),
    "q27o_model_reset": ([VP], None), "q27o_model_prefill": ([VP, VP, I], I),
    "q27o_model_prefill_gemm": ([VP, VP, I, I], I), "q27o_debug_plant": ([I], None),
    "q27o_model_set_scales": ([VP, I, VP], None),
    "q27o_quant_tok_groups_g": ([VP, I, I, I, I, F, VP, VP], None),
    "q27o_e4m3": ([ctypes.c_uint8], F),
    "q27o_fp8_to_i8g64": ([VP, I, I, I, VP, VP], None),
    "q27o_nvfp4_to_i8g64": ([VP, VP, I, I, VP, VP], None),
    "q27o_nvfp4_to_bf16": ([VP, VP, F, I, I, VP], None),
    "q27o_bf16_to_i8g64": ([VP, I, I, I, VP, VP], None),
    "q27o_rmsnorm_f32_rows": ([VP, I, I, VP, F, F, I, VP, VP, I, VP, I, I, I], None),
    "q27o_model_decode_step": ([VP], I), "q27o_model_spec_round": ([VP, VP, VP], I),
    "q27o_model_verify_rows": ([VP, I, VP, VP], I),
    "q27o_model_set_pos": ([VP, I], I),
    "q27o_model_verify_logits": ([VP, I, VP, VP, VP, I], I),
    "q27o_model_verify_trace": ([VP, I, VP, VP, VP, I, VP, VP, VP, VP], I),
    "q27o_model_mtp_pass": ([VP, I, VP, VP, I, I, VP, VP], I),
    "q27o_model_weight_bytes": ([VP], D),
    "q27o_model_tensor": ([VP, ctypes.c_char_p, I, VP], VP),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def ptr(a):
    return None if a is None else a.ctypes.data


def f2bf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf2f(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def cfg_from(c):
    """A q27o config from a q27x Config (or a dict with the same fields)."""
    d = c.as_dict() if hasattr(c, "as_dict") else dict(c)
    d.setdefault("pf_gs", 0)           # (configs recorded before the prefill group setting)
    o = Cfg()
    for f, _ in Cfg._fields_:
        setattr(o, f, d[f])
    return o


class Model:
    def __init__(self, cfg, seed):
        self.cfg = cfg_from(cfg)
        self.m = lib().q27o_model_create(ctypes.byref(self.cfg), seed)
        if not self.m:
            raise RuntimeError("q27o_model_create failed")

    def prefill_gemm(self, ids, chunk=0):
        ids = np.ascontiguousarray(ids, np.int32)
        return lib().q27o_model_prefill_gemm(self.m, ids.ctypes.data, len(ids), chunk)

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        return lib().q27o_model_prefill(self.m, ids.ctypes.data, len(ids))

    def decode_step(self):
        return lib().q27o_model_decode_step(self.m)

    def spec_round(self, forced=None):
        out = np.zeros(8, dtype=np.int32)
        f = None if forced is None else np.ascontiguousarray(forced, dtype=np.int32)
        n = lib().q27o_model_spec_round(self.m, out.ctypes.data, ptr(f))
        return out[:n].tolist()

    def verify_rows(self, toks):
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        nx = np.zeros(8, np.int32)
        lib().q27o_model_verify_rows(self.m, len(toks), toks.ctypes.data, nx.ctypes.data)
        return nx[: len(toks)].tolist()

    def verify_logits(self, toks, advance=True):
        """One verify pass over toks at the current position: (argmax per row, logits [nr][vocab],
        final residual rows [nr][H] bf16 bits); advance commits the rows (pos += nr)."""
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        nr = len(toks)
        nx = np.zeros(8, np.int32)
        lg = np.zeros((nr, self.cfg.vocab), np.float32)
        rc = lib().q27o_model_verify_logits(self.m, nr, toks.ctypes.data, nx.ctypes.data, lg.ctypes.data,
                                             1 if advance else 0)
        if rc:
            raise ValueError("verify_logits: bad row count or position")
        hf = self.tensor("hfinal", -1, np.uint16)[: nr * self.cfg.hidden].reshape(nr, self.cfg.hidden)
        return nx[:nr].tolist(), lg, hf

    def verify_trace(self, toks, advance=True):
        """verify_logits plus, per layer, r1 and r2 (fp32 [n_layers][nr][H]) and the post norm's
        codes [n_layers][nr][H] and per-16 scales [n_layers][nr][H/16]."""
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        nr, nl, H = len(toks), self.cfg.n_layers, self.cfg.hidden
        nx = np.zeros(8, np.int32)
        lg = np.zeros((nr, self.cfg.vocab), np.float32)
        r1, r2 = np.zeros((nl, nr, H), np.float32), np.zeros((nl, nr, H), np.float32)
        pq, ps = np.zeros((nl, nr, H), np.int8), np.zeros((nl, nr, H // 16), np.float32)
        rc = lib().q27o_model_verify_trace(self.m, nr, toks.ctypes.data, nx.ctypes.data, lg.ctypes.data,
                                            1 if advance else 0, r1.ctypes.data, r2.ctypes.data, pq.ctypes.data,
                                            ps.ctypes.data)
        if rc:
            raise ValueError("verify_trace: bad row count or position")
        hf = self.tensor("hfinal", -1, np.uint16)[: nr * H].reshape(nr, H)
        return dict(nx=nx[:nr].tolist(), logits=lg, hfinal=hf, r1=r1, r2=r2, pq=pq, ps=ps)

    def mtp_pass(self, hrows, toks, dpos0, head_row):
        """One MTP pass over rows (hrows [nr][H] bf16 bits, toks [nr]) at draft positions
        dpos0..; returns (argmax of head_row, residual rows [nr][H] bf16, head-row logits)."""
        hrows = np.ascontiguousarray(hrows, dtype=np.uint16)
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        nr = len(toks)
        res = np.zeros((nr, self.cfg.hidden), np.uint16)
        logits = np.zeros(self.cfg.vocab, np.float32)
        t = lib().q27o_model_mtp_pass(self.m, nr, hrows.ctypes.data, toks.ctypes.data, dpos0, head_row,
                                      res.ctypes.data, logits.ctypes.data)
        return t, res, logits

    def tensor(self, name, layer, dtype):
        nb = ctypes.c_size_t(0)
        p = lib().q27o_model_tensor(self.m, name.encode(), layer, ctypes.byref(nb))
        if not p:
            raise KeyError(name)
        n = nb.value // np.dtype(dtype).itemsize
        return np.ctypeslib.as_array((ctypes.c_byte * nb.value).from_address(p)).view(dtype)[:n].copy()

    def set_tensor(self, name, layer, arr):
        """Overwrite a named tensor (weights loaded from a checkpoint); the byte count must match."""
        nb = ctypes.c_size_t(0)
        p = lib().q27o_model_tensor(self.m, name.encode(), layer, ctypes.byref(nb))
        if not p:
            raise KeyError(name)
        a = np.ascontiguousarray(arr)
        if a.nbytes != nb.value:
            raise ValueError(f"{name}: {a.nbytes} bytes for a {nb.value}-byte tensor")
        ctypes.memmove(p, a.ctypes.data, a.nbytes)

    def set_scales(self, layer, v):
        a = np.ascontiguousarray(v, np.float32)
        assert a.size == 11
        lib().q27o_model_set_scales(self.m, layer, a.ctypes.data)

    def close(self):
        if self.m:
            lib().q27o_model_destroy(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
