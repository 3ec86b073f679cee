"""ctypes binding of libq27x.so (include/q27x.h) for tests, smoke and bench.

Device memory and streams go through the library's own plumbing entry points, so no framework is
loaded into the process. Every call checks the status code and raises Q27XError with the
library's last error message. The GPU path has no CPU fallback: without the library (or without a
GPU) the calls fail loudly.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq27x.so")

Q27X_OK = 0
ERRORS = {-1: "ARG", -2: "SHAPE", -3: "HIP", -4: "NOMEM", -5: "STATE", -6: "RANGE", -7: "DEVICE", -8: "IO",
          -9: "FORMAT", -10: "MISSING"}


class Q27XError(RuntimeError):
    def __init__(self, rc, msg):
        super().__init__(f"q27x error {rc} ({ERRORS.get(rc, '?')}): {msg}")
        self.rc = rc


class Config(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("vocab", ctypes.c_int),
        ("n_layers", ctypes.c_int), ("attn_period", ctypes.c_int),
        ("gdn_kh", ctypes.c_int), ("gdn_vh", ctypes.c_int), ("gdn_d", ctypes.c_int),
        ("n_q", ctypes.c_int), ("n_kv", ctypes.c_int), ("head_dim", ctypes.c_int),
        ("attn_gate", ctypes.c_int), ("rot_dims", ctypes.c_int), ("rope_theta", ctypes.c_double),
        ("kv_group", ctypes.c_int), ("rms_eps", ctypes.c_float),
        ("head_double_residual", ctypes.c_int), ("mtp_swap", ctypes.c_int),
        ("mtp_plus_one", ctypes.c_int), ("spec", ctypes.c_int), ("spec_k", ctypes.c_int),
        ("ctx", ctypes.c_int), ("pf_gs", ctypes.c_int), ("eos_id", ctypes.c_int), ("eos_id2", ctypes.c_int),
    ]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


class Stats(ctypes.Structure):
    _fields_ = [
        ("rounds", ctypes.c_longlong), ("committed", ctypes.c_longlong),
        ("accepted", ctypes.c_longlong), ("acc_hist", ctypes.c_longlong * 9),
        ("decode_ms", ctypes.c_double), ("prefill_ms", ctypes.c_double),
        ("draft_ms", ctypes.c_double), ("verify_ms", ctypes.c_double),
        ("head_ms", ctypes.c_double), ("tail_ms", ctypes.c_double),
    ]


class I8G(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("s", ctypes.c_void_p), ("alpha", ctypes.c_float),
                ("rows", ctypes.c_int), ("K", ctypes.c_int)]


_lib = None
VP, I, F, SZ, U64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_uint64

_SIGS = {
    "q27x_last_error": ([], ctypes.c_char_p), "q27x_version": ([], ctypes.c_char_p),
    "q27x_device_count": ([VP], I), "q27x_set_device": ([I], I),
    "q27x_device_name": ([I, ctypes.c_char_p, I], I), "q27x_device_cus": ([I, VP], I),
    "q27x_malloc": ([VP, SZ], I), "q27x_free": ([VP], I),
    "q27x_host_malloc": ([VP, SZ], I), "q27x_host_free": ([VP], I),
    "q27x_memcpy_h2d": ([VP, VP, SZ, VP], I), "q27x_memcpy_d2h": ([VP, VP, SZ, VP], I),
    "q27x_memcpy_d2d": ([VP, VP, SZ, VP], I), "q27x_memset": ([VP, I, SZ, VP], I),
    "q27x_stream_create": ([VP], I), "q27x_stream_destroy": ([VP], I),
    "q27x_stream_sync": ([VP], I), "q27x_device_sync": ([], I),
    "q27x_event_create": ([VP], I), "q27x_event_destroy": ([VP], I),
    "q27x_event_record": ([VP, VP], I), "q27x_event_elapsed_ms": ([VP, VP, VP], I),
    "q27x_quant_rows": ([VP, I, VP, I, VP, I, I, F, I, VP], I),
    "q27x_quant_weights_i8g64": ([VP, I, I, VP, VP, VP], I),
    "q27x_proj_rows": ([VP, VP, I, VP, VP, I, I, VP, I, I, F, I, VP], I),
    "q27x_proj_partials": ([VP, VP, I, VP, I, VP], I),
    "q27x_i8g64_to_grp": ([VP, VP, I, I, I, VP, VP, VP], I),
    "q27x_quant_tok_groups": ([VP, I, I, I, I, VP, VP, VP], I),
    "q27x_gemm_i8g": ([VP, VP, I, I, I, F, VP, VP, I, VP, I, VP, I, F, VP], I),
    "q27x_bf16_gemv_rows": ([VP, I, I, VP, I, VP, I, I, I, VP], I),
    "q27x_rmsnorm_quant_rows": ([VP, I, I, VP, F, F, I, VP, VP, I, VP, VP, I, F, I, VP], I),
    "q27x_swiglu_quant_rows": ([VP, VP, I, VP, VP, I, F, I, VP], I),
    "q27x_gdn_pend_bytes": ([I, I, I, I], SZ),
    "q27x_gdn_verify": ([VP, I, VP, I, VP, VP, I, VP, VP, VP, VP, VP, VP, VP, I, I, I, I, VP, I,
                         VP, VP, I, VP], I),
    "q27x_attn_prep_rows": ([VP, I, VP, VP, VP, VP, I, VP, VP, VP, VP, I, VP, I, I, I, I, F, I,
                             I, VP], I),
    "q27x_attn_work_bytes": ([I, I, I, I], SZ),
    "q27x_attn_rows": ([VP, VP, I, VP, VP, VP, VP, I, I, I, I, I, I, I, VP, VP, VP, VP, VP], I),
    "q27x_attn_rows_noalloc": ([VP, VP, I, VP, VP, VP, VP, I, I, I, I, I, I, I, VP, VP, VP, VP], I),
    "q27x_argmax_rows": ([VP, I, I, I, VP, VP, VP], I),
    "q27x_accept": ([VP, VP, I, VP, VP, VP], I),
    "q27x_math_test": ([VP, VP, I, I, VP], I),
    "q27x_config_default": ([VP], I), "q27x_config_tiny": ([VP], I),
    "q27x_spec_config_from_env": ([VP], I),
    "q27x_ctx_create": ([I, VP, VP], I), "q27x_ctx_destroy": ([VP], I),
    "q27x_load_synthetic": ([VP, U64], I), "q27x_weight_bytes": ([VP, VP], I),
    "q27x_reset": ([VP], I), "q27x_prefill": ([VP, VP, I, VP], I), "q27x_prefill_gemm": ([VP, VP, I, VP], I),
    "q27x_decode_step": ([VP, VP], I), "q27x_spec_round": ([VP, VP, VP], I),
    "q27x_set_forced_drafts": ([VP, VP, I], I),
    "q27x_mtp_draft": ([VP, VP, VP, I, I, I, VP, VP, VP], I),
    "q27x_gdn_commit": ([VP, VP, VP, I, I, I, I, VP], I),
    "q27x_generate": ([VP, I, I, VP, VP, VP], I),
    "q27x_bench_verify": ([VP, I, I, VP], I),
    "q27x_run_rounds": ([VP, I, I, VP], I),
    "q27x_bench_kernel": ([VP, I, I, I, I, VP, VP], I),
    "q27x_bench_mixer": ([VP, I, I, I, I, VP, VP], I),
    "q27x_debug_read": ([VP, ctypes.c_char_p, I, VP, SZ], I),
    "q27x_bench_stream": ([I, SZ, I, I, I, VP], I),
    # checkpoint catalog and upload
    "q27x_ckpt_open": ([ctypes.c_char_p, VP, SZ], VP),
    "q27x_ckpt_open_census": ([ctypes.c_char_p, I, ctypes.c_longlong, ctypes.c_longlong, VP, SZ], VP),
    "q27x_ckpt_close": ([VP], None), "q27x_ckpt_tensor_count": ([VP], I),
    "q27x_ckpt_payload_bytes": ([VP], ctypes.c_longlong),
    "q27x_ckpt_host_ptr": ([VP, ctypes.c_char_p, VP, VP, VP, VP], VP),
    "q27x_ckpt_name": ([VP, I], ctypes.c_char_p),
    "q27x_ckpt_info": ([VP, I, VP, VP, VP, VP, VP, VP], I),
    "q27x_ckpt_check": ([VP, VP, VP, SZ], I), "q27x_load_checkpoint": ([VP, VP, VP, SZ], I),
}


def lib():
    """Load libq27x.so once (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Q27XError(-5, f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def check(rc):
    if rc != Q27X_OK:
        raise Q27XError(rc, lib().q27x_last_error().decode())
    return rc


def call(name, *args):
    return check(getattr(lib(), name)(*args))


def gpu_count():
    n = ctypes.c_int(0)
    rc = lib().q27x_device_count(ctypes.byref(n))
    return n.value if rc == 0 else 0


class DevBuf:
    """A device allocation holding one numpy array's bytes."""

    def __init__(self, nbytes=None, array=None):
        if array is not None:
            array = np.ascontiguousarray(array)
            nbytes = array.nbytes
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        call("q27x_malloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value
        if array is not None:
            self.upload(array)

    def upload(self, array):
        array = np.ascontiguousarray(array)
        assert array.nbytes <= self.nbytes
        call("q27x_memcpy_h2d", self.ptr, array.ctypes.data, array.nbytes, None)

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        call("q27x_memcpy_d2h", out.ctypes.data, self.ptr, out.nbytes, None)
        return out

    def zero(self):
        call("q27x_memset", self.ptr, 0, self.nbytes, None)
        call("q27x_device_sync")

    def free(self):
        if self.ptr:
            lib().q27x_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def default_config(**kw):
    c = Config()
    call("q27x_config_default", ctypes.byref(c))
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def tiny_config(**kw):
    c = Config()
    call("q27x_config_tiny", ctypes.byref(c))
    for k, v in kw.items():
        setattr(c, k, v)
    return c


class Checkpoint:
    """A mapped checkpoint catalog (q27x_ckpt_open_census); raises Q27XError with the reason."""

    def __init__(self, path, nshards=3, tensors=-1, payload_bytes=-1):
        err = ctypes.create_string_buffer(512)
        p = lib().q27x_ckpt_open_census(str(path).encode(), nshards, tensors, payload_bytes, err, len(err))
        if not p:
            msg = err.value.decode()
            raise Q27XError(-8 if msg.startswith(("open(", "fstat(", "mmap(")) else -9, msg)
        self.ck = p

    def tensor_count(self):
        return lib().q27x_ckpt_tensor_count(self.ck)

    def payload_bytes(self):
        return lib().q27x_ckpt_payload_bytes(self.ck)

    def names(self):
        return [lib().q27x_ckpt_name(self.ck, i).decode() for i in range(self.tensor_count())]

    def check(self, cfg):
        err = ctypes.create_string_buffer(512)
        rc = lib().q27x_ckpt_check(self.ck, ctypes.byref(cfg), err, len(err))
        return rc, err.value.decode()

    def close(self):
        if self.ck:
            lib().q27x_ckpt_close(self.ck)
            self.ck = None


class Engine:
    """Owns one q27x context (weights, KV, GDN state, scratch) on one device."""

    def __init__(self, cfg, seed=0x51E70003, device=0):
        self.cfg = cfg
        p = ctypes.c_void_p()
        call("q27x_ctx_create", device, ctypes.byref(cfg), ctypes.byref(p))
        self.ctx = p.value
        call("q27x_load_synthetic", self.ctx, seed)

    def load_synthetic(self, seed):
        call("q27x_load_synthetic", self.ctx, seed)

    def load_checkpoint(self, ck):
        err = ctypes.create_string_buffer(512)
        rc = lib().q27x_load_checkpoint(self.ctx, ck.ck, err, len(err))
        if rc != Q27X_OK:
            raise Q27XError(rc, err.value.decode())

    def weight_bytes(self):
        b = ctypes.c_size_t(0)
        call("q27x_weight_bytes", self.ctx, ctypes.byref(b))
        return b.value

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        t = ctypes.c_int32(0)
        call("q27x_prefill", self.ctx, ids.ctypes.data, len(ids), ctypes.byref(t))
        return t.value

    def prefill_gemm(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        t = ctypes.c_int32(0)
        call("q27x_prefill_gemm", self.ctx, ids.ctypes.data, len(ids), ctypes.byref(t))
        return t.value

    def decode_step(self):
        t = ctypes.c_int32(0)
        call("q27x_decode_step", self.ctx, ctypes.byref(t))
        return t.value

    def spec_round(self):
        out = np.zeros(8, dtype=np.int32)
        n = ctypes.c_int(0)
        call("q27x_spec_round", self.ctx, out.ctypes.data, ctypes.byref(n))
        return out[: n.value].tolist()

    def set_forced(self, toks):
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        call("q27x_set_forced_drafts", self.ctx, toks.ctypes.data if len(toks) else None, len(toks))

    def generate(self, max_new, spec=True):
        out = np.zeros(max_new, dtype=np.int32)
        n = ctypes.c_int(0)
        st = Stats()
        call("q27x_generate", self.ctx, max_new, 1 if spec else 0, out.ctypes.data, ctypes.byref(n),
             ctypes.byref(st))
        return out[: n.value].tolist(), st

    def run_rounds(self, n, spec=True):
        st = Stats()
        call("q27x_run_rounds", self.ctx, n, 1 if spec else 0, ctypes.byref(st))
        return st

    def bench_verify(self, nr, iters):
        ms = ctypes.c_float(0)
        call("q27x_bench_verify", self.ctx, nr, iters, ctypes.byref(ms))
        return ms.value

    def bench_kernel(self, layer, which, nr, iters):
        ms = ctypes.c_float(0)
        b = ctypes.c_double(0)
        call("q27x_bench_kernel", self.ctx, layer, which, nr, iters, ctypes.byref(ms), ctypes.byref(b))
        return ms.value, b.value

    def mtp_draft(self, hrows, toks, dpos0, head_row):
        """One MTP pass (q27x_mtp_draft) on host arrays: hrows [nr][hidden] bf16 bits, toks [nr];
        returns (head-row argmax or None, residual rows [nr][hidden] bf16)."""
        hrows = np.ascontiguousarray(hrows, dtype=np.uint16)
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        nr = len(toks)
        dh, dt = DevBuf(array=hrows), DevBuf(array=toks)
        dres, dtok = DevBuf(nr * self.cfg.hidden * 2), DevBuf(4)
        call("q27x_mtp_draft", self.ctx, dh.ptr, dt.ptr, nr, dpos0, head_row, dres.ptr,
             dtok.ptr if head_row >= 0 else None, None)
        call("q27x_device_sync")
        res = dres.download(np.uint16, (nr, self.cfg.hidden))
        tok = int(dtok.download(np.int32, (1,))[0]) if head_row >= 0 else None
        for b in (dh, dt, dres, dtok):
            b.free()
        return tok, res

    def bench_mixer(self, attn, pos, nr, iters):
        ms = ctypes.c_float(0)
        b = ctypes.c_double(0)
        call("q27x_bench_mixer", self.ctx, 1 if attn else 0, pos, nr, iters, ctypes.byref(ms), ctypes.byref(b))
        return ms.value, b.value

    def read(self, name, layer, dtype, count):
        out = np.empty(count, dtype=dtype)
        call("q27x_debug_read", self.ctx, name.encode(), layer, out.ctypes.data, out.nbytes)
        return out

    def close(self):
        if self.ctx:
            lib().q27x_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
