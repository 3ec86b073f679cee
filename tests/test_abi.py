"""C-ABI checks that need no GPU: libq27x.so loads, exports every function include/q27x.h
declares, and the host-side argument checks and the Q27_SPEC / Q27_SPEC_K parser behave like the
reference's (include/q27.h:189-206, src/q27_main.cpp:3360-3361)."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "q27x.h")


def declared():
    src = open(HDR).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(q27x_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported(X):
    names = declared()
    assert len(names) >= 50
    L = X.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", X.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    assert not [n for n in names if n not in exported]


def test_binding_signatures_cover_the_header(X):
    """The ctypes table names exactly the header's functions (no stale or missing binding)."""
    assert sorted(X._SIGS) == declared()


def test_library_has_gfx950_code_object(X):
    data = open(X.LIB_PATH, "rb").read()
    assert b"gfx950" in data
    assert b"gfx906" not in data


def test_version_and_error_strings(X):
    assert X.lib().q27x_version()
    assert X.lib().q27x_last_error() is not None


def test_argument_errors_without_gpu(X):
    """Null pointers and bad row counts are rejected on the host, before any HIP call."""
    L = X.lib()
    assert L.q27x_quant_rows(None, 16, None, 16, None, 1, 16, 1.0, 1, None) == -1
    h = X.I8G(None, None, 1.0, 64, 64)
    assert L.q27x_proj_rows(ctypes.byref(h), None, 64, None, None, 64, 0, None, 0, 0, 0.0, 1, None) == -1
    assert L.q27x_ctx_create(0, None, None) == -1
    err = L.q27x_last_error().decode()
    assert "q27x_ctx_create" in err


def test_ctx_create_rejects_unsupported_geometry(X):
    c = X.default_config()
    c.gdn_d = 64
    p = ctypes.c_void_p()
    assert X.lib().q27x_ctx_create(0, ctypes.byref(c), ctypes.byref(p)) == -2
    assert p.value is None
    c = X.default_config(spec_k=8)
    assert X.lib().q27x_ctx_create(0, ctypes.byref(c), ctypes.byref(p)) == -2
    # an input width the projection kernels have no instance for (3 x 1024) is refused up front
    c = X.tiny_config(inter=3072)
    assert X.lib().q27x_ctx_create(0, ctypes.byref(c), ctypes.byref(p)) == -2
    assert "input width of 3072" in X.lib().q27x_last_error().decode()
    assert p.value is None


def test_default_config_is_baseline_config3(X):
    c = X.default_config()
    assert (c.hidden, c.inter, c.vocab, c.n_layers, c.attn_period) == (5120, 17408, 62080, 64, 4)
    assert (c.gdn_kh, c.gdn_vh, c.gdn_d) == (16, 48, 128)
    assert (c.n_q, c.n_kv, c.head_dim, c.kv_group) == (32, 8, 128, 32)
    assert c.rope_theta == 1e7
    n_attn = sum(1 for L in range(c.n_layers) if L % c.attn_period == c.attn_period - 1)
    assert n_attn == 16


def _env_config(env):
    code = ("import sys, ctypes; sys.path.insert(0, %r); import importlib.util as u;"
            "s = u.spec_from_file_location('q27x', %r); m = u.module_from_spec(s); s.loader.exec_module(m);"
            "c = m.default_config(); m.call('q27x_spec_config_from_env', ctypes.byref(c));"
            "print(c.spec, c.spec_k, c.pf_gs, c.eos_id, c.eos_id2)") % (ROOT, os.path.join(ROOT, "qwen3.8-27b-mi50-cpp-engine_amd", "q27x.py"))
    e = {k: v for k, v in os.environ.items() if not k.startswith("Q27_")}
    e.update(env)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=e, timeout=120)


@pytest.mark.parametrize("env,expect", [
    ({}, (1, 1)),                                   # defaults: spec on, K = 1 (src/q27_main.cpp:3360-3361)
    ({"Q27_SPEC": "0"}, (0, 1)),
    ({"Q27_SPEC": "off", "Q27_SPEC_K": "2"}, (0, 2)),
    ({"Q27_SPEC": "yes", "Q27_SPEC_K": "7"}, (1, 7)),
    ({"Q27_SPEC_K": "0"}, (1, 1)),                  # clamped to [1, 7]
    ({"Q27_SPEC_K": "-3"}, (1, 1)),
    ({"Q27_SPEC_K": "12"}, (1, 7)),
    ({"Q27_SPEC": ""}, (1, 1)),                     # empty = unset
])
def test_spec_env_semantics(env, expect):
    r = _env_config(env)
    assert r.returncode == 0, r.stderr
    assert tuple(int(v) for v in r.stdout.split())[:2] == expect


@pytest.mark.parametrize("env,expect", [({}, 0), ({"Q27_Q8_GS": "0"}, 0), ({"Q27_Q8_GS": "1024"}, 1024),
                                        ({"Q27_Q8_GS": ""}, 0)])
def test_prefill_group_env(env, expect):
    """Q27_Q8_GS (src/q27_load.cpp:1623, src/q27_main.cpp:4020): 0 = the whole K, the default; 1024."""
    r = _env_config(env)
    assert r.returncode == 0, r.stderr
    assert int(r.stdout.split()[2]) == expect


@pytest.mark.parametrize("env,expect", [({}, (248044, -1)), ({"Q27_EOS_IM_END": "1"}, (248044, 248046)),
                                        ({"Q27_EOS_IM_END": "0"}, (248044, -1))])
def test_stop_token_env(env, expect):
    """q27_is_eos (src/q27_main.cpp:709-710): 248044 always, <|im_end|> 248046 with Q27_EOS_IM_END."""
    r = _env_config(env)
    assert r.returncode == 0, r.stderr
    assert tuple(int(v) for v in r.stdout.split()[3:5]) == expect


@pytest.mark.parametrize("env", [{"Q27_SPEC": "maybe"}, {"Q27_SPEC_K": "2x"}, {"Q27_SPEC_K": "two"},
                                 {"Q27_Q8_GS": "512"}, {"Q27_Q8_GS": "full"}, {"Q27_EOS_IM_END": "sometimes"}])
def test_spec_env_fails_closed(env):
    """An unparseable value prints FATAL and aborts (include/q27.h:189-206), never guesses."""
    r = _env_config(env)
    assert r.returncode != 0
    assert "FATAL" in r.stderr
