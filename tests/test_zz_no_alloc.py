"""The allocation-free attention entry point q27x_attn_rows_noalloc (split partials in the
library's file-scope device array) against q27x_attn_rows (partials in a caller-owned work
buffer), through the C ABI: bit-identical outputs, codes and scales on two calls in a row, the
second smaller than the first (so stale partials of the first call sit in the array), and a call
past the array's limit rejected on the host."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NQ, NKV, HD, GROUP = 32, 8, 128, 32


def kv_cache(rng, O, L, ctx):
    kv = NKV * HD
    out = []
    for _ in range(2):
        x = rng.standard_normal((L, kv)).astype(np.float32)
        q = np.zeros((ctx, kv), np.int8)
        s = np.zeros((ctx, kv // GROUP), np.float32)
        qq, ss = np.empty(L * kv, np.int8), np.empty(L * kv // GROUP, np.float32)
        O.lib().q27o_quant_f32(x.ctypes.data, L * kv, GROUP, qq.ctypes.data, ss.ctypes.data)
        q[:L], s[:L] = qq.reshape(L, kv), ss.reshape(L, kv // GROUP)
        out += [q, s]
    return out


def run_pair(X, O, rng, L0, nr):
    ctx = L0 + nr
    kc, ks, vc, vs = kv_cache(rng, O, ctx, ctx)          # the rows' own positions are filled too
    qh = O.f2bf(rng.standard_normal((nr, NQ * HD)).astype(np.float32))
    qkv_rows = NQ * 2 * HD + 2 * NKV * HD
    gate = O.f2bf(rng.standard_normal((nr, qkv_rows)).astype(np.float32))
    bufs = [X.DevBuf(array=a) for a in (qh, gate, kc, ks, vc, vs)]
    dqh, dg, dk, dks, dv, dvs = (b.ptr for b in bufs)
    n = nr * NQ * HD
    res = []
    for noalloc in (False, True):
        out, xq, xs = X.DevBuf(n * 2), X.DevBuf(n), X.DevBuf(n // 4)
        if noalloc:
            X.call("q27x_attn_rows_noalloc", dqh, dg, qkv_rows, dk, dks, dv, dvs, GROUP, NQ, NKV, HD, 1, L0, nr,
                   out.ptr, xq.ptr, xs.ptr, None)
        else:
            work = X.DevBuf(X.lib().q27x_attn_work_bytes(NQ, HD, ctx, nr))
            X.call("q27x_attn_rows", dqh, dg, qkv_rows, dk, dks, dv, dvs, GROUP, NQ, NKV, HD, 1, L0, nr, work.ptr,
                   out.ptr, xq.ptr, xs.ptr, None)
        X.call("q27x_device_sync")
        res.append((out.download(np.uint16, (nr, NQ * HD)), xq.download(np.int8, (nr, NQ * HD)),
                    xs.download(np.float32, (nr, NQ * HD // 16))))
        for b in (out, xq, xs):
            b.free()
        if not noalloc:
            work.free()
    for b in bufs:
        b.free()
    (o0, q0, s0), (o1, q1, s1) = res
    assert np.array_equal(o1, o0), f"L0={L0} nr={nr}: outputs differ"
    assert np.array_equal(q1, q0), f"L0={L0} nr={nr}: codes differ"
    assert np.array_equal(s1.view(np.uint32), s0.view(np.uint32)), f"L0={L0} nr={nr}: scales differ"


def test_noalloc_attention_matches_the_work_buffer_entry(gpu, O):
    X = gpu
    rng = np.random.default_rng(0x51E7B000)
    print("no-alloc: call 1, 8 rows at 16376 (the array's full size)", flush=True)
    run_pair(X, O, rng, 16376, 8)
    print("no-alloc: call 2, 3 rows at 1021 (smaller, stale partials in the array)", flush=True)
    run_pair(X, O, rng, 1021, 3)


def test_noalloc_attention_rejects_calls_past_its_limit(gpu):
    X = gpu
    small = [X.DevBuf(4096) for _ in range(9)]
    p = [b.ptr for b in small]
    # 8 rows x 32 heads x ceil((16377 + 8) / 64) = 257 splits > 65536 triples: refused on the host
    rc = X.lib().q27x_attn_rows_noalloc(p[0], p[1], 8192, p[2], p[3], p[4], p[5], GROUP, NQ, NKV, HD, 1, 16377, 8,
                                        p[6], p[7], p[8], None)
    assert rc == -6, rc
    assert "scratch" in X.lib().q27x_last_error().decode()
    for b in small:
        b.free()
