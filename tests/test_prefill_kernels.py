"""Prefill-shaped twins of the decode kernels (kernels/llm_sampling.cl:496-736)
and the reference's own checks of them (examples/llm/sampling_test.cpp:
725-1016): T = 37 rows (not a multiple of 64), 4 query heads over 1 KV head,
head_dim 256, hidden 1152; softmax rows sum to 1; the causal and sliding-window
(8) masks; "prefill == decode" (one query at q_offset = pos reproduces the
decode scores, RMSNorm, QK-norm and RoPE); the plumbing copies.

CPU: the oracle's twins against float64 closed forms and, bit for bit, against
the oracle's decode kernels where the reference compares the two paths. GPU:
each product kernel against the oracle (sentinel-prefilled outputs: every
element written), rtol 1e-5 of the largest magnitude for arithmetic, exact for
masks and copies; a whole one-query prefill attention against the product's
decode attention over the same fp16 values."""
import ctypes as C

import numpy as np
import pytest

T, SEQ, HEADS, KVH, HD, HIDDEN, EPS = 37, 37, 4, 1, 256, 1152, 1e-6
SCALE = 1.0 / 16.0
SENTINEL = np.float32(-1.0e30)


def rnd(n, seed, lo=-1.0, hi=1.0):
    return np.random.default_rng(seed).uniform(lo, hi, n).astype(np.float32)


def f16r(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def np_scores(q, k, n_query, q_offset, window):
    q = q.reshape(HEADS, n_query, HD).astype(np.float64)
    k = k.reshape(SEQ, KVH, HD).astype(np.float64)
    s = np.einsum("hqd,td->hqt", q, k[:, 0, :]) * SCALE
    t = np.arange(SEQ)[None, :]
    qpos = q_offset + np.arange(n_query)[:, None]
    mask = (t > qpos) | ((window != 0) & (t + window <= qpos))
    s = np.where(mask[None], -np.inf, s)
    return s, mask


def rel(got, want):
    want = np.asarray(want, np.float64)
    return np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30)


# ---------------------------------------------------------------- CPU ----

def test_oracle_softmax_rows(xo):
    rows, cols = HEADS * T, SEQ
    x = rnd(rows * cols, 1, -4.0, 4.0)
    x[5 * cols:6 * cols] = -np.inf                      # a fully masked row -> zeros
    st = np.empty(2 * rows, np.float32)
    xo.lib().xo_softmax_rows_stats(st, x, rows, cols)
    assert st[10] == 0.0 and st[11] == 1.0
    y = x.copy()
    xo.lib().xo_softmax_rows_apply(y, st, rows, cols)
    y = y.reshape(rows, cols)
    x2 = x.reshape(rows, cols).astype(np.float64)
    live = np.arange(rows) != 5
    e = np.exp(x2[live] - x2[live].max(1, keepdims=True))
    assert rel(y[live], e / e.sum(1, keepdims=True)) < 1e-6
    assert np.abs(y[live].sum(1) - 1.0).max() < 1e-5 and not y[5].any()


@pytest.mark.parametrize("window", [0, 8])
def test_oracle_attention_prefill(xo, window):
    q, k, v = rnd(HEADS * T * HD, 2), rnd(SEQ * KVH * HD, 3), rnd(SEQ * KVH * HD, 4)
    sc = np.empty(HEADS * T * SEQ, np.float32)
    xo.lib().xo_attention_scores_prefill(sc, q, k, HEADS, KVH, HD, T, SEQ, 0, window, SCALE)
    want, mask = np_scores(q, k, T, 0, window)
    sc3 = sc.reshape(HEADS, T, SEQ)
    assert np.array_equal(np.isneginf(sc3), np.broadcast_to(mask, sc3.shape))
    assert rel(sc3[~np.isneginf(sc3)], want[~np.isneginf(want)]) < 1e-5
    # softmax + apply against float64
    st = np.empty(2 * HEADS * T, np.float32)
    xo.lib().xo_softmax_rows_stats(st, sc, HEADS * T, SEQ)
    xo.lib().xo_softmax_rows_apply(sc, st, HEADS * T, SEQ)
    out = np.empty(HEADS * T * HD, np.float32)
    xo.lib().xo_attention_apply_prefill(out, sc, v, HEADS, KVH, HD, T, SEQ)
    p = np.exp(want - want.max(2, keepdims=True))
    p /= p.sum(2, keepdims=True)
    o = np.einsum("hqt,td->hqd", p, v.reshape(SEQ, HD).astype(np.float64))
    assert rel(out, o.reshape(-1)) < 1e-5


def test_oracle_prefill_equals_decode(xo):
    """One query at q_offset = pos reproduces the decode kernels bit for bit
    (sampling_test.cpp:862-880), and row r of the row kernels equals the
    decode kernel on row r."""
    lib = xo.lib()
    pos = SEQ - 1
    q1, k = rnd(HEADS * HD, 5), rnd(SEQ * KVH * HD, 6)
    a = np.empty(HEADS * SEQ, np.float32)
    b = np.empty(HEADS * SEQ, np.float32)
    lib.xo_attention_scores_prefill(a, q1, k, HEADS, KVH, HD, 1, SEQ, pos, 0, SCALE)
    lib.xo_attention_scores(b, q1, k, HEADS, KVH, HD, SEQ, SCALE, 0)
    assert np.array_equal(a, b)
    # QK-norm over tokens == decode per-head norm token by token
    x, w = rnd(T * HEADS * HD, 7), rnd(HD, 8)
    y = np.empty_like(x)
    lib.xo_rmsnorm_heads_rows_gemma(y, x, w, T, HEADS, HD, EPS)
    for t in range(T):
        z = np.empty(HEADS * HD, np.float32)
        lib.xo_rmsnorm_heads_gemma(z, np.ascontiguousarray(x[t * HEADS * HD:(t + 1) * HEADS * HD]), w,
                                   HEADS, HD, EPS)
        assert np.array_equal(z, y[t * HEADS * HD:(t + 1) * HEADS * HD])
    # RoPE over tokens == decode rope at each position
    xr = x.copy()
    lib.xo_rope_prefill(xr, T, HEADS, HD, 100, 10000.0)
    for t in range(T):
        z = np.ascontiguousarray(x[t * HEADS * HD:(t + 1) * HEADS * HD])
        lib.xo_rope(z, HEADS, HD, 100 + t, 10000.0)
        assert np.array_equal(z, xr[t * HEADS * HD:(t + 1) * HEADS * HD])
    # row RMSNorm == numpy per row
    xin, wn = rnd(T * HIDDEN, 9), rnd(HIDDEN, 10, -0.2, 0.2)
    ss = np.empty(T, np.float32)
    out = np.empty_like(xin)
    lib.xo_rmsnorm_rows_sumsq(ss, xin, T, HIDDEN)
    lib.xo_rmsnorm_rows_apply_gemma(out, xin, wn, ss, T, HIDDEN, EPS)
    x2 = xin.reshape(T, HIDDEN).astype(np.float64)
    want = x2 / np.sqrt((x2 * x2).mean(1, keepdims=True) + EPS) * (1.0 + wn)
    assert rel(out, want.reshape(-1)) < 1e-6


def test_oracle_plumbing(xo):
    lib = xo.lib()
    cache = np.zeros(SEQ * HD, np.float32)
    src = rnd(5 * HD, 11)
    lib.xo_kv_append_rows(cache, src, 5, HD, 7)
    assert np.array_equal(cache[7 * HD:12 * HD], src) and not cache[:7 * HD].any()
    vocab = 97
    table = rnd(vocab * 64, 12)
    toks = ((np.arange(T) * 251 + 13) % vocab).astype(np.uint32)
    out = np.empty(T * 64, np.float32)
    lib.xo_embed_lookup_rows(out, table, toks, T, 64)
    assert np.array_equal(out.reshape(T, 64), table.reshape(vocab, 64)[toks])


# ---------------------------------------------------------------- GPU ----

def dev(X, a):
    return X.DeviceBuffer.from_array(np.ascontiguousarray(a))


def sentinel(X, n):
    d = X.DeviceBuffer(n * 4)
    d.upload(np.full(n, SENTINEL, np.float32))
    return d


@pytest.mark.gpu
def test_gpu_softmax_rows(xp, xo):
    X = xp
    print("case prefill softmax rows", flush=True)
    rows, cols = HEADS * T, SEQ
    x = rnd(rows * cols, 21, -4.0, 4.0)
    x[5 * cols:6 * cols] = -np.inf
    dx, dst = dev(X, x), sentinel(X, 2 * rows)
    X.call("xp_softmax_rows_stats", dst.vp, dx.vp, rows, cols, None)
    X.call("xp_softmax_rows_apply", dx.vp, dst.vp, rows, cols, None)
    X.synchronize()
    st = np.empty(2 * rows, np.float32)
    xo.lib().xo_softmax_rows_stats(st, x, rows, cols)
    want = x.copy()
    xo.lib().xo_softmax_rows_apply(want, st, rows, cols)
    got_st = dst.download(np.float32)
    assert got_st[10] == 0.0 and got_st[11] == 1.0
    assert rel(got_st, st) < 1e-5
    got = dx.download(np.float32)
    assert not (got == SENTINEL).any() and rel(got, want) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("window", [0, 8])
def test_gpu_attention_prefill(xp, xo, window):
    X = xp
    print(f"case prefill attention window={window}", flush=True)
    q, k, v = rnd(HEADS * T * HD, 22), rnd(SEQ * KVH * HD, 23), rnd(SEQ * KVH * HD, 24)
    lib = xo.lib()
    want = np.empty(HEADS * T * SEQ, np.float32)
    lib.xo_attention_scores_prefill(want, q, k, HEADS, KVH, HD, T, SEQ, 0, window, SCALE)
    dq, dk, dv = dev(X, q), dev(X, k), dev(X, v)
    ds = sentinel(X, HEADS * T * SEQ)
    X.call("xp_attention_scores_prefill", ds.vp, dq.vp, dk.vp, HEADS, KVH, HD, T, SEQ, 0, window,
           SCALE, None)
    X.synchronize()
    got = ds.download(np.float32)
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    live = ~np.isneginf(want)
    assert rel(got[live], want[live]) < 1e-5
    # softmax + apply on the device against the oracle chain
    dst, do = sentinel(X, 2 * HEADS * T), sentinel(X, HEADS * T * HD)
    X.call("xp_softmax_rows_stats", dst.vp, ds.vp, HEADS * T, SEQ, None)
    X.call("xp_softmax_rows_apply", ds.vp, dst.vp, HEADS * T, SEQ, None)
    X.call("xp_attention_apply_prefill", do.vp, ds.vp, dv.vp, HEADS, KVH, HD, T, SEQ, None)
    X.synchronize()
    st = np.empty(2 * HEADS * T, np.float32)
    lib.xo_softmax_rows_stats(st, want, HEADS * T, SEQ)
    lib.xo_softmax_rows_apply(want, st, HEADS * T, SEQ)
    out = np.empty(HEADS * T * HD, np.float32)
    lib.xo_attention_apply_prefill(out, want, v, HEADS, KVH, HD, T, SEQ)
    assert rel(do.download(np.float32), out) < 1e-5


@pytest.mark.gpu
def test_gpu_prefill_attention_equals_decode(xp):
    """One query at q_offset = pos through scores -> softmax -> apply equals
    the product's decode attention over the same (fp16-valued) K / V."""
    X = xp
    print("case prefill == decode attention", flush=True)
    span = 300
    pos = span - 1
    q1 = rnd(HEADS * HD, 25)
    k, v = f16r(rnd(span * HD, 26)), f16r(rnd(span * HD, 27))
    dq, dk, dv = dev(X, q1), dev(X, k), dev(X, v)
    ds, dst, do = X.DeviceBuffer(HEADS * span * 4), X.DeviceBuffer(2 * HEADS * 4), sentinel(X, HEADS * HD)
    X.call("xp_attention_scores_prefill", ds.vp, dq.vp, dk.vp, HEADS, KVH, HD, 1, span, pos, 0, SCALE,
           None)
    X.call("xp_softmax_rows_stats", dst.vp, ds.vp, HEADS, span, None)
    X.call("xp_softmax_rows_apply", ds.vp, dst.vp, HEADS, span, None)
    X.call("xp_attention_apply_prefill", do.vp, ds.vp, dv.vp, HEADS, KVH, HD, 1, span, None)
    dk16, dv16 = dev(X, k.astype(np.float16).view(np.uint16)), dev(X, v.astype(np.float16).view(np.uint16))
    dd = sentinel(X, HEADS * HD)
    X.call("xp_attention_decode", dd.vp, dq.vp, dk16.vp, dv16.vp, HEADS, KVH, HD, span, 0, SCALE, None)
    X.synchronize()
    a, b = do.download(np.float32), dd.download(np.float32)
    assert not (a == SENTINEL).any() and not (b == SENTINEL).any()
    assert rel(a, b) < 1e-5


@pytest.mark.gpu
def test_gpu_prefill_norms_and_rope(xp, xo):
    X = xp
    print("case prefill norms and rope", flush=True)
    lib = xo.lib()
    xin, wn = rnd(T * HIDDEN, 31), rnd(HIDDEN, 32, -0.2, 0.2)
    ss = np.empty(T, np.float32)
    want = np.empty_like(xin)
    lib.xo_rmsnorm_rows_sumsq(ss, xin, T, HIDDEN)
    lib.xo_rmsnorm_rows_apply_gemma(want, xin, wn, ss, T, HIDDEN, EPS)
    dx, dw, dss, do = dev(X, xin), dev(X, wn), sentinel(X, T), sentinel(X, T * HIDDEN)
    X.call("xp_rmsnorm_rows_sumsq", dss.vp, dx.vp, T, HIDDEN, None)
    X.call("xp_rmsnorm_rows_apply_gemma", do.vp, dx.vp, dw.vp, dss.vp, T, HIDDEN, C.c_float(EPS), None)
    X.synchronize()
    assert rel(dss.download(np.float32), ss) < 1e-5
    got = do.download(np.float32)
    assert not (got == SENTINEL).any() and rel(got, want) < 1e-5
    # per-head QK-norm over tokens
    xh, wh = rnd(T * HEADS * HD, 33), rnd(HD, 34, -0.2, 0.2)
    wanth = np.empty_like(xh)
    lib.xo_rmsnorm_heads_rows_gemma(wanth, xh, wh, T, HEADS, HD, EPS)
    dxh, dwh, doh = dev(X, xh), dev(X, wh), sentinel(X, T * HEADS * HD)
    X.call("xp_rmsnorm_heads_rows_gemma", doh.vp, dxh.vp, dwh.vp, T, HEADS, HD, C.c_float(EPS), None)
    X.synchronize()
    goth = doh.download(np.float32)
    assert not (goth == SENTINEL).any() and rel(goth, wanth) < 1e-5
    # RoPE at positions 4090.. (large angles) and 0..: row t equals the
    # product's decode rope at position pos0 + t bit for bit (the reference's
    # check, sampling_test.cpp:943-975), and the oracle to sin / cos rounding
    # of angles up to ~4.1k rad (fp32 angle spacing there is 4.9e-4)
    for pos0, theta, tol in [(4090, 1e6, 2e-3), (0, 1e4, 1e-5)]:
        wr = xh.copy()
        lib.xo_rope_prefill(wr, T, HEADS, HD, pos0, theta)
        dr = dev(X, xh)
        X.call("xp_rope_prefill", dr.vp, T, HEADS, HD, pos0, C.c_float(theta), None)
        X.synchronize()
        got = dr.download(np.float32)
        assert rel(got, wr) < tol, pos0
        for t in (0, 17, T - 1):
            dd = dev(X, xh[t * HEADS * HD:(t + 1) * HEADS * HD])
            X.call("xp_rope", dd.vp, HEADS, HD, pos0 + t, C.c_float(theta), None)
            X.synchronize()
            assert np.array_equal(dd.download(np.float32), got[t * HEADS * HD:(t + 1) * HEADS * HD]), (pos0, t)


@pytest.mark.gpu
def test_gpu_prefill_plumbing(xp, xo):
    X = xp
    print("case prefill plumbing", flush=True)
    cache0 = rnd(SEQ * HD, 41)
    src = rnd(5 * HD, 42)
    dc, ds = dev(X, cache0), dev(X, src)
    X.call("xp_kv_append_rows", dc.vp, ds.vp, 5, HD, 7, None)
    X.synchronize()
    want = cache0.copy()
    want[7 * HD:12 * HD] = src
    assert np.array_equal(dc.download(np.float32), want)
    vocab, n = 97, 64
    table = rnd(vocab * n, 43)
    toks = ((np.arange(T) * 251 + 13) % vocab).astype(np.uint32)
    toks[3] = vocab + 5                                  # past the table: a zero row
    dt, dk, do = dev(X, table), dev(X, toks), sentinel(X, T * n)
    X.call("xp_embed_lookup_rows", do.vp, dt.vp, dk.vp, T, n, vocab, None)
    X.synchronize()
    got = do.download(np.float32).reshape(T, n)
    ok = np.arange(T) != 3
    assert np.array_equal(got[ok], table.reshape(vocab, n)[toks[ok]]) and not got[3].any()


@pytest.mark.gpu
def test_gpu_prefill_argument_errors(xp):
    X = xp
    d = X.DeviceBuffer(1 << 16)
    with pytest.raises(X.XposeError):
        X.call("xp_attention_scores_prefill", d.vp, d.vp, d.vp, 3, 2, HD, 1, 4, 0, 0, SCALE, None)
    with pytest.raises(X.XposeError):
        X.call("xp_rope_prefill", d.vp, 1, 1, 3, 0, C.c_float(1e4), None)
    with pytest.raises(X.XposeError):
        X.call("xp_rmsnorm_heads_rows_gemma", d.vp, d.vp, d.vp, 1, 1, HD, C.c_float(EPS), None)
    with pytest.raises(X.XposeError):
        X.call("xp_softmax_rows_stats", None, d.vp, 4, 4, None)
