"""Transformer ops: the oracle pinned by closed forms and invariants (CPU), the
gfx950 kernels against the oracle (GPU).

Follows examples/llm/kernel_tests.cpp: Gemma shapes, seed 20260719, U(-1.5,
1.5) inputs, kSeqLen = 131 (not a multiple of 64), numpy allclose rtol 1e-4 /
atol 1e-6 (:43-89, :136-142), sentinel liveness, the windowed kv_start = 43
case with its negative control (:483-621), and the chained attention block
(:713-799).
"""
import ctypes as C
import numpy as np
import pytest

from conftest import allclose_report, hold

HIDDEN, FFN, HEADS, KV_HEADS, HEAD_DIM, SEQ = 1152, 6912, 4, 1, 256, 131
EPS = 1e-6
SENT = np.float32(-1e30)
RTOL, ATOL = 1e-4, 1e-6


def rng():
    return np.random.default_rng(20260719)


def u(r, n):
    return r.uniform(-1.5, 1.5, n).astype(np.float32)


def f16_bits(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def f16_vals(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- CPU ----

def test_oracle_rmsnorm_closed_form(xo):
    r = rng()
    x, w = u(r, HIDDEN), u(r, HIDDEN)
    got = xo.rmsnorm_gemma(x, w, EPS)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean() + EPS) * (1.0 + w.astype(np.float64))
    ok, msg = allclose_report(got, want, 1e-5, 1e-6)
    assert ok, msg


def test_oracle_heads_norm_closed_form(xo):
    r = rng()
    x, w = u(r, HEADS * HEAD_DIM), u(r, HEAD_DIM)
    out = np.empty_like(x)
    xo.lib().xo_rmsnorm_heads_gemma(out, x, w, HEADS, HEAD_DIM, EPS)
    xd = x.astype(np.float64).reshape(HEADS, HEAD_DIM)
    want = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + EPS) * (1.0 + w.astype(np.float64))
    ok, msg = allclose_report(out, want.ravel(), 1e-5, 1e-6)
    assert ok, msg


def oracle_rope(xo, x, pos, theta, heads=HEADS):
    y = np.array(x, np.float32)
    xo.lib().xo_rope(y, heads, HEAD_DIM, pos, theta)
    return y


def test_oracle_rope_invariants(xo):
    """Rotation keeps each pair's norm, pos 0 is the identity, and rotating by
    a then by b equals rotating by a + b (to fp32 rounding)."""
    r = rng()
    x = u(r, HEADS * HEAD_DIM)
    assert np.array_equal(oracle_rope(xo, x, 0, 1e4), x)
    half = HEAD_DIM // 2
    for pos in (17, 511, 4095):
        y = oracle_rope(xo, x, pos, 1e6)
        a = x.reshape(HEADS, 2, half)
        b = y.reshape(HEADS, 2, half)
        np.testing.assert_allclose((b ** 2).sum(1), (a ** 2).sum(1), rtol=2e-6, atol=1e-6)
    # Composition: angle(a) + angle(b) vs angle(a+b) for small positions
    # where the fp32 angle products are exact enough to compare at 1e-5.
    y2 = oracle_rope(xo, oracle_rope(xo, x, 3, 1e4), 5, 1e4)
    y8 = oracle_rope(xo, x, 8, 1e4)
    np.testing.assert_allclose(y2, y8, rtol=1e-5, atol=1e-5)
    # Textbook rotate-half with float64 angles.
    d = np.arange(half)
    inv = 10000.0 ** (-2.0 * d / HEAD_DIM)
    ang = 17 * inv
    a = x.reshape(HEADS, 2, half).astype(np.float64)
    want = np.stack([a[:, 0] * np.cos(ang) - a[:, 1] * np.sin(ang),
                     a[:, 0] * np.sin(ang) + a[:, 1] * np.cos(ang)], 1).ravel()
    np.testing.assert_allclose(oracle_rope(xo, x, 17, 1e4), want, rtol=1e-4, atol=1e-5)


def test_oracle_geglu_closed_form(xo):
    r = rng()
    g, up = u(r, FFN) * 4, u(r, FFN)
    out = np.empty_like(g)
    xo.lib().xo_geglu(out, g, up, FFN)
    gd = g.astype(np.float64)
    want = 0.5 * gd * (1 + np.tanh(0.7978845608028654 * (gd + 0.044715 * gd ** 3))) * up
    ok, msg = allclose_report(out, want, 1e-5, 1e-6)
    assert ok, msg


def np_attention(q, k, v, span, kv0, scale):
    qd = q.astype(np.float64).reshape(HEADS, HEAD_DIM)
    K = k.astype(np.float64).reshape(-1, HEAD_DIM)[kv0:kv0 + span]
    V = v.astype(np.float64).reshape(-1, HEAD_DIM)[kv0:kv0 + span]
    s = qd @ K.T * scale
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    return (p @ V).ravel(), p


def test_oracle_attention_closed_form(xo):
    r = rng()
    q = u(r, HEADS * HEAD_DIM)
    kb, vb = f16_bits(u(r, SEQ * HEAD_DIM)), f16_bits(u(r, SEQ * HEAD_DIM))
    scale = np.float32(1 / 16)
    for kv0 in (0, SEQ // 3):
        span = SEQ - kv0
        out = np.empty(HEADS * HEAD_DIM, np.float32)
        xo.lib().xo_attention_f16(out, q, kb, vb, HEADS, KV_HEADS, HEAD_DIM, span, kv0, scale)
        want, p = np_attention(q, f16_vals(kb), f16_vals(vb), span, kv0, float(scale))
        ok, msg = allclose_report(out, want, 1e-4, 1e-6)
        assert ok, msg
        np.testing.assert_allclose(p.sum(1), 1.0, atol=1e-12)


def test_oracle_softmax_rows_sum_to_one(xo):
    r = rng()
    x = u(r, HEADS * SEQ) * 8
    xo.lib().xo_softmax_rows(x, HEADS, SEQ)
    assert np.abs(x.reshape(HEADS, SEQ).sum(1) - 1).max() < 1e-5


def test_oracle_kv_append_f16(xo):
    row, cap, pos = HEAD_DIM, 8, 5
    cache = np.full(row * cap, 0x4700, np.uint16)   # 7.0
    src = u(rng(), row)
    xo.lib().xo_kv_append_f16(cache, src, row, pos)
    want = np.full(row * cap, 0x4700, np.uint16)
    want[pos * row:(pos + 1) * row] = f16_bits(src)
    assert np.array_equal(cache, want)


def test_fp16_rne_matches_numpy(xh, xo):
    """The product's and the oracle's fp32 -> fp16 rounding against numpy
    (round to nearest even) on 200k values spanning subnormals to overflow."""
    r = np.random.default_rng(5)
    v = np.concatenate([r.standard_normal(100000) * 10.0 ** r.uniform(-9, 5, 100000),
                        np.array([65504, 65519.99, 65520, 1e6, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                                  0.0, -0.0, np.inf, -np.inf])]).astype(np.float32)
    want = v.astype(np.float16).view(np.uint16)
    got_o = np.array([xo.lib().xo_fp32_to_fp16(float(f)) for f in v[:20000]], np.uint16)
    got_p = np.array([xh.f32_to_f16_bits(float(f)) for f in v[-20000:]], np.uint16)
    assert np.array_equal(got_o, want[:20000])
    assert np.array_equal(got_p, want[-20000:])


# ---------------------------------------------------------------- GPU ----

def dev(xp, a):
    return xp.DeviceBuffer.from_array(np.ascontiguousarray(a))


def sentinel(xp, n):
    b = xp.DeviceBuffer(n * 4)
    b.upload(np.full(n, SENT, np.float32))
    return b


@pytest.mark.gpu
def test_gpu_rmsnorm(xp, xo):
    print("case rmsnorm", flush=True)
    r = rng()
    x, w = u(r, HIDDEN), u(r, HIDDEN)
    dx, dw, do = dev(xp, x), dev(xp, w), sentinel(xp, HIDDEN)
    xp.call("xp_rmsnorm_gemma", do.vp, dx.vp, dw.vp, HIDDEN, EPS, None)
    xp.synchronize()
    ok, msg = allclose_report(do.download(np.float32), xo.rmsnorm_gemma(x, w, EPS), RTOL, ATOL)
    assert ok, msg


@pytest.mark.gpu
def test_gpu_heads_norm_and_rope(xp, xo):
    print("case heads_norm+rope", flush=True)
    r = rng()
    x, w = u(r, HEADS * HEAD_DIM), u(r, HEAD_DIM)
    want = np.empty_like(x)
    xo.lib().xo_rmsnorm_heads_gemma(want, x, w, HEADS, HEAD_DIM, EPS)
    dx, dw, do = dev(xp, x), dev(xp, w), sentinel(xp, x.size)
    xp.call("xp_rmsnorm_heads_gemma", do.vp, dx.vp, dw.vp, HEADS, HEAD_DIM, EPS, None)
    xp.synchronize()
    got = do.download(np.float32)
    ok, msg = allclose_report(got, want, RTOL, ATOL)
    assert ok, msg
    for pos, theta in ((17, 1e6), (4095, 1e4), (8191, 1e6)):
        d = dev(xp, want)
        xp.call("xp_rope", d.vp, HEADS, HEAD_DIM, pos, theta, None)
        xp.synchronize()
        g = d.download(np.float32)
        assert (g != want).sum() > want.size // 2, "rope changed nothing"
        ok, msg = allclose_report(g, oracle_rope(xo, want, pos, theta), RTOL, ATOL)
        assert ok, f"pos {pos}: {msg}"


@pytest.mark.gpu
@pytest.mark.parametrize("pos,theta", [(17, 1e6), (512, 1e4), (4096, 1e6), (8191, 1e4)])
def test_gpu_qk_norm_rope_append(xp, xo, pos, theta):
    print(f"case qk_norm_rope_append pos={pos}", flush=True)
    r = rng()
    qr, kr, v = u(r, HEADS * HEAD_DIM), u(r, HEAD_DIM), u(r, HEAD_DIM)
    qw, kw = u(r, HEAD_DIM) * 0.1, u(r, HEAD_DIM) * 0.1
    cap = pos + 2
    qn = np.empty_like(qr)
    kn = np.empty_like(kr)
    xo.lib().xo_rmsnorm_heads_gemma(qn, qr, qw, HEADS, HEAD_DIM, EPS)
    xo.lib().xo_rmsnorm_heads_gemma(kn, kr, kw, 1, HEAD_DIM, EPS)
    xo.lib().xo_rope(qn, HEADS, HEAD_DIM, pos, theta)
    xo.lib().xo_rope(kn, 1, HEAD_DIM, pos, theta)
    kc = np.full(cap * HEAD_DIM, 0x4700, np.uint16)
    vc = kc.copy()
    dq, dk = sentinel(xp, qr.size), sentinel(xp, kr.size)
    dkc, dvc = dev(xp, kc), dev(xp, vc)
    xp.call("xp_qk_norm_rope_append", dq.vp, dk.vp, hold(dev(xp, qr)), hold(dev(xp, kr)),
            hold(dev(xp, v)), hold(dev(xp, qw)), hold(dev(xp, kw)), dkc.vp, dvc.vp, HEADS, 1, HEAD_DIM,
            pos, theta, EPS, None)
    xp.synchronize()
    for got, want in ((dq.download(np.float32), qn), (dk.download(np.float32), kn)):
        ok, msg = allclose_report(got, want, RTOL, ATOL)
        assert ok, msg
    gk, gv = dkc.download(np.uint16), dvc.download(np.uint16)
    # Neighbouring rows untouched; the appended rows within one fp16 ulp of the oracle's.
    assert np.all(np.delete(gk, np.s_[pos * HEAD_DIM:(pos + 1) * HEAD_DIM]) == 0x4700)
    assert np.array_equal(gv[pos * HEAD_DIM:(pos + 1) * HEAD_DIM], f16_bits(v))
    kb = gk[pos * HEAD_DIM:(pos + 1) * HEAD_DIM].astype(np.int32)
    assert np.abs(kb - f16_bits(kn).astype(np.int32)).max() <= 1


def run_attention(xp, q, kb, vb, span, kv0, scale, timed=False):
    """xp_attention_decode (its splits combine through the arrival tickets),
    or with timed the measuring entry, whose launches take the exchange mode
    when every split fits a CU at once (its error word checked after)."""
    d = sentinel(xp, HEADS * HEAD_DIM)
    if timed:
        K = (C.c_void_p * 1)(hold(dev(xp, kb)).value)
        V = (C.c_void_p * 1)(hold(dev(xp, vb)).value)
        ms = C.c_float()
        xp.call("xp_attention_decode_timed", d.vp, hold(dev(xp, q)), K, V, 1, HEADS, KV_HEADS, HEAD_DIM,
                span, kv0, scale, 2, None, C.byref(ms))
    else:
        xp.call("xp_attention_decode", d.vp, hold(dev(xp, q)), hold(dev(xp, kb)), hold(dev(xp, vb)), HEADS,
                KV_HEADS, HEAD_DIM, span, kv0, scale, None)
    xp.synchronize()
    return d.download(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("seq,kv0", [(131, 0), (131, 43), (1, 0), (512, 0), (513, 1),
                                     (1100, 0), (2047, 0), (3600, 0), (4097, 0), (8192, 0),
                                     (8192, 7680)])
def test_gpu_attention(xp, xo, seq, kv0):
    """Spans 1..8192: up to 128 splits of at least 32 keys, combined in one
    level (at most 16 splits) or two (groups of 16; 1100 keys: 35 splits,
    the last group of 3; 3600: 113 splits, the last group of 1; 4097 and
    8192: 128 splits of 33 and 64 keys) through the kernel-level entry's
    tickets, and through the exchange mode of the timed entry (more than 16
    splits, all resident: tagged records, one poll)."""
    print(f"case attention seq={seq} kv0={kv0}", flush=True)
    r = rng()
    q = u(r, HEADS * HEAD_DIM)
    kb, vb = f16_bits(u(r, seq * HEAD_DIM)), f16_bits(u(r, seq * HEAD_DIM))
    span = seq - kv0
    scale = np.float32(1 / 16)
    want = np.empty(HEADS * HEAD_DIM, np.float32)
    xo.lib().xo_attention_f16(want, q, kb, vb, HEADS, KV_HEADS, HEAD_DIM, span, kv0, scale)
    got = run_attention(xp, q, kb, vb, span, kv0, scale)
    ok, msg = allclose_report(got, want, RTOL, 1e-5)
    assert ok, msg
    # the combine sums in a fixed order: the same call gives the same bits
    again = run_attention(xp, q, kb, vb, span, kv0, scale)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    xg = run_attention(xp, q, kb, vb, span, kv0, scale, timed=True)
    ok, msg = allclose_report(xg, want, RTOL, 1e-5)
    assert ok, "exchange mode: " + msg
    assert np.array_equal(xg.view(np.uint32), run_attention(xp, q, kb, vb, span, kv0, scale,
                                                            timed=True).view(np.uint32))
    if kv0:
        # Negative control (kernel_tests.cpp:538-552): ignoring kv_start gives
        # a measurably different answer, so the check above can see it.
        wrong = np.empty_like(want)
        xo.lib().xo_attention_f16(wrong, q, kb, vb, HEADS, KV_HEADS, HEAD_DIM, span, 0, scale)
        assert np.abs(wrong - want).max() > 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads", [(1, 1), (4, 4), (4, 2), (8, 2)])
@pytest.mark.parametrize("seq", [131, 4097, 8192])
def test_gpu_attention_head_groups(xp, xo, heads, kv_heads, seq):
    """Query heads per KV head 1, 2 and 4 over one to four KV heads: both
    entries against the oracle. At spans 4097 and 8192 the splits number more
    than 16 and the timed entry's launches take the exchange mode (128 splits
    over one or two KV heads, 64 over four), whose per-slice items then hold
    one head's statistics beside 1, 2 or 4 heads' dims."""
    print(f"case attention groups heads={heads} kv={kv_heads} seq={seq}", flush=True)
    r = rng()
    q = u(r, heads * HEAD_DIM)
    kb = f16_bits(u(r, seq * kv_heads * HEAD_DIM))
    vb = f16_bits(u(r, seq * kv_heads * HEAD_DIM))
    scale = np.float32(1 / 16)
    want = np.empty(heads * HEAD_DIM, np.float32)
    xo.lib().xo_attention_f16(want, q, kb, vb, heads, kv_heads, HEAD_DIM, seq, 0, scale)
    dq, dk, dv = dev(xp, q), dev(xp, kb), dev(xp, vb)
    outs = []
    for timed in (False, True, True):
        d = sentinel(xp, heads * HEAD_DIM)
        if timed:
            K, V, ms = (C.c_void_p * 1)(dk.ptr), (C.c_void_p * 1)(dv.ptr), C.c_float()
            xp.call("xp_attention_decode_timed", d.vp, dq.vp, K, V, 1, heads, kv_heads, HEAD_DIM,
                    seq, 0, scale, 2, None, C.byref(ms))
        else:
            xp.call("xp_attention_decode", d.vp, dq.vp, dk.vp, dv.vp, heads, kv_heads, HEAD_DIM,
                    seq, 0, scale, None)
        xp.synchronize()
        outs.append(d.download(np.float32))
        ok, msg = allclose_report(outs[-1], want, RTOL, 1e-5)
        assert ok, ("timed: " if timed else "") + msg
    assert np.array_equal(outs[1].view(np.uint32), outs[2].view(np.uint32))


@pytest.mark.gpu
def test_gpu_attention_ticket_levels():
    """XP_ATTN_EXCHANGE=0 in the environment turns the exchange mode off: the
    cases above of more than 16 splits (six spans, and the head groupings at
    spans 4097 and 8192) in a child process, where the timed entry's launches
    take the two-level ticket chain too."""
    import os
    import subprocess
    import sys
    print("case attention ticket levels", flush=True)
    env = dict(os.environ, XP_ATTN_EXCHANGE="0")
    here = os.path.dirname(os.path.abspath(__file__))
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.join(here, "test_transformer.py"), "-q",
                        "-m", "gpu", "-p", "no:cacheprovider",
                        "-k", "test_gpu_attention and (1100 or 2047 or 3600 or 4097 or 8192)"],
                       env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "14 passed" in r.stdout, r.stdout[-2000:]


@pytest.mark.gpu
def test_gpu_attention_block_chain(xp, xo):
    """norm -> rope -> attention chained on the device against the oracle's
    chain (kernel_tests.cpp:713-799)."""
    print("case attention block", flush=True)
    r = rng()
    q, qw = u(r, HEADS * HEAD_DIM), u(r, HEAD_DIM)
    kb, vb = f16_bits(u(r, SEQ * HEAD_DIM)), f16_bits(u(r, SEQ * HEAD_DIM))
    pos, theta, scale = SEQ - 1, 1e6, np.float32(1 / 16)
    qn = np.empty_like(q)
    xo.lib().xo_rmsnorm_heads_gemma(qn, q, qw, HEADS, HEAD_DIM, EPS)
    xo.lib().xo_rope(qn, HEADS, HEAD_DIM, pos, theta)
    want = np.empty_like(q)
    xo.lib().xo_attention_f16(want, qn, kb, vb, HEADS, KV_HEADS, HEAD_DIM, SEQ, 0, scale)
    dq, dqn, dout = dev(xp, q), sentinel(xp, q.size), sentinel(xp, q.size)
    xp.call("xp_rmsnorm_heads_gemma", dqn.vp, dq.vp, hold(dev(xp, qw)), HEADS, HEAD_DIM, EPS, None)
    xp.call("xp_rope", dqn.vp, HEADS, HEAD_DIM, pos, theta, None)
    xp.call("xp_attention_decode", dout.vp, dqn.vp, hold(dev(xp, kb)), hold(dev(xp, vb)), HEADS,
            KV_HEADS, HEAD_DIM, SEQ, 0, scale, None)
    xp.synchronize()
    ok, msg = allclose_report(dout.download(np.float32), want, RTOL, 1e-5)
    assert ok, msg


@pytest.mark.gpu
def test_gpu_geglu_residual_kv_append(xp, xo):
    print("case geglu/residual/kv_append", flush=True)
    r = rng()
    g, up = u(r, FFN) * 4, u(r, FFN)
    want = np.empty_like(g)
    xo.lib().xo_geglu(want, g, up, FFN)
    do = sentinel(xp, FFN)
    xp.call("xp_geglu", do.vp, hold(dev(xp, g)), hold(dev(xp, up)), FFN, None)
    x, y = u(r, HIDDEN), u(r, HIDDEN)
    dx = dev(xp, x)
    xp.call("xp_add_residual", dx.vp, hold(dev(xp, y)), HIDDEN, None)
    cache = np.full(HEAD_DIM * 8, 0x4700, np.uint16)
    src = u(r, HEAD_DIM)
    dc = dev(xp, cache)
    xp.call("xp_kv_append_f16", dc.vp, hold(dev(xp, src)), HEAD_DIM, 5, None)
    xp.synchronize()
    ok, msg = allclose_report(do.download(np.float32), want, RTOL, ATOL)
    assert ok, msg
    assert np.array_equal(dx.download(np.float32), x + y)
    cw = cache.copy()
    xo.lib().xo_kv_append_f16(cw, src, HEAD_DIM, 5)
    assert np.array_equal(dc.download(np.uint16), cw)


@pytest.mark.gpu
def test_gpu_attention_timed_equals_single_launch(xp, xo):
    """The measurement loop leaves the output of its last launch: equal to one
    xp_attention_decode over the same K/V copy, to the oracle's bar."""
    print("case attention timed", flush=True)
    r = rng()
    span = 700
    q = u(r, HEADS * HEAD_DIM)
    ks = [f16_bits(u(r, span * HEAD_DIM)) for _ in range(3)]
    vs = [f16_bits(u(r, span * HEAD_DIM)) for _ in range(3)]
    dk = [dev(xp, k) for k in ks]
    dv = [dev(xp, v) for v in vs]
    d = sentinel(xp, HEADS * HEAD_DIM)
    K = (C.c_void_p * 3)(*[b.ptr for b in dk])
    V = (C.c_void_p * 3)(*[b.ptr for b in dv])
    ms = C.c_float()
    iters = 5                                   # last launch uses copy (5 - 1) % 3 = 1
    xp.call("xp_attention_decode_timed", d.vp, hold(dev(xp, q)), K, V, 3, HEADS, KV_HEADS,
            HEAD_DIM, span, 0, np.float32(1 / 16), iters, None, C.byref(ms))
    xp.synchronize()
    assert ms.value > 0
    want = np.empty(HEADS * HEAD_DIM, np.float32)
    xo.lib().xo_attention_f16(want, q, ks[1], vs[1], HEADS, KV_HEADS, HEAD_DIM, span, 0,
                              np.float32(1 / 16))
    ok, msg = allclose_report(d.download(np.float32), want, RTOL, 1e-5)
    assert ok, msg
    with pytest.raises(xp.XposeError):
        xp.call("xp_attention_decode_timed", d.vp, d.vp, K, V, 0, HEADS, KV_HEADS, HEAD_DIM,
                span, 0, np.float32(1 / 16), iters, None, C.byref(ms))
