"""Sampling: argmax tie rule, top-k, top-p, multinomial, the host draw and the
Philox stream.

Known answers come from examples/llm/sampling_test.cpp: planted maximum at
190037 = 99.5 and ties at {7, 190037, 262141} -> 7 (:136-178), top-k against a
CPU sort with a duplicated 3.25 at 1234/9999 (:424-500), top-p on
probs ~ exp(-0.35 j) with ids 1000 + 37 j (:537-577) and the CDF walk at
u = s/32 (:579-607).
"""
import math

import numpy as np
import pytest

from conftest import allclose_report, hold

VOCAB = 262144
PLANTED = 190037


def logits_with_plant():
    r = np.random.default_rng(20260719)
    x = r.uniform(-1.5, 1.5, VOCAB).astype(np.float32)
    x[PLANTED] = 99.5
    return x


def serial_argmax(x):
    best, bv = 0, -np.inf
    for k, v in enumerate(x):
        if v > bv:
            bv, best = v, k
    return best


# ---------------------------------------------------------------- CPU ----

def test_philox_known_answers(xh, xo):
    """Random123's published philox4x32-10 vectors."""
    kat = [((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
           ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
           ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
            (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1))]
    for ctr, key, want in kat:
        assert tuple(int(v) for v in xh.philox4x32_10(ctr, key)) == want
        o = np.empty(4, np.uint32)
        xo.lib().xo_philox4x32_10(np.array(ctr, np.uint32), np.array(key, np.uint32), o)
        assert tuple(int(v) for v in o) == want


def test_synthetic_distributions(xh):
    """Nibbles uniform on [0,15]; scales |N(0,0.02)| in fp16; normals N(0,1)."""
    w = xh.synth_nibbles(1152, 1024, 9, 1)
    nib = np.stack([(w >> (4 * i)) & 15 for i in range(8)]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.size == 16 and np.abs(counts / counts.mean() - 1).max() < 0.02
    s = xh.synth_scales(1152, 1024, 9, 2).view(np.float16).astype(np.float64)
    assert (s >= 0).all() and abs(s.mean() - 0.02 * np.sqrt(2 / np.pi)) < 3e-4
    n = xh.synth_normal(200000, 9, 3)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1) < 0.01
    # Counter-based: any element regenerates alone and tensors are independent.
    assert np.array_equal(xh.synth_nibbles(1152, 1024, 9, 1), w)
    assert not np.array_equal(xh.synth_nibbles(1152, 1024, 9, 2), w)


def test_oracle_argmax_known_answers(xo):
    x = logits_with_plant()
    assert xo.argmax_tree(x) == (PLANTED, 99.5)
    t = x.copy()
    t[PLANTED] = t[7] = t[VOCAB - 3] = 42.0
    assert xo.argmax_tree(t)[0] == 7
    # Ties placed so each lands in a different strided chain, and ties that
    # share a chain: the tree always agrees with the serial scan.
    r = np.random.default_rng(1)
    for _ in range(20):
        y = np.round(r.uniform(-3, 3, 8192), 1).astype(np.float32)   # many duplicates
        assert xo.argmax_tree(y)[0] == serial_argmax(y)


def test_oracle_topk_vs_sort(xo):
    x = logits_with_plant()
    x[1234] = x[9999] = 3.25
    order = np.lexsort((np.arange(VOCAB), -x))[:64]
    for k, np_ in ((40, 256), (1, 256), (64, 256)):
        cv = np.empty(np_ * k, np.float32)
        ci = np.empty(np_ * k, np.uint32)
        xo.lib().xo_topk_partial(cv, ci, x, VOCAB, np_, k)
        ov = np.full(k, -1e30, np.float32)
        oi = np.empty(k, np.uint32)
        xo.lib().xo_topk_rank_select(ov, oi, cv, ci, np_ * k, k)
        assert np.array_equal(oi, order[:k])
        assert np.array_equal(ov, x[order[:k]])


def test_oracle_topp_and_multinomial_known_answers(xo):
    K = 40
    probs = np.exp(-0.35 * np.arange(K, dtype=np.float32)).astype(np.float32)
    probs = (probs / probs.astype(np.float64).sum()).astype(np.float32)
    ids = (1000 + 37 * np.arange(K)).astype(np.uint32)
    for p in (0.5, 0.9, 0.99):
        w = probs.copy()
        xo.lib().xo_topp_cutoff(w, K, p)
        total = float(np.float32(probs.sum(dtype=np.float32)))
        c = probs.copy()
        cum = np.float32(0)
        for j in range(K):
            if cum >= np.float32(p) * np.float32(total):
                c[j] = 0
            else:
                cum = np.float32(cum + c[j])
        assert np.array_equal(w, c)
        assert 0 < int((w > 0).sum()) < K
    for s in range(32):
        uu = np.float32(s / 32)
        out = np.empty(2, np.float32)
        oi = np.empty(1, np.uint32)
        xo.lib().xo_multinomial_sample(out, oi, probs, ids, K, uu)
        total = probs.sum(dtype=np.float32)
        target, cum, chosen = np.float32(uu * total), np.float32(0), 0
        for j in range(K):
            cum = np.float32(cum + probs[j])
            chosen = ids[j]
            if cum > target:
                break
        assert oi[0] == chosen


def test_draw_product_matches_oracle(xh, xo):
    """The session's host draw (xp_draw) and the oracle's restatement of
    DecodeSession::draw give the same token for the same candidates and u."""
    r = np.random.default_rng(3)
    for trial in range(300):
        n = int(r.integers(1, 200))
        v = np.round(r.normal(0, 2, n), 2).astype(np.float32)   # duplicates on purpose
        i = r.choice(VOCAB, n, replace=False).astype(np.uint32)
        temp = float(r.choice([0.0, 0.5, 0.8, 1.0, 2.0]))
        tk = int(r.choice([0, 1, 5, 64]))
        tp = float(r.choice([1.0, 0.95, 0.5, 0.01]))
        u = float(r.random())
        got = xh.draw(v, i, temp, tk, tp, u)
        want = xo.lib().xo_draw(v.copy(), i.copy(), n, temp, tk, tp, u)
        assert got == want, (trial, n, temp, tk, tp, u)


def test_draw_known_answers_and_distribution(xh):
    v = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    i = np.array([10, 20, 30, 5], np.uint32)
    # Ties on value break to the lower id; top_k=1 / tiny top_p = greedy.
    assert xh.draw(v, i, 1.0, 1, 1.0, 0.99) == 5
    assert xh.draw(v, i, 1.0, 0, 0.01, 0.99) == 5
    assert xh.draw(v, i, 1.0, 0, 1.0, 0.0) == 5
    # Empirical frequencies match softmax(v / T) over top-3 within 3 sigma.
    T, N = 0.8, 20000
    counts = {}
    for s in range(N):
        t = xh.draw(v, i, T, 3, 1.0, xh.philox_uniform(1234, 0, s))
        counts[t] = counts.get(t, 0) + 1
    top = np.array([3.0, 3.0, 2.0])
    p = np.exp((top - 3) / T)
    p /= p.sum()
    for tok, pr in zip((5, 20, 30), p):
        sd = np.sqrt(pr * (1 - pr) / N)
        assert abs(counts.get(tok, 0) / N - pr) < 4 * sd
    assert 10 not in counts


# ---------------------------------------------------------------- GPU ----

def gpu_argmax(xp, x):
    d = xp.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    oi = xp.DeviceBuffer(4)
    ov = xp.DeviceBuffer(4)
    oi.upload(np.array([0xDEADBEEF], np.uint32))
    xp.call("xp_argmax", oi.vp, ov.vp, d.vp, x.size, None)
    xp.synchronize()
    return int(oi.download(np.uint32)[0]), float(ov.download(np.float32)[0])


@pytest.mark.gpu
def test_gpu_argmax(xp, xo):
    print("case argmax", flush=True)
    x = logits_with_plant()
    assert gpu_argmax(xp, x) == (PLANTED, 99.5)
    t = x.copy()
    t[PLANTED] = t[7] = t[VOCAB - 3] = 42.0
    assert gpu_argmax(xp, t)[0] == 7
    r = np.random.default_rng(2)
    for n in (1, 5, 4096, 8192, 100003, VOCAB):
        y = np.round(r.uniform(-3, 3, n), 1).astype(np.float32)
        assert gpu_argmax(xp, y)[0] == xo.argmax_tree(y)[0]
    y = np.full(VOCAB, -np.inf, np.float32)
    assert gpu_argmax(xp, y)[0] == 0
    y[[5, 77]] = np.nan
    y[300] = -1.0
    assert gpu_argmax(xp, y)[0] == 300


@pytest.mark.gpu
@pytest.mark.parametrize("nparts", [1024, 4096, 100000])
def test_gpu_topk4_harvest_bit_exact(xp, xo, nparts):
    print(f"case topk4 nparts={nparts}", flush=True)
    x = logits_with_plant()
    x[1234] = x[9999] = 3.25
    wv = np.empty(4 * nparts, np.float32)
    wi = np.empty(4 * nparts, np.uint32)
    xo.lib().xo_topk4_partial(wv, wi, x, VOCAB, nparts)
    dv, di = xp.DeviceBuffer(wv.nbytes), xp.DeviceBuffer(wi.nbytes)
    xp.call("xp_topk4_harvest", dv.vp, di.vp, hold(xp.DeviceBuffer.from_array(x)), VOCAB, nparts,
            None)
    xp.synchronize()
    assert np.array_equal(dv.download(np.float32).view(np.uint32), wv.view(np.uint32))
    assert np.array_equal(di.download(np.uint32), wi)


# ------------------------------------------- full-vocabulary chain (a22) ----
# The reference's device sampling chain (llm_sampling.cl:130-225, 257-281,
# 349-386, 399-488). CPU: the oracle against numpy closed forms and
# invariants. GPU: each kernel against the oracle on the same inputs —
# bit-exact except exp (softmax_exp_partial, rtol 2e-6), with every later
# step fed the device's own inputs so its output is compared bit for bit.

def vocab_logits(seed=7, n=VOCAB):
    r = np.random.default_rng(seed)
    x = r.normal(0.0, 3.0, n).astype(np.float32)
    x[1234 % n] = x[9999 % n] = 11.25  # a tie at the top
    return x


def chain_view(x, nparts):
    """Element k of chain p is x[p + j * nparts]; returns a list of chains."""
    return [x[p::nparts] for p in range(nparts)]


def test_oracle_vocab_softmax_chain(xo):
    L = xo.lib()
    inv_t = np.float32(1.0 / 0.8)
    for nparts in (256, 4096, 1):
        x = vocab_logits(nparts)
        t = x.copy()
        L.xo_apply_temperature(t, inv_t, t.size)
        assert np.array_equal(t, x * inv_t)                      # one fp32 product each
        pmax = np.empty(nparts, np.float32)
        L.xo_reduce_max_partial(pmax, t, t.size, nparts)
        assert np.array_equal(pmax, np.array([c.max() for c in chain_view(t, nparts)]))
        stats = np.zeros(2, np.float32)
        L.xo_reduce_max_final(stats, pmax, nparts)
        assert stats[0] == t.max()
        e = np.empty_like(t)
        psum = np.empty(nparts, np.float32)
        L.xo_softmax_exp_partial(e, psum, t, stats, t.size, nparts)
        # exp of the fp32 difference the chain forms: only expf's own rounding
        want = np.exp((t - t.max()).astype(np.float64))
        assert np.allclose(e, want, rtol=1e-6, atol=0)
        # a serial fp32 sum of m terms is within (m - 1) 2^-24 sum|x| of the
        # exact sum (Higham's bound): tight for 1024-term chains, loose for one
        # 262144-term chain
        for c, got in zip(chain_view(want, nparts), psum):
            assert abs(got - math.fsum(c)) <= (c.size - 1) * 2.0 ** -24 * c.sum() + 1e-30
        rs = np.empty(nparts, np.float32)
        L.xo_reduce_sum_partial(rs, e, e.size, nparts)
        assert np.array_equal(rs, psum)                          # same chains, same order
        L.xo_reduce_sum_final(stats, psum, nparts)
        bound = (VOCAB / nparts + nparts) * 2.0 ** -24 * want.sum()
        assert abs(stats[1] - math.fsum(want)) <= bound
        L.xo_softmax_normalize(e, stats, e.size)
        rel = bound / want.sum() + 1e-6
        assert abs(math.fsum(e.astype(np.float64)) - 1.0) < rel      # rows sum to 1
        assert np.allclose(e, want / want.sum(), rtol=rel, atol=0)
    # max subtraction: a constant shift leaves the probabilities unchanged
    x = vocab_logits(3, 4096)
    probs = []
    for shift in (0.0, 40.0):
        y = (x + np.float32(shift)).astype(np.float32)
        pm, st = np.empty(64, np.float32), np.zeros(2, np.float32)
        L.xo_reduce_max_partial(pm, y, y.size, 64)
        L.xo_reduce_max_final(st, pm, 64)
        e, ps = np.empty_like(y), np.empty(64, np.float32)
        L.xo_softmax_exp_partial(e, ps, y, st, y.size, 64)
        L.xo_reduce_sum_final(st, ps, 64)
        L.xo_softmax_normalize(e, st, e.size)
        probs.append(e)
    assert np.allclose(probs[0], probs[1], rtol=1e-4, atol=1e-9)


def test_oracle_topk_mask(xo):
    x = vocab_logits(11)
    for k in (1, 40, 64):
        order = np.lexsort((np.arange(VOCAB), -x))
        tv = x[order[:k]].astype(np.float32)
        m = x.copy()
        xo.lib().xo_topk_mask(m, tv, k, VOCAB)
        keep = x >= tv[k - 1]
        assert np.array_equal(np.isfinite(m), keep)
        assert np.array_equal(m[keep], x[keep])


def strided_cdf64(w, nparts):
    """float64 CDF of w in chain order (chain 0's elements, chain 1's, ...)."""
    order = np.concatenate([np.arange(p, w.size, nparts) for p in range(nparts)])
    pos = np.empty(w.size, np.int64)
    pos[order] = np.arange(w.size)
    return np.cumsum(w[order].astype(np.float64)), pos


def test_oracle_multinomial_strided(xo):
    L = xo.lib()
    n, nparts = 4096, 64
    x = vocab_logits(5, n)
    st, pm = np.zeros(2, np.float32), np.empty(nparts, np.float32)
    L.xo_reduce_max_partial(pm, x, n, nparts)
    L.xo_reduce_max_final(st, pm, nparts)
    w, ps = np.empty_like(x), np.empty(nparts, np.float32)
    L.xo_softmax_exp_partial(w, ps, x, st, n, nparts)
    L.xo_reduce_sum_final(st, ps, nparts)
    out, oi = np.empty(2, np.float32), np.empty(1, np.uint32)
    cdf, pos = strided_cdf64(w, nparts)
    T = cdf[-1]
    S = 20000
    counts = np.zeros(n)
    for s in range(S):
        u = np.float32((s + 0.5) / S)
        L.xo_multinomial_strided(out, oi, w, ps, st, n, nparts, u)
        j = int(oi[0])
        # the chosen element's CDF step holds u * total, up to fp32 rounding
        lo = cdf[pos[j] - 1] if pos[j] > 0 else 0.0
        assert lo - 1e-4 * T <= float(u) * T <= cdf[pos[j]] + 1e-4 * T
        assert out[0] == np.float32(j) and out[1] == w[j]
        counts[j] += 1
    # evenly spaced u: each element is drawn its weight's share of the grid
    p = w.astype(np.float64) / T
    assert np.all(np.abs(counts / S - p) < 2.0 / S + 2e-4)


def test_sampling_chain_argument_errors(xh):
    """Entry points validate before launching: no GPU needed for these."""
    X = xh
    with pytest.raises(X.XposeError) as e:
        X.call("xp_topk_partial", 1, 1, 1, 16, 4, 65, None)
    assert "k=65" in str(e.value)
    with pytest.raises(X.XposeError):
        X.call("xp_topk_partial", None, 1, 1, 16, 4, 8, None)
    with pytest.raises(X.XposeError):
        X.call("xp_apply_temperature", 1, float("inf"), 16, None)
    with pytest.raises(X.XposeError):
        X.call("xp_multinomial_strided", 1, 1, 1, 1, 1, 16, 32, 0.5, None)
    with pytest.raises(X.XposeError):
        X.call("xp_reduce_sum_final", 1, 1, 0, None)


def dbuf(xp, a):
    return xp.DeviceBuffer.from_array(np.ascontiguousarray(a))


@pytest.mark.gpu
@pytest.mark.parametrize("nparts", [256, 4096])
def test_gpu_vocab_softmax_chain(xp, xo, nparts):
    print(f"case vocab softmax chain nparts={nparts}", flush=True)
    L = xo.lib()
    x = vocab_logits(nparts)
    inv_t = np.float32(1.0 / 0.8)
    dx = dbuf(xp, x)
    xp.call("xp_apply_temperature", dx.vp, float(inv_t), VOCAB, None)
    xp.synchronize()
    t = x.copy()
    L.xo_apply_temperature(t, inv_t, VOCAB)
    assert np.array_equal(dx.download(np.float32), t)
    dpm, dst = xp.DeviceBuffer(4 * nparts), dbuf(xp, np.zeros(2, np.float32))
    xp.call("xp_reduce_max_partial", dpm.vp, dx.vp, VOCAB, nparts, None)
    xp.call("xp_reduce_max_final", dst.vp, dpm.vp, nparts, None)
    xp.synchronize()
    pm, st = np.empty(nparts, np.float32), np.zeros(2, np.float32)
    L.xo_reduce_max_partial(pm, t, VOCAB, nparts)
    L.xo_reduce_max_final(st, pm, nparts)
    assert np.array_equal(dpm.download(np.float32), pm)
    assert dst.download(np.float32)[0] == st[0]
    # exp: device libm against the host's, within 2 ulp-ish
    de, dps = xp.DeviceBuffer(4 * VOCAB), xp.DeviceBuffer(4 * nparts)
    xp.call("xp_softmax_exp_partial", de.vp, dps.vp, dx.vp, dst.vp, VOCAB, nparts, None)
    xp.synchronize()
    e, ps = np.empty_like(t), np.empty(nparts, np.float32)
    L.xo_softmax_exp_partial(e, ps, t, st, VOCAB, nparts)
    ge, gps = de.download(np.float32), dps.download(np.float32)
    ok, msg = allclose_report(ge, e, 2e-6, 1e-30)
    assert ok, msg
    ok, msg = allclose_report(gps, ps, 1e-5, 0)
    assert ok, msg
    # from here on the oracle gets the device's inputs: bit-exact
    L.xo_softmax_exp_partial(e, ps, t, st, VOCAB, nparts)
    drs = xp.DeviceBuffer(4 * nparts)
    xp.call("xp_reduce_sum_partial", drs.vp, de.vp, VOCAB, nparts, None)
    xp.call("xp_reduce_sum_final", dst.vp, dps.vp, nparts, None)
    xp.synchronize()
    rs = np.empty(nparts, np.float32)
    L.xo_reduce_sum_partial(rs, ge, VOCAB, nparts)
    assert np.array_equal(drs.download(np.float32), rs)
    assert np.array_equal(rs, gps)
    st2 = st.copy()
    L.xo_reduce_sum_final(st2, gps, nparts)
    gst = dst.download(np.float32)
    assert gst[1] == st2[1]
    for s in range(16):
        u = np.float32((s + 0.25) / 16)
        do, di = xp.DeviceBuffer(8), xp.DeviceBuffer(4)
        xp.call("xp_multinomial_strided", do.vp, di.vp, de.vp, dps.vp, dst.vp, VOCAB, nparts,
                float(u), None)
        xp.synchronize()
        out, oi = np.empty(2, np.float32), np.empty(1, np.uint32)
        L.xo_multinomial_strided(out, oi, ge, gps, gst, VOCAB, nparts, u)
        assert int(di.download(np.uint32)[0]) == int(oi[0])
        assert np.array_equal(do.download(np.float32), out)
    xp.call("xp_softmax_normalize", de.vp, dst.vp, VOCAB, None)
    xp.synchronize()
    L.xo_softmax_normalize(ge, gst, VOCAB)
    got = de.download(np.float32)
    assert np.array_equal(got, ge)
    assert abs(got.astype(np.float64).sum() - 1.0) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("k,nparts", [(1, 256), (40, 256), (64, 256), (40, 4096), (64, 33)])
def test_gpu_topk_chain_bit_exact(xp, xo, k, nparts):
    print(f"case topk chain k={k} nparts={nparts}", flush=True)
    L = xo.lib()
    x = logits_with_plant()
    x[1234] = x[9999] = 3.25
    r = np.random.default_rng(k)
    x[r.integers(0, VOCAB, 200)] = 2.5                     # many exact ties
    ncand = nparts * k
    cv, ci = np.empty(ncand, np.float32), np.empty(ncand, np.uint32)
    L.xo_topk_partial(cv, ci, x, VOCAB, nparts, k)
    dx = dbuf(xp, x)
    dcv, dci = xp.DeviceBuffer(4 * ncand), xp.DeviceBuffer(4 * ncand)
    xp.call("xp_topk_partial", dcv.vp, dci.vp, dx.vp, VOCAB, nparts, k, None)
    xp.synchronize()
    assert np.array_equal(dcv.download(np.float32).view(np.uint32), cv.view(np.uint32))
    assert np.array_equal(dci.download(np.uint32), ci)
    ov, oi = np.full(k, -7.0, np.float32), np.full(k, 7, np.uint32)
    L.xo_topk_rank_select(ov, oi, cv, ci, ncand, k)
    dov, doi = dbuf(xp, np.full(k, -7.0, np.float32)), dbuf(xp, np.full(k, 7, np.uint32))
    xp.call("xp_topk_rank_select", dov.vp, doi.vp, dcv.vp, dci.vp, ncand, k, None)
    xp.synchronize()
    assert np.array_equal(doi.download(np.uint32), oi)
    assert np.array_equal(dov.download(np.float32), ov)
    assert np.array_equal(oi, np.lexsort((np.arange(VOCAB), -x))[:k])
    xp.call("xp_topk_mask", dx.vp, dov.vp, k, VOCAB, None)
    xp.synchronize()
    m = x.copy()
    L.xo_topk_mask(m, ov, k, VOCAB)
    assert np.array_equal(dx.download(np.float32), m)


@pytest.mark.gpu
def test_gpu_topp_multinomial_known_answers(xp, xo):
    """sampling_test.cpp:537-607: probs ~ exp(-0.35 j), K = 40, ids 1000 + 37 j,
    p in {0.5, 0.9, 0.99}, u = s / 32."""
    print("case topp/multinomial", flush=True)
    L = xo.lib()
    K = 40
    probs = np.exp(-0.35 * np.arange(K, dtype=np.float32)).astype(np.float32)
    probs = (probs / probs.astype(np.float64).sum()).astype(np.float32)
    ids = (1000 + 37 * np.arange(K)).astype(np.uint32)
    for p in (0.5, 0.9, 0.99):
        w = probs.copy()
        L.xo_topp_cutoff(w, K, np.float32(p))
        dw = dbuf(xp, probs)
        xp.call("xp_topp_cutoff", dw.vp, K, p, None)
        xp.synchronize()
        assert np.array_equal(dw.download(np.float32), w)
        for s in range(32):
            u = np.float32(s / 32)
            out, oi = np.empty(2, np.float32), np.empty(1, np.uint32)
            L.xo_multinomial_sample(out, oi, w, ids, K, u)
            do, di = xp.DeviceBuffer(8), xp.DeviceBuffer(4)
            xp.call("xp_multinomial_sample", do.vp, di.vp, dw.vp, hold(dbuf(xp, ids)), K, float(u), None)
            xp.synchronize()
            assert int(di.download(np.uint32)[0]) == int(oi[0])
            assert np.array_equal(do.download(np.float32), out)
