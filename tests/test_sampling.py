"""Sampling: argmax tie rule, top-k, top-p, multinomial, the host draw and the
Philox stream.

Known answers come from examples/llm/sampling_test.cpp: planted maximum at
190037 = 99.5 and ties at {7, 190037, 262141} -> 7 (:136-178), top-k against a
CPU sort with a duplicated 3.25 at 1234/9999 (:424-500), top-p on
probs ~ exp(-0.35 j) with ids 1000 + 37 j (:537-577) and the CDF walk at
u = s/32 (:579-607).
"""
import numpy as np
import pytest

from conftest import hold

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
