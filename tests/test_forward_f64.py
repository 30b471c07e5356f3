"""Pins the oracle's whole-token forward (xo_forward, xo_generate_greedy) and
its layer policy against an independent float64 restatement written from the
reference's engine (tests/f64_model.py: decode.cpp:1668-1752, decode.hpp:
327-352, the .cl kernels), on a small Gemma-3-shaped model whose layers mix
global and sliding-window attention, at positions on both sides of the
window. Each planted misreading of the reference (a swapped post-norm, the
wrong theta on a layer, an off-by-one kv_start, ...) must fail the same
comparison, so the check has the power to see them.

Also pins xo_mv_km4_bs (the reference's shipped quad-sum order,
llm_matvec.cl:412-434) against float64.
"""
import types

import numpy as np
import pytest

from f64_model import MISTAKES, F64Model, dequant, pack_km4, random_model, unpack_km4

TOL = 5e-5          # relative to max|logits|: oracle (fp32, reference order) vs float64
                    # (measured 9.6e-6 on these inputs)

SHAPE = dict(n_layers=3, hidden=256, ffn=512, n_heads=4, n_kv_heads=1, head_dim=64, vocab=2048,
             max_seq=40, global_every=2, sliding_window=8, rms_eps=1e-6,
             rope_theta_global=1e6, rope_theta_local=1e4)


def shape(**kw):
    d = dict(SHAPE)
    d.update(kw)
    return types.SimpleNamespace(**d)


def oracle_pair(X, xo, p, seed, untied=False):
    """(oracle model, the packed tensors' get) on random weights of shape p."""
    get, embed, ints = random_model(p, seed, untied)
    cfg = X.XpConfig.gemma3_1b(**{k: getattr(p, k) for k in SHAPE},
                               scale_fmt=X.XP_SCALE_F16_QUAD)
    names = {X.T_Q: "q", X.T_K: "k", X.T_V: "v", X.T_O: "o", X.T_GATE: "gate", X.T_UP: "up",
             X.T_DOWN: "down", X.T_LM_HEAD: "lm_head"}
    norms = {X.T_ATTN_NORM: "attn_norm", X.T_POST_ATTN_NORM: "post_attn_norm",
             X.T_FFN_NORM: "ffn_norm", X.T_POST_FFN_NORM: "post_ffn_norm", X.T_Q_NORM: "q_norm",
             X.T_K_NORM: "k_norm", X.T_FINAL_NORM: "final_norm"}

    def oget(l, t):
        base = t & ~X.T_SCALES
        if base in names:
            return get(l, names[base])[1 if t & X.T_SCALES else 0]
        return get(l, norms[base])

    return xo.OracleModel(cfg, oget, embed=embed), get, embed, ints


def rel_err(a, b):
    b = np.asarray(b, np.float64)
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


# ---------------------------------------------------------------- packer ----

def test_km4_pack_unpack_matches_the_oracle_unpacker(xo):
    r = np.random.default_rng(1)
    w = r.integers(-8, 8, (256, 192))
    wq = pack_km4(w)
    assert np.array_equal(unpack_km4(wq, 256, 192), w)
    got = np.empty(256 * 192, np.int8)
    xo.lib().xo_unpack_km4(got, wq, 256, 192)   # pinned by its own closed form
    assert np.array_equal(got.reshape(256, 192), w)


@pytest.mark.parametrize("rows,cols", [(128, 64), (1152, 256), (384, 1024)])
def test_mv_km4_bs_matches_float64(xo, rows, cols):
    """The quad-sum order of the shipped kernel (each quad's four block sums
    added to the accumulator at once) against the float64 product."""
    r = np.random.default_rng(rows + cols)
    w = r.integers(-8, 8, (rows, cols))
    s = np.abs(r.normal(0, 0.02, (rows // 32, cols))).astype(np.float16)
    quad = np.ascontiguousarray(s.reshape(rows // 128, 4, cols).transpose(0, 2, 1).reshape(-1)
                                .view(np.uint16))
    x = r.normal(0, 1, rows).astype(np.float32)
    want = x.astype(np.float64) @ dequant(pack_km4(w), quad, rows, cols)
    for quad_sum in (True, False):
        got = xo.mv_km4(x, pack_km4(w), quad, rows, cols, fmt=0, quad_sum=quad_sum)
        assert rel_err(got, want) < 1e-5, quad_sum
    a = xo.mv_km4(x, pack_km4(w), quad, rows, cols, fmt=0, quad_sum=True)
    b = xo.mv_km4(x, pack_km4(w), quad, rows, cols, fmt=0, quad_sum=False)
    assert rel_err(a, b) < 1e-5


# ---------------------------------------------------------------- forward ----

def test_oracle_forward_matches_float64(xh, xo):
    """Logits at every position 0..20 (the window of 8 is passed at
    position 8; layer 1 is global, layers 0 and 2 local) within 5e-5 of
    max|logits| (the benchmark bar is 1e-3), and the fp16 KV rows the two
    wrote agree within an fp16 ulp of each row's scale."""
    X = xh
    p = shape()
    om, get, embed, _ = oracle_pair(X, xo, p, seed=3)
    fm = F64Model(p, get)
    toks = np.random.default_rng(4).integers(0, p.vocab, 21)
    for pos, t in enumerate(toks):
        a = om.forward(int(t), pos, True)
        b = fm.forward(int(t), pos, True)
        assert rel_err(a, b) < TOL, (pos, rel_err(a, b))
    kvd = p.n_kv_heads * p.head_dim
    for l in range(p.n_layers):
        for oc, fc in ((om.kcache[l], fm.kc[l]), (om.vcache[l], fm.vc[l])):
            o = oc[:21 * kvd].view(np.float16).astype(np.float64).reshape(21, kvd)
            f = fc[:21].astype(np.float64)
            # one fp16 rounding of a value whose fp32 and float64 forms differ
            # in the last fp32 bits: within an fp16 ulp of the row's scale
            assert (np.abs(o - f) <= 2.0 ** -10 * np.abs(f).max(axis=1, keepdims=True)).all(), l


@pytest.mark.parametrize("mistake", MISTAKES)
def test_planted_mistakes_fail_the_forward_check(xh, xo, mistake):
    """The same comparison with one misreading planted in the float64 model:
    it must fail (error at least twice the bar) at some position."""
    X = xh
    p = shape()
    om, get, _, _ = oracle_pair(X, xo, p, seed=3)
    fm = F64Model(p, get, mistakes=(mistake,))
    toks = np.random.default_rng(4).integers(0, p.vocab, 21)
    worst = max(rel_err(om.forward(int(t), pos, True), fm.forward(int(t), pos, True))
                for pos, t in enumerate(toks))
    assert worst > 2 * TOL, (mistake, worst)


def test_oracle_greedy_stream_matches_float64_and_varies(xh, xo):
    """Greedy ids (sample first, decode.cpp:1830-1861) from an untied fp32
    embedding table, so that the stream does not settle on one fixed point:
    the oracle's xo_generate_greedy equals the float64 model's argmax loop,
    the stream holds several distinct ids, and every decision is made by a
    top-2 gap far above the logit tolerance."""
    X = xh
    p = shape()
    om, get, embed, _ = oracle_pair(X, xo, p, seed=5, untied=True)
    fm = F64Model(p, get, embed=embed)
    prompt = np.random.default_rng(6).integers(0, p.vocab, 6).astype(np.uint32)
    n_gen = 16
    got = om.generate_greedy(prompt, n_gen)
    lg = None
    for i, t in enumerate(prompt):
        lg = fm.forward(int(t), i, i == len(prompt) - 1)
    want, gaps = [], []
    for s in range(n_gen):
        order = np.argsort(-lg, kind="stable")
        want.append(int(order[0]))
        gaps.append(float((lg[order[0]] - lg[order[1]]) / np.abs(lg).max()))
        lg = fm.forward(want[-1], len(prompt) + s, True)
    print("top-2 gaps / max|logits|:", " ".join(f"{g:.2e}" for g in gaps))
    assert list(got) == want
    assert len(set(want)) >= 6, want
    assert min(gaps) > 10 * TOL, gaps
