"""Batched decode (xp_batch_*): up to 16 sequences per step on one session's
weights, the matvecs as M = 16 MFMA GEMMs (benchmark config 5).

Every sequence is checked against the oracle run alone on the same packed
weights, its own KV cache and its own token ids: logits within 1e-3 relative
(|d| <= 1e-3 max|logits|), the appended K/V rows likewise (|d| <= 1e-3 max|row|;
the activations enter the GEMM as two bf16 terms, 2^-18 relative), the
device's 64 best candidates equal to the reference harvest (best 4 of 4096
strided chains, llm_sampling.cl:318-347) of the same logits reduced to its
64 best, bit for bit, and the drawn tokens equal to the host draw
(decode.cpp:1873-1917) over that harvest with Philox(seed, seq_id + i, step).
"""
import numpy as np
import pytest

from test_session import all_tensors, logits_close

HARVEST = 4096


def build(X, xo, cfg, seed=0x5EED0005):
    t = all_tensors(X, cfg, seed)
    sess = X.DecodeSession(cfg)
    for (l, k), a in t.items():
        sess.upload(l, k, a)
    return sess, t


def harvest_best(xo, logits, k=64):
    """The reference harvest of `logits`, then its k best by (value desc, index asc)."""
    n = logits.size
    cv = np.empty(4 * HARVEST, np.float32)
    ci = np.empty(4 * HARVEST, np.uint32)
    xo.lib().xo_topk4_partial(cv, ci, logits, n, HARVEST)
    keep = ci != 0xFFFFFFFF
    cv, ci = cv[keep], ci[keep]
    order = np.lexsort((ci, -cv))[:k]
    return cv, ci, cv[order], ci[order]


# ---------------------------------------------------------------- CPU ----

def test_batch_argument_errors(xh):
    X = xh
    with pytest.raises(X.XposeError):
        X.call("xp_batch_create", None, 4, 128, None)


# ---------------------------------------------------------------- GPU ----

@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["gemma3", "narrow"])
def test_gpu_batch_matches_oracle_per_sequence(xp, xo, shape):
    """Five sequences at different depths (two past the 512-position window of
    the local layers), greedy, three steps; the oracle runs each sequence
    alone. narrow: hidden 512, ffn 1024, 2 query heads, so the GEMMs take 2
    k blocks a wave (the loads under the chunk test) except the down
    projection's 4, and the lm_head is a plain GEMM, not the streamed one."""
    X = xp
    print(f"case batch vs oracle {shape}", flush=True)
    if shape == "gemma3":
        cfg = X.XpConfig.gemma3_1b(n_layers=6, vocab=32768, max_seq=1024)
    else:
        cfg = X.XpConfig.gemma3_1b(n_layers=3, hidden=512, ffn=1024, n_heads=2, n_kv_heads=1,
                                   vocab=32768, max_seq=1024, global_every=3)
    sess, t = build(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    depths = [3, 130, 511, 600, 1000]
    B = len(depths)
    batch = X.DecodeBatch(sess, B, cfg.max_seq)
    models = []
    for i, d in enumerate(depths):
        m = xo.OracleModel(cfg, lambda l, k: t[(l, k)])
        for l in range(cfg.n_layers):
            k = X.synth_normal_f16(d * kvd, 1000 + i, 2 * l)
            v = X.synth_normal_f16(d * kvd, 1000 + i, 2 * l + 1)
            batch.kv_upload(i, l, 0, 0, k)
            batch.kv_upload(i, l, 1, 0, v)
            m.kcache[l][:d * kvd] = k
            m.vcache[l][:d * kvd] = v
        models.append(m)
    batch.set_positions(depths)
    toks = np.array([7, 31000, 4242, 17, 9999], np.uint32)
    pos = np.array(depths)
    batch.forward(toks)
    for step in range(3):
        assert np.array_equal(batch.positions(), pos + 1)
        nxt = np.empty(B, np.uint32)
        for i in range(B):
            want = models[i].forward(int(toks[i]), int(pos[i]), True)
            got = batch.last_logits(i)
            ok, msg = logits_close(got, want)
            assert ok, f"step {step} seq {i} depth {pos[i]}: {msg}"
            for which, ref in ((0, models[i].kcache), (1, models[i].vcache)):
                row = batch.kv_download(i, 0, which, int(pos[i]), 1).view(np.float16)
                want_row = ref[0][pos[i] * kvd:(pos[i] + 1) * kvd].view(np.float16)
                err = np.abs(row.astype(np.float64) - want_row.astype(np.float64)).max()
                assert err <= 1e-3 * np.abs(want_row.astype(np.float64)).max(), (step, i, which, err)
            _, _, bv, bi = harvest_best(xo, got)
            gv, gi = batch.last_candidates(i)
            assert np.array_equal(gi, bi), (step, i)
            assert np.array_equal(gv.view(np.uint32), bv.view(np.uint32)), (step, i)
            nxt[i] = gi[0]
        # greedy: the drawn token is the best candidate; decode_step then
        # runs the network on it at the next position
        assert np.array_equal(batch.decode_step(), nxt)
        toks, pos = nxt, pos + 1
    batch.close()
    sess.close()


@pytest.mark.gpu
def test_gpu_batch_sampling_draws(xp, xo):
    """Temperature 0.8 / top-k 64 / top-p 0.95 per sequence, Philox key
    (seed, seq_id + i): the drawn tokens equal the host draw over the
    reference harvest of each sequence's device logits."""
    X = xp
    print("case batch sampling", flush=True)
    cfg = X.XpConfig.gemma3_1b(n_layers=2, vocab=65536, max_seq=512, sample_mode=1,
                               temperature=0.8, top_k=64, top_p=0.95, seed=1234, seq_id=40)
    sess, t = build(X, xo, cfg)
    B = 16
    batch = X.DecodeBatch(sess, B, cfg.max_seq)
    r = np.random.default_rng(5)
    batch.set_positions(r.integers(0, 300, B))
    batch.forward(r.integers(0, cfg.vocab, B))
    for step in range(6):
        want = np.empty(B, np.uint32)
        for i in range(B):
            cv, ci, _, _ = harvest_best(xo, batch.last_logits(i))
            u = xo.lib().xo_philox_uniform(1234, 40 + i, step)
            want[i] = xo.lib().xo_draw(cv.copy(), ci.copy(), cv.size, 0.8, 64, 0.95, u)
        got = batch.decode_step()
        assert np.array_equal(got, want), step
    batch.close()
    sess.close()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["sample", "greedy"])
def test_gpu_batch_decode_steps_equals_steps(xp, xo, mode):
    """xp_batch_decode_steps (the draws after the first on the device, the
    steps queued back to back) gives the tokens, positions, last candidates
    and appended K/V rows of as many xp_batch_decode_step calls on a batch
    built alike: 270 steps, i.e. a chain of 257 and one of 13 (the device
    keeps 256 draws between host reads), then one more step each way."""
    X = xp
    print(f"case batch decode_steps {mode}", flush=True)
    sample = mode == "sample"
    # an untied fp32 N(0, 1) embedding table and temperature 2 so that the
    # streams move and the draws spread over several candidates
    cfg = X.XpConfig.gemma3_1b(n_layers=2, vocab=16384, max_seq=512, sample_mode=1 if sample else 0,
                               temperature=2.0, top_k=64, top_p=0.95, seed=1234, seq_id=40)
    sess, t = build(X, xo, cfg)
    emb = np.random.default_rng(11).normal(0, 1, (cfg.vocab, cfg.hidden)).astype(np.float32)
    sess.upload(-1, X.T_EMBED, emb)
    B = 16
    r = np.random.default_rng(7)
    pos0 = r.integers(0, 200, B)
    tok0 = r.integers(0, cfg.vocab, B)
    a = X.DecodeBatch(sess, B, cfg.max_seq)
    b = X.DecodeBatch(sess, B, cfg.max_seq)
    for x in (a, b):
        x.set_positions(pos0)
        x.forward(tok0)
    n = 270
    want = np.stack([a.decode_step() for _ in range(n)])
    got = b.decode_steps(n)
    assert np.array_equal(got, want)
    # the streams move
    assert min(len(np.unique(want[:, i])) for i in range(B)) > 5
    assert np.array_equal(a.positions(), b.positions())
    for i in range(B):
        va, ia = a.last_candidates(i)
        vb, ib = b.last_candidates(i)
        assert np.array_equal(ia, ib) and np.array_equal(va.view(np.uint32), vb.view(np.uint32)), i
    for i in (0, 7, 15):
        for layer in (0, 1):
            for which in (0, 1):
                ka = a.kv_download(i, layer, which, int(pos0[i]), n + 1)
                kb = b.kv_download(i, layer, which, int(pos0[i]), n + 1)
                assert np.array_equal(ka, kb), (i, layer, which)
    assert np.array_equal(a.decode_step(), b.decode_step())
    a.close()
    b.close()
    sess.close()


@pytest.mark.gpu
def test_gpu_batch_full_size_cfg5(xp, xo):
    """Benchmark config 5 at full size: 26 layers, vocab 262144, 16 sequences
    at the benchmark's Philox depths in [128, 4096] (global-layer spans to
    ~4000), T 0.8 / top-k 64 / top-p 0.95. Each sequence against the oracle
    run alone on its own KV cache for two steps: logits, appended K/V rows,
    the 64 device candidates and the drawn tokens."""
    X = xp
    print("case batch full-size cfg5", flush=True)
    seed = 0x5EED0005
    cfg = X.XpConfig.gemma3_1b(max_seq=4104, sample_mode=1, temperature=0.8, top_k=64,
                               top_p=0.95, seed=seed, seq_id=0)
    sess, t = build(X, xo, cfg)
    n_seq = 16
    u = np.array([X.philox_uniform(seed, i, 0) for i in range(n_seq)])
    depths = (128 + np.floor(u * (4096 - 128 + 1))).astype(np.int64)   # as bench.py's cfg5 leg
    assert depths.max() > 3000 and depths.min() < 1000, depths
    kvd = cfg.n_kv_heads * cfg.head_dim
    batch = X.DecodeBatch(sess, n_seq, cfg.max_seq)
    models = []
    for i, d in enumerate(depths):
        m = xo.OracleModel(cfg, lambda l, k: t[(l, k)])
        for l in range(cfg.n_layers):
            for which, cache in ((0, m.kcache), (1, m.vcache)):
                rows = X.synth_normal_f16(int(d) * kvd, 5000 + i, 2 * l + which)
                batch.kv_upload(i, l, which, 0, rows)
                cache[l][:int(d) * kvd] = rows
        models.append(m)
    batch.set_positions(depths)
    toks = (np.arange(n_seq) * 16381 + 7).astype(np.uint32) % cfg.vocab
    pos = depths.copy()
    batch.forward(toks)
    for step in range(2):
        want_tok = np.empty(n_seq, np.uint32)
        for i in range(n_seq):
            want = models[i].forward(int(toks[i]), int(pos[i]), True, 16)
            got = batch.last_logits(i)
            ok, msg = logits_close(got, want)
            assert ok, f"step {step} seq {i} depth {pos[i]}: {msg}"
            for which, ref in ((0, models[i].kcache), (1, models[i].vcache)):
                for l in (0, 5, 25):
                    row = batch.kv_download(i, l, which, int(pos[i]), 1).view(np.float16)
                    want_row = ref[l][pos[i] * kvd:(pos[i] + 1) * kvd].view(np.float16)
                    err = np.abs(row.astype(np.float64) - want_row.astype(np.float64)).max()
                    assert err <= 1e-3 * np.abs(want_row.astype(np.float64)).max(), (step, i, l, which)
            cv, ci, bv, bi = harvest_best(xo, got)
            gv, gi = batch.last_candidates(i)
            assert np.array_equal(gi, bi), (step, i)
            assert np.array_equal(gv.view(np.uint32), bv.view(np.uint32)), (step, i)
            uu = xo.lib().xo_philox_uniform(seed, i, step)
            want_tok[i] = xo.lib().xo_draw(cv.copy(), ci.copy(), cv.size, 0.8, 64, 0.95, uu)
        got_tok = batch.decode_step()
        assert np.array_equal(got_tok, want_tok), step
        toks, pos = got_tok, pos + 1
    print("cfg5 draws distinct per step:", len(set(toks.tolist())), flush=True)
    batch.close()
    sess.close()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["window", "global3"])
def test_gpu_batch_step_kernel_equals_graph(xp, xo, shape):
    """The persistent step kernel (XP_EXEC_TOKEN) against the graph of
    per-op kernels (XP_EXEC_GRAPH) on the same weights, caches, positions and
    tokens: both run the same tile code in the same order, so logits,
    candidates, appended K/V rows and greedy ids are equal bit for bit.
    window: 6 layers (one global), 16 sequences at depths 3..1000, most past
    the 512-position window. global3: 4 layers, every second global, max_seq
    4104 with the benchmark's depths (global attention in splits of three
    128-key passes, the U = 8 tile)."""
    X = xp
    print(f"case batch step kernel vs graph {shape}", flush=True)
    n_seq = 16
    if shape == "window":
        cfg = X.XpConfig.gemma3_1b(n_layers=6, vocab=32768, max_seq=1024)
        depths = np.linspace(3, 1000, n_seq).astype(np.int64)
    else:
        seed = 0x5EED0005
        cfg = X.XpConfig.gemma3_1b(n_layers=4, global_every=2, vocab=32768, max_seq=4104)
        u = np.array([X.philox_uniform(seed, i, 0) for i in range(n_seq)])
        depths = (128 + np.floor(u * (4096 - 128 + 1))).astype(np.int64)
    sess, t = build(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    bt = X.DecodeBatch(sess, n_seq, cfg.max_seq, X.XP_EXEC_TOKEN)
    bg = X.DecodeBatch(sess, n_seq, cfg.max_seq, X.XP_EXEC_GRAPH)
    assert bt.exec_mode() == X.XP_EXEC_TOKEN and bg.exec_mode() == X.XP_EXEC_GRAPH
    for i, d in enumerate(depths):
        for l in range(cfg.n_layers):
            for which in (0, 1):
                rows = X.synth_normal_f16(int(d) * kvd, 7000 + i, 2 * l + which)
                bt.kv_upload(i, l, which, 0, rows)
                bg.kv_upload(i, l, which, 0, rows)
    bt.set_positions(depths)
    bg.set_positions(depths)
    toks = (np.arange(n_seq) * 7919 + 11).astype(np.uint32) % cfg.vocab
    bt.forward(toks)
    bg.forward(toks)
    pos = depths.copy()
    for step in range(3):
        for i in range(n_seq):
            a, b = bt.last_logits(i), bg.last_logits(i)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (step, i, np.abs(a - b).max())
            va, ia = bt.last_candidates(i)
            vb, ib = bg.last_candidates(i)
            assert np.array_equal(ia, ib) and np.array_equal(va.view(np.uint32), vb.view(np.uint32)), (step, i)
            for l in range(cfg.n_layers):
                for which in (0, 1):
                    ka = bt.kv_download(i, l, which, int(pos[i]), 1)
                    kb = bg.kv_download(i, l, which, int(pos[i]), 1)
                    assert np.array_equal(ka, kb), (step, i, l, which)
        if step < 2:
            ta, tb = bt.decode_step(), bg.decode_step()
            assert np.array_equal(ta, tb), step
            pos = pos + 1
    assert np.array_equal(bt.positions(), bg.positions())
    bt.close()
    bg.close()
    sess.close()


@pytest.mark.gpu
def test_gpu_batch_exec_modes(xp, xo):
    """xp_batch_create2's modes: AUTO takes the graph (the faster), TOKEN the
    step kernel on a free GPU, an unknown mode is refused."""
    X = xp
    print("case batch exec modes", flush=True)
    cfg = X.XpConfig.gemma3_1b(n_layers=1, vocab=16384, max_seq=256)
    sess, _ = build(X, xo, cfg)
    b = X.DecodeBatch(sess, 3, 256)
    assert b.exec_mode() == X.XP_EXEC_GRAPH
    b.close()
    b = X.DecodeBatch(sess, 3, 256, X.XP_EXEC_TOKEN)
    assert b.exec_mode() == X.XP_EXEC_TOKEN
    b.close()
    with pytest.raises(X.XposeError):
        X.DecodeBatch(sess, 3, 256, X.XP_EXEC_LAUNCH)
    sess.close()


@pytest.mark.gpu
def test_gpu_batch_step_kernel_timeout_recovers(xp, xo):
    """The step kernel's bounded waits, forced from the host: with a spin
    limit of 0 a wait gives up at its first incomplete poll, every
    workgroup still finishes, and the step returns XP_E_DEVICE with the
    positions unchanged; with the default limit back, the same step gives the
    graph's results bit for bit (its KV rows rewritten)."""
    X = xp
    print("case batch step kernel forced timeout", flush=True)
    cfg = X.XpConfig.gemma3_1b(n_layers=2, vocab=16384, max_seq=512)
    sess, _ = build(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    n_seq = 4
    depths = np.array([5, 100, 300, 511 - 8], np.int64)
    bt = X.DecodeBatch(sess, n_seq, 512, X.XP_EXEC_TOKEN)
    bg = X.DecodeBatch(sess, n_seq, 512, X.XP_EXEC_GRAPH)
    for i, d in enumerate(depths):
        for l in range(cfg.n_layers):
            for which in (0, 1):
                rows = X.synth_normal_f16(int(d) * kvd, 900 + i, 2 * l + which)
                bt.kv_upload(i, l, which, 0, rows)
                bg.kv_upload(i, l, which, 0, rows)
    bt.set_positions(depths)
    bg.set_positions(depths)

    def same(pos):
        for i in range(n_seq):
            a, b = bt.last_logits(i), bg.last_logits(i)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (i, np.abs(a - b).max())
            for l in range(cfg.n_layers):
                for which in (0, 1):
                    assert np.array_equal(bt.kv_download(i, l, which, int(pos[i]), 1),
                                          bg.kv_download(i, l, which, int(pos[i]), 1)), (i, l, which)

    toks = [11, 222, 3333, 4444]
    bt.forward(toks)
    bg.forward(toks)
    same(depths)
    toks = [5, 66, 777, 8888]
    bt.set_spin_limit(0)
    with pytest.raises(X.XposeError) as ei:
        bt.forward(toks)
    assert "limit" in str(ei.value), ei.value
    assert np.array_equal(bt.positions(), depths + 1)
    bt.set_spin_limit(1 << 20)
    bt.forward(toks)
    bg.forward(toks)
    same(depths + 1)
    assert np.array_equal(bt.positions(), depths + 2)
    bt.close()
    bg.close()
    sess.close()


@pytest.mark.gpu
def test_gpu_batch_one_sequence_equals_session(xp, xo):
    """A batch of one sequence and the single-sequence session (persistent
    token kernel) on the same weights and KV give the same logits to the
    end-to-end bar."""
    X = xp
    print("case batch of one vs session", flush=True)
    cfg = X.XpConfig.gemma3_1b(n_layers=4, vocab=32768, max_seq=1024)
    sess, t = build(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    batch = X.DecodeBatch(sess, 1, cfg.max_seq)
    for l in range(cfg.n_layers):
        for which in (0, 1):
            rows = X.synth_normal_f16(700 * kvd, 3, 2 * l + which)
            sess.kv_upload(l, which, 0, rows)
            batch.kv_upload(0, l, which, 0, rows)
    sess.set_position(700)
    batch.set_positions([700])
    sess.prefill([555])
    batch.forward([555])
    ok, msg = logits_close(batch.last_logits(0), sess.last_logits())
    assert ok, msg
    batch.close()
    sess.close()


@pytest.mark.gpu
def test_gpu_batch_error_paths(xp, xo):
    X = xp
    print("case batch errors", flush=True)
    cfg = X.XpConfig.gemma3_1b(n_layers=1, vocab=16384, max_seq=256)
    sess, _ = build(X, xo, cfg)
    for n in (0, 17):
        with pytest.raises(X.XposeError):
            X.DecodeBatch(sess, n, 256)
    with pytest.raises(X.XposeError):
        X.DecodeBatch(sess, 2, 9000)
    b = X.DecodeBatch(sess, 2, 256)
    with pytest.raises(X.XposeError):
        b.set_positions([0, 256])
    with pytest.raises(X.XposeError):
        b.decode_step()                       # no logits yet
    b.set_positions([254, 255])
    b.forward([1, 2])
    with pytest.raises(X.XposeError):
        b.forward([1, 2])                     # sequence 1 is at max_seq
    with pytest.raises(X.XposeError):
        b.forward([1, 99999])                 # token >= vocab
    b.close()
    sess.close()


@pytest.mark.gpu
def test_gpu_batch_graph_attention_timeout_recovers(xp, xo):
    """The batched graph's exchange-mode decode attention (the global layer of
    a 6-layer model at max_seq 1024: 2 sequences x 32 splits, all resident)
    with its spin limit forced to 0: the step returns XP_E_DEVICE, the
    positions stay, the records and tickets start over, and the same step
    run again with the default limit equals a second batch's, bit for bit."""
    X = xp
    print("case batch graph attention forced timeout", flush=True)
    cfg = X.XpConfig.gemma3_1b(n_layers=6, vocab=16384, max_seq=1024)
    sess, _ = build(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    depths = np.array([300, 700], np.int64)
    ba = X.DecodeBatch(sess, 2, 1024, X.XP_EXEC_GRAPH)
    bb = X.DecodeBatch(sess, 2, 1024, X.XP_EXEC_GRAPH)
    for i, d in enumerate(depths):
        for l in range(cfg.n_layers):
            for which in (0, 1):
                rows = X.synth_normal_f16(int(d) * kvd, 50 + i, 2 * l + which)
                ba.kv_upload(i, l, which, 0, rows)
                bb.kv_upload(i, l, which, 0, rows)
    ba.set_positions(depths)
    bb.set_positions(depths)
    ba.forward([11, 22])
    bb.forward([11, 22])
    ba.set_spin_limit(0)
    with pytest.raises(X.XposeError) as ei:
        ba.forward([33, 44])
    assert ei.value.code == -5 and "limit" in str(ei.value), ei.value
    assert np.array_equal(ba.positions(), depths + 1)
    ba.set_spin_limit(1 << 18)
    ba.forward([33, 44])
    bb.forward([33, 44])
    for i in range(2):
        assert np.array_equal(ba.last_logits(i).view(np.uint32), bb.last_logits(i).view(np.uint32)), i
        for l in range(cfg.n_layers):
            for which in (0, 1):
                assert np.array_equal(ba.kv_download(i, l, which, int(depths[i]) + 1, 1),
                                      bb.kv_download(i, l, which, int(depths[i]) + 1, 1)), (i, l, which)
    ba.close()
    bb.close()
    sess.close()
