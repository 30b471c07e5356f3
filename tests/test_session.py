"""The decode session (engine level): the token step of DecodeSession
(examples/llm/decode.cpp:1634-1866) on the GPU against the oracle's
xo_forward on the same packed weights, KV contents and token ids.

Bars (the benchmark specification): greedy token ids bit-exact; logits within 1e-3
relative (|d| <= 1e-3 * max|logits|); KV rows within one fp16 ulp.
"""
import numpy as np
import pytest

LOGIT_TOL = 1e-3

# Every engine-level GPU test runs on both executions of the token step: the
# persistent token kernel (token_kernel.hip) and the captured graph of per-op
# kernels. XP_EXEC_TOKEN makes session creation fail rather than fall back.
EXEC_MODES = [pytest.param(3, id="token"), pytest.param(1, id="graph")]


@pytest.fixture(params=EXEC_MODES)
def mode(request):
    return request.param


def cfg_small(X, **kw):
    base = dict(n_layers=6, vocab=32768, max_seq=1024)
    base.update(kw)
    return X.XpConfig.gemma3_1b(**base)


def all_tensors(X, cfg, seed):
    t = {}
    for l in range(cfg.n_layers):
        for m in X.MATRICES:
            t[(l, m)] = X.synth_tensor(cfg, seed, l, m)
            t[(l, m | X.T_SCALES)] = X.synth_tensor(cfg, seed, l, m | X.T_SCALES)
        for n in X.NORMS:
            t[(l, n)] = X.synth_tensor(cfg, seed, l, n)
    for k in (X.T_LM_HEAD, X.T_LM_HEAD | X.T_SCALES, X.T_FINAL_NORM):
        t[(-1, k)] = X.synth_tensor(cfg, seed, -1, k)
    return t


def make_pair(X, xo, cfg, seed=0x5EED0002):
    t = all_tensors(X, cfg, seed)
    sess = X.DecodeSession(cfg)
    assert sess.exec_mode == cfg.exec_mode
    for (l, k), a in t.items():
        sess.upload(l, k, a)
    model = xo.OracleModel(cfg, lambda l, k: t[(l, k)])
    return sess, model


def logits_close(got, want):
    err = np.abs(got.astype(np.float64) - want).max()
    return err <= LOGIT_TOL * np.abs(want).max(), f"max_abs={err:.3e} max|want|={np.abs(want).max():.3e}"


def top5(x):
    return np.lexsort((np.arange(x.size), -x))[:5]


# ---------------------------------------------------------------- CPU ----

def test_weight_bytes_match_the_algorithmic_count(xh):
    """Nibbles + fp16 scales of one Gemma-3-1B token = 562,360,320 B, the
    figure the HBM roofline is priced on (reference: 536.3 MiB,
    agent-docs/llm-inference.md:105)."""
    X = xh
    cfg = X.XpConfig.gemma3_1b()
    total = 0
    for l in range(cfg.n_layers):
        for m in X.MATRICES:
            total += X.tensor_bytes(cfg, l, m) + X.tensor_bytes(cfg, l, m | X.T_SCALES)
    total += X.tensor_bytes(cfg, -1, X.T_LM_HEAD) + X.tensor_bytes(cfg, -1, X.T_LM_HEAD | X.T_SCALES)
    assert total == 562_360_320
    assert X.tensor_bytes(cfg, 0, X.T_GATE) == 1152 * 6912 // 2
    assert X.tensor_bytes(cfg, 0, X.T_GATE | X.T_SCALES) == 36 * 6912 * 2


def test_synth_tensor_is_deterministic(xh):
    X = xh
    cfg = cfg_small(X, n_layers=2)
    a = X.synth_tensor(cfg, 5, 1, X.T_DOWN)
    assert np.array_equal(a, X.synth_tensor(cfg, 5, 1, X.T_DOWN))
    assert not np.array_equal(a, X.synth_tensor(cfg, 6, 1, X.T_DOWN))
    n = X.synth_tensor(cfg, 5, 0, X.T_Q_NORM)
    assert n.size == 256 and abs(n.mean()) < 0.03 and 0.07 < n.std() < 0.13


def test_config_and_tensor_errors(xh):
    X = xh
    bad = X.XpConfig.gemma3_1b(head_dim=1024)
    with pytest.raises(X.XposeError) as e:
        X.DecodeSession(bad)
    assert "head_dim" in str(e.value)
    cfg = X.XpConfig.gemma3_1b()
    with pytest.raises(X.XposeError):
        X.tensor_bytes(cfg, 26, X.T_Q)
    with pytest.raises(X.XposeError):
        X.tensor_bytes(cfg, 0, X.T_LM_HEAD)


def test_oracle_embedding_closed_form(xh, xo):
    X = xh
    cfg = cfg_small(X, n_layers=1, vocab=4096)
    t = all_tensors(X, cfg, 11)
    model = xo.OracleModel(cfg, lambda l, k: t[(l, k)])
    import ctypes as C
    tok = 3001
    x = np.empty(cfg.hidden, np.float32)
    xo.lib().xo_embed(x, C.byref(model.model), tok)
    W = np.empty(cfg.hidden * cfg.vocab, np.int8)
    xo.lib().xo_unpack_km4(W, t[(-1, X.T_LM_HEAD)], cfg.hidden, cfg.vocab)
    W = W.reshape(cfg.hidden, cfg.vocab)
    sc = t[(-1, X.T_LM_HEAD | X.T_SCALES)].reshape(cfg.hidden // 128, cfg.vocab, 4)
    s = sc.transpose(0, 2, 1).reshape(cfg.hidden // 32, cfg.vocab).view(np.float16)
    col = W[:, tok].astype(np.float32) * np.repeat(s[:, tok].astype(np.float32), 32)
    assert np.array_equal(x, (col * np.float32(np.sqrt(np.float32(1152)))).astype(np.float32))


def test_oracle_generate_matches_forward_loop(xh, xo):
    """xo_generate_greedy == prefill + sample-first decode written out."""
    X = xh
    cfg = cfg_small(X, n_layers=2, vocab=4096, max_seq=64)
    t = all_tensors(X, cfg, 12)
    ids = xo.OracleModel(cfg, lambda l, k: t[(l, k)]).generate_greedy([5, 9, 3], 4)
    m = xo.OracleModel(cfg, lambda l, k: t[(l, k)])
    m.forward(5, 0, False)
    m.forward(9, 1, False)
    lg = m.forward(3, 2, True)
    out = []
    for pos in range(3, 7):
        tok = xo.argmax_tree(lg)[0]
        out.append(tok)
        lg = m.forward(tok, pos, True)
    assert list(ids) == out


# ---------------------------------------------------------------- GPU ----

@pytest.mark.gpu
def test_gpu_one_layer_cfg2(xp, xo, mode):
    """benchmark config 2: one local Gemma-3-1B layer, 512 prior fp16 KV rows
    ~ N(0,1), decode at position 512 (kv_start 1, span 512)."""
    X = xp
    print("case session one-layer cfg2", flush=True)
    cfg = X.XpConfig.gemma3_1b(n_layers=1, max_seq=1024, exec_mode=mode)
    sess, model = make_pair(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    k = X.synth_normal_f16(512 * kvd, 77, 1)
    v = X.synth_normal_f16(512 * kvd, 77, 2)
    sess.kv_upload(0, 0, 0, k)
    sess.kv_upload(0, 1, 0, v)
    model.kcache[0][:512 * kvd] = k
    model.vcache[0][:512 * kvd] = v
    sess.set_position(512)
    sess.prefill([123456])
    want = model.forward(123456, 512, True)
    ok, msg = logits_close(sess.last_logits(), want)
    assert ok, msg
    for which, ref in ((0, model.kcache[0]), (1, model.vcache[0])):
        row = sess.kv_download(0, which, 512, 1).astype(np.int32)
        assert np.abs(row - ref[512 * kvd:513 * kvd].astype(np.int32)).max() <= 1
        assert np.array_equal(sess.kv_download(0, which, 0, 512), ref[:512 * kvd])


@pytest.mark.gpu
def test_gpu_small_model_greedy(xp, xo, mode):
    X = xp
    print("case session small greedy", flush=True)
    cfg = cfg_small(X, exec_mode=mode)
    sess, model = make_pair(X, xo, cfg)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 32).astype(np.uint32)
    want = model.generate_greedy(prompt, 24)
    sess.prefill(prompt)
    got = [sess.decode_step() for _ in range(24)]
    assert list(want) == got
    assert sess.position == 32 + 24


@pytest.mark.gpu
def test_gpu_small_model_logits_every_step(xp, xo, mode):
    X = xp
    print("case session small logits", flush=True)
    cfg = cfg_small(X, n_layers=7, vocab=16384, exec_mode=mode)
    sess, model = make_pair(X, xo, cfg)
    prompt = [7, 1000, 16000, 3]
    for i, t in enumerate(prompt[:-1]):
        model.forward(t, i, False)
    lg = model.forward(prompt[-1], len(prompt) - 1, True)
    sess.prefill(prompt)
    ok, msg = logits_close(sess.last_logits(), lg)
    assert ok, msg
    pos = len(prompt)
    for step in range(12):
        tok = sess.decode_step()
        assert tok == xo.argmax_tree(lg)[0]
        lg = model.forward(tok, pos, True)
        got = sess.last_logits()
        ok, msg = logits_close(got, lg)
        assert ok, f"step {step}: {msg}"
        assert np.array_equal(top5(got), top5(lg)), step
        pos += 1


@pytest.mark.gpu
def test_gpu_decode_steps_equals_decode_step(xp, xo, mode):
    X = xp
    print("case session decode_steps", flush=True)
    cfg = cfg_small(X, n_layers=3, exec_mode=mode)
    t = all_tensors(X, cfg, 21)
    a, b = X.DecodeSession(cfg), X.DecodeSession(cfg)
    assert a.exec_mode == b.exec_mode == mode
    for (l, k), arr in t.items():
        a.upload(l, k, arr)
        b.upload(l, k, arr)
    a.prefill([1, 2, 3])
    b.prefill([1, 2, 3])
    many = a.decode_steps(20)
    one = [b.decode_step() for _ in range(20)]
    assert list(many) == one
    assert np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32))


@pytest.mark.gpu
def test_gpu_full_model_greedy_cfg3(xp, xo, mode):
    """benchmark config 3 (shortened): full Gemma-3-1B architecture, random
    int4 weights, tied 262144 x 1152 table; prefill then greedy decode."""
    X = xp
    print("case session full model cfg3", flush=True)
    cfg = X.XpConfig.gemma3_1b(max_seq=2048, exec_mode=mode)
    sess, model = make_pair(X, xo, cfg)
    prompt = np.random.default_rng(32).integers(0, cfg.vocab, 8).astype(np.uint32)
    for i, t in enumerate(prompt[:-1]):
        model.forward(int(t), i, False, 16)
    lg = model.forward(int(prompt[-1]), len(prompt) - 1, True, 16)
    sess.prefill(prompt)
    ok, msg = logits_close(sess.last_logits(), lg)
    assert ok, msg
    pos = len(prompt)
    for step in range(6):
        tok = sess.decode_step()
        assert tok == xo.argmax_tree(lg)[0], step
        lg = model.forward(tok, pos, True, 16)
        ok, msg = logits_close(sess.last_logits(), lg)
        assert ok, f"step {step}: {msg}"
        pos += 1


@pytest.mark.gpu
def test_gpu_full_model_deep_context_cfg4(xp, xo, mode):
    """benchmark config 4 (shortened): KV of all 26 layers pre-filled with fp16
    N(0,1) to position 4096; decode from 4096 (global layers span 4097,
    local layers the last 512)."""
    X = xp
    print("case session full model cfg4", flush=True)
    deep_context_check(X, xo, X.XpConfig.gemma3_1b(max_seq=4160, exec_mode=mode))


@pytest.mark.gpu
def test_gpu_token_device_placement_cfg4(xp, xo):
    """Config 4 on the token kernel with XP_PLACE_DEVICE: every exchange
    through the device coherence point and 32-key attention chunks in the
    local layers, the path a device whose workgroup placement the session's
    probe cannot verify takes."""
    X = xp
    print("case session token device placement cfg4", flush=True)
    deep_context_check(X, xo, X.XpConfig.gemma3_1b(max_seq=4160, exec_mode=X.XP_EXEC_TOKEN,
                                                     placement=X.XP_PLACE_DEVICE))


def deep_context_check(X, xo, cfg, fill=4096, steps=3):
    sess, model = make_pair(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    for l in range(cfg.n_layers):
        for which, cache in ((0, model.kcache), (1, model.vcache)):
            rows = X.synth_normal_f16(fill * kvd, 4096, 2 * l + which)
            sess.kv_upload(l, which, 0, rows)
            cache[l][:fill * kvd] = rows
    sess.set_position(fill)
    sess.prefill([4242])
    lg = model.forward(4242, fill, True, 16)
    ok, msg = logits_close(sess.last_logits(), lg)
    assert ok, msg
    pos = fill + 1
    for step in range(steps):
        tok = sess.decode_step()
        assert tok == xo.argmax_tree(lg)[0]
        lg = model.forward(tok, pos, True, 16)
        ok, msg = logits_close(sess.last_logits(), lg)
        assert ok, f"step {step}: {msg}"
        pos += 1
    return sess


DEEP_MODES = [pytest.param(3, 0, id="token-auto"), pytest.param(3, 1, id="token-device"),
              pytest.param(1, 0, id="graph")]


@pytest.mark.gpu
@pytest.mark.parametrize("exec_mode,placement", DEEP_MODES)
def test_gpu_full_model_max_context_8192(xp, xo, exec_mode, placement):
    """The deep end of benchmark config 4 at the default max_seq 8192: KV of
    all 26 layers pre-filled to position 8190, then positions 8190 and 8191
    (the last the cache holds): the global layers attend 8191 and 8192
    keys, which on the token kernel is 256 attention chunks, every
    workgroup of the global combine."""
    X = xp
    print(f"case session max context 8192 exec {exec_mode} placement {placement}", flush=True)
    cfg = X.XpConfig.gemma3_1b(exec_mode=exec_mode, placement=placement)
    assert cfg.max_seq == 8192
    sess = deep_context_check(X, xo, cfg, fill=8190, steps=1)
    assert sess.position == 8192
    with pytest.raises(X.XposeError):
        sess.decode_step()                   # the cache is full
    sess.close()


def untied_pair(X, xo, cfg, seed, embed_seed):
    """make_pair plus an fp32 N(0, 1) embedding table (XP_T_EMBED) that is not
    the lm_head: a greedy stream then moves from token to token instead of
    settling on the fixed point a tied random table has."""
    t = all_tensors(X, cfg, seed)
    emb = np.random.default_rng(embed_seed).normal(0, 1, (cfg.vocab, cfg.hidden)).astype(np.float32)
    sess = X.DecodeSession(cfg)
    assert sess.exec_mode == cfg.exec_mode
    for (l, k), a in t.items():
        sess.upload(l, k, a)
    sess.upload(-1, X.T_EMBED, emb)
    model = xo.OracleModel(cfg, lambda l, k: t[(l, k)], embed=emb)
    return sess, model


def greedy_stream_check(xo, sess, model, prompt, n_gen, min_distinct):
    """Sample-first greedy decode (decode.cpp:1830-1861) against the oracle:
    every id equal, logits within 1e-3 at every step, the stream holding at
    least min_distinct ids; prints the oracle's top-2 gap of each decision."""
    lg = None
    for i, t in enumerate(prompt):
        lg = model.forward(int(t), i, i == len(prompt) - 1, 16)
    sess.prefill(prompt)
    ids, gaps = [], []
    for step in range(n_gen):
        ok, msg = logits_close(sess.last_logits(), lg)
        assert ok, f"step {step}: {msg}"
        order = top5(lg)
        gaps.append(float((lg[order[0]] - lg[order[1]]) / np.abs(lg).max()))
        tok = sess.decode_step()
        assert tok == int(order[0]), (step, tok, int(order[0]))
        ids.append(tok)
        lg = model.forward(tok, len(prompt) + step, True, 16)
    print("ids", ids, "top-2 gaps / max|logits|:", " ".join(f"{g:.1e}" for g in gaps), flush=True)
    assert len(set(ids)) >= min_distinct, ids


@pytest.mark.gpu
def test_gpu_greedy_stream_varies(xp, xo, mode):
    """24 greedy tokens after a 32-token prompt on a 6-layer model with an
    untied table: 24 distinct ids on the oracle (smallest top-2 gap 5e-3 of
    max|logits|), each equal on the GPU."""
    X = xp
    print("case session varying greedy stream", flush=True)
    cfg = cfg_small(X, exec_mode=mode)
    sess, model = untied_pair(X, xo, cfg, 0x5EED0002, 17)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 32).astype(np.uint32)
    greedy_stream_check(xo, sess, model, prompt, 24, 16)
    sess.close()


@pytest.mark.gpu
def test_gpu_full_model_greedy_stream_varies(xp, xo, mode):
    """The full Gemma-3-1B shape with an untied 262144 x 1152 fp32 table: 12
    greedy tokens after an 8-token prompt, 10 distinct ids on the oracle
    (smallest top-2 gap 4e-3 of max|logits|), each equal on the GPU."""
    X = xp
    print("case session full model varying greedy stream", flush=True)
    cfg = X.XpConfig.gemma3_1b(max_seq=2048, exec_mode=mode)
    sess, model = untied_pair(X, xo, cfg, 0x5EED0002, 18)
    prompt = np.random.default_rng(32).integers(0, cfg.vocab, 8).astype(np.uint32)
    greedy_stream_check(xo, sess, model, prompt, 12, 8)
    sess.close()


@pytest.mark.gpu
def test_gpu_temperature_sampling(xp, xo, mode):
    """Temperature 0.8 / top-k 64 / top-p 0.95 over the top-4-per-chain
    harvest, Philox uniform per (sequence, step) (benchmark config 5 draw)."""
    X = xp
    print("case session temperature", flush=True)
    cfg = cfg_small(X, n_layers=4, sample_mode=1, temperature=0.8, top_k=64, top_p=0.95,
                    seed=99, seq_id=3, topk_parts=1024, exec_mode=mode)
    sess, model = make_pair(X, xo, cfg)
    prompt = [11, 22, 33]
    for i, t in enumerate(prompt[:-1]):
        model.forward(t, i, False)
    lg = model.forward(prompt[-1], 2, True)
    sess.prefill(prompt)
    pos = 3
    for step in range(16):
        # Logits agree with the oracle to the end-to-end bar; the harvest is
        # then checked bit for bit on the same (device) logits, since logits
        # that differ in the last bits may legitimately swap near-tied
        # candidates of a chain.
        got = sess.last_logits()
        ok, msg = logits_close(got, lg)
        assert ok, f"step {step}: {msg}"
        cv = np.empty(4096, np.float32)
        ci = np.empty(4096, np.uint32)
        xo.lib().xo_topk4_partial(cv, ci, got, cfg.vocab, 1024)
        gv, gi = sess.last_candidates()
        assert np.array_equal(gi, ci), step          # same candidate set
        assert np.array_equal(gv.view(np.uint32), cv.view(np.uint32)), step
        keep = ci != 0xFFFFFFFF
        u = xo.lib().xo_philox_uniform(99, 3, step)
        want = xo.lib().xo_draw(cv[keep].copy(), ci[keep].copy(), int(keep.sum()), 0.8, 64,
                                0.95, u)
        tok = sess.decode_step()
        assert tok == want, step
        lg = model.forward(tok, pos, True)
        pos += 1


@pytest.mark.gpu
def test_gpu_session_error_paths(xp):
    X = xp
    cfg = cfg_small(X, n_layers=1, max_seq=16)
    s = X.DecodeSession(cfg)
    s.synthesize(1)
    with pytest.raises(X.XposeError) as e:
        s.decode_step()
    assert e.value.code == -4
    with pytest.raises(X.XposeError):
        s.prefill(list(range(17)))
    with pytest.raises(X.XposeError):
        s.prefill([cfg.vocab])
    s.prefill(list(range(15)))
    s.decode_step()
    with pytest.raises(X.XposeError) as e:
        s.decode_step()
    assert "full" in str(e.value)
    with pytest.raises(X.XposeError) as e:
        X.DecodeSession(cfg_small(X, n_layers=1, max_seq=16, placement=7))
    assert "placement" in str(e.value)


@pytest.mark.gpu
def test_gpu_batched_prefill(xp, xo, mode):
    """xp_session_prefill with XP_PREFILL_AUTO runs the first n - 1 prompt
    tokens through the batched step (16 positions per pass on the session's
    KV cache): against the oracle's token-by-token prefill, every appended
    K/V row within 1e-3 of its row's max (the batched GEMM's A operand is two
    bf16 terms), the last logits within 1e-3; against XP_PREFILL_TOKENS the
    same; rows past the prompt untouched. The prompt (37 tokens) is not a
    multiple of 16 and starts at 490, so it crosses the 512-position window
    of the local layers."""
    X = xp
    print("case batched prefill", flush=True)
    pos0, n = 490, 37
    kvd = 256
    outs = {}
    for pm in (X.XP_PREFILL_AUTO, X.XP_PREFILL_TOKENS):
        cfg = cfg_small(X, n_layers=6, vocab=16384, exec_mode=mode, prefill_mode=pm)
        sess, model = make_pair(X, xo, cfg)
        for l in range(cfg.n_layers):
            for which in (0, 1):
                rows = X.synth_normal_f16(cfg.max_seq * kvd, 77, 2 * l + which)
                sess.kv_upload(l, which, 0, rows)
                (model.kcache if which == 0 else model.vcache)[l][:] = rows
        sess.set_position(pos0)
        prompt = np.random.default_rng(8).integers(0, cfg.vocab, n).astype(np.uint32)
        sess.prefill(prompt)
        assert sess.position == pos0 + n
        want = None
        for i, t in enumerate(prompt):
            want = model.forward(int(t), pos0 + i, i == n - 1)
        ok, msg = logits_close(sess.last_logits(), want)
        assert ok, f"prefill mode {pm}: {msg}"
        for l in range(cfg.n_layers):
            for which, ref in ((0, model.kcache[l]), (1, model.vcache[l])):
                got = sess.kv_download(l, which, pos0, n).view(np.float16).astype(np.float64)
                exp = ref[pos0 * kvd:(pos0 + n) * kvd].view(np.float16).astype(np.float64)
                err = np.abs(got - exp).reshape(n, kvd).max(axis=1)
                assert np.all(err <= 1e-3 * np.abs(exp).reshape(n, kvd).max(axis=1)), (pm, l, which)
                past = sess.kv_download(l, which, pos0 + n, 8)
                assert np.array_equal(past, ref[(pos0 + n) * kvd:(pos0 + n + 8) * kvd]), (pm, l)
        outs[pm] = ([sess.decode_step() for _ in range(4)], sess.last_logits())
        sess.close()
    a, b = outs[X.XP_PREFILL_AUTO], outs[X.XP_PREFILL_TOKENS]
    assert a[0] == b[0]
    ok, msg = logits_close(a[1], b[1])
    assert ok, msg


@pytest.mark.gpu
def test_gpu_token_trace_timeline(xp):
    """xp_session_trace: stage ends are ordered (each stage's last finisher
    after the previous one's), every stage has working workgroups, and a
    workgroup's input arrival precedes its stage end."""
    X = xp
    from xpose_amd.trace import arrivals, timeline
    cfg = cfg_small(X, n_layers=3, exec_mode=3)
    sess = X.DecodeSession(cfg)
    sess.synthesize(0x5EED0003)
    sess.prefill(np.array([7, 8, 9], np.uint32))
    sess.trace(True)
    sess.decode_steps(1)
    tr = sess.last_trace().astype(np.int64)
    n = cfg.n_layers
    assert tr.shape[0] == 12 * n + 3 and (tr[0] > 0).all()
    ends = [tr[1 + e].max() for e in range(6 * n + 2)]
    assert all(b >= a for a, b in zip(ends, ends[1:])), ends
    for l in range(n):
        for k in range(6):
            arr, end = tr[3 + 6 * n + 6 * l + k], tr[1 + 6 * l + k]
            w = arr > 0
            assert w.any(), (l, k)
            assert (arr[w] <= end[w]).all(), (l, k)
    rows, lm, am, total = timeline(tr, n)
    assert total > 0 and lm > 0 and (rows >= 0).all()
    a = arrivals(tr, n)
    assert (a[:, :, 1] >= 0).all() and (a[:, :, 2] >= 0).all()
    sess.trace(False)
    sess.close()


@pytest.mark.gpu
def test_gpu_token_kernel_timeout_recovers(xp):
    """The token kernel's bounded waits, forced from the host: with a spin
    limit of 0 every wait that its first read does not satisfy gives up,
    every workgroup still finishes, and the step returns XP_E_DEVICE with the
    position unchanged; after xp_session_set_position (which clears the
    status word) and the default limit back, the session recomputes the
    same context and its logits and next greedy ids are bit-equal to a fresh
    session's (the reference errors, never hangs: decode.cpp:1824-1826)."""
    X = xp
    print("case session token kernel forced timeout", flush=True)
    cfg = cfg_small(X, n_layers=3, vocab=16384, max_seq=64, exec_mode=X.XP_EXEC_TOKEN)
    a, b = X.DecodeSession(cfg), X.DecodeSession(cfg)
    for s in (a, b):
        s.synthesize(0x5EED0006)
        s.prefill([7, 8, 9])
    a.set_spin_limit(0)
    with pytest.raises(X.XposeError) as ei:
        a.decode_step()
    assert ei.value.code == -5 and "limit" in str(ei.value), ei.value
    assert a.position == 3
    with pytest.raises(X.XposeError):
        a.decode_step()                      # the status stays set until a position is set
    a.set_spin_limit(1 << 18)
    a.set_position(2)
    a.prefill([9])
    assert np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32))
    got = [a.decode_step() for _ in range(3)]
    want = [b.decode_step() for _ in range(3)]
    assert got == want
    assert np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32))
    with pytest.raises(X.XposeError):
        a.set_spin_limit(1 << 25)
    a.close()
    b.close()


@pytest.mark.gpu
def test_gpu_graph_attention_timeout_recovers(xp):
    """The graph path's exchange-mode decode attention (a global layer at
    max_seq 1024: 32 splits, all resident, combining through tagged records)
    with its spin limit forced to 0: the step returns XP_E_DEVICE instead of
    NaN logits reported as success, the records and tickets start over, and
    after xp_session_set_position the session's logits and next greedy ids
    are bit-equal to a fresh session's."""
    X = xp
    print("case session graph attention forced timeout", flush=True)
    cfg = cfg_small(X, n_layers=6, vocab=16384, max_seq=1024, exec_mode=X.XP_EXEC_GRAPH)
    a, b = X.DecodeSession(cfg), X.DecodeSession(cfg)
    for s in (a, b):
        s.synthesize(0x5EED0007)
        s.prefill([5, 6, 7, 8])
    a.set_spin_limit(0)
    with pytest.raises(X.XposeError) as ei:
        a.decode_step()
    assert ei.value.code == -5 and "limit" in str(ei.value), ei.value
    assert a.position == 4
    a.set_spin_limit(1 << 18)
    a.set_position(3)
    a.prefill([8])
    assert np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32))
    got = [a.decode_step() for _ in range(3)]
    want = [b.decode_step() for _ in range(3)]
    assert got == want
    assert np.array_equal(a.last_logits().view(np.uint32), b.last_logits().view(np.uint32))
    a.close()
    b.close()


@pytest.mark.gpu
def test_gpu_cfg3_full_length(xp, xo, mode):
    """Benchmark config 3 at its stated length: full Gemma-3-1B, the tied
    262144 x 1152 int4 table, a 32-token prompt of uniform random ids from
    position 0, then 128 greedy tokens in the reference's sample-first order
    (decode.cpp:1830-1861); every id equal to the oracle's generation."""
    X = xp
    print(f"case session cfg3 32 + 128 mode {mode}", flush=True)
    cfg = X.XpConfig.gemma3_1b(max_seq=512, exec_mode=mode)
    sess, model = make_pair(X, xo, cfg)
    prompt = np.random.default_rng(0x5EED0003).integers(0, cfg.vocab, 32).astype(np.uint32)
    want = model.generate_greedy(prompt, 128, 16)
    sess.prefill(prompt)
    got = sess.decode_steps(128)
    assert np.array_equal(got, want), int(np.argmax(got != want))
    assert sess.position == 32 + 128
    sess.close()


@pytest.mark.gpu
@pytest.mark.parametrize("exec_mode,placement", DEEP_MODES)
def test_gpu_cfg4_chunk_switch_and_buckets(xp, xo, exec_mode, placement):
    """Benchmark config 4's positions the shortened checks do not reach: the
    token kernel's switch of global attention from 64-key to 128-key head-pair
    chunks (global span 6656 -> 6657, positions 6655 and 6656) and one
    position per 512-position bucket of the 4097 -> 8192 run (4097, 4609, ...,
    7681, and 8191); KV of all 26 layers pre-filled with fp16 N(0,1) rows, each position
    run as a one-token prefill against the oracle at the same position (the
    positions run deepest first, so the row each run appends lies past every
    later context). Logits within 1e-3 and the greedy id equal."""
    X = xp
    print(f"case session cfg4 positions exec {exec_mode} placement {placement}", flush=True)
    cfg = X.XpConfig.gemma3_1b(exec_mode=exec_mode, placement=placement)
    sess, model = make_pair(X, xo, cfg)
    kvd = cfg.n_kv_heads * cfg.head_dim
    fill = cfg.max_seq - 1
    for l in range(cfg.n_layers):
        for which, cache in ((0, model.kcache), (1, model.vcache)):
            rows = X.synth_normal_f16(fill * kvd, 4096, 2 * l + which)
            sess.kv_upload(l, which, 0, rows)
            cache[l][:fill * kvd] = rows
    positions = sorted([6655, 6656] + [4097 + 512 * k for k in range(8)] + [8191], reverse=True)
    for p in positions:
        tok = 1000 + p
        sess.set_position(p)
        sess.prefill([tok])
        want = model.forward(tok, p, True, 16)
        got = sess.last_logits()
        ok, msg = logits_close(got, want)
        assert ok, f"position {p}: {msg}"
        assert xo.argmax_tree(got)[0] == xo.argmax_tree(want)[0], p
    sess.close()
