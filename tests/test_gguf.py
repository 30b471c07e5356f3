"""The GGUF load path: reader, ggml block dequantisers, the requantising packer
and the packed-weight cache (examples/llm/model/gguf.cpp, decode.cpp:60-229,
710-1328, 2580-2661), product against the oracle and against known answers.

Pins:
* the reference's own GGUF self-test (model/selftest.cpp:128-299): the same
  file built byte by byte, every value it checks (header, config keys,
  head_dim fallback, vocab from the token array, F32 values, the hand-computed
  Q4_0 and Q5_0 blocks, malformed files rejected);
* every other block format: blocks encoded from explicit parameters (scales,
  mins, quants) whose values are known in closed form (tests/gguf_util.py);
* the product's dequantisers (element-wise) equal the oracle's (the
  reference's loop order) bit for bit on random blocks;
* the packer: exact-grid blocks pack to their own nibbles and scale; the
  chosen bf16 scale is the better of its two neighbours (brute force); every
  reconstruction is within half a scale step; product == oracle bit for bit;
* the cache: pack -> verify byte for byte; a flipped byte, a touched model
  file and a truncated cache are all caught.
"""
import os
import struct

import numpy as np
import pytest

import gguf_util as G

HERE = os.path.dirname(os.path.abspath(__file__))


# ---------------------------------------------------------------- helpers ----

def selftest_file(path):
    """The file of model/selftest.cpp:128-215: 16 metadata keys (13 written),
    3 tensors (f32_t {4, 2}, q4_0_t {32}, q5_0_t {32})."""
    toks = ["<unk>", "<bos>", "<eos>"] + [f"<0x{i:02X}>" for i in range(256)]
    toks += ["h", "e", "l", "o", "▁", "▁h", "▁he", "ll", "llo", "▁hello"]
    scores = [0.0] * 3 + [0.0] * 256 + [-10.0] * 5 + [-3.0, -2.0, -4.0, -1.0, 0.0]
    f32 = struct.pack("<8f", *[i * 1.5 - 3.0 for i in range(8)])
    q4 = struct.pack("<H", 0x3800) + bytes(j | ((15 - j) << 4) for j in range(16))
    q5 = struct.pack("<HI", 0x3800, 0xFFFF0000) + bytes(j | ((15 - j) << 4) for j in range(16))
    meta = [("general.architecture", G.STR, "llama"), ("general.name", G.STR, "selftest"),
            ("llama.block_count", G.U32, 7), ("llama.attention.head_count", G.U32, 4),
            ("llama.attention.head_count_kv", G.U32, 2), ("llama.embedding_length", G.U32, 64),
            ("llama.feed_forward_length", G.U32, 172), ("llama.context_length", G.U32, 512),
            ("llama.rope.freq_base", G.F32, 1000000.0), ("tokenizer.ggml.model", G.STR, "llama"),
            ("tokenizer.ggml.add_space_prefix", G.BOOL, True),
            ("tokenizer.ggml.unknown_token_id", G.U32, 0), ("tokenizer.ggml.bos_token_id", G.U32, 1),
            ("tokenizer.ggml.eos_token_id", G.U32, 2),
            ("tokenizer.ggml.tokens", G.ARR, (G.STR, toks)),
            ("tokenizer.ggml.scores", G.ARR, (G.F32, scores))]
    tensors = [("f32_t", (4, 2), 0, f32), ("q4_0_t", (32,), 2, q4), ("q5_0_t", (32,), 6, q5)]
    return G.write_gguf(path, meta, tensors), len(toks)


def rand_blocks(r, typ, nblocks):
    """Random raw blocks of a ggml type with finite fp16 fields."""
    size = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 12: 144, 14: 210}[typ]
    raw = r.integers(0, 256, (nblocks, size), dtype=np.uint8)
    halves = {2: [0], 3: [0, 2], 6: [0], 7: [0, 2], 8: [0], 12: [0, 2], 14: [208]}[typ]
    for off in halves:
        v = G.f16(r.uniform(-2, 2, nblocks)).view(np.uint8).reshape(-1, 2)
        raw[:, off:off + 2] = v
    return raw


# ------------------------------------------------------------------ CPU ----

def test_reference_selftest_file(xh, tmp_path):
    """Every check of model/selftest.cpp:217-282 that concerns the reader."""
    X = xh
    path = str(tmp_path / "selftest.gguf")
    data, n_tok = selftest_file(path)
    g = X.Gguf(path)
    info = g.info()
    assert info.version == 3 and info.n_tensors == 3 and info.n_meta == 16
    # the data blob starts at the first 32-byte boundary after the descriptors
    assert info.data_offset == len(data) - (32 + 32 + 32 - 10)   # f32 32 B, q4_0 18 -> 32, q5_0 22
    m = g.model()
    assert m.arch == b"llama" and m.n_layers == 7 and m.n_heads == 4 and m.n_kv_heads == 2
    assert m.hidden == 64 and m.ffn == 172 and m.rope_freq_base == 1e6
    assert m.head_dim == 16                       # key_length absent: 64 / 4
    assert m.vocab == n_tok                       # the token array's length
    assert g.array_length("tokenizer.ggml.tokens") == n_tok
    assert g.string("general.name") == "selftest"
    assert g.number("llama.context_length") == 512
    typ, dims, nb = g.tensor("f32_t")
    assert typ == 0 and dims == (4, 2) and nb == 32
    assert np.array_equal(g.rows("f32_t").reshape(-1), np.arange(8, dtype=np.float32) * 1.5 - 3.0)
    typ, dims, nb = g.tensor("q4_0_t")
    assert typ == 2 and nb == 18
    v = g.rows("q4_0_t").reshape(-1)
    j = np.arange(16)
    assert np.array_equal(v[:16], (j - 8) * 0.5) and np.array_equal(v[16:], ((15 - j) - 8) * 0.5)
    assert v[0] == -4.0 and v[15] == 3.5 and v[16] == 3.5
    typ, dims, nb = g.tensor("q5_0_t")
    assert typ == 6 and nb == 22
    v = g.rows("q5_0_t").reshape(-1)
    assert np.array_equal(v[:16], (j - 16) * 0.5) and np.array_equal(v[16:], (15 - j) * 0.5)
    assert v[0] == -8.0 and v[16] == 7.5
    g.close()
    # malformed files are errors, not crashes (selftest.cpp:283-305)
    for bad, what in ((b"NOTGGUF!", "magic"), (data[:24], "header"),
                      (data[:len(data) // 2], "body")):
        p = str(tmp_path / f"bad_{what}.gguf")
        with open(p, "wb") as f:
            f.write(bad)
        with pytest.raises(X.XposeError):
            X.Gguf(p)


def test_oracle_reference_selftest_blocks(xo):
    """The oracle's Q4_0 / Q5_0 against the same hand-computed blocks."""
    q4 = np.frombuffer(struct.pack("<H", 0x3800) + bytes(j | ((15 - j) << 4) for j in range(16)),
                       np.uint8)
    q5 = np.frombuffer(struct.pack("<HI", 0x3800, 0xFFFF0000) +
                       bytes(j | ((15 - j) << 4) for j in range(16)), np.uint8)
    j = np.arange(16)
    v = xo.dequantize(2, q4, 32)
    assert np.array_equal(v, np.concatenate([(j - 8) * 0.5, ((15 - j) - 8) * 0.5]))
    v = xo.dequantize(6, q5, 32)
    assert np.array_equal(v, np.concatenate([(j - 16) * 0.5, (15 - j) * 0.5]))


def test_oracle_dequantize_known_blocks(xo):
    """Blocks encoded from explicit parameters decode to their closed form."""
    r = np.random.default_rng(11)
    for _ in range(20):
        d, m = r.uniform(-1, 1), r.uniform(-1, 1)
        q4, q5, q6 = r.integers(0, 16, 32), r.integers(0, 32, 32), r.integers(0, 64, 256)
        q8 = r.integers(-128, 128, 32)
        cases = [
            (2, G.q4_0_block(d, q4), G.q4_0_values(d, q4)),
            (3, G.q4_1_block(d, m, q4), G.q4_1_values(d, m, q4)),
            (6, G.q5_0_block(d, q5), G.q5_0_values(d, q5)),
            (7, G.q5_1_block(d, m, q5), G.q5_1_values(d, m, q5)),
            (8, G.q8_0_block(d, q8), G.q8_0_values(d, q8)),
        ]
        sc, mn, qk = r.integers(0, 64, 8), r.integers(0, 64, 8), r.integers(0, 16, 256)
        cases.append((12, G.q4_k_block(d, m, sc, mn, qk), G.q4_k_values(d, m, sc, mn, qk)))
        s6 = r.integers(-128, 128, 16)
        cases.append((14, G.q6_k_block(d, s6, q6), G.q6_k_values(d, s6, q6)))
        h = r.standard_normal(64).astype(np.float32)
        cases.append((1, G.f16(h).tobytes(), G.f16(h).astype(np.float32)))
        bf = (h.view(np.uint32) >> 16).astype(np.uint16)
        cases.append((30, bf.tobytes(), (bf.astype(np.uint32) << 16).view(np.float32)))
        cases.append((0, h.tobytes(), h))
        for typ, raw, want in cases:
            got = xo.dequantize(typ, np.frombuffer(raw, np.uint8), want.size)
            assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32)), typ


def test_dequantize_product_equals_oracle(xh, xo):
    X = xh
    r = np.random.default_rng(3)
    for typ, per in ((2, 32), (3, 32), (6, 32), (7, 32), (8, 32), (12, 256), (14, 256)):
        raw = rand_blocks(r, typ, 64)
        n = 64 * per
        got = X.dequantize(typ, raw, n)
        want = xo.dequantize(typ, raw, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), typ
    h = r.integers(0, 65536, 4096).astype(np.uint16)      # every fp16 class, NaN included
    for typ in (1, 30):
        got = X.dequantize(typ, h, h.size)
        want = xo.dequantize(typ, h, h.size)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), typ
    with pytest.raises(X.XposeError):
        X.dequantize(10, np.zeros(84, np.uint8), 256)         # Q2_K: not implemented
    with pytest.raises(X.XposeError):
        X.dequantize(8, np.zeros(34, np.uint8), 31)           # partial block


def lround(x):
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def block_error(v, s):
    if s <= 0:
        return np.inf
    inv = np.float32(1.0) / np.float32(s)
    q = np.clip(lround((v * inv).astype(np.float32)) + 8, 0, 15)
    return float(np.sum(((q - 8) * np.float64(s) - v.astype(np.float64)) ** 2))


def test_oracle_packer_pins(xo):
    r = np.random.default_rng(5)
    rows, cols = 256, 128
    # exact grid: v = k s with s a bf16 value and max |k| = 7 -> scale s, nibbles k + 8
    s = np.float32(0.15625)                                       # 0x3E20 in bf16
    k = r.integers(-7, 8, (cols, rows))
    k[:, ::32] = 7                                                 # amax = 7 s in every block
    w = (k * s).astype(np.float32)
    wq, sc = xo.pack_int4(w, True)
    nib = np.empty(rows * cols, np.int8)
    xo.lib().xo_unpack_km4(nib, wq, rows, cols)
    assert np.array_equal(nib.reshape(rows, cols), k.T)
    assert np.all(sc == 0x3E20)
    # random blocks: the scale is the better bf16 neighbour of amax / 7 and every
    # element reconstructs within half a step
    w = (r.standard_normal((cols, rows)) * r.uniform(0.01, 3, (cols, 1))).astype(np.float32)
    w[3, 64:96] = 0.0                                             # an all-zero block
    w[5, 100] = 40.0                                              # an outlier
    wq, sc = xo.pack_int4(w, True)
    xo.lib().xo_unpack_km4(nib, wq, rows, cols)
    nib = nib.reshape(rows, cols).astype(np.float64)
    for c in range(cols):
        for b in range(rows // 32):
            blk = w[c, 32 * b:32 * b + 32]
            got = float(xo.lib().xo_bf16_to_fp32(int(sc[((b // 4) * cols + c) * 4 + b % 4])))
            s0 = np.float32(np.abs(blk).max()) / np.float32(7.0)
            if s0 == 0:
                assert got == 0.0 and np.all(nib[32 * b:32 * b + 32, c] == 0)
                continue
            lo = (np.array([s0], np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)[0]
            hi = (np.array([lo], np.float32).view(np.uint32) + 0x10000).view(np.float32)[0]
            assert got in (lo, hi)
            assert block_error(blk, got) <= block_error(blk, hi if got == lo else lo)
            rec = nib[32 * b:32 * b + 32, c] * got
            assert np.all(np.abs(rec - blk) <= got * 0.5 * (1 + 1e-6))
    # fp32 scales: s = amax / 7 exactly
    wq, scf = xo.pack_int4(w, False)
    assert np.array_equal(scf.reshape(rows // 32, cols)[1, 7],
                          np.float32(np.abs(w[7, 32:64]).max()) / np.float32(7.0))


def test_pack_product_equals_oracle(xh, xo):
    X = xh
    r = np.random.default_rng(9)
    for rows, cols in ((256, 128), (1152, 192)):
        w = (r.standard_normal((cols, rows)) * r.uniform(1e-3, 2, (cols, 1))).astype(np.float32)
        w[0, :32] = 0.0
        w[1, 5] = -50.0
        w[2, 40:72] = 1e-30                                       # tiny blocks
        for fmt, bf in ((X.XP_SCALE_BF16_QUAD, True), (X.XP_SCALE_F32, False)):
            wq, sc = X.pack_int4(w, fmt)
            owq, osc = xo.pack_int4(w, bf)
            assert np.array_equal(wq, owq), (rows, cols, fmt)
            assert np.array_equal(sc.view(np.uint8), osc.view(np.uint8)), (rows, cols, fmt)
    with pytest.raises(X.XposeError):
        X.pack_int4(np.zeros((64, 96), np.float32))               # rows not a multiple of 128
    with pytest.raises(X.XposeError):
        X.pack_int4(np.zeros((32, 128), np.float32))              # cols not a multiple of 64


SMALL = dict(n_layers=2, hidden=256, ffn=512, n_heads=1, vocab=1024)


def small_cfg(X, **kw):
    c = X.XpConfig.gemma3_1b(n_layers=SMALL["n_layers"], hidden=SMALL["hidden"], ffn=SMALL["ffn"],
                             n_heads=SMALL["n_heads"], vocab=SMALL["vocab"], max_seq=512,
                             scale_fmt=X.XP_SCALE_BF16_QUAD, **kw)
    return c


def test_cache_roundtrip_and_damage(xh, xo, tmp_path):
    X = xh
    model = str(tmp_path / "m.gguf")
    vals = G.gemma_model(model, **SMALL)
    g = X.Gguf(model)
    cfg = g.config(small_cfg(X))
    assert (cfg.n_layers, cfg.hidden, cfg.ffn, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
            cfg.vocab, cfg.sliding_window) == (2, 256, 512, 1, 1, 256, 1024, 512)
    assert cfg.rope_theta_global == 1e6
    cache = str(tmp_path / "m.xpack")
    st = g.pack_model(cfg, cache, threads=4)
    assert st.cache_written == 1 and st.n_tensors == 2 * 7 + 1
    assert g.verify_cache(cfg, cache) == 0
    # the cached bytes of a matrix are the packer's output on the file's values,
    # and the oracle packs the same bytes
    rows = g.rows("blk.1.ffn_down.weight")
    assert np.array_equal(rows, vals["blk.1.ffn_down.weight"])
    wq, sc = X.pack_int4(rows)
    owq, osc = xo.pack_int4(rows, True)
    assert np.array_equal(wq, owq) and np.array_equal(sc, osc)
    data = open(cache, "rb").read()
    assert data.find(wq.tobytes() + sc.tobytes()) > 0
    # a flipped payload byte is a mismatch (the header still validates)
    bad = bytearray(data)
    bad[4096] ^= 0x10
    with open(cache, "wb") as f:
        f.write(bad)
    assert g.verify_cache(cfg, cache) >= 1
    # a truncated cache, and a touched model file, are not valid caches
    with open(cache, "wb") as f:
        f.write(data[:len(data) // 2])
    with pytest.raises(X.XposeError):
        g.verify_cache(cfg, cache)
    with open(cache, "wb") as f:
        f.write(data)
    assert g.verify_cache(cfg, cache) == 0
    st_ = os.stat(model)
    os.utime(model, ns=(st_.st_atime_ns, st_.st_mtime_ns + 1_000_000_000))
    with pytest.raises(X.XposeError) as e:
        g.verify_cache(cfg, cache)
    assert "changed" in str(e.value)
    g.close()


def test_load_errors(xh, tmp_path):
    X = xh
    model = str(tmp_path / "m.gguf")
    G.gemma_model(model, **SMALL)
    g = X.Gguf(model)
    cfg = g.config(small_cfg(X))
    bad = g.config(small_cfg(X))
    bad.ffn = 1024
    with pytest.raises(X.XposeError) as e:
        g.pack_model(bad, str(tmp_path / "x.xpack"))
    assert "ffn" in str(e.value)
    f16 = g.config(small_cfg(X))
    f16.scale_fmt = X.XP_SCALE_F16_QUAD
    with pytest.raises(X.XposeError):
        g.pack_model(f16, str(tmp_path / "x.xpack"))
    with pytest.raises(X.XposeError):
        g.tensor("no.such.tensor")
    g.close()
    # a matrix in a type the loader does not dequantise
    G.write_gguf(str(tmp_path / "q2k.gguf"),
                 [("general.architecture", G.STR, "gemma3"), ("gemma3.block_count", G.U32, 1)],
                 [("blk.0.attn_q.weight", (256, 256), 10, bytes(84 * 256))])
    g2 = X.Gguf(str(tmp_path / "q2k.gguf"))
    c2 = small_cfg(X)
    c2.n_layers = 1
    with pytest.raises(X.XposeError) as e:
        g2.pack_model(c2, str(tmp_path / "y.xpack"))
    assert "Q2_K" in str(e.value)
    g2.close()


# ------------------------------------------------------------------ GPU ----

def oracle_from_gguf(X, xo, g, cfg, vals):
    """The oracle model of a GGUF file: the oracle's packer on the file's
    values, norms minus 1, the fp32 embedding rows."""
    names = {X.T_Q: "attn_q", X.T_K: "attn_k", X.T_V: "attn_v", X.T_O: "attn_output",
             X.T_GATE: "ffn_gate", X.T_UP: "ffn_up", X.T_DOWN: "ffn_down"}
    norms = {X.T_ATTN_NORM: "attn_norm", X.T_POST_ATTN_NORM: "post_attention_norm",
             X.T_FFN_NORM: "ffn_norm", X.T_POST_FFN_NORM: "post_ffw_norm",
             X.T_Q_NORM: "attn_q_norm", X.T_K_NORM: "attn_k_norm"}
    packed = {}

    def get(layer, t):
        base = t & ~X.T_SCALES
        if base == X.T_FINAL_NORM:
            return vals["output_norm.weight"] - 1.0
        if base in norms:
            return vals[f"blk.{layer}.{norms[base]}.weight"] - 1.0
        name = "token_embd.weight" if base == X.T_LM_HEAD else f"blk.{layer}.{names[base]}.weight"
        if name not in packed:
            packed[name] = xo.pack_int4(vals[name], True)
        return packed[name][1 if t & X.T_SCALES else 0]

    return xo.OracleModel(cfg, get, embed=vals["token_embd.weight"])


def check_load(X, xo, tmp_path, shape, steps, seed):
    from test_session import logits_close
    model = str(tmp_path / "m.gguf")
    vals = G.gemma_model(model, seed=seed, **shape)
    g = X.Gguf(model)
    cfg = g.config(X.XpConfig.gemma3_1b(max_seq=512, scale_fmt=X.XP_SCALE_BF16_QUAD))
    cache = str(tmp_path / "m.xpack")
    sess = X.DecodeSession(cfg)
    st = sess.load_gguf(g, cache)
    assert st.from_cache == 0 and st.cache_written == 1
    om = oracle_from_gguf(X, xo, g, cfg, vals)
    prompt = [5, 77, cfg.vocab - 1]
    want = None
    for i, t in enumerate(prompt):
        want = om.forward(t, i, i == len(prompt) - 1)
    sess.prefill(prompt)
    ok, msg = logits_close(sess.last_logits(), want)
    assert ok, msg
    first = sess.last_logits()
    for s in range(steps):
        nxt = int(np.argmax(want))   # greedy; ties are measure-zero on these logits
        tok = sess.decode_step()
        assert tok == nxt, s
        want = om.forward(tok, len(prompt) + s, True)
        ok, msg = logits_close(sess.last_logits(), want)
        assert ok, f"step {s}: {msg}"
    sess.close()
    # the same model from the cache: identical logits
    sess = X.DecodeSession(cfg)
    st = sess.load_gguf(g, cache)
    assert st.from_cache == 1
    sess.prefill(prompt)
    assert np.array_equal(sess.last_logits().view(np.uint32), first.view(np.uint32))
    # the batched path embeds from the same table
    om2 = oracle_from_gguf(X, xo, g, cfg, vals)
    b = X.DecodeBatch(sess, 2, 64)
    b.set_positions([0, 0])
    b.forward([prompt[0], prompt[2]])
    for i, t in enumerate((prompt[0], prompt[2])):
        want = om2.forward(t, 0, True)
        ok, msg = logits_close(b.last_logits(i), want)
        assert ok, f"batch seq {i}: {msg}"
    b.close()
    sess.close()
    g.close()


@pytest.mark.gpu
def test_gpu_load_gguf_small_model(xp, xo, tmp_path):
    """A small Gemma-3-architecture GGUF (graph path): requantised on load,
    logits within 1e-3 of the oracle on the oracle's packing of the same file
    values, with the file's fp32 embedding rows; greedy ids equal."""
    print("case gguf small", flush=True)
    check_load(xp, xo, tmp_path, SMALL, steps=3, seed=21)


@pytest.mark.gpu
def test_gpu_load_gguf_gemma_shapes(xp, xo, tmp_path):
    """Gemma-3-1B layer shapes, 2 layers, vocab 16384 (the persistent token
    kernel with the fp32 embedding table)."""
    print("case gguf gemma shapes", flush=True)
    check_load(xp, xo, tmp_path, dict(n_layers=2, hidden=1152, ffn=6912, n_heads=4, vocab=16384),
               steps=2, seed=22)


def test_config_window_merge(xh, tmp_path):
    """The file's sliding_window replaces the default 512; a window the caller
    set to anything else survives (decode.cpp:1427-1434)."""
    X = xh
    path = str(tmp_path / "w.gguf")
    G.write_gguf(path, [("general.architecture", G.STR, "gemma3"),
                        ("gemma3.block_count", G.U32, 3),
                        ("gemma3.attention.sliding_window", G.U32, 1024)], [])
    g = X.Gguf(path)
    assert g.config(X.XpConfig.gemma3_1b()).sliding_window == 1024
    c = g.config(X.XpConfig.gemma3_1b(sliding_window=128, global_every=4))
    assert (c.sliding_window, c.global_every, c.n_layers) == (128, 4, 3)
    g.close()
