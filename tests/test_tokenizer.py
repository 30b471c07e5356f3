"""The GGUF tokenizer (model/tokenizer.cpp:70-374): the reference's own
self-test cases (model/selftest.cpp:259-282) on the product and the oracle,
then product == oracle (oracle/tokenizer.py, the reference's loops restated)
on a synthetic Gemma-like vocabulary over random text, and decode(encode(s))
== s wherever byte fallback makes the tokenizer total."""
import numpy as np
import pytest

import gguf_util as G
from oracle.tokenizer import Tokenizer as OTok
from test_gguf import selftest_file

CONTROL, UNKNOWN, BYTE, USER = 3, 2, 6, 4


def test_reference_selftest_vocabulary(xh, tmp_path):
    X = xh
    path = str(tmp_path / "s.gguf")
    _, n = selftest_file(path)
    g = X.Gguf(path)
    t = X.Tokenizer(g)
    assert t.ids.vocab == n and t.ids.add_space_prefix == 1 and t.ids.unk == 0 and t.ids.bos == 1
    assert t.kind(3) == 1                         # no token_type array: every token NORMAL
    sp_hello, sp_h = n - 1, n - 5
    assert t.encode("hello") == [sp_hello]        # the scored merge path ends in _hello
    assert t.decode([sp_hello]) == b"hello"       # the dummy prefix is stripped
    assert t.encode("hq") == [sp_h, 0]            # 'q': no spelling, no byte tokens -> <unk>
    assert t.encode("hello", add_bos=True) == [1, sp_hello]
    # the oracle on the same vocabulary
    toks = ["<unk>", "<bos>", "<eos>"] + [f"<0x{i:02X}>" for i in range(256)]
    toks += ["h", "e", "l", "o", "▁", "▁h", "▁he", "ll", "llo", "▁hello"]
    scores = [0.0] * 259 + [-10.0] * 5 + [-3.0, -2.0, -4.0, -1.0, 0.0]
    o = OTok(toks, scores, None, bos=1, eos=2, unk=0)
    assert o.encode(b"hello") == [sp_hello] and o.encode(b"hq") == [sp_h, 0]
    assert o.decode([sp_hello]) == b"hello"
    t.close()
    g.close()


def synthetic_vocab(seed=3):
    """Control tokens, an unknown token, 256 byte tokens, whitespace runs
    (user-defined), single characters (some multi-byte) and random 2-4
    character pieces with random scores; one duplicate spelling."""
    r = np.random.default_rng(seed)
    toks = ["<pad>", "<eos>", "<bos>", "<unk>", "<start_of_turn>", "<end_of_turn>", "<s>"]
    types = [CONTROL, CONTROL, CONTROL, UNKNOWN, CONTROL, CONTROL, CONTROL]
    toks += [f"<0x{i:02X}>" for i in range(256)]
    types += [BYTE] * 256
    toks += ["\n", "\n\n", "▁▁", "▁▁▁▁"]
    types += [USER] * 4
    alphabet = list("abcdefghijklmnopqrstuvwxyzABC,.!?") + ["▁", "é", "中", "文", "🙂"]
    toks += alphabet
    types += [1] * len(alphabet)
    seen = set(toks)
    while len(toks) < 1200:
        k = int(r.integers(2, 5))
        p = "".join(r.choice(alphabet, k))
        if p not in seen:
            seen.add(p)
            toks.append(p)
            types.append(1)
    toks.append("▁a")                  # a duplicate spelling: the lower id is the one used
    types.append(1)
    if "▁a" not in seen:
        toks.insert(300, "▁a")
        types.insert(300, 1)
    scores = list(-np.abs(r.standard_normal(len(toks))).astype(np.float32))
    scores[-1] = 5.0
    return toks, scores, types


def write_vocab(path, toks, scores, types, prefix=True):
    meta = [("general.architecture", G.STR, "gemma3"),
            ("tokenizer.ggml.model", G.STR, "llama"),
            ("tokenizer.ggml.tokens", G.ARR, (G.STR, toks)),
            ("tokenizer.ggml.scores", G.ARR, (G.F32, scores)),
            ("tokenizer.ggml.token_type", G.ARR, (G.I32, types)),
            ("tokenizer.ggml.bos_token_id", G.U32, 2), ("tokenizer.ggml.eos_token_id", G.U32, 1),
            ("tokenizer.ggml.unknown_token_id", G.U32, 3),
            ("tokenizer.ggml.padding_token_id", G.U32, 0),
            ("tokenizer.ggml.add_space_prefix", G.BOOL, prefix)]
    G.write_gguf(path, meta, [])


def random_text(r, n):
    parts = ["a", "b", "c", "ab", "é", "中文", "🙂", " ", "  ", "\n", "\n\n", "xyz", ",", "!",
             "<start_of_turn>", "<end_of_turn>", "<s>", "<unk>", "q", "Z", "ÿ"]
    s = "".join(r.choice(parts, n))
    b = s.encode()
    if r.random() < 0.2:                          # an invalid UTF-8 byte somewhere
        i = int(r.integers(0, len(b) + 1))
        b = b[:i] + bytes([int(r.integers(0x80, 0x100))]) + b[i:]
    return b


@pytest.mark.parametrize("prefix,tied", [(True, False), (False, False), (True, True)])
def test_tokenizer_matches_oracle(xh, tmp_path, prefix, tied):
    """tied: every score equal, so the leftmost-pair rule decides every merge."""
    X = xh
    toks, scores, types = synthetic_vocab()
    if tied:
        scores = [0.0] * len(scores)
    path = str(tmp_path / "v.gguf")
    write_vocab(path, toks, scores, types, prefix)
    g = X.Gguf(path)
    t = X.Tokenizer(g)
    o = OTok(toks, scores, types, bos=2, eos=1, unk=3, pad=0, add_space_prefix=prefix)
    assert t.find("▁a") == o.token_to_id["▁a".encode()]
    r = np.random.default_rng(7)
    for i in range(300):
        text = random_text(r, int(r.integers(0, 40)))
        bos, eos = bool(i % 3 == 0), bool(i % 5 == 0)
        ids = t.encode(text, bos, eos)
        assert ids == o.encode(text, bos, eos), text
        assert t.decode(ids) == o.decode(ids), text
        assert t.decode(ids, False) == o.decode(ids, False), text
    for tid in range(len(toks)):
        assert t.piece(tid) == o.decode_one(tid)
    t.close()
    g.close()


def test_tokenizer_round_trip(xh, tmp_path):
    """Text with no special spellings decodes back to itself (byte fallback
    covers every byte; the one added prefix space is removed)."""
    X = xh
    toks, scores, types = synthetic_vocab(5)
    path = str(tmp_path / "v.gguf")
    write_vocab(path, toks, scores, types)
    g = X.Gguf(path)
    t = X.Tokenizer(g)
    r = np.random.default_rng(9)
    parts = ["a", "b", "é", "中", "🙂", " ", "\n", "xyz", ",", "ñ", "\t", "Ω"]
    for _ in range(200):
        s = "".join(r.choice(parts, int(r.integers(1, 30)))).encode()
        assert t.decode(t.encode(s)) == s, s
    t.close()
    g.close()


def test_tokenizer_errors(xh, tmp_path):
    X = xh
    path = str(tmp_path / "none.gguf")
    G.write_gguf(path, [("general.architecture", G.STR, "gemma3")], [])
    g = X.Gguf(path)
    with pytest.raises(X.XposeError):
        X.Tokenizer(g)
    g.close()
    path = str(tmp_path / "bad.gguf")
    G.write_gguf(path, [("tokenizer.ggml.tokens", G.ARR, (G.STR, ["a", "b"])),
                        ("tokenizer.ggml.scores", G.ARR, (G.F32, [0.0]))], [])
    g = X.Gguf(path)
    with pytest.raises(X.XposeError):
        X.Tokenizer(g)
    g.close()
