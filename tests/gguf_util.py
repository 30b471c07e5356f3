"""Test helpers for the GGUF load path: a GGUF v3 writer and encoders for the
ggml block formats, written from the published layouts (the inverse of what
examples/llm/model/gguf.cpp:448-645 decodes). The encoders take explicit
block parameters (scales, mins, quants), so a test knows every value the
decoder must produce."""
from __future__ import annotations

import struct

import numpy as np

# metadata value kinds
U32, F32, BOOL, STR, ARR = 4, 6, 7, 8, 9
I32 = 5


def _s(b: bytearray, text: str | bytes) -> None:
    raw = text.encode() if isinstance(text, str) else text
    b += struct.pack("<Q", len(raw)) + raw


def write_gguf(path: str, meta: list, tensors: list, alignment: int = 32, version: int = 3) -> bytes:
    """meta: [(key, kind, value)] with kind U32 / I32 / F32 / BOOL / STR, or
    (key, ARR, (elem_kind, values)); tensors: [(name, dims, ggml_type, raw)]
    with dims fastest-first. Returns the file bytes (also written to path)."""
    h = bytearray(b"GGUF")
    h += struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, kind, val in meta:
        _s(h, key)
        h += struct.pack("<I", kind)
        if kind == U32:
            h += struct.pack("<I", val)
        elif kind == I32:
            h += struct.pack("<i", val)
        elif kind == F32:
            h += struct.pack("<f", val)
        elif kind == BOOL:
            h += struct.pack("<B", 1 if val else 0)
        elif kind == STR:
            _s(h, val)
        elif kind == ARR:
            ek, vals = val
            h += struct.pack("<IQ", ek, len(vals))
            for v in vals:
                if ek == STR:
                    _s(h, v)
                elif ek == F32:
                    h += struct.pack("<f", v)
                elif ek == I32:
                    h += struct.pack("<i", v)
                else:
                    h += struct.pack("<I", v)
        else:
            raise ValueError(kind)
    blob = bytearray()
    offsets = []
    for _, _, _, raw in tensors:
        while len(blob) % alignment:
            blob += b"\0"
        offsets.append(len(blob))
        blob += bytes(raw)
    for (name, dims, typ, _), off in zip(tensors, offsets):
        _s(h, name)
        h += struct.pack("<I", len(dims))
        for d in dims:
            h += struct.pack("<Q", d)
        h += struct.pack("<IQ", typ, off)
    while len(h) % alignment:
        h += b"\0"
    data = bytes(h + blob)
    if path:
        with open(path, "wb") as f:
            f.write(data)
    return data


def f16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16)


# ---- block encoders (explicit parameters -> bytes) ----------------------------

def q4_0_block(d: float, q: np.ndarray) -> bytes:
    """q: 32 unsigned 4-bit quants; element e < 16 is the low nibble of byte e,
    element e >= 16 the high nibble of byte e - 16."""
    q = np.asarray(q, np.uint8)
    return f16(d).tobytes() + (q[:16] | (q[16:] << 4)).astype(np.uint8).tobytes()


def q4_1_block(d: float, m: float, q: np.ndarray) -> bytes:
    q = np.asarray(q, np.uint8)
    return f16(d).tobytes() + f16(m).tobytes() + (q[:16] | (q[16:] << 4)).astype(np.uint8).tobytes()


def _qh(q: np.ndarray) -> bytes:
    bits = (np.asarray(q, np.uint32) >> 4) & 1
    return struct.pack("<I", int(np.sum(bits << np.arange(32, dtype=np.uint32))))


def q5_0_block(d: float, q: np.ndarray) -> bytes:
    """q: 32 unsigned 5-bit quants; bit e of qh is the fifth bit of element e."""
    q = np.asarray(q, np.uint8)
    lo = q & 15
    return f16(d).tobytes() + _qh(q) + (lo[:16] | (lo[16:] << 4)).astype(np.uint8).tobytes()


def q5_1_block(d: float, m: float, q: np.ndarray) -> bytes:
    q = np.asarray(q, np.uint8)
    lo = q & 15
    return (f16(d).tobytes() + f16(m).tobytes() + _qh(q) +
            (lo[:16] | (lo[16:] << 4)).astype(np.uint8).tobytes())


def q8_0_block(d: float, q: np.ndarray) -> bytes:
    return f16(d).tobytes() + np.asarray(q, np.int8).tobytes()


def q4_k_block(d: float, dmin: float, sc: np.ndarray, mn: np.ndarray, q: np.ndarray) -> bytes:
    """sc, mn: 8 six-bit sub-block scales / mins; q: 256 four-bit quants.
    Scales: bytes 0-3 hold sc[0..3] (low 6 bits), bytes 4-7 mn[0..3]; for
    j >= 4, byte j + 4 holds sc[j] & 15 | (mn[j] & 15) << 4 and the top two bits
    of sc[j] / mn[j] go to bits 6-7 of byte j - 4 / byte j. Quants: the
    64-element run r uses bytes 32 r .. 32 r + 31, low nibbles for its first 32
    elements and high nibbles for the next 32."""
    sc = np.asarray(sc, np.uint8)
    mn = np.asarray(mn, np.uint8)
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = sc[j] & 63
        s[j + 4] = mn[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (mn[j] >> 4) << 6
    q = np.asarray(q, np.uint8).reshape(4, 2, 32)          # run, half, lane
    qs = (q[:, 0, :] | (q[:, 1, :] << 4)).reshape(128).astype(np.uint8)
    return f16(d).tobytes() + f16(dmin).tobytes() + s.tobytes() + qs.tobytes()


def q6_k_block(d: float, sc: np.ndarray, q: np.ndarray) -> bytes:
    """sc: 16 int8 scales; q: 256 six-bit quants (stored unsigned, value q - 32).
    Element e = 128 h + 32 t + l: low nibble in byte 64 h + l + 32 (t & 1)
    (low half for t < 2, high half for t >= 2), top two bits at bits 2 t of
    byte 32 h + l, scale index 8 h + 2 t + l // 16."""
    q = np.asarray(q, np.uint8)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e in range(256):
        h, t, l = e // 128, (e % 128) // 32, e % 32
        ql[64 * h + l + 32 * (t & 1)] |= (q[e] & 15) << (4 * (t >> 1))
        qh[32 * h + l] |= (q[e] >> 4) << (2 * t)
    return ql.tobytes() + qh.tobytes() + np.asarray(sc, np.int8).tobytes() + f16(d).tobytes()


# ---- closed-form values of the blocks above (float32, two roundings) -----------

def q4_0_values(d, q):
    d = np.float32(f16(d))
    return (np.asarray(q, np.int32) - 8).astype(np.float32) * d


def q4_1_values(d, m, q):
    d, m = np.float32(f16(d)), np.float32(f16(m))
    return np.asarray(q, np.float32) * d + m


def q5_0_values(d, q):
    return (np.asarray(q, np.int32) - 16).astype(np.float32) * np.float32(f16(d))


def q5_1_values(d, m, q):
    d, m = np.float32(f16(d)), np.float32(f16(m))
    return np.asarray(q, np.float32) * d + m


def q8_0_values(d, q):
    return np.asarray(q, np.float32) * np.float32(f16(d))


def q4_k_values(d, dmin, sc, mn, q):
    d, dmin = np.float32(f16(d)), np.float32(f16(dmin))
    j = np.arange(256) // 32
    return ((d * np.asarray(sc, np.float32)[j]) * np.asarray(q, np.float32)
            - dmin * np.asarray(mn, np.float32)[j]).astype(np.float32)


def q6_k_values(d, sc, q):
    d = np.float32(f16(d))
    e = np.arange(256)
    idx = 8 * (e // 128) + 2 * ((e % 128) // 32) + (e % 32) // 16
    return ((d * np.asarray(sc, np.float32)[idx]) *
            (np.asarray(q, np.int32) - 32).astype(np.float32)).astype(np.float32)


# ---- whole-tensor encoders for test models ------------------------------------

def encode_q8_0(x: np.ndarray) -> bytes:
    """Rows of x (fastest axis a multiple of 32) as Q8_0: d = amax / 127."""
    b = np.asarray(x, np.float32).reshape(-1, 32)
    d = (np.abs(b).max(axis=1) / 127.0).astype(np.float16)
    inv = np.where(d.astype(np.float32) > 0, 1.0 / np.maximum(d.astype(np.float32), 1e-30), 0.0)
    q = np.clip(np.rint(b * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((b.shape[0], 34), np.uint8)
    out[:, :2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.tobytes()


def chat_vocab(vocab: int):
    """A Gemma-like vocabulary of `vocab` entries: <pad> <eos> <bos> <unk>
    <start_of_turn> <end_of_turn>, 256 byte tokens, letters, then fillers.
    Returns (tokens, types); bos = 2, eos = 1, unk = 3."""
    toks = ["<pad>", "<eos>", "<bos>", "<unk>", "<start_of_turn>", "<end_of_turn>"]
    types = [3, 3, 3, 2, 3, 3]
    toks += [f"<0x{i:02X}>" for i in range(256)]
    types += [6] * 256
    for c in "abcdefghijklmnopqrstuvwxyz":
        toks += [c, "▁" + c]
        types += [1, 1]
    toks += ["▁", "\n"]
    types += [1, 1]
    while len(toks) < vocab:
        toks.append(f"w{len(toks)}")
        types.append(1)
    return toks[:vocab], types[:vocab]


def gemma_model(path: str, n_layers: int, hidden: int, ffn: int, n_heads: int, vocab: int,
                seed: int = 7, head_dim: int = 256, mat_type: str = "q8_0",
                chat: bool = False) -> dict:
    """A small Gemma-3-architecture GGUF: Q8_0 (or F32) matrices ~ N(0, 0.05),
    norms 1 + N(0, 0.1) (the file stores 1 + w), token_embd tied. Returns the
    fp32 values the file holds as {name: array [rows][row_len]}."""
    r = np.random.default_rng(seed)
    qd, kvd = n_heads * head_dim, head_dim
    meta = [("general.architecture", STR, "gemma3"), ("general.name", STR, "test"),
            ("gemma3.block_count", U32, n_layers), ("gemma3.embedding_length", U32, hidden),
            ("gemma3.feed_forward_length", U32, ffn), ("gemma3.attention.head_count", U32, n_heads),
            ("gemma3.attention.head_count_kv", U32, 1), ("gemma3.attention.key_length", U32, head_dim),
            ("gemma3.attention.value_length", U32, head_dim), ("gemma3.context_length", U32, 8192),
            ("gemma3.attention.sliding_window", U32, 512), ("gemma3.rope.freq_base", F32, 1e6),
            ("gemma3.attention.layer_norm_rms_epsilon", F32, 1e-6),
            ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(vocab)]))]
    if chat:
        toks, types = chat_vocab(vocab)
        meta[-1] = ("tokenizer.ggml.tokens", ARR, (STR, toks))
        meta += [("tokenizer.ggml.token_type", ARR, (I32, types)),
                 ("tokenizer.ggml.scores", ARR, (F32, [0.0] * vocab)),
                 ("tokenizer.ggml.bos_token_id", U32, 2), ("tokenizer.ggml.eos_token_id", U32, 1),
                 ("tokenizer.ggml.unknown_token_id", U32, 3)]
    tensors, values = [], {}

    def mat(name, rows_in, cols_out):
        w = (r.standard_normal((cols_out, rows_in)) * 0.05).astype(np.float32)
        if mat_type == "q8_0":
            raw = encode_q8_0(w)
            typ = 8
            blocks = np.frombuffer(raw, np.uint8).reshape(-1, 34)
            d = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
            q = blocks[:, 2:].copy().view(np.int8).astype(np.float32)
            vals = (q * d[:, None]).reshape(cols_out, rows_in)
        else:
            raw, typ, vals = w.tobytes(), 0, w
        tensors.append((name, (rows_in, cols_out), typ, raw))
        values[name] = vals

    def norm(name, n):
        v = (1.0 + r.standard_normal(n) * 0.1).astype(np.float32)
        tensors.append((name, (n,), 0, v.tobytes()))
        values[name] = v

    for l in range(n_layers):
        p = f"blk.{l}."
        mat(p + "attn_q.weight", hidden, qd)
        mat(p + "attn_k.weight", hidden, kvd)
        mat(p + "attn_v.weight", hidden, kvd)
        mat(p + "attn_output.weight", qd, hidden)
        mat(p + "ffn_gate.weight", hidden, ffn)
        mat(p + "ffn_up.weight", hidden, ffn)
        mat(p + "ffn_down.weight", ffn, hidden)
        for n, size in (("attn_norm", hidden), ("post_attention_norm", hidden),
                        ("ffn_norm", hidden), ("post_ffw_norm", hidden),
                        ("attn_q_norm", head_dim), ("attn_k_norm", head_dim)):
            norm(p + n + ".weight", size)
    norm("output_norm.weight", hidden)
    mat("token_embd.weight", hidden, vocab)
    write_gguf(path, meta, tensors)
    return values
