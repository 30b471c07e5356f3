"""An independent float64 restatement of one Gemma-3 decode token, written
from the reference's engine and kernel sources, not from the oracle:

* token order: DecodeSession::record_token, examples/llm/decode.cpp:1668-1752
  (attn norm -> q | k | v -> QK-norm -> RoPE -> KV append -> scores over
  [kv_start, seq_len) -> softmax -> apply -> o -> post-attn norm -> residual;
  ffn norm -> gate, up -> GeGLU -> down -> post-ffw norm -> residual), then
  the final norm and the lm_head (:1754-1755);
* layer policy: DecodeConfig::layer_is_global / rope_theta / layer_window /
  attn_kv_start, examples/llm/decode.hpp:327-352 (global iff
  (l + 1) % global_every == 0; kv_start = 0 when the window is 0 or
  seq_len <= window, else seq_len - window);
* scales: effective_embed_scale sqrt(hidden), effective_attn_scale
  1 / sqrt(head_dim), decode.cpp:277-282;
* kernels: rmsnorm_apply_gemma x * rsqrt(mean(x^2) + eps) * (1 + w) and its
  per-head form, llm_transformer.cl:96-134; rotate-half RoPE with
  inv = exp2(-log2(theta) * 2d / head_dim), :158-179; GeGLU with the tanh
  GELU, :213-231; attention_scores / attention_apply with kv head
  h / (n_heads / kv_heads), :287-305, :478-500;
* the packed weights: KM4 nibble plane uint4 wq[(g nblk + b) 64 + t] for
  column j = 64 g + t, block b = k / 32, word (k >> 3) & 3, nibble (k & 7) 4,
  value nibble - 8 (decode.hpp:45-48); fp16 scale quads
  sc[((b / 4) cols + j) 4 + b % 4] (decode.hpp:369-370, fp16 payload).

Everything is float64 except the KV cache, which holds fp16 rows as the
build's cache does (the benchmark specification asks for an fp16 cache; the
reference's is fp32). Test infrastructure only: it checks the oracle's
whole-token forward, with `mistakes` to show that the comparison fails for
plausible misreadings of the reference.
"""
from __future__ import annotations

import numpy as np

# Plausible misreadings of the reference, each planted on demand.
MISTAKES = (
    "global_policy_l_mod",      # global iff l % global_every == 0
    "theta_swapped",            # global layers rotate with the local theta
    "kv_start_off_by_one",      # kv_start = seq_len - window + 1
    "post_norms_swapped",       # post-attn and post-ffw norm weights exchanged
    "no_one_plus_w",            # x_hat * w instead of x_hat * (1 + w)
    "rope_interleaved",         # (2d, 2d + 1) pairs instead of (d, d + hd / 2)
    "embed_unscaled",           # no sqrt(hidden) on the embedding
    "gelu_erf",                 # exact GELU instead of the tanh form
    "no_qk_norm",               # QK-norm skipped
)


def unpack_km4(wq: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """int [rows (k)][cols (j)] weight values in [-8, 7] from a KM4 plane."""
    nblk = rows // 32
    w = np.asarray(wq, np.uint32).reshape(cols // 64, nblk, 64, 4)   # [g][b][t][word]
    nib = np.stack([(w >> np.uint32(4 * n)) & np.uint32(15) for n in range(8)], axis=-1)
    # nib[g][b][t][word][n] is k = 32 b + 8 word + n of column 64 g + t
    vals = nib.astype(np.int64) - 8
    return vals.transpose(1, 3, 4, 0, 2).reshape(rows, cols)


def pack_km4(w: np.ndarray) -> np.ndarray:
    """The KM4 plane of int values w[k][j] in [-8, 7] (inverse of unpack_km4)."""
    rows, cols = w.shape
    nib = (np.asarray(w, np.int64) + 8).astype(np.uint32)
    nib = nib.reshape(rows // 32, 4, 8, cols // 64, 64).transpose(3, 0, 4, 1, 2)  # [g][b][t][word][n]
    out = np.zeros(nib.shape[:4], np.uint32)
    for n in range(8):
        out |= nib[..., n] << np.uint32(4 * n)
    return out.reshape(-1)


def scales_f64(sc: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """float64 [rows / 32][cols] group scales from an fp16 quad plane."""
    q = np.asarray(sc, np.uint16).reshape(rows // 128, cols, 4)      # [b / 4][j][b % 4]
    s = q.transpose(0, 2, 1).reshape(rows // 32, cols)
    return s.view(np.float16).astype(np.float64)


def dequant(wq, sc, rows: int, cols: int) -> np.ndarray:
    """float64 W[k][j] = (nibble - 8) * scale of k's 32-block."""
    return unpack_km4(wq, rows, cols) * np.repeat(scales_f64(sc, rows, cols), 32, axis=0)


def _fp16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float64).astype(np.float16)


class F64Model:
    """Weights as float64 matrices, an fp16 KV cache, the residual stream in
    float64. `p` holds the shape (n_layers, hidden, ffn, n_heads, n_kv_heads,
    head_dim, vocab, max_seq, global_every, sliding_window, rms_eps,
    rope_theta_global, rope_theta_local) as attributes; `get(layer, name)`
    returns packed planes ('q', 'k', ..., 'lm_head': (wq, sc)) or norm weights
    stored as multiplier - 1 ('attn_norm', ..., 'final_norm')."""

    MATS = ("q", "k", "v", "o", "gate", "up", "down")
    NORMS = ("attn_norm", "post_attn_norm", "ffn_norm", "post_ffn_norm", "q_norm", "k_norm")

    def __init__(self, p, get, embed=None, mistakes=()):
        self.p = p
        self.mistakes = set(mistakes)
        unknown = self.mistakes - set(MISTAKES)
        assert not unknown, unknown
        H, F, qd = p.hidden, p.ffn, p.n_heads * p.head_dim
        kvd = p.n_kv_heads * p.head_dim
        dims = {"q": (H, qd), "k": (H, kvd), "v": (H, kvd), "o": (qd, H), "gate": (H, F),
                "up": (H, F), "down": (F, H)}
        self.W = []
        self.N = []
        for l in range(p.n_layers):
            self.W.append({m: dequant(*get(l, m), *dims[m]) for m in self.MATS})
            self.N.append({n: np.asarray(get(l, n), np.float64) for n in self.NORMS})
        self.lm = dequant(*get(-1, "lm_head"), H, p.vocab)
        self.final_norm = np.asarray(get(-1, "final_norm"), np.float64)
        self.embed = None if embed is None else np.asarray(embed, np.float64)
        self.kc = [np.zeros((p.max_seq, kvd), np.float16) for _ in range(p.n_layers)]
        self.vc = [np.zeros((p.max_seq, kvd), np.float16) for _ in range(p.n_layers)]

    # ---- the reference's kernels, float64 ----
    def _norm(self, x, w):
        mult = w if "no_one_plus_w" in self.mistakes else 1.0 + w
        return x / np.sqrt(np.mean(x * x) + self.p.rms_eps) * mult

    def _rope(self, v, pos, theta):
        hd = self.p.head_dim
        half = hd // 2
        d = np.arange(half, dtype=np.float64)
        ang = pos * np.exp2(-np.log2(theta) * (2.0 * d / hd))
        c, s = np.cos(ang), np.sin(ang)
        out = v.copy()
        for h in range(v.size // hd):
            r = v[h * hd:(h + 1) * hd]
            if "rope_interleaved" in self.mistakes:
                lo, hi = r[0::2], r[1::2]
                out[h * hd:(h + 1) * hd][0::2] = lo * c - hi * s
                out[h * hd:(h + 1) * hd][1::2] = lo * s + hi * c
            else:
                lo, hi = r[:half], r[half:]
                out[h * hd:h * hd + half] = lo * c - hi * s
                out[h * hd + half:(h + 1) * hd] = lo * s + hi * c
        return out

    def _gelu(self, g):
        if "gelu_erf" in self.mistakes:
            from scipy.special import erf
            return 0.5 * g * (1.0 + erf(g / np.sqrt(2.0)))
        return 0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3)))

    def is_global(self, l):
        ge = self.p.global_every
        if ge == 0:
            return True
        if "global_policy_l_mod" in self.mistakes:
            return l % ge == 0
        return (l + 1) % ge == 0

    def kv_start(self, l, seq_len):
        w = 0 if self.is_global(l) else self.p.sliding_window
        if w == 0 or seq_len <= w:
            return 0
        return seq_len - w + (1 if "kv_start_off_by_one" in self.mistakes else 0)

    def embed_row(self, token):
        sc = 1.0 if "embed_unscaled" in self.mistakes else np.sqrt(self.p.hidden)
        row = self.embed[token] if self.embed is not None else self.lm[:, token]
        return row * sc

    def forward(self, token: int, pos: int, want_logits: bool = True):
        p = self.p
        hd, nh, nkv = p.head_dim, p.n_heads, p.n_kv_heads
        qd = nh * hd
        seq_len = pos + 1
        x = self.embed_row(token).copy()
        for l in range(p.n_layers):
            W, N = self.W[l], self.N[l]
            glob = self.is_global(l)
            theta = p.rope_theta_global if glob and "theta_swapped" not in self.mistakes \
                else p.rope_theta_local
            kv0 = self.kv_start(l, seq_len)
            xb = self._norm(x, N["attn_norm"])
            q, k, v = xb @ W["q"], xb @ W["k"], xb @ W["v"]
            if "no_qk_norm" not in self.mistakes:
                q = np.concatenate([self._norm(q[h * hd:(h + 1) * hd], N["q_norm"]) for h in range(nh)])
                k = np.concatenate([self._norm(k[h * hd:(h + 1) * hd], N["k_norm"]) for h in range(nkv)])
            q, k = self._rope(q, pos, theta), self._rope(k, pos, theta)
            self.kc[l][pos] = _fp16(k)
            self.vc[l][pos] = _fp16(v)
            K = self.kc[l][kv0:seq_len].astype(np.float64)
            V = self.vc[l][kv0:seq_len].astype(np.float64)
            att = np.empty(qd)
            group = nh // nkv
            for h in range(nh):
                kh = h // group
                s = K[:, kh * hd:(kh + 1) * hd] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
                e = np.exp(s - s.max())
                att[h * hd:(h + 1) * hd] = (e / e.sum()) @ V[:, kh * hd:(kh + 1) * hd]
            a = att @ W["o"]
            post_a, post_f = N["post_attn_norm"], N["post_ffn_norm"]
            if "post_norms_swapped" in self.mistakes:
                post_a, post_f = post_f, post_a
            x = x + self._norm(a, post_a)
            xb = self._norm(x, N["ffn_norm"])
            h_ = self._gelu(xb @ W["gate"]) * (xb @ W["up"])
            x = x + self._norm(h_ @ W["down"], post_f)
        if not want_logits:
            return None
        return self._norm(x, self.final_norm) @ self.lm


def random_model(p, seed: int, untied_embed: bool = False):
    """Random packed tensors for shape `p`: nibbles uniform in [0, 15], fp16
    scales |N(0, 0.02)|, norm multipliers N(1, 0.1) stored as m - 1, and
    optionally an fp32 N(0, 1) embedding table. Returns (get, embed, ints)
    where get(layer, name) is what F64Model takes and ints holds the int
    weight values for checking the packer."""
    r = np.random.default_rng(seed)
    H, F, qd = p.hidden, p.ffn, p.n_heads * p.head_dim
    kvd = p.n_kv_heads * p.head_dim
    dims = {"q": (H, qd), "k": (H, kvd), "v": (H, kvd), "o": (qd, H), "gate": (H, F),
            "up": (H, F), "down": (F, H)}
    t = {}
    ints = {}

    def mat(key, rows, cols):
        w = r.integers(-8, 8, (rows, cols))
        s = np.abs(r.normal(0.0, 0.02, (rows // 32, cols))).astype(np.float16)
        quad = s.reshape(rows // 128, 4, cols).transpose(0, 2, 1).reshape(-1).view(np.uint16)
        t[key] = (pack_km4(w), np.ascontiguousarray(quad))
        ints[key] = w

    for l in range(p.n_layers):
        for m, (rows, cols) in dims.items():
            mat((l, m), rows, cols)
        for n, size in (("attn_norm", H), ("post_attn_norm", H), ("ffn_norm", H),
                        ("post_ffn_norm", H), ("q_norm", p.head_dim), ("k_norm", p.head_dim)):
            t[(l, n)] = (r.normal(1.0, 0.1, size) - 1.0).astype(np.float32)
    mat((-1, "lm_head"), H, p.vocab)
    t[(-1, "final_norm")] = (r.normal(1.0, 0.1, H) - 1.0).astype(np.float32)
    embed = r.normal(0.0, 1.0, (p.vocab, H)).astype(np.float32) if untied_embed else None
    return (lambda l, n: t[(l, n)]), embed, ints
