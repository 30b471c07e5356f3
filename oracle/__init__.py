"""ctypes binding of oracle/liboracle.so — the CPU restatement of the
reference arithmetic.

TEST INFRASTRUCTURE ONLY: imported by tests/, by the graft entry's smoke()
(as the checker) and by bench.py's cpu_baseline leg (as the timed CPU
baseline). The product path (xpose_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
I8P = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")


class QWeight(C.Structure):
    _fields_ = [("wq", C.c_void_p), ("sc", C.c_void_p), ("rows", C.c_uint32),
                ("cols", C.c_uint32)]


class Layer(C.Structure):
    _fields_ = [(n, QWeight) for n in ("q", "k", "v", "o", "gate", "up", "down")] + \
               [(n, C.c_void_p) for n in ("attn_norm", "post_attn_norm", "ffn_norm",
                                          "post_ffn_norm", "q_norm", "k_norm", "kcache",
                                          "vcache")]


class Model(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "hidden", "ffn", "n_heads",
                                          "n_kv_heads", "head_dim", "vocab", "max_seq",
                                          "global_every", "sliding_window")] + \
               [("rms_eps", C.c_float), ("theta_global", C.c_float),
                ("theta_local", C.c_float), ("layers", C.c_void_p),
                ("lm_head", QWeight), ("final_norm", C.c_void_p), ("scale_fmt", C.c_int32),
                ("embed", C.c_void_p)]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run `python -m xpose_amd.build --oracle-only`")
        l = C.CDLL(LIB_PATH)
        u32, f32, i32, vp, f64 = C.c_uint32, C.c_float, C.c_int, C.c_void_p, C.c_double
        decl = {
            "xo_fp16_to_fp32": (f32, [u32]),
            "xo_fp32_to_fp16": (C.c_uint16, [f32]),
            "xo_bf16_to_fp32": (f32, [u32]),
            "xo_q4dot8": (f32, [u32, F32P]),
            "xo_mv_km4": (None, [F32P, F32P, U32P, vp, i32, u32, u32]),
            "xo_mv_km4_bs": (None, [F32P, F32P, U32P, vp, i32, u32, u32]),
            "xo_mv_km4_split": (None, [F32P, F32P, U32P, vp, i32, u32, u32, u32]),
            "xo_mv_reduce": (None, [F32P, F32P, u32, u32]),
            "xo_matvec_q4_col": (None, [F32P, F32P, U32P, F32P, u32, u32]),
            "xo_nib_hash": (u32, [u32, u32]),
            "xo_pack_km4_hash": (None, [U32P, u32, u32]),
            "xo_pack_col_hash": (None, [U32P, u32, u32]),
            "xo_unpack_km4": (None, [I8P, U32P, u32, u32]),
            "xo_rmsnorm_gemma2": (None, [F32P, F32P, F32P, u32, u32, f32]),
            "xo_rmsnorm_heads_gemma": (None, [F32P, F32P, F32P, u32, u32, f32]),
            "xo_rope": (None, [F32P, u32, u32, u32, f32]),
            "xo_geglu": (None, [F32P, F32P, F32P, u32]),
            "xo_add_residual": (None, [F32P, F32P, u32]),
            "xo_kv_append_f16": (None, [U16P, F32P, u32, u32]),
            "xo_attention_scores": (None, [F32P, F32P, F32P, u32, u32, u32, u32, f32, u32]),
            "xo_softmax_rows": (None, [F32P, u32, u32]),
            "xo_attention_apply": (None, [F32P, F32P, F32P, u32, u32, u32, u32, u32]),
            "xo_attention_f16": (None, [F32P, F32P, U16P, U16P, u32, u32, u32, u32, u32, f32]),
            "xo_argmax_partial": (None, [F32P, U32P, F32P, u32, u32]),
            "xo_argmax_reduce": (None, [F32P, U32P, F32P, U32P, u32, u32]),
            "xo_argmax_final": (None, [F32P, U32P, F32P, U32P, u32]),
            "xo_argmax_tree": (u32, [F32P, u32, C.POINTER(f32)]),
            "xo_apply_temperature": (None, [F32P, f32, u32]),
            "xo_reduce_max_partial": (None, [F32P, F32P, u32, u32]),
            "xo_reduce_max_final": (None, [F32P, F32P, u32]),
            "xo_softmax_exp_partial": (None, [F32P, F32P, F32P, F32P, u32, u32]),
            "xo_reduce_sum_partial": (None, [F32P, F32P, u32, u32]),
            "xo_reduce_sum_final": (None, [F32P, F32P, u32]),
            "xo_softmax_normalize": (None, [F32P, F32P, u32]),
            "xo_topk_mask": (None, [F32P, F32P, u32, u32]),
            "xo_multinomial_strided": (None, [F32P, U32P, F32P, F32P, F32P, u32, u32, f32]),
            "xo_topk4_partial": (None, [F32P, U32P, F32P, u32, u32]),
            "xo_topk_partial": (None, [F32P, U32P, F32P, u32, u32, u32]),
            "xo_topk_rank_select": (None, [F32P, U32P, F32P, U32P, u32, u32]),
            "xo_topp_cutoff": (None, [F32P, u32, f32]),
            "xo_multinomial_sample": (None, [F32P, U32P, F32P, U32P, u32, f32]),
            "xo_draw": (u32, [F32P, U32P, u32, f32, u32, f32, f64]),
            "xo_philox_uniform": (f64, [u32, u32, u32]),
            "xo_philox4x32_10": (None, [U32P, U32P, U32P]),
            "xo_embed": (None, [F32P, C.POINTER(Model), u32]),
            "xo_dequantize": (i32, [u32, vp, F32P, C.c_uint64]),
            "xo_pack_int4": (None, [F32P, u32, u32, i32, U32P, vp]),
            "xo_quantise": (u32, [f32, f32]),
            "xo_best_bf16_scale": (f32, [F32P, f32]),
            "xo_rq_repack": (i32, [u32, vp, u32, u32, U32P, vp, F32P, vp]),
            "xo_softmax_rows_stats": (None, [F32P, F32P, u32, u32]),
            "xo_softmax_rows_apply": (None, [F32P, F32P, u32, u32]),
            "xo_attention_scores_prefill": (None, [F32P, F32P, F32P, u32, u32, u32, u32, u32, u32, u32, f32]),
            "xo_attention_apply_prefill": (None, [F32P, F32P, F32P, u32, u32, u32, u32, u32]),
            "xo_rmsnorm_rows_sumsq": (None, [F32P, F32P, u32, u32]),
            "xo_rmsnorm_rows_apply_gemma": (None, [F32P, F32P, F32P, F32P, u32, u32, f32]),
            "xo_rmsnorm_heads_rows_gemma": (None, [F32P, F32P, F32P, u32, u32, u32, f32]),
            "xo_rope_prefill": (None, [F32P, u32, u32, u32, u32, f32]),
            "xo_kv_append_rows": (None, [F32P, F32P, u32, u32, u32]),
            "xo_embed_lookup_rows": (None, [F32P, F32P, U32P, u32, u32]),
            "xo_rq_reconstruct": (f32, [u32, u32, U32P, vp, F32P, vp, u32, u32]),
            "xo_forward": (i32, [C.POINTER(Model), u32, u32, vp, i32]),
            "xo_generate_greedy": (i32, [C.POINTER(Model), U32P, u32, u32, U32P, i32]),
        }
        for name, (res, args) in decl.items():
            fn = getattr(l, name)
            fn.restype, fn.argtypes = res, args
        _lib = l
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def mv_km4(x, wq, sc, rows: int, cols: int, fmt: int = 0, quad_sum: bool = False) -> np.ndarray:
    out = np.empty(cols, np.float32)
    sc = np.ascontiguousarray(sc)
    fn = lib().xo_mv_km4_bs if quad_sum else lib().xo_mv_km4
    fn(out, _f32(x), np.ascontiguousarray(wq, np.uint32), sc.ctypes.data, fmt, rows, cols)
    return out


def rmsnorm_gemma(x, w, eps: float = 1e-6, nparts: int = 64) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().xo_rmsnorm_gemma2(out, x, _f32(w), x.size, nparts, eps)
    return out


def dequantize(ggml_type: int, raw, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    raw = np.ascontiguousarray(raw)
    if lib().xo_dequantize(ggml_type, raw.ctypes.data, out, n) != 0:
        raise ValueError(f"xo_dequantize: type {ggml_type} / {n} elements")
    return out


def pack_int4(w_cols, bf16: bool = True):
    """The reference packer over w[cols][rows]: (KM4 plane, scale plane)."""
    w_cols = _f32(w_cols)
    cols, rows = w_cols.shape
    wq = np.empty(rows * cols // 8, np.uint32)
    sc = np.empty(rows // 32 * cols, np.uint16 if bf16 else np.float32)
    lib().xo_pack_int4(w_cols, rows, cols, 1 if bf16 else 0, wq, sc.ctypes.data)
    return wq, sc


RQ_TYPES = {8: (8, 0, 1, False), 6: (4, 1, 1, False), 12: (4, 0, 1, True), 14: (4, 2, 2, False)}


def rq_repack(ggml_type: int, raw, rows: int, cols: int) -> dict:
    """repack() of quant_repack.cpp: the planes of a rows x cols native
    matrix as numpy arrays (quant, high, scale, bias; None where absent)."""
    qw, hw, sw, has_bias = RQ_TYPES[ggml_type]
    slots = (rows + 63) // 64 * (cols // 32) * 64
    quant = np.empty(slots * qw, np.uint32)
    high = np.empty(slots * hw, np.uint32) if hw else None
    scale = np.empty(slots * sw, np.float32)
    bias = np.empty(slots, np.float32) if has_bias else None
    raw = np.ascontiguousarray(raw)
    rc = lib().xo_rq_repack(ggml_type, raw.ctypes.data, rows, cols, quant,
                            None if high is None else high.ctypes.data, scale,
                            None if bias is None else bias.ctypes.data)
    if rc != 0:
        raise ValueError(f"xo_rq_repack refused type {ggml_type} {rows} x {cols}")
    return {"quant": quant, "high": high, "scale": scale, "bias": bias}


def rq_reconstruct(ggml_type: int, planes: dict, rows: int, cols: int) -> np.ndarray:
    """reconstruct() at every (r, k): float32 [rows][cols]."""
    out = np.empty((rows, cols), np.float32)
    f = lib().xo_rq_reconstruct
    h = None if planes["high"] is None else planes["high"].ctypes.data
    b = None if planes["bias"] is None else planes["bias"].ctypes.data
    for r in range(rows):
        for k in range(cols):
            out[r, k] = f(ggml_type, cols // 32, planes["quant"], h, planes["scale"], b, r, k)
    return out


def argmax_tree(logits) -> tuple[int, float]:
    v = C.c_float()
    i = lib().xo_argmax_tree(_f32(logits), np.asarray(logits).size, C.byref(v))
    return int(i), float(v.value)


class OracleModel:
    """The oracle's model: the same packed tensors the GPU session holds
    (fp16 quad scales), an fp16 KV cache, and xo_forward in record_token
    order. `get(layer, tensor)` supplies each tensor as a numpy array."""

    def __init__(self, cfg, get, embed=None):
        """`embed`: optional fp32 [vocab][hidden] embedding rows (a GGUF
        model's table); the scale planes are in cfg.scale_fmt."""
        import xpose_amd as X
        self.cfg = cfg
        self._keep = []
        L = cfg.n_layers
        kvd = cfg.n_kv_heads * cfg.head_dim
        self.kcache = [np.zeros(cfg.max_seq * kvd, np.uint16) for _ in range(L)]
        self.vcache = [np.zeros(cfg.max_seq * kvd, np.uint16) for _ in range(L)]
        layers = (Layer * L)()

        def qw(layer, m):
            from xpose_amd import MATRICES  # noqa: F401
            w = np.ascontiguousarray(get(layer, m))
            s = np.ascontiguousarray(get(layer, m | X.T_SCALES))
            self._keep += [w, s]
            rows = {X.T_Q: cfg.hidden, X.T_K: cfg.hidden, X.T_V: cfg.hidden,
                    X.T_O: cfg.n_heads * cfg.head_dim, X.T_GATE: cfg.hidden,
                    X.T_UP: cfg.hidden, X.T_DOWN: cfg.ffn, X.T_LM_HEAD: cfg.hidden}[m]
            return QWeight(w.ctypes.data, s.ctypes.data, rows, w.size * 8 // rows)

        for l in range(L):
            ly = layers[l]
            for name, m in (("q", X.T_Q), ("k", X.T_K), ("v", X.T_V), ("o", X.T_O),
                            ("gate", X.T_GATE), ("up", X.T_UP), ("down", X.T_DOWN)):
                setattr(ly, name, qw(l, m))
            for name, t in (("attn_norm", X.T_ATTN_NORM), ("post_attn_norm", X.T_POST_ATTN_NORM),
                            ("ffn_norm", X.T_FFN_NORM), ("post_ffn_norm", X.T_POST_FFN_NORM),
                            ("q_norm", X.T_Q_NORM), ("k_norm", X.T_K_NORM)):
                a = np.ascontiguousarray(get(l, t), np.float32)
                self._keep.append(a)
                setattr(ly, name, a.ctypes.data)
            ly.kcache = self.kcache[l].ctypes.data
            ly.vcache = self.vcache[l].ctypes.data
        self._layers = layers
        fn = np.ascontiguousarray(get(-1, X.T_FINAL_NORM), np.float32)
        self._keep.append(fn)
        m = Model()
        for f in ("n_layers", "hidden", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab",
                  "max_seq", "global_every", "sliding_window", "rms_eps"):
            setattr(m, f, getattr(cfg, f))
        m.theta_global = cfg.rope_theta_global
        m.theta_local = cfg.rope_theta_local
        m.layers = C.cast(layers, C.c_void_p)
        m.lm_head = qw(-1, X.T_LM_HEAD)
        m.final_norm = fn.ctypes.data
        m.scale_fmt = cfg.scale_fmt
        if embed is not None:
            e = np.ascontiguousarray(embed, np.float32)
            self._keep.append(e)
            m.embed = e.ctypes.data
        self.model = m

    def forward(self, token: int, pos: int, want_logits: bool = True, threads: int = 0):
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        rc = lib().xo_forward(C.byref(self.model), token, pos,
                              logits.ctypes.data if want_logits else None, threads)
        if rc != 0:
            raise RuntimeError(f"xo_forward failed ({rc})")
        return logits

    def generate_greedy(self, prompt, n_gen: int, threads: int = 0) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(n_gen, np.uint32)
        rc = lib().xo_generate_greedy(C.byref(self.model), prompt, prompt.size, n_gen, out,
                                      threads)
        if rc != 0:
            raise RuntimeError(f"xo_generate_greedy failed ({rc})")
        return out
