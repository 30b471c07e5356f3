"""xpose_amd — MI355X (gfx950) Gemma-3 int4 decode hot path.

Python binding of the C ABI in include/xpose.h (libxpose.so, built in-tree by
xpose_amd/build.py). The binding is ctypes + numpy only: device memory and
streams come from the library itself, so no second HIP runtime is loaded.
Loading fails loudly if the shared object is missing; there is no CPU
fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libxpose.so")

XP_SCALE_F16_QUAD = 0
XP_SCALE_BF16_QUAD = 1
XP_SCALE_F32 = 2

XP_EXEC_AUTO, XP_EXEC_GRAPH, XP_EXEC_LAUNCH, XP_EXEC_TOKEN = 0, 1, 2, 3
XP_PREFILL_AUTO, XP_PREFILL_TOKENS = 0, 1
XP_PLACE_AUTO, XP_PLACE_DEVICE = 0, 1

_lib = None

# Tensor ids (enum xp_tensor in include/xpose.h).
T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN = range(7)
T_ATTN_NORM, T_POST_ATTN_NORM, T_FFN_NORM, T_POST_FFN_NORM, T_Q_NORM, T_K_NORM = range(16, 22)
T_LM_HEAD, T_FINAL_NORM, T_EMBED = 32, 33, 34
T_SCALES = 0x100
MATRICES = (T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN)
NORMS = (T_ATTN_NORM, T_POST_ATTN_NORM, T_FFN_NORM, T_POST_FFN_NORM, T_Q_NORM, T_K_NORM)


class XpConfig(C.Structure):
    """xp_config (include/xpose.h), the reference's DecodeConfig + Sampling."""
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "hidden", "ffn", "n_heads", "n_kv_heads",
                                          "head_dim", "vocab", "max_seq", "global_every",
                                          "sliding_window")] + \
               [(n, C.c_float) for n in ("rms_eps", "rope_theta_global", "rope_theta_local",
                                         "embed_scale", "attn_scale")] + \
               [("scale_fmt", C.c_int32), ("sample_mode", C.c_int32),
                ("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("seed", C.c_uint32), ("seq_id", C.c_uint32), ("topk_parts", C.c_uint32),
                ("exec_mode", C.c_int32), ("prefill_mode", C.c_int32), ("placement", C.c_int32)]

    @classmethod
    def gemma3_1b(cls, **overrides) -> "XpConfig":
        c = cls()
        lib().xp_config_gemma3_1b(C.byref(c))
        for k, v in overrides.items():
            setattr(c, k, v)
        return c

    def is_global(self, layer: int) -> bool:
        return self.global_every == 0 or (layer + 1) % self.global_every == 0


class GgufInfo(C.Structure):
    _fields_ = [("version", C.c_uint32)] + [(n, C.c_uint64) for n in (
        "n_tensors", "n_meta", "alignment", "data_offset", "file_size")]


class GgufModel(C.Structure):
    _fields_ = [("arch", C.c_char * 32)] + [(n, C.c_uint32) for n in (
        "n_layers", "n_heads", "n_kv_heads", "hidden", "ffn", "context_length", "key_length",
        "value_length", "vocab", "sliding_window", "head_dim")] + [
        ("rope_freq_base", C.c_float), ("rms_eps", C.c_float)]


class LoadStats(C.Structure):
    _fields_ = [(n, C.c_double) for n in ("total_ms", "pack_ms", "cache_ms", "upload_ms")] + [
        ("packed_bytes", C.c_uint64), ("from_cache", C.c_int32), ("cache_written", C.c_int32),
        ("threads", C.c_uint32), ("n_tensors", C.c_uint32)]


class TokenizerIds(C.Structure):
    _fields_ = [("vocab", C.c_uint32)] + [(n, C.c_int32) for n in (
        "bos", "eos", "unk", "pad", "add_bos", "add_eos", "add_space_prefix")]


# enum xp_ggml_type / xp_load_flags
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q5_0, GGML_Q5_1, GGML_Q8_0 = 0, 1, 2, 3, 6, 7, 8
GGML_Q4_K, GGML_Q6_K, GGML_BF16 = 12, 14, 30
LOAD_REPACK, LOAD_NORM_RAW, LOAD_NO_EMBED = 1, 2, 4


class RqLayout(C.Structure):
    """xp_rq_layout: plane sizes of a repacked native-format matrix."""
    _fields_ = [("type", C.c_uint32), ("rows", C.c_uint32), ("padded_rows", C.c_uint32),
                ("cols", C.c_uint32), ("nkb", C.c_uint32), ("reserved", C.c_uint32),
                ("quant_bytes", C.c_uint64), ("high_bytes", C.c_uint64),
                ("scale_bytes", C.c_uint64), ("bias_bytes", C.c_uint64),
                ("native_bytes", C.c_uint64)]


class RqTensor(C.Structure):
    """xp_rq_tensor: device planes of one repacked matrix."""
    _fields_ = [("type", C.c_uint32), ("rows", C.c_uint32), ("cols", C.c_uint32),
                ("reserved", C.c_uint32), ("quant", C.c_void_p), ("high", C.c_void_p),
                ("scale", C.c_void_p), ("bias", C.c_void_p)]


class XpMetrics(C.Structure):
    _fields_ = [("ms", C.c_double), ("gpu_ms", C.c_double), ("sample_ms", C.c_double),
                ("tokens_per_sec", C.c_double), ("position", C.c_uint32),
                ("launches", C.c_uint32), ("exec_mode", C.c_int32)]


class XposeError(RuntimeError):
    """A libxpose entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def _declare(lib: C.CDLL) -> None:
    vp, u32, i32, f32, sz = C.c_void_p, C.c_uint32, C.c_int, C.c_float, C.c_size_t
    P = C.POINTER
    sig = {
        "xp_last_error": (C.c_char_p, []),
        "xp_version": (C.c_char_p, []),
        "xp_init": (i32, [i32]),
        "xp_device_info": (i32, [C.c_char_p, sz, P(i32), P(sz), C.c_char_p, sz]),
        "xp_malloc": (i32, [P(vp), sz]),
        "xp_free": (i32, [vp]),
        "xp_memcpy_htod": (i32, [vp, vp, sz]),
        "xp_memcpy_dtoh": (i32, [vp, vp, sz]),
        "xp_memcpy_dtod": (i32, [vp, vp, sz]),
        "xp_memset": (i32, [vp, i32, sz]),
        "xp_synchronize": (i32, []),
        "xp_stream_create": (i32, [P(vp)]),
        "xp_stream_destroy": (i32, [vp]),
        "xp_stream_synchronize": (i32, [vp]),
        "xp_event_create": (i32, [P(vp)]),
        "xp_event_destroy": (i32, [vp]),
        "xp_event_record": (i32, [vp, vp]),
        "xp_event_elapsed_ms": (i32, [vp, vp, P(f32)]),
        "xp_mv_int4": (i32, [vp, vp, vp, vp, i32, u32, u32, u32, vp]),
        "xp_mv_int4_noalloc": (i32, [vp, vp, vp, vp, i32, u32, u32, u32, vp]),
        "xp_mv_int4_multi": (i32, [u32, P(vp), vp, P(vp), P(vp), P(u32), i32, u32, vp]),
        "xp_unpack_km4": (i32, [vp, vp, u32, u32, vp]),
        "xp_mv_int4_timed": (i32, [vp, vp, P(vp), P(vp), u32, i32, u32, u32, u32, u32, vp,
                                   P(f32)]),
        "xp_mv_int4_batch_timed": (i32, [vp, vp, P(vp), P(vp), u32, i32, u32, u32, u32, u32, u32,
                                         vp, P(f32)]),
        "xp_fp16_decode": (i32, [vp, vp, u32, vp]),
        "xp_stream_read_timed": (i32, [vp, sz, u32, vp, P(f32)]),
        "xp_stream_read_rot_timed": (i32, [P(vp), u32, sz, u32, u32, vp, P(f32)]),
        "xp_stream_read_rot_batch_timed": (i32, [P(vp), u32, sz, u32, u32, u32, vp, P(f32)]),
        "xp_exchange_chain_timed": (i32, [u32, u32, u32, i32, vp, P(f32)]),
        "xp_handoff_pingpong_timed": (i32, [u32, u32, i32, u32, vp, P(f32), P(u32)]),
        "xp_load_latency": (i32, [u32, u32, i32, vp, P(f32)]),
        "xp_copy": (i32, [vp, vp, sz, vp]),
        "xp_philox4x32_10": (None, [P(u32), P(u32), P(u32)]),
        "xp_synth_nibbles": (i32, [vp, u32, u32, u32, u32]),
        "xp_synth_scales": (i32, [vp, i32, u32, u32, f32, u32, u32]),
        "xp_synth_normal": (i32, [vp, sz, f32, f32, u32, u32]),
        "xp_synth_normal_f16": (i32, [vp, sz, f32, f32, u32, u32]),
        "xp_f32_to_f16": (C.c_uint16, [f32]),
        "xp_config_gemma3_1b": (None, [P(XpConfig)]),
        "xp_session_create": (i32, [P(XpConfig), P(vp)]),
        "xp_session_destroy": (i32, [vp]),
        "xp_batch_create": (i32, [vp, u32, u32, P(vp)]),
        "xp_batch_create2": (i32, [vp, u32, u32, i32, P(vp)]),
        "xp_batch_exec_mode": (i32, [vp, P(i32)]),
        "xp_batch_step_trace": (i32, [vp, i32]),
        "xp_batch_set_spin_limit": (i32, [vp, u32]),
        "xp_batch_step_trace_read": (i32, [vp, vp, C.c_size_t, P(C.c_size_t)]),
        "xp_batch_destroy": (i32, [vp]),
        "xp_batch_kv_upload": (i32, [vp, u32, i32, i32, u32, u32, vp]),
        "xp_batch_kv_download": (i32, [vp, u32, i32, i32, u32, u32, vp]),
        "xp_batch_set_positions": (i32, [vp, vp]),
        "xp_batch_positions": (i32, [vp, vp]),
        "xp_batch_forward": (i32, [vp, vp]),
        "xp_batch_decode_step": (i32, [vp, vp]),
        "xp_batch_decode_steps": (i32, [vp, u32, vp]),
        "xp_batch_last_logits": (i32, [vp, u32, vp, u32]),
        "xp_batch_last_candidates": (i32, [vp, u32, vp, vp, u32]),
        "xp_batch_last_ms": (i32, [vp, P(f32)]),
        "xp_tensor_bytes": (i32, [P(XpConfig), i32, i32, P(sz)]),
        "xp_session_upload": (i32, [vp, i32, i32, vp, sz]),
        "xp_session_upload_part": (i32, [vp, i32, i32, sz, vp, sz]),
        "xp_gguf_open": (i32, [C.c_char_p, P(vp)]),
        "xp_gguf_close": (i32, [vp]),
        "xp_gguf_get_info": (i32, [vp, P(GgufInfo)]),
        "xp_gguf_get_model": (i32, [vp, P(GgufModel)]),
        "xp_gguf_tensor_count": (i32, [vp, P(C.c_uint64)]),
        "xp_gguf_tensor_at": (i32, [vp, C.c_uint64, C.c_char_p, sz]),
        "xp_gguf_tensor_info": (i32, [vp, C.c_char_p, P(u32), P(u32), P(C.c_uint64),
                                      P(C.c_uint64)]),
        "xp_gguf_meta_number": (i32, [vp, C.c_char_p, P(C.c_double)]),
        "xp_gguf_meta_string": (i32, [vp, C.c_char_p, C.c_char_p, sz, P(sz)]),
        "xp_gguf_meta_array_length": (i32, [vp, C.c_char_p, P(C.c_uint64)]),
        "xp_dequantize": (i32, [u32, vp, vp, C.c_uint64]),
        "xp_softmax_rows_stats": (i32, [vp, vp, u32, u32, vp]),
        "xp_softmax_rows_apply": (i32, [vp, vp, u32, u32, vp]),
        "xp_attention_scores_prefill": (i32, [vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, f32, vp]),
        "xp_attention_apply_prefill": (i32, [vp, vp, vp, u32, u32, u32, u32, u32, vp]),
        "xp_rmsnorm_rows_sumsq": (i32, [vp, vp, u32, u32, vp]),
        "xp_rmsnorm_rows_apply_gemma": (i32, [vp, vp, vp, vp, u32, u32, f32, vp]),
        "xp_rmsnorm_heads_rows_gemma": (i32, [vp, vp, vp, u32, u32, u32, f32, vp]),
        "xp_rope_prefill": (i32, [vp, u32, u32, u32, u32, f32, vp]),
        "xp_kv_append_rows": (i32, [vp, vp, u32, u32, u32, vp]),
        "xp_embed_lookup_rows": (i32, [vp, vp, vp, u32, u32, u32, vp]),
        "xp_rq_layout_of": (i32, [u32, u32, u32, P(RqLayout)]),
        "xp_rq_repack": (i32, [P(RqLayout), vp, u32, vp, vp, vp, vp]),
        "xp_rq_reconstruct": (i32, [P(RqLayout), vp, vp, vp, vp, vp]),
        "xp_mv_rq": (i32, [vp, vp, P(RqTensor), u32, vp]),
        "xp_mv_rq_timed": (i32, [vp, vp, P(RqTensor), u32, u32, u32, vp, P(f32)]),
        "xp_dequant_native": (i32, [vp, vp, u32, C.c_uint64, vp]),
        "xp_mv_native": (i32, [vp, vp, vp, u32, u32, u32, vp]),
        "xp_gguf_dequantize_rows": (i32, [vp, C.c_char_p, C.c_uint64, C.c_uint64, vp]),
        "xp_config_from_gguf": (i32, [vp, P(XpConfig)]),
        "xp_pack_int4": (i32, [vp, u32, u32, i32, u32, vp, vp]),
        "xp_gguf_pack_model": (i32, [vp, P(XpConfig), C.c_char_p, u32, P(LoadStats)]),
        "xp_gguf_verify_cache": (i32, [vp, P(XpConfig), C.c_char_p, u32, P(u32)]),
        "xp_session_load_gguf": (i32, [vp, vp, C.c_char_p, u32, u32, P(LoadStats)]),
        "xp_tokenizer_create": (i32, [vp, P(vp)]),
        "xp_tokenizer_destroy": (i32, [vp]),
        "xp_tokenizer_info": (i32, [vp, P(TokenizerIds)]),
        "xp_tokenize": (i32, [vp, C.c_char_p, sz, i32, i32, vp, sz, P(sz)]),
        "xp_detokenize": (i32, [vp, vp, sz, i32, C.c_char_p, sz, P(sz)]),
        "xp_token_piece": (i32, [vp, i32, C.c_char_p, sz, P(sz)]),
        "xp_token_text": (i32, [vp, i32, C.c_char_p, sz, P(sz)]),
        "xp_token_find": (i32, [vp, C.c_char_p, sz, P(i32)]),
        "xp_token_kind": (i32, [vp, i32, P(i32), P(f32)]),
        "xp_synth_tensor": (i32, [P(XpConfig), u32, i32, i32, vp, sz]),
        "xp_session_synthesize": (i32, [vp, u32]),
        "xp_session_kv_upload": (i32, [vp, i32, i32, u32, u32, vp]),
        "xp_session_kv_download": (i32, [vp, i32, i32, u32, u32, vp]),
        "xp_session_set_position": (i32, [vp, u32]),
        "xp_session_set_spin_limit": (i32, [vp, u32]),
        "xp_session_prefill": (i32, [vp, vp, u32]),
        "xp_session_decode_step": (i32, [vp, P(u32)]),
        "xp_session_decode_steps": (i32, [vp, u32, vp]),
        "xp_session_reset": (i32, [vp]),
        "xp_session_position": (i32, [vp, P(u32)]),
        "xp_session_last_logits": (i32, [vp, vp, u32]),
        "xp_session_last_candidates": (i32, [vp, vp, vp, u32]),
        "xp_session_last_metrics": (i32, [vp, P(XpMetrics)]),
        "xp_session_weight_bytes": (i32, [vp, P(sz)]),
        "xp_session_kv_bytes": (i32, [vp, P(sz)]),
        "xp_session_trace": (i32, [vp, i32]),
        "xp_session_exec_mode": (i32, [vp, P(C.c_int32)]),
        "xp_session_last_trace": (i32, [vp, vp, sz, P(u32)]),
        "xp_draw": (u32, [vp, vp, u32, f32, u32, f32, C.c_double]),
        "xp_philox_uniform": (C.c_double, [u32, u32, u32]),
    }
    optional = {
        "xp_rmsnorm_gemma": (i32, [vp, vp, vp, u32, f32, vp]),
        "xp_rmsnorm_heads_gemma": (i32, [vp, vp, vp, u32, u32, f32, vp]),
        "xp_rope": (i32, [vp, u32, u32, u32, f32, vp]),
        "xp_qk_norm_rope_append": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32,
                                         u32, f32, f32, vp]),
        "xp_attention_decode": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, f32, vp]),
        "xp_attention_decode_timed": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, f32, u32,
                                            vp, C.POINTER(C.c_float)]),
        "xp_geglu": (i32, [vp, vp, vp, u32, vp]),
        "xp_add_residual": (i32, [vp, vp, u32, vp]),
        "xp_kv_append_f16": (i32, [vp, vp, u32, u32, vp]),
        "xp_argmax": (i32, [vp, vp, vp, u32, vp]),
        "xp_topk4_harvest": (i32, [vp, vp, vp, u32, u32, vp]),
        "xp_apply_temperature": (i32, [vp, f32, u32, vp]),
        "xp_reduce_max_partial": (i32, [vp, vp, u32, u32, vp]),
        "xp_reduce_max_final": (i32, [vp, vp, u32, vp]),
        "xp_softmax_exp_partial": (i32, [vp, vp, vp, vp, u32, u32, vp]),
        "xp_reduce_sum_partial": (i32, [vp, vp, u32, u32, vp]),
        "xp_reduce_sum_final": (i32, [vp, vp, u32, vp]),
        "xp_softmax_normalize": (i32, [vp, vp, u32, vp]),
        "xp_topk_partial": (i32, [vp, vp, vp, u32, u32, u32, vp]),
        "xp_topk_rank_select": (i32, [vp, vp, vp, vp, u32, u32, vp]),
        "xp_topk_mask": (i32, [vp, vp, u32, u32, vp]),
        "xp_topp_cutoff": (i32, [vp, u32, f32, vp]),
        "xp_multinomial_sample": (i32, [vp, vp, vp, vp, u32, f32, vp]),
        "xp_multinomial_strided": (i32, [vp, vp, vp, vp, vp, u32, u32, f32, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    for name, (res, args) in optional.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args


def lib() -> C.CDLL:
    """The loaded libxpose.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m xpose_amd.build` "
                "(the HIP path has no CPU fallback)")
        l = C.CDLL(LIB_PATH)
        _declare(l)
        _lib = l
    return _lib


def check(name: str, code: int) -> None:
    if code != 0:
        raise XposeError(name, code, lib().xp_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    """Calls a status-returning entry point and raises XposeError on failure."""
    check(name, getattr(lib(), name)(*args))


def init(dev: int = 0) -> None:
    call("xp_init", dev)


def device_info() -> dict:
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(64)
    cu = C.c_int()
    hbm = C.c_size_t()
    call("xp_device_info", name, 256, C.byref(cu), C.byref(hbm), arch, 64)
    return {"name": name.value.decode(), "arch": arch.value.decode(), "n_cu": cu.value,
            "hbm_bytes": hbm.value}


class DeviceBuffer:
    """A device allocation owned by Python (freed on close / garbage collection)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        call("xp_malloc", C.byref(p), self.nbytes)
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes, "upload past the end of the buffer"
        call("xp_memcpy_htod", C.c_void_p(self.ptr + offset), a.ctypes.data, a.nbytes)

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        out = np.empty(count, dtype=dt)
        assert offset + out.nbytes <= self.nbytes, "download past the end of the buffer"
        call("xp_memcpy_dtoh", out.ctypes.data, C.c_void_p(self.ptr + offset), out.nbytes)
        return out

    def fill_bytes(self, value: int) -> None:
        call("xp_memset", C.c_void_p(self.ptr), value, self.nbytes)

    def close(self) -> None:
        if self.ptr and _lib is not None:
            _lib.xp_free(C.c_void_p(self.ptr))
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def vp(self) -> C.c_void_p:
        return C.c_void_p(self.ptr)


def synchronize() -> None:
    call("xp_synchronize")


# ---- synthetic inputs (host side; no GPU needed) ---------------------------

def philox4x32_10(ctr, key) -> np.ndarray:
    c = (C.c_uint32 * 4)(*[int(v) & 0xFFFFFFFF for v in ctr])
    k = (C.c_uint32 * 2)(*[int(v) & 0xFFFFFFFF for v in key])
    o = (C.c_uint32 * 4)()
    lib().xp_philox4x32_10(c, k, o)
    return np.array(list(o), dtype=np.uint32)


def synth_nibbles(rows: int, cols: int, seed: int, tensor_id: int) -> np.ndarray:
    """KM4 nibble plane as uint32[rows*cols/8] (4 words per 32-weight block)."""
    w = np.empty(rows * cols // 8, dtype=np.uint32)
    call("xp_synth_nibbles", w.ctypes.data, rows, cols, seed, tensor_id)
    return w


def synth_scales(rows: int, cols: int, seed: int, tensor_id: int, sigma: float = 0.02,
                 fmt: int = XP_SCALE_F16_QUAD) -> np.ndarray:
    nblk = rows // 32
    if fmt == XP_SCALE_F16_QUAD:
        s = np.empty(nblk * cols, dtype=np.uint16)
    else:
        s = np.empty(nblk * cols, dtype=np.float32)
    call("xp_synth_scales", s.ctypes.data, fmt, rows, cols, sigma, seed, tensor_id)
    return s


def synth_normal(n: int, seed: int, tensor_id: int, mean: float = 0.0,
                 sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    call("xp_synth_normal", out.ctypes.data, n, mean, sigma, seed, tensor_id)
    return out


def synth_normal_f16(n: int, seed: int, tensor_id: int, mean: float = 0.0,
                     sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    call("xp_synth_normal_f16", out.ctypes.data, n, mean, sigma, seed, tensor_id)
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib().xp_f32_to_f16(float(x)))


# ---- synthetic model tensors (bit-identical to what a session synthesizes) --

def tensor_bytes(cfg: XpConfig, layer: int, tensor: int) -> int:
    b = C.c_size_t()
    call("xp_tensor_bytes", C.byref(cfg), layer, tensor, C.byref(b))
    return b.value


def synth_tensor(cfg: XpConfig, seed: int, layer: int, tensor: int) -> np.ndarray:
    """uint32 nibble planes, uint16 (fp16 quad) / float32 scale planes, float32 norms."""
    nb = tensor_bytes(cfg, layer, tensor)
    base = tensor & ~T_SCALES
    if base in MATRICES or base == T_LM_HEAD:
        if tensor & T_SCALES:
            dt = np.float32 if cfg.scale_fmt == XP_SCALE_F32 else np.uint16
        else:
            dt = np.uint32
    else:
        dt = np.float32
    out = np.empty(nb // np.dtype(dt).itemsize, dtype=dt)
    call("xp_synth_tensor", C.byref(cfg), seed, layer, tensor, out.ctypes.data, nb)
    return out


class DecodeBatch:
    """Up to 16 sequences decoded together on a DecodeSession's weights
    (xp_batch_*). The session must stay open while the batch lives."""

    def __init__(self, sess: "DecodeSession", n_seq: int, max_seq: int, exec_mode: int = 0):
        """exec_mode: XP_EXEC_AUTO (0), XP_EXEC_GRAPH (1) or XP_EXEC_TOKEN (3, the
        persistent step kernel), as xp_batch_create2."""
        self.sess = sess
        self.n = n_seq
        self.max_seq = max_seq
        h = C.c_void_p()
        call("xp_batch_create2", sess.h, n_seq, max_seq, exec_mode, C.byref(h))
        self.h = h

    def exec_mode(self) -> int:
        m = C.c_int32()
        call("xp_batch_exec_mode", self.h, C.byref(m))
        return m.value

    def set_spin_limit(self, rounds: int) -> None:
        call("xp_batch_set_spin_limit", self.h, rounds)

    def step_trace(self, enable: bool) -> None:
        call("xp_batch_step_trace", self.h, 1 if enable else 0)

    def step_trace_read(self) -> np.ndarray:
        """The step kernel's stage timeline, [n_layers][7][2][grid] then
        [grid] start times (100 MHz ticks), as xp_batch_step_trace."""
        n = C.c_size_t()
        call("xp_batch_step_trace_read", self.h, None, 0, C.byref(n))
        out = np.empty(n.value, np.uint64)
        call("xp_batch_step_trace_read", self.h, out.ctypes.data, out.size, C.byref(n))
        return out

    def close(self) -> None:
        if self.h and self.h.value and _lib is not None:
            _lib.xp_batch_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kv_upload(self, seq: int, layer: int, which: int, pos0: int, rows: np.ndarray) -> None:
        rows = np.ascontiguousarray(rows, np.uint16)
        kvd = self.sess.cfg.n_kv_heads * self.sess.cfg.head_dim
        call("xp_batch_kv_upload", self.h, seq, layer, which, pos0, rows.size // kvd, rows.ctypes.data)

    def kv_download(self, seq: int, layer: int, which: int, pos0: int, n: int) -> np.ndarray:
        kvd = self.sess.cfg.n_kv_heads * self.sess.cfg.head_dim
        out = np.empty(n * kvd, np.uint16)
        call("xp_batch_kv_download", self.h, seq, layer, which, pos0, n, out.ctypes.data)
        return out

    def set_positions(self, pos) -> None:
        pos = np.ascontiguousarray(pos, np.uint32)
        assert pos.size == self.n
        call("xp_batch_set_positions", self.h, pos.ctypes.data)

    def positions(self) -> np.ndarray:
        out = np.empty(self.n, np.uint32)
        call("xp_batch_positions", self.h, out.ctypes.data)
        return out

    def forward(self, tokens) -> None:
        t = np.ascontiguousarray(tokens, np.uint32)
        assert t.size == self.n
        call("xp_batch_forward", self.h, t.ctypes.data)

    def decode_step(self) -> np.ndarray:
        out = np.empty(self.n, np.uint32)
        call("xp_batch_decode_step", self.h, out.ctypes.data)
        return out

    def decode_steps(self, steps: int) -> np.ndarray:
        """steps sample-first steps queued back to back (the draws after the
        first on the device): [steps][n_seq] tokens, those of as many
        decode_step calls."""
        out = np.empty((steps, self.n), np.uint32)
        call("xp_batch_decode_steps", self.h, steps, out.ctypes.data)
        return out

    def last_logits(self, seq: int) -> np.ndarray:
        out = np.empty(self.sess.cfg.vocab, np.float32)
        call("xp_batch_last_logits", self.h, seq, out.ctypes.data, out.size)
        return out

    def last_candidates(self, seq: int, n: int = 64):
        v = np.empty(n, np.float32)
        i = np.empty(n, np.uint32)
        call("xp_batch_last_candidates", self.h, seq, v.ctypes.data, i.ctypes.data, n)
        return v, i

    def last_ms(self) -> float:
        ms = C.c_float()
        call("xp_batch_last_ms", self.h, C.byref(ms))
        return ms.value


class DecodeSession:
    """The engine-level entry points of the reference DecodeSession
    (examples/llm/decode.hpp:605-676) over the C ABI."""

    def __init__(self, cfg: XpConfig):
        self.cfg = cfg
        h = C.c_void_p()
        call("xp_session_create", C.byref(cfg), C.byref(h))
        self.h = h

    def close(self) -> None:
        if self.h and self.h.value and _lib is not None:
            _lib.xp_session_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synthesize(self, seed: int) -> None:
        call("xp_session_synthesize", self.h, seed)

    def load_gguf(self, g: "Gguf", cache: str | None = None, flags: int = 0,
                  threads: int = 0) -> LoadStats:
        """Requantises and uploads a GGUF model (xp_session_load_gguf)."""
        st = LoadStats()
        call("xp_session_load_gguf", self.h, g.h, cache.encode() if cache else None, flags,
             threads, C.byref(st))
        return st

    def upload(self, layer: int, tensor: int, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        call("xp_session_upload", self.h, layer, tensor, a.ctypes.data, a.nbytes)

    def kv_upload(self, layer: int, which: int, pos0: int, rows: np.ndarray) -> None:
        rows = np.ascontiguousarray(rows, np.uint16)
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        call("xp_session_kv_upload", self.h, layer, which, pos0, rows.size // kvd,
             rows.ctypes.data)

    def kv_download(self, layer: int, which: int, pos0: int, n: int) -> np.ndarray:
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        out = np.empty(n * kvd, np.uint16)
        call("xp_session_kv_download", self.h, layer, which, pos0, n, out.ctypes.data)
        return out

    def set_position(self, pos: int) -> None:
        call("xp_session_set_position", self.h, pos)

    def set_spin_limit(self, rounds: int) -> None:
        """Poll rounds a token-kernel wait takes before the step fails with
        XP_E_DEVICE (0: every wait not satisfied by its first read fails)."""
        call("xp_session_set_spin_limit", self.h, rounds)

    def prefill(self, ids) -> None:
        ids = np.ascontiguousarray(ids, np.uint32)
        call("xp_session_prefill", self.h, ids.ctypes.data, ids.size)

    def decode_step(self) -> int:
        t = C.c_uint32()
        call("xp_session_decode_step", self.h, C.byref(t))
        return t.value

    def decode_steps(self, n: int) -> np.ndarray:
        out = np.empty(n, np.uint32)
        call("xp_session_decode_steps", self.h, n, out.ctypes.data)
        return out

    def reset(self) -> None:
        call("xp_session_reset", self.h)

    @property
    def position(self) -> int:
        p = C.c_uint32()
        call("xp_session_position", self.h, C.byref(p))
        return p.value

    def last_logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.float32)
        call("xp_session_last_logits", self.h, out.ctypes.data, out.size)
        return out

    def last_candidates(self):
        n = 4 * self.cfg.topk_parts
        v = np.empty(n, np.float32)
        i = np.empty(n, np.uint32)
        call("xp_session_last_candidates", self.h, v.ctypes.data, i.ctypes.data, n)
        return v, i

    def last_metrics(self) -> XpMetrics:
        m = XpMetrics()
        call("xp_session_last_metrics", self.h, C.byref(m))
        return m

    def weight_bytes(self) -> int:
        b = C.c_size_t()
        call("xp_session_weight_bytes", self.h, C.byref(b))
        return b.value

    @property
    def exec_mode(self) -> int:
        """XP_EXEC_TOKEN (3), XP_EXEC_GRAPH (1) or XP_EXEC_LAUNCH (2)."""
        m = C.c_int32()
        call("xp_session_exec_mode", self.h, C.byref(m))
        return m.value

    def trace(self, enable: bool = True) -> None:
        """Record the persistent kernel's barrier timeline from now on."""
        call("xp_session_trace", self.h, 1 if enable else 0)

    def last_trace(self) -> np.ndarray:
        """[12 * n_layers + 3][grid] ticks (100 MHz) of the last launch: kernel
        start, the end of each layer's six stages, lm_head, argmax, then each
        stage's input arrival; 0 where a workgroup had no work in a stage."""
        g = C.c_uint32()
        probe = np.empty(1, np.uint64)
        call("xp_session_last_trace", self.h, probe.ctypes.data, 1, C.byref(g))
        ne = 12 * self.cfg.n_layers + 3
        out = np.empty(ne * g.value, np.uint64)
        call("xp_session_last_trace", self.h, out.ctypes.data, out.size, C.byref(g))
        return out.reshape(ne, g.value)


def draw(val, idx, temperature: float, top_k: int, top_p: float, u: float) -> int:
    v = np.array(val, np.float32)
    i = np.array(idx, np.uint32)
    return int(lib().xp_draw(v.ctypes.data, i.ctypes.data, v.size, temperature, top_k, top_p, u))


def philox_uniform(seed: int, seq: int, step: int) -> float:
    return float(lib().xp_philox_uniform(seed, seq, step))


class Gguf:
    """An open GGUF model file (xp_gguf_*): metadata, tensor table,
    dequantisation, and the packed-weight cache."""

    def __init__(self, path: str):
        h = C.c_void_p()
        call("xp_gguf_open", path.encode(), C.byref(h))
        self.h = h
        self.path = path

    def close(self) -> None:
        if self.h and self.h.value and _lib is not None:
            _lib.xp_gguf_close(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> GgufInfo:
        i = GgufInfo()
        call("xp_gguf_get_info", self.h, C.byref(i))
        return i

    def model(self) -> GgufModel:
        m = GgufModel()
        call("xp_gguf_get_model", self.h, C.byref(m))
        return m

    def tensor_names(self) -> list[str]:
        n = C.c_uint64()
        call("xp_gguf_tensor_count", self.h, C.byref(n))
        buf = C.create_string_buffer(256)
        out = []
        for i in range(n.value):
            call("xp_gguf_tensor_at", self.h, i, buf, 256)
            out.append(buf.value.decode())
        return out

    def tensor(self, name: str) -> tuple[int, tuple, int]:
        """(ggml type, dims (fastest first, n_dims of them), bytes)."""
        t, nd, nb = C.c_uint32(), C.c_uint32(), C.c_uint64()
        dims = (C.c_uint64 * 4)()
        call("xp_gguf_tensor_info", self.h, name.encode(), C.byref(t), C.byref(nd), dims,
             C.byref(nb))
        return t.value, tuple(dims[i] for i in range(nd.value)), nb.value

    def number(self, key: str) -> float:
        v = C.c_double()
        call("xp_gguf_meta_number", self.h, key.encode(), C.byref(v))
        return v.value

    def string(self, key: str) -> str:
        n = C.c_size_t()
        call("xp_gguf_meta_string", self.h, key.encode(), None, 0, C.byref(n))
        buf = C.create_string_buffer(n.value + 1)
        call("xp_gguf_meta_string", self.h, key.encode(), buf, n.value + 1, None)
        return buf.raw[:n.value].decode(errors="replace")

    def array_length(self, key: str) -> int:
        n = C.c_uint64()
        call("xp_gguf_meta_array_length", self.h, key.encode(), C.byref(n))
        return n.value

    def rows(self, name: str, row0: int = 0, nrows: int | None = None) -> np.ndarray:
        """Rows of a 2-D tensor dequantised to fp32 [nrows][dims[0]]."""
        _, dims, _ = self.tensor(name)
        total = 1
        for d in dims[1:]:
            total *= d
        if nrows is None:
            nrows = total - row0
        out = np.empty((nrows, dims[0]), np.float32)
        call("xp_gguf_dequantize_rows", self.h, name.encode(), row0, nrows, out.ctypes.data)
        return out

    def config(self, base: XpConfig | None = None) -> XpConfig:
        """The shapes of this file over `base` (default the Gemma-3-1B config)."""
        c = base if base is not None else XpConfig.gemma3_1b()
        call("xp_config_from_gguf", self.h, C.byref(c))
        return c

    def pack_model(self, cfg: XpConfig, cache: str, threads: int = 0) -> LoadStats:
        st = LoadStats()
        call("xp_gguf_pack_model", self.h, C.byref(cfg), cache.encode(), threads, C.byref(st))
        return st

    def verify_cache(self, cfg: XpConfig, cache: str, threads: int = 0) -> int:
        bad = C.c_uint32()
        call("xp_gguf_verify_cache", self.h, C.byref(cfg), cache.encode(), threads, C.byref(bad))
        return bad.value


def dequantize(ggml_type: int, raw: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    raw = np.ascontiguousarray(raw)
    call("xp_dequantize", ggml_type, raw.ctypes.data, out.ctypes.data, n)
    return out


def pack_int4(w_cols: np.ndarray, scale_fmt: int = XP_SCALE_BF16_QUAD, threads: int = 0):
    """Requantises w[cols][rows] (GGUF row order) to (KM4 plane, scale plane)."""
    w_cols = np.ascontiguousarray(w_cols, np.float32)
    cols, rows = w_cols.shape
    wq = np.empty(rows * cols // 8, np.uint32)
    sc = np.empty(rows // 32 * cols, np.uint16 if scale_fmt == XP_SCALE_BF16_QUAD else np.float32)
    call("xp_pack_int4", w_cols.ctypes.data, rows, cols, scale_fmt, threads, wq.ctypes.data,
         sc.ctypes.data)
    return wq, sc


def rq_layout(ggml_type: int, rows: int, cols: int) -> RqLayout:
    l = RqLayout()
    call("xp_rq_layout_of", ggml_type, rows, cols, C.byref(l))
    return l


def _ptr(a):
    return None if a is None else a.ctypes.data


def rq_repack(ggml_type: int, raw: np.ndarray, rows: int, cols: int, threads: int = 0) -> dict:
    """xp_rq_repack: host planes {layout, quant, high, scale, bias} (None
    where the type has no such plane) of rows x cols native blocks."""
    l = rq_layout(ggml_type, rows, cols)
    planes = {"layout": l,
              "quant": np.empty(l.quant_bytes // 4, np.uint32),
              "high": np.empty(l.high_bytes // 4, np.uint32) if l.high_bytes else None,
              "scale": np.empty(l.scale_bytes // 4, np.float32),
              "bias": np.empty(l.bias_bytes // 4, np.float32) if l.bias_bytes else None}
    raw = np.ascontiguousarray(raw)
    call("xp_rq_repack", C.byref(l), raw.ctypes.data, threads, _ptr(planes["quant"]),
         _ptr(planes["high"]), _ptr(planes["scale"]), _ptr(planes["bias"]))
    return planes


def rq_reconstruct(planes: dict) -> np.ndarray:
    """xp_rq_reconstruct: float32 [rows][cols]."""
    l = planes["layout"]
    out = np.empty((l.rows, l.cols), np.float32)
    call("xp_rq_reconstruct", C.byref(l), _ptr(planes["quant"]), _ptr(planes["high"]),
         _ptr(planes["scale"]), _ptr(planes["bias"]), out.ctypes.data)
    return out


class RqWeights:
    """A repacked matrix's planes in device memory; .tensor is the
    xp_rq_tensor that xp_mv_rq takes."""

    def __init__(self, planes: dict):
        l = planes["layout"]
        self.layout = l
        self.bufs = {k: DeviceBuffer.from_array(planes[k])
                     for k in ("quant", "high", "scale", "bias") if planes[k] is not None}
        t = RqTensor()
        t.type, t.rows, t.cols = l.type, l.rows, l.cols
        for k in ("quant", "high", "scale", "bias"):
            setattr(t, k, self.bufs[k].ptr if k in self.bufs else None)
        self.tensor = t

    def close(self) -> None:
        for b in self.bufs.values():
            b.close()
        self.bufs = {}


class Tokenizer:
    """The SentencePiece tokenizer of a GGUF file (xp_tokenizer_*). Keep the
    Gguf open while the tokenizer is in use."""

    def __init__(self, g: Gguf):
        h = C.c_void_p()
        call("xp_tokenizer_create", g.h, C.byref(h))
        self.h = h
        self.g = g
        i = TokenizerIds()
        call("xp_tokenizer_info", h, C.byref(i))
        self.ids = i

    def close(self) -> None:
        if self.h and self.h.value and _lib is not None:
            _lib.xp_tokenizer_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text: str | bytes, add_bos: bool = False, add_eos: bool = False) -> list[int]:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        n = C.c_size_t()
        call("xp_tokenize", self.h, raw, len(raw), int(add_bos), int(add_eos), None, 0, C.byref(n))
        out = (C.c_int32 * max(1, n.value))()
        call("xp_tokenize", self.h, raw, len(raw), int(add_bos), int(add_eos), out, n.value,
             C.byref(n))
        return list(out[:n.value])

    def decode(self, ids, skip_special: bool = True) -> bytes:
        a = (C.c_int32 * max(1, len(ids)))(*ids)
        n = C.c_size_t()
        call("xp_detokenize", self.h, a, len(ids), int(skip_special), None, 0, C.byref(n))
        buf = C.create_string_buffer(n.value + 1)
        call("xp_detokenize", self.h, a, len(ids), int(skip_special), buf, n.value + 1, C.byref(n))
        return buf.raw[:n.value]

    def piece(self, token: int) -> bytes:
        n = C.c_size_t()
        call("xp_token_piece", self.h, token, None, 0, C.byref(n))
        buf = C.create_string_buffer(n.value + 1)
        call("xp_token_piece", self.h, token, buf, n.value + 1, C.byref(n))
        return buf.raw[:n.value]

    def find(self, spelling: str | bytes) -> int:
        raw = spelling.encode() if isinstance(spelling, str) else bytes(spelling)
        i = C.c_int32()
        call("xp_token_find", self.h, raw, len(raw), C.byref(i))
        return i.value

    def kind(self, token: int) -> int:
        k, s = C.c_int32(), C.c_float()
        call("xp_token_kind", self.h, token, C.byref(k), C.byref(s))
        return k.value

