"""ctypes binding of libmimizuku_amd.so (the C ABI declared in include/mimizuku.h).

The library is the only compute path: if it is missing this module raises, it never falls back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmimizuku_amd.so")

u64, i32, i64, f32, sz = C.c_uint64, C.c_int, C.c_long, C.c_float, C.c_size_t
P = C.c_void_p


class MzError(RuntimeError):
    """A nonzero status from the library, with its mz_last_error() message."""


class Dims(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("d", "ff", "nh", "enc_layers", "dec_layers", "n_mels", "vocab", "max_t")]


class GenCfgC(C.Structure):
    _fields_ = [("sot", C.c_int), ("eos", C.c_int), ("no_timestamps", C.c_int),
                ("suppress", C.POINTER(C.c_int32)), ("n_suppress", C.c_int),
                ("begin_suppress", C.POINTER(C.c_int32)), ("n_begin_suppress", C.c_int),
                ("lang_tokens", C.POINTER(C.c_int32)), ("n_langs", C.c_int),
                ("align_heads", C.POINTER(C.c_int32)), ("n_align", C.c_int)]


class LinearArgs(C.Structure):
    _fields_ = [("epilogue", C.c_int), ("a", u64), ("lda", C.c_long), ("w", u64), ("bias", u64),
                ("m", C.c_int), ("n", C.c_int), ("k", C.c_int), ("out", u64), ("ldo", C.c_long), ("pos", u64),
                ("heads", u64), ("blocks_per_clip", C.c_int), ("nh", C.c_int), ("kind", C.c_int), ("slot0", C.c_int),
                ("conv_cin", C.c_int), ("conv_tin", C.c_int), ("conv_tout", C.c_int), ("conv_stride", C.c_int)]


class Times(C.Structure):
    _fields_ = [("enc", C.c_double), ("dec", C.c_double), ("post", C.c_double), ("steps", C.c_int)]


EPI_F16, EPI_GELU_F16, EPI_RESID_F32, EPI_GELU_POS, EPI_HEADS = range(5)
(BUF_TOK, BUF_DONE, BUF_CTR, BUF_ALIGN, BUF_ENC_OUT, BUF_LOGITS, BUF_TRACE, BUF_XKV, BUF_DEC_X, BUF_ENC_X,
 BUF_DEC_TRACE, BUF_SELF_K, BUF_SELF_V, BUF_ALIGN_H) = range(14)
DT_F16, DT_F32 = 0, 1
# kernel classes of mz_engine_profile_read
K_NAMES = ["mel", "conv1", "conv2", "ln", "qkv", "attn", "oproj", "fc1", "fc2", "xkv", "step",
           "dec_embed", "dec_qkv", "dec_self", "dec_oproj", "dec_addln", "dec_cross", "dec_xo", "dec_fc1", "dec_fc2",
           "dec_lm", "dec_argmax"]

# name -> (restype, argtypes); every int-returning function is a status
SIGNATURES = {
    "mz_last_error": (C.c_char_p, []),
    "mz_version": (C.c_char_p, []),
    "mz_init": (i32, [i32, C.POINTER(P)]),
    "mz_ctx_free": (i32, [P]),
    "mz_alloc": (i32, [P, sz, C.POINTER(u64)]),
    "mz_free": (i32, [P, u64]),
    "mz_mem_info": (i32, [P, C.POINTER(sz), C.POINTER(sz)]),
    "mz_upload": (i32, [P, u64, P, sz]),
    "mz_download": (i32, [P, P, u64, sz]),
    "mz_copy": (i32, [P, u64, u64, sz]),
    "mz_sync": (i32, [P]),
    "mz_event_create": (i32, [P, C.POINTER(u64)]),
    "mz_event_record": (i32, [P, u64]),
    "mz_event_elapsed_ms": (i32, [u64, u64, C.POINTER(f32)]),
    "mz_event_destroy": (i32, [u64]),
    "mz_graph_begin": (i32, [P]),
    "mz_graph_end": (i32, [P, C.POINTER(P)]),
    "mz_graph_launch": (i32, [P, P]),
    "mz_graph_free": (i32, [P]),
    "mz_gemm": (i32, [P, u64, i32, u64, u64, i32, i32, i32, i32, u64]),
    "mz_linear": (i32, [P, C.POINTER(LinearArgs)]),
    "mz_layernorm": (i32, [P, u64, i64, u64, u64, u64, i64, i32, i32, f32]),
    "mz_add_layernorm": (i32, [P, u64, u64, u64, u64, u64, i32, i32, f32]),
    "mz_enc_attention": (i32, [P, u64, u64, i32, i32]),
    "mz_mel_transpose": (i32, [P, u64, u64, i32, i32]),
    "mz_scratch_bytes": (sz, [C.POINTER(Dims), i32, i32, i32]),
    "mz_engine_new": (i32, [P, C.POINTER(Dims), C.POINTER(GenCfgC), i32, i32, C.POINTER(P)]),
    "mz_engine_put": (i32, [P, C.c_char_p, i32, P, C.POINTER(C.c_int64), i32]),
    "mz_engine_finish": (i32, [P]),
    "mz_engine_load": (i32, [P, C.c_char_p]),
    "mz_engine_open": (i32, [P, C.c_char_p, i32, i32, C.POINTER(P)]),
    "mz_st_open": (i32, [C.c_char_p, C.POINTER(P)]),
    "mz_st_count": (i32, [P, C.POINTER(i32)]),
    "mz_st_info": (i32, [P, i32, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.POINTER(i32),
                         C.POINTER(C.POINTER(C.c_int64)), C.POINTER(P), C.POINTER(u64)]),
    "mz_st_find": (i32, [P, C.c_char_p, C.POINTER(i32)]),
    "mz_st_meta": (i32, [P, C.c_char_p, C.POINTER(C.c_char_p)]),
    "mz_st_close": (i32, [P]),
    "mz_json_check": (i32, [C.c_char_p, sz]),
    "mz_model_open": (i32, [C.c_char_p, C.POINTER(P)]),
    "mz_model_dims": (i32, [P, C.POINTER(Dims)]),
    "mz_model_gencfg": (i32, [P, C.POINTER(GenCfgC)]),
    "mz_model_lang": (i32, [P, i32, C.POINTER(C.c_char_p), C.POINTER(C.c_int32)]),
    "mz_model_task": (i32, [P, i32, C.POINTER(C.c_char_p), C.POINTER(C.c_int32)]),
    "mz_model_free": (i32, [P]),
    "mz_engine_encode": (i32, [P, P, i32, i32]),
    "mz_engine_encode_device": (i32, [P, u64, i32, i32]),
    "mz_engine_profile": (i32, [P, i32]),
    "mz_engine_profile_read": (i32, [P, i32, C.POINTER(C.c_double), C.POINTER(i32)]),
    "mz_engine_reset": (i32, [P, P, i32, i32]),
    "mz_engine_detect": (i32, [P, i32, P]),
    "mz_engine_step": (i32, [P, i32, i32, i32]),
    "mz_engine_capture": (i32, [P, i32, i32]),
    "mz_engine_replay": (i32, [P]),
    "mz_engine_set_trace": (i32, [P, i32]),
    "mz_engine_buffer": (i32, [P, i32, C.POINTER(u64), C.POINTER(sz)]),
    "mz_engine_read": (i32, [P, i32, P, sz, sz]),
    "mz_engine_free": (i32, [P]),
    "mz_transcribe": (i32, [P, P, P, i32, P, i32, i32, i32, i32, i32, P, P, P, P, C.POINTER(Times)]),
    "mz_transcribe_device": (i32, [P, u64, P, i32, P, i32, i32, i32, i32, i32, P, P, P, P, C.POINTER(Times)]),
    "mz_transcribe_submit": (i32, [P, P, i32]),
    "mz_transcribe_submit_device": (i32, [P, u64, i32]),
    "mz_transcribe_collect": (i32, [P, P, i32, P, i32, i32, i32, i32, i32, P, P, P, P, C.POINTER(Times)]),
    "mz_wav_read": (i32, [C.c_char_p, P, sz, C.POINTER(sz), C.POINTER(i32)]),
    "mz_resample_16k": (i32, [P, sz, i32, P, sz, C.POINTER(sz)]),
    "mz_mel_tables": (i32, [i32, P, P, P]),
    "mz_log_mel": (i32, [P, u64, P, i32, i32, u64, P]),
    "mz_tok_open": (i32, [C.c_char_p, i32, i32, C.POINTER(P)]),
    "mz_tok_from_bytes": (i32, [P, P, i32, C.POINTER(P)]),
    "mz_tok_free": (i32, [P]),
    "mz_tok_decode": (i32, [P, P, i32, P, sz, C.POINTER(sz)]),
    "mz_tok_pieces": (i32, [P, P, P, i32, i32, P, sz, C.POINTER(sz), P, P, P, C.POINTER(i32)]),
    "mz_json_time": (i32, [f32, P, sz, C.POINTER(sz)]),
    "mz_results_json": (i32, [P, P, i32, P, P, P, i32, P, P, P, sz, C.POINTER(sz)]),
    "mz_cli": (i32, [i32, P]),
    "mz_jump_times": (i32, [P, i32, i32, i32, i32, i32, i32, P]),
    "mz_align_cost": (i32, [P, i32, i32, i32, i32, i32, i32, P]),
    "mz_jump_times_device": (i32, [P, u64, C.c_int64, i32, P, P, i32, i32, i32, i32, P, C.c_int64]),
    "mz_jump_times_device_noalloc": (i32, [P, u64, C.c_int64, i32, P, P, i32, i32, i32, i32, P, C.c_int64]),
    "mz_dtw": (i32, [P, i32, i32, P, P, P]),
    "mz_f2h": (C.c_uint16, [f32]),
    "mz_h2f": (f32, [C.c_uint16]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library (raises MzError with a build hint if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MzError(f"{LIB_PATH} is not built: run `python -m mimizuku_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise MzError(lib().mz_last_error().decode(errors="replace"))


def ptr(a) -> C.c_void_p:
    """Host pointer of a C-contiguous numpy array."""
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return C.c_void_p(a.ctypes.data)
