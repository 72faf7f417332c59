"""ctypes binding of libmarian_hip.so (include/marian_hip.h, include/marian_hip_util.h).

The library is loaded from this directory only; a missing library is an error,
never a reason to fall back to another implementation.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmarian_hip.so"

OK = 0
ERR_INVALID_INPUT = -1
ERR_MODEL = -2
ERR_INFERENCE = -3
ERR_DEVICE = -4
ERR_BUFFER = -5
ERR_NOT_READY = -6

FLAG_IGNORE_EOS = 1 << 0
FLAG_NO_GENERATION_MASK = 1 << 1
FLAG_FAST_REDUCTIONS = 1 << 2


class Linear(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("mult", C.c_void_p), ("bias", C.c_void_p)]


class EncoderLayer(C.Structure):
    _fields_ = [
        ("qkv", Linear), ("out", Linear),
        ("ln1_scale", C.c_void_p), ("ln1_bias", C.c_void_p),
        ("ffn1", Linear), ("ffn2", Linear),
        ("ln2_scale", C.c_void_p), ("ln2_bias", C.c_void_p),
    ]


class DecoderLayer(C.Structure):
    _fields_ = [
        ("self_qkv", Linear), ("self_out", Linear),
        ("ln1_scale", C.c_void_p), ("ln1_bias", C.c_void_p),
        ("cross_q", Linear), ("cross_kv", Linear), ("cross_out", Linear),
        ("ln2_scale", C.c_void_p), ("ln2_bias", C.c_void_p),
        ("ffn1", Linear), ("ffn2", Linear),
        ("ln3_scale", C.c_void_p), ("ln3_bias", C.c_void_p),
    ]


class Model(C.Structure):
    _fields_ = [
        ("vocab", C.c_uint32), ("dim", C.c_uint32), ("heads", C.c_uint32),
        ("ffn_dim", C.c_uint32), ("encoder_layers", C.c_uint32), ("decoder_layers", C.c_uint32),
        ("embedding", C.c_void_p), ("embedding_mult", C.c_void_p), ("output_bias", C.c_void_p),
        ("encoder", C.POINTER(EncoderLayer)), ("decoder", C.POINTER(DecoderLayer)),
    ]


class StaticLinear(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("weight_mult", C.c_float), ("act_mult", C.c_float),
                ("bias", C.c_void_p)]


class SsruEncoderLayer(C.Structure):
    _fields_ = [
        ("wq", StaticLinear), ("wk", StaticLinear), ("wv", StaticLinear), ("wo", StaticLinear),
        ("attn_ln_scale", C.c_void_p), ("attn_ln_bias", C.c_void_p),
        ("w1", StaticLinear), ("w2", StaticLinear),
        ("ffn_ln_scale", C.c_void_p), ("ffn_ln_bias", C.c_void_p),
    ]


class SsruDecoderLayer(C.Structure):
    _fields_ = [
        ("ssru_w", StaticLinear), ("ssru_wf", StaticLinear),
        ("ssru_ln_scale", C.c_void_p), ("ssru_ln_bias", C.c_void_p),
        ("wq", StaticLinear), ("wk", StaticLinear), ("wv", StaticLinear), ("wo", StaticLinear),
        ("context_ln_scale", C.c_void_p), ("context_ln_bias", C.c_void_p),
        ("w1", StaticLinear), ("w2", StaticLinear),
        ("ffn_ln_scale", C.c_void_p), ("ffn_ln_bias", C.c_void_p),
    ]


class SsruModel(C.Structure):
    _fields_ = [
        ("source_vocab", C.c_uint32), ("target_vocab", C.c_uint32), ("dim", C.c_uint32),
        ("heads", C.c_uint32), ("ffn_dim", C.c_uint32), ("encoder_layers", C.c_uint32),
        ("decoder_layers", C.c_uint32),
        ("encoder_embedding", C.c_void_p), ("encoder_embedding_mult", C.c_float),
        ("decoder_embedding", C.c_void_p), ("decoder_embedding_mult", C.c_float),
        ("output_act_mult", C.c_float), ("output_bias", C.c_void_p),
        ("encoder", C.POINTER(SsruEncoderLayer)), ("decoder", C.POINTER(SsruDecoderLayer)),
    ]


class Limits(C.Structure):
    _fields_ = [
        ("max_length_factor", C.c_uint32), ("max_generation_steps", C.c_uint32),
        ("max_position", C.c_uint32), ("max_batch", C.c_uint32),
        ("max_source_tokens", C.c_uint32), ("max_padded_cells", C.c_uint64),
    ]


class Stats(C.Structure):
    _fields_ = [
        ("total_ms", C.c_double), ("encoder_ms", C.c_double), ("decode_ms", C.c_double),
        ("vocab_kernel_ms", C.c_double), ("vocab_kernel_launches", C.c_uint32),
        ("decode_steps", C.c_uint32), ("max_active_rows", C.c_uint32),
        ("generated_tokens", C.c_uint64), ("launched_steps", C.c_uint32),
        ("allocations", C.c_uint32),
    ]


class Capacity(C.Structure):
    _fields_ = [
        ("sentences", C.c_uint32), ("source_tokens", C.c_uint32), ("output_tokens", C.c_uint32),
        ("steps", C.c_uint32), ("candidate_ids", C.c_uint32), ("max_candidates", C.c_uint32),
    ]


_P = C.c_void_p
_I64 = C.c_int64
_SZ = C.c_size_t

# name -> (restype, argtypes); every symbol declared in include/*.h.
SIGNATURES = {
    # marian_hip.h
    "marian_hip_engine_create": (C.c_int, [C.POINTER(Model), C.POINTER(Limits), C.c_int, C.POINTER(_P)]),
    "marian_hip_engine_destroy": (None, [_P]),
    "marian_hip_translate_token_ids": (C.c_int, [_P, _P, _SZ, _P, _SZ, _P, C.c_uint32, _P, _SZ, _P, C.POINTER(_SZ)]),
    "marian_hip_translate_probe": (C.c_int, [_P, _P, _SZ, _P, _SZ, _P, C.c_uint32, _P, _SZ, _P, C.POINTER(_SZ),
                                             C.c_uint32, _P, _P, _P]),
    "marian_hip_engine_create_ssru": (C.c_int, [C.POINTER(SsruModel), C.POINTER(Limits), C.c_int,
                                                 C.POINTER(_P)]),
    "marian_hip_translate_shortlisted": (C.c_int, [_P, _P, _SZ, _P, _SZ, _P, C.c_uint32, _P, _P, _P, _SZ,
                                                   _P, C.POINTER(_SZ)]),
    "marian_hip_warmup": (C.c_int, [_P]),
    "marian_hip_reserve": (C.c_int, [_P, C.POINTER(Capacity)]),
    "marian_hip_validate_batch": (C.c_int, [C.POINTER(Limits), C.c_uint32, C.c_uint32, _P, _SZ, _P, _SZ, _P, _P,
                                            C.c_char_p, _SZ]),
    "marian_hip_is_ready": (C.c_int, [_P]),
    "marian_hip_last_error": (C.c_char_p, [_P]),
    "marian_hip_info": (C.c_int, [_P, C.c_char_p, _SZ]),
    "marian_hip_last_stats": (C.c_int, [_P, C.POINTER(Stats)]),
    "marian_hip_set_timing": (C.c_int, [_P, C.c_uint32]),
    "marian_hip_last_step_trace": (C.c_int, [_P, _P, _P, _SZ, C.POINTER(_SZ)]),
    "marian_hip_last_kernel_trace": (C.c_int, [_P, _P, _P, _P, _P, _SZ, C.POINTER(_SZ)]),
    "marian_hip_quantize_rows": (C.c_int, [_P, _I64, _I64, _P, _P, _P, _P]),
    "marian_hip_q8_linear": (C.c_int, [_P, _P, _P, _I64, _I64, _P, _P, _P, _I64, C.c_int, _P, _P, _P, _P]),
    "marian_hip_q8_linear_static": (C.c_int, [_P, _I64, _I64, C.c_float, _P, _P, _P, _I64, C.c_int, _P, _P, _P, _P]),
    "marian_hip_ssru_layer_norm": (C.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P]),
    "marian_hip_residual_layer_norm": (C.c_int, [_P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P]),
    "marian_hip_attention": (C.c_int, [_P, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, C.c_int, _P, _I64, _P]),
    "marian_hip_vocab_argmax": (C.c_int, [_P, _P, _I64, _I64, _P, _P, _P, _I64, C.c_uint32, _P, _P, _P]),
    "marian_hip_candidate_argmax": (C.c_int, [_P, _P, _I64, _I64, _P, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _P]),
    "marian_hip_vocab_argmax_noalloc": (C.c_int, [_P, _P, _I64, _I64, _P, _P, _P, _I64, C.c_uint32, _P, _P, _P]),
    "marian_hip_positions": (C.c_int, [C.c_uint32, C.c_uint32, _P]),
    # marian_hip_util.h
    "marian_hip_device_count": (C.c_int, []),
    "marian_hip_device_name": (C.c_int, [C.c_int, C.c_char_p, _SZ]),
    "marian_hip_set_device": (C.c_int, [C.c_int]),
    "marian_hip_device_alloc": (_P, [_SZ]),
    "marian_hip_device_free": (C.c_int, [_P]),
    "marian_hip_memcpy_h2d": (C.c_int, [_P, _P, _SZ]),
    "marian_hip_memcpy_d2h": (C.c_int, [_P, _P, _SZ]),
    "marian_hip_memcpy_d2d": (C.c_int, [_P, _P, _SZ]),
    "marian_hip_memset": (C.c_int, [_P, C.c_int, _SZ]),
    "marian_hip_stream_create": (_P, []),
    "marian_hip_stream_destroy": (C.c_int, [_P]),
    "marian_hip_stream_sync": (C.c_int, [_P]),
    "marian_hip_device_sync": (C.c_int, []),
    "marian_hip_event_create": (_P, []),
    "marian_hip_event_destroy": (C.c_int, [_P]),
    "marian_hip_event_record": (C.c_int, [_P, _P]),
    "marian_hip_event_sync": (C.c_int, [_P]),
    "marian_hip_event_elapsed": (C.c_int, [_P, _P, C.POINTER(C.c_float)]),
    "marian_hip_last_op_error": (C.c_char_p, []),
    "marian_hip_build_id": (C.c_char_p, []),
}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def load() -> C.CDLL:
    """Loads the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LibraryMissing(
            f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
            "(the marian-hip backend has no other implementation to fall back on)"
        )
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def build_id() -> str:
    """Source hash the loaded library was built from."""
    return load().marian_hip_build_id().decode()


def op_error() -> str:
    return load().marian_hip_last_op_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise RuntimeError(f"{what} failed ({rc}): {op_error()}")
