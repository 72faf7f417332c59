"""ctypes wrapper of liboracle.so — the CPU restatement of marian-cpu's Q8 path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker and the timed CPU baseline.  The
product never imports it.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

# Reduction orders (oracle.h).  REFERENCE, the reference's own order, is the
# default and the one the HIP kernels reproduce; CANONICAL is kept to measure
# how sensitive greedy outputs are to the fp32 summation order; FAST_DECODER is
# the order of the engine's opt-in fast-reduction flag (encoder as REFERENCE,
# the decoder's LayerNorm and softmax sums as lane partials + butterfly).
CANONICAL = 0
REFERENCE = 1
FAST_DECODER = 2
FLAG_IGNORE_EOS = 1
FLAG_NO_GENERATION_MASK = 2


def build() -> Path:
    res = subprocess.run(["make", "-C", str(HERE)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


class Linear(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("mult", C.c_void_p), ("bias", C.c_void_p)]


class EncoderLayer(C.Structure):
    _fields_ = [("qkv", Linear), ("out", Linear), ("ln1_scale", C.c_void_p),
                ("ln1_bias", C.c_void_p), ("ffn1", Linear), ("ffn2", Linear),
                ("ln2_scale", C.c_void_p), ("ln2_bias", C.c_void_p)]


class DecoderLayer(C.Structure):
    _fields_ = [("self_qkv", Linear), ("self_out", Linear), ("ln1_scale", C.c_void_p),
                ("ln1_bias", C.c_void_p), ("cross_q", Linear), ("cross_kv", Linear),
                ("cross_out", Linear), ("ln2_scale", C.c_void_p), ("ln2_bias", C.c_void_p),
                ("ffn1", Linear), ("ffn2", Linear), ("ln3_scale", C.c_void_p),
                ("ln3_bias", C.c_void_p)]


class Model(C.Structure):
    _fields_ = [("vocab", C.c_uint32), ("dim", C.c_uint32), ("heads", C.c_uint32),
                ("ffn_dim", C.c_uint32), ("encoder_layers", C.c_uint32),
                ("decoder_layers", C.c_uint32), ("embedding", C.c_void_p),
                ("embedding_mult", C.c_void_p), ("output_bias", C.c_void_p),
                ("encoder", C.POINTER(EncoderLayer)), ("decoder", C.POINTER(DecoderLayer))]


class StaticLinear(C.Structure):
    _fields_ = [("weight", C.c_void_p), ("weight_mult", C.c_float), ("act_mult", C.c_float),
                ("bias", C.c_void_p)]


class SsruEncoderLayer(C.Structure):
    _fields_ = [("wq", StaticLinear), ("wk", StaticLinear), ("wv", StaticLinear),
                ("wo", StaticLinear), ("attn_ln_scale", C.c_void_p), ("attn_ln_bias", C.c_void_p),
                ("w1", StaticLinear), ("w2", StaticLinear), ("ffn_ln_scale", C.c_void_p),
                ("ffn_ln_bias", C.c_void_p)]


class SsruDecoderLayer(C.Structure):
    _fields_ = [("ssru_w", StaticLinear), ("ssru_wf", StaticLinear),
                ("ssru_ln_scale", C.c_void_p), ("ssru_ln_bias", C.c_void_p),
                ("wq", StaticLinear), ("wk", StaticLinear), ("wv", StaticLinear),
                ("wo", StaticLinear), ("context_ln_scale", C.c_void_p),
                ("context_ln_bias", C.c_void_p), ("w1", StaticLinear), ("w2", StaticLinear),
                ("ffn_ln_scale", C.c_void_p), ("ffn_ln_bias", C.c_void_p)]


class SsruModelStruct(C.Structure):
    _fields_ = [("source_vocab", C.c_uint32), ("target_vocab", C.c_uint32), ("dim", C.c_uint32),
                ("heads", C.c_uint32), ("ffn_dim", C.c_uint32), ("encoder_layers", C.c_uint32),
                ("decoder_layers", C.c_uint32), ("encoder_embedding", C.c_void_p),
                ("encoder_embedding_mult", C.c_float), ("decoder_embedding", C.c_void_p),
                ("decoder_embedding_mult", C.c_float), ("output_act_mult", C.c_float),
                ("output_bias", C.c_void_p), ("encoder", C.POINTER(SsruEncoderLayer)),
                ("decoder", C.POINTER(SsruDecoderLayer))]


class Limits(C.Structure):
    _fields_ = [("max_length_factor", C.c_uint32), ("max_generation_steps", C.c_uint32),
                ("max_position", C.c_uint32), ("max_batch", C.c_uint32),
                ("max_source_tokens", C.c_uint32), ("max_padded_cells", C.c_uint64)]


_P, _SZ = C.c_void_p, C.c_size_t
_SIG = {
    "oracle_build_info": (C.c_char_p, []),
    "oracle_expf": (C.c_float, [C.c_float, C.c_int]),
    "oracle_row_sum": (C.c_float, [_P, _SZ, C.c_int]),
    "oracle_positions": (C.c_int, [C.c_uint32, C.c_uint32, _P]),
    "oracle_quantize_rows": (C.c_int, [_P, _SZ, _SZ, _P, _P]),
    "oracle_quantize_static_u8": (C.c_int, [_P, _SZ, C.c_float, _P]),
    "oracle_gemm_i32": (C.c_int, [_P, _SZ, _SZ, _P, _SZ, _P, C.c_int]),
    "oracle_gemm_u8_i8_avx2": (C.c_int, [_P, _SZ, _SZ, _P, _SZ, C.c_uint8, _P, C.c_int]),
    "oracle_dot_u8_i8": (C.c_int32, [_P, _P, _SZ]),
    "oracle_linear_forward": (C.c_int, [_P, _SZ, _SZ, C.POINTER(Linear), _SZ, C.c_int, _P, _P,
                                        _P, _P, C.c_int]),
    "oracle_residual_layer_norm": (C.c_int, [_P, _P, _P, _P, _SZ, _SZ, C.c_int, _P]),
    "oracle_linear_forward_static": (C.c_int, [_P, _SZ, _SZ, C.POINTER(Linear), _SZ, C.c_float,
                                               C.c_int, _P, _P, _P, C.c_int]),
    "oracle_candidate_argmax": (C.c_int, [_P, _P, _SZ, _SZ, _P, _P, _P, _SZ, _P, _P, _P, _P]),
    "oracle_ssru_layer_norm": (C.c_int, [_P, _P, _P, _P, _P, _P, _SZ, _SZ, C.c_int, _P]),
    "oracle_attention": (C.c_int, [_P, _SZ, _P, _SZ, _P, _SZ, _P, _P, _SZ, _SZ, _SZ, C.c_int, _P,
                                   _SZ]),
    "oracle_translate": (C.c_int, [C.POINTER(Model), _P, _SZ, _P, _SZ, _P, C.POINTER(Limits),
                                   C.c_uint32, C.c_int, C.c_int, _P, _SZ, _P, C.POINTER(_SZ),
                                   C.c_char_p, _SZ]),
    "oracle_translate_reference_schedule": (C.c_int, [C.POINTER(Model), _P, _SZ, _P, _SZ, _P,
                                                      C.POINTER(Limits), C.c_uint32, C.c_int,
                                                      C.c_int, _P, _SZ, _P, C.POINTER(_SZ),
                                                      C.c_char_p, _SZ]),
    "oracle_translate_probe": (C.c_int, [C.POINTER(Model), _P, _SZ, _P, _SZ, _P, C.POINTER(Limits),
                                         C.c_uint32, C.c_int, C.c_int, _P, _SZ, _P, C.POINTER(_SZ),
                                         C.c_char_p, _SZ, C.c_uint32, _P, _P, _P]),
    "oracle_encode": (C.c_int, [C.POINTER(Model), _P, _SZ, _P, _SZ, C.c_int, C.c_int, _P]),
    "oracle_translate_shortlisted": (C.c_int, [C.POINTER(Model), _P, _SZ, _P, _SZ, _P,
                                               C.POINTER(Limits), C.c_uint32, C.c_int, C.c_int, _P,
                                               _P, _P, _SZ, _P, C.POINTER(_SZ), C.c_char_p, _SZ]),
    "oracle_translate_ssru": (C.c_int, [C.POINTER(SsruModelStruct), _P, _SZ, _P, _SZ, _P,
                                        C.POINTER(Limits), C.c_uint32, C.c_int, C.c_int, _P, _P,
                                        _P, _SZ, _P, C.POINTER(_SZ), C.c_char_p, _SZ, C.c_uint32,
                                        _P, _P, _P]),
    "oracle_translate_ssru_reference_schedule": (C.c_int, [C.POINTER(SsruModelStruct), _P, _SZ, _P, _SZ,
                                                           _P, C.POINTER(Limits), C.c_uint32, C.c_int,
                                                           C.c_int, _P, _P, _P, _SZ, _P, C.POINTER(_SZ),
                                                           C.c_char_p, _SZ]),
    "oracle_last_step_logits": (C.c_int, [C.POINTER(Model), _P, _SZ, C.c_uint32, C.c_uint32,
                                          C.c_int, _P]),
}

_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


class OracleModel:
    """ctypes view of a seeded model (any object with the SeededModel fields)."""

    def __init__(self, m):
        keep = []

        def arr(a, dtype):
            a = np.ascontiguousarray(a, dtype=dtype)
            keep.append(a)
            return a.ctypes.data

        def lin(d):
            return Linear(arr(d["weight"], np.int8), arr(d["mult"], np.float32),
                          arr(d["bias"], np.float32))

        g = m.geometry
        enc = (EncoderLayer * max(1, len(m.encoder)))()
        for i, L in enumerate(m.encoder):
            enc[i] = EncoderLayer(lin(L["qkv"]), lin(L["out"]), arr(L["ln1"]["scale"], np.float32),
                                  arr(L["ln1"]["bias"], np.float32), lin(L["ffn1"]), lin(L["ffn2"]),
                                  arr(L["ln2"]["scale"], np.float32),
                                  arr(L["ln2"]["bias"], np.float32))
        dec = (DecoderLayer * max(1, len(m.decoder)))()
        for i, L in enumerate(m.decoder):
            dec[i] = DecoderLayer(
                lin(L["self_qkv"]), lin(L["self_out"]), arr(L["ln1"]["scale"], np.float32),
                arr(L["ln1"]["bias"], np.float32), lin(L["cross_q"]), lin(L["cross_kv"]),
                lin(L["cross_out"]), arr(L["ln2"]["scale"], np.float32),
                arr(L["ln2"]["bias"], np.float32), lin(L["ffn1"]), lin(L["ffn2"]),
                arr(L["ln3"]["scale"], np.float32), arr(L["ln3"]["bias"], np.float32))
        self.struct = Model(g.vocab, g.dim, g.heads, g.ffn_dim, len(m.encoder), len(m.decoder),
                            arr(m.embedding, np.int8), arr(m.embedding_mult, np.float32),
                            arr(m.output_bias, np.float32), enc, dec)
        self.geometry = g
        self._keep = (keep, enc, dec)


class OracleSsruModel:
    """ctypes view of a Transformer-SSRU model (the SsruModel fields)."""

    def __init__(self, m):
        keep = []

        def arr(a, dtype):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dtype)
            keep.append(a)
            return a.ctypes.data

        def lin(d):
            return StaticLinear(arr(d["weight"], np.int8), d["weight_mult"], d["act_mult"],
                                arr(d["bias"], np.float32))

        def ln(d):
            return arr(d["scale"], np.float32), arr(d["bias"], np.float32)

        g = m.geometry
        enc = (SsruEncoderLayer * max(1, len(m.encoder)))()
        for i, L in enumerate(m.encoder):
            enc[i] = SsruEncoderLayer(lin(L["wq"]), lin(L["wk"]), lin(L["wv"]), lin(L["wo"]),
                                      *ln(L["attn_ln"]), lin(L["w1"]), lin(L["w2"]),
                                      *ln(L["ffn_ln"]))
        dec = (SsruDecoderLayer * max(1, len(m.decoder)))()
        for i, L in enumerate(m.decoder):
            dec[i] = SsruDecoderLayer(lin(L["ssru_w"]), lin(L["ssru_wf"]), *ln(L["ssru_ln"]),
                                      lin(L["wq"]), lin(L["wk"]), lin(L["wv"]), lin(L["wo"]),
                                      *ln(L["context_ln"]), lin(L["w1"]), lin(L["w2"]),
                                      *ln(L["ffn_ln"]))
        self.struct = SsruModelStruct(
            g.source_vocab, g.target_vocab, g.dim, g.heads, g.ffn_dim, len(m.encoder),
            len(m.decoder), arr(m.encoder_embedding, np.int8), m.encoder_embedding_mult,
            arr(m.decoder_embedding, np.int8), m.decoder_embedding_mult, m.output_act_mult,
            arr(m.output_bias, np.float32), enc, dec)
        self.geometry = g
        self._keep = (keep, enc, dec)


def translate_ssru(model: OracleSsruModel, tokens, offsets, max_output_tokens, limits: dict,
                   flags=0, candidates=None, candidate_offsets=None, probe_step=None,
                   order=REFERENCE, threads=8, schedule="ragged"):
    """Greedy translation over the Transformer-SSRU graph.  Returns the token
    lists; with probe_step also the encoder states [T, d], the logits [B, Vt]
    of that step (ids not scored are -inf) and the rows that reached it.
    schedule="reference" runs the reference x86 engine's schedule instead (a
    padded batch, every row decoded every step, `threads` splitting the
    GEMMs' rows; the timed CPU baseline; no probe): the same tokens."""
    lib = load()
    toks = np.ascontiguousarray(tokens, np.int32)
    offs = np.ascontiguousarray(offsets, np.uint32)
    req = np.ascontiguousarray(max_output_tokens, np.uint32)
    B = offs.size - 1
    g = model.geometry
    cap = int(np.minimum(req.astype(np.int64), 4096).sum()) + 1
    out = np.zeros(cap, np.int32)
    out_offs = np.zeros(offs.size, np.uint32)
    n = C.c_size_t(0)
    err = C.create_string_buffer(512)
    lim = make_limits(limits)
    cand = None if candidates is None else np.ascontiguousarray(candidates, np.uint32)
    coff = None if candidate_offsets is None else np.ascontiguousarray(candidate_offsets, np.uint32)
    enc = logits = active = None
    if schedule != "ragged":
        if schedule != "reference" or probe_step is not None:
            raise ValueError("schedule is 'ragged' or 'reference' (the latter without a probe)")
        rc = lib.oracle_translate_ssru_reference_schedule(
            C.byref(model.struct), _ptr(toks) if toks.size else None, toks.size, _ptr(offs), offs.size,
            _ptr(req), C.byref(lim), flags, order, threads, _ptr(cand), _ptr(coff), _ptr(out), cap,
            _ptr(out_offs), C.byref(n), err, 512)
        if rc != 0:
            raise OracleError(rc, err.value.decode())
        return [out[out_offs[i]:out_offs[i + 1]].tolist() for i in range(B)]
    if probe_step is not None:
        enc = np.zeros((max(toks.size, 1), g.dim), np.float32)
        logits = np.zeros((max(B, 1), g.target_vocab), np.float32)
        active = np.zeros(max(B, 1), np.uint8)
    rc = lib.oracle_translate_ssru(
        C.byref(model.struct), _ptr(toks) if toks.size else None, toks.size, _ptr(offs), offs.size,
        _ptr(req), C.byref(lim), flags, order, threads, _ptr(cand), _ptr(coff), _ptr(out), cap,
        _ptr(out_offs), C.byref(n), err, 512,
        0xFFFFFFFF if probe_step is None else int(probe_step), _ptr(enc), _ptr(logits),
        _ptr(active))
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    rows = [out[out_offs[i]:out_offs[i + 1]].tolist() for i in range(B)]
    if probe_step is None:
        return rows
    return rows, enc[:toks.size], logits[:B], active[:B].astype(bool)


def make_limits(d: dict) -> Limits:
    return Limits(d["max_length_factor"], d["max_generation_steps"], d["max_position"],
                  d["max_batch"], d["max_source_tokens"], d["max_padded_cells"])


class OracleError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"oracle error {code}: {msg}")
        self.code = code


def translate(model: OracleModel, tokens, offsets, max_output_tokens, limits: dict, flags=0,
              order=REFERENCE, threads=8, schedule="ragged"):
    """Returns a list of token lists, one per row."""
    lib = load()
    toks = np.ascontiguousarray(tokens, np.int32)
    offs = np.ascontiguousarray(offsets, np.uint32)
    req = np.ascontiguousarray(max_output_tokens, np.uint32)
    cap = int(np.minimum(req.astype(np.int64), 4096).sum()) + 1
    out = np.zeros(cap, np.int32)
    out_offs = np.zeros(offs.size, np.uint32)
    n = C.c_size_t(0)
    err = C.create_string_buffer(512)
    lim = make_limits(limits)
    fn = lib.oracle_translate if schedule == "ragged" else lib.oracle_translate_reference_schedule
    rc = fn(C.byref(model.struct), _ptr(toks) if toks.size else None, toks.size, _ptr(offs),
            offs.size, _ptr(req), C.byref(lim), flags, order, threads, _ptr(out), cap,
            _ptr(out_offs), C.byref(n), err, 512)
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    return [out[out_offs[i]:out_offs[i + 1]].tolist() for i in range(offs.size - 1)]


def translate_shortlisted(model: OracleModel, tokens, offsets, max_output_tokens, limits: dict,
                          candidates, candidate_offsets, flags=0, order=REFERENCE, threads=8):
    """translate() with each sentence scored over its candidate list."""
    lib = load()
    toks = np.ascontiguousarray(tokens, np.int32)
    offs = np.ascontiguousarray(offsets, np.uint32)
    req = np.ascontiguousarray(max_output_tokens, np.uint32)
    cand = np.ascontiguousarray(candidates, np.uint32)
    coff = np.ascontiguousarray(candidate_offsets, np.uint32)
    cap = int(np.minimum(req.astype(np.int64), 4096).sum()) + 1
    out = np.zeros(cap, np.int32)
    out_offs = np.zeros(offs.size, np.uint32)
    n = C.c_size_t(0)
    err = C.create_string_buffer(512)
    lim = make_limits(limits)
    rc = lib.oracle_translate_shortlisted(
        C.byref(model.struct), _ptr(toks) if toks.size else None, toks.size, _ptr(offs), offs.size,
        _ptr(req), C.byref(lim), flags, order, threads, _ptr(cand), _ptr(coff), _ptr(out), cap,
        _ptr(out_offs), C.byref(n), err, 512)
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    return [out[out_offs[i]:out_offs[i + 1]].tolist() for i in range(offs.size - 1)]


def translate_probe(model: OracleModel, tokens, offsets, max_output_tokens, limits: dict,
                    flags=0, probe_step=0, order=REFERENCE, threads=8):
    """translate() plus the final encoder states [T, d] and, for decode step
    probe_step, the logits [B, V] of the rows that reach it (active[b] = 1)."""
    lib = load()
    toks = np.ascontiguousarray(tokens, np.int32)
    offs = np.ascontiguousarray(offsets, np.uint32)
    req = np.ascontiguousarray(max_output_tokens, np.uint32)
    B = offs.size - 1
    g = model.geometry
    cap = int(np.minimum(req.astype(np.int64), 4096).sum()) + 1
    out = np.zeros(cap, np.int32)
    out_offs = np.zeros(offs.size, np.uint32)
    n = C.c_size_t(0)
    err = C.create_string_buffer(512)
    lim = make_limits(limits)
    enc = np.zeros((max(toks.size, 1), g.dim), np.float32)
    logits = np.zeros((max(B, 1), g.vocab), np.float32)
    active = np.zeros(max(B, 1), np.uint8)
    rc = lib.oracle_translate_probe(
        C.byref(model.struct), _ptr(toks) if toks.size else None, toks.size, _ptr(offs), offs.size,
        _ptr(req), C.byref(lim), flags, order, threads, _ptr(out), cap, _ptr(out_offs), C.byref(n),
        err, 512, probe_step, _ptr(enc), _ptr(logits), _ptr(active))
    if rc != 0:
        raise OracleError(rc, err.value.decode())
    rows = [out[out_offs[i]:out_offs[i + 1]].tolist() for i in range(B)]
    return rows, enc[:toks.size], logits[:B], active[:B].astype(bool)


def build_info() -> str:
    return load().oracle_build_info().decode()


def expf(x: float, order=REFERENCE) -> float:
    return load().oracle_expf(x, order)


def row_sum(x: np.ndarray, order=REFERENCE) -> float:
    x = np.ascontiguousarray(x, np.float32)
    return load().oracle_row_sum(_ptr(x), x.size, order)


def positions(dim: int, count: int) -> np.ndarray:
    out = np.zeros((count, dim), np.float32)
    if load().oracle_positions(dim, count, _ptr(out)) != 0:
        raise OracleError(-1, "invalid positions dimension")
    return out


def quantize_rows(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    q = np.zeros((rows, cols), np.int8)
    a = np.zeros(rows, np.float32)
    rc = load().oracle_quantize_rows(_ptr(x), rows, cols, _ptr(q), _ptr(a))
    if rc != 0:
        raise OracleError(rc, "non-finite activation")
    return q, a


def quantize_static_u8(x: np.ndarray, mult: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size, np.uint8)
    rc = load().oracle_quantize_static_u8(_ptr(x), x.size, mult, _ptr(out))
    if rc != 0:
        raise OracleError(rc, "invalid quantization input")
    return out


def gemm_i32(qa: np.ndarray, qw: np.ndarray, threads=8) -> np.ndarray:
    qa = np.ascontiguousarray(qa, np.int8)
    qw = np.ascontiguousarray(qw, np.int8)
    M, K = qa.shape
    N = qw.shape[0]
    acc = np.zeros((M, N), np.int32)
    rc = load().oracle_gemm_i32(_ptr(qa), M, K, _ptr(qw), N, _ptr(acc), threads)
    if rc != 0:
        raise OracleError(rc, "accumulator overflow")
    return acc


def gemm_u8_i8_avx2(a: np.ndarray, w: np.ndarray, zero_point=127, threads=1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.uint8)
    w = np.ascontiguousarray(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    acc = np.zeros((M, N), np.int32)
    rc = load().oracle_gemm_u8_i8_avx2(_ptr(a), M, K, _ptr(w), N, zero_point, _ptr(acc), threads)
    if rc != 0:
        raise OracleError(rc, "AVX2 unavailable or accumulator overflow")
    return acc


def dot_u8_i8(a: np.ndarray, w: np.ndarray) -> int:
    a = np.ascontiguousarray(a, np.uint8)
    w = np.ascontiguousarray(w, np.int8)
    return int(load().oracle_dot_u8_i8(_ptr(a), _ptr(w), a.size))


def linear_forward(x: np.ndarray, weight, mult, bias, relu=False, threads=8):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(weight, np.int8)
    mult = np.ascontiguousarray(mult, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    M, K = x.shape
    N = w.shape[0]
    y = np.zeros((M, N), np.float32)
    acc = np.zeros((M, N), np.int32)
    q = np.zeros((M, K), np.int8)
    a = np.zeros(M, np.float32)
    lin = Linear(_ptr(w), _ptr(mult), _ptr(bias))
    rc = load().oracle_linear_forward(_ptr(x), M, K, C.byref(lin), N, int(relu), _ptr(y), _ptr(acc),
                                      _ptr(q), _ptr(a), threads)
    if rc != 0:
        raise OracleError(rc, "non-finite activation or accumulator overflow")
    return y, acc, q, a


def linear_forward_static(x: np.ndarray, weight, mult, bias, act_mult: float, relu=False,
                          threads=8):
    """Q8 linear with one static activation multiplier: (y, acc, q)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(weight, np.int8)
    mult = np.ascontiguousarray(mult, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    M, K = x.shape
    N = w.shape[0]
    y = np.zeros((M, N), np.float32)
    acc = np.zeros((M, N), np.int32)
    q = np.zeros((M, K), np.int8)
    lin = Linear(_ptr(w), _ptr(mult), _ptr(bias))
    rc = load().oracle_linear_forward_static(_ptr(x), M, K, C.byref(lin), N, act_mult, int(relu),
                                             _ptr(y), _ptr(acc), _ptr(q), threads)
    if rc != 0:
        raise OracleError(rc, "non-finite input, invalid multiplier or accumulator overflow")
    return y, acc, q


def candidate_argmax(xq, xa, emb, mult, bias, cand, offsets):
    """select_token over candidate lists: (tokens [M], logits per list position)."""
    xq = np.ascontiguousarray(xq, np.int8)
    xa = np.ascontiguousarray(xa, np.float32)
    emb = np.ascontiguousarray(emb, np.int8)
    mult = np.ascontiguousarray(mult, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    cand = np.ascontiguousarray(cand, np.uint32)
    offs = np.ascontiguousarray(offsets, np.uint32)
    M, K = xq.shape
    tok = np.zeros(M, np.int32)
    lg = np.zeros(max(cand.size, 1), np.float32)
    rc = load().oracle_candidate_argmax(_ptr(xq), _ptr(xa), M, K, _ptr(emb), _ptr(mult), _ptr(bias),
                                        emb.shape[0], _ptr(cand), _ptr(offs), _ptr(tok), _ptr(lg))
    if rc != 0:
        raise OracleError(rc, "empty candidate list or id outside the vocabulary")
    return tok, lg[:cand.size]


def ssru_layer_norm(cand, forget, state, residual, scale, bias, order=REFERENCE):
    """Returns (out, updated state); the inputs are not modified."""
    cand, forget, residual = (np.ascontiguousarray(t, np.float32) for t in (cand, forget, residual))
    st = np.array(state, np.float32, copy=True, order="C")
    scale = np.ascontiguousarray(scale, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    rows, d = cand.shape
    out = np.zeros_like(cand)
    load().oracle_ssru_layer_norm(_ptr(cand), _ptr(forget), _ptr(st), _ptr(residual), _ptr(scale),
                                  _ptr(bias), rows, d, order, _ptr(out))
    return out, st


def residual_layer_norm(x, r, scale, bias, order=REFERENCE):
    x = np.ascontiguousarray(x, np.float32)
    r = np.ascontiguousarray(r, np.float32)
    scale = np.ascontiguousarray(scale, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    rows, d = x.shape
    out = np.zeros_like(x)
    load().oracle_residual_layer_norm(_ptr(x), _ptr(r), _ptr(scale), _ptr(bias), rows, d, order,
                                      _ptr(out))
    return out


def attention(q, k, v, cu_q, cu_k, heads, order=REFERENCE):
    """Packed multi-head attention; q/k/v are fp32 [rows, heads*64] arrays."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    cu_q = np.ascontiguousarray(cu_q, np.uint32)
    cu_k = np.ascontiguousarray(cu_k, np.uint32)
    out = np.zeros((q.shape[0], q.shape[1]), np.float32)
    dh = q.shape[1] // heads
    rc = load().oracle_attention(_ptr(q), q.shape[1], _ptr(k), k.shape[1], _ptr(v), v.shape[1],
                                 _ptr(cu_q), _ptr(cu_k), cu_q.size - 1, heads, dh, order, _ptr(out),
                                 out.shape[1])
    if rc != 0:
        raise OracleError(rc, "empty key range")
    return out


def encode(model: OracleModel, tokens, offsets, order=REFERENCE, threads=8):
    toks = np.ascontiguousarray(tokens, np.int32)
    offs = np.ascontiguousarray(offsets, np.uint32)
    out = np.zeros((toks.size, model.geometry.dim), np.float32)
    rc = load().oracle_encode(C.byref(model.struct), _ptr(toks), toks.size, _ptr(offs), offs.size,
                              order, threads, _ptr(out))
    if rc != 0:
        raise OracleError(rc, "encode failed")
    return out


def last_step_logits(model: OracleModel, tokens, steps: int, flags=0, order=REFERENCE):
    toks = np.ascontiguousarray(tokens, np.int32)
    out = np.zeros(model.geometry.vocab, np.float32)
    rc = load().oracle_last_step_logits(C.byref(model.struct), _ptr(toks), toks.size, steps, flags,
                                        order, _ptr(out))
    if rc != 0:
        raise OracleError(rc, "last_step_logits failed")
    return out
