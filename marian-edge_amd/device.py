"""Device buffers and op-level calls through the C ABI (no framework needed).

DeviceArray holds HBM allocated by libmarian_hip.so; the op functions take
DeviceArrays and mirror the op-level entry points of include/marian_hip.h.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


class DeviceArray:
    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._lib = _lib.load()
        self.ptr = self._lib.marian_hip_device_alloc(max(self.nbytes, 1))
        if not self.ptr:
            raise MemoryError(f"device allocation of {self.nbytes} bytes failed: {_lib.op_error()}")

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            _lib.check(d._lib.marian_hip_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes), "h2d")
        return d

    @classmethod
    def zeros(cls, shape, dtype) -> "DeviceArray":
        d = cls(shape, dtype)
        _lib.check(d._lib.marian_hip_memset(d.ptr, 0, max(d.nbytes, 1)), "memset")
        return d

    def fill_bytes(self, value: int) -> None:
        _lib.check(self._lib.marian_hip_memset(self.ptr, value, max(self.nbytes, 1)), "memset")

    def host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            _lib.check(self._lib.marian_hip_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes), "d2h")
        return out

    def free(self) -> None:
        if self.ptr:
            self._lib.marian_hip_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(x):
    return None if x is None else x.ptr


def device_count() -> int:
    return _lib.load().marian_hip_device_count()


def device_name(device: int = 0) -> str:
    buf = C.create_string_buffer(256)
    _lib.check(_lib.load().marian_hip_device_name(device, buf, 256), "device_name")
    return buf.value.decode()


def copy(dst: DeviceArray, src: DeviceArray) -> None:
    """Device-to-device copy of src's bytes into dst."""
    n = min(dst.nbytes, src.nbytes)
    _lib.check(_lib.load().marian_hip_memcpy_d2d(dst.ptr, src.ptr, n), "d2d")


def synchronize() -> None:
    _lib.check(_lib.load().marian_hip_device_sync(), "device_sync")


def quantize_rows(x: DeviceArray, q: DeviceArray, a: DeviceArray, err: DeviceArray | None = None,
                  stream=None) -> None:
    rows, cols = x.shape
    _lib.check(_lib.load().marian_hip_quantize_rows(x.ptr, rows, cols, q.ptr, a.ptr, _p(err), stream),
               "quantize_rows")


def q8_linear(x: DeviceArray | None, w: DeviceArray, mult: DeviceArray, bias: DeviceArray,
              out_i32: DeviceArray | None, out_f32: DeviceArray | None, relu: bool = False,
              xq: DeviceArray | None = None, xa: DeviceArray | None = None,
              err: DeviceArray | None = None, stream=None) -> None:
    M, K = (x.shape if x is not None else xq.shape)
    N = w.shape[0]
    _lib.check(_lib.load().marian_hip_q8_linear(
        _p(x), _p(xq), _p(xa), M, K, w.ptr, mult.ptr, bias.ptr, N, int(relu), _p(out_i32),
        _p(out_f32), _p(err), stream), "q8_linear")


def q8_linear_static(x: DeviceArray, act_mult: float, w: DeviceArray, mult: DeviceArray,
                     bias: DeviceArray, out_i32: DeviceArray | None, out_f32: DeviceArray | None,
                     relu: bool = False, err: DeviceArray | None = None, stream=None) -> None:
    M, K = x.shape
    N = w.shape[0]
    _lib.check(_lib.load().marian_hip_q8_linear_static(
        x.ptr, M, K, float(act_mult), w.ptr, mult.ptr, bias.ptr, N, int(relu), _p(out_i32),
        _p(out_f32), _p(err), stream), "q8_linear_static")


def ssru_layer_norm(cand, forget, state, residual, scale, bias, out, q=None, a=None, err=None,
                    stream=None) -> None:
    rows, dim = cand.shape
    _lib.check(_lib.load().marian_hip_ssru_layer_norm(
        cand.ptr, forget.ptr, state.ptr, residual.ptr, scale.ptr, bias.ptr, rows, dim, out.ptr,
        _p(q), _p(a), _p(err), stream), "ssru_layer_norm")


def residual_layer_norm(x, r, scale, bias, out, q=None, a=None, err=None, stream=None) -> None:
    rows, dim = x.shape
    _lib.check(_lib.load().marian_hip_residual_layer_norm(
        x.ptr, r.ptr, scale.ptr, bias.ptr, rows, dim, out.ptr, _p(q), _p(a), _p(err), stream),
        "residual_layer_norm")


def attention(q, k, v, seq_of_row, cu, out, heads: int, max_keys: int, ldq=None, ldkv=None,
              ldo=None, bf16: bool = False, packed_self: bool = True, head_dim: int = 64,
              stream=None) -> None:
    """packed_self: the query rows are the key rows of the cu-packed sequences
    (passes the sequence count, which allows the key-staging kernel)."""
    rows = seq_of_row.shape[0]
    n_seqs = cu.shape[0] - 1 if packed_self else 0
    _lib.check(_lib.load().marian_hip_attention(
        q.ptr, ldq or q.shape[1], k.ptr, v.ptr, ldkv or k.shape[1], seq_of_row.ptr, cu.ptr, n_seqs,
        rows, heads, head_dim, max_keys, int(bf16), out.ptr, ldo or out.shape[1], stream),
        "attention")


def vocab_argmax(xq, xa, emb, emb_mult, bias, token, logits=None, flags: int = 0, stream=None):
    M, K = xq.shape
    V = emb.shape[0]
    _lib.check(_lib.load().marian_hip_vocab_argmax(
        xq.ptr, xa.ptr, M, K, emb.ptr, emb_mult.ptr, bias.ptr, V, flags, token.ptr, _p(logits),
        stream), "vocab_argmax")


def candidate_argmax(xq, xa, emb, emb_mult, bias, cand, cand_offsets, max_cands: int, token,
                     logits=None, err=None, stream=None):
    M, K = xq.shape
    V = emb.shape[0]
    _lib.check(_lib.load().marian_hip_candidate_argmax(
        xq.ptr, xa.ptr, M, K, emb.ptr, emb_mult.ptr, bias.ptr, V, cand.ptr, cand_offsets.ptr,
        int(max_cands), token.ptr, _p(logits), _p(err), stream), "candidate_argmax")


def positions(dim: int, count: int) -> np.ndarray:
    out = np.zeros((count, dim), np.float32)
    _lib.check(_lib.load().marian_hip_positions(dim, count, out.ctypes.data), "positions")
    return out


class Stream:
    def __init__(self):
        self._lib = _lib.load()
        self.handle = self._lib.marian_hip_stream_create()
        if not self.handle:
            raise RuntimeError(f"stream creation failed: {_lib.op_error()}")

    def sync(self):
        _lib.check(self._lib.marian_hip_stream_sync(self.handle), "stream_sync")

    def close(self):
        if self.handle:
            self._lib.marian_hip_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        self._lib = _lib.load()
        self.handle = self._lib.marian_hip_event_create()
        if not self.handle:
            raise RuntimeError(f"event creation failed: {_lib.op_error()}")

    def record(self, stream=None):
        _lib.check(self._lib.marian_hip_event_record(self.handle, stream), "event_record")

    def sync(self):
        _lib.check(self._lib.marian_hip_event_sync(self.handle), "event_sync")

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float(0)
        _lib.check(self._lib.marian_hip_event_elapsed(self.handle, later.handle, C.byref(ms)),
                   "event_elapsed")
        return float(ms.value)

    def close(self):
        if self.handle:
            self._lib.marian_hip_event_destroy(self.handle)
            self.handle = None
