"""Python mirror of the reference's token-level engine and backend interface.

HipEngine.translate_token_ids mirrors CpuTokenEngine::translate_token_ids
(crates/marian-cpu/src/backend.rs:48-57, q8_engine.rs:353-466): packed token ids
and cu_seqlens offsets in, BatchOutput{tokens, offsets} out, errors raised with
the reference's BackendError categories (crates/marian-core/src/types.rs:60-70).
HipBackend carries the TranslationBackend surface that does not need a
tokenizer: info() and is_ready() (crates/marian-core/src/backend.rs:7-38).
Every call goes through libmarian_hip.so.
"""

from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass

import numpy as np

from . import _lib
from .synthetic import SeededModel, SsruModel, REFERENCE_LIMITS


class BackendError(RuntimeError):
    """Base of the reference's BackendError variants."""


class InvalidInput(BackendError):
    pass


class ModelError(BackendError):
    pass


class InferenceError(BackendError):
    pass


class DeviceError(InferenceError):
    """A HIP runtime failure; the engine is not ready afterwards."""


class BufferTooSmall(BackendError):
    pass


_ERRORS = {
    _lib.ERR_INVALID_INPUT: InvalidInput,
    _lib.ERR_MODEL: ModelError,
    _lib.ERR_INFERENCE: InferenceError,
    _lib.ERR_DEVICE: DeviceError,
    _lib.ERR_BUFFER: BufferTooSmall,
    _lib.ERR_NOT_READY: DeviceError,
}


@dataclass
class BatchOutput:
    """crates/marian-cpu/src/engine.rs:80-85"""

    tokens: np.ndarray
    offsets: np.ndarray

    def rows(self) -> list[list[int]]:
        return [self.tokens[self.offsets[i]:self.offsets[i + 1]].tolist()
                for i in range(len(self.offsets) - 1)]


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class _ModelStructs:
    """ctypes model description pointing into the SeededModel's numpy arrays."""

    def __init__(self, m: SeededModel):
        g = m.geometry
        keep = []

        def arr(a, dtype):
            a = np.ascontiguousarray(a, dtype=dtype)
            keep.append(a)
            return _ptr(a)

        def lin(d):
            return _lib.Linear(arr(d["weight"], np.int8), arr(d["mult"], np.float32),
                               arr(d["bias"], np.float32))

        enc = (_lib.EncoderLayer * max(1, len(m.encoder)))()
        for i, L in enumerate(m.encoder):
            enc[i] = _lib.EncoderLayer(
                lin(L["qkv"]), lin(L["out"]), arr(L["ln1"]["scale"], np.float32),
                arr(L["ln1"]["bias"], np.float32), lin(L["ffn1"]), lin(L["ffn2"]),
                arr(L["ln2"]["scale"], np.float32), arr(L["ln2"]["bias"], np.float32))
        dec = (_lib.DecoderLayer * max(1, len(m.decoder)))()
        for i, L in enumerate(m.decoder):
            dec[i] = _lib.DecoderLayer(
                lin(L["self_qkv"]), lin(L["self_out"]), arr(L["ln1"]["scale"], np.float32),
                arr(L["ln1"]["bias"], np.float32), lin(L["cross_q"]), lin(L["cross_kv"]),
                lin(L["cross_out"]), arr(L["ln2"]["scale"], np.float32),
                arr(L["ln2"]["bias"], np.float32), lin(L["ffn1"]), lin(L["ffn2"]),
                arr(L["ln3"]["scale"], np.float32), arr(L["ln3"]["bias"], np.float32))
        self.model = _lib.Model(
            g.vocab, g.dim, g.heads, g.ffn_dim, len(m.encoder), len(m.decoder),
            arr(m.embedding, np.int8), arr(m.embedding_mult, np.float32),
            arr(m.output_bias, np.float32), enc, dec)
        self._keep = (keep, enc, dec)


class _SsruModelStructs:
    """ctypes description of a Transformer-SSRU model (synthetic.SsruModel)."""

    def __init__(self, m: SsruModel):
        g = m.geometry
        keep = []

        def arr(a, dtype):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dtype)
            keep.append(a)
            return _ptr(a)

        def lin(d):
            return _lib.StaticLinear(arr(d["weight"], np.int8), d["weight_mult"], d["act_mult"],
                                     arr(d["bias"], np.float32))

        def ln(d):
            return arr(d["scale"], np.float32), arr(d["bias"], np.float32)

        enc = (_lib.SsruEncoderLayer * max(1, len(m.encoder)))()
        for i, L in enumerate(m.encoder):
            enc[i] = _lib.SsruEncoderLayer(lin(L["wq"]), lin(L["wk"]), lin(L["wv"]), lin(L["wo"]),
                                           *ln(L["attn_ln"]), lin(L["w1"]), lin(L["w2"]),
                                           *ln(L["ffn_ln"]))
        dec = (_lib.SsruDecoderLayer * max(1, len(m.decoder)))()
        for i, L in enumerate(m.decoder):
            dec[i] = _lib.SsruDecoderLayer(lin(L["ssru_w"]), lin(L["ssru_wf"]), *ln(L["ssru_ln"]),
                                           lin(L["wq"]), lin(L["wk"]), lin(L["wv"]), lin(L["wo"]),
                                           *ln(L["context_ln"]), lin(L["w1"]), lin(L["w2"]),
                                           *ln(L["ffn_ln"]))
        self.model = _lib.SsruModel(
            g.source_vocab, g.target_vocab, g.dim, g.heads, g.ffn_dim, len(m.encoder), len(m.decoder),
            arr(m.encoder_embedding, np.int8), m.encoder_embedding_mult,
            arr(m.decoder_embedding, np.int8), m.decoder_embedding_mult, m.output_act_mult,
            arr(m.output_bias, np.float32), enc, dec)
        self._keep = (keep, enc, dec)


def make_limits(limits: dict | None) -> _lib.Limits:
    d = dict(REFERENCE_LIMITS)
    if limits:
        d.update(limits)
    return _lib.Limits(d["max_length_factor"], d["max_generation_steps"], d["max_position"],
                       d["max_batch"], d["max_source_tokens"], d["max_padded_cells"])


def capacity_for(batches) -> dict:
    """The marian_hip_reserve capacity that covers every batch in `batches`
    (objects with tokens, offsets and max_output_tokens, e.g. synthetic.Batch),
    with the generation limits as requested (caps may only lower them)."""
    cap = dict(sentences=0, source_tokens=0, output_tokens=0, steps=0)
    for b in batches:
        lim = np.asarray(b.max_output_tokens, np.int64)
        cap["sentences"] = max(cap["sentences"], len(b.offsets) - 1)
        cap["source_tokens"] = max(cap["source_tokens"], int(np.asarray(b.tokens).size))
        cap["output_tokens"] = max(cap["output_tokens"], int(np.minimum(lim, 4096).sum()))
        cap["steps"] = max(cap["steps"], int(np.minimum(lim, 4096).max(initial=0)))
    return cap


def validate_batch(tokens, offsets, limits: dict | None = None, source_vocab: int = 32000,
                   target_vocab: int = 32000, candidates=None, candidate_offsets=None) -> None:
    """The library's host-only batch checks (marian_hip_validate_batch, the
    reference's validate_batch, q8_engine.rs:468-509); raises InvalidInput
    with the reference's message.  Needs no device."""
    lib = _lib.load()
    toks = np.ascontiguousarray(tokens, np.int32)
    offs = np.ascontiguousarray(offsets, np.uint32)
    lim = make_limits(limits)
    cand = coff = None
    if candidates is not None or candidate_offsets is not None:
        cand = np.ascontiguousarray(candidates, np.uint32)
        coff = np.ascontiguousarray(candidate_offsets, np.uint32)
    msg = C.create_string_buffer(512)
    rc = lib.marian_hip_validate_batch(
        C.byref(lim), source_vocab, target_vocab, _ptr(toks) if toks.size else None, toks.size,
        _ptr(offs) if offs.size else None, offs.size,
        _ptr(cand) if cand is not None and cand.size else None,
        _ptr(coff) if coff is not None and coff.size else None, msg, len(msg))
    if rc != _lib.OK:
        raise _ERRORS.get(rc, BackendError)(msg.value.decode(errors="replace"))


class HipEngine:
    """Owns one marian_hip_engine (one device, one stream, one owner thread)."""

    def __init__(self, model: SeededModel | SsruModel, limits: dict | None = None, device: int = 0,
                 capacity: dict | None = None):
        """A SeededModel gives the transformer-decoder engine
        (marian_hip_engine_create), an SsruModel the reference's
        Transformer-SSRU graph (marian_hip_engine_create_ssru).  `capacity`
        (marian_hip_capacity fields, e.g. from capacity_for) sizes the decode
        buffers at creation, so calls within it allocate nothing."""
        self._lib = _lib.load()
        self._limits = make_limits(limits)
        handle = C.c_void_p()
        if isinstance(model, SsruModel):
            structs = _SsruModelStructs(model)
            create = self._lib.marian_hip_engine_create_ssru
            self.target_vocab = model.geometry.target_vocab
        else:
            structs = _ModelStructs(model)
            create = self._lib.marian_hip_engine_create
            self.target_vocab = model.geometry.vocab
        rc = create(C.byref(structs.model), C.byref(self._limits), device, C.byref(handle))
        if rc != _lib.OK:
            raise _ERRORS.get(rc, BackendError)(
                f"engine creation failed ({rc}): {self._lib.marian_hip_last_op_error().decode(errors='replace')}")
        self._h = handle
        self.geometry = model.geometry
        if capacity:
            self.reserve(**capacity)

    def reserve(self, sentences: int, source_tokens: int, output_tokens: int, steps: int,
                candidate_ids: int = 0, max_candidates: int = 0) -> None:
        """marian_hip_reserve: size the buffers for calls up to this capacity."""
        cap = _lib.Capacity(int(sentences), int(source_tokens), int(output_tokens), int(steps),
                            int(candidate_ids), int(max_candidates))
        rc = self._lib.marian_hip_reserve(self._h, C.byref(cap))
        if rc != _lib.OK:
            self._raise(rc)

    def warmup(self) -> None:
        """Q8CpuEngine::warmup (q8_engine.rs:349-351): the batch [2, 0], at
        most 4 output tokens."""
        rc = self._lib.marian_hip_warmup(self._h)
        if rc != _lib.OK:
            self._raise(rc)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.marian_hip_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _raise(self, rc: int):
        msg = self._lib.marian_hip_last_error(self._h).decode(errors="replace")
        raise _ERRORS.get(rc, BackendError)(msg)

    def translate_token_ids(self, tokens, offsets, max_output_tokens, flags: int = 0,
                            candidates=None, candidate_offsets=None) -> BatchOutput:
        """With candidates (concatenated per-sentence lists and their offsets
        [B + 1], e.g. from shortlist.pack_candidates) each sentence is scored
        only over its list (marian_hip_translate_shortlisted)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        offs = np.ascontiguousarray(offsets, np.uint32)
        lim = np.ascontiguousarray(max_output_tokens, np.uint32)
        if lim.shape[0] != max(0, offs.shape[0] - 1):
            raise InvalidInput("max_output_tokens does not match packed batch")
        cap = int(np.minimum(lim.astype(np.int64), 4096).sum())
        out = np.zeros(max(cap, 1), np.int32)
        out_offs = np.zeros(max(offs.shape[0], 1), np.uint32)
        n = C.c_size_t(0)
        if candidates is not None or candidate_offsets is not None:
            cand = np.ascontiguousarray(candidates, np.uint32)
            coff = np.ascontiguousarray(candidate_offsets, np.uint32)
            if coff.shape[0] != offs.shape[0]:
                raise InvalidInput("candidate offsets do not match the packed batch")
            rc = self._lib.marian_hip_translate_shortlisted(
                self._h, _ptr(toks) if toks.size else None, toks.size, _ptr(offs), offs.size,
                _ptr(lim), flags, _ptr(cand) if cand.size else None, _ptr(coff), _ptr(out), out.size,
                _ptr(out_offs), C.byref(n))
        else:
            rc = self._lib.marian_hip_translate_token_ids(
                self._h, _ptr(toks) if toks.size else None, toks.size, _ptr(offs), offs.size,
                _ptr(lim), flags, _ptr(out), out.size, _ptr(out_offs), C.byref(n))
        if rc != _lib.OK:
            self._raise(rc)
        return BatchOutput(out[:n.value].copy(), out_offs.copy())

    def translate_probe(self, tokens, offsets, max_output_tokens, flags: int = 0,
                        probe_step: int = 0):
        """translate_token_ids plus what the engine computed below the token
        level: (BatchOutput, encoder states [T, d], logits [B, V] of decode step
        probe_step, active [B] = rows whose logits were captured)."""
        toks = np.ascontiguousarray(tokens, np.int32)
        offs = np.ascontiguousarray(offsets, np.uint32)
        lim = np.ascontiguousarray(max_output_tokens, np.uint32)
        B = max(0, offs.shape[0] - 1)
        if lim.shape[0] != B:
            raise InvalidInput("max_output_tokens does not match packed batch")
        g = self.geometry
        cap = int(np.minimum(lim.astype(np.int64), 4096).sum())
        out = np.zeros(max(cap, 1), np.int32)
        out_offs = np.zeros(max(offs.shape[0], 1), np.uint32)
        enc = np.zeros((max(toks.size, 1), g.dim), np.float32)
        logits = np.zeros((max(B, 1), self.target_vocab), np.float32)
        active = np.zeros(max(B, 1), np.uint8)
        n = C.c_size_t(0)
        rc = self._lib.marian_hip_translate_probe(
            self._h, _ptr(toks) if toks.size else None, toks.size, _ptr(offs), offs.size,
            _ptr(lim), flags, _ptr(out), out.size, _ptr(out_offs), C.byref(n), int(probe_step),
            _ptr(enc), _ptr(logits), _ptr(active))
        if rc != _lib.OK:
            self._raise(rc)
        return (BatchOutput(out[:n.value].copy(), out_offs.copy()), enc[:toks.size], logits[:B],
                active[:B].astype(bool))

    TIME_STEPS, TIME_KERNELS = 1, 2

    def set_timing(self, flags: int) -> None:
        """TIME_STEPS: per-step end times (last_step_trace); TIME_KERNELS: per
        launch durations of the vocabulary and attention-block kernels
        (last_kernel_trace), at several microseconds of device time each."""
        rc = self._lib.marian_hip_set_timing(self._h, int(flags))
        if rc != _lib.OK:
            self._raise(rc)

    def last_stats(self) -> dict:
        s = _lib.Stats()
        self._lib.marian_hip_last_stats(self._h, C.byref(s))
        return {f: getattr(s, f) for f, _ in _lib.Stats._fields_}

    def last_step_trace(self) -> tuple[np.ndarray, np.ndarray]:
        """(active rows per decode step, device ms at each step's end)."""
        n = C.c_size_t(0)
        self._lib.marian_hip_last_step_trace(self._h, None, None, 0, C.byref(n))
        rows = np.zeros(max(n.value, 1), np.uint32)
        ms = np.zeros(max(n.value, 1), np.float32)
        self._lib.marian_hip_last_step_trace(self._h, _ptr(rows), _ptr(ms), n.value, C.byref(n))
        return rows[:n.value], ms[:n.value]

    KERNEL_VOCAB, KERNEL_SELF_BLOCK, KERNEL_CROSS_BLOCK, KERNEL_SELF_ATTN, KERNEL_CROSS_ATTN = 0, 1, 2, 3, 4

    def last_kernel_trace(self) -> dict:
        """Per timed decode launch of the last call (kernel timing on):
        kind (KERNEL_*), decode step, decoder layer, device microseconds."""
        n = C.c_size_t(0)
        self._lib.marian_hip_last_kernel_trace(self._h, None, None, None, None, 0, C.byref(n))
        m = max(n.value, 1)
        kind, step, layer = (np.zeros(m, np.uint32) for _ in range(3))
        us = np.zeros(m, np.float32)
        self._lib.marian_hip_last_kernel_trace(self._h, _ptr(kind), _ptr(step), _ptr(layer), _ptr(us),
                                               n.value, C.byref(n))
        k = n.value
        return dict(kind=kind[:k], step=step[:k], layer=layer[:k], us=us[:k])

    def is_ready(self) -> bool:
        return bool(self._lib.marian_hip_is_ready(self._h))

    def info(self) -> dict:
        buf = C.create_string_buffer(1024)
        rc = self._lib.marian_hip_info(self._h, buf, len(buf))
        if rc != _lib.OK:
            self._raise(rc)
        return json.loads(buf.value.decode())


class HipBackend:
    """TranslationBackend surface at the token level (backend.rs:7-38).

    duplicate_batch_width: how many physical rows a logical input repeated by
    the scheduler may occupy (translate_batch_with_repetitions, backend.rs:25-37;
    the Metal backend materializes up to this many copies to reach its device's
    occupancy knee, crates/marian-metal/src/backend.rs:319-354).  The default 1
    materializes none: a decode step here costs about the same from 1 to 4 rows
    and more above, so copies of a row only add work."""

    def __init__(self, engine: HipEngine, duplicate_batch_width: int = 1, warmup: bool = True):
        """Like the reference's backends, warms the engine up once at load
        (backend.rs:448); a failure there is an InferenceError."""
        if duplicate_batch_width < 1:
            raise InvalidInput("duplicate_batch_width must be at least 1")
        self.engine = engine
        self.duplicate_batch_width = int(duplicate_batch_width)
        if warmup:
            try:
                engine.warmup()
            except BackendError as e:
                raise InferenceError(f"HIP warmup failed: {e}") from e

    def info(self) -> dict:
        return self.engine.info()

    def is_ready(self) -> bool:
        return self.engine.is_ready()

    def translate_token_batch(self, sentences: list[list[int]], max_output_tokens: list[int],
                              repetitions: list[int] | None = None, flags: int = 0):
        """One output per logical input, like translate_batch_with_repetitions
        (backend.rs:30-37): logical input i is run as min(repetitions[i],
        duplicate_batch_width) physical rows and the first copy's output is
        returned; repetitions do not change the result."""
        if repetitions is None:
            repetitions = [1] * len(sentences)
        if len(repetitions) != len(sentences) or any(int(c) <= 0 for c in repetitions):
            raise InvalidInput("logical batch repetitions are malformed")
        if len(max_output_tokens) != len(sentences):
            raise InvalidInput("max_output_tokens does not match inputs")
        physical, limits, first = [], [], []
        for sent, lim, count in zip(sentences, max_output_tokens, repetitions):
            first.append(len(physical))
            for _ in range(min(int(count), self.duplicate_batch_width)):
                physical.append(sent)
                limits.append(lim)
        offs = np.zeros(len(physical) + 1, np.uint32)
        offs[1:] = np.cumsum([len(s) for s in physical])
        toks = np.concatenate([np.asarray(s, np.int32) for s in physical]) if physical else \
            np.zeros(0, np.int32)
        out = self.engine.translate_token_ids(toks, offs, limits, flags)
        rows = out.rows()
        if len(rows) != len(physical):
            raise InferenceError(f"backend returned {len(rows)} physical outputs for "
                                 f"{len(physical)} rows")
        return [rows[i] for i in first]
