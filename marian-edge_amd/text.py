"""Text-side callers of the token engine: bounded segmentation of long source
text and the text-to-text translation flow with one output budget per input.

Host-side restatements of
  segment_text            crates/marian-core/src/segmenter.rs:122-196 (and its
                          helpers :198-727), on UTF-8 byte offsets like the
                          reference's ranges;
  translate_with_engine   crates/marian-cpu/src/backend.rs:107-348: segments
                          each input, encodes with EOS, and runs the segments in
                          rounds (at most one per input per round) so that each
                          segment gets what is left of its input's
                          max_output_tokens after the segments before it;
  TranslationBackend      crates/marian-core/src/backend.rs:7-38, as
                          HipTextBackend over a HipEngine (or any token engine).

The token engine is anything with translate_token_ids(tokens, offsets,
max_output_tokens) returning an object with `tokens` and `offsets`
(HipEngine, or HipTokenEngine when a lexical shortlist gives the candidates).
Outputs are batch-invariant, so which segments share a round does not change a
result; the reference's padded-attention cap on a round (a CPU cost bound) is
kept as the default and can be lifted for the GPU engine.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Protocol

import numpy as np

from .engine import BackendError, InferenceError, InvalidInput

# segmenter.rs:13-22
MAX_SEGMENTER_INPUT_BYTES = 4 * 1024 * 1024
MAX_SEGMENTS = 4096
MAX_ENCODING_CALLS = 32_768
MAX_ENCODING_BYTES = 64 * 1024 * 1024
MAX_COUNTED_PIECES = 8 * 1024 * 1024
# crates/marian-cpu/src/limits.rs:3-7
MAXIMUM_SOURCE_TOKENS = 256
MAXIMUM_ENGINE_BATCH = 256
MAXIMUM_PADDED_ATTENTION_CELLS = 65_536
MAXIMUM_TRANSLATION_SEGMENTS = 4096


class UnsupportedDirection(BackendError):
    """BackendError::UnsupportedDirection (crates/marian-core/src/types.rs:60-70)."""


class SegmentError(ValueError):
    """segmenter.rs:48-108; `kind` names the variant, `fields` its values."""

    def __init__(self, kind: str, text: str, **fields):
        super().__init__(text)
        self.kind = kind
        self.fields = fields


@dataclass
class TextSegment:
    """Byte ranges of one content fragment and the separator after it."""
    content_range: range
    separator_range: range
    source_pieces: int

    def content(self, text: str) -> str:
        return text.encode("utf-8")[self.content_range.start:self.content_range.stop].decode("utf-8")

    def separator(self, text: str) -> str:
        return text.encode("utf-8")[self.separator_range.start:self.separator_range.stop].decode("utf-8")

    def full_range(self) -> range:
        return range(self.content_range.start, self.separator_range.stop)


# Unicode White_Space, the set Rust's char::is_whitespace tests (Python's
# str.isspace also accepts U+001C..U+001F, which Rust does not).
_WHITE_SPACE = frozenset(
    [0x09, 0x0A, 0x0B, 0x0C, 0x0D, 0x20, 0x85, 0xA0, 0x1680, 0x2028, 0x2029, 0x202F, 0x205F, 0x3000]
    + list(range(0x2000, 0x200B)))
_TERMINATORS = frozenset(".!?\u3002\uff01\uff1f\u2026")
_CLOSING = frozenset("\"'\u2019\u201d\u00bb)]}\u3009\u300b\u300d\u300f\u3011\u3015\u3017\u3019\u301b")
_TITLE = frozenset("capt. col. dr. gen. gov. lt. mr. mrs. ms. prof. rep. rev. sen. sgt. sr. st.".split())
_NON_TERMINAL = frozenset(
    "e.g. i.e. fig. no. vs. jan. feb. mar. apr. jun. jul. aug. sep. sept. oct. nov. dec.".split())
_COMMON = frozenset("approx. co. corp. dept. ed. eds. est. etc. inc. ltd. misc. p. pp. vol.".split())


def _ws(c: str) -> bool:
    return ord(c) in _WHITE_SPACE


def _ascii_digit(c) -> bool:
    return c is not None and "0" <= c <= "9"


class _Text:
    """A string viewed as UTF-8 bytes, with scalar stepping by byte offset."""

    def __init__(self, text: str):
        self.s = text
        self.b = text.encode("utf-8")
        self.n = len(self.b)

    def boundary(self, i: int) -> bool:
        return i <= 0 or i >= self.n or (self.b[i] & 0xC0) != 0x80

    def next(self, i: int) -> tuple[str, int]:
        lead = self.b[i]
        w = 1 if lead < 0x80 else 2 if lead < 0xE0 else 3 if lead < 0xF0 else 4
        return self.b[i:i + w].decode("utf-8"), i + w

    def prev(self, end: int) -> tuple[int, str]:
        i = end - 1
        while i > 0 and (self.b[i] & 0xC0) == 0x80:
            i -= 1
        return i, self.b[i:end].decode("utf-8")

    def slice(self, a: int, b: int) -> str:
        return self.b[a:b].decode("utf-8")

    def consume(self, i: int, end: int, pred) -> int:
        while i < end:
            c, nx = self.next(i)
            if not pred(c):
                break
            i = nx
        return i


class _Counter:
    """Cached, bounded piece counting (PieceCounter, segmenter.rs:186-265)."""

    def __init__(self, t: _Text, count: Callable[[str], int]):
        self.t, self.count_fn = t, count
        self.cache: dict[tuple[int, int], int] = {}
        self.calls = self.bytes = self.pieces = 0

    def count(self, a: int, b: int) -> int:
        key = (a, b)
        if key in self.cache:
            return self.cache[key]
        self.calls += 1
        if self.calls > MAX_ENCODING_CALLS:
            raise SegmentError("EncodingWorkLimit", f"source segmentation exceeded tokenizer calls safety "
                               f"limit {MAX_ENCODING_CALLS}", resource="tokenizer calls",
                               maximum=MAX_ENCODING_CALLS)
        self.bytes += b - a
        if self.bytes > MAX_ENCODING_BYTES:
            raise SegmentError("EncodingWorkLimit", f"source segmentation exceeded encoded bytes safety "
                               f"limit {MAX_ENCODING_BYTES}", resource="encoded bytes",
                               maximum=MAX_ENCODING_BYTES)
        try:
            pieces = int(self.count_fn(self.t.slice(a, b)))
        except SegmentError:
            raise
        except Exception as e:  # the closure's error becomes SegmentError::Encoding
            raise SegmentError("Encoding", f"source tokenizer failed for byte range {a}..{b}: {e}",
                               start=a, end=b, message=str(e)) from e
        self.pieces += pieces
        if self.pieces > MAX_COUNTED_PIECES:
            raise SegmentError("EncodingWorkLimit", f"source segmentation exceeded counted pieces safety "
                               f"limit {MAX_COUNTED_PIECES}", resource="counted pieces",
                               maximum=MAX_COUNTED_PIECES)
        self.cache[key] = pieces
        return pieces


def _push(result: list, seg: TextSegment) -> None:
    if len(result) >= MAX_SEGMENTS:
        raise SegmentError("TooManySegments", f"source requires more than {MAX_SEGMENTS} segments",
                           maximum=MAX_SEGMENTS)
    result.append(seg)


def _initial_or_acronym(token: str) -> bool:
    parts = token.rstrip(".").split(".")
    return 0 < len(parts) <= 8 and all(len(p) == 1 and p.isascii() and p.isalpha() for p in parts)


def _period_ends_sentence(t: _Text, index: int, quoted_end: int) -> bool:
    """segmenter.rs:601-661: decimals, titles, fixed abbreviations, common
    abbreviations before lowercase or digits, initials before uppercase."""
    prev = t.prev(index)[1] if index > 0 else None
    nxt = t.next(index + 1)[0] if index + 1 < t.n else None
    if _ascii_digit(prev) and _ascii_digit(nxt):
        return False
    token_start = 0
    j = index
    while j > 0:
        k, c = t.prev(j)
        if _ws(c) or c in "([{\"\u201c":
            token_start = j
            break
        j = k
    # ASCII-lowercased, keeping ASCII alphanumerics and periods only
    token = "".join(c.lower() for c in t.slice(token_start, index + 1)
                    if (c.isascii() and c.isalnum()) or c == ".")
    following = t.slice(quoted_end, t.n)
    k = 0
    while k < len(following) and _ws(following[k]):
        k += 1
    fc = following[k] if k < len(following) else None
    if token in _TITLE and fc is not None:
        return False
    if token in _NON_TERMINAL and fc is not None:
        return False
    if token in _COMMON and fc is not None and ((fc.isascii() and fc.islower()) or _ascii_digit(fc)):
        return False
    if _initial_or_acronym(token) and fc is not None and fc.isascii() and fc.isupper():
        return False
    return True


def _sentence_units(t: _Text, content_end: int) -> list[list[range]]:
    """segmenter.rs:267-320: sentence ends (terminators, closing marks, then
    whitespace or the end) and line breaks delimit units."""
    units: list[list[range]] = []
    cursor = index = 0
    while index < content_end:
        c, nx = t.next(index)
        if c in _TERMINATORS:
            p_end = t.consume(index, content_end, lambda ch: ch in _TERMINATORS)
            q_end = t.consume(p_end, content_end, lambda ch: ch in _CLOSING)
            follows = q_end == content_end or (q_end < content_end and _ws(t.next(q_end)[0]))
            if follows and (c != "." or _period_ends_sentence(t, index, q_end)):
                s_end = t.consume(q_end, content_end, _ws)
                units.append([range(cursor, q_end), range(q_end, s_end)])
                cursor = index = s_end
                continue
            index = max(p_end, nx)
            continue
        if _ws(c):
            w_end = t.consume(index, content_end, _ws)
            if any(ch in "\n\r" for ch in t.slice(index, w_end)):
                units.append([range(cursor, index), range(index, w_end)])
                cursor = w_end
            index = w_end
            continue
        index = nx
    if cursor < content_end:
        units.append([range(cursor, content_end), range(content_end, t.n)])
    elif units:
        units[-1][1] = range(units[-1][1].start, t.n)
    return units


def _dash_boundary(t: _Text, index: int, start: int, end: int) -> bool:
    repeated = index + 1 < end and t.b[index + 1] == ord("-")
    before = index == start or _ws(t.prev(index)[1])
    after = index + 1 >= end or _ws(t.next(index + 1)[0])
    return repeated or before or after


def _break_points(t: _Text, start: int, end: int) -> list[tuple[int, int, int]]:
    """(content_end, next_start, priority): 0 clause punctuation and dashes,
    1 commas, 2 whitespace (segmenter.rs:475-516)."""
    points = []
    index = start
    while index < end:
        c, nx = t.next(index)
        if _ws(c):
            w_end = t.consume(index, end, _ws)
            points.append((index, w_end, 2))
            index = w_end
            continue
        if c in ";\uff1b:\uff1a/\u2013\u2014" or (c == "-" and _dash_boundary(t, index, start, end)):
            prio = 0
        elif c in ",\uff0c":
            prio = 1
        else:
            index = nx
            continue
        p_end = nx
        if c == "-":
            while p_end < end and t.b[p_end] == ord("-"):
                p_end += 1
        points.append((p_end, t.consume(p_end, end, _ws), prio))
        index = p_end
    return points


def _rightmost_fitting(points, prio, start, end, max_pieces, counter):
    cands = [p for p in points if p[2] == prio and p[0] > start and p[1] > start and p[1] < end]
    lo, hi, best = 0, len(cands), None
    while lo < hi:
        mid = lo + (hi - lo) // 2
        pieces = counter.count(start, cands[mid][0])
        if pieces <= max_pieces:
            best = (cands[mid], pieces)
            lo = mid + 1
        else:
            hi = mid
    return best


def _largest_scalar_prefix(t: _Text, start, end, max_pieces, counter):
    first_end = t.next(start)[1]
    first = counter.count(start, first_end)
    if first > max_pieces:
        raise SegmentError("UnsplitableScalar", f"UTF-8 scalar at byte range {start}..{first_end} encodes "
                           f"to {first} pieces; maximum is {max_pieces}", start=start, end=first_end,
                           pieces=first, maximum=max_pieces)
    lo, hi, best = first_end, end, (first_end, first)
    while lo < hi:
        mid = lo + (hi - lo + 1) // 2
        while mid > start and not t.boundary(mid):  # floor_char_boundary
            mid -= 1
        if mid <= best[0]:
            break
        pieces = counter.count(start, mid)
        if pieces <= max_pieces:
            best = (mid, pieces)
            lo = mid
        else:  # previous_char_boundary
            p = mid - 1 if mid > start else start
            while p > start and not t.boundary(p):
                p -= 1
            hi = p
    return best


def _split_oversize(t: _Text, unit, max_pieces, counter, result) -> None:
    """segmenter.rs:322-390 with :392-473: rightmost fitting break of the best priority,
    else the largest fitting UTF-8 prefix."""
    content, sep = unit
    points = _break_points(t, content.start, content.stop)
    start = content.start
    while start < content.stop:
        rem = counter.count(start, content.stop)
        if rem <= max_pieces:
            _push(result, TextSegment(range(start, content.stop), sep, rem))
            return
        sel = None
        for prio in (0, 1, 2):
            sel = _rightmost_fitting(points, prio, start, content.stop, max_pieces, counter)
            if sel:
                break
        if sel:
            (c_end, n_start, _), pieces = sel
        else:
            c_end, pieces = _largest_scalar_prefix(t, start, content.stop, max_pieces, counter)
            n_start = c_end
        _push(result, TextSegment(range(start, c_end), range(c_end, n_start), pieces))
        start = n_start
    if sep.start < sep.stop and result:
        last = result[-1]
        last.separator_range = range(last.separator_range.start, sep.stop)


def segment_text(text: str, max_pieces: int, count_pieces: Callable[[str], int]) -> list[TextSegment]:
    """Splits text into ordered, lossless byte ranges whose content fits
    max_pieces (segmenter.rs:122-173).  count_pieces returns the exact piece
    count of a string, or raises (reported as an Encoding error)."""
    if max_pieces == 0:
        raise SegmentError("ZeroPieceLimit", "source piece limit must be non-zero")
    t = _Text(text)
    if t.n > MAX_SEGMENTER_INPUT_BYTES:
        raise SegmentError("InputTooLarge", f"source contains {t.n} bytes; segmenter maximum is "
                           f"{MAX_SEGMENTER_INPUT_BYTES}", bytes=t.n, maximum=MAX_SEGMENTER_INPUT_BYTES)
    content_end = t.n
    while content_end > 0:
        k, c = t.prev(content_end)
        if not _ws(c):
            break
        content_end = k
    counter = _Counter(t, count_pieces)
    whole = counter.count(0, content_end)
    units = _sentence_units(t, content_end)
    if whole <= max_pieces and len(units) <= 1:
        return [TextSegment(range(0, content_end), range(content_end, t.n), whole)]
    result: list[TextSegment] = []
    for unit in units:
        pieces = counter.count(unit[0].start, unit[0].stop)
        if pieces <= max_pieces:
            _push(result, TextSegment(unit[0], unit[1], pieces))
        else:
            _split_oversize(t, unit, max_pieces, counter, result)
    return result


# ---------------------------------------------------------------------------
# Text-level translation (crates/marian-cpu/src/backend.rs:107-348).
# ---------------------------------------------------------------------------
class TextTokenizer(Protocol):
    """crates/marian-cpu/src/backend.rs:26-32."""

    def vocabulary_size(self) -> int: ...

    def encode(self, text: str) -> list[int]: ...

    def decode(self, token_ids: list[int]) -> str: ...


@dataclass
class TranslationInput:
    """crates/marian-core/src/types.rs:6-25 (max_output_tokens defaults to 512)."""
    text: str
    source_lang: str
    target_lang: str
    max_output_tokens: int = 512


@dataclass
class TranslationOutput:
    text: str
    input_tokens: int
    output_tokens: int
    score: float | None = None


@dataclass
class _Planned:
    translated: str | None
    separator: str
    input_tokens: int
    output_tokens: int = 0


@dataclass
class _Work:
    input_index: int
    segment_index: int
    tokens: list = field(default_factory=list)


def translate_with_engine(engine, source: TextTokenizer, target: TextTokenizer, source_lang: str,
                          target_lang: str, eos_id: int, inputs: list[TranslationInput], *,
                          label: str = "HIP", max_engine_batch: int = MAXIMUM_ENGINE_BATCH,
                          max_padded_cells: int = MAXIMUM_PADDED_ATTENTION_CELLS) -> list[TranslationOutput]:
    """The reference's text flow over a token engine.  max_padded_cells = 0
    lifts the padded-attention cap on a round (the GPU engine packs rows
    without padding); results do not depend on it."""
    if not inputs:
        return []
    for inp in inputs:
        if inp.source_lang != source_lang or inp.target_lang != target_lang:
            raise UnsupportedDirection(f"{inp.source_lang} -> {inp.target_lang}; loaded model is "
                                       f"{source_lang} -> {target_lang}")
    planned: list[list[_Planned]] = []
    work: list[list[_Work]] = [[] for _ in inputs]
    total = 0
    vocab = source.vocabulary_size()
    for ii, inp in enumerate(inputs):
        try:
            segments = segment_text(inp.text, MAXIMUM_SOURCE_TOKENS - 1, lambda s: len(source.encode(s)))
        except SegmentError as e:
            raise InvalidInput(str(e)) from e
        plan: list[_Planned] = []
        for seg in segments:
            content, sep = seg.content(inp.text), seg.separator(inp.text)
            si = len(plan)
            if not content:
                plan.append(_Planned("", sep, 0))
                continue
            if total >= MAXIMUM_TRANSLATION_SEGMENTS:
                raise InvalidInput(f"batch requires more than {MAXIMUM_TRANSLATION_SEGMENTS} translated segments")
            try:
                pieces = list(source.encode(content))
            except Exception as e:
                raise InvalidInput(f"tokenizer encoding failed: {e}") from e
            if len(pieces) != seg.source_pieces:
                raise InferenceError(f"source tokenizer returned {len(pieces)} pieces after sizing the "
                                     f"segment as {seg.source_pieces}")
            bad = [p for p in pieces if p < 0 or p >= vocab]
            if bad:
                raise InvalidInput(f"tokenizer returned source token {bad[0]} outside vocabulary {vocab}")
            pieces.append(eos_id)
            if len(pieces) > MAXIMUM_SOURCE_TOKENS:
                raise InferenceError(f"segmented source has {len(pieces)} tokens including EOS; maximum is "
                                     f"{MAXIMUM_SOURCE_TOKENS}")
            plan.append(_Planned(None, sep, len(pieces)))
            work[ii].append(_Work(ii, si, pieces))
            total += 1
        planned.append(plan)

    pos = [0] * len(work)
    remaining = [int(inp.max_output_tokens) for inp in inputs]
    while True:
        # An input whose budget is spent gets empty translations for the rest.
        for ii in range(len(work)):
            if remaining[ii] != 0:
                continue
            while pos[ii] < len(work[ii]):
                dst = planned[ii][work[ii][pos[ii]].segment_index]
                if dst.translated is not None:
                    raise InferenceError(f"{label} segment was translated more than once")
                dst.translated = ""
                pos[ii] += 1
        batch: list[_Work] = []
        longest = 0
        for ii, segs in enumerate(work):
            if pos[ii] >= len(segs):
                continue
            if len(batch) >= max_engine_batch:
                break
            seg = segs[pos[ii]]
            cand = max(longest, len(seg.tokens))
            if max_padded_cells and (len(batch) + 1) * cand * cand > max_padded_cells:
                continue
            longest = cand
            batch.append(seg)
        if not batch:
            if all(p == len(s) for p, s in zip(pos, work)):
                break
            raise InferenceError(f"unable to construct a bounded {label} inference batch")
        tokens = np.concatenate([np.asarray(w.tokens, np.int32) for w in batch])
        offsets = np.zeros(len(batch) + 1, np.uint32)
        offsets[1:] = np.cumsum([len(w.tokens) for w in batch])
        limits = [min(remaining[w.input_index], 0xFFFFFFFF) for w in batch]
        out = engine.translate_token_ids(tokens, offsets, limits)
        o_off = [int(v) for v in out.offsets]
        o_tok = [int(v) for v in out.tokens]
        if len(o_off) != len(batch) + 1:
            raise InferenceError(f"{label} engine returned malformed batch offsets")
        for row, w in enumerate(batch):
            a, b = o_off[row], o_off[row + 1]
            if b < a or b > len(o_tok):
                raise InferenceError(f"{label} engine returned out-of-range token offsets")
            if b - a > remaining[w.input_index]:
                raise InferenceError(f"{label} engine exceeded the original max_output_tokens budget")
            remaining[w.input_index] -= b - a
            ids = [t for t in o_tok[a:b] if t != eos_id]
            try:
                text = target.decode(ids)
            except Exception as e:
                raise InferenceError(f"tokenizer decoding failed: {e}") from e
            dst = planned[w.input_index][w.segment_index]
            if dst.translated is not None:
                raise InferenceError(f"{label} segment was translated more than once")
            dst.translated = text
            dst.output_tokens = len(ids)
            pos[w.input_index] += 1

    outputs = []
    for plan in planned:
        if any(p.translated is None for p in plan):
            raise InferenceError(f"{label} segment has no translation result")
        outputs.append(TranslationOutput(text="".join(p.translated + p.separator for p in plan),
                                         input_tokens=sum(p.input_tokens for p in plan),
                                         output_tokens=sum(p.output_tokens for p in plan)))
    return outputs


class HipTokenEngine:
    """A HipEngine plus the model's lexical shortlist: each sentence is scored
    over its shortlist candidates (Q8CpuEngine::prepare_candidates,
    crates/marian-cpu/src/q8_engine.rs:576-584); without a shortlist, the
    whole vocabulary."""

    def __init__(self, engine, shortlist=None):
        self.engine = engine
        self.shortlist = shortlist

    def translate_token_ids(self, tokens, offsets, max_output_tokens, flags: int = 0):
        if self.shortlist is None:
            return self.engine.translate_token_ids(tokens, offsets, max_output_tokens, flags)
        from .shortlist import pack_candidates
        lists = [self.shortlist.candidates(tokens[offsets[b]:offsets[b + 1]])
                 for b in range(len(offsets) - 1)]
        cand, coff, _ = pack_candidates(lists)
        return self.engine.translate_token_ids(tokens, offsets, max_output_tokens, flags,
                                               candidates=cand, candidate_offsets=coff)


class HipTextBackend:
    """TranslationBackend at the text level (crates/marian-core/src/backend.rs:7-38;
    the reference's Q8CpuBackend, crates/marian-cpu/src/backend.rs:497-968, over
    the HIP engine).  Rounds are not capped by padded attention cells: the
    engine packs rows without padding."""

    def __init__(self, engine, source: TextTokenizer, target: TextTokenizer, source_lang: str,
                 target_lang: str, eos_id: int = 0, shortlist=None, model_id: str = "marian-q8",
                 duplicate_batch_width: int = 1, warmup: bool = True):
        if duplicate_batch_width < 1:
            raise InvalidInput("duplicate_batch_width must be at least 1")
        self.engine = engine
        if warmup:  # Q8CpuBackend warms its engine at load (backend.rs:810-814)
            try:
                engine.warmup()
            except BackendError as e:
                raise InferenceError(f"HIP warmup failed: {e}") from e
        self.token_engine = HipTokenEngine(engine, shortlist)
        self.source, self.target = source, target
        self.source_lang, self.target_lang = source_lang, target_lang
        self.eos_id = eos_id
        self.model_id = model_id
        self.duplicate_batch_width = duplicate_batch_width

    def info(self) -> dict:
        info = dict(self.engine.info())
        info.update(model=self.model_id, supports_batching=True)
        return info

    def is_ready(self) -> bool:
        return self.engine.is_ready()

    def translate_batch(self, inputs: list[TranslationInput]) -> list[TranslationOutput]:
        return translate_with_engine(self.token_engine, self.source, self.target, self.source_lang,
                                     self.target_lang, self.eos_id, inputs, max_padded_cells=0,
                                     max_engine_batch=4096)

    def translate_batch_with_repetitions(self, inputs, repetitions) -> list[TranslationOutput]:
        """One output per logical input; input i runs as min(repetitions[i],
        duplicate_batch_width) physical inputs (backend.rs:25-37)."""
        if len(inputs) != len(repetitions) or any(int(r) <= 0 for r in repetitions):
            raise InvalidInput("logical batch repetitions are malformed")
        physical, first = [], []
        for inp, r in zip(inputs, repetitions):
            first.append(len(physical))
            physical.extend([inp] * min(int(r), self.duplicate_batch_width))
        outs = self.translate_batch(physical)
        if len(outs) != len(physical):
            raise InferenceError(f"HIP backend returned {len(outs)} outputs for {len(physical)} rows")
        return [outs[i] for i in first]
