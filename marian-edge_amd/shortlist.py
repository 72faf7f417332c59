"""Lexical shortlist: the per-sentence candidate ids the output scoring runs over.

Host-side restatement of crates/marian-model/src/shortlist.rs (the reference
builds candidates on the CPU too): the binary format of `from_bytes`
(:55-139: a 48-byte header with the magic, firstNum, the offset and target
counts, then u64 offsets[source_vocab + 1] and u32 targets) and
`candidates` (:150-198).  The candidate list feeds
marian_hip_candidate_argmax (`device.candidate_argmax`), which scores only
those ids on the GPU.
"""

from __future__ import annotations

import struct

import numpy as np

MAGIC = 17_373_278_592_220_534_773
MAX_TARGET_ENTRIES = 4_000_000


class ShortlistError(ValueError):
    pass


class LexicalShortlist:
    def __init__(self, source_vocab: int, target_vocab: int, first_num: int = 0,
                 offsets=None, targets=None):
        self.source_vocab = int(source_vocab)
        self.target_vocab = int(target_vocab)
        self.first_num = int(first_num)
        self.offsets = np.zeros(0, np.int64) if offsets is None else np.asarray(offsets, np.int64)
        self.targets = np.zeros(0, np.uint32) if targets is None else np.asarray(targets, np.uint32)

    @classmethod
    def from_bytes(cls, data: bytes | None, source_vocab: int, target_vocab: int) -> "LexicalShortlist":
        """shortlist.rs:55-139; None = no shortlist (every id is a candidate)."""
        if data is None:
            return cls(source_vocab, target_vocab)
        max_bytes = 48 + (source_vocab + 1) * 8 + MAX_TARGET_ENTRIES * 4
        if len(data) > max_bytes:
            raise ShortlistError(f"lexical shortlist has {len(data)} bytes; maximum is {max_bytes}")
        if len(data) < 48:
            raise ShortlistError("truncated lexical shortlist header")
        magic, _, first_num, _, offset_count, target_count = struct.unpack_from("<6Q", data, 0)
        if (magic != MAGIC or offset_count != source_vocab + 1 or first_num > target_vocab
                or target_count > MAX_TARGET_ENTRIES):
            raise ShortlistError("unsupported lexical shortlist format")
        expected = 48 + offset_count * 8 + target_count * 4
        if len(data) != expected:
            raise ShortlistError(f"lexical shortlist has {len(data)} bytes, expected {expected}")
        offsets = np.frombuffer(data, "<u8", offset_count, 48).astype(np.int64)
        if (offsets[0] != 0 or offsets[-1] != target_count or np.any(np.diff(offsets) < 0)):
            raise ShortlistError("lexical shortlist offsets are invalid")
        targets = np.frombuffer(data, "<u4", target_count, 48 + offset_count * 8).astype(np.uint32)
        bad = targets >= target_vocab
        if bad.any():
            raise ShortlistError(f"lexical shortlist target {int(targets[bad][0])} exceeds "
                                 f"vocabulary {target_vocab}")
        return cls(source_vocab, target_vocab, first_num, offsets, targets)

    @staticmethod
    def to_bytes(first_num: int, offsets, targets) -> bytes:
        """The binary layout from_bytes reads (for tests and tools)."""
        head = struct.pack("<6Q", MAGIC, 0, first_num, 0, len(offsets), len(targets))
        return (head + np.asarray(offsets, "<u8").tobytes() + np.asarray(targets, "<u4").tobytes())

    def candidates(self, tokens) -> np.ndarray:
        """shortlist.rs:150-198: the ids a sentence's output may use, ascending."""
        present = np.full(self.target_vocab, self.offsets.size == 0, bool)
        if self.offsets.size:
            present[:self.first_num] = True
            for t in tokens:
                t = int(t)
                if t < 0:
                    raise ShortlistError("source token ID is negative")
                if t >= self.source_vocab:
                    raise ShortlistError(f"source token {t} exceeds vocabulary {self.source_vocab}")
                present[self.targets[self.offsets[t]:self.offsets[t + 1]]] = True
        # The generation mask: UNK and the byte/control ids never become output.
        if self.target_vocab > 1:
            present[1] = False
        if self.target_vocab > 7:
            present[7:min(self.target_vocab, 39)] = False
        cands = list(np.flatnonzero(present))
        # Padded with the lowest absent ids from 50 up to a multiple of 8.
        for i in range(50, self.target_vocab):
            if len(cands) % 8 == 0:
                break
            if not present[i]:
                cands.append(i)
        cands = np.array(sorted(cands), np.uint32)
        if cands.size == 0:
            raise ShortlistError("lexical shortlist produced no candidates")
        if cands[0] != 0:
            raise ShortlistError("lexical shortlist does not contain EOS token 0")
        return cands


def pack_candidates(lists) -> tuple[np.ndarray, np.ndarray, int]:
    """Concatenated candidate lists, their offsets [B + 1] and the longest length."""
    offs = np.zeros(len(lists) + 1, np.uint32)
    offs[1:] = np.cumsum([len(c) for c in lists])
    flat = np.concatenate(lists).astype(np.uint32) if lists else np.zeros(0, np.uint32)
    return flat, offs, int(max((len(c) for c in lists), default=0))
