"""The library's host-only batch checks (marian_hip_validate_batch), no GPU.

They are the checks the translate entry points run before touching the
device: Q8CpuEngine::validate_batch (crates/marian-cpu/src/q8_engine.rs:468-509)
and validate_work_shape (:1103-1119) with the caps as parameters, plus the
shortlisted call's candidate lists (LexicalShortlist::candidates returns them
sorted and without repeats, crates/marian-model/src/shortlist.rs:150-198; the
strict '>' scan of select_token, q8_engine.rs:770-788, picks the first maximum
in list order, which the device's lowest-id tie rule equals only on ascending
lists)."""

import numpy as np
import pytest

REF = None  # the reference's caps (NULL limits)


def check(pkg, toks, offs, limits=REF, cand=None, coff=None, vs=100, vt=100):
    pkg.validate_batch(np.asarray(toks, np.int32), np.asarray(offs, np.uint32), limits, vs, vt, cand, coff)


def test_valid_batches_pass(pkg):
    check(pkg, [5, 6, 7], [0, 2, 3])
    check(pkg, [5, 6, 7], [0, 2, 3], cand=[0, 3, 9, 1, 4], coff=[0, 3, 5])


@pytest.mark.parametrize("offs, msg", [
    ([0, 2], "invalid packed batch offsets"),          # offsets[B] != n_tokens
    ([1, 3], "invalid packed batch offsets"),          # offsets[0] != 0
    ([0], "invalid packed batch offsets"),             # no sentence
    ([0, 0, 3], "each input must contain at least one token"),
])
def test_offsets_are_checked_like_the_reference(pkg, offs, msg):
    with pytest.raises(pkg.InvalidInput, match=msg):
        check(pkg, [5, 6, 7], offs)


def test_source_ids_and_caps(pkg):
    with pytest.raises(pkg.InvalidInput, match="source token 100 is outside vocabulary 100"):
        check(pkg, [5, 100], [0, 2])
    with pytest.raises(pkg.InvalidInput, match="source token -1"):
        check(pkg, [-1, 5], [0, 2])
    # 300 tokens > the reference's 256-token source cap; lifted caps accept it
    toks, offs = [5] * 300, [0, 300]
    with pytest.raises(pkg.InvalidInput, match="source has 300 tokens; maximum is 256"):
        check(pkg, toks, offs)
    check(pkg, toks, offs, limits=dict(pkg.LIFTED_LIMITS))
    # batch * L^2 = 5 * 120^2 = 72000 > 65536 padded cells
    toks, offs = [5] * 600, np.arange(0, 601, 120)
    with pytest.raises(pkg.InvalidInput, match="padded attention work is 72000 cells"):
        check(pkg, toks, offs)
    with pytest.raises(pkg.InvalidInput, match="maximum is 256"):
        check(pkg, [5] * 257, np.arange(258))


def test_candidate_lists(pkg):
    ok = dict(cand=[0, 3, 9, 1, 4], coff=[0, 3, 5])
    check(pkg, [5, 6, 7], [0, 2, 3], **ok)
    with pytest.raises(pkg.InvalidInput, match="not strictly ascending at position 2"):
        check(pkg, [5, 6, 7], [0, 2, 3], cand=[0, 9, 3, 1, 4], coff=[0, 3, 5])
    with pytest.raises(pkg.InvalidInput, match="list 1 is not strictly ascending at position 1"):
        check(pkg, [5, 6, 7], [0, 2, 3], cand=[0, 3, 9, 4, 4], coff=[0, 3, 5])
    with pytest.raises(pkg.InvalidInput, match="empty candidate list"):
        check(pkg, [5, 6, 7], [0, 2, 3], cand=[0, 3, 9], coff=[0, 3, 3])
    with pytest.raises(pkg.InvalidInput, match="output candidate 100 exceeds vocabulary 100"):
        check(pkg, [5, 6, 7], [0, 2, 3], cand=[0, 3, 100, 1, 4], coff=[0, 3, 5])
    with pytest.raises(pkg.InvalidInput, match="invalid candidate offsets"):
        check(pkg, [5, 6, 7], [0, 2, 3], cand=[0, 3, 9, 1, 4], coff=[1, 3, 5])


def test_shortlist_candidates_pass(pkg):
    """Lists built by the restated LexicalShortlist::candidates are accepted."""
    import importlib
    sl = importlib.import_module(pkg.__name__ + ".shortlist")
    short = sl.LexicalShortlist.from_bytes(None, 100, 100)
    lists = [short.candidates([5, 6]), short.candidates([7])]
    flat, offs, _ = sl.pack_candidates(lists)
    check(pkg, [5, 6, 7], [0, 2, 3], cand=flat, coff=offs)
