"""Host-side logic of HipBackend (no GPU): repetitions -> physical rows.

translate_batch_with_repetitions (crates/marian-core/src/backend.rs:25-37) must
return one output per logical input; the Metal backend expands repeated
inputs into physical rows up to its duplicate width and maps the outputs back
(crates/marian-metal/src/backend.rs:319-354).  A stub engine records the
packed batch it receives.
"""

import numpy as np
import pytest


class StubEngine:
    def __init__(self, pkg, warmup_error=None):
        self.pkg = pkg
        self.calls = []
        self.warmups = 0
        self.warmup_error = warmup_error

    def warmup(self):
        self.warmups += 1
        if self.warmup_error:
            raise self.warmup_error

    def translate_token_ids(self, toks, offs, limits, flags=0):
        self.calls.append((np.asarray(toks).copy(), np.asarray(offs).copy(), list(limits), flags))
        rows = [list(toks[offs[i]:offs[i + 1]])[::-1] for i in range(len(offs) - 1)]
        tokens = np.array([t for r in rows for t in r], np.int32)
        out_offs = np.zeros(len(rows) + 1, np.uint32)
        out_offs[1:] = np.cumsum([len(r) for r in rows])
        return self.pkg.BatchOutput(tokens, out_offs)


def test_repetitions_expand_to_physical_rows(pkg):
    eng = StubEngine(pkg)
    be = pkg.HipBackend(eng, duplicate_batch_width=2)
    sents = [[5, 6], [7], [8, 9, 10]]
    out = be.translate_token_batch(sents, [4, 4, 4], repetitions=[1, 3, 2])
    assert out == [[6, 5], [7], [10, 9, 8]]
    toks, offs, limits, _ = eng.calls[-1]
    # input 1 repeated 3 times but capped at width 2; input 2 twice
    assert np.diff(offs).tolist() == [2, 1, 1, 3, 3]
    assert limits == [4, 4, 4, 4, 4]


def test_default_width_materializes_no_copies(pkg):
    eng = StubEngine(pkg)
    be = pkg.HipBackend(eng)
    out = be.translate_token_batch([[5, 6], [7]], [3, 3], repetitions=[4, 9])
    assert out == [[6, 5], [7]]
    assert np.diff(eng.calls[-1][1]).tolist() == [2, 1]


@pytest.mark.parametrize("reps", [[1], [1, 0], [1, -2]])
def test_malformed_repetitions_are_invalid_input(pkg, reps):
    be = pkg.HipBackend(StubEngine(pkg))
    with pytest.raises(pkg.InvalidInput):
        be.translate_token_batch([[5], [6]], [1, 1], repetitions=reps)


def test_backend_warms_its_engine_up_once_at_load(pkg):
    """Q8CpuBackend warms its engine at load (crates/marian-cpu/src/backend.rs:810-813)."""
    eng = StubEngine(pkg)
    be = pkg.HipBackend(eng)
    assert eng.warmups == 1
    be.translate_token_batch([[5]], [2])
    assert eng.warmups == 1 and len(eng.calls) == 1


def test_warmup_failure_is_an_inference_error(pkg):
    with pytest.raises(pkg.InferenceError, match="HIP warmup failed"):
        pkg.HipBackend(StubEngine(pkg, warmup_error=pkg.DeviceError("no device")))
