"""Text-side callers: segment_text and translate_with_engine.

The segmentation tests are the reference's own (crates/marian-cpu/tests/
segmenter.rs), restated against marian_edge_amd.text with the same inputs,
piece counters and expectations; the budget test is the reference's
`segmented_text_shares_one_original_output_budget`
(crates/marian-cpu/src/backend.rs:1104-1128).  The pipeline tests run the
text flow over the oracle as token engine (CPU) and check what the
reference's text flow guarantees: lossless reassembly with separators kept
outside the model, segments within 255 pieces plus EOS, and one output budget
shared across an input's segments in order."""

import importlib

import numpy as np
import pytest


@pytest.fixture(scope="module")
def text(pkg):
    return importlib.import_module(pkg.__name__ + ".text")


def word_pieces(s):
    return len(s.split())


def scalar_pieces(s):
    return sum(1 for c in s if not c.isspace())


def rebuilt(t, segs):
    return "".join(s.content(t) + s.separator(t) for s in segs)


def test_short_text_stays_in_one_lossless_segment(text):
    t = "Hello world.  \r\n"
    segs = text.segment_text(t, 255, word_pieces)
    assert len(segs) == 1
    assert segs[0].content(t) == "Hello world."
    assert segs[0].separator(t) == "  \r\n"
    assert segs[0].full_range() == range(0, len(t.encode()))
    assert rebuilt(t, segs) == t


def test_abbreviations_decimals_versions_domains_emails_do_not_split(text):
    prefix = "Dr. Smith used e.g. version 1.2.3 at example.com and a.b@example.org. "
    t = prefix + "word " * 260 + " End."
    segs = text.segment_text(t, 255, word_pieces)
    assert segs[0].content(t) == prefix.rstrip()
    assert not any(s.content(t) in ("Dr.", "e.g.", "version 1.2.", "example.", "a.b@example.")
                   for s in segs)
    assert rebuilt(t, segs) == t
    assert all(s.source_pieces <= 255 for s in segs)


def test_quotes_cjk_terminators_crlf_and_blank_lines(text):
    t = "word " * 256 + " \r\n\r\nHe asked, \"Ready?!\"  中文句子。\n下一句！  Final…”"
    segs = text.segment_text(t, 255, word_pieces)
    assert rebuilt(t, segs) == t
    assert all(s.source_pieces <= 255 for s in segs)
    assert any(s.separator(t) == "  \r\n\r\n" for s in segs)
    assert any(s.content(t).endswith("Ready?!\"") for s in segs)
    assert any(s.content(t).endswith("中文句子。") for s in segs)


def test_short_multiline_text_keeps_separators_outside(text):
    t = "Line one.\nLine two?\r\nLine three!"
    segs = text.segment_text(t, 255, word_pieces)
    assert [s.separator(t) for s in segs] == ["\n", "\r\n", ""]
    assert rebuilt(t, segs) == t


def test_seven_hundred_tokens_split_at_preferred_boundaries(text):
    t = " ".join(f"token{i}" for i in range(700))
    segs = text.segment_text(t, 255, word_pieces)
    assert [s.source_pieces for s in segs] == [255, 255, 190]
    assert rebuilt(t, segs) == t


@pytest.mark.parametrize("delim", [";", ":", "/", " —", " --", ","])
def test_falls_back_through_punctuation(text, delim):
    t = "a" * 140 + delim + " " + "b" * 140 + delim + " " + "c" * 40
    segs = text.segment_text(t, 150, scalar_pieces)
    assert rebuilt(t, segs) == t
    assert segs[0].content(t).endswith(delim.lstrip())


def test_falls_back_to_utf8_scalars(text):
    t = "界" * 260 + "🙂" * 260 + "文" * 180
    segs = text.segment_text(t, 255, scalar_pieces)
    b = t.encode()
    assert len(segs) == 3
    assert rebuilt(t, segs) == t

    def boundary(i):
        return i == len(b) or (b[i] & 0xC0) != 0x80

    assert all(s.source_pieces <= 255 and boundary(s.content_range.start) and
               boundary(s.content_range.stop) for s in segs)


def test_leading_period_and_leading_newline_remain_lossless(text):
    t = "\r\n. Hidden start. " + "x" * 300
    segs = text.segment_text(t, 100, scalar_pieces)
    assert rebuilt(t, segs) == t
    assert all(s.source_pieces <= 100 for s in segs)


@pytest.mark.parametrize("pieces,expected", [(254, 1), (255, 1), (256, 2)])
def test_exact_piece_limit_boundaries(text, pieces, expected):
    t = " ".join(["x"] * pieces)
    segs = text.segment_text(t, 255, word_pieces)
    assert len(segs) == expected
    assert all(s.source_pieces <= 255 for s in segs)
    assert rebuilt(t, segs) == t


def test_whitespace_only_input(text):
    t = " \t\r\n\n "
    segs = text.segment_text(t, 255, word_pieces)
    assert len(segs) == 1
    assert segs[0].content(t) == "" and segs[0].separator(t) == t and segs[0].source_pieces == 0


def test_rejects_zero_limit_encoder_failure_and_unsplitable_scalar(text):
    with pytest.raises(text.SegmentError) as e:
        text.segment_text("text", 0, word_pieces)
    assert e.value.kind == "ZeroPieceLimit"

    def broken(_):
        raise RuntimeError("broken model")

    with pytest.raises(text.SegmentError) as e:
        text.segment_text("bad", 3, broken)
    assert e.value.kind == "Encoding" and e.value.fields["start"] == 0 and e.value.fields["end"] == 3
    with pytest.raises(text.SegmentError) as e:
        text.segment_text("🙂🙂", 1, lambda s: 2 * len(s))
    assert e.value.kind == "UnsplitableScalar"
    assert e.value.fields == dict(start=0, end=4, pieces=2, maximum=1)


def test_enforces_input_and_segment_safety_limits(text):
    with pytest.raises(text.SegmentError) as e:
        text.segment_text("x" * (text.MAX_SEGMENTER_INPUT_BYTES + 1), 255, scalar_pieces)
    assert e.value.kind == "InputTooLarge"
    with pytest.raises(text.SegmentError) as e:
        text.segment_text("x" * (text.MAX_SEGMENTS + 1), 1, scalar_pieces)
    assert e.value.kind in ("TooManySegments", "EncodingWorkLimit")


def test_rust_whitespace_not_python_isspace(text):
    # U+001F is whitespace to Python's isspace but not to Rust's char::is_whitespace:
    # it is content, not a separator.
    t = "a\x1fb"
    segs = text.segment_text(t, 255, lambda s: len(s))
    assert segs[0].content(t) == t


# ---- translate_with_engine ----
class WordTokenizer:
    """The reference test's tokenizer: every word is id 2, decode gives one x per id."""

    def vocabulary_size(self):
        return 32

    def encode(self, s):
        return [2] * len(s.split())

    def decode(self, ids):
        return "x" * len(ids)


class LimitEngine:
    """Emits min(limit, 2) tokens of id 7 per row."""

    def translate_token_ids(self, tokens, offsets, limits):
        out, offs = [], [0]
        assert len(offsets) == len(limits) + 1
        for lim in limits:
            out += [7] * min(int(lim), 2)
            offs.append(len(out))
        return type("B", (), {"tokens": out, "offsets": offs})()


def test_segmented_text_shares_one_original_output_budget(text):
    first = text.TranslationInput("One. Two.", "en", "zh", max_output_tokens=1)
    second = text.TranslationInput("Three. Four.", "en", "zh", max_output_tokens=1)
    outs = text.translate_with_engine(LimitEngine(), WordTokenizer(), WordTokenizer(), "en", "zh", 0,
                                      [first, second])
    assert [o.text for o in outs] == ["x ", "x "]
    assert [o.output_tokens for o in outs] == [1, 1]


def test_direction_and_empty_inputs(text):
    assert text.translate_with_engine(LimitEngine(), WordTokenizer(), WordTokenizer(), "en", "zh", 0, []) == []
    with pytest.raises(text.UnsupportedDirection):
        text.translate_with_engine(LimitEngine(), WordTokenizer(), WordTokenizer(), "en", "zh", 0,
                                   [text.TranslationInput("a", "de", "zh")])


class HashTokenizer:
    """Words to ids 3..V-1 by a fixed hash; ids decode to "w<id>" joined by spaces."""

    def __init__(self, vocab):
        self.V = vocab

    def vocabulary_size(self):
        return self.V

    def encode(self, s):
        return [3 + (sum(map(ord, w)) * 31 + len(w)) % (self.V - 3) for w in s.split()]

    def decode(self, ids):
        return " ".join(f"w{i}" for i in ids)


class OracleTokenEngine:
    """The oracle as token engine (test only): oracle_translate per call."""

    def __init__(self, orc, om, limits):
        self.orc, self.om, self.limits = orc, om, limits
        self.calls = []

    def translate_token_ids(self, tokens, offsets, limits):
        self.calls.append(len(offsets) - 1)
        rows = self.orc.translate(self.om, tokens, offsets, limits, self.limits, threads=8)
        offs = np.zeros(len(rows) + 1, np.uint32)
        offs[1:] = np.cumsum([len(r) for r in rows])
        return type("B", (), {"tokens": [t for r in rows for t in r], "offsets": offs.tolist()})()


def long_inputs(text, budget):
    paragraph = " ".join(f"word{i % 97} and more{i % 13}." for i in range(120))  # > 255 pieces
    return [text.TranslationInput("Short one.", "en", "de", budget),
            text.TranslationInput(paragraph + "\r\n\r\nSecond paragraph here!", "en", "de", budget),
            text.TranslationInput("   ", "en", "de", budget)]


def test_text_flow_over_the_oracle(pkg, orc, text):
    g = pkg.Geometry(vocab=500, dim=128, heads=2, ffn_dim=256, encoder_layers=1, decoder_layers=1)
    om = orc.OracleModel(pkg.seeded_model(seed=8, geometry=g, std=0.3))
    tok = HashTokenizer(500)
    eng = OracleTokenEngine(orc, om, pkg.LIFTED_LIMITS)
    ins = long_inputs(text, 40)
    outs = text.translate_with_engine(eng, tok, tok, "en", "de", 0, ins)
    assert len(outs) == 3
    assert outs[2].text == "   " and outs[2].input_tokens == 0 and outs[2].output_tokens == 0
    assert all(o.output_tokens <= 40 for o in outs)
    assert outs[1].input_tokens > 256          # split into several segments
    assert outs[1].text.endswith("!") is False  # decoded ids, the separators kept verbatim
    assert "\r\n\r\n" in outs[1].text
    # rounds take at most one segment per input
    assert max(eng.calls) <= 3
    # every non-empty segment of input 1 spent budget in order: the output
    # tokens are the budget that was used
    assert outs[1].output_tokens <= 40


def test_budget_is_shared_in_segment_order(pkg, orc, text):
    """With IGNORE_EOS-like behaviour absent, budgets shrink by what each
    segment generated (EOS included); once spent, later segments are empty."""
    g = pkg.Geometry(vocab=500, dim=128, heads=2, ffn_dim=256, encoder_layers=1, decoder_layers=1)
    om = orc.OracleModel(pkg.seeded_model(seed=8, geometry=g, std=0.3))
    tok = HashTokenizer(500)
    for budget in (1, 3, 7):
        eng = OracleTokenEngine(orc, om, pkg.LIFTED_LIMITS)
        inp = text.TranslationInput("Alpha beta. Gamma delta. Epsilon zeta.", "en", "de", budget)
        out = text.translate_with_engine(eng, tok, tok, "en", "de", 0, [inp])[0]
        assert out.output_tokens <= budget
        # three segments, each followed by its separator
        assert out.text.count(" ") >= 2
