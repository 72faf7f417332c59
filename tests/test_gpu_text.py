"""GPU: the text-level backend (HipTextBackend: segmentation, EOS, the shared
output budget, shortlist candidates) over the HIP engine gives the same texts
and token counts as the same text flow over the oracle, for the
Transformer-SSRU graph with a lexical shortlist and for the transformer graph
over the full vocabulary; repetitions do not change an output."""

import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class HashTokenizer:
    def __init__(self, vocab):
        self.V = vocab

    def vocabulary_size(self):
        return self.V

    def encode(self, s):
        return [3 + (sum(map(ord, w)) * 31 + len(w)) % (self.V - 3) for w in s.split()]

    def decode(self, ids):
        return " ".join(f"w{i}" for i in ids)


class OracleEngine:
    """Token engine over the oracle (test only)."""

    def __init__(self, orc, om, limits, ssru, shortlist=None):
        self.orc, self.om, self.limits, self.ssru, self.shortlist = orc, om, limits, ssru, shortlist

    def translate_token_ids(self, tokens, offsets, limits):
        if self.ssru:
            kw = {}
            if self.shortlist is not None:
                lists = [self.shortlist.candidates(tokens[offsets[b]:offsets[b + 1]])
                         for b in range(len(offsets) - 1)]
                flat = np.concatenate(lists).astype(np.uint32)
                coff = np.zeros(len(lists) + 1, np.uint32)
                coff[1:] = np.cumsum([len(c) for c in lists])
                kw = dict(candidates=flat, candidate_offsets=coff)
            rows = self.orc.translate_ssru(self.om, tokens, offsets, limits, self.limits, threads=16, **kw)
        else:
            rows = self.orc.translate(self.om, tokens, offsets, limits, self.limits, threads=16)
        offs = np.zeros(len(rows) + 1, np.uint32)
        offs[1:] = np.cumsum([len(r) for r in rows])
        return type("B", (), {"tokens": [t for r in rows for t in r], "offsets": offs.tolist()})()


def inputs(text, n=12, budget=60):
    rng = np.random.default_rng(5)
    out = []
    for i in range(n):
        k = int(rng.integers(3, 40))
        words = " ".join(f"w{int(x)}" for x in rng.integers(0, 500, size=k))
        body = f"{words}. Next {i}?" if i % 3 else f"{words}\r\n\r\n{words[:20]}!"
        out.append(text.TranslationInput(body, "en", "de", budget if i % 4 else 7))
    out.append(text.TranslationInput(" ".join(f"long{i % 57}" for i in range(400)), "en", "de", budget))
    out.append(text.TranslationInput("  \n ", "en", "de", budget))
    return out


def test_text_backend_ssru_with_shortlist(pkg, orc):
    text = importlib.import_module(pkg.__name__ + ".text")
    sl = importlib.import_module(pkg.__name__ + ".shortlist")
    g = pkg.SsruGeometry(source_vocab=3000, target_vocab=3200, encoder_layers=2, decoder_layers=2)
    model = pkg.seeded_ssru_model(seed=51, geometry=g, std=0.05)
    rng = np.random.default_rng(9)
    targets = rng.integers(0, g.target_vocab, size=16 * g.source_vocab).astype(np.uint32)
    shortlist = sl.LexicalShortlist.from_bytes(
        sl.LexicalShortlist.to_bytes(60, np.arange(g.source_vocab + 1, dtype=np.uint64) * 16, targets),
        g.source_vocab, g.target_vocab)
    tok = HashTokenizer(3000)
    ins = inputs(text)
    want = text.translate_with_engine(OracleEngine(orc, orc.OracleSsruModel(model), pkg.LIFTED_LIMITS, True,
                                                   shortlist), tok, tok, "en", "de", 0, ins)
    with pkg.HipEngine(model, limits=pkg.LIFTED_LIMITS) as e:
        be = text.HipTextBackend(e, tok, tok, "en", "de", eos_id=0, shortlist=shortlist,
                                 duplicate_batch_width=3)
        got = be.translate_batch(ins)
        rep = be.translate_batch_with_repetitions(ins, [1 + (i % 4) for i in range(len(ins))])
        print(f"{sum(o.output_tokens for o in got)} output tokens, "
              f"{sum(o.input_tokens for o in got)} input tokens", flush=True)
        assert got == want
        assert rep == want
        assert be.is_ready()


def test_text_backend_transformer_full_vocabulary(pkg, orc, small_model):
    text = importlib.import_module(pkg.__name__ + ".text")
    tok = HashTokenizer(small_model.geometry.vocab)
    ins = inputs(text, n=20)
    want = text.translate_with_engine(OracleEngine(orc, orc.OracleModel(small_model), pkg.LIFTED_LIMITS,
                                                   False), tok, tok, "en", "de", 0, ins)
    with pkg.HipEngine(small_model, limits=pkg.LIFTED_LIMITS) as e:
        got = text.HipTextBackend(e, tok, tok, "en", "de", eos_id=0).translate_batch(ins)
        print(f"{sum(o.output_tokens for o in got)} output tokens", flush=True)
        assert got == want
