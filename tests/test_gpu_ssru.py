"""GPU parity for the reference's own graph: Transformer encoder + SSRU decoder
with static per-tensor activation multipliers (marian_hip_engine_create_ssru),
and shortlisted scoring (marian_hip_translate_shortlisted) on both graphs.

Every case is compared with the oracle (oracle_translate_ssru /
oracle_translate_shortlisted) token for token; the probe cases also compare
the encoder states and one step's logits bit for bit.  The geometries cover
the reference's supported shape (d = 384, 8 heads of 48, FFN 1536, 6 encoder
and 4 SSRU decoder layers, crates/marian-model/src/manifest.rs:27-36), a
64-wide-head shape, layers whose inputs share one static multiplier (one
quantization and one fused GEMM per group) and layers that do not (one per
layer), and candidate lists from a lexical shortlist.
"""

import importlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ORACLE_THREADS = 16


@pytest.fixture(scope="module")
def sl(pkg):
    return importlib.import_module(pkg.__name__ + ".shortlist")


def shortlist_lists(sl, toks, offs, Vs, Vt, per_source=12, first=40, seed=3):
    """A random lexical shortlist and the candidate lists of the batch."""
    rng = np.random.default_rng(seed)
    targets = rng.integers(0, Vt, size=per_source * Vs).astype(np.uint32)
    offsets = np.arange(Vs + 1, dtype=np.uint64) * per_source
    s = sl.LexicalShortlist.from_bytes(sl.LexicalShortlist.to_bytes(first, offsets, targets), Vs, Vt)
    return sl.pack_candidates([s.candidates(toks[offs[b]:offs[b + 1]]) for b in range(len(offs) - 1)])


def run_both(pkg, orc, engine, om, b, flags, cand=None, coff=None):
    got = engine.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, flags,
                                     candidates=cand, candidate_offsets=coff).rows()
    want = orc.translate_ssru(om, b.tokens, b.offsets, b.max_output_tokens, b.limits, flags,
                              candidates=cand, candidate_offsets=coff, threads=ORACLE_THREADS)
    return got, want


SHAPES = {
    "d384-dh48": dict(dim=384, heads=8, ffn_dim=1536),
    "d256-dh64": dict(dim=256, heads=4, ffn_dim=1024),
    "d384-dh64": dict(dim=384, heads=6, ffn_dim=1536),
    "d512-dh64": dict(dim=512, heads=8, ffn_dim=2048),
    "d128-dh64": dict(dim=128, heads=2, ffn_dim=512),
    "d192-dh48": dict(dim=192, heads=4, ffn_dim=768),
}


@pytest.mark.parametrize("shared", [True, False], ids=["shared-mults", "own-mults"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_ssru_engine_token_exact(pkg, orc, sl, shape, shared):
    g = pkg.SsruGeometry(source_vocab=3000, target_vocab=3200, encoder_layers=2, decoder_layers=2,
                         **SHAPES[shape])
    model = pkg.seeded_ssru_model(seed=31, geometry=g, std=0.05, shared_input_mults=shared)
    om = orc.OracleSsruModel(model)
    b = pkg.ragged_batch(seed=19, n=12, vocab=g.source_vocab)
    cand, coff, _ = shortlist_lists(sl, b.tokens, b.offsets, g.source_vocab, g.target_vocab)
    with pkg.HipEngine(model, limits=b.limits) as e:
        for name, c, co in (("full vocabulary", None, None), ("shortlist", cand, coff)):
            got, want = run_both(pkg, orc, e, om, b, 0, c, co)
            print(f"{shape} {'shared' if shared else 'own'} {name}: {sum(map(len, got))} tokens",
                  flush=True)
            assert got == want
        assert e.is_ready()


@pytest.mark.parametrize("step", [0, 5, 17])
def test_ssru_probe_bit_exact(pkg, orc, step):
    g = pkg.SsruGeometry(source_vocab=3000, target_vocab=3200, encoder_layers=2, decoder_layers=3)
    model = pkg.seeded_ssru_model(seed=41, geometry=g, std=0.05)
    om = orc.OracleSsruModel(model)
    b = pkg.ragged_batch(seed=23, n=9, vocab=g.source_vocab)
    lim = np.minimum(b.max_output_tokens.astype(np.int64), step + 1).astype(np.uint32)
    with pkg.HipEngine(model, limits=b.limits) as e:
        out, enc, lg, act = e.translate_probe(b.tokens, b.offsets, lim, pkg.FLAG_IGNORE_EOS,
                                              probe_step=step)
    rows, enc_o, lg_o, act_o = orc.translate_ssru(om, b.tokens, b.offsets, lim, b.limits,
                                                  pkg.FLAG_IGNORE_EOS, probe_step=step,
                                                  threads=ORACLE_THREADS)
    print(f"step {step}: {int(act.sum())} active rows", flush=True)
    assert out.rows() == rows
    assert np.array_equal(act, act_o)
    assert np.array_equal(enc.view(np.uint32), enc_o.view(np.uint32))
    assert np.array_equal(lg[act_o].view(np.uint32), lg_o[act_o].view(np.uint32))


def test_ssru_long_sentences_token_exact(pkg, orc):
    """Sentences longer than 128 tokens and an FFN width that is not a
    multiple of 128: every step's SSRU LayerNorm, query projection and
    cross-attention run as separate kernels (the fused decode block holds at
    most 128 encoder keys per row), and so do the residual LayerNorms and the
    linears that read them (the fused LayerNorm + linear kernel takes 128
    output columns per workgroup).  The other cases use the fused kernels.
    Both read the recurrent state of step t from one buffer and write it to
    the other."""
    g = pkg.SsruGeometry(source_vocab=3000, target_vocab=3200, encoder_layers=2, decoder_layers=2,
                         ffn_dim=960)
    model = pkg.seeded_ssru_model(seed=37, geometry=g, std=0.05)
    om = orc.OracleSsruModel(model)
    rng = np.random.default_rng(13)
    seqs = [rng.integers(3, g.source_vocab, size=L).astype(np.int32) for L in (150, 12, 131, 40)]
    b = pkg.synthetic._pack("long", seqs, [30, 9, 25, 20], 0, dict(pkg.synthetic.LIFTED_LIMITS))
    with pkg.HipEngine(model, limits=b.limits) as e:
        got, want = run_both(pkg, orc, e, om, b, pkg.FLAG_IGNORE_EOS)
        print(f"long sentences: {sum(map(len, got))} tokens", flush=True)
        assert got == want
        assert e.is_ready()


def test_ssru_many_rows_token_exact(pkg, orc, sl):
    """200 sentences: the fused SSRU kernels over 25 row groups and 800
    (row, head) workgroups, with the active set shrinking step by step."""
    g = pkg.SsruGeometry(source_vocab=3000, target_vocab=3200, encoder_layers=1, decoder_layers=2,
                         dim=256, heads=4, ffn_dim=1024)
    model = pkg.seeded_ssru_model(seed=43, geometry=g, std=0.05)
    om = orc.OracleSsruModel(model)
    b = pkg.ragged_batch(seed=31, n=200, vocab=g.source_vocab)
    cand, coff, _ = shortlist_lists(sl, b.tokens, b.offsets, g.source_vocab, g.target_vocab)
    with pkg.HipEngine(model, limits=b.limits) as e:
        for name, c, co in (("full vocabulary", None, None), ("shortlist", cand, coff)):
            got, want = run_both(pkg, orc, e, om, b, 0, c, co)
            print(f"200 rows, {name}: {sum(map(len, got))} tokens", flush=True)
            assert got == want


@pytest.mark.parametrize("ffn_dim", [1536, 960], ids=["fused", "generic"])
def test_ssru_non_finite_activation_is_an_inference_error(pkg, orc, ffn_dim):
    """A decoder FFN whose weight multiplier makes its output overflow: the
    quantization of the hidden rows rejects the infinities, as the oracle's
    static quantization does (error -2); the call fails with an inference
    error and the engine stays ready.  FFN 1536 runs the fused kernels, 960
    the generic ones."""
    g = pkg.SsruGeometry(source_vocab=3000, target_vocab=3200, encoder_layers=1, decoder_layers=2,
                         ffn_dim=ffn_dim)
    model = pkg.seeded_ssru_model(seed=47, geometry=g, std=0.05)
    model.decoder[1]["w1"]["weight_mult"] = 1e-37  # acc / (act * 1e-37) overflows
    om = orc.OracleSsruModel(model)
    b = pkg.ragged_batch(seed=5, n=6, vocab=g.source_vocab)
    with pytest.raises(orc.OracleError) as ei:
        orc.translate_ssru(om, b.tokens, b.offsets, b.max_output_tokens, b.limits, 0,
                           threads=ORACLE_THREADS)
    assert ei.value.code == -2
    with pkg.HipEngine(model, limits=b.limits) as e:
        with pytest.raises(pkg.InferenceError, match="not finite"):
            e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, 0)
        assert e.is_ready()


def test_ssru_reference_shape_ragged_64(pkg, orc, sl):
    """The reference's supported shape at full size (32000-id vocabularies,
    6 encoder / 4 SSRU decoder layers) on the 64-sentence ragged batch, with
    and without a shortlist."""
    g = pkg.SsruGeometry()
    model = pkg.seeded_ssru_model(geometry=g)
    om = orc.OracleSsruModel(model)
    b = pkg.ragged_batch()
    cand, coff, _ = shortlist_lists(sl, b.tokens, b.offsets, g.source_vocab, g.target_vocab,
                                    per_source=40, first=100)
    with pkg.HipEngine(model, limits=b.limits) as e:
        for name, c, co in (("full vocabulary", None, None), ("shortlist", cand, coff)):
            got, want = run_both(pkg, orc, e, om, b, b.flags, c, co)
            print(f"reference shape, {name}: {sum(map(len, got))} tokens", flush=True)
            assert got == want


def test_transformer_engine_shortlisted(pkg, orc, sl, small_model):
    """Candidate scoring on the transformer graph (dynamic multipliers), at
    step row counts that use the fused decode kernels and the generic ones."""
    g = small_model.geometry
    om = orc.OracleModel(small_model)
    b = pkg.ragged_batch(seed=29, n=40, vocab=g.vocab)
    cand, coff, _ = shortlist_lists(sl, b.tokens, b.offsets, g.vocab, g.vocab)
    with pkg.HipEngine(small_model, limits=b.limits) as e:
        got = e.translate_token_ids(b.tokens, b.offsets, b.max_output_tokens, b.flags,
                                    candidates=cand, candidate_offsets=coff).rows()
        want = orc.translate_shortlisted(om, b.tokens, b.offsets, b.max_output_tokens, b.limits,
                                         cand, coff, b.flags, threads=ORACLE_THREADS)
        print(f"transformer shortlisted: {sum(map(len, got))} tokens", flush=True)
        assert got == want
        assert e.is_ready()


def test_shortlisted_input_errors_keep_the_engine_ready(pkg, small_model):
    b = pkg.ragged_batch(seed=3, n=2, vocab=small_model.geometry.vocab)
    with pkg.HipEngine(small_model, limits=b.limits) as e:
        with pytest.raises(pkg.InvalidInput, match="empty candidate"):
            e.translate_token_ids(b.tokens, b.offsets, [4, 4], candidates=[0, 5],
                                  candidate_offsets=[0, 2, 2])
        with pytest.raises(pkg.InvalidInput, match="exceeds vocabulary"):
            e.translate_token_ids(b.tokens, b.offsets, [4, 4], candidates=[0, 5, 2048],
                                  candidate_offsets=[0, 2, 3])
        with pytest.raises(pkg.InvalidInput, match="not strictly ascending"):
            e.translate_token_ids(b.tokens, b.offsets, [4, 4], candidates=[5, 0, 2],
                                  candidate_offsets=[0, 2, 3])
        assert e.is_ready()
        out = e.translate_token_ids(b.tokens, b.offsets, [4, 4], pkg.FLAG_IGNORE_EOS,
                                    candidates=[7, 9], candidate_offsets=[0, 1, 2]).rows()
        assert out == [[7] * 4, [9] * 4]
