"""Pins the oracle's model composition (embedding, layer wiring, decode loop).

The op-level functions of the oracle are pinned by the reference's known-answer
tests (test_oracle.py).  These tests pin how it wires them together
(crates/marian-cpu/src/q8_engine.rs:526-558 encoder layer, :410-432 context
block, :632-651 FFN, :586-630 embedding and decoder input, :749-790 scoring):

1. Closed forms.  With every int8 weight of the layers zero, each linear layer
   returns its bias, so the attention output no longer matters and a layer is
   x1 = LN1(b_o + x), x = LN2(b_2 + x1).  The float64 closed form, the
   position table and sqrt(d) included, must agree with the oracle's encoder
   output and logits to fp32 rounding.  In the decoder each step's state
   depends only on (previous token, step), so the greedy tokens follow too.
2. An independent float64 model (tests/fp64_model.py) with random weights.
   Its quantization decisions can differ from fp32 only near rounding ties,
   so it agrees with the oracle to a small tolerance; each planted wiring
   mistake (a wrong residual operand, swapped LayerNorm parameters, Q/K/V slot
   order, a missing sqrt(d), a position off by one, cross K/V from the wrong
   source, ...) moves the result far outside that tolerance.
"""

import copy

import numpy as np
import pytest

import fp64_model as F

GEOM = dict(vocab=300, dim=128, heads=2, ffn_dim=256, encoder_layers=2, decoder_layers=2)


def batch(pkg, n=5, seed=17, vocab=300):
    rng = np.random.default_rng(seed)
    lens = rng.integers(3, 14, size=n)
    seqs = [rng.integers(3, vocab, size=int(L)).astype(np.int32) for L in lens]
    offs = np.zeros(n + 1, np.uint32)
    offs[1:] = np.cumsum(lens)
    return np.concatenate(seqs), offs


def zero_layers(m):
    z = copy.deepcopy(m)
    for L in z.encoder + z.decoder:
        for name, part in L.items():
            if "weight" in part:
                part["weight"][:] = 0
    return z


def ln64(z, p):
    mean = z.mean(-1, keepdims=True)
    var = ((z - mean) ** 2).mean(-1, keepdims=True)
    return (z - mean) / np.sqrt(var + 1e-6) * p["scale"].astype(np.float64) + p["bias"].astype(np.float64)


def closed_form_encoder(m, toks, offs):
    d = m.geometry.dim
    pos = F.positions(d, 4096)
    p = np.concatenate([np.arange(offs[i + 1] - offs[i]) for i in range(len(offs) - 1)])
    x = m.embedding[toks].astype(np.float64) / m.embedding_mult[toks].astype(np.float64)[:, None]
    x = x * np.sqrt(d) + pos[p]
    for L in m.encoder:
        x1 = ln64(L["out"]["bias"].astype(np.float64) + x, L["ln1"])
        x = ln64(L["ffn2"]["bias"].astype(np.float64) + x1, L["ln2"])
    return x


def closed_form_decoder_state(m, prev, t):
    d = m.geometry.dim
    pos = F.positions(d, 4096)
    x = pos[t].copy()
    if prev >= 0:
        x += m.embedding[prev].astype(np.float64) / np.float64(m.embedding_mult[prev]) * np.sqrt(d)
    for L in m.decoder:
        x1 = ln64(L["self_out"]["bias"].astype(np.float64) + x, L["ln1"])
        x2 = ln64(L["cross_out"]["bias"].astype(np.float64) + x1, L["ln2"])
        x = ln64(L["ffn2"]["bias"].astype(np.float64) + x2, L["ln3"])
    return x


@pytest.fixture(scope="module")
def zmodel(pkg):
    return zero_layers(pkg.seeded_model(seed=9, geometry=pkg.Geometry(**GEOM), std=0.3))


def test_zero_weight_encoder_closed_form(pkg, orc, zmodel):
    toks, offs = batch(pkg)
    got = orc.encode(orc.OracleModel(zmodel), toks, offs)
    want = closed_form_encoder(zmodel, toks, offs)
    err = np.abs(got - want).max()
    print(f"zero-weight encoder: max |oracle - closed form| = {err:.2e}")
    assert err < 2e-5


def test_zero_weight_decoder_closed_form(pkg, orc, zmodel):
    toks, offs = batch(pkg, n=3)
    om = orc.OracleModel(zmodel)
    steps = 9
    # greedy tokens from the closed form: state(prev, t) -> logits -> argmax
    fm = F.Fp64Model(zmodel)
    want_rows = []
    for b in range(3):
        prev, row = -1, []
        for t in range(steps):
            lg = fm.logits(closed_form_decoder_state(zmodel, prev, t))
            prev = int(np.argmax(lg))
            row.append(prev)
        want_rows.append(row)
    got = orc.translate(om, toks, offs, [steps] * 3, pkg.LIFTED_LIMITS, flags=1)
    assert got == want_rows
    # the logits of the last step, against the closed form of its state
    seq = toks[offs[0]:offs[1]]
    lg = orc.last_step_logits(om, seq, steps, flags=0)
    want = fm.logits(closed_form_decoder_state(zmodel, want_rows[0][-2], steps - 1))
    live = np.isfinite(want)
    assert np.array_equal(np.isfinite(lg), live)
    err = np.abs(lg[live] - want[live]) / np.maximum(np.abs(want[live]), 1e-3)
    print(f"zero-weight logits: max rel err {err.max():.2e}")
    assert err.max() < 1e-5


@pytest.fixture(scope="module")
def rmodel(pkg):
    return pkg.seeded_model(seed=12, geometry=pkg.Geometry(**GEOM), std=0.3)


@pytest.fixture(scope="module")
def oracle_run(pkg, orc, rmodel):
    toks, offs = batch(pkg, n=4, seed=23)
    om = orc.OracleModel(rmodel)
    enc = orc.encode(om, toks, offs)
    steps = 6
    rows = orc.translate(om, toks, offs, [steps] * 4, pkg.LIFTED_LIMITS, flags=1)
    seq = toks[offs[1]:offs[2]]
    lg = orc.last_step_logits(om, seq, 4, flags=0)
    return toks, offs, enc, rows, lg


def fp64_run(model, toks, offs, mistake=None):
    fm = F.Fp64Model(model, mistake)
    enc = fm.encode(toks, offs)
    rows = []
    for b in range(len(offs) - 1):
        sl = slice(int(offs[b]), int(offs[b + 1]))
        r, _ = fm.decode(enc[sl], toks[sl], 6, flags=1)
        rows.append(r)
    sl = slice(int(offs[1]), int(offs[2]))
    _, lg = fm.decode(enc[sl], toks[sl], 4, flags=1, probe_step=3)
    return enc, rows, lg


# fp32 vs float64 rounding plus rare quantization flips near ties: measured
# 1.1e-6 (encoder) and 3.5e-7 (logits) on this model.
ENC_TOL = 1e-4    # encoder states are O(1) after LayerNorm
LOGIT_TOL = 1e-4  # relative, on the unmasked logits


def distance(oracle_run, fp):
    _, _, enc, rows, lg = oracle_run
    e_enc = float(np.abs(fp[0] - enc).max())
    live = np.isfinite(lg)
    e_lg = float((np.abs(fp[2][live] - lg[live]) / np.maximum(np.abs(lg[live]), 1e-2)).max())
    return e_enc, e_lg, fp[1] == rows


def test_fp64_model_agrees_with_oracle(orc, rmodel, oracle_run):
    toks, offs = oracle_run[0], oracle_run[1]
    e_enc, e_lg, same = distance(oracle_run, fp64_run(rmodel, toks, offs))
    print(f"fp64 model vs oracle: encoder {e_enc:.2e}, logits {e_lg:.2e}, tokens same {same}")
    assert e_enc < ENC_TOL and e_lg < LOGIT_TOL and same


@pytest.mark.parametrize("mistake", F.MISTAKES)
def test_planted_wiring_mistake_is_caught(orc, rmodel, oracle_run, mistake):
    toks, offs = oracle_run[0], oracle_run[1]
    e_enc, e_lg, same = distance(oracle_run, fp64_run(rmodel, toks, offs, mistake))
    print(f"{mistake}: encoder {e_enc:.2e}, logits {e_lg:.2e}, tokens same {same}")
    assert e_enc > 100 * ENC_TOL or e_lg > 100 * LOGIT_TOL
