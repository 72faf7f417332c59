"""marian_hip_engine_create rejects invalid models before it touches the device.

The reference refuses these at load time: a -128 weight or a multiplier that is
not finite and positive (Q8Linear::new, crates/marian-cpu/src/q8_gemm.rs:96-110,
validate_quant_mult :592-600; the intgemm8 loader, legacy_q8.rs:384-395).  The
engine also refuses geometries its kernels do not run.  These tests need no
GPU: a model that passed validation would go on to select the device, which
fails here with a device error instead of the model error asserted.
"""

import copy

import numpy as np
import pytest


@pytest.fixture(scope="module")
def tiny(pkg):
    g = pkg.Geometry(vocab=96, dim=128, heads=2, ffn_dim=256, encoder_layers=1, decoder_layers=1)
    return pkg.seeded_model(seed=3, geometry=g)


def rejected(pkg, model, needle):
    with pytest.raises(pkg.ModelError) as ei:
        pkg.HipEngine(model)
    assert needle in str(ei.value), str(ei.value)


@pytest.mark.parametrize("where", [("encoder", 0, "qkv"), ("encoder", 0, "ffn2"),
                                   ("decoder", 0, "self_out"), ("decoder", 0, "cross_kv"),
                                   ("decoder", 0, "ffn1")])
@pytest.mark.parametrize("bad", [0.0, -1.0, float("nan"), float("inf")])
def test_layer_multiplier_must_be_finite_and_positive(pkg, tiny, where, bad):
    m = copy.deepcopy(tiny)
    part, idx, name = where
    getattr(m, part)[idx][name]["mult"][5] = bad
    rejected(pkg, m, "multiplier")


@pytest.mark.parametrize("where", [("encoder", 0, "out"), ("decoder", 0, "cross_q"),
                                   ("decoder", 0, "ffn2")])
def test_layer_weight_minus_128_is_rejected(pkg, tiny, where):
    m = copy.deepcopy(tiny)
    part, idx, name = where
    getattr(m, part)[idx][name]["weight"][3, 7] = -128
    rejected(pkg, m, "[-127, 127]")


def test_embedding_checks(pkg, tiny):
    m = copy.deepcopy(tiny)
    m.embedding[10, 0] = -128
    rejected(pkg, m, "embedding")
    m = copy.deepcopy(tiny)
    m.embedding_mult[0] = 0.0
    rejected(pkg, m, "embedding")


@pytest.mark.parametrize("geom,needle", [
    (dict(dim=576, heads=9), "heads"),          # 9 heads: more than the kernels hold
    (dict(dim=100, heads=2), "heads"),          # head width 50
    (dict(dim=256, heads=8), "heads"),          # head width 32
    (dict(dim=576, heads=12), "heads"),         # width 48 but d > 512
    (dict(ffn_dim=96), "ffn_dim"),              # not a multiple of 64
    (dict(ffn_dim=2112), "ffn_dim"),            # above the skinny kernel's K
    (dict(decoder_layers=0), "decoder layer"),  # nothing for the vocabulary to score
])
def test_unsupported_geometry_is_a_model_error(pkg, geom, needle):
    g = dict(vocab=96, dim=128, heads=2, ffn_dim=256, encoder_layers=1, decoder_layers=1)
    g.update(geom)
    m = pkg.seeded_model(seed=4, geometry=pkg.Geometry(**g))
    rejected(pkg, m, needle)


def test_valid_tiny_model_passes_validation(pkg, tiny):
    # A valid model gets past validation to device selection: on a machine
    # without a GPU that is a device error, never a model error.
    if pkg._lib.load().marian_hip_device_count() > 0:
        pytest.skip("a GPU is visible: the engine would be created")
    with pytest.raises(pkg.DeviceError):
        pkg.HipEngine(tiny)


# ---- the Transformer-SSRU graph (marian_hip_engine_create_ssru) ----
@pytest.fixture(scope="module")
def tiny_ssru(pkg):
    g = pkg.SsruGeometry(source_vocab=90, target_vocab=96, dim=128, heads=2, ffn_dim=256,
                         encoder_layers=1, decoder_layers=1)
    return pkg.seeded_ssru_model(seed=3, geometry=g)


@pytest.mark.parametrize("where", [("encoder", 0, "wk"), ("decoder", 0, "ssru_wf"),
                                   ("decoder", 0, "wv"), ("decoder", 0, "w2")])
@pytest.mark.parametrize("field", ["act_mult", "weight_mult"])
@pytest.mark.parametrize("bad", [0.0, -2.0, float("nan"), float("inf")])
def test_ssru_multipliers_must_be_finite_and_positive(pkg, tiny_ssru, where, field, bad):
    m = copy.deepcopy(tiny_ssru)
    part, idx, name = where
    getattr(m, part)[idx][name][field] = bad
    rejected(pkg, m, "multiplier")


def test_ssru_weight_and_table_checks(pkg, tiny_ssru):
    m = copy.deepcopy(tiny_ssru)
    m.decoder[0]["ssru_w"]["weight"][1, 2] = -128
    rejected(pkg, m, "[-127, 127]")
    m = copy.deepcopy(tiny_ssru)
    m.encoder_embedding[5, 5] = -128
    rejected(pkg, m, "encoder embedding")
    m = copy.deepcopy(tiny_ssru)
    m.decoder_embedding_mult = 0.0
    rejected(pkg, m, "decoder embedding")
    m = copy.deepcopy(tiny_ssru)
    m.output_act_mult = float("nan")
    rejected(pkg, m, "output multiplier")
    m = copy.deepcopy(tiny_ssru)
    m.decoder[0]["context_ln"]["scale"] = None
    rejected(pkg, m, "LayerNorm")


@pytest.mark.parametrize("geom,needle", [
    (dict(dim=576, heads=12), "heads"),
    (dict(ffn_dim=100), "ffn_dim"),
    (dict(decoder_layers=0), "decoder layer"),
])
def test_ssru_unsupported_geometry_is_a_model_error(pkg, geom, needle):
    g = dict(source_vocab=90, target_vocab=96, dim=128, heads=2, ffn_dim=256, encoder_layers=1,
             decoder_layers=1)
    g.update(geom)
    m = pkg.seeded_ssru_model(seed=4, geometry=pkg.SsruGeometry(**g))
    rejected(pkg, m, needle)


def test_valid_tiny_ssru_model_passes_validation(pkg, tiny_ssru):
    if pkg._lib.load().marian_hip_device_count() > 0:
        pytest.skip("a GPU is visible: the engine would be created")
    with pytest.raises(pkg.DeviceError):
        pkg.HipEngine(tiny_ssru)
