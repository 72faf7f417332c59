"""marian-hip: MI355X (gfx950) backend for Marian Edge's Q8 greedy translation path.

The compute lives in libmarian_hip.so (hand-written HIP kernels behind the C
ABI in include/marian_hip.h).  This package is the host-side mirror of the
reference's token-level engine interface plus synthetic-model generators.
"""

from . import _lib
from .engine import (BackendError, BatchOutput, BufferTooSmall, DeviceError, HipBackend,
                     HipEngine, InferenceError, InvalidInput, ModelError, capacity_for, make_limits,
                     validate_batch)
from .text import (HipTextBackend, HipTokenEngine, SegmentError, TextSegment, TranslationInput,
                   TranslationOutput, UnsupportedDirection, segment_text, translate_with_engine)
from .synthetic import (Batch, Geometry, LIFTED_LIMITS, REFERENCE_LIMITS, SeededModel,
                        SsruGeometry, SsruModel, attention_inputs, gemm_inputs, ragged_batch,
                        seeded_model, seeded_ssru_model, single_sentence_batch, stress_batch,
                        GEMM_SHAPES, GEMM_ROWS)

FLAG_IGNORE_EOS = _lib.FLAG_IGNORE_EOS
FLAG_NO_GENERATION_MASK = _lib.FLAG_NO_GENERATION_MASK
FLAG_FAST_REDUCTIONS = _lib.FLAG_FAST_REDUCTIONS

__all__ = [
    "BackendError", "BatchOutput", "BufferTooSmall", "DeviceError", "HipBackend", "HipEngine",
    "InferenceError", "InvalidInput", "ModelError", "make_limits", "capacity_for", "validate_batch",
    "Batch", "Geometry",
    "LIFTED_LIMITS", "REFERENCE_LIMITS", "SeededModel", "SsruGeometry", "SsruModel",
    "seeded_ssru_model", "attention_inputs", "gemm_inputs",
    "ragged_batch", "seeded_model", "single_sentence_batch", "stress_batch", "GEMM_SHAPES",
    "GEMM_ROWS", "FLAG_IGNORE_EOS", "FLAG_NO_GENERATION_MASK", "FLAG_FAST_REDUCTIONS", "load_library",
    "HipTextBackend", "HipTokenEngine", "SegmentError", "TextSegment", "TranslationInput",
    "TranslationOutput", "UnsupportedDirection", "segment_text", "translate_with_engine",
]


def load_library():
    """Loads libmarian_hip.so; raises if it is missing."""
    return _lib.load()
