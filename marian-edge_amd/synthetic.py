"""Seeded random-init models and synthetic workloads.

Every array is drawn from numpy.random.Generator(PCG64(seed)) in a fixed order,
so the same seed gives the same bytes on every machine with this numpy
release (2.2).  Weights are N(0, 0.02) fp32 quantized per output channel:
mult_n = 127 / max_k |w[n, k]| (fp32 division), q = clamp(rint(w * mult_n),
-127, 127) — the offline rule of the reference's Q8 artifacts
(crates/marian-cpu/tests/q8_fp32_artifact.rs:130-132) with one multiplier per
output channel instead of per tensor.  Biases are N(0, 0.02); LayerNorm scales
are 1 + N(0, 0.02) and LayerNorm biases N(0, 0.02).

Draw order: embedding [V, d], output bias [V]; then per encoder layer qkv, out,
ln1, ffn1, ffn2, ln2; then per decoder layer self_qkv, self_out, ln1, cross_q,
cross_kv, cross_out, ln2, ffn1, ffn2, ln3.  A linear draws weight then bias; a
LayerNorm draws scale then bias.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

DEFAULT_SEED = 20251201


@dataclass
class Geometry:
    vocab: int = 32000
    dim: int = 512
    heads: int = 8
    ffn_dim: int = 2048
    encoder_layers: int = 6
    decoder_layers: int = 2


def quantize_weights(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row (output channel) symmetric int8 quantization of fp32 weights."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    absmax = np.abs(w).max(axis=1)
    safe = np.where(absmax > 0, absmax, np.float32(1)).astype(np.float32)
    mult = np.where(absmax > 0, np.float32(127) / safe, np.float32(1)).astype(np.float32)
    q = np.clip(np.rint(w * mult[:, None]), -127, 127).astype(np.int8)
    return q, mult


@dataclass
class SeededModel:
    geometry: Geometry
    seed: int
    embedding: np.ndarray = field(repr=False)
    embedding_mult: np.ndarray = field(repr=False)
    output_bias: np.ndarray = field(repr=False)
    encoder: list = field(repr=False)
    decoder: list = field(repr=False)

    def weight_bytes(self) -> int:
        total = self.embedding.nbytes + self.embedding_mult.nbytes + self.output_bias.nbytes
        for layer in self.encoder + self.decoder:
            for v in layer.values():
                total += sum(a.nbytes for a in v.values())
        return total


def seeded_model(seed: int = DEFAULT_SEED, geometry: Geometry | None = None,
                 std: float = 0.02) -> SeededModel:
    """std scales every draw (0.02 is the benchmark model; tests use larger
    values to make attention peaked)."""
    g = geometry or Geometry()
    rng = np.random.Generator(np.random.PCG64(seed))

    def normal(*shape: int) -> np.ndarray:
        return (rng.standard_normal(shape) * std).astype(np.float32)

    def linear(out_dim: int, in_dim: int) -> dict:
        q, mult = quantize_weights(normal(out_dim, in_dim))
        return {"weight": q, "mult": mult, "bias": normal(out_dim)}

    def norm() -> dict:
        scale = (np.float32(1) + normal(g.dim)).astype(np.float32)
        return {"scale": scale, "bias": normal(g.dim)}

    d, f = g.dim, g.ffn_dim
    emb_q, emb_mult = quantize_weights(normal(g.vocab, d))
    out_bias = normal(g.vocab)
    encoder = []
    for _ in range(g.encoder_layers):
        layer = {}
        layer["qkv"] = linear(3 * d, d)
        layer["out"] = linear(d, d)
        layer["ln1"] = norm()
        layer["ffn1"] = linear(f, d)
        layer["ffn2"] = linear(d, f)
        layer["ln2"] = norm()
        encoder.append(layer)
    decoder = []
    for _ in range(g.decoder_layers):
        layer = {}
        layer["self_qkv"] = linear(3 * d, d)
        layer["self_out"] = linear(d, d)
        layer["ln1"] = norm()
        layer["cross_q"] = linear(d, d)
        layer["cross_kv"] = linear(2 * d, d)
        layer["cross_out"] = linear(d, d)
        layer["ln2"] = norm()
        layer["ffn1"] = linear(f, d)
        layer["ffn2"] = linear(d, f)
        layer["ln3"] = norm()
        decoder.append(layer)
    return SeededModel(g, seed, emb_q, emb_mult, out_bias, encoder, decoder)


# ---------------------------------------------------------------------------
# The reference's own graph: Transformer encoder + SSRU decoder with one weight
# multiplier and one static activation multiplier per dense layer
# (crates/marian-cpu/src/q8_engine.rs:76-114, legacy_q8.rs:544-552).
# ---------------------------------------------------------------------------
@dataclass
class SsruGeometry:
    """Defaults: the reference's supported shape (crates/marian-model/src/
    manifest.rs:27-36), 384 wide, 8 heads, 6 encoder and 4 SSRU decoder layers,
    FFN 1536."""
    source_vocab: int = 32000
    target_vocab: int = 32000
    dim: int = 384
    heads: int = 8
    ffn_dim: int = 1536
    encoder_layers: int = 6
    decoder_layers: int = 4


@dataclass
class SsruModel:
    geometry: SsruGeometry
    seed: int
    encoder_embedding: np.ndarray = field(repr=False)
    encoder_embedding_mult: float = field(repr=False)
    decoder_embedding: np.ndarray = field(repr=False)
    decoder_embedding_mult: float = field(repr=False)
    output_act_mult: float = field(repr=False)
    output_bias: np.ndarray = field(repr=False)
    encoder: list = field(repr=False)
    decoder: list = field(repr=False)


def quantize_tensor(w: np.ndarray) -> tuple[np.ndarray, float]:
    """One multiplier for the whole tensor: mult = 127 / max|w| (fp32),
    q = clamp(rint(w * mult), -127, 127) (q8_fp32_artifact.rs:130-132)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    m = np.float32(np.abs(w).max())
    mult = np.float32(127) / m if m > 0 else np.float32(1)
    return np.clip(np.rint(w * mult), -127, 127).astype(np.int8), float(mult)


def seeded_ssru_model(seed: int = DEFAULT_SEED, geometry: SsruGeometry | None = None,
                      std: float = 0.02, shared_input_mults: bool = True) -> SsruModel:
    """Random-init Transformer-SSRU model.  Draw order: encoder embedding
    [Vs, d], decoder embedding [Vt, d], output bias [Vt]; per encoder layer
    wq, wk, wv, wo, attn_ln, w1, w2, ffn_ln; per decoder layer ssru_w (no bias),
    ssru_wf, ssru_ln, wq, wk, wv, wo, context_ln, w1, w2, ffn_ln; then the
    static activation multipliers.  A multiplier is 127 / (the role's expected
    largest |input|) times a draw from U(0.85, 1.15): LayerNorm outputs 4.5,
    embedding + position 4 std sqrt(d) + 1, attention outputs and FFN hidden
    4 std sqrt(d).  With shared_input_mults the layers that read the same input
    (wq/wk/wv of an encoder layer, ssru_w/ssru_wf, a context layer's wk/wv)
    share one multiplier, as calibration from the same activations gives."""
    g = geometry or SsruGeometry()
    rng = np.random.Generator(np.random.PCG64(seed))
    d, f = g.dim, g.ffn_dim

    def normal(*shape: int) -> np.ndarray:
        return (rng.standard_normal(shape) * std).astype(np.float32)

    def linear(out_dim: int, in_dim: int, bias: bool = True) -> dict:
        q, mult = quantize_tensor(normal(out_dim, in_dim))
        return {"weight": q, "weight_mult": mult, "act_mult": 1.0,
                "bias": normal(out_dim) if bias else None}

    def norm() -> dict:
        return {"scale": (np.float32(1) + normal(d)).astype(np.float32), "bias": normal(d)}

    enc_q, enc_mult = quantize_tensor(normal(g.source_vocab, d))
    dec_q, dec_mult = quantize_tensor(normal(g.target_vocab, d))
    out_bias = normal(g.target_vocab)
    encoder = []
    for _ in range(g.encoder_layers):
        L = {k: linear(d, d) for k in ("wq", "wk", "wv", "wo")}
        L["attn_ln"] = norm()
        L["w1"] = linear(f, d)
        L["w2"] = linear(d, f)
        L["ffn_ln"] = norm()
        encoder.append(L)
    decoder = []
    for _ in range(g.decoder_layers):
        L = {"ssru_w": linear(d, d, bias=False), "ssru_wf": linear(d, d), "ssru_ln": norm()}
        for k in ("wq", "wk", "wv", "wo"):
            L[k] = linear(d, d)
        L["context_ln"] = norm()
        L["w1"] = linear(f, d)
        L["w2"] = linear(d, f)
        L["ffn_ln"] = norm()
        decoder.append(L)

    spread = 4.0 * std * math.sqrt(d)
    ln_in, emb_in, proj_in = 4.5, spread + 1.0, spread

    def mult(base: float) -> float:
        return float(np.float32(127.0 / (base * rng.uniform(0.85, 1.15))))

    def assign(layers, group, base):
        if shared_input_mults:
            m = mult(base)
            for k in group:
                layers[k]["act_mult"] = m
        else:
            for k in group:
                layers[k]["act_mult"] = mult(base)

    for i, L in enumerate(encoder):
        assign(L, ("wq", "wk", "wv"), emb_in if i == 0 else ln_in)
        L["wo"]["act_mult"] = mult(proj_in)
        L["w1"]["act_mult"] = mult(ln_in)
        L["w2"]["act_mult"] = mult(proj_in)
    for i, L in enumerate(decoder):
        assign(L, ("ssru_w", "ssru_wf"), emb_in if i == 0 else ln_in)
        L["wq"]["act_mult"] = mult(ln_in)
        assign(L, ("wk", "wv"), ln_in)
        L["wo"]["act_mult"] = mult(proj_in)
        L["w1"]["act_mult"] = mult(ln_in)
        L["w2"]["act_mult"] = mult(proj_in)
    out_act = mult(ln_in)
    return SsruModel(g, seed, enc_q, enc_mult, dec_q, dec_mult, out_act, out_bias, encoder, decoder)


# ---------------------------------------------------------------------------
# Workloads.  A batch is (tokens int32[T], offsets uint32[B+1], limits
# uint32[B]) plus the flags and work limits it is run with.
# ---------------------------------------------------------------------------
REFERENCE_LIMITS = dict(max_length_factor=2, max_generation_steps=256, max_position=4096,
                        max_batch=256, max_source_tokens=256, max_padded_cells=65536)
# The ragged configurations lift the padded-batch caps (their batches exceed
# them) and allow up to 512 generated tokens per row.
LIFTED_LIMITS = dict(max_length_factor=0, max_generation_steps=512, max_position=4096,
                     max_batch=0, max_source_tokens=0, max_padded_cells=0)


@dataclass
class Batch:
    name: str
    tokens: np.ndarray
    offsets: np.ndarray
    max_output_tokens: np.ndarray
    flags: int
    limits: dict

    @property
    def lengths(self) -> np.ndarray:
        return np.diff(self.offsets.astype(np.int64))

    def subset(self, rows) -> "Batch":
        rows = list(rows)
        parts = [self.tokens[self.offsets[r]:self.offsets[r + 1]] for r in rows]
        toks = np.concatenate(parts).astype(np.int32) if parts else np.zeros(0, np.int32)
        offs = np.zeros(len(rows) + 1, np.uint32)
        offs[1:] = np.cumsum([len(p) for p in parts])
        return Batch(self.name, toks, offs, self.max_output_tokens[rows].astype(np.uint32),
                     self.flags, self.limits)


def _pack(name, seqs, limits_per_row, flags, limits) -> Batch:
    offs = np.zeros(len(seqs) + 1, np.uint32)
    offs[1:] = np.cumsum([len(s) for s in seqs])
    toks = np.concatenate(seqs).astype(np.int32)
    return Batch(name, toks, offs, np.asarray(limits_per_row, np.uint32), flags, limits)


def single_sentence_batch(seed: int = 1, vocab: int = 32000) -> Batch:
    """One sentence of 24 ids ~U[3, vocab), exactly 32 greedy steps, EOS ignored."""
    rng = np.random.Generator(np.random.PCG64(seed))
    toks = rng.integers(3, vocab, size=24).astype(np.int32)
    return _pack("single-sentence-24x32", [toks], [32], 1, dict(REFERENCE_LIMITS))


def ragged_batch(seed: int = 3, n: int = 64, vocab: int = 32000) -> Batch:
    """64 sentences, L ~ lognormal(3.0, 0.5) clipped to [5, 128], ids ~U[3, vocab);
    row i stops at a forced step ~U_int[ceil(0.8 L), floor(1.5 L + 10)], capped at 512."""
    rng = np.random.Generator(np.random.PCG64(seed))
    lens = np.clip(np.rint(rng.lognormal(3.0, 0.5, size=n)), 5, 128).astype(np.int64)
    seqs = [rng.integers(3, vocab, size=int(L)).astype(np.int32) for L in lens]
    stops = [min(512, int(rng.integers(math.ceil(0.8 * L), math.floor(1.5 * L + 10) + 1)))
             for L in lens]
    return _pack(f"ragged-{n}", seqs, stops, 0, dict(LIFTED_LIMITS))


def stress_batch(seed: int = 4, n: int = 256, vocab: int = 32000, split: int = 256) -> Batch:
    """256 draws from 0.7*lognormal(2.5, 0.5) + 0.3*U[128, 400], split into
    segments of at most `split` tokens; each segment stops at a forced step
    ~U_int[1, 512]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    seqs = []
    for _ in range(n):
        if rng.random() < 0.7:
            L = int(np.clip(np.rint(rng.lognormal(2.5, 0.5)), 1, None))
        else:
            L = int(rng.integers(128, 401))
        while L > 0:
            seg = min(L, split)
            seqs.append(seg)
            L -= seg
    toks = [rng.integers(3, vocab, size=s).astype(np.int32) for s in seqs]
    stops = [int(rng.integers(1, 513)) for _ in seqs]
    return _pack(f"stress-{n}", toks, stops, 0, dict(LIFTED_LIMITS))


def attention_inputs(seed: int = 2, n: int = 256, heads: int = 8):
    """256 packed sentences, L ~ lognormal(3.2, 0.6) clipped to [4, 256];
    Q, K, V ~ N(0, 1) fp32 [T, heads*64]."""
    rng = np.random.Generator(np.random.PCG64(seed))
    lens = np.clip(np.rint(rng.lognormal(3.2, 0.6, size=n)), 4, 256).astype(np.int64)
    cu = np.zeros(n + 1, np.uint32)
    cu[1:] = np.cumsum(lens)
    T = int(cu[-1])
    d = heads * 64
    q = rng.standard_normal((T, d)).astype(np.float32)
    k = rng.standard_normal((T, d)).astype(np.float32)
    v = rng.standard_normal((T, d)).astype(np.float32)
    return q, k, v, cu


GEMM_SHAPES = [(512, 1536), (512, 512), (512, 2048), (2048, 512), (512, 32000)]
GEMM_ROWS = [1, 8, 64, 256, 4096]


def gemm_inputs(M: int, K: int, N: int, seed: int = 5):
    """A ~ N(0,1) fp32 [M, K]; W ~ U_int[-127, 127] [N, K]; per-column scale
    s_n ~ U(0.001, 0.02) given as the multiplier 1/s_n; bias ~ N(0, 0.02)."""
    rng = np.random.Generator(np.random.PCG64(seed * 1000003 + M * 131 + K * 7 + N))
    a = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, size=N).astype(np.float32)
    mult = (np.float32(1) / s).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32)
    return a, w, mult, bias


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bfloat16 (ties to even), returned as uint16 bits."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)
