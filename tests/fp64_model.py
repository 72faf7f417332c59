"""A float64 restatement of the Q8 Transformer's composition, for pinning the oracle.

Written from the mathematics of the path, not from the oracle's code: numpy
float64 throughout, every layer a textbook expression.  Quantization follows
the same rule as the path (per-row a = 127 / max|x|, q = clamp(rint(x a), -127,
127), y = acc / (a w_mult) + bias) but in float64, so its decisions can differ
from an fp32 implementation only where x a lies within rounding of a .5 tie.
The wiring it states (crates/marian-cpu/src/q8_engine.rs):
  embedding      x = (q / mult) sqrt(d) + pos[p]                      :53-74, 586-603
  encoder layer  x1 = LN1(Wo attn(Wq x, Wk x, Wv x) + x)              :526-558
                 x  = LN2(W2 relu(W1 x1) + x1)                        :632-651
  decoder input  pos[0] at step 0, else emb(prev) sqrt(d) + pos[t]    :605-630
  decoder layer  self-attention over the row's steps 0..t, then
                 x2 = LN2(Wo_c attn(Wq_c x1, K_c enc, V_c enc) + x1)  :410-432
                 then the FFN as in the encoder, with LN3
  scoring        logit_v = acc_v / (a mult_v) + bias_v, ids 1 and 7..38
                 masked, first maximum wins                           :749-790
`mistake` plants one wiring error at a time, so a test can show that the
comparison would catch it.
"""

from __future__ import annotations

import numpy as np

MISTAKES = (
    "no_sqrt_d",          # embedding not scaled by sqrt(d)
    "gamma_beta_swap",    # LayerNorm scale and shift exchanged
    "ln_params_swap",     # first and second LayerNorm of a layer exchanged
    "residual_from_y",    # LN(y + y) instead of LN(y + x)
    "ffn_residual_x",     # the FFN residual taken from the layer input, not x1
    "qk_swap",            # query and key rows of the fused projection exchanged
    "kv_swap",            # key and value rows exchanged
    "no_attn_scale",      # scores not scaled by 1/sqrt(dh)
    "no_relu",            # FFN hidden without ReLU
    "attend_whole_batch", # encoder attention across sentences of the batch
    "pos_off_by_one",     # decoder step t uses pos[t + 1]
    "cross_from_embedding",  # cross K/V computed from the encoder input
    "cross_q_from_input", # cross query from the layer input instead of x1
    "no_self_cache",      # decoder self-attention over the current step only
    "sin_cos_swap",       # positions with cos in the first half
)


def positions(d: int, count: int) -> np.ndarray:
    half = d // 2
    f = np.exp(-np.arange(half) * np.log(10000.0) / (half - 1))
    p = np.arange(count)[:, None] * f[None, :]
    return np.concatenate([np.sin(p), np.cos(p)], axis=1)


def quantize(x: np.ndarray):
    m = np.abs(x).max(axis=-1, keepdims=True)
    a = np.where(m > 0, 127.0 / np.where(m > 0, m, 1.0), 1.0)
    q = np.clip(np.rint(x * a), -127, 127)
    return q, a


def linear(x, lin, relu=False):
    q, a = quantize(x)
    acc = q @ lin["weight"].astype(np.float64).T
    y = acc / (a * lin["mult"].astype(np.float64)[None, :]) + lin["bias"].astype(np.float64)
    return np.maximum(y, 0.0) if relu else y


def layer_norm(z, p, mistake=None):
    g, b = p["scale"].astype(np.float64), p["bias"].astype(np.float64)
    if mistake == "gamma_beta_swap":
        g, b = b, g
    mean = z.mean(axis=-1, keepdims=True)
    var = ((z - mean) ** 2).mean(axis=-1, keepdims=True)
    return (z - mean) / np.sqrt(var + 1e-6) * g + b


def attend(q, k, v, heads, mistake=None):
    """q [n, d] over keys k/v [m, d]; heads of width d / heads."""
    n, d = q.shape
    dh = d // heads
    out = np.zeros((n, d))
    scale = 1.0 if mistake == "no_attn_scale" else 1.0 / np.sqrt(dh)
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        s = q[:, sl] @ k[:, sl].T * scale
        s = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, sl] = (s / s.sum(axis=1, keepdims=True)) @ v[:, sl]
    return out


class Fp64Model:
    def __init__(self, model, mistake=None):
        assert mistake is None or mistake in MISTAKES, mistake
        self.m = model
        self.g = model.geometry
        self.mistake = mistake
        self.pos = positions(self.g.dim, 4096)
        if mistake == "sin_cos_swap":
            h = self.g.dim // 2
            self.pos = np.concatenate([self.pos[:, h:], self.pos[:, :h]], axis=1)

    def embed(self, tok):
        e = self.m.embedding[tok].astype(np.float64) / self.m.embedding_mult[tok].astype(np.float64)[..., None]
        return e if self.mistake == "no_sqrt_d" else e * np.sqrt(self.g.dim)

    def _ln(self, z, layer, which):
        names = {"ln1": "ln2", "ln2": "ln1"} if self.mistake == "ln_params_swap" else {}
        return layer_norm(z, layer[names.get(which, which)], self.mistake)

    def _res(self, y, x):
        return y + y if self.mistake == "residual_from_y" else y + x

    def _split_qkv(self, qkv):
        d = self.g.dim
        q, k, v = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
        if self.mistake == "qk_swap":
            q, k = k, q
        if self.mistake == "kv_swap":
            k, v = v, k
        return q, k, v

    def _ffn(self, x1, layer, ln, residual):
        h = linear(x1, layer["ffn1"], relu=self.mistake != "no_relu")
        y = linear(h, layer["ffn2"])
        return self._ln(self._res(y, residual), layer, ln)

    def encode(self, tokens, offsets):
        """Packed rows [T, d]; each sentence attends over its own rows."""
        H = self.g.heads
        x = self.embed(np.asarray(tokens)) + self.pos[np.concatenate(
            [np.arange(offsets[i + 1] - offsets[i]) for i in range(len(offsets) - 1)])]
        for L in self.m.encoder:
            q, k, v = self._split_qkv(linear(x, L["qkv"]))
            att = np.zeros_like(x)
            if self.mistake == "attend_whole_batch":
                att = attend(q, k, v, H, self.mistake)
            else:
                for i in range(len(offsets) - 1):
                    sl = slice(int(offsets[i]), int(offsets[i + 1]))
                    att[sl] = attend(q[sl], k[sl], v[sl], H, self.mistake)
            x1 = self._ln(self._res(linear(att, L["out"]), x), L, "ln1")
            x = self._ffn(x1, L, "ln2", x if self.mistake == "ffn_residual_x" else x1)
        return x

    def logits(self, state, flags=0):
        q, a = quantize(state[None, :])
        acc = q @ self.m.embedding.astype(np.float64).T
        lg = (acc / (a * self.m.embedding_mult.astype(np.float64)[None, :]))[0] + \
            self.m.output_bias.astype(np.float64)
        if not flags & 2:
            lg[1] = -np.inf
            lg[7:39] = -np.inf
        return lg

    def decode(self, enc, tokens, steps, flags=1, probe_step=None):
        """Greedy decode of one sentence (enc: its encoder rows, tokens: its
        source ids); returns the generated ids and the logits of probe_step."""
        d, H = self.g.dim, self.g.heads
        src = self.embed(np.asarray(tokens)) + self.pos[:len(tokens)] \
            if self.mistake == "cross_from_embedding" else enc
        ckv = [linear(src, L["cross_kv"]) for L in self.m.decoder]
        kc = [np.zeros((0, d)) for _ in self.m.decoder]
        vc = [np.zeros((0, d)) for _ in self.m.decoder]
        prev, out, probed = -1, [], None
        for t in range(steps):
            p = self.pos[t + 1 if self.mistake == "pos_off_by_one" else t]
            x = (p if prev < 0 else self.embed(prev) + p)[None, :]
            for li, L in enumerate(self.m.decoder):
                q, k, v = self._split_qkv(linear(x, L["self_qkv"]))
                if self.mistake == "no_self_cache":
                    kc[li], vc[li] = k, v
                else:
                    kc[li] = np.vstack([kc[li], k])
                    vc[li] = np.vstack([vc[li], v])
                att = attend(q, kc[li], vc[li], H, self.mistake)
                x1 = self._ln(self._res(linear(att, L["self_out"]), x), L, "ln1")
                qc = linear(x if self.mistake == "cross_q_from_input" else x1, L["cross_q"])
                att = attend(qc, ckv[li][:, :d], ckv[li][:, d:], H, self.mistake)
                x2 = layer_norm(self._res(linear(att, L["cross_out"]), x1), L["ln2"], self.mistake)
                x = self._ffn(x2, L, "ln3", x2)
            lg = self.logits(x[0], flags)
            if probe_step == t:
                probed = lg
            tok = int(np.argmax(lg))
            out.append(tok)
            prev = tok
            if tok == 0 and not flags & 1:
                break
        return out, probed


# ---------------------------------------------------------------------------
# The reference's own graph: Transformer encoder + SSRU decoder with static
# per-tensor activation multipliers (q8_engine.rs:76-114, 382-451, 511-574;
# tensor.rs:184-218).
#   linear         q = clamp(rint(x a), -127, 127), y = acc / (a w) + b
#   embedding      x = (q / mult) sqrt(d) + pos, separate encoder/decoder tables
#   encoder layer  Q, K, V each from its own layer (and multiplier)
#   SSRU           c = W x, f = Wf x + bf, g = 1 / (1 + exp(-f)),
#                  s = g s + (1 - g) c, x1 = LN(relu(s) + x)
#   context        x2 = LN(Wo attn(Wq x1, Wk enc, Wv enc) + x1), then the FFN
#   scoring        the state quantized with the output multiplier; candidates
#                  scanned in order (or every id with the generation mask)
# ---------------------------------------------------------------------------
SSRU_MISTAKES = (
    "gate_inverted",          # s = (1 - g) s + g c
    "state_not_carried",      # the recurrent state restarts at zero every step
    "ssru_no_relu",           # LN(s + x) instead of LN(relu(s) + x)
    "ssru_no_residual",       # LN(relu(s)) without the layer input
    "context_q_from_input",   # the context query from x instead of the SSRU output
    "cross_from_embedding",   # context K/V from the encoder input
    "decoder_table_swap",     # decoder input from the encoder embedding table
    "output_mult_dynamic",    # output row quantized per row instead of statically
    "kv_mult_swap",           # wk quantized with wv's multiplier and back
    "ffn_residual_x",         # FFN residual from the SSRU output instead of x2
    "no_sqrt_d",
    "pos_off_by_one",
)


def slinear(x, lin, relu=False, act=None):
    a = lin["act_mult"] if act is None else act
    q = np.clip(np.rint(x * np.float64(a)), -127, 127)
    acc = q @ lin["weight"].astype(np.float64).T
    y = acc / (np.float64(a) * np.float64(lin["weight_mult"]))
    if lin["bias"] is not None:
        y = y + lin["bias"].astype(np.float64)
    return np.maximum(y, 0.0) if relu else y


class Fp64SsruModel:
    def __init__(self, model, mistake=None):
        assert mistake is None or mistake in SSRU_MISTAKES, mistake
        self.m = model
        self.g = model.geometry
        self.mistake = mistake
        self.pos = positions(self.g.dim, 4096)

    def _embed(self, table, mult, tok):
        e = table[tok].astype(np.float64) / np.float64(mult)
        return e if self.mistake == "no_sqrt_d" else e * np.sqrt(self.g.dim)

    def encode(self, tokens, offsets):
        H = self.g.heads
        toks = np.asarray(tokens)
        p = np.concatenate([np.arange(offsets[i + 1] - offsets[i]) for i in range(len(offsets) - 1)])
        x = self._embed(self.m.encoder_embedding, self.m.encoder_embedding_mult, toks) + self.pos[p]
        for L in self.m.encoder:
            q, k, v = slinear(x, L["wq"]), slinear(x, L["wk"]), slinear(x, L["wv"])
            att = np.zeros_like(x)
            for i in range(len(offsets) - 1):
                sl = slice(int(offsets[i]), int(offsets[i + 1]))
                att[sl] = attend(q[sl], k[sl], v[sl], H)
            x1 = layer_norm(slinear(att, L["wo"]) + x, L["attn_ln"])
            h = slinear(x1, L["w1"], relu=True)
            x = layer_norm(slinear(h, L["w2"]) + x1, L["ffn_ln"])
        return x

    def logits(self, state, flags=0, candidates=None):
        if self.mistake == "output_mult_dynamic":
            q, a = quantize(state[None, :])
            q, a = q[0], float(a[0, 0])
        else:
            a = np.float64(self.m.output_act_mult)
            q = np.clip(np.rint(state * a), -127, 127)
        acc = self.m.decoder_embedding.astype(np.float64) @ q
        lg = acc / (a * np.float64(self.m.decoder_embedding_mult)) + self.m.output_bias.astype(np.float64)
        out = np.full_like(lg, -np.inf)
        if candidates is not None:
            out[candidates] = lg[candidates]
        else:
            out[:] = lg
            if not flags & 2:
                out[1] = -np.inf
                out[7:39] = -np.inf
        return out

    def decode(self, enc, tokens, steps, flags=1, candidates=None, probe_step=None):
        d, H = self.g.dim, self.g.heads
        src = enc
        if self.mistake == "cross_from_embedding":
            src = self._embed(self.m.encoder_embedding, self.m.encoder_embedding_mult,
                              np.asarray(tokens)) + self.pos[:len(tokens)]
        kv = []
        for L in self.m.decoder:
            if self.mistake == "kv_mult_swap":
                kv.append((slinear(src, L["wk"], act=L["wv"]["act_mult"]),
                           slinear(src, L["wv"], act=L["wk"]["act_mult"])))
            else:
                kv.append((slinear(src, L["wk"]), slinear(src, L["wv"])))
        state = [np.zeros(d) for _ in self.m.decoder]
        prev, out, probed = -1, [], None
        cand = None if candidates is None else np.asarray(candidates, np.int64)
        for t in range(steps):
            p = self.pos[t + 1 if self.mistake == "pos_off_by_one" else t]
            if prev < 0:
                x = p.copy()
            elif self.mistake == "decoder_table_swap":
                x = self._embed(self.m.encoder_embedding, self.m.encoder_embedding_mult, prev) + p
            else:
                x = self._embed(self.m.decoder_embedding, self.m.decoder_embedding_mult, prev) + p
            x = x[None, :]
            for li, L in enumerate(self.m.decoder):
                c = slinear(x, L["ssru_w"])
                f = slinear(x, L["ssru_wf"])
                gate = 1.0 / (1.0 + np.exp(-f))
                if self.mistake == "gate_inverted":
                    gate = 1.0 - gate
                s0 = np.zeros(d) if self.mistake == "state_not_carried" else state[li]
                s = gate * s0 + (1.0 - gate) * c
                state[li] = s[0]
                z = s if self.mistake == "ssru_no_relu" else np.maximum(s, 0.0)
                x1 = layer_norm(z if self.mistake == "ssru_no_residual" else z + x, L["ssru_ln"])
                qc = slinear(x if self.mistake == "context_q_from_input" else x1, L["wq"])
                att = attend(qc, kv[li][0], kv[li][1], H)
                x2 = layer_norm(slinear(att, L["wo"]) + x1, L["context_ln"])
                h = slinear(x2, L["w1"], relu=True)
                x = layer_norm(slinear(h, L["w2"]) + (x1 if self.mistake == "ffn_residual_x" else x2),
                               L["ffn_ln"])
            lg = self.logits(x[0], flags, cand)
            if probe_step == t:
                probed = lg
            if cand is not None:
                tok = int(cand[np.argmax(lg[cand])])
            else:
                tok = int(np.argmax(lg))
            out.append(tok)
            prev = tok
            if tok == 0 and not flags & 1:
                break
        return out, probed
