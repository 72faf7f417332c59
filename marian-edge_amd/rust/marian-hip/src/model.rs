//! Borrowed model descriptions handed to the engine constructors.  They point
//! at already-quantized weights (the caller's parsed model); the engine copies
//! everything to device memory during creation, so the borrows end there.

use crate::ffi;

/// A dense layer of the transformer-decoder graph: int8 [out, in] weights,
/// one multiplier per output channel, fp32 bias.
#[derive(Clone, Copy)]
pub struct Linear<'a> {
    pub weight: &'a [i8],
    pub mult: &'a [f32],
    pub bias: &'a [f32],
}

#[derive(Clone, Copy)]
pub struct Norm<'a> {
    pub scale: &'a [f32],
    pub bias: &'a [f32],
}

pub struct EncoderLayer<'a> {
    pub qkv: Linear<'a>,
    pub out: Linear<'a>,
    pub ln1: Norm<'a>,
    pub ffn1: Linear<'a>,
    pub ffn2: Linear<'a>,
    pub ln2: Norm<'a>,
}

pub struct DecoderLayer<'a> {
    pub self_qkv: Linear<'a>,
    pub self_out: Linear<'a>,
    pub ln1: Norm<'a>,
    pub cross_q: Linear<'a>,
    pub cross_kv: Linear<'a>,
    pub cross_out: Linear<'a>,
    pub ln2: Norm<'a>,
    pub ffn1: Linear<'a>,
    pub ffn2: Linear<'a>,
    pub ln3: Norm<'a>,
}

/// The transformer-decoder graph (tied embedding and output projection).
pub struct TransformerModel<'a> {
    pub vocab: u32,
    pub dim: u32,
    pub heads: u32,
    pub ffn_dim: u32,
    pub embedding: &'a [i8],
    pub embedding_mult: &'a [f32],
    pub output_bias: &'a [f32],
    pub encoder: Vec<EncoderLayer<'a>>,
    pub decoder: Vec<DecoderLayer<'a>>,
}

/// A dense layer of the reference's per-tensor scheme (Q8Linear,
/// crates/marian-cpu/src/q8_gemm.rs): one weight multiplier, one static
/// activation multiplier, optional bias.
#[derive(Clone, Copy)]
pub struct StaticLinear<'a> {
    pub weight: &'a [i8],
    pub weight_mult: f32,
    pub act_mult: f32,
    pub bias: Option<&'a [f32]>,
}

pub struct SsruEncoderLayer<'a> {
    pub wq: StaticLinear<'a>,
    pub wk: StaticLinear<'a>,
    pub wv: StaticLinear<'a>,
    pub wo: StaticLinear<'a>,
    pub attn_ln: Norm<'a>,
    pub w1: StaticLinear<'a>,
    pub w2: StaticLinear<'a>,
    pub ffn_ln: Norm<'a>,
}

pub struct SsruDecoderLayer<'a> {
    pub ssru_w: StaticLinear<'a>,
    pub ssru_wf: StaticLinear<'a>,
    pub ssru_ln: Norm<'a>,
    pub wq: StaticLinear<'a>,
    pub wk: StaticLinear<'a>,
    pub wv: StaticLinear<'a>,
    pub wo: StaticLinear<'a>,
    pub context_ln: Norm<'a>,
    pub w1: StaticLinear<'a>,
    pub w2: StaticLinear<'a>,
    pub ffn_ln: Norm<'a>,
}

/// The reference's Transformer-SSRU graph (Q8CpuEngine,
/// crates/marian-cpu/src/q8_engine.rs:76-114).
pub struct SsruModel<'a> {
    pub source_vocab: u32,
    pub target_vocab: u32,
    pub dim: u32,
    pub heads: u32,
    pub ffn_dim: u32,
    pub encoder_embedding: &'a [i8],
    pub encoder_embedding_mult: f32,
    pub decoder_embedding: &'a [i8],
    pub decoder_embedding_mult: f32,
    pub output_act_mult: f32,
    pub output_bias: &'a [f32],
    pub encoder: Vec<SsruEncoderLayer<'a>>,
    pub decoder: Vec<SsruDecoderLayer<'a>>,
}

impl<'a> SsruModel<'a> {
    /// The loaded Q8 model of marian-cpu (`Q8CpuEngine::weights_view`, added by
    /// marian-edge-wiring.patch), one to one: `encoder_Wemb` / `decoder_Wemb`,
    /// `decoder_output_activation_mult`, and per layer the Q8Linear weights
    /// ([out, in] int8), weight and activation multipliers and optional bias,
    /// with the LayerNorms in the graph's order (q8_engine.rs:76-114).
    pub fn from_q8_view(view: &marian_cpu::Q8ModelView<'a>) -> Self {
        fn st<'a>(l: &'a marian_cpu::Q8Linear) -> StaticLinear<'a> {
            StaticLinear {
                weight: l.weights(),
                weight_mult: l.weight_quant_mult(),
                act_mult: l.activation_quant_mult(),
                bias: l.bias(),
            }
        }
        fn nm<'a>(n: &marian_cpu::Q8LayerNormView<'a>) -> Norm<'a> {
            Norm { scale: n.scale, bias: n.bias }
        }
        let ffn_dim = view.encoder.first().map_or(0, |l| l.w1.output_dim());
        let dim = view.dim.max(1);
        SsruModel {
            source_vocab: (view.encoder_embedding.len() / dim) as u32,
            target_vocab: (view.decoder_embedding.len() / dim) as u32,
            dim: view.dim as u32,
            heads: view.heads as u32,
            ffn_dim: ffn_dim as u32,
            encoder_embedding: view.encoder_embedding,
            encoder_embedding_mult: view.encoder_embedding_mult,
            decoder_embedding: view.decoder_embedding,
            decoder_embedding_mult: view.decoder_embedding_mult,
            output_act_mult: view.decoder_output_activation_mult,
            output_bias: view.output_bias,
            encoder: view
                .encoder
                .iter()
                .map(|l| SsruEncoderLayer {
                    wq: st(l.wq),
                    wk: st(l.wk),
                    wv: st(l.wv),
                    wo: st(l.wo),
                    attn_ln: nm(&l.attention_norm),
                    w1: st(l.w1),
                    w2: st(l.w2),
                    ffn_ln: nm(&l.ffn_norm),
                })
                .collect(),
            decoder: view
                .decoder
                .iter()
                .map(|l| SsruDecoderLayer {
                    ssru_w: st(l.ssru_w),
                    ssru_wf: st(l.ssru_wf),
                    ssru_ln: nm(&l.ssru_norm),
                    wq: st(l.wq),
                    wk: st(l.wk),
                    wv: st(l.wv),
                    wo: st(l.wo),
                    context_ln: nm(&l.context_norm),
                    w1: st(l.w1),
                    w2: st(l.w2),
                    ffn_ln: nm(&l.ffn_norm),
                })
                .collect(),
        }
    }
}

fn lin(l: &Linear<'_>) -> ffi::marian_hip_linear {
    ffi::marian_hip_linear { weight: l.weight.as_ptr(), mult: l.mult.as_ptr(), bias: l.bias.as_ptr() }
}

fn slin(l: &StaticLinear<'_>) -> ffi::marian_hip_static_linear {
    ffi::marian_hip_static_linear {
        weight: l.weight.as_ptr(),
        weight_mult: l.weight_mult,
        act_mult: l.act_mult,
        bias: l.bias.map_or(std::ptr::null(), |b| b.as_ptr()),
    }
}

/// Slice lengths are checked here; value checks (multipliers finite and
/// positive, no -128 weight, supported geometry) are the library's.
fn check_len(what: &str, got: usize, want: usize) -> Result<(), String> {
    if got == want {
        Ok(())
    } else {
        Err(format!("{what} has {got} values, expected {want}"))
    }
}

impl TransformerModel<'_> {
    /// The C description plus the layer arrays it points into (keep both alive
    /// for the create call).
    pub(crate) fn raw(
        &self,
    ) -> Result<(ffi::marian_hip_model, Vec<ffi::marian_hip_encoder_layer>, Vec<ffi::marian_hip_decoder_layer>), String>
    {
        let (d, f, v) = (self.dim as usize, self.ffn_dim as usize, self.vocab as usize);
        check_len("embedding", self.embedding.len(), v * d)?;
        check_len("embedding multipliers", self.embedding_mult.len(), v)?;
        check_len("output bias", self.output_bias.len(), v)?;
        let check = |name: &str, l: &Linear<'_>, n: usize, k: usize| -> Result<(), String> {
            check_len(name, l.weight.len(), n * k)?;
            check_len(name, l.mult.len(), n)?;
            check_len(name, l.bias.len(), n)
        };
        let norm = |name: &str, p: &Norm<'_>| -> Result<(), String> {
            check_len(name, p.scale.len(), d)?;
            check_len(name, p.bias.len(), d)
        };
        let mut enc = Vec::with_capacity(self.encoder.len());
        for l in &self.encoder {
            check("encoder qkv", &l.qkv, 3 * d, d)?;
            check("encoder out", &l.out, d, d)?;
            check("encoder ffn1", &l.ffn1, f, d)?;
            check("encoder ffn2", &l.ffn2, d, f)?;
            norm("encoder ln1", &l.ln1)?;
            norm("encoder ln2", &l.ln2)?;
            enc.push(ffi::marian_hip_encoder_layer {
                qkv: lin(&l.qkv),
                out: lin(&l.out),
                ln1_scale: l.ln1.scale.as_ptr(),
                ln1_bias: l.ln1.bias.as_ptr(),
                ffn1: lin(&l.ffn1),
                ffn2: lin(&l.ffn2),
                ln2_scale: l.ln2.scale.as_ptr(),
                ln2_bias: l.ln2.bias.as_ptr(),
            });
        }
        let mut dec = Vec::with_capacity(self.decoder.len());
        for l in &self.decoder {
            check("decoder self_qkv", &l.self_qkv, 3 * d, d)?;
            check("decoder self_out", &l.self_out, d, d)?;
            check("decoder cross_q", &l.cross_q, d, d)?;
            check("decoder cross_kv", &l.cross_kv, 2 * d, d)?;
            check("decoder cross_out", &l.cross_out, d, d)?;
            check("decoder ffn1", &l.ffn1, f, d)?;
            check("decoder ffn2", &l.ffn2, d, f)?;
            norm("decoder ln1", &l.ln1)?;
            norm("decoder ln2", &l.ln2)?;
            norm("decoder ln3", &l.ln3)?;
            dec.push(ffi::marian_hip_decoder_layer {
                self_qkv: lin(&l.self_qkv),
                self_out: lin(&l.self_out),
                ln1_scale: l.ln1.scale.as_ptr(),
                ln1_bias: l.ln1.bias.as_ptr(),
                cross_q: lin(&l.cross_q),
                cross_kv: lin(&l.cross_kv),
                cross_out: lin(&l.cross_out),
                ln2_scale: l.ln2.scale.as_ptr(),
                ln2_bias: l.ln2.bias.as_ptr(),
                ffn1: lin(&l.ffn1),
                ffn2: lin(&l.ffn2),
                ln3_scale: l.ln3.scale.as_ptr(),
                ln3_bias: l.ln3.bias.as_ptr(),
            });
        }
        let model = ffi::marian_hip_model {
            vocab: self.vocab,
            dim: self.dim,
            heads: self.heads,
            ffn_dim: self.ffn_dim,
            encoder_layers: enc.len() as u32,
            decoder_layers: dec.len() as u32,
            embedding: self.embedding.as_ptr(),
            embedding_mult: self.embedding_mult.as_ptr(),
            output_bias: self.output_bias.as_ptr(),
            encoder: enc.as_ptr(),
            decoder: dec.as_ptr(),
        };
        Ok((model, enc, dec))
    }
}

impl SsruModel<'_> {
    pub(crate) fn raw(
        &self,
    ) -> Result<
        (ffi::marian_hip_ssru_model, Vec<ffi::marian_hip_ssru_encoder_layer>, Vec<ffi::marian_hip_ssru_decoder_layer>),
        String,
    > {
        let (d, f) = (self.dim as usize, self.ffn_dim as usize);
        check_len("encoder embedding", self.encoder_embedding.len(), self.source_vocab as usize * d)?;
        check_len("decoder embedding", self.decoder_embedding.len(), self.target_vocab as usize * d)?;
        check_len("output bias", self.output_bias.len(), self.target_vocab as usize)?;
        let check = |name: &str, l: &StaticLinear<'_>, n: usize, k: usize| -> Result<(), String> {
            check_len(name, l.weight.len(), n * k)?;
            l.bias.map_or(Ok(()), |b| check_len(name, b.len(), n))
        };
        let norm = |name: &str, p: &Norm<'_>| -> Result<(), String> {
            check_len(name, p.scale.len(), d)?;
            check_len(name, p.bias.len(), d)
        };
        let mut enc = Vec::with_capacity(self.encoder.len());
        for l in &self.encoder {
            for (name, x) in [("encoder Wq", &l.wq), ("encoder Wk", &l.wk), ("encoder Wv", &l.wv), ("encoder Wo", &l.wo)] {
                check(name, x, d, d)?;
            }
            check("encoder W1", &l.w1, f, d)?;
            check("encoder W2", &l.w2, d, f)?;
            norm("encoder attention norm", &l.attn_ln)?;
            norm("encoder ffn norm", &l.ffn_ln)?;
            enc.push(ffi::marian_hip_ssru_encoder_layer {
                wq: slin(&l.wq),
                wk: slin(&l.wk),
                wv: slin(&l.wv),
                wo: slin(&l.wo),
                attn_ln_scale: l.attn_ln.scale.as_ptr(),
                attn_ln_bias: l.attn_ln.bias.as_ptr(),
                w1: slin(&l.w1),
                w2: slin(&l.w2),
                ffn_ln_scale: l.ffn_ln.scale.as_ptr(),
                ffn_ln_bias: l.ffn_ln.bias.as_ptr(),
            });
        }
        let mut dec = Vec::with_capacity(self.decoder.len());
        for l in &self.decoder {
            for (name, x) in [
                ("SSRU W", &l.ssru_w),
                ("SSRU Wf", &l.ssru_wf),
                ("context Wq", &l.wq),
                ("context Wk", &l.wk),
                ("context Wv", &l.wv),
                ("context Wo", &l.wo),
            ] {
                check(name, x, d, d)?;
            }
            check("decoder W1", &l.w1, f, d)?;
            check("decoder W2", &l.w2, d, f)?;
            norm("SSRU norm", &l.ssru_ln)?;
            norm("context norm", &l.context_ln)?;
            norm("decoder ffn norm", &l.ffn_ln)?;
            dec.push(ffi::marian_hip_ssru_decoder_layer {
                ssru_w: slin(&l.ssru_w),
                ssru_wf: slin(&l.ssru_wf),
                ssru_ln_scale: l.ssru_ln.scale.as_ptr(),
                ssru_ln_bias: l.ssru_ln.bias.as_ptr(),
                wq: slin(&l.wq),
                wk: slin(&l.wk),
                wv: slin(&l.wv),
                wo: slin(&l.wo),
                context_ln_scale: l.context_ln.scale.as_ptr(),
                context_ln_bias: l.context_ln.bias.as_ptr(),
                w1: slin(&l.w1),
                w2: slin(&l.w2),
                ffn_ln_scale: l.ffn_ln.scale.as_ptr(),
                ffn_ln_bias: l.ffn_ln.bias.as_ptr(),
            });
        }
        let model = ffi::marian_hip_ssru_model {
            source_vocab: self.source_vocab,
            target_vocab: self.target_vocab,
            dim: self.dim,
            heads: self.heads,
            ffn_dim: self.ffn_dim,
            encoder_layers: enc.len() as u32,
            decoder_layers: dec.len() as u32,
            encoder_embedding: self.encoder_embedding.as_ptr(),
            encoder_embedding_mult: self.encoder_embedding_mult,
            decoder_embedding: self.decoder_embedding.as_ptr(),
            decoder_embedding_mult: self.decoder_embedding_mult,
            output_act_mult: self.output_act_mult,
            output_bias: self.output_bias.as_ptr(),
            encoder: enc.as_ptr(),
            decoder: dec.as_ptr(),
        };
        Ok((model, enc, dec))
    }
}
