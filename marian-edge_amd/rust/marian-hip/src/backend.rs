//! marian-core's TranslationBackend over the HIP engine.  The text side
//! (tokenizers, segmentation, output budgets) is marian-cpu's own
//! `translate_with_engine` (crates/marian-cpu/src/backend.rs:107-348), which
//! takes any `CpuTokenEngine`; both need `pub` in marian-cpu (see the
//! integration notes).

use std::sync::Arc;

use marian_core::{BackendError, BackendInfo, TranslationBackend, TranslationInput, TranslationOutput};
use marian_cpu::{BatchOutput, CpuTokenEngine, TextTokenizer, translate_with_engine};
use marian_model::LexicalShortlist;

use crate::engine::HipEngine;

/// The token-level engine the text pipeline drives: the HIP engine plus the
/// model's lexical shortlist, whose candidates each sentence is scored over
/// (Q8CpuEngine::prepare_candidates, crates/marian-cpu/src/q8_engine.rs:576-584).
pub struct HipTokenEngine {
    pub engine: HipEngine,
    /// None scores the whole vocabulary under the generation mask, which is
    /// what the reference's engine does without a shortlist file.
    pub shortlist: Option<Arc<LexicalShortlist>>,
}

impl CpuTokenEngine for HipTokenEngine {
    fn translate_token_ids(
        &self,
        tokens: &[i32],
        offsets: &[u32],
        max_output_tokens: &[usize],
    ) -> Result<BatchOutput, String> {
        let Some(shortlist) = &self.shortlist else {
            return self.engine.translate_token_ids(tokens, offsets, max_output_tokens);
        };
        let mut candidates = Vec::new();
        let mut candidate_offsets = Vec::with_capacity(offsets.len());
        candidate_offsets.push(0u32);
        for pair in offsets.windows(2) {
            let list = shortlist.candidates(&tokens[pair[0] as usize..pair[1] as usize])?;
            candidates.extend_from_slice(&list);
            candidate_offsets.push(
                u32::try_from(candidates.len()).map_err(|_| "candidate lists exceed u32".to_string())?,
            );
        }
        self.engine.translate_shortlisted(tokens, offsets, max_output_tokens, &candidates, &candidate_offsets)
    }

    fn label(&self) -> &'static str {
        "HIP"
    }
}

pub struct HipBackend {
    engine: HipTokenEngine,
    source: Arc<dyn TextTokenizer>,
    target: Arc<dyn TextTokenizer>,
    source_lang: String,
    target_lang: String,
    model_id: String,
    eos_id: i32,
    /// How many physical rows a logical input repeated by the scheduler may
    /// occupy (translate_batch_with_repetitions).  1 materializes none: a
    /// decode step costs about the same from 1 to 4 rows on this device and
    /// more above, so copies of a row only add work.
    duplicate_batch_width: usize,
}

impl HipBackend {
    /// Builds the backend and warms its engine up once, as the reference's
    /// backends do at load (Q8CpuBackend, crates/marian-cpu/src/backend.rs:810-813);
    /// a warmup failure is BackendError::Inference.
    #[allow(clippy::too_many_arguments)]
    pub fn new(
        engine: HipEngine,
        shortlist: Option<Arc<LexicalShortlist>>,
        source: Arc<dyn TextTokenizer>,
        target: Arc<dyn TextTokenizer>,
        source_lang: impl Into<String>,
        target_lang: impl Into<String>,
        model_id: impl Into<String>,
        eos_id: i32,
    ) -> Result<Self, BackendError> {
        engine
            .warmup()
            .map_err(|error| BackendError::Inference(format!("HIP warmup failed: {error}")))?;
        Ok(Self {
            engine: HipTokenEngine { engine, shortlist },
            source,
            target,
            source_lang: source_lang.into(),
            target_lang: target_lang.into(),
            model_id: model_id.into(),
            eos_id,
            duplicate_batch_width: 1,
        })
    }

    pub fn with_duplicate_batch_width(mut self, width: usize) -> Self {
        self.duplicate_batch_width = width.max(1);
        self
    }

    pub fn engine(&self) -> &HipEngine {
        &self.engine.engine
    }
}

impl TranslationBackend for HipBackend {
    fn info(&self) -> BackendInfo {
        // The library reports the device (e.g. "AMD Instinct MI355X (gfx950)").
        let json = self.engine.engine.info_json();
        let device = json
            .split("\"device\":\"")
            .nth(1)
            .and_then(|rest| rest.split('"').next())
            .unwrap_or("AMD GPU")
            .to_string();
        BackendInfo {
            name: "hip".into(),
            device,
            model: self.model_id.clone(),
            precision: "q8".into(),
            attention: Some("varlen-fused".into()),
            supports_batching: true,
        }
    }

    /// Not ready after any HIP runtime error: the scheduler then drains
    /// instead of enqueueing (crates/marian-core/src/backend.rs:10-18).
    fn is_ready(&self) -> bool {
        self.engine.engine.is_ready()
    }

    fn translate_batch(&mut self, inputs: &[TranslationInput]) -> Result<Vec<TranslationOutput>, BackendError> {
        translate_with_engine(
            &self.engine,
            self.source.as_ref(),
            self.target.as_ref(),
            &self.source_lang,
            &self.target_lang,
            self.eos_id,
            inputs,
        )
    }

    /// One output per logical input; input i runs as min(repetitions[i],
    /// duplicate_batch_width) physical rows and its first copy's output is
    /// returned (outputs are batch-invariant, so the copies agree).
    fn translate_batch_with_repetitions(
        &mut self,
        inputs: &[TranslationInput],
        repetitions: &[usize],
    ) -> Result<Vec<TranslationOutput>, BackendError> {
        if inputs.len() != repetitions.len() || repetitions.iter().any(|&r| r == 0) {
            return Err(BackendError::InvalidInput("logical batch repetitions are malformed".into()));
        }
        if self.duplicate_batch_width == 1 {
            return self.translate_batch(inputs);
        }
        let mut physical = Vec::new();
        let mut first_copy = Vec::with_capacity(inputs.len());
        for (input, &count) in inputs.iter().zip(repetitions) {
            first_copy.push(physical.len());
            for _ in 0..count.min(self.duplicate_batch_width) {
                physical.push(input.clone());
            }
        }
        let outputs = self.translate_batch(&physical)?;
        if outputs.len() != physical.len() {
            return Err(BackendError::Inference(format!(
                "HIP backend returned {} outputs for {} physical rows",
                outputs.len(),
                physical.len()
            )));
        }
        Ok(first_copy.into_iter().map(|i| outputs[i].clone()).collect())
    }
}

/// Scheduler settings for a HIP worker (marian-core's `SchedulerConfig`,
/// crates/marian-core/src/scheduler.rs:22-44).  Measured on one MI355X with
/// batches of 1 to 256 sentences of the 64-sentence ragged distribution: a
/// decode step costs nearly the same from 1 to 64 rows, so throughput grows
/// from 11.7k target tokens/s at 1 sentence to 267k at 64 and 498k at 256
/// (profiles/batch_sweep_ragged.md).  A model of `worker_loop` over those
/// batch times gives the lowest median latency at 10/50/90% load with 256
/// requests per batch and a 100 us window; the CLI's 16 and 750 us saturate
/// the worker at about a fifth of that load.  The length-bucket cap is raised
/// so that it never limits a batch below 256 (the engine does not pad).
pub fn recommended_scheduler_config() -> marian_core::SchedulerConfig {
    marian_core::SchedulerConfig {
        max_batch_size: 256,
        max_padded_source_chars: 256 * 1024,
        batch_window: std::time::Duration::from_micros(100),
        ..marian_core::SchedulerConfig::default()
    }
}
