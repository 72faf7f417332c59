//! Safe wrapper of one marian_hip_engine: one device, one HIP stream, one
//! owner thread.  Like every marian-edge backend object it is deliberately
//! neither Send nor Sync (crates/marian-core/src/backend.rs:3-6).

use std::{
    ffi::{CStr, c_int},
    marker::PhantomData,
    ptr::NonNull,
};

use marian_core::BackendError;
use marian_cpu::BatchOutput;

use crate::{
    ffi,
    model::{SsruModel, TransformerModel},
};

/// Work limits (crates/marian-cpu/src/limits.rs:3-7); 0 disables a cap.
pub type Limits = ffi::marian_hip_limits;

/// The largest call a serving worker will make, for `HipEngine::reserve`.
pub type Capacity = ffi::marian_hip_capacity;

/// The reference's caps.
pub const REFERENCE_LIMITS: Limits = Limits {
    max_length_factor: 2,
    max_generation_steps: 256,
    max_position: 4096,
    max_batch: 256,
    max_source_tokens: 256,
    max_padded_cells: 65536,
};

pub struct HipEngine {
    raw: NonNull<ffi::marian_hip_engine>,
    _owner_thread: PhantomData<*const ()>,
}

fn op_error() -> String {
    // SAFETY: the library returns a NUL-terminated thread-local string.
    unsafe { CStr::from_ptr(ffi::marian_hip_last_op_error()) }.to_string_lossy().into_owned()
}

fn creation_error(code: c_int) -> BackendError {
    let msg = format!("marian-hip engine creation failed ({code}): {}", op_error());
    match code {
        ffi::ERR_MODEL => BackendError::Model(msg),
        ffi::ERR_INVALID_INPUT => BackendError::InvalidInput(msg),
        _ => BackendError::Inference(msg),
    }
}

impl HipEngine {
    /// The transformer-decoder graph (marian_hip_engine_create).
    pub fn new(model: &TransformerModel<'_>, limits: &Limits, device: i32) -> Result<Self, BackendError> {
        let (raw_model, _enc, _dec) = model.raw().map_err(BackendError::Model)?;
        let mut out = std::ptr::null_mut();
        // SAFETY: raw_model and the layer arrays it points into live until the
        // call returns; the library copies everything it keeps.
        let rc = unsafe { ffi::marian_hip_engine_create(&raw_model, limits, device, &mut out) };
        Self::wrap(rc, out)
    }

    /// The reference's Transformer-SSRU graph (marian_hip_engine_create_ssru).
    pub fn new_ssru(model: &SsruModel<'_>, limits: &Limits, device: i32) -> Result<Self, BackendError> {
        let (raw_model, _enc, _dec) = model.raw().map_err(BackendError::Model)?;
        let mut out = std::ptr::null_mut();
        // SAFETY: as in `new`.
        let rc = unsafe { ffi::marian_hip_engine_create_ssru(&raw_model, limits, device, &mut out) };
        Self::wrap(rc, out)
    }

    fn wrap(rc: c_int, out: *mut ffi::marian_hip_engine) -> Result<Self, BackendError> {
        match (rc, NonNull::new(out)) {
            (ffi::OK, Some(raw)) => Ok(Self { raw, _owner_thread: PhantomData }),
            (ffi::OK, None) => Err(creation_error(ffi::ERR_DEVICE)),
            (code, _) => Err(creation_error(code)),
        }
    }

    /// Q8CpuEngine::warmup (crates/marian-cpu/src/q8_engine.rs:349-351): the
    /// batch [2, 0] with at most 4 output tokens, so the first request does not
    /// pay for code-object loading or the first buffer allocations.
    pub fn warmup(&self) -> Result<(), String> {
        // SAFETY: self.raw is a live engine handle.
        match unsafe { ffi::marian_hip_warmup(self.raw.as_ptr()) } {
            ffi::OK => Ok(()),
            _ => Err(self.last_error()),
        }
    }

    /// Sizes the engine's decode buffers for calls up to `capacity`, so that
    /// such calls allocate nothing (`last_stats().allocations == 0`).
    pub fn reserve(&self, capacity: &Capacity) -> Result<(), String> {
        // SAFETY: self.raw is a live engine handle; capacity is read during the call.
        match unsafe { ffi::marian_hip_reserve(self.raw.as_ptr(), capacity) } {
            ffi::OK => Ok(()),
            _ => Err(self.last_error()),
        }
    }

    pub fn is_ready(&self) -> bool {
        // SAFETY: self.raw is a live engine handle.
        unsafe { ffi::marian_hip_is_ready(self.raw.as_ptr()) != 0 }
    }

    pub fn last_error(&self) -> String {
        // SAFETY: the engine owns the returned string until its next call.
        unsafe { CStr::from_ptr(ffi::marian_hip_last_error(self.raw.as_ptr())) }
            .to_string_lossy()
            .into_owned()
    }

    /// The BackendInfo fields the library fills, as JSON
    /// ({"name", "device", "model", "precision", "attention", "supports_batching"}).
    pub fn info_json(&self) -> String {
        let mut buf = vec![0u8; 1024];
        // SAFETY: buf is writable for its length.
        let rc = unsafe { ffi::marian_hip_info(self.raw.as_ptr(), buf.as_mut_ptr().cast(), buf.len()) };
        if rc != ffi::OK {
            return String::from("{}");
        }
        let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
        String::from_utf8_lossy(&buf[..end]).into_owned()
    }

    pub fn last_stats(&self) -> ffi::marian_hip_stats {
        let mut s = ffi::marian_hip_stats::default();
        // SAFETY: s is a valid out-parameter.
        unsafe { ffi::marian_hip_last_stats(self.raw.as_ptr(), &mut s) };
        s
    }

    /// Q8CpuEngine::translate_token_ids (crates/marian-cpu/src/q8_engine.rs:353-358):
    /// greedy outputs of a packed batch, scored over the whole vocabulary.
    pub fn translate_token_ids(
        &self,
        tokens: &[i32],
        offsets: &[u32],
        max_output_tokens: &[usize],
    ) -> Result<BatchOutput, String> {
        self.translate(tokens, offsets, max_output_tokens, None)
    }

    /// The same, each sentence scored over its own candidate list
    /// (LexicalShortlist::candidates of its source ids).
    pub fn translate_shortlisted(
        &self,
        tokens: &[i32],
        offsets: &[u32],
        max_output_tokens: &[usize],
        candidates: &[u32],
        candidate_offsets: &[u32],
    ) -> Result<BatchOutput, String> {
        self.translate(tokens, offsets, max_output_tokens, Some((candidates, candidate_offsets)))
    }

    fn translate(
        &self,
        tokens: &[i32],
        offsets: &[u32],
        max_output_tokens: &[usize],
        candidates: Option<(&[u32], &[u32])>,
    ) -> Result<BatchOutput, String> {
        if max_output_tokens.len() + 1 != offsets.len().max(1) {
            return Err("max_output_tokens does not match packed batch".into());
        }
        if let Some((_, coff)) = candidates {
            if coff.len() != offsets.len() {
                return Err("candidate offsets do not match packed batch".into());
            }
        }
        let budgets: Vec<u32> = max_output_tokens.iter().map(|&v| v.min(u32::MAX as usize) as u32).collect();
        // Σ min(budget, 4096) is always enough (positions cap every row at 4096).
        let mut cap = budgets.iter().map(|&v| v.min(4096) as usize).sum::<usize>().max(1);
        let mut out_offsets = vec![0u32; offsets.len()];
        loop {
            let mut out = vec![0i32; cap];
            let mut len = 0usize;
            // SAFETY: every slice is valid for the length passed with it.
            let rc = unsafe {
                match candidates {
                    None => ffi::marian_hip_translate_token_ids(
                        self.raw.as_ptr(),
                        tokens.as_ptr(),
                        tokens.len(),
                        offsets.as_ptr(),
                        offsets.len(),
                        budgets.as_ptr(),
                        0,
                        out.as_mut_ptr(),
                        out.len(),
                        out_offsets.as_mut_ptr(),
                        &mut len,
                    ),
                    Some((cand, coff)) => ffi::marian_hip_translate_shortlisted(
                        self.raw.as_ptr(),
                        tokens.as_ptr(),
                        tokens.len(),
                        offsets.as_ptr(),
                        offsets.len(),
                        budgets.as_ptr(),
                        0,
                        cand.as_ptr(),
                        coff.as_ptr(),
                        out.as_mut_ptr(),
                        out.len(),
                        out_offsets.as_mut_ptr(),
                        &mut len,
                    ),
                }
            };
            match rc {
                ffi::OK => {
                    out.truncate(len);
                    return Ok(BatchOutput { tokens: out, offsets: out_offsets });
                }
                ffi::ERR_BUFFER if len > cap => cap = len,
                _ => return Err(self.last_error()),
            }
        }
    }
}

impl Drop for HipEngine {
    fn drop(&mut self) {
        // SAFETY: the handle is live and dropped exactly once, on its owner thread.
        unsafe { ffi::marian_hip_engine_destroy(self.raw.as_ptr()) }
    }
}
