//! marian-hip: the AMD Instinct MI355X (gfx950) backend of marian-edge.
//!
//! The compute is libmarian_hip.so, hand-written HIP kernels behind the C ABI
//! of include/marian_hip.h; this crate is its Rust side: `ffi` declares the
//! ABI, `HipEngine` owns one device engine, `HipBackend` implements
//! marian-core's `TranslationBackend` over it with marian-cpu's text pipeline.

pub mod backend;
pub mod engine;
pub mod ffi;
pub mod model;

pub use backend::{HipBackend, HipTokenEngine, recommended_scheduler_config};
pub use engine::{Capacity, HipEngine, Limits, REFERENCE_LIMITS};
pub use model::{
    DecoderLayer, EncoderLayer, Linear, Norm, SsruDecoderLayer, SsruEncoderLayer, SsruModel, StaticLinear,
    TransformerModel,
};

/// Number of HIP devices visible to this process (0 without a GPU).
pub fn device_count() -> usize {
    // SAFETY: no arguments; the call only queries the runtime.
    let n = unsafe { ffi::marian_hip_device_count() };
    n.max(0) as usize
}
