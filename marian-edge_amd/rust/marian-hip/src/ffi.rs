//! Raw declarations of the engine-level C ABI in include/marian_hip.h.
//! Struct layouts are #[repr(C)] mirrors of the header's; every pointer
//! argument is host memory owned by the caller for the duration of the call.

#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int};

pub const MARIAN_HIP_ABI_VERSION: u32 = 4;

pub const OK: c_int = 0;
pub const ERR_INVALID_INPUT: c_int = -1;
pub const ERR_MODEL: c_int = -2;
pub const ERR_INFERENCE: c_int = -3;
pub const ERR_DEVICE: c_int = -4;
pub const ERR_BUFFER: c_int = -5;
pub const ERR_NOT_READY: c_int = -6;

pub const FLAG_IGNORE_EOS: u32 = 1 << 0;
pub const FLAG_NO_GENERATION_MASK: u32 = 1 << 1;
pub const FLAG_FAST_REDUCTIONS: u32 = 1 << 2;

#[repr(C)]
#[derive(Clone, Copy)]
pub struct marian_hip_linear {
    pub weight: *const i8,
    pub mult: *const f32,
    pub bias: *const f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct marian_hip_encoder_layer {
    pub qkv: marian_hip_linear,
    pub out: marian_hip_linear,
    pub ln1_scale: *const f32,
    pub ln1_bias: *const f32,
    pub ffn1: marian_hip_linear,
    pub ffn2: marian_hip_linear,
    pub ln2_scale: *const f32,
    pub ln2_bias: *const f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct marian_hip_decoder_layer {
    pub self_qkv: marian_hip_linear,
    pub self_out: marian_hip_linear,
    pub ln1_scale: *const f32,
    pub ln1_bias: *const f32,
    pub cross_q: marian_hip_linear,
    pub cross_kv: marian_hip_linear,
    pub cross_out: marian_hip_linear,
    pub ln2_scale: *const f32,
    pub ln2_bias: *const f32,
    pub ffn1: marian_hip_linear,
    pub ffn2: marian_hip_linear,
    pub ln3_scale: *const f32,
    pub ln3_bias: *const f32,
}

#[repr(C)]
pub struct marian_hip_model {
    pub vocab: u32,
    pub dim: u32,
    pub heads: u32,
    pub ffn_dim: u32,
    pub encoder_layers: u32,
    pub decoder_layers: u32,
    pub embedding: *const i8,
    pub embedding_mult: *const f32,
    pub output_bias: *const f32,
    pub encoder: *const marian_hip_encoder_layer,
    pub decoder: *const marian_hip_decoder_layer,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct marian_hip_static_linear {
    pub weight: *const i8,
    pub weight_mult: f32,
    pub act_mult: f32,
    pub bias: *const f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct marian_hip_ssru_encoder_layer {
    pub wq: marian_hip_static_linear,
    pub wk: marian_hip_static_linear,
    pub wv: marian_hip_static_linear,
    pub wo: marian_hip_static_linear,
    pub attn_ln_scale: *const f32,
    pub attn_ln_bias: *const f32,
    pub w1: marian_hip_static_linear,
    pub w2: marian_hip_static_linear,
    pub ffn_ln_scale: *const f32,
    pub ffn_ln_bias: *const f32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct marian_hip_ssru_decoder_layer {
    pub ssru_w: marian_hip_static_linear,
    pub ssru_wf: marian_hip_static_linear,
    pub ssru_ln_scale: *const f32,
    pub ssru_ln_bias: *const f32,
    pub wq: marian_hip_static_linear,
    pub wk: marian_hip_static_linear,
    pub wv: marian_hip_static_linear,
    pub wo: marian_hip_static_linear,
    pub context_ln_scale: *const f32,
    pub context_ln_bias: *const f32,
    pub w1: marian_hip_static_linear,
    pub w2: marian_hip_static_linear,
    pub ffn_ln_scale: *const f32,
    pub ffn_ln_bias: *const f32,
}

#[repr(C)]
pub struct marian_hip_ssru_model {
    pub source_vocab: u32,
    pub target_vocab: u32,
    pub dim: u32,
    pub heads: u32,
    pub ffn_dim: u32,
    pub encoder_layers: u32,
    pub decoder_layers: u32,
    pub encoder_embedding: *const i8,
    pub encoder_embedding_mult: f32,
    pub decoder_embedding: *const i8,
    pub decoder_embedding_mult: f32,
    pub output_act_mult: f32,
    pub output_bias: *const f32,
    pub encoder: *const marian_hip_ssru_encoder_layer,
    pub decoder: *const marian_hip_ssru_decoder_layer,
}

#[repr(C)]
#[derive(Clone, Copy, Default)]
pub struct marian_hip_limits {
    pub max_length_factor: u32,
    pub max_generation_steps: u32,
    pub max_position: u32,
    pub max_batch: u32,
    pub max_source_tokens: u32,
    pub max_padded_cells: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Default, Debug)]
pub struct marian_hip_stats {
    pub total_ms: f64,
    pub encoder_ms: f64,
    pub decode_ms: f64,
    pub vocab_kernel_ms: f64,
    pub vocab_kernel_launches: u32,
    pub decode_steps: u32,
    pub max_active_rows: u32,
    pub generated_tokens: u64,
    pub launched_steps: u32,
    pub allocations: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Default, Debug)]
pub struct marian_hip_capacity {
    pub sentences: u32,
    pub source_tokens: u32,
    pub output_tokens: u32,
    pub steps: u32,
    pub candidate_ids: u32,
    pub max_candidates: u32,
}

/// Opaque engine handle.
#[repr(C)]
pub struct marian_hip_engine {
    _private: [u8; 0],
}

extern "C" {
    pub fn marian_hip_engine_create(
        model: *const marian_hip_model,
        limits: *const marian_hip_limits,
        device: c_int,
        out_engine: *mut *mut marian_hip_engine,
    ) -> c_int;
    pub fn marian_hip_engine_create_ssru(
        model: *const marian_hip_ssru_model,
        limits: *const marian_hip_limits,
        device: c_int,
        out_engine: *mut *mut marian_hip_engine,
    ) -> c_int;
    pub fn marian_hip_engine_destroy(engine: *mut marian_hip_engine);
    pub fn marian_hip_translate_token_ids(
        engine: *mut marian_hip_engine,
        tokens: *const i32,
        n_tokens: usize,
        offsets: *const u32,
        n_offsets: usize,
        max_output_tokens: *const u32,
        flags: u32,
        out_tokens: *mut i32,
        out_cap: usize,
        out_offsets: *mut u32,
        out_len: *mut usize,
    ) -> c_int;
    pub fn marian_hip_translate_shortlisted(
        engine: *mut marian_hip_engine,
        tokens: *const i32,
        n_tokens: usize,
        offsets: *const u32,
        n_offsets: usize,
        max_output_tokens: *const u32,
        flags: u32,
        candidates: *const u32,
        candidate_offsets: *const u32,
        out_tokens: *mut i32,
        out_cap: usize,
        out_offsets: *mut u32,
        out_len: *mut usize,
    ) -> c_int;
    pub fn marian_hip_warmup(engine: *mut marian_hip_engine) -> c_int;
    pub fn marian_hip_reserve(engine: *mut marian_hip_engine, capacity: *const marian_hip_capacity) -> c_int;
    pub fn marian_hip_validate_batch(
        limits: *const marian_hip_limits,
        source_vocab: u32,
        target_vocab: u32,
        tokens: *const i32,
        n_tokens: usize,
        offsets: *const u32,
        n_offsets: usize,
        candidates: *const u32,
        candidate_offsets: *const u32,
        msg: *mut c_char,
        msg_cap: usize,
    ) -> c_int;
    pub fn marian_hip_is_ready(engine: *const marian_hip_engine) -> c_int;
    pub fn marian_hip_last_error(engine: *const marian_hip_engine) -> *const c_char;
    pub fn marian_hip_last_op_error() -> *const c_char;
    pub fn marian_hip_info(engine: *const marian_hip_engine, buf: *mut c_char, cap: usize) -> c_int;
    pub fn marian_hip_last_stats(engine: *const marian_hip_engine, stats: *mut marian_hip_stats) -> c_int;
    pub fn marian_hip_device_count() -> c_int;
    pub fn marian_hip_build_id() -> *const c_char;
}
