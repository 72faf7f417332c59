/*
 * marian_hip.h — C ABI of the MI355X (gfx950) Q8 greedy translation backend.
 *
 * The ABI sits at the reference's token-level engine boundary, below its
 * text adapter.  Reference interfaces each entry point replaces (paths relative
 * to the marian-edge checkout):
 *
 *   marian_hip_engine_create   Q8CpuEngine::load / load_owned
 *                              crates/marian-cpu/src/q8_engine.rs:162-174, 828-877
 *                              (the caller hands over parsed, already-quantized
 *                              weights; the engine copies them to HBM)
 *   marian_hip_translate_token_ids
 *                              Q8CpuEngine::translate_token_ids
 *                              crates/marian-cpu/src/q8_engine.rs:353-466, and the
 *                              CpuTokenEngine trait crates/marian-cpu/src/backend.rs:48-57;
 *                              output = BatchOutput crates/marian-cpu/src/engine.rs:80-85
 *   marian_hip_is_ready        TranslationBackend::is_ready
 *                              crates/marian-core/src/backend.rs:16-18
 *   marian_hip_info            TranslationBackend::info / BackendInfo
 *                              crates/marian-core/src/backend.rs:8, types.rs:49-58
 *   marian_hip_last_error      BackendError message (types.rs:60-70); the wasm
 *                              ABI's error slot (marian-worker-wasm/src/lib.rs:381-389)
 *   marian_hip_engine_destroy  Drop of the engine on its owner thread
 *                              (crates/marian-core/src/backend.rs:3-6)
 *   marian_hip_engine_create_ssru
 *                              Q8CpuEngine::from_model over the reference's own
 *                              Transformer-SSRU graph, q8_engine.rs:195-212, 828-877
 *   marian_hip_translate_shortlisted
 *                              translate_token_ids with the lexical shortlist's
 *                              candidates, q8_engine.rs:361-362, 576-584, 749-790
 *   marian_hip_warmup          Q8CpuEngine::warmup q8_engine.rs:349-351 (called by
 *                              the backends at load, marian-cpu/src/backend.rs:448,
 *                              812, 853, 896)
 *   marian_hip_validate_batch  Q8CpuEngine::validate_batch q8_engine.rs:468-509 and
 *                              validate_work_shape :1103-1119, host only
 *   marian_hip_reserve         no counterpart: sizes the engine's grow-only decode
 *                              buffers (the reference's pooled scratch,
 *                              q8_engine.rs:733-747) for a serving worker's
 *                              largest batch at load time
 *
 * Op-level entry points (device pointers, caller's stream) replace the
 * reference's building blocks and exist so each kernel can be checked and timed
 * on its own:
 *   marian_hip_quantize_rows   quantize_symmetric_u8_into q8_gemm.rs:569-590
 *   marian_hip_q8_linear       Q8Linear::run_into q8_gemm.rs:380-448 (+ the
 *                              exact kernel q8_avx2.rs:125-229)
 *   marian_hip_q8_linear_static  the same with the static activation multiplier
 *                              of the reference's Q8 models (legacy_q8.rs:544-552)
 *   marian_hip_residual_layer_norm  residual_layer_norm_into tensor.rs:132-155
 *   marian_hip_ssru_layer_norm ssru_update_layer_norm_into tensor.rs:184-218
 *   marian_hip_attention       attention_into tensor.rs:251-318
 *   marian_hip_vocab_argmax    select_token q8_engine.rs:749-790
 *   marian_hip_candidate_argmax  select_token over a lexical shortlist's candidates
 *                              (shortlist.rs:150-198)
 *   marian_hip_positions       sinusoidal_positions crates/marian-model/src/position.rs:5-21
 * The op-level entry points that need intermediate device buffers keep them
 * in library scratch, one set per (device, stream), kept until the process
 * ends: calls on different streams do not share it, and calls on one stream
 * are ordered by that stream (two threads that issue calls on the same
 * stream at once must serialize their calls themselves).
 * marian_hip_vocab_argmax_noalloc has no reference counterpart (see there).
 *
 * Threading: one engine handle belongs to one owner thread (the reference
 * backend is deliberately !Send, backend.rs:3-6).  The engine owns one HIP
 * stream.  Nothing here locks.
 *
 * Status codes: 0 success; negative values below.  Invalid input and
 * output-buffer errors do not affect readiness; a HIP runtime error makes the
 * engine permanently not ready (like the Metal backend's poisoning,
 * crates/marian-metal/src/engine.rs:113-125).
 */
#ifndef MARIAN_HIP_H
#define MARIAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MARIAN_HIP_ABI_VERSION 4 /* 2: marian_hip_attention takes head_dim;
                                    3: the Transformer-SSRU engine, shortlisted translate;
                                    4: warmup, reserve, validate_batch, stats
                                       launched_steps and allocations */

enum {
  MARIAN_HIP_OK = 0,
  MARIAN_HIP_ERR_INVALID_INPUT = -1, /* BackendError::InvalidInput */
  MARIAN_HIP_ERR_MODEL = -2,         /* BackendError::Model */
  MARIAN_HIP_ERR_INFERENCE = -3,     /* BackendError::Inference (e.g. non-finite activation) */
  MARIAN_HIP_ERR_DEVICE = -4,        /* HIP runtime failure; engine becomes not ready */
  MARIAN_HIP_ERR_BUFFER = -5,        /* caller's output buffer too small */
  MARIAN_HIP_ERR_NOT_READY = -6      /* engine was poisoned by an earlier device error */
};

/* Translate flags. */
enum {
  MARIAN_HIP_FLAG_IGNORE_EOS = 1u << 0,         /* token 0 does not finish a row */
  MARIAN_HIP_FLAG_NO_GENERATION_MASK = 1u << 1, /* also score ids 1 and 7..38
                                                   (shortlist.rs:169-176 masks them) */
  /* Opt-in, no counterpart in the reference: the decoder's LayerNorm sums and
   * softmax denominators as 64 lane partials (lane l: elements l, l + 64, ...
   * in order from 0.0) combined by an xor butterfly over lane distances 32,
   * 16, ..., 1, instead of the reference's left-to-right folds
   * (tensor.rs:372-385, 745-754).  The encoder, every other sum, exp and the
   * integer work are unchanged.  Results then differ from the reference in the
   * last bits of those sums; greedy outputs are compared with the exact mode in
   * tests/test_gpu_fast.py.  Transformer graph only (the SSRU engine rejects
   * it). */
  MARIAN_HIP_FLAG_FAST_REDUCTIONS = 1u << 2
};

/* One Q8 dense layer.  weight is [out, in] int8, input-contiguous (the
 * reference's canonical layout, legacy_q8.rs:82-89); mult[n] is the
 * per-output-channel multiplier with real_w = q / mult (legacy_q8.rs:466-495
 * uses one multiplier per tensor); bias is fp32 [out]. */
typedef struct {
  const int8_t* weight;
  const float* mult;
  const float* bias;
} marian_hip_linear;

typedef struct {
  marian_hip_linear qkv; /* [3d, d] rows Q, K, V (q8_engine.rs:528-530 as one GEMM) */
  marian_hip_linear out; /* [d, d] */
  const float* ln1_scale;
  const float* ln1_bias;
  marian_hip_linear ffn1; /* [F, d], ReLU */
  marian_hip_linear ffn2; /* [d, F] */
  const float* ln2_scale;
  const float* ln2_bias;
} marian_hip_encoder_layer;

typedef struct {
  marian_hip_linear self_qkv; /* [3d, d] */
  marian_hip_linear self_out; /* [d, d] */
  const float* ln1_scale;
  const float* ln1_bias;
  marian_hip_linear cross_q;   /* [d, d] (q8_engine.rs:410) */
  marian_hip_linear cross_kv;  /* [2d, d] on the encoder output (q8_engine.rs:560-567) */
  marian_hip_linear cross_out; /* [d, d] */
  const float* ln2_scale;
  const float* ln2_bias;
  marian_hip_linear ffn1;
  marian_hip_linear ffn2;
  const float* ln3_scale;
  const float* ln3_bias;
} marian_hip_decoder_layer;

/* Host-side model description; every pointer is host memory owned by the
 * caller and only read during marian_hip_engine_create. */
typedef struct {
  uint32_t vocab, dim, heads, ffn_dim, encoder_layers, decoder_layers;
  const int8_t* embedding;     /* [vocab, dim]: source and target embedding and
                                  the tied output projection */
  const float* embedding_mult; /* [vocab] per-row multiplier */
  const float* output_bias;    /* [vocab] */
  const marian_hip_encoder_layer* encoder;
  const marian_hip_decoder_layer* decoder;
} marian_hip_model;

/* Work limits (crates/marian-cpu/src/limits.rs:3-7 and q8_engine.rs:369-379).
 * 0 disables a cap.  Reference values: factor 2, steps 256, position 4096,
 * batch 256, source tokens 256, padded cells 65536. */
typedef struct {
  uint32_t max_length_factor;
  uint32_t max_generation_steps;
  uint32_t max_position; /* must be <= 4096 (the position table) */
  uint32_t max_batch;
  uint32_t max_source_tokens;
  uint64_t max_padded_cells;
} marian_hip_limits;

typedef struct marian_hip_engine marian_hip_engine;

/* Copies the model to device `device` and builds the position table.
 * Supported geometry: 1-8 heads of width 64 or 48 (dim = 64 * heads or
 * 48 * heads, a multiple of 64, at most 512: 384 with 8 heads of 48 is the
 * reference's small production shape), ffn_dim a multiple of 64 up to 2048,
 * at least one decoder layer, vocab < 2^31.  The
 * model is checked before the device is touched: every weight multiplier
 * finite and positive, no weight -128, every tensor present (Q8Linear::new,
 * crates/marian-cpu/src/q8_gemm.rs:96-110); otherwise MARIAN_HIP_ERR_MODEL,
 * with the reason in marian_hip_last_op_error() on the calling thread. */
int marian_hip_engine_create(const marian_hip_model* model, const marian_hip_limits* limits,
                             int device, marian_hip_engine** out_engine);
void marian_hip_engine_destroy(marian_hip_engine* engine);

/* Greedy translation of a packed batch.
 *   tokens[n_tokens]: source ids; offsets[n_offsets]: cu_seqlens with
 *   offsets[0] = 0, offsets[B] = n_tokens, every row >= 1 token;
 *   max_output_tokens[B]: requested budget per row.
 * Outputs (host memory): out_tokens (capacity out_cap) receives the generated
 * ids of every row back to back, including a final EOS 0 when one is emitted;
 * out_offsets[B+1] the row boundaries; *out_len the total.  On
 * MARIAN_HIP_ERR_BUFFER, *out_len holds the capacity needed.  The bound
 * sum_b min(max_output_tokens[b], caps) is always enough. */
int marian_hip_translate_token_ids(marian_hip_engine* engine, const int32_t* tokens,
                                   size_t n_tokens, const uint32_t* offsets, size_t n_offsets,
                                   const uint32_t* max_output_tokens, uint32_t flags,
                                   int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets,
                                   size_t* out_len);

/* marian_hip_translate_token_ids that also copies out intermediate values, for
 * checks below the token level.  No counterpart in the reference: it exposes
 * what the reference's own tests read from its engine (the encoder states of
 * Q8CpuEngine::encode, q8_engine.rs:511-574, and the logits that select_token
 * scores, q8_engine.rs:749-790).  Same arguments and results as the plain call,
 * plus (host memory, each may be NULL):
 *   enc_out[n_tokens, dim]   the final encoder state of every packed row (fp32);
 *   logits_out[B, vocab]     for decode step `probe_step` (0-based), the logits
 *                            of every row still active at that step, masked ids
 *                            -inf (rows not active there are left untouched);
 *   active_out[B]            1 for the rows whose logits were written, else 0
 *                            (needs logits_out).
 * The extra copies synchronize the stream, so its timings are not
 * representative. */
int marian_hip_translate_probe(marian_hip_engine* engine, const int32_t* tokens, size_t n_tokens,
                               const uint32_t* offsets, size_t n_offsets,
                               const uint32_t* max_output_tokens, uint32_t flags,
                               int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets,
                               size_t* out_len, uint32_t probe_step, float* enc_out,
                               float* logits_out, uint8_t* active_out);

/* ---- The reference's own graph: Transformer encoder, SSRU decoder ----
 *
 * Q8CpuEngine's fixed graph (crates/marian-cpu/src/q8_engine.rs:76-114,
 * 511-574, 382-451) over a Marian binary model: every dense layer has ONE
 * weight multiplier and ONE static activation multiplier (the intgemm8
 * payload's quantization multiplier and the <name>_QuantMultA tensor,
 * legacy_q8.rs:390-403, 544-552, 646-674), so a layer computes
 *   q = clamp(rne(x * act_mult), -127, 127),  y = acc * (1 / (act_mult * weight_mult)) + bias
 * (q8_gemm.rs:380-448, 569-590).  Encoder and decoder embeddings are separate
 * tables, each with one multiplier; the decoder embedding is also the tied
 * output projection, whose input is quantized with output_act_mult.  A decoder
 * layer is SSRU (tensor.rs:184-218), then cross-attention, then the FFN. */
typedef struct {
  const int8_t* weight; /* [out, in] int8 in [-127, 127], input-contiguous */
  float weight_mult;    /* real weight = q / weight_mult */
  float act_mult;       /* static activation multiplier */
  const float* bias;    /* [out], or NULL: no bias (adds 0.0, q8_gemm.rs:444) */
} marian_hip_static_linear;

typedef struct {
  marian_hip_static_linear wq, wk, wv, wo; /* [d, d] each (q8_engine.rs:528-544) */
  const float* attn_ln_scale;
  const float* attn_ln_bias;
  marian_hip_static_linear w1; /* [F, d], ReLU */
  marian_hip_static_linear w2; /* [d, F] */
  const float* ffn_ln_scale;
  const float* ffn_ln_bias;
} marian_hip_ssru_encoder_layer;

typedef struct {
  marian_hip_static_linear ssru_w;  /* [d, d] candidate, no bias (q8_engine.rs:394, 942-958) */
  marian_hip_static_linear ssru_wf; /* [d, d] forget gate input (q8_engine.rs:395) */
  const float* ssru_ln_scale;
  const float* ssru_ln_bias;
  marian_hip_static_linear wq, wk, wv, wo; /* context attention; wk/wv on the encoder output */
  const float* context_ln_scale;
  const float* context_ln_bias;
  marian_hip_static_linear w1, w2;
  const float* ffn_ln_scale;
  const float* ffn_ln_bias;
} marian_hip_ssru_decoder_layer;

typedef struct {
  uint32_t source_vocab, target_vocab, dim, heads, ffn_dim, encoder_layers, decoder_layers;
  const int8_t* encoder_embedding; /* [source_vocab, dim] */
  float encoder_embedding_mult;
  const int8_t* decoder_embedding; /* [target_vocab, dim]; also the output projection */
  float decoder_embedding_mult;
  float output_act_mult;           /* decoder_output_activation_mult, the QuantMultA of
                                      decoder_Wemb (q8_engine.rs:834-836) */
  const float* output_bias;        /* [target_vocab] */
  const marian_hip_ssru_encoder_layer* encoder;
  const marian_hip_ssru_decoder_layer* decoder;
} marian_hip_ssru_model;

/* Engine for the graph above (Q8CpuEngine::from_model, q8_engine.rs:195-212).
 * Same geometry rules as marian_hip_engine_create; multipliers must be finite
 * and positive, weights in [-127, 127].  marian_hip_translate_token_ids and
 * marian_hip_translate_probe on it score the full target vocabulary with the
 * generation mask, which is what the reference's engine does without a
 * shortlist file (LexicalShortlist::from_bytes(None), shortlist.rs:55-65). */
int marian_hip_engine_create_ssru(const marian_hip_ssru_model* model,
                                  const marian_hip_limits* limits, int device,
                                  marian_hip_engine** out_engine);

/* marian_hip_translate_token_ids with per-sentence output candidates: sentence
 * b is scored only over candidates[candidate_offsets[b] .. candidate_offsets[b+1]),
 * in list order, the first maximum winning (select_token over
 * LexicalShortlist::candidates: prepare_candidates, q8_engine.rs:576-584, and
 * :749-790).  The lists come from the caller (the reference builds them from
 * the source ids with its shortlist, shortlist.rs:150-198, sorted and without
 * repeats); no generation mask is applied to them.  An empty list, a list that
 * is not strictly ascending or an id >= the target vocabulary is
 * MARIAN_HIP_ERR_INVALID_INPUT.  Works on either engine kind. */
int marian_hip_translate_shortlisted(marian_hip_engine* engine, const int32_t* tokens,
                                     size_t n_tokens, const uint32_t* offsets, size_t n_offsets,
                                     const uint32_t* max_output_tokens, uint32_t flags,
                                     const uint32_t* candidates,
                                     const uint32_t* candidate_offsets, int32_t* out_tokens,
                                     size_t out_cap, uint32_t* out_offsets, size_t* out_len);

/* Q8CpuEngine::warmup (crates/marian-cpu/src/q8_engine.rs:349-351): translates
 * the one-sentence batch [2, 0] with at most 4 output tokens, so the first
 * request does not pay for loading the kernels' code objects or allocating
 * the decode buffers.  The reference's backends call it once after loading
 * (crates/marian-cpu/src/backend.rs:448, 812, 853, 896); a failure there is
 * BackendError::Inference.  Needs a vocabulary of at least 3 ids. */
int marian_hip_warmup(marian_hip_engine* engine);

/* Capacity of a serving worker's largest call, for marian_hip_reserve. */
typedef struct {
  uint32_t sentences;      /* sentences (packed rows) of one call, 1..4096 */
  uint32_t source_tokens;  /* source tokens of one call (sum over sentences) */
  uint32_t output_tokens;  /* sum over sentences of the generation limits */
  uint32_t steps;          /* longest generation limit */
  uint32_t candidate_ids;  /* shortlisted calls: candidate ids of one call (0: none) */
  uint32_t max_candidates; /* shortlisted calls: longest candidate list */
} marian_hip_capacity;
/* No counterpart in the reference (its scratch is pooled per call,
 * q8_engine.rs:733-747, and grows on the heap as needed): sizes the engine's
 * grow-only device buffers and pinned host staging for calls up to
 * `capacity`, so that such calls allocate nothing (marian_hip_stats.allocations
 * = 0) and a serving worker never allocates in the middle of a request.
 * Larger calls still work and grow the buffers.  Buffers never shrink. */
int marian_hip_reserve(marian_hip_engine* engine, const marian_hip_capacity* capacity);

/* The host checks marian_hip_translate_token_ids and
 * marian_hip_translate_shortlisted run before they touch the device, with no
 * engine or device: Q8CpuEngine::validate_batch (q8_engine.rs:468-509) and
 * validate_work_shape (:1103-1119) under `limits` (NULL: the reference's
 * values; 0 disables a cap), source ids below source_vocab, and, when
 * candidate_offsets is given, candidate lists that are non-empty, strictly
 * ascending (as LexicalShortlist::candidates returns them,
 * shortlist.rs:150-198) and below target_vocab.  Returns MARIAN_HIP_OK or
 * MARIAN_HIP_ERR_INVALID_INPUT with the reason written to msg (may be NULL). */
int marian_hip_validate_batch(const marian_hip_limits* limits, uint32_t source_vocab,
                              uint32_t target_vocab, const int32_t* tokens, size_t n_tokens,
                              const uint32_t* offsets, size_t n_offsets,
                              const uint32_t* candidates, const uint32_t* candidate_offsets,
                              char* msg, size_t msg_cap);

int marian_hip_is_ready(const marian_hip_engine* engine);
/* Last error message of this engine ("" if none); valid until the next call. */
const char* marian_hip_last_error(const marian_hip_engine* engine);
/* BackendInfo fields, e.g. name "hip", device "AMD Instinct MI355X (gfx950)",
 * precision "q8". Writes a NUL-terminated JSON object into buf. */
int marian_hip_info(const marian_hip_engine* engine, char* buf, size_t cap);

/* Timing of the last translate call, in milliseconds (events on the engine's
 * stream): total (from the upload of the packed batch to the generated tokens
 * in host memory), encoder (upload included), decode loop, the summed device
 * time of the vocabulary projection + argmax kernel and the number of its
 * launches, and the number of decode steps that ran on rows.
 * launched_steps counts the steps enqueued: rows that end on EOS are seen by
 * the host a few steps late, and steps enqueued after the last row finished
 * run on no rows.  allocations counts the device and pinned host buffers the
 * call had to (re)allocate: 0 once marian_hip_reserve (or an earlier call)
 * sized them for the batch. */
typedef struct {
  double total_ms, encoder_ms, decode_ms;
  double vocab_kernel_ms;
  uint32_t vocab_kernel_launches;
  uint32_t decode_steps;
  uint32_t max_active_rows;
  uint64_t generated_tokens;
  uint32_t launched_steps;
  uint32_t allocations;
} marian_hip_stats;
int marian_hip_last_stats(const marian_hip_engine* engine, marian_hip_stats* stats);
/* Timing of later translate calls (default 0: none).
 * MARIAN_HIP_TIME_STEPS: one event at the end of every decode step
 *   (marian_hip_last_step_trace reports the times); cheap.
 * MARIAN_HIP_TIME_KERNELS: the vocabulary, attention-block and decode
 *   attention launches record events from their own dispatches (marian_hip_stats.vocab_kernel_ms and
 *   marian_hip_last_kernel_trace are filled); this adds several microseconds
 *   of device time per timed launch, so throughput is measured without it. */
#define MARIAN_HIP_TIME_STEPS 1u
#define MARIAN_HIP_TIME_KERNELS 2u
int marian_hip_set_timing(marian_hip_engine* engine, uint32_t flags);
/* Kernel kinds of marian_hip_last_kernel_trace. */
#define MARIAN_HIP_KERNEL_VOCAB 0       /* vocabulary projection + argmax partials */
#define MARIAN_HIP_KERNEL_SELF_BLOCK 1  /* decoder self-attention block */
#define MARIAN_HIP_KERNEL_CROSS_BLOCK 2 /* decoder cross-attention block */
#define MARIAN_HIP_KERNEL_SELF_ATTN 3   /* decoder self-attention kernel (steps the blocks do not cover) */
#define MARIAN_HIP_KERNEL_CROSS_ATTN 4  /* decoder cross-attention kernel (likewise) */
/* With MARIAN_HIP_TIME_KERNELS: one record per timed decode launch of the last
 * translate call, in launch order: its kind, decode step, decoder layer and
 * device duration in microseconds (from events its own dispatch recorded).
 * Writes min(cap, launches) entries and the launch count to *n. */
int marian_hip_last_kernel_trace(const marian_hip_engine* engine, uint32_t* kind, uint32_t* step,
                                 uint32_t* layer, float* us, size_t cap, size_t* n);
/* Per decode step of the last translate call: the number of active rows the
 * step ran on and, with MARIAN_HIP_TIME_STEPS, the device time at which
 * the step's tokens were final (ms from the batch start, else 0).  Writes
 * min(cap, steps) entries and the step count to *n_steps.  A row that
 * produced c tokens completed at step c-1. */
int marian_hip_last_step_trace(const marian_hip_engine* engine, uint32_t* active_rows,
                               float* step_end_ms, size_t cap, size_t* n_steps);

/* ---- op-level entry points: device pointers, `stream` is a hipStream_t or
 * NULL for the default stream.  They return MARIAN_HIP_ERR_INVALID_INPUT for
 * shapes the kernels do not support. ------------------------------------- */

/* q[m,:] = clamp(rne(x[m,:]*a[m]), -127, 127), a[m] = 127/max|x[m,:]| (1 for
 * an all-zero row).  err (device int, may be NULL) is set to 1 when a
 * non-finite value is seen. */
int marian_hip_quantize_rows(const float* x, int64_t rows, int64_t cols, int8_t* q, float* a,
                             int* err, void* stream);

/* y = (x quantized per row) @ W^T dequantized + bias (+ReLU).
 * x fp32 [M,K] (NULL when xq/xa are given pre-quantized), W int8 [N,K],
 * out_i32 [M,N] optional (exact accumulators), out_f32 [M,N] optional.
 * K must be a multiple of 64. */
int marian_hip_q8_linear(const float* x, const int8_t* xq, const float* xa, int64_t M,
                         int64_t K, const int8_t* w, const float* w_mult, const float* bias,
                         int64_t N, int relu, int32_t* out_i32, float* out_f32, int* err,
                         void* stream);

/* marian_hip_q8_linear with the reference's static activation multiplier
 * (Q8Linear::run_into with activation_quant_mult, q8_gemm.rs:380-448 and
 * quantize_symmetric_u8_into :569-590; the model's per-tensor QuantMultA,
 * legacy_q8.rs:544-552): q = clamp(rne(x * act_mult), -127, 127) for every row,
 * y = acc * (1 / (act_mult * w_mult[n])) + bias[n].  act_mult must be finite
 * and positive; a non-finite x sets *err. */
int marian_hip_q8_linear_static(const float* x, int64_t M, int64_t K, float act_mult,
                                const int8_t* w, const float* w_mult, const float* bias, int64_t N,
                                int relu, int32_t* out_i32, float* out_f32, int* err, void* stream);

/* SSRU update + LayerNorm of the reference's SSRU decoder
 * (ssru_update_layer_norm_into, crates/marian-cpu/src/tensor.rs:184-218):
 * per element gate = 1 / (1 + exp(-forget)), state = gate * state +
 * (1 - gate) * cand (in place); out = LN(relu(state) + residual) (eps 1e-6),
 * optionally quantized per row into q / a.  All rows [rows, dim], dim a
 * multiple of 64 up to 1024. */
int marian_hip_ssru_layer_norm(const float* cand, const float* forget, float* state,
                               const float* residual, const float* scale, const float* bias,
                               int64_t rows, int64_t dim, float* out, int8_t* q, float* a, int* err,
                               void* stream);

/* out = LN(x + r) (eps 1e-6), optional int8 quantization of out (q, a). */
int marian_hip_residual_layer_norm(const float* x, const float* r, const float* scale,
                                   const float* bias, int64_t rows, int64_t dim, float* out,
                                   int8_t* q, float* a, int* err, void* stream);

/* Variable-length attention: query row i belongs to sequence seq_of_row[i]
 * and attends over key rows [cu_k[s], cu_k[s+1]); max_keys bounds every range
 * (at most 4096); heads <= 16 of width head_dim (64, or 48 as in the
 * reference's 384-wide model; head h is columns [h*head_dim, (h+1)*head_dim)).
 * Row strides in elements.  in_bf16 != 0 reads q/k/v as bfloat16 (converted
 * exactly to fp32); out is fp32 [rows, heads*head_dim].
 * n_seqs > 0 declares packed self-attention: the query rows are the key rows
 * (row i lies in [cu_k[s], cu_k[s+1]) for s = seq_of_row[i]), cu_k has
 * n_seqs + 1 entries, rows = cu_k[n_seqs]; then ranges of at most 256 keys
 * run on the kernel that stages each sequence's keys once per 16 queries.
 * n_seqs = 0: one (row, head) wave each, for any query/key pairing. */
int marian_hip_attention(const void* q, int64_t ldq, const void* k, const void* v, int64_t ldkv,
                         const int32_t* seq_of_row, const uint32_t* cu_k, int64_t n_seqs,
                         int64_t rows, int64_t heads, int64_t head_dim, int64_t max_keys,
                         int in_bf16, float* out, int64_t ldo, void* stream);

/* Vocabulary projection + bias + generation mask + argmax per row:
 * token[m] = argmax_v (acc[m,v] * (1/(xa[m]*mult[v])) + bias[v]) with ties to
 * the lowest id; logits [M,V] optional.  xq/xa are the quantized rows;
 * K (the model width) must be a multiple of 64 and at most 512. */
int marian_hip_vocab_argmax(const int8_t* xq, const float* xa, int64_t M, int64_t K,
                            const int8_t* emb, const float* emb_mult, const float* bias,
                            int64_t V, uint32_t flags, int32_t* token, float* logits,
                            void* stream);

/* Output scoring over per-row candidate lists, e.g. a lexical shortlist's
 * (select_token over LexicalShortlist::candidates, q8_engine.rs:749-790 and
 * crates/marian-model/src/shortlist.rs:150-198): row m scores the vocabulary
 * ids cand[cand_offsets[m] .. cand_offsets[m+1]) (device arrays, ids sorted
 * ascending, every list non-empty) as logit = acc * (1/(xa[m]*mult[id])) +
 * bias[id] and token[m] = the first maximum in list order (a row whose logits
 * are all -inf or NaN gets its first candidate).  max_cands bounds every list's
 * length (grid size).  logits (optional) receives each candidate's logit at
 * its position in cand.  An id >= V sets *err (may be NULL) and is skipped.
 * K a multiple of 64 up to 4096, M <= 65535. */
int marian_hip_candidate_argmax(const int8_t* xq, const float* xa, int64_t M, int64_t K,
                                const int8_t* emb, const float* emb_mult, const float* bias,
                                int64_t V, const uint32_t* cand, const uint32_t* cand_offsets,
                                int64_t max_cands, int32_t* token, float* logits, int* err,
                                void* stream);

/* marian_hip_vocab_argmax without any device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops that forbid hipMalloc).  Same
 * arguments and results; the per-row partial argmax keys live in a fixed
 * 1 MiB device array of the library (131072 keys, one per row and 128-column
 * vocabulary group: M * ceil(V / 128) <= 131072, e.g. up to 524 rows at
 * V = 32000; larger inputs return MARIAN_HIP_ERR_INVALID_INPUT and launch
 * nothing).  Each device holds its own copy of that array until the process
 * ends, and every call on a device shares it: calls that overlap on one
 * device (two streams, two threads) race and must be serialized by the
 * caller.  Nothing in it needs clearing between calls. */
int marian_hip_vocab_argmax_noalloc(const int8_t* xq, const float* xa, int64_t M, int64_t K,
                                    const int8_t* emb, const float* emb_mult, const float* bias,
                                    int64_t V, uint32_t flags, int32_t* token, float* logits,
                                    void* stream);

/* Host: sinusoidal position table [count, dim] (fp32), as the engine builds it. */
int marian_hip_positions(uint32_t dim, uint32_t count, float* out);

#ifdef __cplusplus
}
#endif
#endif
