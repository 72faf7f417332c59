/*
 * oracle.h — CPU restatement of marian-edge's `marian-cpu` Q8 greedy
 * translation path.  TEST INFRASTRUCTURE ONLY: this library is the checker
 * that the HIP backend is compared against, and the CPU baseline it is timed
 * beside.  Nothing in the product (the marian-hip library or its Python
 * mirror) may link, load or call it.
 *
 * The model/limits structs below have the same field order as the ones in
 * include/marian_hip.h so one host-side description can be handed to both
 * libraries; the oracle does not include that header on purpose (it must not
 * depend on product code).
 *
 * Reference semantics followed (paths relative to the reference checkout):
 *   quantize            crates/marian-cpu/src/q8_gemm.rs:569-590
 *   exact i32 GEMM      crates/marian-cpu/src/q8_gemm.rs:539-553 (closed form),
 *                       crates/marian-cpu/src/q8_avx2.rs:125-358 (x86 kernel)
 *   dequant + bias      crates/marian-cpu/src/q8_gemm.rs:438-446
 *   residual LayerNorm  crates/marian-cpu/src/tensor.rs:132-155, 372-425
 *   SSRU + LayerNorm    crates/marian-cpu/src/tensor.rs:184-218, 718-724
 *   static activation   crates/marian-cpu/src/legacy_q8.rs:544-552 (QuantMultA)
 *   attention           crates/marian-cpu/src/tensor.rs:251-318, 594-637, 745-754
 *   positions           crates/marian-model/src/position.rs:5-21
 *   embedding           crates/marian-cpu/src/q8_engine.rs:53-74, 586-630
 *   greedy loop         crates/marian-cpu/src/q8_engine.rs:353-466
 *   output scoring      crates/marian-cpu/src/q8_engine.rs:749-790
 *   generation mask     crates/marian-model/src/shortlist.rs:169-176
 *
 * Reduction order.  `order` selects how fp32 sums are rounded:
 *   ORACLE_ORDER_REFERENCE (1): the x86 reference order (strictly sequential
 *     LayerNorm and softmax sums, the C library's expf).  This is the mode
 *     the HIP kernels reproduce bit for bit.
 *   ORACLE_ORDER_CANONICAL (0): an alternative (64 strided lane partials +
 *     xor butterfly, exp via a double-precision Cody-Waite/Taylor routine),
 *     kept to measure how sensitive greedy outputs are to the fp32 summation
 *     order.
 *   ORACLE_ORDER_FAST_DECODER (2): the order of the HIP engine's opt-in
 *     MARIAN_HIP_FLAG_FAST_REDUCTIONS: the encoder exactly as REFERENCE; in
 *     the decoder the LayerNorm sums and softmax denominators as 64 strided
 *     lane partials + xor butterfly (canon_sum), exp still the C library's.
 * Everything else (dot products, PV accumulation, dequant, LN affine, embedding)
 * uses the reference's sequential op order in every mode.
 */
#ifndef MARIAN_ORACLE_H
#define MARIAN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_ORDER_CANONICAL = 0, ORACLE_ORDER_REFERENCE = 1, ORACLE_ORDER_FAST_DECODER = 2 };

/* Translate flags (same values as MARIAN_HIP_FLAG_*). */
enum {
  ORACLE_FLAG_IGNORE_EOS = 1u << 0,         /* token 0 does not finish a row */
  ORACLE_FLAG_NO_GENERATION_MASK = 1u << 1  /* score ids 1 and 7..38 too */
};

typedef struct {
  const int8_t* weight; /* [out, in], input-contiguous */
  const float* mult;    /* [out] per-output-channel multiplier (q = w*mult) */
  const float* bias;    /* [out] */
} oracle_linear;

typedef struct {
  oracle_linear qkv; /* [3d, d] rows: Q, K, V */
  oracle_linear out; /* [d, d] */
  const float* ln1_scale;
  const float* ln1_bias;
  oracle_linear ffn1; /* [F, d] */
  oracle_linear ffn2; /* [d, F] */
  const float* ln2_scale;
  const float* ln2_bias;
} oracle_encoder_layer;

typedef struct {
  oracle_linear self_qkv; /* [3d, d] */
  oracle_linear self_out; /* [d, d] */
  const float* ln1_scale;
  const float* ln1_bias;
  oracle_linear cross_q;   /* [d, d]  applied to the decoder state */
  oracle_linear cross_kv;  /* [2d, d] applied to the encoder output */
  oracle_linear cross_out; /* [d, d] */
  const float* ln2_scale;
  const float* ln2_bias;
  oracle_linear ffn1; /* [F, d] */
  oracle_linear ffn2; /* [d, F] */
  const float* ln3_scale;
  const float* ln3_bias;
} oracle_decoder_layer;

typedef struct {
  uint32_t vocab, dim, heads, ffn_dim, encoder_layers, decoder_layers;
  const int8_t* embedding;     /* [vocab, dim] tied source/target/output */
  const float* embedding_mult; /* [vocab] */
  const float* output_bias;    /* [vocab] */
  const oracle_encoder_layer* encoder;
  const oracle_decoder_layer* decoder;
} oracle_model;

/* The reference's own graph (q8_engine.rs:76-114): Transformer encoder, SSRU
 * decoder, one weight multiplier and one static activation multiplier per
 * dense layer, separate encoder/decoder embeddings (the decoder's is the tied
 * output projection).  Same field order as marian_hip_ssru_model. */
typedef struct {
  const int8_t* weight; /* [out, in] */
  float weight_mult;
  float act_mult;
  const float* bias; /* [out] or NULL */
} oracle_static_linear;

typedef struct {
  oracle_static_linear wq, wk, wv, wo;
  const float* attn_ln_scale;
  const float* attn_ln_bias;
  oracle_static_linear w1, w2;
  const float* ffn_ln_scale;
  const float* ffn_ln_bias;
} oracle_ssru_encoder_layer;

typedef struct {
  oracle_static_linear ssru_w, ssru_wf;
  const float* ssru_ln_scale;
  const float* ssru_ln_bias;
  oracle_static_linear wq, wk, wv, wo;
  const float* context_ln_scale;
  const float* context_ln_bias;
  oracle_static_linear w1, w2;
  const float* ffn_ln_scale;
  const float* ffn_ln_bias;
} oracle_ssru_decoder_layer;

typedef struct {
  uint32_t source_vocab, target_vocab, dim, heads, ffn_dim, encoder_layers, decoder_layers;
  const int8_t* encoder_embedding;
  float encoder_embedding_mult;
  const int8_t* decoder_embedding;
  float decoder_embedding_mult;
  float output_act_mult;
  const float* output_bias;
  const oracle_ssru_encoder_layer* encoder;
  const oracle_ssru_decoder_layer* decoder;
} oracle_ssru_model;

/* Work limits; 0 disables a cap (reference values in brackets). */
typedef struct {
  uint32_t max_length_factor;    /* [2] limit <= len * factor */
  uint32_t max_generation_steps; /* [256] */
  uint32_t max_position;         /* [4096] must be <= 4096 */
  uint32_t max_batch;            /* [256] */
  uint32_t max_source_tokens;    /* [256] */
  uint64_t max_padded_cells;     /* [65536] batch * Lmax^2 */
} oracle_limits;

/* Compiler and flags this library was built with (for the CPU-baseline record). */
const char* oracle_build_info(void);

/* ---- elementary ops ---------------------------------------------------- */
float oracle_expf(float x, int order);
float oracle_row_sum(const float* x, size_t n, int order);
/* sinusoidal table [count, dim] */
int oracle_positions(uint32_t dim, uint32_t count, float* out);

/* Per-row dynamic quantization: a[m] = 127/max|x[m,:]| (1 if the row is 0),
 * q = clamp(rne(x*a), -127, 127).  Returns 0, or -1 on a non-finite input. */
int oracle_quantize_rows(const float* x, size_t rows, size_t cols, int8_t* q, float* a);
/* Static multiplier, reference u8 encoding (q + 127). */
int oracle_quantize_static_u8(const float* x, size_t n, float mult, uint8_t* out);

/* Exact closed-form i32 GEMM: acc[m,n] = sum_k qa[m,k]*qw[n,k]. */
int oracle_gemm_i32(const int8_t* qa, size_t M, size_t K, const int8_t* qw, size_t N,
                    int32_t* acc, int threads);
/* The reference x86 kernel's arithmetic: u8 activations with a zero point,
 * widened i16 madd, i64 flush (q8_avx2.rs:125-358). threads<=1 is serial. */
int oracle_gemm_u8_i8_avx2(const uint8_t* a, size_t M, size_t K, const int8_t* w, size_t N,
                           uint8_t zero_point, int32_t* acc, int threads);
/* Scalar u8.i8 dot (q8_arm.rs:50-55). */
int32_t oracle_dot_u8_i8(const uint8_t* a, const int8_t* w, size_t n);

/* Full Q8 linear: quantize rows, exact GEMM, dequant + bias (+ReLU).
 * Any of acc/qa/a may be NULL. */
int oracle_linear_forward(const float* x, size_t M, size_t K, const oracle_linear* lin,
                          size_t N, int relu, float* y, int32_t* acc, int8_t* qa, float* a,
                          int threads);

/* Q8 linear with a static activation multiplier for every row (the
 * reference's own mode): q = clamp(rne(x*act_mult), -127, 127).  -1 on a
 * non-finite input or multiplier.  acc/qa may be NULL. */
int oracle_linear_forward_static(const float* x, size_t M, size_t K, const oracle_linear* lin,
                                 size_t N, float act_mult, int relu, float* y, int32_t* acc,
                                 int8_t* qa, int threads);

/* SSRU update + LayerNorm (tensor.rs:184-218): state updated in place,
 * out = LN(relu(state) + residual). */
int oracle_ssru_layer_norm(const float* cand, const float* forget, float* state,
                           const float* residual, const float* scale, const float* bias,
                           size_t rows, size_t d, int order, float* out);

/* select_token over candidate lists: row m scores cand[offs[m] .. offs[m+1])
 * (logits per list position, optional); -1 on an empty list or an id >= V. */
int oracle_candidate_argmax(const int8_t* xq, const float* xa, size_t M, size_t K,
                            const int8_t* emb, const float* mult, const float* bias, size_t V,
                            const uint32_t* cand, const uint32_t* offs, int32_t* token,
                            float* logits);

/* out = LN(x + r) per row of length d (eps 1e-6). */
int oracle_residual_layer_norm(const float* x, const float* r, const float* scale,
                               const float* bias, size_t rows, size_t d, int order,
                               float* out);

/* Variable-length multi-head attention.  Sequence b owns query rows
 * [cu_q[b], cu_q[b+1]) and key/value rows [cu_k[b], cu_k[b+1]); row strides
 * are in floats; head h uses columns [h*dh, (h+1)*dh) of each operand. */
int oracle_attention(const float* q, size_t ldq, const float* k, size_t ldk, const float* v,
                     size_t ldv, const uint32_t* cu_q, const uint32_t* cu_k, size_t batch,
                     size_t heads, size_t head_dim, int order, float* out, size_t ldo);

/* Greedy translation of a packed batch (q8_engine.rs:353-466).
 * out_tokens receives the concatenated outputs (capacity out_cap), out_offsets
 * batch+1 entries.  Returns 0, -1 invalid input, -2 model/arithmetic error,
 * -3 output buffer too small.  A message is written to err (if non-NULL). */
int oracle_translate(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                     const uint32_t* offsets, size_t n_offsets,
                     const uint32_t* max_output_tokens, const oracle_limits* limits,
                     uint32_t flags, int order, int threads, int32_t* out_tokens,
                     size_t out_cap, uint32_t* out_offsets, size_t* out_len, char* err,
                     size_t err_cap);

/* oracle_translate that also returns intermediate values (each may be NULL):
 * enc_out[n_tokens, dim] the final encoder state of every packed row;
 * logits_out[B, vocab] the logits of decode step probe_step (0-based) of every
 * row that reaches it (masked ids -inf), active_out[B] = 1 for those rows. */
int oracle_translate_probe(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                           const uint32_t* offsets, size_t n_offsets,
                           const uint32_t* max_output_tokens, const oracle_limits* limits,
                           uint32_t flags, int order, int threads, int32_t* out_tokens,
                           size_t out_cap, uint32_t* out_offsets, size_t* out_len, char* err,
                           size_t err_cap, uint32_t probe_step, float* enc_out,
                           float* logits_out, uint8_t* active_out);

/* oracle_translate with per-sentence output candidates (select_token over
 * LexicalShortlist::candidates, q8_engine.rs:576-584, 749-790): sentence b
 * scores candidates[cand_offsets[b] .. cand_offsets[b+1]) in list order, the
 * first maximum winning, without the generation mask.  -1 for an empty list
 * or an id out of the vocabulary. */
int oracle_translate_shortlisted(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                                 const uint32_t* offsets, size_t n_offsets,
                                 const uint32_t* max_output_tokens, const oracle_limits* limits,
                                 uint32_t flags, int order, int threads, const uint32_t* candidates,
                                 const uint32_t* cand_offsets, int32_t* out_tokens, size_t out_cap,
                                 uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap);

/* Same contract, executed the way the reference x86 engine schedules the work
 * (padded encoder batch, all rows every decode step, AVX2 madd GEMM row-split
 * over `threads` when rows>1 && rows*N >= 8192, scalar output scoring).  Its
 * results equal oracle_translate's; it exists to be timed. */
int oracle_translate_reference_schedule(
    const oracle_model* model, const int32_t* tokens, size_t n_tokens, const uint32_t* offsets,
    size_t n_offsets, const uint32_t* max_output_tokens, const oracle_limits* limits,
    uint32_t flags, int order, int threads, int32_t* out_tokens, size_t out_cap,
    uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap);

/* Encoder only (packed rows): writes the final encoder states [T, d]. */
int oracle_encode(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                  const uint32_t* offsets, size_t n_offsets, int order, int threads,
                  float* out);

/* One decoder step for a single sequence given explicit state, used by tests
 * to compare logits: runs `steps` greedy steps for sequence 0 of the packed
 * batch and writes the logits of the last step [vocab] (mask applied as -inf
 * unless NO_GENERATION_MASK). */
int oracle_last_step_logits(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                            uint32_t steps, uint32_t flags, int order, float* logits);

/* Q8CpuEngine::translate_token_ids over the Transformer-SSRU graph
 * (q8_engine.rs:353-466 with encode :511-574, the SSRU decoder layer
 * :394-432, select_token :749-790).  candidates/cand_offsets[B+1] give each
 * sentence's output candidates in scan order; NULL scores the whole target
 * vocabulary in ascending order with the generation mask (what
 * LexicalShortlist::from_bytes(None) yields).  enc_out, logits_out[B,
 * target_vocab] (probe_step; ids not scored are -inf) and active_out as in
 * oracle_translate_probe; each may be NULL.  Same return codes as
 * oracle_translate, plus -1 for an empty candidate list or an id out of the
 * target vocabulary. */
int oracle_translate_ssru(const oracle_ssru_model* model, const int32_t* tokens, size_t n_tokens,
                          const uint32_t* offsets, size_t n_offsets,
                          const uint32_t* max_output_tokens, const oracle_limits* limits,
                          uint32_t flags, int order, int threads, const uint32_t* candidates,
                          const uint32_t* cand_offsets, int32_t* out_tokens, size_t out_cap,
                          uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap,
                          uint32_t probe_step, float* enc_out, float* logits_out,
                          uint8_t* active_out);

/* oracle_translate_ssru executed the way the reference x86 engine schedules
 * the work (padded batch, every row decoded every step, u8 AVX2 GEMMs, scalar
 * scoring); the same tokens.  Timed CPU baseline. */
int oracle_translate_ssru_reference_schedule(
    const oracle_ssru_model* model, const int32_t* tokens, size_t n_tokens, const uint32_t* offsets,
    size_t n_offsets, const uint32_t* max_output_tokens, const oracle_limits* limits, uint32_t flags,
    int order, int threads, const uint32_t* candidates, const uint32_t* cand_offsets,
    int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets, size_t* out_len, char* err,
    size_t err_cap);

#ifdef __cplusplus
}
#endif
#endif
