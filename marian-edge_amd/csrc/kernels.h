// kernels.h — host-side launch interface of the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mh {

// Input-row prologue of the decode attention block: the workgroup builds its
// row itself instead of reading a quantized row, so the producer of that row
// needs no kernel of its own.
//   PRO_LN:  row = LayerNorm(y + r) with gamma/beta (the post-norm residual
//            LayerNorm of a sublayer's output),
//   PRO_EMB: row = emb[prev]/mult * scale + pos[step] (the decoder input; a
//            negative prev gives pos[step] alone).
// The head-0 workgroup of each row also stores the fp32 row to `out` (the
// next residual).
enum ProKind { PRO_NONE = 0, PRO_LN = 1, PRO_EMB = 2 };
struct RowPrologue {
  int kind = PRO_NONE;
  const float* y = nullptr;
  const float* r = nullptr;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  const int8_t* emb = nullptr;
  const float* emb_mult = nullptr;
  const float* pos = nullptr;  // [kMaxPosition, K]
  float scale = 1.0f;
  const int32_t* row_prev = nullptr;  // position row: the consumer's step
  float* out = nullptr;  // fp32 [M, K], or nullptr when nothing reads the rows again
  int* err = nullptr;    // set to 1 on a non-finite row value
  int fast = 0;          // PRO_LN: the LayerNorm sums in the fast-reduction tree order
};

// Quantized activations times an int8 weight matrix [N, K] (K-contiguous).
struct GemmArgs {
  const int8_t* A = nullptr;  // [M, lda] int8 activations
  const float* a = nullptr;   // [M] per-row activation multipliers
  int64_t lda = 0;
  int M = 0;                  // row count (host) ...
  const int* M_dev = nullptr; // ... or read on the device (decode active rows)
  int K = 0;                  // multiple of 64
  const int8_t* W = nullptr;  // [N, K], K-contiguous
  const int8_t* Wf = nullptr; // optional, skinny and vocabulary kernels: W in fragment order
  const float* wmult = nullptr;
  const float* bias = nullptr;
  int N = 0;
  // Alternative A source (skinny kernel only): fp32 rows Af[M, ldaf] that are
  // quantized while loading, with row multiplier 127 / max_p Aamax[m*parts+p]
  // (the per-part |max| written by the producer: one per attention head;
  // 1 to 16 parts, K <= 512).  Store epilogue only; each workgroup takes 16
  // rows.  Without Aamax the kernel finds each row's |max| over all of K itself
  // (K <= 2048: the FFN down-projection), as the row quantization would, and sets
  // *err to 1 on a non-finite value.
  const float* Af = nullptr;
  int64_t ldaf = 0;
  const float* Aamax = nullptr;
  int amax_parts = 0;
  int* err = nullptr;
  // Vocabulary kernel only: with pro.kind == PRO_LN the rows (at most
  // kVocabLnMaxRows, K = 512) are LayerNorm(pro.y + pro.r), built in the
  // kernel instead of read from A (pro.out is not written).
  RowPrologue pro;
};
constexpr int kVocabLnMaxRows = 4;
// Whether the vocabulary kernel can build LayerNorm rows of width K itself.
bool vocab_ln_supported(int K);

enum EpiMode { EPI_STORE = 0, EPI_QKV_CACHE = 1, EPI_ARGMAX = 2 };

struct Epilogue {
  // EPI_STORE (and the Q columns of EPI_QKV_CACHE)
  float* out = nullptr;
  int64_t ldo = 0;
  int32_t* out_i32 = nullptr;
  int64_t ldi = 0;
  int relu = 0;
  // EPI_QKV_CACHE: columns [d, 2d) -> kcache, [2d, 3d) -> vcache, at cache row
  // row_kv0[m] + step (the row's sequence's first cache row).
  float* kcache = nullptr;
  float* vcache = nullptr;
  const int64_t* row_kv0 = nullptr;
  int step = 0;
  int d = 0;
  // EPI_ARGMAX: per-row best key of each 64-column group -> partials[m*ld + g]
  uint64_t* partials = nullptr;
  int partial_ld = 0;
  float* logits = nullptr;  // optional [M, N]
  int64_t ldl = 0;
  uint32_t flags = 0;  // bit 1: no generation mask
  // EPI_STORE, int8 A (skinny) or tile GEMM: the output also quantized with a
  // static multiplier for the next layer, q = clamp(rne(y * qmult), -127, 127)
  // into out_q [M, ldq], and out_qa[m] = qmult.
  int8_t* out_q = nullptr;
  int64_t ldq = 0;
  float qmult = 0.0f;
  float* out_qa = nullptr;
};

// Column groups of the skinny kernel, and the argmax partial count per row.
int skinny_groups(int N);
int argmax_groups(int N, int K);
// Skinny (M up to a few hundred, weights streamed once per 64 rows) MFMA GEMM.
hipError_t launch_gemm_skinny(const GemmArgs& g, int mode, const Epilogue& e, hipStream_t s);
// The vocabulary kernel (EPI_ARGMAX); when ev_start/ev_stop are given they are
// recorded by the kernel's own dispatch (start and end of the kernel).
hipError_t launch_vocab_argmax(const GemmArgs& g, const Epilogue& e, hipStream_t s,
                               hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);
// LDS-tiled 64x64 MFMA GEMM for large M (EPI_STORE only); lda a multiple of 16.
hipError_t launch_gemm_tile(const GemmArgs& g, const Epilogue& e, hipStream_t s);
// Picks the kernel by M (host-known M only).
hipError_t launch_gemm_store(const GemmArgs& g, const Epilogue& e, hipStream_t s);

hipError_t launch_quantize_rows(const float* x, int64_t ldx, int rows, const int* rows_dev,
                                int cols, int8_t* q, int64_t ldq, float* a, int* err,
                                hipStream_t s);

// qmult > 0: q is quantized with that static multiplier (the next layer's)
// instead of each row's own.
// fast: the LayerNorm sums in the fast-reduction tree order (decoder only).
hipError_t launch_residual_ln(const float* y, const float* r, const float* g, const float* b,
                              int rows, const int* rows_dev, int d, float* out, int8_t* q,
                              float* a, int* err, hipStream_t s, float qmult = 0.0f,
                              bool fast = false);

// Quantization with one static activation multiplier for every row (a[row] =
// mult); rejects a multiplier that is not finite and positive.
hipError_t launch_quantize_rows_static(const float* x, int64_t ldx, int rows, int cols, float mult,
                                       int8_t* q, int64_t ldq, float* a, int* err, hipStream_t s,
                                       const int* rows_dev = nullptr);

// SSRU update + LayerNorm: state <- gate * state + (1 - gate) * cand with
// gate = sigmoid(forget); out = LN(relu(state) + resid) (+ quantization, with
// qmult when > 0).  cand/forget rows are ldc floats apart (0: d); row r's
// state is state row state_row[r] when state_row is set; rows at or past
// *rows_dev are skipped.  The new state goes to state_out when set (another
// buffer than state), else over the old one.
hipError_t launch_ssru_ln(const float* cand, const float* forget, float* state, const float* resid,
                          const float* g, const float* b, int rows, int d, float* out, int8_t* q,
                          float* a, int* err, hipStream_t s, int64_t ldc = 0,
                          const int* rows_dev = nullptr, const int* state_row = nullptr,
                          float qmult = 0.0f, float* state_out = nullptr);

// SSRU input (Transformer-SSRU decoder, static multipliers): the layer input
// x of each row (pro: PRO_LN, LayerNorm(y + r), the previous layer's last
// sublayer; PRO_EMB, the decoder input embedding at position `step`), its
// candidate and forget-gate projections (W [2d, d] in fragment order: rows
// [0, d) the candidate, [d, 2d) the forget gate, each input quantized with its
// own static multiplier act_c / act_f), and the SSRU update of each state
// column: state_out[seq] = gate * state_in[seq] + (1 - gate) * c with gate =
// 1 / (1 + exp(-f)), z = relu(state') + x.  d = 256, 384 or 512; state_out
// must not alias state_in.
struct SsruInputArgs {
  RowPrologue pro;
  int step = 0;  // PRO_EMB: the position row
  int rows = 0;
  const int* rows_dev = nullptr;
  int d = 0;
  float act_c = 0.0f, act_f = 0.0f;
  const int8_t* W = nullptr;
  const float* wmult = nullptr;  // [2d]
  const float* bias = nullptr;   // [2d]
  const float* state_in = nullptr;  // [sequences, d]
  float* state_out = nullptr;
  const int* state_row = nullptr;   // sequence of each row
  int64_t state_rows = 0;           // sequences held by the state buffers
  float* z = nullptr;               // [rows, d]
  int* err = nullptr;
};
hipError_t launch_ssru_input(const SsruInputArgs& a, hipStream_t s);

// SSRU decode block: per (row, head) one workgroup takes z (from
// launch_ssru_input), applies the SSRU LayerNorm (the head-0 workgroup stores
// the LayerNorm row to x_out), quantizes the row with the query projection's
// static multiplier xq_mult, projects it onto the head's query with int8 MFMA
// (static dequantization), attends over the row's encoder keys
// row_key0[r] + [0, row_nk[r]) (at most kSsruBlockMaxKeys), and stores the
// head's output quantized with the output projection's static multiplier
// (qout [rows, ldqout], qa[r] = qmult).  One launch replaces the LayerNorm,
// query projection and cross-attention kernels.
struct SsruBlockArgs {
  const float* z = nullptr;  // [rows, d]
  const float* gamma = nullptr;
  const float* beta = nullptr;
  float* x_out = nullptr;  // [rows, d] the LayerNorm rows
  float xq_mult = 0.0f;    // the query projection's activation multiplier
  const int8_t* Wq = nullptr;  // [d, d] in fragment order (frag_load)
  const float* wq_mult = nullptr;
  const float* wq_bias = nullptr;
  const float* k = nullptr;  // encoder key / value rows, stride ldkv
  const float* v = nullptr;
  int64_t ldkv = 0;
  const int64_t* row_key0 = nullptr;
  const int32_t* row_nk = nullptr;
  int64_t max_row = 0;  // key rows of k / v are < max_row
  int max_keys = 0;     // upper bound on keys per row
  int d = 0, heads = 0, rows = 0;
  const int* rows_dev = nullptr;
  int8_t* qout = nullptr;
  int64_t ldqout = 0;
  float qmult = 0.0f;
  float* qa = nullptr;
  int* err = nullptr;
};
constexpr int kSsruBlockMaxKeys = 128;

// Residual LayerNorm + Q8 linear for groups of eight rows: out[m] = (relu of)
// Q8Linear(LN(y[m] + r[m])) with the row quantized by xq_mult[0] for output
// columns below part_n and xq_mult[1] from it (a row group of two layers with
// their own static multipliers; part_n = N: one), or with each row's own
// multiplier when dyn is set (xq_mult unused).
// Optional outputs: fp32 `out`, and/or `out_q` quantized with qmult (the next
// layer's static multiplier, out_qa[m] = qmult); x_out receives the
// LayerNorm rows.  Eight rows and 128 output columns per workgroup;
// K = 256, 384 or 512, N a multiple of 128.
struct LnGemmRowsArgs {
  const float* y = nullptr;  // [rows, K], or computed from ya:
  // y = the static Q8 linear of the int8 rows ya [rows, K] with multiplier
  // ya_mult and Wy [K, K] in fragment order (ymult, ybias): the attention
  // output projection, computed by every workgroup for its rows.
  const int8_t* ya = nullptr;
  float ya_mult = 0.0f;
  const int8_t* Wy = nullptr;
  const float* ymult = nullptr;
  const float* ybias = nullptr;
  const float* r = nullptr;  // [rows, K]
  const float* gamma = nullptr;
  const float* beta = nullptr;
  int rows = 0;
  const int* rows_dev = nullptr;
  float* x_out = nullptr;  // optional [rows, K]
  float xq_mult[2] = {0.0f, 0.0f};
  int part_n = 0;
  int dyn = 0;
  const int8_t* W = nullptr;  // [N, K] in fragment order (frag_load)
  const float* wmult = nullptr;
  const float* bias = nullptr;
  int K = 0, N = 0;
  int relu = 0;
  float* out = nullptr;
  int64_t ldo = 0;
  int8_t* out_q = nullptr;
  int64_t ldq = 0;
  float qmult = 0.0f;
  float* out_qa = nullptr;
  int* err = nullptr;
  int fast = 0;  // dyn only: the LayerNorm sums in the fast-reduction tree order
};
bool ln_gemm_rows_supported(int K, int N);
hipError_t launch_ln_gemm_rows(const LnGemmRowsArgs& a, hipStream_t s);
bool ssru_block_supported(int d, int heads, int max_keys);
hipError_t launch_ssru_block(const SsruBlockArgs& a, hipStream_t s);

struct EmbedArgs {
  const int8_t* emb = nullptr;
  const float* emb_mult = nullptr;
  const float* pos = nullptr;  // [kMaxPosition, d]
  float scale = 1.0f;
  int d = 0;
  // encoder rows: token and position per row
  const int32_t* tokens = nullptr;
  const int32_t* positions = nullptr;
  // decoder rows: token = row_prev[r] (negative: position only), position = step
  const int32_t* row_prev = nullptr;
  int step = 0;
  int rows = 0;
  const int* rows_dev = nullptr;
  float* x = nullptr;
  int8_t* xq = nullptr;  // null: no quantized copy
  float* xa = nullptr;
  float qmult = 0.0f;    // > 0: quantize with this static multiplier
  int* err = nullptr;
};
hipError_t launch_embed(const EmbedArgs& a, hipStream_t s);

enum AttnMode { ATT_SEQ = 0, ATT_CROSS = 1, ATT_SELF = 2 };
struct AttnArgs {
  int mode = ATT_SEQ;
  const void* q = nullptr;
  int64_t ldq = 0;
  const void* k = nullptr;
  const void* v = nullptr;
  int64_t ldkv = 0;
  int bf16 = 0;
  int heads = 0;
  int head_dim = 64;  // 64 or 48; head h is columns [h * head_dim, (h + 1) * head_dim)
  int rows = 0;
  const int* rows_dev = nullptr;
  // ATT_SEQ: keys of row r are [cu[seq_of_row[r]], cu[seq_of_row[r]+1])
  const int* seq_of_row = nullptr;
  const uint32_t* cu = nullptr;
  // ATT_CROSS: keys of row r are row_key0[r] + [0, row_nk[r]);
  // ATT_SELF: keys are row_key0[r] + [0, step]
  const int64_t* row_key0 = nullptr;
  const int32_t* row_nk = nullptr;
  int step = 0;
  // ATT_CROSS / ATT_SELF: key rows of the K/V buffers are < max_row.  Rows at
  // or past the device row count read their (stale) ranges clamped to this
  // bound before the count is known, and are then discarded.
  int64_t max_row = 0;
  int max_keys = 0;  // upper bound on keys per row (selects the kernel variant)
  float* out = nullptr;   // fp32 [rows, ldo], head h at columns [64h, 64h+64)
  int64_t ldo = 0;
  float* amax = nullptr;  // optional [rows, heads]: max |out| of each head's slice
  int* err = nullptr;
  // Optional: the output also quantized with a static multiplier into qout
  // [rows, ldqout] (head h at its columns), and qa[row] = qmult.
  int8_t* qout = nullptr;
  int64_t ldqout = 0;
  float qmult = 0.0f;
  float* qa = nullptr;
  // ATT_SEQ with max_keys <= 256: the query-tile list written by
  // launch_seq_tiles (tiles_cap = its bound) selects the tiled kernel (no amax).
  const uint32_t* tiles = nullptr;
  int tiles_cap = 0;
  int fast = 0;  // ATT_CROSS / ATT_SELF: the softmax denominator in the fast-reduction tree order
};
// ev_start / ev_stop as in launch_vocab_argmax (single-wave kernel only).
hipError_t launch_attention(const AttnArgs& a, hipStream_t s, hipEvent_t ev_start = nullptr,
                            hipEvent_t ev_stop = nullptr);
// Query tiles of packed sequences cu[0..nseq] for the tiled ATT_SEQ kernel:
// at most seq_tiles_bound(rows, nseq) entries; tiles needs 1 + 2 * cap words.
int seq_tiles_bound(int rows, int nseq);
hipError_t launch_seq_tiles(const uint32_t* cu, int nseq, uint32_t* tiles, int cap, hipStream_t s);

// Decode attention block (one launch per attention sublayer on steps with few
// rows): per (row, head) it builds the row's input with `pro` (PRO_LN, or
// PRO_EMB for the first self-attention), projects it onto the head's query
// (ATT_SELF: query, key and value rows h*64.., d + h*64.., 2d + h*64.. of W),
// and attends.  ATT_SELF attends over cache rows row_key0[r] + [0, step) plus
// this step's key and value, which it also writes to kc_out / vc_out at row
// row_key0[r] + step; ATT_CROSS attends over row_key0[r] + [0, row_nk[r]).
// d = 512, head_dim 64, at most 128 keys per row (max_keys).
struct BlockArgs {
  int mode = ATT_SELF;
  RowPrologue pro;
  int rows = 0;
  const int* rows_dev = nullptr;
  int heads = 0;
  const int8_t* W = nullptr;  // [3d or d, d] in fragment order (frag_load)
  const float* wmult = nullptr;
  const float* bias = nullptr;
  const float* k = nullptr;  // key rows (ATT_SELF: the cache), stride ldkv
  const float* v = nullptr;
  float* kc_out = nullptr;  // ATT_SELF: this step's key / value rows
  float* vc_out = nullptr;
  int64_t ldkv = 0;
  const int64_t* row_key0 = nullptr;
  const int32_t* row_nk = nullptr;
  int step = 0;
  int64_t max_row = 0;  // key rows of k / v are < max_row
  int max_keys = 0;     // upper bound on keys attended per row
  float* out = nullptr;  // [rows, ldo], head h at columns [64h, 64h+64)
  int64_t ldo = 0;
  float* amax = nullptr;  // [rows, heads]
  int* err = nullptr;
  int fast = 0;  // the softmax denominator (and, with pro.fast, the LayerNorm) in the tree order
};
bool attn_block_supported(int d, int heads, int max_keys);

// LayerNorm + up-projection block: out[r, :] = (relu of) the Q8 linear of the
// row `pro` builds (PRO_LN), one workgroup per (row, 128 output columns); the
// column-slice-0 workgroup also stores the LayerNorm row to pro.out.
// K = 512, N a multiple of 128.
struct LnGemmArgs {
  RowPrologue pro;
  int rows = 0;
  const int* rows_dev = nullptr;
  const int8_t* W = nullptr;  // [N, K] in fragment order (frag_load)
  const float* wmult = nullptr;
  const float* bias = nullptr;
  int K = 0, N = 0;
  int relu = 0;
  float* out = nullptr;  // [rows, ldo]
  int64_t ldo = 0;
  int* err = nullptr;
};
bool ln_gemm_block_supported(int K, int N);
hipError_t launch_ln_gemm_block(const LnGemmArgs& a, hipStream_t s);
// ev_start / ev_stop as in launch_vocab_argmax.
hipError_t launch_attn_block(const BlockArgs& b, hipStream_t s, hipEvent_t ev_start = nullptr,
                             hipEvent_t ev_stop = nullptr);

// Per-row decode metadata, rebuilt in active-row order by the finalizer.
struct RowMeta {
  int* slot = nullptr;        // sequence of each active row
  int64_t* kv0 = nullptr;     // first KV-cache (and output) row of that sequence
  int64_t* src0 = nullptr;    // first encoder row of that sequence
  int32_t* srcn = nullptr;    // its source length
  int32_t* prev = nullptr;    // its last emitted token (-1 before the first step)
  uint32_t* limit = nullptr;  // its generation limit
};

struct FinalizeArgs {
  const uint64_t* partials = nullptr;
  int nparts = 0;
  RowMeta rows;
  int* n_active = nullptr;
  int rows_ub = 0;                   // host bound on *n_active; rows below it are allocated
  int* err = nullptr;                // set to 3 if *n_active exceeds rows_ub
  int32_t* out_tok = nullptr;        // row kv0 + step
  uint32_t* count = nullptr;
  int step = 0;
  uint32_t flags = 0;
  uint32_t* active_hist = nullptr;  // optional: active_hist[step] = rows this step ran on
  int* host_active = nullptr;       // optional, pinned host memory: the new active count
};
hipError_t launch_finalize(const FinalizeArgs& f, hipStream_t s);

// Output scoring over per-row candidate lists (a lexical shortlist): row m
// scores the ids cand[off[m] .. off[m+1]) (ascending) against its quantized
// state xq / xa; one argmax key per (row, 128 candidates) goes to
// partials[m * nparts + chunk] (nparts >= cand_groups(max_cands)).  logits
// (optional) receives each candidate's logit at its position in cand.  An id
// outside the vocabulary sets *err to 1 and is not scored.
struct CandArgs {
  const int8_t* xq = nullptr;  // [M, K]
  const float* xa = nullptr;   // [M]
  int M = 0, K = 0, V = 0;
  const int8_t* emb = nullptr;  // [V, K] row-major
  const float* mult = nullptr;
  const float* bias = nullptr;
  const uint32_t* cand = nullptr;
  const uint32_t* off = nullptr;  // [M + 1], or [sequences + 1] with row_slot
  const int* row_slot = nullptr;  // decode loop: row m scores sequence row_slot[m]'s list
  const int* rows_dev = nullptr;  // decode loop: rows at or past *rows_dev are skipped
  int max_cands = 0;              // host bound on the lists' lengths
  uint64_t* partials = nullptr;
  int nparts = 0;
  float* logits = nullptr;
  int* err = nullptr;
  // pro.kind == PRO_LN (K = 256, 384 or 512): the rows are LayerNorm(pro.y +
  // pro.r), built in the kernel and quantized with qmult (> 0, static) or each
  // row's own multiplier (0); xq / xa are not read.
  RowPrologue pro;
  float qmult = 0.0f;
};
int cand_groups(int max_cands);
bool cand_ln_supported(int K);
hipError_t launch_cand_argmax(const CandArgs& c, hipStream_t s);

// Reduces argmax partials to token ids (op-level argmax).
// Records the message marian_hip_last_op_error returns on this thread.
void note_op_error(const char* msg);

hipError_t launch_argmax_reduce(const uint64_t* partials, int nparts, int rows, int32_t* token,
                                hipStream_t s);

}  // namespace mh
