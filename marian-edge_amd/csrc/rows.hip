// rows.hip — one-wavefront-per-row kernels: activation quantization, residual
// LayerNorm (+ quantization for the next GEMM), embedding gather, and the
// per-step token selection / active-set compaction of the decode loop.
#include "device_common.h"
#include "kernels.h"

namespace mh {
namespace {


// Row quantization for the next GEMM: absmax -> multiplier -> int8
// (q8_gemm.rs:569-590 with a per-row multiplier).  Non-finite input sets *err.
__global__ __launch_bounds__(256) void k_quantize_rows(const float* x, int64_t ldx, int rows,
                                                       const int* rows_dev, int cols, int8_t* q,
                                                       int64_t ldq, float* a, int* err) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = rows_dev ? *rows_dev : rows;
  if (row >= n) return;
  const float* xr = x + (int64_t)row * ldx;
  float m = 0.0f;
  bool bad = false;
  for (int i = lane; i < cols; i += 64) {
    const float v = xr[i];
    bad |= !isfinite(v);
    m = fmaxf(m, fabsf(v));
  }
  m = wave_max(m);
  const float sc = row_multiplier(m);
  int8_t* qr = q + (int64_t)row * ldq;
  for (int i = lane; i < cols; i += 64) qr[i] = (int8_t)quantize_one(xr[i], sc);
  if (lane == 0) a[row] = sc;
  if (__any(bad) && lane == 0 && err) *err = 1;
}

// Quantization with a static per-tensor activation multiplier (the reference's
// own mode, quantize_symmetric_u8_into q8_gemm.rs:569-590 with the model's
// QuantMultA, legacy_q8.rs:544-552): q = clamp(rne(x * mult), -127, 127), and
// a[row] = mult so the GEMM epilogue dequantizes with 1 / (mult * w).
__global__ __launch_bounds__(256) void k_quantize_rows_static(const float* x, int64_t ldx, int rows,
                                                              const int* rows_dev, int cols,
                                                              float mult, int8_t* q, int64_t ldq,
                                                              float* a, int* err) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= (rows_dev ? min(*rows_dev, rows) : rows)) return;
  const float* xr = x + (int64_t)row * ldx;
  int8_t* qr = q + (int64_t)row * ldq;
  bool bad = false;
  for (int i = lane; i < cols; i += 64) {
    const float v = xr[i];
    bad |= !isfinite(v);
    qr[i] = (int8_t)quantize_one(v, mult);
  }
  if (lane == 0) a[row] = mult;
  if (__any(bad) && lane == 0 && err) *err = 1;
}

// Same, for rows of V4*256 values held in registers: one 16-byte load and one
// 4-byte store per lane per 256 columns.
template <int V4>
__global__ __launch_bounds__(256) void k_quantize_rows_v4(const float* x, int64_t ldx, int rows,
                                                          const int* rows_dev, int8_t* q,
                                                          int64_t ldq, float* a, int* err) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;  // host bound: rows below it are allocated
  const float4* xr = (const float4*)(x + (int64_t)row * ldx);
  float4 v[V4];
#pragma unroll
  for (int j = 0; j < V4; ++j) v[j] = xr[lane + 64 * j];
  const int n = rows_dev ? *rows_dev : rows;
  if (row >= n) return;
  float m = 0.0f;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    bad |= !isfinite(v[j].x) || !isfinite(v[j].y) || !isfinite(v[j].z) || !isfinite(v[j].w);
    m = fmaxf(fmaxf(m, fmaxf(fabsf(v[j].x), fabsf(v[j].y))), fmaxf(fabsf(v[j].z), fabsf(v[j].w)));
  }
  m = wave_max(m);
  const float sc = row_multiplier(m);
  uint32_t* qr = (uint32_t*)(q + (int64_t)row * ldq);
#pragma unroll
  for (int j = 0; j < V4; ++j) {
    const uint32_t b0 = (uint32_t)(quantize_one(v[j].x, sc) & 0xFF);
    const uint32_t b1 = (uint32_t)(quantize_one(v[j].y, sc) & 0xFF);
    const uint32_t b2 = (uint32_t)(quantize_one(v[j].z, sc) & 0xFF);
    const uint32_t b3 = (uint32_t)(quantize_one(v[j].w, sc) & 0xFF);
    qr[lane + 64 * j] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
  }
  if (lane == 0) a[row] = sc;
  if (__any(bad) && lane == 0 && err) *err = 1;
}

// LayerNorm of one row z (lane holds z[lane + 64 j]) by one wave, stored to
// out (and quantized into q / a when q is set, with the row's own multiplier
// or, when qmult > 0, the next layer's static one): normalize_row
// (tensor.rs:372-385) sums the row strictly left to right: the wave parks z in
// LDS (zr, kLnRow<PER> floats) and folds it with fold_row_wave (speculative
// 128-element chunks for even PER, with the sequential fold's exact result);
// the centred squares are formed lane-parallel and folded the same way.
// FAST: both sums in the fast-reduction tree order instead (tree_sum_wave).
template <int PER, bool FAST = false>
__device__ __forceinline__ void ln_row_wave(const float (&z)[PER], float* zr, const float (&gv)[PER],
                                            const float (&bv)[PER], int row, int lane, float* out,
                                            int8_t* q, float* a, int* err, float qmult) {
  constexpr int D = PER * 64;
  const float mean = (FAST ? tree_sum_wave<PER>(z) : fold_row_wave<PER>(z, zr, lane)) / (float)D;
  float t[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float c = z[j] - mean;
    t[j] = c * c;
  }
  const float var = (FAST ? tree_sum_wave<PER>(t) : fold_row_wave<PER>(t, zr, lane)) / (float)D;
  const float inv = 1.0f / sqrtf(var + kLayerNormEpsilon);
  float o[PER];
  float m = 0.0f;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    o[j] = ((z[j] - mean) * inv) * gv[j] + bv[j];
    bad |= !isfinite(o[j]);
    m = fmaxf(m, fabsf(o[j]));
    out[(int64_t)row * D + i] = o[j];
  }
  if (q) {
    m = wave_max(m);
    const float sc = qmult > 0.0f ? qmult : row_multiplier(m);
#pragma unroll
    for (int j = 0; j < PER; ++j) q[(int64_t)row * D + lane + 64 * j] = (int8_t)quantize_one(o[j], sc);
    if (lane == 0) a[row] = sc;
  }
  if (__any(bad) && lane == 0 && err) *err = 1;
}

// out = LN(y + r), optionally quantized for the next GEMM.  One wave per row.
template <int PER, bool FAST = false>
__global__ __launch_bounds__(256) void k_residual_ln(const float* y, const float* r,
                                                     const float* gamma, const float* beta,
                                                     int rows, const int* rows_dev, float* out,
                                                     int8_t* q, float* a, int* err, float qmult) {
  constexpr int D = PER * 64;
  __shared__ __attribute__((aligned(16))) float sZ[4][kLnRow<PER>];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave;
  if (row >= rows) return;  // uniform per wave; the waves share no barrier
  // Rows below the host bound are always backed by memory, so every load is
  // issued before the device row count arrives.
  const float* yr = y + (int64_t)row * D;
  const float* rr = r + (int64_t)row * D;
  float yv[PER], rv[PER], gv[PER], bv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    yv[j] = yr[lane + 64 * j];
    rv[j] = rr[lane + 64 * j];
    gv[j] = gamma[lane + 64 * j];
    bv[j] = beta[lane + 64 * j];
  }
  const int n = rows_dev ? *rows_dev : rows;
  if (row >= n) return;
  float z[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) z[j] = yv[j] + rv[j];
  ln_row_wave<PER, FAST>(z, sZ[wave], gv, bv, row, lane, out, q, a, err, qmult);
}

// SSRU state update + LayerNorm (ssru_update_layer_norm_into, tensor.rs:184-218,
// the reference's SSRU decoder, q8_engine.rs:394-408).  Per element: gate =
// 1 / (1 + exp(-f)) with the C library's expf, s' = gate * s + (1 - gate) * c
// (each product, the difference and the sum rounded on their own), s' is
// stored to state_out (the state itself, or the other buffer of a pair); then
// out = LN(relu(s') + residual) (relu_residual
// :718-724, relu as max(x, 0) with NaN and -0.0 giving +0.0) with the
// sequential folds of normalize_row.  One wave per row.  In the decode loop
// the state of active row r is state row state_row[r] (its sequence), and
// rows at or past *rows_dev are skipped.
__constant__ uint64_t kRowsExp2Tab[32] = {MH_EXP2_TABLE_32};
template <int PER>
__global__ __launch_bounds__(256) void k_ssru_ln(const float* cand, const float* forget, int64_t ldc,
                                                 float* state, const float* resid, const float* gamma,
                                                 const float* beta, int rows, const int* rows_dev,
                                                 const int* state_row, float* out, int8_t* q,
                                                 float* a, int* err, float qmult, float* state_out) {
  constexpr int D = PER * 64;
  __shared__ __attribute__((aligned(16))) float sZ[4][kLnRow<PER>];
  __shared__ uint64_t sTab[32];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (threadIdx.x < 32) sTab[threadIdx.x] = kRowsExp2Tab[threadIdx.x];
  __syncthreads();
  const int row = blockIdx.x * 4 + wave;
  if (row >= (rows_dev ? min(*rows_dev, rows) : rows)) return;
  const int64_t srow = state_row ? state_row[row] : row;
  float z[PER], gv[PER], bv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e_ = lane + 64 * j;
    const float c = cand[row * ldc + e_], f = forget[row * ldc + e_];
    const float st = state[srow * D + e_], r = resid[(int64_t)row * D + e_];
    gv[j] = gamma[e_];
    bv[j] = beta[e_];
    const float e = ref_expf(-f, sTab);
    const float gate = 1.0f / (1.0f + e);
    const float next = gate * st + (1.0f - gate) * c;
    state_out[srow * D + e_] = next;
    z[j] = (next > 0.0f ? next : 0.0f) + r;
  }
  ln_row_wave<PER>(z, sZ[wave], gv, bv, row, lane, out, q, a, err, qmult);
}

// x = (q/mult)*sqrt(d) + pos[p] (q8_engine.rs:53-74, 586-630); token < 0 gives
// pos[p] alone (the decoder's first step).  Fused quantization of x with its
// own multiplier or, when a.qmult > 0, the next layer's static one; none
// when a.xq is null.
template <int PER>
__global__ __launch_bounds__(256) void k_embed(EmbedArgs a) {
  constexpr int D = PER * 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= a.rows) return;  // host bound: rows below it are allocated
  int token, p;
  if (a.tokens) {
    token = a.tokens[row];
    p = a.positions[row];
  } else {
    token = a.row_prev[row];  // read before the device row count is known
    p = a.step;
  }
  const float* pr = a.pos + (int64_t)p * D;
  float pv[PER], ev[PER];
  const int tk = token < 0 ? 0 : token;
  const int8_t* er = a.emb + (int64_t)tk * D;
  const float mult = a.emb_mult[tk];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    pv[j] = pr[lane + 64 * j];
    ev[j] = (float)er[lane + 64 * j];
  }
  const int n = a.rows_dev ? *a.rows_dev : a.rows;
  if (row >= n) return;
  float o[PER];
  float m = 0.0f;
  bool bad = false;
  if (token < 0) {
#pragma unroll
    for (int j = 0; j < PER; ++j) o[j] = pv[j];
  } else {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const float v = ev[j] / mult;
      o[j] = v * a.scale + pv[j];
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    bad |= !isfinite(o[j]);
    m = fmaxf(m, fabsf(o[j]));
    a.x[(int64_t)row * D + lane + 64 * j] = o[j];
  }
  if (a.xq) {
    m = wave_max(m);
    const float sc = a.qmult > 0.0f ? a.qmult : row_multiplier(m);
#pragma unroll
    for (int j = 0; j < PER; ++j) a.xq[(int64_t)row * D + lane + 64 * j] = (int8_t)quantize_one(o[j], sc);
    if (lane == 0) a.xa[row] = sc;
  }
  if (__any(bad) && lane == 0 && a.err) *a.err = 1;
}

// End of a decode step for at most W * R rows (R <= 8 rows per wave, W
// waves): the same work as k_finalize with no LDS scan.  Every partial key of
// the wave's rows is requested at once (rows past the host bound are clamped
// to the last one; partials past 4 x 64 come in a second pass), the rows'
// maxima are taken across the wave together (rows_max_u64), and lane i keeps
// row R * wave + i for the stop rules.  The kept rows are compacted in order
// with a ballot and a prefix count, across waves through one barrier.
constexpr int kFinalizeWaveRows = 64;

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Maxima over the wave of R (a power of two <= 64) values per lane: a
// transposed butterfly.  At lane distance d = 32, 16, ... the lanes with bit
// d set keep the upper half of their rows and trade the lower half with
// their partner, so each step halves the rows per lane with one exchange per
// kept row (R - 1 exchanges in all instead of 6 R); the remaining lane bits
// are plain maxima.  Lane l ends with the maximum of row l >> (6 - log2 R).
template <int R>
__device__ __forceinline__ uint64_t rows_max_u64(uint64_t (&b)[R], int lane) {
  static_assert(R >= 1 && R <= 64 && (R & (R - 1)) == 0, "R: a power of two");
  int d = 32;
#pragma unroll
  for (int cur = R; cur > 1; cur >>= 1, d >>= 1) {
    const bool up = lane & d;
#pragma unroll
    for (int i = 0; i < cur / 2; ++i) {
      const uint64_t keep = up ? b[i + cur / 2] : b[i];
      const uint64_t give = up ? b[i] : b[i + cur / 2];
      b[i] = umax64(keep, shfl_xor_u64(give, d));
    }
  }
  uint64_t m = b[0];
#pragma unroll
  for (; d >= 1; d >>= 1) m = umax64(m, shfl_xor_u64(m, d));
  return m;
}

template <int W, int R>
__global__ __launch_bounds__(W * 64) void k_finalize_wave(FinalizeArgs f) {
  touch_kernargs<sizeof(FinalizeArgs)>();
  constexpr int KP = 4;  // partials per row and lane requested up front
  __shared__ int s_cnt[W];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ub = min(f.rows_ub, W * R);
  const int np = f.nparts;
  const int r = R * wave + lane;  // this lane's row (lane < R)
  // Row state and partials are requested before the device row count is
  // needed (rows below the host bound are allocated).
  const int rl = min(r, ub - 1);
  const int slot = f.rows.slot[rl];
  const int64_t kv0 = f.rows.kv0[rl];
  const int64_t src0 = f.rows.src0[rl];
  const int srcn = f.rows.srcn[rl];
  const uint32_t lim = f.rows.limit[rl];
  uint64_t v[R][KP];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint64_t* pr = f.partials + (int64_t)min(R * wave + i, ub - 1) * np;
#pragma unroll
    for (int k = 0; k < KP; ++k) {
      const int p = lane + 64 * k;
      const uint64_t x = pr[min(p, np - 1)];
      v[i][k] = p < np ? x : 0;
    }
  }
  if (np > 64 * KP) {  // uniform: vocabularies over 32768 ids
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint64_t* pr = f.partials + (int64_t)min(R * wave + i, ub - 1) * np;
      for (int p = lane + 64 * KP; p < np; p += 64) v[i][0] = umax64(v[i][0], pr[p]);
    }
  }
  uint64_t b[R];
#pragma unroll
  for (int i = 0; i < R; ++i) b[i] = umax64(umax64(v[i][0], v[i][1]), umax64(v[i][2], v[i][3]));
  // Lane l holds row l >> (6 - log2 R); lane i < R fetches row i's maximum.
  constexpr int kShift = R == 1 ? 6 : R == 2 ? 5 : R == 4 ? 4 : R == 8 ? 3 : R == 16 ? 2 : R == 32 ? 1 : 0;
  const uint64_t red = rows_max_u64<R>(b, lane);
  const int src = (min(lane, R - 1) << kShift) * 4;  // byte address of the source lane
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)red);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)(red >> 32));
  const uint64_t mine = ((uint64_t)hi << 32) | lo;
  const int n_dev = *f.n_active;
  const int n = min(n_dev, ub);
  const int32_t tok = argmax_key_id(mine);
  bool keep = false;
  if (lane < R && r < n) {
    f.out_tok[kv0 + f.step] = tok;
    f.count[slot] = (uint32_t)f.step + 1u;
    const bool fin = (tok == 0 && !(f.flags & 1u)) || (uint32_t)f.step + 1u >= lim;
    keep = !fin;
  }
  const uint64_t kept = __ballot(keep);
  int base = 0, total = __popcll(kept);
  if constexpr (W > 1) {
    // A wave's compacted rows can land on rows an earlier wave read: every
    // wave's row-state loads complete (vmcnt(0)) before the barrier, after
    // which the stores start.
    if (lane == 0) s_cnt[wave] = total;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    total = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const int c = s_cnt[w];
      base += w < wave ? c : 0;
      total += c;
    }
  }
  const int pos = base + __popcll(kept & ((1ull << lane) - 1ull));  // kept rows before this one
  if (keep) {
    f.rows.slot[pos] = slot;
    f.rows.kv0[pos] = kv0;
    f.rows.src0[pos] = src0;
    f.rows.srcn[pos] = srcn;
    f.rows.limit[pos] = lim;
    f.rows.prev[pos] = tok;
  }
  if (threadIdx.x == 0) {
    if (n_dev > ub && f.err) *f.err = 3;
    if (f.active_hist) f.active_hist[f.step] = (uint32_t)n;
    *f.n_active = total;
    if (f.host_active) *f.host_active = total;
  }
}

// End of a decode step: reduce each active row's argmax partials to a token,
// append it, apply the stop rules of q8_engine.rs:383-390, 444-448, and
// compact the active list in order.  One workgroup; rows <= kMaxRowsPerCall.
// WIDE: more than 256 partials per row (vocabularies above 32768 ids), the
// ones past 256 reduced by a loop after the registers' (a loop with loads
// would make every wait before it drain all loads in flight).
constexpr int kFinalizeKP = 4;  // partials per row and lane held in registers
template <bool WIDE>
__global__ __launch_bounds__(1024) void k_finalize(FinalizeArgs f) {
  __shared__ int s_slot[kMaxRowsPerCall];
  __shared__ int s_tok[kMaxRowsPerCall];
  __shared__ int64_t s_kv0[kMaxRowsPerCall];
  __shared__ int64_t s_src0[kMaxRowsPerCall];
  __shared__ int s_srcn[kMaxRowsPerCall];
  __shared__ uint32_t s_lim[kMaxRowsPerCall];
  __shared__ unsigned char s_keep[kMaxRowsPerCall];
  __shared__ int s_wsum[16];
  __shared__ int s_total;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // Wave w takes rows 4w..4w+3 of each 64-row pass; lane i < 4 owns row
  // r0 + i.  Rows below the host bound are allocated, so the passes run as a
  // two-deep pipeline: the next pass's partials and row state are requested
  // (from clamped, always valid rows) before this pass is reduced, and no
  // global store is issued before the last load (a store counts among the
  // memory operations a load's wait covers): the tokens, counts and the
  // compacted list are written in the second phase, from LDS.
  const int ub = min(f.rows_ub, kMaxRowsPerCall);
  const int np = f.nparts;
  constexpr int KP = kFinalizeKP;
  struct Pass {
    uint64_t v[4][KP];
    int slot, srcn;
    int64_t kv0, src0;
    uint32_t lim;
  };
  auto load_pass = [&](int r0, Pass& P) {
    const int rl = min(r0 + (lane & 3), ub - 1);
    P.slot = f.rows.slot[rl];
    P.kv0 = f.rows.kv0[rl];
    P.src0 = f.rows.src0[rl];
    P.srcn = f.rows.srcn[rl];
    P.lim = f.rows.limit[rl];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint64_t* pr = f.partials + (int64_t)min(r0 + i, ub - 1) * np;
#pragma unroll
      for (int k = 0; k < KP; ++k) P.v[i][k] = pr[min(lane + 64 * k, np - 1)];  // repeats leave the max
    }
  };
  auto finish_pass = [&](int r0, const Pass& P, int n) {
    uint64_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      b[i] = P.v[i][0];
#pragma unroll
      for (int k = 1; k < KP; ++k) b[i] = umax64(b[i], P.v[i][k]);
      if constexpr (WIDE) {
        const uint64_t* pr = f.partials + (int64_t)min(r0 + i, ub - 1) * np;
        for (int q = lane + 64 * KP; q < np; q += 64) b[i] = umax64(b[i], pr[q]);
      }
      b[i] = wave_max_u64(b[i]);
    }
    const uint64_t best = lane == 0 ? b[0] : lane == 1 ? b[1] : lane == 2 ? b[2] : b[3];
    const int r = r0 + lane;
    if (lane < 4 && r < n) {
      const int32_t tok = argmax_key_id(best);
      const bool fin = (tok == 0 && !(f.flags & 1u)) || (uint32_t)f.step + 1u >= P.lim;
      s_slot[r] = P.slot;
      s_tok[r] = tok;
      s_kv0[r] = P.kv0;
      s_src0[r] = P.src0;
      s_srcn[r] = P.srcn;
      s_lim[r] = P.lim;
      s_keep[r] = fin ? 0 : 1;
    }
  };
  const int n_dev = *f.n_active;  // a scalar load: its wait covers no vector load
  int n = min(n_dev, ub);
  Pass pa, pb;
  int r0 = 4 * __builtin_amdgcn_readfirstlane(wave);  // uniform loop: no exec-masked waits
  load_pass(r0, pa);
  for (; r0 < ub; r0 += 128) {
    load_pass(r0 + 64, pb);
    __builtin_amdgcn_sched_barrier(0);  // the next pass's loads go out before this pass is reduced
    finish_pass(r0, pa, n);
    if (r0 + 64 >= ub) break;
    load_pass(r0 + 128, pa);
    __builtin_amdgcn_sched_barrier(0);
    finish_pass(r0 + 64, pb, n);
  }
  __syncthreads();
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * tid + i;
    if (r < n) cnt += s_keep[r];
  }
  int incl = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < 16; ++w) {
      const int t = s_wsum[w];
      s_wsum[w] = run;
      run += t;
    }
    s_total = run;
  }
  __syncthreads();
  int pos = s_wsum[wave] + incl - cnt;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * tid + i;
    if (r < n) {
      f.out_tok[s_kv0[r] + f.step] = s_tok[r];
      f.count[s_slot[r]] = (uint32_t)f.step + 1u;
    }
    if (r < n && s_keep[r]) {
      f.rows.slot[pos] = s_slot[r];
      f.rows.kv0[pos] = s_kv0[r];
      f.rows.src0[pos] = s_src0[r];
      f.rows.srcn[pos] = s_srcn[r];
      f.rows.limit[pos] = s_lim[r];
      f.rows.prev[pos] = s_tok[r];
      ++pos;
    }
  }
  if (tid == 0) {
    if (n_dev > ub && f.err) *f.err = 3;
    if (f.active_hist) f.active_hist[f.step] = (uint32_t)n;
    *f.n_active = s_total;
    if (f.host_active) *f.host_active = s_total;
  }
}

__global__ __launch_bounds__(256) void k_argmax_reduce(const uint64_t* partials, int nparts,
                                                       int rows, int32_t* token) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;
  uint64_t best = 0;
  for (int p = lane; p < nparts; p += 64) {
    const uint64_t k = partials[(int64_t)row * nparts + p];
    best = k > best ? k : best;
  }
  best = wave_max_u64(best);
  if (lane == 0) token[row] = argmax_key_id(best);
}

}  // namespace

hipError_t launch_quantize_rows(const float* x, int64_t ldx, int rows, const int* rows_dev,
                                int cols, int8_t* q, int64_t ldq, float* a, int* err,
                                hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  const dim3 grid((rows + 3) / 4), block(256);
  const bool vec = cols % 256 == 0 && ldx % 4 == 0 && ldq % 4 == 0 &&
                   ((uintptr_t)x % 16) == 0 && ((uintptr_t)q % 4) == 0;
  if (vec && cols == 2048)
    hipLaunchKernelGGL(k_quantize_rows_v4<8>, grid, block, 0, s, x, ldx, rows, rows_dev, q, ldq, a, err);
  else if (vec && cols == 512)
    hipLaunchKernelGGL(k_quantize_rows_v4<2>, grid, block, 0, s, x, ldx, rows, rows_dev, q, ldq, a, err);
  else if (vec && cols == 1536)
    hipLaunchKernelGGL(k_quantize_rows_v4<6>, grid, block, 0, s, x, ldx, rows, rows_dev, q, ldq, a, err);
  else
    hipLaunchKernelGGL(k_quantize_rows, grid, block, 0, s, x, ldx, rows, rows_dev, cols, q, ldq, a, err);
  return hipGetLastError();
}

// Row widths d = 64 * PER: every width the engine accepts (PER 1-8) and the
// op-level LayerNorm's up to 1024 (PER 9-16).
#define MH_PER_DISPATCH_8(PER_VALUE, CALL) \
  case 1: CALL(1); break;                  \
  case 2: CALL(2); break;                  \
  case 3: CALL(3); break;                  \
  case 4: CALL(4); break;                  \
  case 5: CALL(5); break;                  \
  case 6: CALL(6); break;                  \
  case 7: CALL(7); break;                  \
  case 8: CALL(8); break;
#define MH_PER_DISPATCH(PER_VALUE, CALL)  \
  switch (PER_VALUE) {                    \
    MH_PER_DISPATCH_8(PER_VALUE, CALL)    \
    default: return hipErrorInvalidValue; \
  }
#define MH_PER_DISPATCH_16(PER_VALUE, CALL) \
  switch (PER_VALUE) {                      \
    MH_PER_DISPATCH_8(PER_VALUE, CALL)      \
    case 9: CALL(9); break;                 \
    case 10: CALL(10); break;               \
    case 11: CALL(11); break;               \
    case 12: CALL(12); break;               \
    case 13: CALL(13); break;               \
    case 14: CALL(14); break;               \
    case 15: CALL(15); break;               \
    case 16: CALL(16); break;               \
    default: return hipErrorInvalidValue;   \
  }

hipError_t launch_residual_ln(const float* y, const float* r, const float* g, const float* b,
                              int rows, const int* rows_dev, int d, float* out, int8_t* q,
                              float* a, int* err, hipStream_t s, float qmult, bool fast) {
  if (rows <= 0) return hipSuccess;
  if (d % 64) return hipErrorInvalidValue;
  // One wave per row, four rows per workgroup: widths of 256, 384 and 512
  // fold with the one-wave speculative folds, others sequentially; with
  // `fast` (the decoder's widths) the sums take the tree order.
  const dim3 grid((rows + 3) / 4), block(256);
#define MH_LN(P) \
  hipLaunchKernelGGL(k_residual_ln<P>, grid, block, 0, s, y, r, g, b, rows, rows_dev, out, q, a, err, qmult)
#define MH_LNF(P)                                                                                            \
  hipLaunchKernelGGL((k_residual_ln<P, true>), grid, block, 0, s, y, r, g, b, rows, rows_dev, out, q, a, err, \
                     qmult)
  if (fast) {
    MH_PER_DISPATCH(d / 64, MH_LNF)
  } else {
    MH_PER_DISPATCH_16(d / 64, MH_LN)
  }
#undef MH_LNF
#undef MH_LN
  return hipGetLastError();
}

hipError_t launch_quantize_rows_static(const float* x, int64_t ldx, int rows, int cols, float mult,
                                       int8_t* q, int64_t ldq, float* a, int* err, hipStream_t s,
                                       const int* rows_dev) {
  if (rows <= 0) return hipSuccess;
  if (!(mult > 0.0f) || !(mult < __builtin_huge_valf())) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_quantize_rows_static, dim3((rows + 3) / 4), dim3(256), 0, s, x, ldx, rows, rows_dev,
                     cols, mult, q, ldq, a, err);
  return hipGetLastError();
}

hipError_t launch_ssru_ln(const float* cand, const float* forget, float* state, const float* resid,
                          const float* g, const float* b, int rows, int d, float* out, int8_t* q,
                          float* a, int* err, hipStream_t s, int64_t ldc, const int* rows_dev,
                          const int* state_row, float qmult, float* state_out) {
  if (rows <= 0) return hipSuccess;
  if (d % 64) return hipErrorInvalidValue;
  const dim3 grid((rows + 3) / 4), block(256);
  float* so = state_out ? state_out : state;
#define MH_SSRU(P) \
  hipLaunchKernelGGL(k_ssru_ln<P>, grid, block, 0, s, cand, forget, ldc > 0 ? ldc : d, state, resid, g, b, rows, \
                     rows_dev, state_row, out, q, a, err, qmult, so)
  MH_PER_DISPATCH_16(d / 64, MH_SSRU)
#undef MH_SSRU
  return hipGetLastError();
}

hipError_t launch_embed(const EmbedArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (a.d % 64) return hipErrorInvalidValue;
  const dim3 grid((a.rows + 3) / 4), block(256);
#define MH_EMB(P) hipLaunchKernelGGL(k_embed<P>, grid, block, 0, s, a)
  MH_PER_DISPATCH(a.d / 64, MH_EMB)
#undef MH_EMB
  return hipGetLastError();
}

hipError_t launch_finalize(const FinalizeArgs& f, hipStream_t s) {
  if (f.rows_ub <= 0 || f.rows_ub > kMaxRowsPerCall || f.nparts <= 0) return hipErrorInvalidValue;
  // One wave per 8 rows (4 on the smallest steps), up to kFinalizeWaveRows;
  // the workgroup scan above that.  Eight rows keep a wave's 4 x 8 partial
  // loads and its row state within the 63 loads a wave can have in flight
  // (16 rows per wave measured 5.9 µs against 3.8 µs for 8).
  if (f.rows_ub <= 4)
    hipLaunchKernelGGL((k_finalize_wave<1, 4>), dim3(1), dim3(64), 0, s, f);
  else if (f.rows_ub <= 8)
    hipLaunchKernelGGL((k_finalize_wave<1, 8>), dim3(1), dim3(64), 0, s, f);
  else if (f.rows_ub <= 16)
    hipLaunchKernelGGL((k_finalize_wave<2, 8>), dim3(1), dim3(128), 0, s, f);
  else if (f.rows_ub <= 32)
    hipLaunchKernelGGL((k_finalize_wave<4, 8>), dim3(1), dim3(256), 0, s, f);
  else if (f.rows_ub <= kFinalizeWaveRows)
    hipLaunchKernelGGL((k_finalize_wave<8, 8>), dim3(1), dim3(512), 0, s, f);
  else if (f.nparts > 64 * kFinalizeKP)
    hipLaunchKernelGGL(k_finalize<true>, dim3(1), dim3(1024), 0, s, f);
  else
    hipLaunchKernelGGL(k_finalize<false>, dim3(1), dim3(1024), 0, s, f);
  return hipGetLastError();
}

hipError_t launch_argmax_reduce(const uint64_t* partials, int nparts, int rows, int32_t* token,
                                hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_argmax_reduce, dim3((rows + 3) / 4), dim3(256), 0, s, partials, nparts,
                     rows, token);
  return hipGetLastError();
}

}  // namespace mh
