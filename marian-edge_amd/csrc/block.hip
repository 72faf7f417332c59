// block.hip — decode attention block for steps with few active rows: one
// 256-thread workgroup per (row, head) builds the row's input (the residual
// LayerNorm of the previous sublayer, or the decoder input embedding),
// projects it onto this head's query (self-attention: query, key and value)
// with int8 MFMA, and attends over the row's keys.  One launch replaces the
// LayerNorm, projection and attention kernels; the weight and K/V loads are
// issued first, so they overlap the LayerNorm's sequential folds.
//
// Every value is produced by the same operations, in the same order, as the
// separate kernels (and the reference):
//   LayerNorm       normalize_row, tensor.rs:372-385 (sequential folds)
//   quantization    q8_gemm.rs:569-590 (per-row multiplier)
//   projection      exact i32 MFMA, dequant q8_gemm.rs:438-446
//   attention       attention_into, tensor.rs:251-318 (sequential dot, max,
//                   C-library expf, sequential sum from 0.0, PV in key order)
#include "device_common.h"
#include "kernels.h"
#include <hip/hip_ext.h>

namespace mh {
namespace {

constexpr int kBlkRowWaves = 4;   // waves 0-3: the input row (wave 0; 1-3 exit)
constexpr int kBlkLoadWaves = 4;  // waves 4-7 load weights and keys, then project
constexpr int kBlkThreads = 64 * (kBlkRowWaves + kBlkLoadWaves);
constexpr int kBlkD = 512;             // model width handled (8 heads x 64)
constexpr int kBlkMaxKeys = 128;       // keys staged in LDS
constexpr int kBlkRow = kHeadDim + 4;  // padded LDS key row (floats)
constexpr int kPvRow = kBlkMaxKeys + 4;  // padded LDS row of one dimension's PV products
static_assert(kHeadDim * kPvRow <= kBlkMaxKeys * kBlkRow, "the PV products fit in the key rows");

__constant__ uint64_t kBlkExp2Tab[32] = {MH_EXP2_TABLE_32};

__device__ __forceinline__ v4i zero4b() { return v4i{0, 0, 0, 0}; }

// Ends a batch of a software-pipelined loop: neither the IR optimizer nor the
// scheduler moves memory accesses across it, so only one batch is read ahead.
__device__ __forceinline__ void batch_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}


// ---- the input row, built by one wave: lane l holds elements 4l..4l+3 and
// 256+4l..256+4l+3 of the kBlkD-wide row ---------------------------------------
template <int PK>
struct RowLoads {
  f4v a[2], b[2], g[2], bb[2];  // LN: y, r, gamma, beta; embedding: pos in a
  uint32_t e4[2];               // embedding: four int8 entries
  float mu = 1.0f;              // embedding: the token's multiplier
  int tok = -1;
};

// Loads of row r (issued before the device row count is known).
template <int PK>
__device__ __forceinline__ void row_load(const RowPrologue& p, int r, int step, int lane, RowLoads<PK>& L) {
  if constexpr (PK == PRO_LN) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = 4 * lane + 256 * j;
      L.a[j] = *(const f4v*)(p.y + (int64_t)r * kBlkD + e);
      L.b[j] = *(const f4v*)(p.r + (int64_t)r * kBlkD + e);
      L.g[j] = *(const f4v*)(p.gamma + e);
      L.bb[j] = *(const f4v*)(p.beta + e);
    }
  } else {
    L.tok = p.row_prev[r];
    const int tk = max(L.tok, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int e = 4 * lane + 256 * j;
      L.a[j] = *(const f4v*)(p.pos + (int64_t)step * kBlkD + e);
      L.e4[j] = *(const uint32_t*)(p.emb + (int64_t)tk * kBlkD + e);
    }
    L.mu = p.emb_mult[tk];
  }
}

// The row's values built by one wave: LayerNorm(y + r) with its two
// sequential folds over an LDS copy (sZ), or the scaled embedding plus the
// position row.
template <int PK>
__device__ __forceinline__ void row_build(const RowPrologue& p, const RowLoads<PK>& L, float* sZ,
                                          int lane, f4v (&o)[2]) {
  if constexpr (PK == PRO_LN) {
    f4v z[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      z[j] = L.a[j] + L.b[j];  // add_slices
      *(f4v*)(sZ + 4 * lane + 256 * j) = z[j];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes land
    __builtin_amdgcn_wave_barrier();
    const float mean = seq_fold_lds<kBlkD / 4>((const float4*)sZ, -0.0f) / (float)kBlkD;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const f4v c = z[j] - mean;
      *(f4v*)(sZ + 4 * lane + 256 * j) = c * c;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    const float var = seq_fold_lds<kBlkD / 4>((const float4*)sZ, -0.0f) / (float)kBlkD;
    const float inv = 1.0f / sqrtf(var + kLayerNormEpsilon);
#pragma unroll
    for (int j = 0; j < 2; ++j) o[j] = ((z[j] - mean) * inv) * L.g[j] + L.bb[j];
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (L.tok < 0) {
        o[j] = L.a[j];
      } else {
        f4v v;
        v.x = (float)(int8_t)(L.e4[j] & 0xFF) / L.mu;
        v.y = (float)(int8_t)((L.e4[j] >> 8) & 0xFF) / L.mu;
        v.z = (float)(int8_t)((L.e4[j] >> 16) & 0xFF) / L.mu;
        v.w = (float)(int8_t)(L.e4[j] >> 24) / L.mu;
        o[j] = v * p.scale + L.a[j];
      }
    }
  }
}

// Quantizes the row into sX with its row multiplier (returned); `bad` tells
// whether any value is not finite.
__device__ __forceinline__ float row_quantize(const f4v (&o)[2], int8_t* sX, int lane, bool& bad) {
  bad = false;
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    bad |= !isfinite(o[j].x) || !isfinite(o[j].y) || !isfinite(o[j].z) || !isfinite(o[j].w);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(o[j].x), fabsf(o[j].y)), fmaxf(fabsf(o[j].z), fabsf(o[j].w))));
  }
  const float a_row = row_multiplier(wave_max(m));
#pragma unroll
  for (int j = 0; j < 2; ++j)
    *(uint32_t*)(sX + 4 * lane + 256 * j) = (uint32_t)(quantize_one(o[j].x, a_row) & 0xFF) |
                                            ((uint32_t)(quantize_one(o[j].y, a_row) & 0xFF) << 8) |
                                            ((uint32_t)(quantize_one(o[j].z, a_row) & 0xFF) << 16) |
                                            ((uint32_t)(quantize_one(o[j].w, a_row) & 0xFF) << 24);
  return a_row;
}

// Row 0 of 16-row MFMA tiles against T column tiles whose weight fragments
// are in registers.  Every lane reads the row's 16-byte k-slice from LDS (a
// broadcast: rows 1-15 of the A tile repeat row 0, and their outputs are never
// used), k-step outer, so one LDS read feeds every tile and the tiles' chains
// run interleaved; with one or two tiles the k-steps alternate between two
// chains per tile.  The sums are exact i32, so the split does not change them.
// Returns row 0 (lanes 0-15: the tile's 16 columns).
template <int T>
__device__ __forceinline__ void row_tiles_mfma(const int8_t* sX, const v4i (&bf)[T][kBlkD / 64], int kq,
                                               int32_t (&out)[T]) {
  constexpr int CH = T <= 2 ? 2 : 1;
  v4i acc[T][CH];
#pragma unroll
  for (int i = 0; i < T; ++i)
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[i][c] = zero4b();
#pragma unroll
  for (int s = 0; s < kBlkD / 64; ++s) {
    const v4i af = *(const v4i*)(sX + s * 64 + kq);
#pragma unroll
    for (int i = 0; i < T; ++i)
      acc[i][s % CH] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[i][s], acc[i][s % CH], 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < T; ++i) out[i] = CH == 2 ? acc[i][0][0] + acc[i][1][0] : acc[i][0][0];
}

// Work split: wave 0 builds the input row (a LayerNorm with the one-wave
// speculative folds, or the embedding row), waves 1-3 exit at once; waves
// 4-7 meanwhile load this head's weight rows and stage the row's keys and
// values in LDS, then run the projection; wave 0 attends, helped by waves 4-7
// (wave 5: a second chunk of scores; all four: the PV products).
constexpr int kBlkLoaders = 64 * kBlkLoadWaves;
static_assert(kBlkRow % 4 == 0 && kBlkMaxKeys * (kBlkRow / 4) % 64 == 0, "key staging by wave instructions");

// FAST: the LayerNorm sums and the softmax denominator in the fast-reduction
// tree order (tree_sum_wave / tree_combine_wave) instead of the folds.
template <int MODE, int PK, bool FAST>
__global__ __launch_bounds__(kBlkThreads) void k_attn_block(BlockArgs b) {
  constexpr bool SELF = MODE == ATT_SELF;
  constexpr int NT = SELF ? 12 : 4;        // 16-column projection tiles: Q (+ K, V)
  constexpr int TPW = NT / kBlkLoadWaves;  // tiles per loader wave
  static_assert(NT % kBlkLoadWaves == 0, "every loader wave owns whole tiles");
  __shared__ __attribute__((aligned(16))) float sK[kBlkMaxKeys * kBlkRow];
  __shared__ __attribute__((aligned(16))) float sV[kBlkMaxKeys * kBlkRow];
  constexpr int PER = kBlkD / 64;  // LayerNorm row: lane l holds elements l + 64j
  __shared__ __attribute__((aligned(16))) float sZ[PK == PRO_LN ? kLnRow<PER> : kBlkD];
  __shared__ __attribute__((aligned(16))) int8_t sX[kBlkD];
  __shared__ __attribute__((aligned(16))) float sQ[kHeadDim];
  __shared__ __attribute__((aligned(16))) float sP[kBlkMaxKeys];
  __shared__ uint64_t sTab[32];
  __shared__ float sA;
  __shared__ float sS[64];

  touch_kernargs<sizeof(BlockArgs)>();
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // Row-major ids: workgroups are dealt to the 8 XCDs in turn, so head h of
  // every row runs on XCD h and each XCD reads one head's weights.
  const int h = blockIdx.x % b.heads, r = blockIdx.x / b.heads;  // r < b.rows (host bound)
  const int step = b.step;
  // Key range of this row (read before the device row count is known; rows
  // past it read clamped stale ranges and are discarded below).  Each wave
  // reads it, and the device row count, only after its first loads are
  // issued: a load whose value a branch needs is waited for there, and the
  // compiler would otherwise sink the wave's other loads below that wait.
  int64_t key0;
  int nk_row, nkm, nk_ld, nkey;
  auto key_range = [&]() {
    key0 = b.row_key0[r];
    nk_row = SELF ? step : b.row_nk[r];
    key0 = min(max(key0, (int64_t)0), b.max_row - 1);
    nkm = max(min(nk_row, kBlkMaxKeys - (SELF ? 1 : 0)), SELF ? 0 : 1);  // keys from memory
    nk_ld = (int)min((int64_t)nkm, b.max_row - key0);                   // readable rows
    nkey = SELF ? nkm + 1 : nkm;                                       // keys attended
  };

  if (wave < kBlkRowWaves) {
    // ---- the input row ----------------------------------------------------------
    if (wave != 0) return;  // wave 0 builds the row
    const uint64_t tab_v = kBlkExp2Tab[lane & 31];
    bool bad;
    float a_row;
    if constexpr (PK == PRO_LN) {
      // LayerNorm(y + r) with the one-wave speculative folds (ln_wave).
      float y[PER], rr[PER], gv[PER], bv[PER];
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int64_t e = (int64_t)r * kBlkD + lane + 64 * j;
        y[j] = b.pro.y[e];
        rr[j] = b.pro.r[e];
        gv[j] = b.pro.gamma[lane + 64 * j];
        bv[j] = b.pro.beta[lane + 64 * j];
      }
      asm volatile("" ::: "memory");  // the row loads are issued first
      if (r >= bounded_rows(b.rows_dev, b.rows)) return;
      key_range();
      float z[PER], o[PER];
#pragma unroll
      for (int j = 0; j < PER; ++j) z[j] = y[j] + rr[j];  // add_slices
      ln_wave<PER, FAST>(z, sZ, gv, bv, lane, o);
      bad = false;
      float mx = 0.0f;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        bad |= !isfinite(o[j]);
        mx = fmaxf(mx, fabsf(o[j]));
      }
      a_row = row_multiplier(wave_max(mx));
#pragma unroll
      for (int j = 0; j < PER; ++j) sX[lane + 64 * j] = (int8_t)quantize_one(o[j], a_row);
      if (h == 0 && b.pro.out) {
#pragma unroll
        for (int j = 0; j < PER; ++j) b.pro.out[(int64_t)r * kBlkD + lane + 64 * j] = o[j];
      }
    } else {
      RowLoads<PK> in;
      row_load<PK>(b.pro, r, step, lane, in);
      asm volatile("" ::: "memory");  // the row loads are issued first
      if (r >= bounded_rows(b.rows_dev, b.rows)) return;
      key_range();
      f4v o[2];
      row_build<PK>(b.pro, in, sZ, lane, o);
      a_row = row_quantize(o, sX, lane, bad);
      if (h == 0 && b.pro.out) {
#pragma unroll
        for (int j = 0; j < 2; ++j) *(f4v*)(b.pro.out + (int64_t)r * kBlkD + 4 * lane + 256 * j) = o[j];
      }
    }
    if (lane == 0) sA = a_row;
    if (lane < 32) sTab[lane] = tab_v;
    if (__any(bad) && lane == 0 && b.err) *b.err = 1;
    if (lane == 0 && nk_row > nkm && b.err) *b.err = 2;  // more keys than the LDS stages
    __syncthreads();  // input row published; keys staged
    __syncthreads();  // projection done
  } else {
    // ---- waves 4-7: weights, then the keys and values into LDS -----------------
    const int lw = wave - kBlkRowWaves;  // loader wave
    const int kq = (lane >> 4) * 16;
    v4i bf[TPW][kBlkD / 64];
    float wm[TPW], bi[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = lw + kBlkLoadWaves * i;  // 16 columns of Q, K or V
      const int c0 = (tile / 4) * kBlkD + h * kHeadDim + (tile % 4) * 16;
      const int n_w = c0 + (lane & 15);
#pragma unroll
      for (int s = 0; s < kBlkD / 64; ++s) bf[i][s] = frag_load(b.W, c0 / 16, kBlkD / 64, s, lane);
      wm[i] = b.wmult[n_w];
      bi[i] = b.bias[n_w];
    }
    asm volatile("" ::: "memory");  // the weight loads are issued first
    key_range();
    // Key and value rows go straight from memory into the padded LDS rows
    // (global_load_lds, 16 bytes per lane, no registers): an LDS row is 17
    // 16-byte slots, the last one padding.  Wave instruction i fills slots
    // [64i, 64i + 64); lanes on padding or past the readable keys are masked
    // off and leave their slot untouched.
    const int64_t base = key0 * b.ldkv + h * kHeadDim;
    constexpr int kSlots = kBlkRow / 4;  // 17
    const int n_inst = (nk_ld * kSlots + 63) >> 6;
    for (int i = lw; i < n_inst; i += kBlkLoadWaves) {
      const int slot = 64 * i + lane, key = slot / kSlots, c = slot - key * kSlots;
      if (c < kHeadDim / 4 && key < nk_ld) {
        const int64_t off = base + (int64_t)key * b.ldkv + c * 4;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(b.k + off),
                                         (__attribute__((address_space(3))) void*)(sK + 256 * i), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(b.v + off),
                                         (__attribute__((address_space(3))) void*)(sV + 256 * i), 16, 0, 0);
      }
    }
    if (r >= bounded_rows(b.rows_dev, b.rows)) {
      __builtin_amdgcn_s_waitcnt(0);  // no LDS write may land after the workgroup ends
      return;
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's key and value rows are in LDS
    // Value rows from the last key up to the next multiple of 16 are zero, so
    // the PV products of the folds' whole batches of 16 keys are +0.
    const int u = tid - 64 * kBlkRowWaves;
    const int zrows = min((nkey + 15) & ~15, kBlkMaxKeys) - nkey;
    for (int idx = u; idx < zrows * 16; idx += kBlkLoaders)
      *(f4v*)(sV + (nkey + (idx >> 4)) * kBlkRow + (idx & 15) * 4) = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();  // the input row (wave 0) is in LDS
    // ---- projection: row 0 of 16-row MFMA tiles; the dequantization scales
    // are computed while the matrix cores run ------------------------------------
    const float a_row = sA;
    float inv[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) inv[i] = dequant_scale(a_row, wm[i]);
    int32_t acc[TPW];
    row_tiles_mfma<TPW>(sX, bf, kq, acc);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tile = lw + kBlkLoadWaves * i;
      if (lane < 16) {  // lanes 0..15 hold row 0 of the tile's 16 columns
        const int c = (tile % 4) * 16 + lane;
        const float yv = dequant_apply(acc[i], inv[i], bi[i]);
        if (tile < 4) {
          sQ[c] = yv;
        } else if (tile < 8) {
          // This step's key: attended now and cached for later steps.
          sK[nkm * kBlkRow + c] = yv;
          b.kc_out[(key0 + step) * b.ldkv + h * kHeadDim + c] = yv;
        } else {
          sV[nkm * kBlkRow + c] = yv;
          b.vc_out[(key0 + step) * b.ldkv + h * kHeadDim + c] = yv;
        }
      }
    }
    __syncthreads();  // query and keys are in LDS
  }

  // ---- attention: wave 0, helped by waves 4-7 ----------------------------------
  // Scores: lane = key of chunk c (keys c*64 + lane), 64-term dot in
  // dimension order, one chain per wave: wave 0 takes chunk 0 and, with more
  // than 64 keys, wave 5 (another SIMD) takes chunk 1, handed to wave 0
  // through LDS.  The key rows and the query (every lane the same address: a
  // broadcast) come from LDS in batches of 8 dimensions, read three batches
  // ahead; the products of the next batch are formed between the dependent
  // adds of the current one (one add and one multiply per scheduling group),
  // so the adds wait only for each other.
  const bool two = nkey > 64;
  const int n16 = (nkey + 15) >> 4;  // the folds' batches of 16 keys
  float sc = -INFINITY;
  if (wave == 0 || (two && wave == kBlkRowWaves + 1)) {
    const int c = wave == 0 ? 0 : 1;
    const float* kr = sK + min(c * 64 + lane, nkey - 1) * kBlkRow;
    constexpr int kNb = kHeadDim / 8;  // batches of 8 dimensions
    f4v kb[4][2], qb[4][2];            // batch b in slot b % 4
    float pr[2][8];                    // products of batch b in pr[b % 2]
    auto rd = [&](int bt) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        kb[bt & 3][i] = *(const f4v*)(kr + 8 * bt + 4 * i);
        qb[bt & 3][i] = *(const f4v*)(sQ + 8 * bt + 4 * i);
      }
    };
    const float scale = 1.0f / sqrtf((float)kHeadDim);
    float da = -0.0f;
    rd(0);
    rd(1);
    rd(2);
    batch_fence();
#pragma unroll
    for (int i = 0; i < 8; ++i) pr[0][i] = qb[0][i >> 2][i & 3] * kb[0][i >> 2][i & 3];
#pragma unroll
    for (int bt = 0; bt < kNb; ++bt) {
      if (bt + 3 < kNb) rd(bt + 3);
      batch_fence();
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        da = da + pr[bt & 1][i];
        if (bt + 1 < kNb) pr[(bt + 1) & 1][i] = qb[(bt + 1) & 3][i >> 2][i & 3] * kb[(bt + 1) & 3][i >> 2][i & 3];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (c * 64 + lane < nkey) sc = da * scale;
    if (c == 1) sS[lane] = sc;
  }
  if (two) wg_lds_barrier();  // chunk 1's scores are in LDS
  if (wave == 0) {
    const float sc1 = two ? sS[lane] : -INFINITY;
    const float mx = wave_max(fmaxf(sc, sc1));
    const float e0 = lane < nkey ? ref_expf(sc - mx, sTab) : 0.0f;
    const float e1 = 64 + lane < nkey ? ref_expf(sc1 - mx, sTab) : 0.0f;
    float inv;
    if constexpr (FAST) {
      // Lane l's keys l and 64 + l in order from 0.0 (0.0 + e0 is e0), then
      // the butterfly; +0.0 past the last key leaves the sums unchanged.
      inv = 1.0f / tree_combine_wave(e0 + e1);
    } else {
      sP[lane] = e0;
      sP[64 + lane] = e1;
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes land
      __builtin_amdgcn_wave_barrier();
      // Denominator: keys in order from 0.0 (softmax_in_place), folded over
      // whole batches of 16 entries: past the last key they hold +0.0, which
      // leaves the (non-negative) sum unchanged.
      inv = 1.0f / seq_fold_lds_upto<kBlkMaxKeys / 16>((const float4*)sP, n16, 0.0f);
      __builtin_amdgcn_wave_barrier();
    }
    // p_k = e_k * inv (scale_in_place)
    sP[lane] = e0 * inv;
    sP[64 + lane] = e1 * inv;
  }
  wg_lds_barrier();  // p is in LDS; the key rows are no longer read
  // PV: out_d = sum_k v_k[d] * p_k in key order.  Waves 4-7 form the
  // products (the same roundings as inside the sum) into the freed key rows,
  // transposed: row d (stride kPvRow) holds dimension d's products in key
  // order.  Lane = key of a 64-key chunk; each wave owns fixed groups of four
  // dimensions, all of its reads issued at once.  Wave 0 then folds its lane's
  // row in key order, over whole batches of 16 keys: past the last key p is +0
  // and the value rows are zero, so those products are +0 and leave the sum
  // (never -0) unchanged.  Products of keys past the batches are not read.
  float* sPv = sK;
  if (wave >= kBlkRowWaves) {
    constexpr int kGroups = kHeadDim / 4 / kBlkLoadWaves;  // 4-dimension groups per wave and chunk
    const int lw = wave - kBlkRowWaves;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      if (c == 1 && !two) break;
      const float pj = sP[c * 64 + lane];
      const float* vr = sV + (c * 64 + lane) * kBlkRow;
      f4v v[kGroups];
#pragma unroll
      for (int g = 0; g < kGroups; ++g) v[g] = *(const f4v*)(vr + 4 * (lw + kBlkLoadWaves * g));
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        const int d0 = 4 * (lw + kBlkLoadWaves * g);
        float* t = sPv + d0 * kPvRow + c * 64 + lane;
        t[0] = v[g].x * pj;
        t[kPvRow] = v[g].y * pj;
        t[2 * kPvRow] = v[g].z * pj;
        t[3 * kPvRow] = v[g].w * pj;
      }
    }
  }
  wg_lds_barrier();  // the products are in LDS
  if (wave != 0) return;
  const float o = seq_fold_lds_upto<kBlkMaxKeys / 16>((const float4*)(sPv + lane * kPvRow), n16, 0.0f);
  b.out[(int64_t)r * b.ldo + h * kHeadDim + lane] = o;
  const bool bad = !isfinite(o);
  const float am = wave_max(fabsf(o));
  if (lane == 0 && b.amax) b.amax[(int64_t)r * b.heads + h] = am;
  if (__any(bad) && lane == 0 && b.err) *b.err = 1;
}


// ---------------------------------------------------------------------------
// LayerNorm + up-projection block (the FFN's first layer on steps with few
// rows): one 512-thread workgroup per (row, 128-column slice).  Wave 0
// builds the row's residual LayerNorm (one-wave speculative folds) and
// quantizes it, as in the attention block; waves 4-7 meanwhile load the
// slice's weight rows into registers, then run the projection on MFMA (row 0
// of a 16-row tile), dequantize, apply ReLU and store.  Replaces the
// LayerNorm kernel and the skinny GEMM that followed it.
// ---------------------------------------------------------------------------
constexpr int kLgCols = 128;                                      // output columns per workgroup
constexpr int kLgTiles = kLgCols / 16;                            // MFMA column tiles per workgroup
constexpr int kLgTpw = kLgTiles / kBlkLoadWaves;  // tiles per loader wave
static_assert(kLgTiles % kBlkLoadWaves == 0, "every loader wave owns whole tiles");

template <bool FAST>
__global__ __launch_bounds__(kBlkThreads) void k_ln_gemm_block(LnGemmArgs a) {
  touch_kernargs<sizeof(LnGemmArgs)>();
  constexpr int PER = kBlkD / 64;  // lane l holds row elements l + 64j
  __shared__ __attribute__((aligned(16))) float sZ[kLnRow<PER>];
  __shared__ __attribute__((aligned(16))) int8_t sX[kBlkD];
  __shared__ float sA;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int slices = a.N / kLgCols;
  const int slice = blockIdx.x % slices, r = blockIdx.x / slices;  // r < a.rows (host bound)
  // The device row count is read after each wave's loads are issued (the
  // compiler would otherwise sink the loads below the wait for it).
  if (wave < kBlkRowWaves) {
    if (wave != 0) return;  // wave 0 builds the row with the one-wave folds
    float y[PER], rr[PER], gv[PER], bv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int64_t e = (int64_t)r * kBlkD + lane + 64 * j;
      y[j] = a.pro.y[e];
      rr[j] = a.pro.r[e];
      gv[j] = a.pro.gamma[lane + 64 * j];
      bv[j] = a.pro.beta[lane + 64 * j];
    }
    asm volatile("" ::: "memory");  // the row loads are issued first
    if (r >= bounded_rows(a.rows_dev, a.rows)) return;
    float z[PER], o[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) z[j] = y[j] + rr[j];  // add_slices
    ln_wave<PER, FAST>(z, sZ, gv, bv, lane, o);
    bool bad = false;
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      bad |= !isfinite(o[j]);
      mx = fmaxf(mx, fabsf(o[j]));
    }
    const float a_row = row_multiplier(wave_max(mx));
#pragma unroll
    for (int j = 0; j < PER; ++j) sX[lane + 64 * j] = (int8_t)quantize_one(o[j], a_row);
    if (slice == 0 && a.pro.out) {
#pragma unroll
      for (int j = 0; j < PER; ++j) a.pro.out[(int64_t)r * kBlkD + lane + 64 * j] = o[j];
    }
    if (lane == 0) sA = a_row;
    if (__any(bad) && lane == 0 && a.err) *a.err = 1;
    __syncthreads();  // the quantized row is in LDS
    return;
  }
  const int lw = wave - kBlkRowWaves;  // loader wave
  const int kq = (lane >> 4) * 16;
  v4i bf[kLgTpw][kBlkD / 64];
  float wm[kLgTpw], bi[kLgTpw];
#pragma unroll
  for (int i = 0; i < kLgTpw; ++i) {
    const int tile = lw + kBlkLoadWaves * i;
    const int col = slice * kLgCols + tile * 16 + (lane & 15);
#pragma unroll
    for (int s = 0; s < kBlkD / 64; ++s) bf[i][s] = frag_load(a.W, slice * kLgTiles + tile, kBlkD / 64, s, lane);
    wm[i] = a.wmult[col];
    bi[i] = a.bias[col];
  }
  asm volatile("" ::: "memory");  // the weight loads are issued first
  if (r >= bounded_rows(a.rows_dev, a.rows)) return;
  __syncthreads();  // the quantized row is in LDS
  const float a_row = sA;
  float inv[kLgTpw];
#pragma unroll
  for (int i = 0; i < kLgTpw; ++i) inv[i] = dequant_scale(a_row, wm[i]);
  int32_t acc[kLgTpw];
  row_tiles_mfma<kLgTpw>(sX, bf, kq, acc);
#pragma unroll
  for (int i = 0; i < kLgTpw; ++i) {
    const int tile = lw + kBlkLoadWaves * i;
    if (lane < 16) {  // lanes 0..15 hold row 0 of the tile's 16 columns
      float y = dequant_apply(acc[i], inv[i], bi[i]);
      if (a.relu) y = y > 0.0f ? y : 0.0f;
      a.out[(int64_t)r * a.ldo + slice * kLgCols + tile * 16 + lane] = y;
    }
  }
}
}  // namespace

bool attn_block_supported(int d, int heads, int max_keys) {
  return d == kBlkD && heads * kHeadDim == kBlkD && max_keys >= 1 && max_keys <= kBlkMaxKeys;
}

hipError_t launch_attn_block(const BlockArgs& b, hipStream_t s, hipEvent_t ev_start,
                             hipEvent_t ev_stop) {
  if (b.rows <= 0) return hipSuccess;
  if (!attn_block_supported(kBlkD, b.heads, b.max_keys) || !b.W || !b.wmult || !b.bias ||
      !b.k || !b.v || !b.out || !b.row_key0 || b.max_row <= 0 ||
      (b.mode == ATT_CROSS && !b.row_nk) ||
      (b.mode == ATT_SELF && (!b.kc_out || !b.vc_out || b.step < 0 || b.step + 1 > kBlkMaxKeys)))
    return hipErrorInvalidValue;
  const RowPrologue& p = b.pro;
  if (p.kind == PRO_LN ? !(p.y && p.r && p.gamma && p.beta)
                       : !(p.kind == PRO_EMB && p.emb && p.emb_mult && p.pos && p.row_prev &&
                           b.step >= 0 && b.step < kMaxPosition))
    return hipErrorInvalidValue;
  if (b.mode == ATT_CROSS && p.kind != PRO_LN) return hipErrorInvalidValue;
  const dim3 grid(b.rows * b.heads), block(kBlkThreads);
  auto kern = b.fast ? (b.mode == ATT_CROSS ? k_attn_block<ATT_CROSS, PRO_LN, true>
                        : p.kind == PRO_LN  ? k_attn_block<ATT_SELF, PRO_LN, true>
                                            : k_attn_block<ATT_SELF, PRO_EMB, true>)
                     : (b.mode == ATT_CROSS ? k_attn_block<ATT_CROSS, PRO_LN, false>
                        : p.kind == PRO_LN  ? k_attn_block<ATT_SELF, PRO_LN, false>
                                            : k_attn_block<ATT_SELF, PRO_EMB, false>);
  // With events the dispatch itself records them at its start and end.
  if (ev_start || ev_stop)
    hipExtLaunchKernelGGL(kern, grid, block, 0, s, ev_start, ev_stop, 0, b);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, s, b);
  return hipGetLastError();
}

bool ln_gemm_block_supported(int K, int N) { return K == kBlkD && N > 0 && N % kLgCols == 0; }

hipError_t launch_ln_gemm_block(const LnGemmArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const RowPrologue& p = a.pro;
  if (!ln_gemm_block_supported(a.K, a.N) || p.kind != PRO_LN || !p.y || !p.r || !p.gamma ||
      !p.beta || !a.W || !a.wmult || !a.bias || !a.out || a.ldo < a.N)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(p.fast ? k_ln_gemm_block<true> : k_ln_gemm_block<false>, dim3(a.rows * (a.N / kLgCols)),
                     dim3(kBlkThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace mh
