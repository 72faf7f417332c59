// gemm.hip — int8 x int8 -> i32 GEMMs on CDNA4 MFMA (v_mfma_i32_16x16x64_i8).
//
// Both operands are K-contiguous: activations A[M, K] row-major and weights
// W[N, K] in the reference's canonical [out, in] layout, so an MFMA operand
// fragment (16 rows x 16 consecutive k per lane) is one 16-byte load from
// either matrix.  Accumulators are exact i32 (|acc| <= 127*127*K < 2^31 for
// K <= 2048+), so the summation order inside the matrix core does not matter:
// the result equals the closed form sum_k qa*qw of q8_gemm.rs:539-553.
//
// Epilogue: y = acc * (1/(a_m * w_n)) + b_n (q8_gemm.rs:438-446), optional
// ReLU (tensor.rs:114-116), optional raw i32 store.
#include "device_common.h"
#include "kernels.h"
#include <hip/hip_ext.h>

namespace mh {
namespace {

constexpr int kSkinnyRows = 64;    // rows per pass of the skinny kernel
constexpr int kSkinnyMaxK = 2048;  // 8 waves x 4 k-steps x 64


__device__ __forceinline__ v4i zero4() { return v4i{0, 0, 0, 0}; }
// v where keep holds, else zero, with v's load issued either way (its address
// must be valid).  The mask goes through an empty asm so that the compiler
// cannot turn the choice back into a select, which it lowers to a branch
// around the load; a load behind a branch is waited for inside it, which
// serializes the loads issued before and after it.
__device__ __forceinline__ v4i keep_or_zero(v4i v, bool keep) {
  int m = keep ? -1 : 0;
  asm("" : "+v"(m));
  return v & v4i{m, m, m, m};
}

// ---------------------------------------------------------------------------
// Skinny GEMM (decode and small M).  One workgroup owns CT*16 output columns
// for every row; its NW waves split K (wave w takes k-steps w, w+NW, ...),
// load their A and B fragments straight from memory (A is small and L2
// resident, B = the weights, streamed once per 64 rows), and add their exact
// i32 partial tiles into LDS with integer atomics, so the reduction order is
// irrelevant.  The epilogue then walks the LDS tile row-major: consecutive
// threads write consecutive columns.
// ---------------------------------------------------------------------------
// Row multiplier of row m of an fp32 A source from its producer's partial
// maxima (`parts` per row, one per attention head).  EIGHT: exactly eight
// parts, read as two 16-byte vectors with no branch, so that the loads issue
// together with the kernel's other prologue loads (a load behind a branch
// is waited for inside the branch).
constexpr int kAfParts = 8;
constexpr int kAfMaxParts = 16;
template <bool EIGHT>
__device__ __forceinline__ float af_row_mult(const float* amax, int m, int parts) {
  float mx = 0.0f;
  if constexpr (EIGHT) {
    const float4* p = (const float4*)(amax + (int64_t)m * kAfParts);
    const float4 u = p[0], v = p[1];
    mx = fmaxf(fmaxf(fmaxf(u.x, u.y), fmaxf(u.z, u.w)), fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
  } else {
#pragma unroll
    for (int i = 0; i < kAfMaxParts; ++i)
      if (i < parts) mx = fmaxf(mx, amax[(int64_t)m * parts + i]);
  }
  return row_multiplier(fmaxf(mx, 0.0f));
}

// 16 consecutive fp32 values quantized with multiplier a, packed as the
// 16 int8 bytes of an MFMA operand fragment (byte j = element j).
__device__ __forceinline__ v4i quantize_frag16(const float4 (&f)[4], float a) {
  v4i r;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    r[w] = (quantize_one(f[w].x, a) & 0xFF) | ((quantize_one(f[w].y, a) & 0xFF) << 8) |
           ((quantize_one(f[w].z, a) & 0xFF) << 16) | ((quantize_one(f[w].w, a) & 0xFF) << 24);
  return r;
}
constexpr int kAfRows = 16;  // fp32 A source: one MFMA row tile per workgroup

// A sources of the skinny kernel: int8 rows with their multipliers, or fp32
// rows quantized while loading, with the row maxima of the producer in eight
// parts (A_F32) or in another number of parts (A_F32_P), or found here over
// all of K (A_F32_MAX).  A_I8_RG: int8 rows in 16-row groups over
// blockIdx.y, as the fp32 sources are (plain stores or the QKV cache; no
// int32 or quantized copies).
enum ASrc { A_I8 = 0, A_F32 = 1, A_F32_MAX = 2, A_I8_RG = 3, A_F32_P = 4 };

// FULL: K is exactly NW x KSW k-steps (every shape the engine uses), so no
// k-step needs a guard and every prologue load is unconditional (guarded
// loads become branches that the compiler waits on one by one).
template <int MODE, int CT, int NW, int KSW, int ASRC, bool FULL>
__global__ __launch_bounds__(NW * 64) void k_gemm_skinny(GemmArgs g, Epilogue e) {
  touch_kernargs<sizeof(GemmArgs) + sizeof(Epilogue)>();
  constexpr bool AF = ASRC == A_F32 || ASRC == A_F32_MAX || ASRC == A_F32_P;  // fp32 A, quantized while loading
  constexpr bool AX = ASRC == A_F32_MAX;   // ... with the row maxima found here
  constexpr bool A8 = ASRC == A_F32;       // ... with the producer's maxima in eight parts
  constexpr bool RG = ASRC != A_I8;        // one 16-row group per workgroup
  constexpr int NT = NW * 64;
  constexpr int COLS = CT * 16;
  constexpr int LDC = COLS + 1;          // padded LDS row (i32)
  constexpr int ROWS_PER_THREAD = kSkinnyRows * COLS / NT;
  __shared__ int32_t sAcc[kSkinnyRows * LDC];
  __shared__ float sRowMax[AX ? NW * kAfRows : 1];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * COLS;
  const int kq = (lane >> 4) * 16;
  const int ksteps = g.K >> 6;
  // An fp32 A source is split into 16-row groups over blockIdx.y: each
  // workgroup quantizes only its own rows (one MFMA row tile).
  const int r0 = RG ? (int)blockIdx.y * kAfRows : 0;
  const float* Af = AF ? g.Af + (int64_t)r0 * g.ldaf : nullptr;
  const int8_t* Ai = AF ? nullptr : g.A + (int64_t)r0 * g.lda;
  const float* ai = AF ? nullptr : g.a + r0;
  const float* Aamax = AF && !AX ? g.Aamax + (int64_t)r0 * g.amax_parts : nullptr;
  float* out = e.out ? e.out + (int64_t)r0 * e.ldo : nullptr;
  // g.M bounds the rows on the host side; every row below it is allocated,
  // so the first row chunk's activations are loaded before the device row
  // count (g.M_dev) is known.
  const int Mh = RG ? min(g.M - r0, kAfRows) : g.M;

  // Every weight fragment of this wave (k-steps wave, wave+NW, ...).
  v4i bf[KSW][CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    // Fragment order: the tile's next k-step is 1 KB further; row-major: 64
    // bytes along the lane's weight row.
    const int n = min(n0 + ct * 16 + (lane & 15), g.N - 1);
    const int tile = min((n0 >> 4) + ct, ((g.N + 15) >> 4) - 1);
    const int8_t* wb = g.Wf ? g.Wf + ((int64_t)tile * ksteps * 64 + lane) * 16 : g.W + (int64_t)n * g.K + kq;
    const int wstep = g.Wf ? 1024 : 64;
    // Loads from clamped (in-bounds) k-steps, zeroed afterwards: no branch
    // around a load, so every load of the prologue is in flight at once.
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      const int s = wave + NW * i;
      const v4i v = *(const v4i*)(wb + (int64_t)min(s, ksteps - 1) * wstep);
      bf[i][ct] = FULL || s < ksteps ? v : zero4();
    }
  }
  // Epilogue operands (each thread always handles the same column) and the
  // row multipliers are requested with the weights, so that they arrive in
  // the same memory round trip.
  const int ec = tid % COLS;
  const int en = min(n0 + ec, g.N - 1);
  const float ewm = g.wmult[en], ebias = g.bias[en];
  float am[ROWS_PER_THREAD];
  int64_t crow[MODE == EPI_QKV_CACHE ? ROWS_PER_THREAD : 1];
#pragma unroll
  for (int k = 0; k < ROWS_PER_THREAD; ++k) {
    const int m = min(tid / COLS + k * (NT / COLS), Mh - 1);
    if constexpr (!AX) am[k] = AF ? af_row_mult<A8>(Aamax, m, g.amax_parts) : ai[m];
    if constexpr (MODE == EPI_QKV_CACHE) crow[k] = e.row_kv0[r0 + m] + e.step;
  }
  int Md;  // the device row count, read after the activation loads are issued

  // First chunk's activation fragments.
  v4i af[KSW][4];
  bool xbad = false;  // A_F32_MAX: a non-finite value in this lane's row (row lane % 16)
  if constexpr (AF) {
    // At most 16 rows (one MFMA row tile): every k-step's fp32 values and the
    // row's maxima are requested together, then quantized.
    const int m = min(lane & 15, Mh - 1);
    const float* ar = Af + (int64_t)m * g.ldaf + kq;
    float4 raw[KSW][4];
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      const int s = min(wave + NW * i, ksteps - 1);  // past K: loaded, then unused
#pragma unroll
      for (int w = 0; w < 4; ++w) raw[i][w] = *(const float4*)(ar + s * 64 + 4 * w);
    }
    float a_m = AX ? 0.0f : af_row_mult<A8>(Aamax, m, g.amax_parts);
    asm volatile("" ::: "memory");  // the loads above are issued first
    Md = bounded_rows(g.M_dev, g.M);
    if constexpr (AX) {
      // Row |max| over all of K: this lane's 16 values per k-step, the four
      // lanes of the row (its k-offsets), then the waves through LDS.
      float mx = 0.0f;
      bool bad = false;
#pragma unroll
      for (int i = 0; i < KSW; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float4 v = raw[i][w];
          bad |= !isfinite(v.x) || !isfinite(v.y) || !isfinite(v.z) || !isfinite(v.w);
          mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      if (lane < kAfRows) sRowMax[wave * kAfRows + lane] = mx;
      xbad = bad;
      __syncthreads();
      float rm = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) rm = fmaxf(rm, sRowMax[w * kAfRows + (lane & 15)]);
      a_m = row_multiplier(rm);
    }
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      af[i][0] = FULL || wave + NW * i < ksteps ? quantize_frag16(raw[i], a_m) : zero4();
#pragma unroll
      for (int mt = 1; mt < 4; ++mt) af[i][mt] = zero4();
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int m = min(mt * 16 + (lane & 15), Mh - 1);
      const int8_t* ar = Ai + (int64_t)m * g.lda + kq;
#pragma unroll
      for (int i = 0; i < KSW; ++i) {
        const int s = wave + NW * i;
        const v4i v = *(const v4i*)(ar + min(s, ksteps - 1) * 64);
        af[i][mt] = ((FULL || s < ksteps) && mt * 16 < Mh) ? v : zero4();
      }
    }
    asm volatile("" ::: "memory");  // the loads above are issued first
    Md = bounded_rows(g.M_dev, g.M);
  }
  if constexpr (AX) {
#pragma unroll
    for (int k = 0; k < ROWS_PER_THREAD; ++k) {
      const int m = min(tid / COLS + k * (NT / COLS), Mh - 1);
      float rm = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) rm = fmaxf(rm, sRowMax[w * kAfRows + m]);
      am[k] = row_multiplier(rm);
    }
  }
  const int M = RG ? min(Md - r0, kAfRows) : Md;  // this workgroup's rows
  // Non-finite values count only in rows below the device row count, as in
  // the row quantization.
  if constexpr (AX)
    if (__any(xbad && (lane & 15) < M) && lane == 0 && g.err) *g.err = 1;

  for (int m0 = 0; m0 < M; m0 += kSkinnyRows) {
    if (!AF && m0 > 0) {  // int8 A: next 64-row chunk
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int m = min(m0 + mt * 16 + (lane & 15), M - 1);
        const int8_t* ar = Ai + (int64_t)m * g.lda + kq;
#pragma unroll
        for (int i = 0; i < KSW; ++i) {
          const int s = wave + NW * i;
          af[i][mt] = (s < ksteps && m0 + mt * 16 < M) ? *(const v4i*)(ar + s * 64) : zero4();
        }
      }
#pragma unroll
      for (int k = 0; k < ROWS_PER_THREAD; ++k) {
        const int m = min(m0 + tid / COLS + k * (NT / COLS), M - 1);
        am[k] = ai[m];
        if constexpr (MODE == EPI_QKV_CACHE) crow[k] = e.row_kv0[r0 + m] + e.step;
      }
    }
    for (int i = tid; i < kSkinnyRows * LDC; i += NT) sAcc[i] = 0;
    __syncthreads();
    const int mt_n = min(4, (M - m0 + 15) >> 4);  // live 16-row tiles (uniform)
    v4i acc[4][CT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[mt][ct] = zero4();
#pragma unroll
    for (int i = 0; i < KSW; ++i) {
      if (FULL || wave + NW * i < ksteps) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          if (mt < mt_n)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
              acc[mt][ct] =
                  __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i][mt], bf[i][ct], acc[mt][ct], 0, 0, 0);
      }
    }
    // Lane l holds rows 4*(l/16)+r of column l%16 of each 16x16 tile.  Rows
    // at or past M carry garbage and are never stored.
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
      if (mt < mt_n)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            atomicAdd(&sAcc[(mt * 16 + (lane >> 4) * 4 + r) * LDC + ct * 16 + (lane & 15)],
                      acc[mt][ct][r]);
    __syncthreads();

    const int n = n0 + ec;
#pragma unroll
    for (int k = 0; k < ROWS_PER_THREAD; ++k) {
      const int row = tid / COLS + k * (NT / COLS);
      const int m = m0 + row;
      if (m >= M || n >= g.N) continue;
      const int32_t iv = sAcc[row * LDC + ec];
      float y = dequant(iv, am[k], ewm, ebias);
      if (e.relu) y = y > 0.0f ? y : 0.0f;
      if (MODE == EPI_QKV_CACHE) {
        if (n < e.d) {
          out[(int64_t)m * e.ldo + n] = y;
        } else {
          if (n < 2 * e.d)
            e.kcache[crow[k] * e.d + (n - e.d)] = y;
          else
            e.vcache[crow[k] * e.d + (n - 2 * e.d)] = y;
        }
      } else {
        if (out) out[(int64_t)m * e.ldo + n] = y;
        if (e.out_i32) e.out_i32[(int64_t)m * e.ldi + n] = iv;
        if (e.out_q) {  // int8 A only (no row offset r0)
          e.out_q[(int64_t)m * e.ldq + n] = (int8_t)quantize_one(y, e.qmult);
          if (n == 0) e.out_qa[m] = e.qmult;
          if (!isfinite(y) && g.err) *g.err = 1;  // quantizing rejects non-finite input
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Vocabulary projection + bias + generation mask + argmax (the tied output
// embedding, N = vocab).  One workgroup = 4 waves = 128 columns; every wave
// owns two 16-column tiles for the whole K, so its weight fragments (all of
// them, issued at once) stay in registers across row chunks and no cross-wave
// reduction of accumulators is needed.  The activation rows are staged once
// per workgroup in LDS.  Each row's best (logit, id) key over the workgroup's
// columns is written as one partial; the step finalizer reduces the partials.
// ---------------------------------------------------------------------------
constexpr int kVocabCols = 128;                   // columns per workgroup
// Waves per workgroup: 8 of one column tile when the kernel builds the rows'
// LayerNorm (at most 4 rows: 7.8 against 9.1 µs per launch with 4 waves), 4
// of two tiles otherwise (10.1 against 10.8 µs at 5-64 rows).
template <bool LNP>
constexpr int kVocabWaves = LNP ? 8 : 4;
constexpr int kVocabMaxK = 512;                   // K held in registers
constexpr int kVocabLds = kVocabMaxK + 16;        // padded LDS row (bytes)

// FULL: K = 512, every k-step live, unconditional weight loads.  LNP: the
// rows (at most kVocabLnMaxRows = 4, K = 512) are the residual LayerNorm of
// g.pro: wave w builds row w with the one-wave speculative folds (ln_wave)
// while the weight loads are in flight (the row's loads are issued before
// the weights'), takes its maximum and quantizes it into the LDS row the
// matrix cores read.
// FAST (with LNP): the LayerNorm sums in the fast-reduction tree order.
template <bool FULL, bool LNP, bool FAST = false>
__global__ __launch_bounds__(64 * kVocabWaves<LNP>) void k_vocab_argmax(GemmArgs g, Epilogue e) {
  touch_kernargs<sizeof(GemmArgs) + sizeof(Epilogue)>();
  constexpr int kVocabThreads = 64 * kVocabWaves<LNP>;
  constexpr int kVocabCT = kVocabCols / (16 * kVocabWaves<LNP>);  // column tiles per wave
  constexpr int KEYS = kVocabWaves<LNP> * 16;  // per row: one key per (wave, lane column)
  static_assert(kVocabCT * 16 * kVocabWaves<LNP> == kVocabCols, "whole tiles per wave");
  static_assert(!LNP || (kVocabLnMaxRows <= kVocabWaves<LNP> && kVocabLnMaxRows <= 4), "a wave per prologue row");
  constexpr int PER = kVocabMaxK / 64;  // prologue rows: lane l holds elements l + 64j
  __shared__ __attribute__((aligned(16))) int8_t sA[kSkinnyRows * kVocabLds];
  __shared__ uint64_t sK[kSkinnyRows * (KEYS + 1)];
  __shared__ float sAm[kSkinnyRows];
  __shared__ __attribute__((aligned(16))) float sZ[LNP ? 4 * kLnRow<PER> : 4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kq = (lane >> 4) * 16;
  const int ksteps = g.K >> 6;
  const int nbase = blockIdx.x * kVocabCols + wave * 16 * kVocabCT;

  // LayerNorm prologue: this wave's row (rows below the host bound are
  // allocated), requested before the weights.
  float wy[LNP ? PER : 1], wr[LNP ? PER : 1], wgm[LNP ? PER : 1], wbt[LNP ? PER : 1];
  if constexpr (LNP) {
    const int64_t ro = (int64_t)min(wave, g.M - 1) * kVocabMaxK;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c = lane + 64 * j;
      wy[j] = g.pro.y[ro + c];
      wr[j] = g.pro.r[ro + c];
      wgm[j] = g.pro.gamma[c];
      wbt[j] = g.pro.beta[c];
    }
  }

  // Weight fragments for the wave's columns over all of K, issued first.
  v4i bf[kVocabCT][kVocabMaxK / 64];
  int ncol[kVocabCT];
#pragma unroll
  for (int ct = 0; ct < kVocabCT; ++ct) {
    ncol[ct] = nbase + ct * 16 + (lane & 15);
    const int tile = min((nbase >> 4) + ct, ((g.N + 15) >> 4) - 1);
    const int8_t* wb = g.Wf ? g.Wf + ((int64_t)tile * ksteps * 64 + lane) * 16
                            : g.W + (int64_t)min(ncol[ct], g.N - 1) * g.K + kq;
    const int wstep = g.Wf ? 1024 : 64;  // fragment order: 1 KB per k-step
#pragma unroll
    for (int s = 0; s < kVocabMaxK / 64; ++s) {
      const v4i v = *(const v4i*)(wb + (int64_t)min(s, ksteps - 1) * wstep);
      bf[ct][s] = FULL || s < ksteps ? v : zero4();
    }
  }
  // Epilogue operands of this lane's columns.
  float wm[kVocabCT], bi[kVocabCT];
  bool live[kVocabCT];
#pragma unroll
  for (int ct = 0; ct < kVocabCT; ++ct) {
    const int n = min(ncol[ct], g.N - 1);
    wm[ct] = g.wmult[n];
    bi[ct] = g.bias[n];
    live[ct] = ncol[ct] < g.N && ((e.flags & 2u) || !generation_masked((uint32_t)ncol[ct]));
  }
  // Activation rows of a 64-row chunk: thread t holds 16-byte pieces
  // t + kVocabThreads j (row = piece / 32, piece % 32 < K / 16), all
  // requested at once.
  // The first chunk is requested for the rows below the host bound g.M (all
  // allocated) before the device row count arrives.
  // Above 64 rows each 64-row group is a row of workgroups (blockIdx.y), so
  // the groups run side by side; every group reads the weights again (from
  // the caches: the vocabulary is 16 MB).
  constexpr int kStage = kSkinnyRows * (kVocabMaxK / 16) / kVocabThreads;
  const int r0 = (int)blockIdx.y * kSkinnyRows;  // this workgroup's first row
  const int cpr = g.K >> 4;
  v4i st[kStage];
  float sa = 0.0f;
  const int rows_h = min(kSkinnyRows, g.M - r0);
  if constexpr (!LNP) {
#pragma unroll
    for (int j = 0; j < kStage; ++j) {
      const int c = tid + kVocabThreads * j, row = c >> 5, cc = c & 31;
      st[j] = (row < rows_h && cc < cpr) ? *(const v4i*)(g.A + (int64_t)(r0 + row) * g.lda + cc * 16)
                                         : zero4();
    }
    if (tid < rows_h) sa = g.a[r0 + tid];
  }
  const int M = min(g.M_dev ? min(*g.M_dev, g.M) : g.M, r0 + kSkinnyRows);  // rows below this group's end
  if constexpr (LNP) {
    // normalize_row (tensor.rs:372-385), one wave per row.
    if (wave < g.M) {
      float z[PER], o[PER];
#pragma unroll
      for (int j = 0; j < PER; ++j) z[j] = wy[j] + wr[j];  // add_slices
      ln_wave<PER, FAST>(z, sZ + wave * kLnRow<PER>, wgm, wbt, lane, o);
      float mx = 0.0f;
      bool bad = false;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        bad |= !isfinite(o[j]);
        mx = fmaxf(mx, fabsf(o[j]));
      }
      const float a_row = row_multiplier(wave_max(mx));
#pragma unroll
      for (int j = 0; j < PER; ++j) sA[wave * kVocabLds + lane + 64 * j] = (int8_t)quantize_one(o[j], a_row);
      if (lane == 0) sAm[wave] = a_row;
      if (__any(bad) && lane == 0 && wave < M && g.pro.err) *g.pro.err = 1;
    }
  }

  for (int m0 = r0; m0 < M; m0 += kSkinnyRows) {
    const int rows = min(kSkinnyRows, M - m0);
    if constexpr (!LNP) {
#pragma unroll
      for (int j = 0; j < kStage; ++j) {
        const int c = tid + kVocabThreads * j;
        *(v4i*)(sA + (c >> 5) * kVocabLds + (c & 31) * 16) = st[j];
      }
      if (tid < kSkinnyRows) sAm[tid] = sa;
      // The next chunk's rows are requested now, from clamped (allocated)
      // rows with the pieces past the chunk masked, so they arrive while this
      // chunk is multiplied instead of after it.
      const int m1 = m0 + kSkinnyRows, rows1 = M - m1;
#pragma unroll
      for (int j = 0; j < kStage; ++j) {
        const int c = tid + kVocabThreads * j, row = c >> 5, cc = c & 31;
        st[j] = keep_or_zero(*(const v4i*)(g.A + (int64_t)min(m1 + row, M - 1) * g.lda + min(cc, cpr - 1) * 16),
                             row < rows1 && cc < cpr);
      }
      sa = g.a[min(m1 + tid, M - 1)];  // read only for rows of the chunk
    }
    __syncthreads();
    const int mt_n = (rows + 15) >> 4;
    v4i acc[4][kVocabCT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int ct = 0; ct < kVocabCT; ++ct) acc[mt][ct] = zero4();
    if (FULL && mt_n == 1) {
      // One row tile (the common decode case): every k-step's A fragment is
      // read at once, then the matrix cores run four independent chains
      // (two column tiles x even / odd k-steps; exact integer sums).
      constexpr int S = kVocabMaxK / 64;
      v4i a1[S];
#pragma unroll
      for (int s = 0; s < S; ++s) a1[s] = *(const v4i*)(sA + (lane & 15) * kVocabLds + kq + s * 64);
      v4i acc2[kVocabCT];
#pragma unroll
      for (int ct = 0; ct < kVocabCT; ++ct) acc2[ct] = zero4();
#pragma unroll
      for (int s = 0; s < S; s += 2)
#pragma unroll
        for (int ct = 0; ct < kVocabCT; ++ct) {
          acc[0][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[s], bf[ct][s], acc[0][ct], 0, 0, 0);
          acc2[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[s + 1], bf[ct][s + 1], acc2[ct], 0, 0, 0);
        }
#pragma unroll
      for (int ct = 0; ct < kVocabCT; ++ct) acc[0][ct] += acc2[ct];
    } else {
      // All live row tiles advance together over K: up to 4 x kVocabCT
      // independent accumulation chains keep the matrix core busy.
#pragma unroll
      for (int s = 0; s < kVocabMaxK / 64; ++s) {
        if (FULL || s < ksteps) {
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            if (mt < mt_n) {
              const v4i af = *(const v4i*)(sA + (mt * 16 + (lane & 15)) * kVocabLds + kq + s * 64);
#pragma unroll
              for (int ct = 0; ct < kVocabCT; ++ct)
                acc[mt][ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[ct][s], acc[mt][ct], 0, 0, 0);
            }
          }
        }
      }
    }
    // Lane holds rows 4*(lane/16)+r of each tile and column lane%16 of each of
    // its column tiles: dequantize in registers, keep the best of its columns
    // per row, and park it in LDS.
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (mt < mt_n) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int lr = mt * 16 + (lane >> 4) * 4 + r;
          uint64_t key = 0;
          if (lr < rows) {
            const int m = m0 + lr;
            const float am = sAm[lr];
#pragma unroll
            for (int ct = 0; ct < kVocabCT; ++ct) {
              const float y = dequant(acc[mt][ct][r], am, wm[ct], bi[ct]);
              if (e.logits && ncol[ct] < g.N)
                e.logits[(int64_t)m * e.ldl + ncol[ct]] = live[ct] ? y : -INFINITY;
              if (live[ct]) {
                const uint64_t k = argmax_key(y, (uint32_t)ncol[ct]);
                key = k > key ? k : key;
              }
            }
          }
          sK[lr * (KEYS + 1) + wave * 16 + (lane & 15)] = key;
        }
      }
    }
    __syncthreads();
    // P threads per row reduce its KEYS parked keys.
    {
      constexpr int P = kVocabThreads / kSkinnyRows;
      static_assert(P == 4 || P == 8, "4 or 8 threads per row");
      const int row = tid / P, part = tid % P;
      uint64_t best = 0;
      if (row < rows) {
#pragma unroll
        for (int j = 0; j < KEYS / P; ++j) {
          const uint64_t k = sK[row * (KEYS + 1) + part * (KEYS / P) + j];
          best = k > best ? k : best;
        }
      }
      best = umax64(best, xor_lane_u64<1>(best));
      best = umax64(best, xor_lane_u64<2>(best));
      if constexpr (P == 8) best = umax64(best, xor_lane_u64<4>(best));
      if (row < rows && part == 0)
        e.partials[(int64_t)(m0 + row) * e.partial_ld + blockIdx.x] = best;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Tile GEMM: 64x64 output tile per workgroup, 4 waves in a 2x2 grid each
// owning 32x32 (2x2 MFMA tiles).  K is staged through LDS in chunks of up to
// 512: the whole chunk of both operands is requested at once (64 KB per
// workgroup in flight), and the next chunk's loads are in flight while the
// MFMAs consume the current one, so a K of 512 costs one memory round trip
// instead of one per 64-wide k-step.  The epilogue dequantizes into LDS and
// stores whole 256-byte row segments.
//
// Tile order: the grid is one-dimensional and workgroups reach the 8 XCDs
// round-robin, so the linear id is remapped to give each XCD a contiguous
// range of tiles, with the column tile varying fastest.  The workgroups in
// flight on one XCD then share their activation rows (in its L2) and write
// adjacent 256-byte pieces of the same output rows: the output is most of
// the traffic, and the row tile varying fastest (writes spread over many
// rows at once) measured 15% slower on 4096 x 32000.  Grids more than
// kTileWideN column tiles wide take the column tiles in groups of
// kTileGroup row tiles (row tile fastest within a group), so a weight tile
// is fetched into an XCD's L2 once for eight row tiles instead of once per
// row tile (4096 x 32000: 360 -> 344 us with both outputs, 272 -> 253 us
// with the fp32 one; the narrow encoder shapes keep their weights in L2
// either way and were within noise).
// The output rows are written with non-temporal stores (they are not read
// again by this kernel): 3-14% faster from M = 1400 to 7400 on the encoder
// and op-level shapes.
// ---------------------------------------------------------------------------
constexpr int kTm = 64;         // tile edge (rows and columns)
constexpr int64_t kTileBigGrid = 256;  // tiles above which K chunks are 256 wide
constexpr int kTout = kTm + 4;  // padded LDS row of the epilogue (words)
constexpr int kTileWideN = 64;  // column tiles above which tiles go in row groups
constexpr int kTileGroup = 8;   // row tiles per group

template <int KC>  // K chunk staged in LDS: 512 (one round trip for K = 512) or 256
__global__ __launch_bounds__(256) void k_gemm_tile(GemmArgs g, Epilogue e, int tiles_n, int tiles) {
  constexpr int LDS_ROW = KC + 16;                // padded LDS row (bytes)
  constexpr int ROW_CH = KC / 16;                 // 16-byte pieces per row
  constexpr int CH = kTm * ROW_CH / 256;          // 16-byte loads per thread per operand
  static_assert(kTm * LDS_ROW >= kTm * kTout * 4, "the epilogue reuses the operand tiles");
  __shared__ __attribute__((aligned(16))) int8_t sA[kTm * LDS_ROW];
  __shared__ __attribute__((aligned(16))) int8_t sB[kTm * LDS_ROW];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  int tile = blockIdx.x;
  const int full = tiles & ~7;
  if (tile < full) tile = (tile & 7) * (full >> 3) + (tile >> 3);
  const int M = g.M, N = g.N, K = g.K;
  int m0 = tile / tiles_n * kTm, n0 = tile % tiles_n * kTm;
  if (tiles_n > kTileWideN) {  // a permutation of the tiles: groups of up to kTileGroup row tiles
    const int tiles_m = (M + kTm - 1) / kTm;
    const int grp = tile / (kTileGroup * tiles_n), first_m = grp * kTileGroup;
    const int gm = min(kTileGroup, tiles_m - first_m), in_g = tile - grp * kTileGroup * tiles_n;
    m0 = (first_m + in_g % gm) * kTm;
    n0 = in_g / gm * kTm;
  }

  // Every load is issued (from an in-bounds address); pieces past M, N or
  // the chunk's K are zeroed when they are stored to LDS.
  v4i ra[CH], rb[CH];
  bool ka[CH], kb[CH];
  auto gload = [&](int k0, int kc) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * 256, row = c / ROW_CH, col = c % ROW_CH * 16;
      const int m = m0 + row, n = n0 + row;
      const int cl = min(col, kc - 16);
      ra[i] = *(const v4i*)(g.A + (int64_t)min(m, M - 1) * g.lda + k0 + cl);
      rb[i] = *(const v4i*)(g.W + (int64_t)min(n, N - 1) * K + k0 + cl);
      ka[i] = col < kc && m < M;
      kb[i] = col < kc && n < N;
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * 256, row = c / ROW_CH, col = c % ROW_CH * 16;
      *(v4i*)(sA + row * LDS_ROW + col) = keep_or_zero(ra[i], ka[i]);
      *(v4i*)(sB + row * LDS_ROW + col) = keep_or_zero(rb[i], kb[i]);
    }
  };

  v4i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero4();

  const int kq = (lane >> 4) * 16;
  const int8_t* pa = sA + (wm * 32 + (lane & 15)) * LDS_ROW + kq;
  const int8_t* pb = sB + (wn * 32 + (lane & 15)) * LDS_ROW + kq;
  gload(0, min(KC, K));
  lstore();
  __syncthreads();
  for (int k0 = 0; k0 < K; k0 += KC) {
    const int ksteps = min(KC, K - k0) >> 6;
    const bool more = k0 + KC < K;
    if (more) gload(k0 + KC, min(KC, K - k0 - KC));
#pragma unroll
    for (int ks = 0; ks < KC / 64; ++ks) {
      if (ks < ksteps) {
        const v4i a0 = *(const v4i*)(pa + ks * 64);
        const v4i a1 = *(const v4i*)(pa + 16 * LDS_ROW + ks * 64);
        const v4i b0 = *(const v4i*)(pb + ks * 64);
        const v4i b1 = *(const v4i*)(pb + 16 * LDS_ROW + ks * 64);
        acc[0][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b1, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b0, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc[1][1], 0, 0, 0);
      }
    }
    if (more) {
      __syncthreads();
      lstore();
      __syncthreads();
    }
  }

  // Epilogue: element (m, n) of the MFMA tile (i, j) is register r of lane
  // (m % 16 / 4) * 16 + n % 16 with r = m % 4.
  float arow[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm * 32 + i * 16 + (lane >> 4) * 4 + r;
      arow[i][r] = m < M ? g.a[m] : 1.0f;
    }
  float* sO = (float*)sA;      // [kTm][kTout] dequantized
  int32_t* sI = (int32_t*)sB;  // [kTm][kTout] accumulators
  __syncthreads();             // the MFMAs' last LDS reads are done
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int nl = wn * 32 + j * 16 + (lane & 15), n = n0 + nl;
    const float wmul = n < N ? g.wmult[n] : 1.0f, bias = n < N ? g.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ml = wm * 32 + i * 16 + (lane >> 4) * 4 + r;
        const int32_t iv = acc[i][j][r];
        float y = dequant(iv, arow[i][r], wmul, bias);
        if (e.relu) y = y > 0.0f ? y : 0.0f;
        sO[ml * kTout + nl] = y;
        sI[ml * kTout + nl] = iv;
      }
  }
  __syncthreads();
  const bool vec_o = e.out && (e.ldo & 3) == 0 && ((uintptr_t)e.out & 15) == 0;
  const bool vec_i = e.out_i32 && (e.ldi & 3) == 0 && ((uintptr_t)e.out_i32 & 15) == 0;
#pragma unroll
  for (int q = 0; q < kTm * kTm / 4 / 256; ++q) {
    const int idx = tid + q * 256, row = idx >> 4, c4 = (idx & 15) * 4;
    const int m = m0 + row, n = n0 + c4;
    if (m >= M || n >= N) continue;
    const float* so = sO + row * kTout + c4;
    const int32_t* si = sI + row * kTout + c4;
    if (e.out) {
      float* o = e.out + (int64_t)m * e.ldo + n;
      if (vec_o && n + 4 <= N) {
        __builtin_nontemporal_store(*(const f4v*)so, (f4v*)o);
      } else {
        for (int t = 0; t < 4 && n + t < N; ++t) o[t] = so[t];
      }
    }
    if (e.out_i32) {
      int32_t* o = e.out_i32 + (int64_t)m * e.ldi + n;
      if (vec_i && n + 4 <= N) {
        __builtin_nontemporal_store(*(const v4i*)si, (v4i*)o);
      } else {
        for (int t = 0; t < 4 && n + t < N; ++t) o[t] = si[t];
      }
    }
    if (e.out_q) {
      int8_t* o = e.out_q + (int64_t)m * e.ldq + n;
      bool bad = false;
      for (int t = 0; t < 4 && n + t < N; ++t) {
        o[t] = (int8_t)quantize_one(so[t], e.qmult);
        bad |= !isfinite(so[t]);
      }
      if (n == 0) e.out_qa[m] = e.qmult;
      if (bad && g.err) *g.err = 1;  // quantizing rejects non-finite input
    }
  }
}

// ---------------------------------------------------------------------------
// Output scoring over a candidate list (the lexical shortlist's ids, sorted
// ascending): select_token (q8_engine.rs:749-790) for row m scores only
// cand[off[m] .. off[m+1]).  One workgroup per (row, 128 candidates): each of
// its 4 waves gathers the embedding rows of two 16-candidate tiles (lane l
// loads 16 bytes of row cand[16t + l % 16] per 64-wide k-step) and runs them
// against the row's quantized state on the matrix cores (every row of the A
// tile is the state, so output row 0 is the dot products).  Keys (logit,
// inverted id) give the first maximum in candidate order, as the strict '>'
// scan does; one key per workgroup goes to partials[m * nparts + chunk]
// (0 from the workgroups past a shorter list, which exit at once).
// ---------------------------------------------------------------------------
constexpr int kCandChunk = 128;
constexpr int kCandKs = 8;  // k-steps requested together (K <= 512: all of them)
// LNP > 0: the row is LayerNorm(pro.y + pro.r) of width 64 LNP, built by wave
// 0 while the candidates' embedding rows are in flight, and quantized with
// c.qmult (> 0, static) or its own multiplier.
// FAST (with LNP): the LayerNorm sums in the fast-reduction tree order.
template <int LNP, bool FAST = false>
__global__ __launch_bounds__(256) void k_cand_argmax(CandArgs c) {
  __shared__ uint64_t sKey[4];
  __shared__ __attribute__((aligned(16))) float sZ[LNP ? kLnRow<LNP> : 1];
  __shared__ __attribute__((aligned(16))) int8_t sX[LNP ? 64 * LNP : 16];
  __shared__ float sA;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = blockIdx.y, chunk = blockIdx.x;
  const int ksteps = c.K >> 6, kq = (lane >> 4) * 16;
  // The first k-steps are requested before the device row count is known
  // (rows below the host bound are backed by memory; a finished row's list is
  // another sequence's, still in bounds), all of them at once.
  float ly[LNP ? LNP : 1], lr[LNP ? LNP : 1], lg[LNP ? LNP : 1], lb[LNP ? LNP : 1];
  if constexpr (LNP > 0) {
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < LNP; ++j) {
        const int e = lane + 64 * j;
        ly[j] = c.pro.y[(int64_t)m * c.K + e];
        lr[j] = c.pro.r[(int64_t)m * c.K + e];
        lg[j] = c.pro.gamma[e];
        lb[j] = c.pro.beta[e];
      }
    }
  }
  const int b = c.row_slot ? c.row_slot[m] : m;
  const int64_t c0 = c.off[b], n = (int64_t)c.off[b + 1] - c0;
  if ((int64_t)chunk * kCandChunk >= n) {  // past the row's list (the grid fits the longest)
    if (tid == 0 && !(c.rows_dev && m >= *c.rows_dev)) c.partials[(int64_t)m * c.nparts + chunk] = 0;
    return;
  }
  const int8_t* xr = LNP ? nullptr : c.xq + (int64_t)m * c.K + kq;
  float am = LNP ? 0.0f : c.xa[m];
  bool live[2], bad = false;
  uint32_t id[2];
  const int8_t* er[2];
  float wm[2], wb[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t i = (int64_t)chunk * kCandChunk + wave * 32 + t * 16 + (lane & 15);
    live[t] = i < n;
    id[t] = live[t] ? c.cand[c0 + i] : 0u;
    if (id[t] >= (uint32_t)c.V) {  // not a vocabulary id: reported, never scored
      bad = true;
      live[t] = false;
      id[t] = 0u;
    }
    er[t] = c.emb + (int64_t)id[t] * c.K + kq;
    wm[t] = c.mult[id[t]];
    wb[t] = c.bias[id[t]];
  }
  v4i xa[kCandKs], bw[2][kCandKs];
  auto load = [&](int s0) {
#pragma unroll
    for (int s = 0; s < kCandKs; ++s) {
      const int64_t o = 64 * min(s0 + s, ksteps - 1);
      if (!LNP) xa[s] = *(const v4i*)(xr + o);
      bw[0][s] = *(const v4i*)(er[0] + o);
      bw[1][s] = *(const v4i*)(er[1] + o);
    }
  };
  load(0);
  if (c.rows_dev && m >= *c.rows_dev) return;  // uniform per workgroup
  if constexpr (LNP > 0) {
    if (wave == 0) {
      float z[LNP], o[LNP];
#pragma unroll
      for (int j = 0; j < LNP; ++j) z[j] = ly[j] + lr[j];
      ln_wave<LNP, FAST>(z, sZ, lg, lb, lane, o);
      float mx = 0.0f;
      bool nf = false;
#pragma unroll
      for (int j = 0; j < LNP; ++j) {
        nf |= !isfinite(o[j]);
        mx = fmaxf(mx, fabsf(o[j]));
      }
      const float sc = c.qmult > 0.0f ? c.qmult : row_multiplier(wave_max(mx));
#pragma unroll
      for (int j = 0; j < LNP; ++j) sX[lane + 64 * j] = (int8_t)quantize_one(o[j], sc);
      if (lane == 0) sA = sc;
      if (__any(nf) && lane == 0 && c.err) *c.err = 1;
    }
    wg_lds_barrier();
    am = sA;
#pragma unroll
    for (int s = 0; s < kCandKs; ++s) xa[s] = *(const v4i*)(sX + 64 * min(s, ksteps - 1) + kq);
  }
  v4i acc[2] = {zero4(), zero4()};
  for (int s0 = 0; s0 < ksteps; s0 += kCandKs) {
    if (s0 > 0) load(s0);
#pragma unroll
    for (int s = 0; s < kCandKs; ++s)
      if (s0 + s < ksteps) {  // uniform
        acc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[s], bw[0][s], acc[0], 0, 0, 0);
        acc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[s], bw[1][s], acc[1], 0, 0, 0);
      }
  }
  uint64_t best = 0;
  // Lanes 0-15 hold row 0 (register 0) for candidates 16t + lane.
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (lane < 16 && live[t]) {
      const float y = dequant(acc[t][0], am, wm[t], wb[t]);
      if (c.logits) c.logits[c0 + chunk * kCandChunk + wave * 32 + t * 16 + lane] = y;
      const uint64_t k = argmax_key(y, id[t]);
      best = k > best ? k : best;
    }
  }
  if (__any(bad) && lane == 0 && c.err) *c.err = 1;
  best = wave_max_u64(best);
  if (lane == 0) sKey[wave] = best;
  __syncthreads();
  if (tid == 0)
    c.partials[(int64_t)m * c.nparts + chunk] = umax64(umax64(sKey[0], sKey[1]), umax64(sKey[2], sKey[3]));
}

}  // namespace

hipError_t launch_cand_argmax(const CandArgs& c, hipStream_t s) {
  if (c.M <= 0) return hipSuccess;
  if (c.K <= 0 || c.K % 64 || c.V <= 0 || c.max_cands <= 0 || c.M > 65535 || !c.partials)
    return hipErrorInvalidValue;
  const int chunks = cand_groups(c.max_cands);
  if (c.nparts < chunks) return hipErrorInvalidValue;
  const dim3 grid(chunks, c.M), block(256);
  if (c.pro.kind == PRO_LN) {
    if (!cand_ln_supported(c.K) || !c.pro.y || !c.pro.r || !c.pro.gamma || !c.pro.beta ||
        !(c.qmult >= 0.0f) || !(c.qmult < __builtin_huge_valf()))
      return hipErrorInvalidValue;
    const bool f = c.pro.fast;
    if (c.K == 256)
      hipLaunchKernelGGL((f ? k_cand_argmax<4, true> : k_cand_argmax<4>), grid, block, 0, s, c);
    else if (c.K == 384)
      hipLaunchKernelGGL((f ? k_cand_argmax<6, true> : k_cand_argmax<6>), grid, block, 0, s, c);
    else
      hipLaunchKernelGGL((f ? k_cand_argmax<8, true> : k_cand_argmax<8>), grid, block, 0, s, c);
  } else {
    if (!c.xq || !c.xa) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cand_argmax<0>, grid, block, 0, s, c);
  }
  return hipGetLastError();
}
int cand_groups(int max_cands) { return (max_cands + kCandChunk - 1) / kCandChunk; }
bool cand_ln_supported(int K) { return K == 256 || K == 384 || K == 512; }

// Columns per skinny workgroup: wide enough that the vocabulary projection
// does not re-read the activations too often, narrow enough that the small
// decode GEMMs still spread over many CUs.
int skinny_cols(int N) { return N >= 8192 ? 64 : (N >= 1024 ? 32 : 16); }
int skinny_groups(int N) { return (N + skinny_cols(N) - 1) / skinny_cols(N); }
int argmax_groups(int N, int /*K*/) { return (N + kVocabCols - 1) / kVocabCols; }
bool vocab_ln_supported(int K) { return K == kVocabMaxK; }

template <int MODE, int NW, int KSW, int ASRC, bool FULL>
static hipError_t launch_skinny_kf(const GemmArgs& g, const Epilogue& e, hipStream_t s) {
  const dim3 grid(skinny_groups(g.N), ASRC != A_I8 ? (g.M + kAfRows - 1) / kAfRows : 1), block(NW * 64);
  switch (skinny_cols(g.N)) {
    case 64: hipLaunchKernelGGL((k_gemm_skinny<MODE, 4, NW, KSW, ASRC, FULL>), grid, block, 0, s, g, e); break;
    case 32: hipLaunchKernelGGL((k_gemm_skinny<MODE, 2, NW, KSW, ASRC, FULL>), grid, block, 0, s, g, e); break;
    default: hipLaunchKernelGGL((k_gemm_skinny<MODE, 1, NW, KSW, ASRC, FULL>), grid, block, 0, s, g, e); break;
  }
  return hipGetLastError();
}
template <int MODE, int NW, int KSW, int ASRC>
static hipError_t launch_skinny_k(const GemmArgs& g, const Epilogue& e, hipStream_t s) {
  return (g.K >> 6) == NW * KSW ? launch_skinny_kf<MODE, NW, KSW, ASRC, true>(g, e, s)
                                : launch_skinny_kf<MODE, NW, KSW, ASRC, false>(g, e, s);
}

// Waves and per-wave k-steps by K: long K (the FFN down-projection) spreads
// over 8 waves; each wave holds its k-steps' fragments in registers.  An
// fp32 A source is supported for K <= 512 (the attention-output projections),
// one k-step per wave over 8 waves (3% faster per launch than 4 waves of two
// at K = 512, measured; 2 and 1 waves are 3-7% slower end to end).
template <int MODE>
static hipError_t launch_skinny_mode(const GemmArgs& g, const Epilogue& e, hipStream_t s) {
  const int ksteps = g.K >> 6;
  if (g.Af && !g.Aamax) {  // row maxima found here: the FFN down-projection (K <= 2048)
    if (MODE != EPI_STORE || ksteps > 32 || g.ldaf % 4 || e.out_i32 || g.M > 65535 * kAfRows)
      return hipErrorInvalidValue;
    return launch_skinny_k<MODE, 16, 2, A_F32_MAX>(g, e, s);
  }
  if (g.Af) {
    if (MODE != EPI_STORE || ksteps > 8 || !g.Aamax || g.amax_parts < 1 || g.amax_parts > kAfMaxParts ||
        g.ldaf % 4 || e.out_i32 ||
        g.M > 65535 * kAfRows)
      return hipErrorInvalidValue;
    return g.amax_parts == kAfParts ? launch_skinny_k<MODE, 8, 1, A_F32>(g, e, s)
                                    : launch_skinny_k<MODE, 8, 1, A_F32_P>(g, e, s);
  }
  // Above 16 rows, K <= 512 takes one 16-row group per workgroup (the groups
  // run side by side instead of one workgroup walking its rows in 64-row
  // chunks, each waiting for its own activation loads); the QKV cache
  // epilogue indexes its cache rows by the group's absolute rows.
  const bool rg8 = !e.out_i32 && !e.out_q && g.M > kAfRows && g.M <= 65535 * kAfRows;
  if (ksteps <= 4)
    return rg8 ? launch_skinny_k<MODE, 4, 1, A_I8_RG>(g, e, s) : launch_skinny_k<MODE, 4, 1, A_I8>(g, e, s);
  if (ksteps <= 8)
    return rg8 ? launch_skinny_k<MODE, 4, 2, A_I8_RG>(g, e, s) : launch_skinny_k<MODE, 4, 2, A_I8>(g, e, s);
  if (ksteps <= 16) return launch_skinny_k<MODE, 4, 4, A_I8>(g, e, s);
  // K = 1536 (the FFN down-projection of a 1536-wide FFN): 16 waves of two
  // k-steps beat 8 of four (measured); K = 2048 the other way round.  Above
  // 16 rows, plain stores take one 16-row group per workgroup: a 64-row
  // chunk of these K is 96-128 KB of activations per workgroup.
  const bool rg = MODE == EPI_STORE && !e.out_i32 && !e.out_q && g.M > kAfRows && g.M <= 65535 * kAfRows;
  if (ksteps <= 24)
    return rg ? launch_skinny_k<MODE, 16, 2, A_I8_RG>(g, e, s) : launch_skinny_k<MODE, 16, 2, A_I8>(g, e, s);
  return rg ? launch_skinny_k<MODE, 8, 4, A_I8_RG>(g, e, s) : launch_skinny_k<MODE, 8, 4, A_I8>(g, e, s);
}

hipError_t launch_gemm_skinny(const GemmArgs& g, int mode, const Epilogue& e, hipStream_t s) {
  if (g.K <= 0 || g.K % 64 || g.K > kSkinnyMaxK || g.N <= 0 || g.M <= 0) return hipErrorInvalidValue;
  if (e.out_q && (mode != EPI_STORE || g.Af || !e.out_qa || e.ldq < g.N || !(e.qmult > 0.0f) ||
                  !(e.qmult < __builtin_huge_valf())))
    return hipErrorInvalidValue;
  switch (mode) {
    case EPI_STORE: return launch_skinny_mode<EPI_STORE>(g, e, s);
    case EPI_QKV_CACHE: return launch_skinny_mode<EPI_QKV_CACHE>(g, e, s);
    case EPI_ARGMAX:
      return launch_vocab_argmax(g, e, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_vocab_argmax(const GemmArgs& g, const Epilogue& e, hipStream_t s,
                               hipEvent_t ev_start, hipEvent_t ev_stop) {
  if (g.K <= 0 || g.K % 64 || g.K > kVocabMaxK || g.N <= 0) return hipErrorInvalidValue;
  const RowPrologue& p = g.pro;
  const dim3 grid((g.N + kVocabCols - 1) / kVocabCols,
                  p.kind == PRO_LN ? 1 : max(1, (g.M + kSkinnyRows - 1) / kSkinnyRows)),
      block(64 * (p.kind == PRO_LN ? kVocabWaves<true> : kVocabWaves<false>));
  if (p.kind != PRO_NONE &&
      (p.kind != PRO_LN || g.K != kVocabMaxK || g.M > kVocabLnMaxRows || !p.y || !p.r || !p.gamma || !p.beta))
    return hipErrorInvalidValue;
  auto kern = p.kind == PRO_LN      ? (p.fast ? k_vocab_argmax<true, true, true> : k_vocab_argmax<true, true>)
              : g.K == kVocabMaxK ? k_vocab_argmax<true, false>
                                  : k_vocab_argmax<false, false>;
  if (ev_start || ev_stop)
    hipExtLaunchKernelGGL(kern, grid, block, 0, s, ev_start, ev_stop, 0, g, e);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, s, g, e);
  return hipGetLastError();
}

hipError_t launch_gemm_tile(const GemmArgs& g, const Epilogue& e, hipStream_t s) {
  if (g.K <= 0 || g.K % 64 || g.N <= 0 || g.M_dev || g.lda % 16) return hipErrorInvalidValue;
  if (e.out_q && (!e.out_qa || e.ldq < g.N || !(e.qmult > 0.0f) || !(e.qmult < __builtin_huge_valf())))
    return hipErrorInvalidValue;
  if (g.M <= 0) return hipSuccess;
  const int64_t tiles = (int64_t)((g.M + kTm - 1) / kTm) * ((g.N + kTm - 1) / kTm);
  if (tiles > (int64_t)INT32_MAX) return hipErrorInvalidValue;
  const int tiles_n = (g.N + kTm - 1) / kTm;
  // Launches of more than one round of 512-wide-chunk workgroups (two per
  // CU) take the 256-wide chunks (34 KB of LDS, four workgroups per CU, more
  // loads in flight per CU: 385 vs 469 us on 4096 x 32000; the encoder's QKV
  // and FFN1 in one round instead of two); smaller ones the 512-wide chunks
  // (one round trip for K = 512).
  if (tiles > kTileBigGrid)
    hipLaunchKernelGGL(k_gemm_tile<256>, dim3((unsigned)tiles), dim3(256), 0, s, g, e, tiles_n, (int)tiles);
  else
    hipLaunchKernelGGL(k_gemm_tile<512>, dim3((unsigned)tiles), dim3(256), 0, s, g, e, tiles_n, (int)tiles);
  return hipGetLastError();
}

hipError_t launch_gemm_store(const GemmArgs& g, const Epilogue& e, hipStream_t s) {
  if (g.M_dev || (g.M <= kSkinnyRows && g.K <= kSkinnyMaxK))
    return launch_gemm_skinny(g, EPI_STORE, e, s);
  return launch_gemm_tile(g, e, s);
}

}  // namespace mh
