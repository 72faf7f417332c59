// lngemm.hip — residual LayerNorm + Q8 linear for groups of eight rows: each
// workgroup builds its rows' LayerNorms (one wave per row, the sequential
// folds of normalize_row, tensor.rs:372-385), quantizes them (a static
// activation multiplier, legacy_q8.rs:544-552, or each row's own, q8_gemm.rs:
// 569-590) and multiplies them by 128 output columns of an int8 weight on the
// matrix cores (exact i32, y = acc * (1 / (a * w)) + b, q8_gemm.rs:438-446).
// Optionally the rows' y is itself a static Q8 linear computed in the
// workgroup (the Transformer-SSRU graph's attention-output projection).
#include "device_common.h"
#include "kernels.h"

namespace mh {
namespace {

// ---------------------------------------------------------------------------
// Residual LayerNorm + Q8 linear: out = (relu of) Q8Linear(LN(y + r)) for
// kLgsRows rows and kLgsCols output columns per workgroup.  Wave w builds
// row w of the group (LayerNorm as launch_residual_ln), quantizes it into
// LDS -- with the static activation multiplier of the column block it feeds
// (xq_mult[0] below part_n, xq_mult[1] from it: the two parts of a row-block
// group with their own multipliers), or (DYN) with the row's own multiplier
// 127 / max|row| -- then runs the MFMA chain of column tile w over the
// group's rows.  Slice-0 workgroups also store the LayerNorm rows (the next
// residual).
// ---------------------------------------------------------------------------
constexpr int kLgsRows = 8;
constexpr int kLgsWaves = 8;
constexpr int kLgsCols = 16 * kLgsWaves;

// YP: y is not read but computed here, the static Q8 linear of the int8 rows
// a.ya with Wy (the attention-output projection): wave w takes its column
// tiles w, w + 8, ... over the group's rows, and the rows meet in LDS.
// FAST (DYN only): the LayerNorm sums in the fast-reduction tree order.
template <int PER, bool YP, bool DYN, bool FAST = false>
__global__ __launch_bounds__(64 * kLgsWaves) void k_ln_gemm_rows(LnGemmRowsArgs a) {
  constexpr int D = PER * 64;
  constexpr int KS = D / 64;
  constexpr int YT = YP ? D / 16 / kLgsWaves : 1;  // y tiles per wave
  __shared__ __attribute__((aligned(16))) float sZ[kLgsWaves][kLnRow<PER>];
  __shared__ __attribute__((aligned(16))) int8_t sX[kLgsRows][D];
  __shared__ __attribute__((aligned(16))) float sY[YP ? kLgsRows : 1][YP ? D : 1];
  __shared__ float sAm[kLgsRows];  // DYN: each row's multiplier
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int slices = a.N / kLgsCols;
  const int slice = blockIdx.x % slices, grp = blockIdx.x / slices;
  const int r = grp * kLgsRows + wave;  // this wave's row
  const int n0 = slice * kLgsCols;
  const float am = n0 < a.part_n ? a.xq_mult[0] : a.xq_mult[1];
  const int ar = lane & 15;  // MFMA A-operand row of this lane
  // Row loads (rows below the host bound are backed by memory).
  float yv[PER], rv[PER], gv[PER], bv[PER];
  const bool row_mem = r < a.rows;
  if (row_mem) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      if (!YP) yv[j] = a.y[(int64_t)r * D + e];
      rv[j] = a.r[(int64_t)r * D + e];
      gv[j] = a.gamma[e];
      bv[j] = a.beta[e];
    }
  }
  // YP: the group's int8 rows (A fragments) and this wave's Wy tiles.
  v4i ya[YP ? KS : 1], by[YT][YP ? KS : 1];
  float ym[YT], yb[YT];
  if constexpr (YP) {
    const int m = min(grp * kLgsRows + (ar & (kLgsRows - 1)), a.rows - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s) ya[s] = *(const v4i*)(a.ya + (int64_t)m * D + 64 * s + (lane >> 4) * 16);
#pragma unroll
    for (int i = 0; i < YT; ++i) {
      const int t = wave + kLgsWaves * i;
#pragma unroll
      for (int s = 0; s < KS; ++s) by[i][s] = frag_load(a.Wy, t, KS, s, lane);
      ym[i] = a.ymult[16 * t + ar];
      yb[i] = a.ybias[16 * t + ar];
    }
  }
  // Tile `wave` of this slice: weight fragments, dequantization operands.
  const int col = n0 + 16 * wave + (lane & 15);
  v4i bf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) bf[s] = frag_load(a.W, (n0 >> 4) + wave, KS, s, lane);
  const float wm = a.wmult[col], wb = a.bias[col];
  const int n_rows = a.rows_dev ? min(*a.rows_dev, a.rows) : a.rows;
  if (grp * kLgsRows >= n_rows) return;  // the whole workgroup alike
  const bool live = r < n_rows;
  if constexpr (YP) {
    // y rows 0..7 = the group's rows (zero past the device count); lane l
    // ends with rows 4(l/16)+i of column l%16 of each tile.
    const bool y_live = ar < kLgsRows && grp * kLgsRows + ar < n_rows;
#pragma unroll
    for (int i = 0; i < YT; ++i) {
      v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(y_live ? ya[s] : v4i{0, 0, 0, 0}, by[i][s], acc, 0, 0, 0);
      if (lane < 32) {
        const float inv = dequant_scale(a.ya_mult, ym[i]);
        const int t = wave + kLgsWaves * i;
#pragma unroll
        for (int k = 0; k < 4; ++k) sY[4 * (lane >> 4) + k][16 * t + ar] = dequant_apply(acc[k], inv, yb[i]);
      }
    }
    wg_lds_barrier();
    if (live) {
#pragma unroll
      for (int j = 0; j < PER; ++j) yv[j] = sY[wave][lane + 64 * j];
    }
  }
  if (live) {
    float z[PER], o[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) z[j] = yv[j] + rv[j];
    ln_wave<PER, FAST>(z, sZ[wave], gv, bv, lane, o);
    bool bad = false;
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      bad |= !isfinite(o[j]);
      mx = fmaxf(mx, fabsf(o[j]));
    }
    const float ar_mult = DYN ? row_multiplier(wave_max(mx)) : am;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      if (slice == 0 && a.x_out) a.x_out[(int64_t)r * D + e] = o[j];
      sX[wave][e] = (int8_t)quantize_one(o[j], ar_mult);
    }
    if (DYN && lane == 0) sAm[wave] = ar_mult;
    if (__any(bad) && lane == 0 && a.err) *a.err = 1;
  }
  wg_lds_barrier();  // LDS only: the LayerNorm row stores stay in flight
  // Rows 0..7 of the A operand are the group's rows (zero past the device
  // count), rows 8..15 zero.  Lane l ends with rows 4(l/16)+i of column l%16.
  const bool a_live = ar < kLgsRows && grp * kLgsRows + ar < n_rows;
  v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const v4i x = a_live ? *(const v4i*)(&sX[ar][64 * s + (lane >> 4) * 16]) : v4i{0, 0, 0, 0};
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x, bf[s], acc, 0, 0, 0);
  }
  if (lane >= 32) return;  // rows 8..15
  const float inv = dequant_scale(am, wm);
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rl = 4 * (lane >> 4) + i, m = grp * kLgsRows + rl;
    if (m >= n_rows) continue;
    float y = DYN ? dequant(acc[i], sAm[rl], wm, wb) : dequant_apply(acc[i], inv, wb);
    if (a.relu) y = y > 0.0f ? y : 0.0f;
    if (a.out) a.out[(int64_t)m * a.ldo + col] = y;
    if (a.out_q) {
      a.out_q[(int64_t)m * a.ldq + col] = (int8_t)quantize_one(y, a.qmult);
      if (col == 0) a.out_qa[m] = a.qmult;
      bad |= !isfinite(y);  // quantizing rejects non-finite input
    }
  }
  if (__any(bad) && lane == 0 && a.err) *a.err = 1;
}

}  // namespace

bool ln_gemm_rows_supported(int K, int N) {
  return (K == 256 || K == 384 || K == 512) && N > 0 && N % kLgsCols == 0;
}

hipError_t launch_ln_gemm_rows(const LnGemmRowsArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const bool yp = a.ya != nullptr;
  if (!ln_gemm_rows_supported(a.K, a.N) || (yp ? !(a.Wy && a.ymult && a.ybias) : !a.y) || !a.r ||
      !a.gamma || !a.beta || !a.W ||
      !a.wmult || !a.bias || (!a.out && !a.out_q) || (a.out && a.ldo < a.N) ||
      (a.out_q && (!a.out_qa || a.ldq < a.N)) || a.part_n < 0 || a.part_n % kLgsCols)
    return hipErrorInvalidValue;
  for (const float m : {a.dyn ? 1.0f : a.xq_mult[0], a.dyn ? 1.0f : a.xq_mult[1], yp ? a.ya_mult : 1.0f})
    if (!(m > 0.0f) || !(m < __builtin_huge_valf())) return hipErrorInvalidValue;
  if ((a.dyn && yp) || (a.fast && !a.dyn)) return hipErrorInvalidValue;
  if (a.out_q && (!(a.qmult > 0.0f) || !(a.qmult < __builtin_huge_valf()))) return hipErrorInvalidValue;
  const int groups = (a.rows + kLgsRows - 1) / kLgsRows;
  if ((int64_t)groups * (a.N / kLgsCols) > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid(groups * (a.N / kLgsCols)), block(64 * kLgsWaves);
#define MH_LG(P)                                                                       \
  if (a.dyn && a.fast)                                                                 \
    hipLaunchKernelGGL((k_ln_gemm_rows<P, false, true, true>), grid, block, 0, s, a);  \
  else if (a.dyn)                                                                      \
    hipLaunchKernelGGL((k_ln_gemm_rows<P, false, true>), grid, block, 0, s, a);        \
  else if (yp)                                                                         \
    hipLaunchKernelGGL((k_ln_gemm_rows<P, true, false>), grid, block, 0, s, a);  \
  else                                                                           \
    hipLaunchKernelGGL((k_ln_gemm_rows<P, false, false>), grid, block, 0, s, a);
  if (a.K == 256) {
    MH_LG(4)
  } else if (a.K == 384) {
    MH_LG(6)
  } else {
    MH_LG(8)
  }
#undef MH_LG
  return hipGetLastError();
}

}  // namespace mh
