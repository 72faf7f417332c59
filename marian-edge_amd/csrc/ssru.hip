// ssru.hip — fused decode kernels of the Transformer-SSRU graph (the
// reference's own model, static per-tensor multipliers).  With static
// multipliers a quantized row needs nothing from other rows or columns, so
// one decoder layer runs as four launches:
//   k_ssru_input      the layer input x (the previous layer's last residual
//                     LayerNorm, or the decoder input embedding), the SSRU's
//                     candidate and forget-gate projections of it and the SSRU
//                     update: state' and z = relu(state') + x;
//   k_ssru_block      per (row, head): the SSRU LayerNorm of z, the head's
//                     query projection and the cross-attention over the row's
//                     sentence, quantized for the output projection;
//   (output projection: the skinny GEMM)
//   k_ln_gemm_rows    (lngemm.hip) the output projection, the context
//                     block's residual LayerNorm and the FFN up-projection;
//   (FFN down-projection: the skinny GEMM).
//
// Every value is produced by the same operations, in the same order, as the
// separate kernels (and the reference):
//   SSRU update       ssru_update_layer_norm_into, tensor.rs:184-218
//   LayerNorm         normalize_row, tensor.rs:372-385 (sequential folds)
//   embedding         (q / mult) * sqrt(d) + pos (q8_engine.rs:586-630)
//   quantization      quantize_static_into (legacy_q8.rs:544-552): q =
//                     clamp(rne(x * act_mult), -127, 127)
//   projection        exact i32 MFMA, y = acc * (1 / (act * w)) + b
//                     (legacy_q8.rs:646-674)
//   attention         attention_into, tensor.rs:251-318 (sequential dot from
//                     -0.0, max, C-library expf, sequential sum from 0.0, PV in
//                     key order from 0.0)
#include "device_common.h"
#include "kernels.h"

namespace mh {
namespace {

constexpr int kSbThreads = 256;
constexpr int kSbLoaders = kSbThreads - 64;  // waves 1-3 stage keys and values

__constant__ uint64_t kSbExp2Tab[32] = {MH_EXP2_TABLE_32};

// ---------------------------------------------------------------------------
// SSRU LayerNorm + query projection + cross-attention, one 256-thread
// workgroup per (row, head).  Wave 0 loads z and normalizes it; waves 1-3
// stage the head's key and value rows in LDS; wave t < head_dim / 16
// projects one 16-column query tile; wave 0 then attends alone (the
// dependent chains are per row).
// ---------------------------------------------------------------------------
template <int PER, int DH>
__global__ __launch_bounds__(kSbThreads) void k_ssru_block(SsruBlockArgs a) {
  constexpr int D = PER * 64;
  constexpr int T = DH / 16;  // query tiles of one head
  constexpr int KS = D / 64;  // k-steps of the projection
  constexpr int KR = DH + 4;  // padded LDS key row (floats), 16-byte aligned
  constexpr int V4 = DH / 4;  // float4 per key row of one head
  constexpr int NL = (kSsruBlockMaxKeys * V4 + kSbLoaders - 1) / kSbLoaders;
  static_assert(T <= 4 && DH % 16 == 0, "one query tile per wave");
  __shared__ __attribute__((aligned(16))) float sK[kSsruBlockMaxKeys * KR];
  __shared__ __attribute__((aligned(16))) float sV[kSsruBlockMaxKeys * KR];
  __shared__ __attribute__((aligned(16))) float sZ[kLnRow<PER>];
  __shared__ __attribute__((aligned(16))) int8_t sX[D];
  __shared__ __attribute__((aligned(16))) float sQ[DH];
  __shared__ __attribute__((aligned(16))) float sP[kSsruBlockMaxKeys];
  __shared__ uint64_t sTab[32];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = blockIdx.x % a.heads, r = blockIdx.x / a.heads;  // r < a.rows, the host bound
  if (wave == 0 && lane < 32) sTab[lane] = kSbExp2Tab[lane];  // wave 0 alone reads it

  // This row's key range, read before the device row count (a stale row's
  // range is clamped into the buffer and its results are discarded).
  int64_t key0 = a.row_key0[r];
  int nk = max(a.row_nk[r], 1);
  key0 = min(max(key0, (int64_t)0), a.max_row - 1);
  // More keys than the block stages: attend over the first 128 (flagged
  // below for live rows; the host bound max_keys rules it out).
  const bool too_long = nk > kSsruBlockMaxKeys;
  nk = min(nk, kSsruBlockMaxKeys);
  const int nk_ld = (int)min((int64_t)nk, a.max_row - key0);

  // wave 0: the row z (relu(s') + x) and the LayerNorm parameters.
  float zv[PER], gv[PER], bv[PER];
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      zv[j] = a.z[(int64_t)r * D + e];
      gv[j] = a.gamma[e];
      bv[j] = a.beta[e];
    }
  }
  // Waves t < T: the weight fragments of query tile t of this head (columns
  // h*DH + 16t ..) and the dequantization operands of lane t's column.
  v4i bf[KS];
  float wm = 1.0f, wb = 0.0f;
  if (wave < T) {
    const int tile = (h * DH >> 4) + wave;
#pragma unroll
    for (int s = 0; s < KS; ++s) bf[s] = frag_load(a.Wq, tile, KS, s, lane);
    const int n = h * DH + 16 * wave + (lane & 15);
    wm = a.wq_mult[n];
    wb = a.wq_bias[n];
  }
  // Waves 1-3: this head's key and value rows (keys past the row's last
  // reload that key, so every load is in bounds; they are not stored).
  f4v kreg[NL], vreg[NL];
  const int lt = tid - 64;
  if (wave > 0) {
    const int64_t base = key0 * a.ldkv + h * DH;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int idx = min(lt + kSbLoaders * i, nk_ld * V4 - 1);
      const int64_t off = base + (int64_t)(idx / V4) * a.ldkv + 4 * (idx % V4);
      kreg[i] = *(const f4v*)(a.k + off);
      vreg[i] = *(const f4v*)(a.v + off);
    }
  }
  const int n_rows = a.rows_dev ? *a.rows_dev : a.rows;
  if (r >= n_rows) return;  // the whole workgroup alike
  if (too_long && tid == 0 && a.err) *a.err = 2;

  if (wave == 0) {
    // LayerNorm(z): the SSRU LayerNorm (ssru_update_layer_norm_into).
    float o[PER];
    ln_wave<PER>(zv, sZ, gv, bv, lane, o);
    bool bad = false;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = lane + 64 * j;
      bad |= !isfinite(o[j]);
      if (h == 0) a.x_out[(int64_t)r * D + e] = o[j];
      sX[e] = (int8_t)quantize_one(o[j], a.xq_mult);
    }
    if (__any(bad) && lane == 0 && a.err) *a.err = 1;
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int idx = lt + kSbLoaders * i;
      if (idx < kSsruBlockMaxKeys * V4) {  // rows past the last key hold finite copies
        const int so = (idx / V4) * KR + 4 * (idx % V4);
        *(f4v*)(sK + so) = kreg[i];
        *(f4v*)(sV + so) = vreg[i];
      }
    }
  }
  wg_lds_barrier();  // LDS only: the state and row stores stay in flight

  // Query tile `wave`: row 0 of the MFMA A operand is the quantized row
  // (lanes 0, 16, 32, 48 hold its 16-byte k-slices), the other rows zero;
  // lane l < 16 ends with column l of row 0 in acc[0].
  if (wave < T) {
    v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const v4i x = (lane & 15) == 0 ? *(const v4i*)(sX + 64 * s + (lane >> 4) * 16) : v4i{0, 0, 0, 0};
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(x, bf[s], acc, 0, 0, 0);
    }
    if (lane < 16) sQ[16 * wave + lane] = dequant(acc[0], a.xq_mult, wm, wb);
  }
  wg_lds_barrier();
  if (wave != 0) return;

  // Scores: lane = key (keys lane and 64 + lane), DH-term dots in dimension
  // order from -0.0; q (an LDS broadcast) and both key rows are read before
  // the two chains run side by side.
  const float scale = 1.0f / sqrtf((float)DH);
  const float* k0 = sK + min(lane, nk - 1) * KR;
  const float* k1 = sK + min(64 + lane, nk - 1) * KR;
  f4v qv[V4], x0[V4], x1[V4];
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    qv[i] = *(const f4v*)(sQ + 4 * i);
    x0[i] = *(const f4v*)(k0 + 4 * i);
    x1[i] = *(const f4v*)(k1 + 4 * i);
  }
  float d0 = -0.0f, d1 = -0.0f;
#pragma unroll
  for (int i = 0; i < V4; ++i) {
    d0 = d0 + qv[i].x * x0[i].x;
    d1 = d1 + qv[i].x * x1[i].x;
    d0 = d0 + qv[i].y * x0[i].y;
    d1 = d1 + qv[i].y * x1[i].y;
    d0 = d0 + qv[i].z * x0[i].z;
    d1 = d1 + qv[i].z * x1[i].z;
    d0 = d0 + qv[i].w * x0[i].w;
    d1 = d1 + qv[i].w * x1[i].w;
  }
  const float s0 = lane < nk ? d0 * scale : -INFINITY;
  const float s1 = 64 + lane < nk ? d1 * scale : -INFINITY;
  const float mx = wave_max(fmaxf(s0, s1));
  const float p0 = lane < nk ? ref_expf(s0 - mx, sTab) : 0.0f;
  const float p1 = 64 + lane < nk ? ref_expf(s1 - mx, sTab) : 0.0f;
  sP[lane] = p0;
  sP[64 + lane] = p1;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  // Denominator: the probabilities in key order from 0.0 (keys past the last
  // hold +0.0, which leaves the non-negative sum unchanged), 16 at a time.
  const float inv = 1.0f / seq_fold_lds_upto<kSsruBlockMaxKeys / 16>((const float4*)sP, (nk + 15) >> 4, 0.0f);
  // out_d = sum_j v[j][d] * (e_j * inv) in key order from 0.0; lane = d.
  // Sixteen keys per batch in two alternating register sets: the next batch
  // is read while this one is added.  Keys past the last have e = +0.0 and
  // finite value rows, so their +-0.0 products leave the sum unchanged.
  constexpr int PB = 16;
  const int dl = min(lane, DH - 1);
  const float* vc = sV + dl;
  const int nb = (nk + PB - 1) / PB;
  float o = 0.0f;
  f4v pA[PB / 4], pB[PB / 4];
  float vA[PB], vB[PB];
  auto read = [&](int b, f4v (&p)[PB / 4], float (&v)[PB]) {
#pragma unroll
    for (int i = 0; i < PB / 4; ++i) p[i] = *(const f4v*)(sP + PB * b + 4 * i);
#pragma unroll
    for (int u = 0; u < PB; ++u) v[u] = vc[(PB * b + u) * KR];
  };
  auto add = [&](const f4v (&p)[PB / 4], const float (&v)[PB]) {
#pragma unroll
    for (int u = 0; u < PB; ++u) o = o + v[u] * (p[u / 4][u % 4] * inv);
  };
  read(0, pA, vA);
#pragma unroll 1
  for (int b = 0;;) {
    read(min(b + 1, nb - 1), pB, vB);  // past the last batch: re-read it, unused
    __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the adds
    add(pA, vA);
    if (++b >= nb) break;
    read(min(b + 1, nb - 1), pA, vA);
    __builtin_amdgcn_sched_barrier(0);
    add(pB, vB);
    if (++b >= nb) break;
  }

  if (lane < DH) a.qout[(int64_t)r * a.ldqout + h * DH + lane] = (int8_t)quantize_one(o, a.qmult);
  if (lane == 0 && h == 0) a.qa[r] = a.qmult;
  if (__any(lane < DH && !isfinite(o)) && lane == 0 && a.err) *a.err = 1;
}

// ---------------------------------------------------------------------------
// SSRU input: for 8 rows and 64 state columns per workgroup, wave w builds
// row w's layer input x (PRO_LN: LayerNorm(y + r); PRO_EMB: the embedding of
// the row's last token at position `step`), quantizes it with the candidate
// and forget projections' multipliers into LDS and keeps x; waves 0-3 then
// project the rows onto candidate tiles 4s .. 4s+3 (columns 64s ..), waves
// 4-7 onto the forget-gate tiles of the same columns, and waves 0-3 apply
// the SSRU update to each (row, column): state' = gate * state + (1 - gate)
// * c with gate = 1 / (1 + exp(-f)), z = relu(state') + x.
// ---------------------------------------------------------------------------
constexpr int kSiRows = 8;
constexpr int kSiCols = 64;  // state columns per workgroup

template <int PER, int PK>
__global__ __launch_bounds__(512) void k_ssru_input(SsruInputArgs a) {
  constexpr int D = PER * 64;
  constexpr int KS = D / 64;
  __shared__ __attribute__((aligned(16))) float sZ[kSiRows][kLnRow<PER>];
  __shared__ __attribute__((aligned(16))) int8_t sXc[kSiRows][D];
  __shared__ __attribute__((aligned(16))) int8_t sXf[kSiRows][D];
  __shared__ float sRes[kSiRows][D];
  __shared__ float sF[kSiRows][kSiCols + 1];
  __shared__ uint64_t sTab[32];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int slices = D / kSiCols;
  const int slice = blockIdx.x % slices, grp = blockIdx.x / slices;
  const int r = grp * kSiRows + wave;  // this wave's row
  if (tid < 32) sTab[tid] = kSbExp2Tab[tid];
  // Row loads (rows below the host bound are backed by memory).
  const RowPrologue& p = a.pro;
  float ya[PER], yb[PER], gv[PER], bv[PER];
  int tok = -1;
  float emult = 1.0f;
  if (r < a.rows) {
    if constexpr (PK == PRO_LN) {
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = lane + 64 * j;
        ya[j] = p.y[(int64_t)r * D + e];
        yb[j] = p.r[(int64_t)r * D + e];
        gv[j] = p.gamma[e];
        bv[j] = p.beta[e];
      }
    } else {
      tok = p.row_prev[r];  // negative: the position row alone
      const int tk = tok < 0 ? 0 : tok;
      emult = p.emb_mult[tk];
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int e = lane + 64 * j;
        ya[j] = p.pos[(int64_t)a.step * D + e];
        yb[j] = (float)p.emb[(int64_t)tk * D + e];
      }
    }
  }
  // Tile of this wave: candidate columns 64 slice + 16 wave (waves 0-3) or the
  // forget-gate columns d + 64 slice + 16 (wave - 4) (waves 4-7).
  const bool fpart = wave >= 4;
  const int tile = (fpart ? D / 16 : 0) + 4 * slice + (wave & 3);
  v4i bf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) bf[s] = frag_load(a.W, tile, KS, s, lane);
  const int col = 16 * tile + (lane & 15);
  const float wm = a.wmult[col], wb = a.bias[col];
  // State column j of the lane's rows 4 (lane / 16) + i (candidate waves).
  const int j = kSiCols * slice + 16 * (wave & 3) + (lane & 15);
  float st[4];
  int64_t sr[4];
  if (!fpart && lane < 32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = min(grp * kSiRows + 4 * (lane >> 4) + i, a.rows - 1);
      // a stale row's sequence is clamped into the state buffer
      sr[i] = a.state_row ? min(max((int64_t)a.state_row[m], (int64_t)0), a.state_rows - 1) : m;
      st[i] = a.state_in[sr[i] * D + j];
    }
  }
  const int n_rows = a.rows_dev ? min(*a.rows_dev, a.rows) : a.rows;
  if (grp * kSiRows >= n_rows) return;  // the whole workgroup alike
  if (r < n_rows) {
    float x[PER];
    if constexpr (PK == PRO_LN) {
      float z[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) z[k] = ya[k] + yb[k];
      ln_wave<PER>(z, sZ[wave], gv, bv, lane, x);
    } else {
#pragma unroll
      for (int k = 0; k < PER; ++k) x[k] = tok < 0 ? ya[k] : (yb[k] / emult) * p.scale + ya[k];
    }
    bool bad = false;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int e = lane + 64 * k;
      bad |= !isfinite(x[k]);
      sRes[wave][e] = x[k];
      sXc[wave][e] = (int8_t)quantize_one(x[k], a.act_c);
      sXf[wave][e] = (int8_t)quantize_one(x[k], a.act_f);
    }
    if (__any(bad) && lane == 0 && a.err) *a.err = 1;
  }
  wg_lds_barrier();
  // Rows 0..7 of the A operand are the group's rows (zero past the device
  // count), rows 8..15 zero.  Lane l ends with rows 4(l/16)+i of column l%16.
  const int ar = lane & 15;
  const bool a_live = ar < kSiRows && grp * kSiRows + ar < n_rows;
  const int8_t* sx = fpart ? &sXf[0][0] : &sXc[0][0];
  v4i acc = v4i{0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const v4i xq = a_live ? *(const v4i*)(sx + ar * D + 64 * s + (lane >> 4) * 16) : v4i{0, 0, 0, 0};
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xq, bf[s], acc, 0, 0, 0);
  }
  const float inv = dequant_scale(fpart ? a.act_f : a.act_c, wm);
  if (fpart && lane < 32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) sF[4 * (lane >> 4) + i][16 * (wave - 4) + (lane & 15)] = dequant_apply(acc[i], inv, wb);
  }
  wg_lds_barrier();
  if (fpart || lane >= 32) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rl = 4 * (lane >> 4) + i, m = grp * kSiRows + rl;
    if (m >= n_rows) continue;
    const float c = dequant_apply(acc[i], inv, wb);
    const float f = sF[rl][16 * wave + (lane & 15)];
    const float e = ref_expf(-f, sTab);
    const float gate = 1.0f / (1.0f + e);
    const float next = gate * st[i] + (1.0f - gate) * c;
    a.state_out[sr[i] * D + j] = next;
    a.z[(int64_t)m * D + j] = (next > 0.0f ? next : 0.0f) + sRes[rl][j];
  }
}

}  // namespace

hipError_t launch_ssru_input(const SsruInputArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const RowPrologue& p = a.pro;
  const bool pro_ok = p.kind == PRO_LN ? (p.y && p.r && p.gamma && p.beta)
                                       : (p.kind == PRO_EMB && p.emb && p.emb_mult && p.pos && p.row_prev &&
                                          a.step >= 0 && a.step < kMaxPosition);
  if ((a.d != 256 && a.d != 384 && a.d != 512) || !pro_ok || !a.W || !a.wmult || !a.bias ||
      !a.state_in || !a.state_out || a.state_in == a.state_out || a.state_rows < a.rows || !a.z)
    return hipErrorInvalidValue;
  for (const float m : {a.act_c, a.act_f})
    if (!(m > 0.0f) || !(m < __builtin_huge_valf())) return hipErrorInvalidValue;
  const int groups = (a.rows + kSiRows - 1) / kSiRows;
  const dim3 grid(groups * (a.d / kSiCols)), block(512);
#define MH_SI(P)                                                                          \
  if (p.kind == PRO_LN)                                                                   \
    hipLaunchKernelGGL((k_ssru_input<P, PRO_LN>), grid, block, 0, s, a);                  \
  else                                                                                    \
    hipLaunchKernelGGL((k_ssru_input<P, PRO_EMB>), grid, block, 0, s, a);
  if (a.d == 256) {
    MH_SI(4)
  } else if (a.d == 384) {
    MH_SI(6)
  } else {
    MH_SI(8)
  }
#undef MH_SI
  return hipGetLastError();
}

bool ssru_block_supported(int d, int heads, int max_keys) {
  if (heads <= 0 || d % heads || max_keys <= 0 || max_keys > kSsruBlockMaxKeys) return false;
  const int dh = d / heads;
  return (d == 256 && dh == 64) || (d == 384 && (dh == 48 || dh == 64)) || (d == 512 && dh == 64);
}

hipError_t launch_ssru_block(const SsruBlockArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (!ssru_block_supported(a.d, a.heads, a.max_keys) || !a.z || !a.gamma || !a.beta ||
      !a.x_out || !a.Wq || !a.wq_mult || !a.wq_bias || !a.k || !a.v || a.ldkv < a.d || !a.row_key0 ||
      !a.row_nk || a.max_row <= 0 || !a.qout || !a.qa || a.ldqout < a.d ||
      (int64_t)a.rows * a.heads > 0x7fffffff)
    return hipErrorInvalidValue;
  for (const float m : {a.xq_mult, a.qmult})
    if (!(m > 0.0f) || !(m < __builtin_huge_valf())) return hipErrorInvalidValue;
  const dim3 grid(a.rows * a.heads), block(kSbThreads);
  const int dh = a.d / a.heads;
  if (a.d == 256)
    hipLaunchKernelGGL((k_ssru_block<4, 64>), grid, block, 0, s, a);
  else if (a.d == 384 && dh == 48)
    hipLaunchKernelGGL((k_ssru_block<6, 48>), grid, block, 0, s, a);
  else if (a.d == 384)
    hipLaunchKernelGGL((k_ssru_block<6, 64>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((k_ssru_block<8, 64>), grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace mh
