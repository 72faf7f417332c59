// rows.hip — one-wavefront-per-row kernels: activation quantization, residual
// LayerNorm (+ quantization for the next GEMM), embedding gather, and the
// per-step token selection / active-set compaction of the decode loop.
#include "device_common.h"
#include "kernels.h"

namespace mh {
namespace {

constexpr float kLayerNormEpsilon = 1.0e-6f;  // tensor.rs:3

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

// out = LN(y + r) with canonical sums; optional quantization of out.
template <int PER>
__global__ __launch_bounds__(256) void k_residual_ln(const float* y, const float* r,
                                                     const float* gamma, const float* beta,
                                                     int rows, const int* rows_dev, float* out,
                                                     int8_t* q, float* a, int* err) {
  constexpr int D = PER * 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = rows_dev ? *rows_dev : rows;
  if (row >= n) return;
  const float* yr = y + (int64_t)row * D;
  const float* rr = r + (int64_t)row * D;
  float z[PER];
  float p = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    z[j] = yr[lane + 64 * j] + rr[lane + 64 * j];
    p = p + z[j];
  }
  const float mean = wave_sum_canon(p) / (float)D;
  float p2 = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float c = z[j] - mean;
    p2 = p2 + c * c;
  }
  const float var = wave_sum_canon(p2) / (float)D;
  const float inv = 1.0f / sqrtf(var + kLayerNormEpsilon);
  float o[PER];
  float m = 0.0f;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    o[j] = ((z[j] - mean) * inv) * gamma[i] + beta[i];
    bad |= !isfinite(o[j]);
    m = fmaxf(m, fabsf(o[j]));
    out[(int64_t)row * D + i] = o[j];
  }
  if (q) {
    m = wave_max(m);
    const float sc = row_multiplier(m);
#pragma unroll
    for (int j = 0; j < PER; ++j) q[(int64_t)row * D + lane + 64 * j] = (int8_t)quantize_one(o[j], sc);
    if (lane == 0) a[row] = sc;
    if (__any(bad) && lane == 0 && err) *err = 1;
  }
}

// x = (q/mult)*sqrt(d) + pos[p] (q8_engine.rs:53-74, 586-630); token < 0 gives
// pos[p] alone (the decoder's first step).  Fused quantization of x.
template <int PER>
__global__ __launch_bounds__(256) void k_embed(EmbedArgs a) {
  constexpr int D = PER * 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = a.rows_dev ? *a.rows_dev : a.rows;
  if (row >= n) return;
  int token, p;
  if (a.tokens) {
    token = a.tokens[row];
    p = a.positions[row];
  } else {
    token = a.prev[a.act[row]];
    p = a.step;
  }
  const float* pr = a.pos + (int64_t)p * D;
  float o[PER];
  float m = 0.0f;
  bool bad = false;
  if (token < 0) {
#pragma unroll
    for (int j = 0; j < PER; ++j) o[j] = pr[lane + 64 * j];
  } else {
    const int8_t* er = a.emb + (int64_t)token * D;
    const float mult = a.emb_mult[token];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const float v = (float)er[lane + 64 * j] / mult;
      o[j] = v * a.scale + pr[lane + 64 * j];
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    bad |= !isfinite(o[j]);
    m = fmaxf(m, fabsf(o[j]));
    a.x[(int64_t)row * D + lane + 64 * j] = o[j];
  }
  m = wave_max(m);
  const float sc = row_multiplier(m);
#pragma unroll
  for (int j = 0; j < PER; ++j) a.xq[(int64_t)row * D + lane + 64 * j] = (int8_t)quantize_one(o[j], sc);
  if (lane == 0) a.xa[row] = sc;
  if (__any(bad) && lane == 0 && a.err) *a.err = 1;
}

// End of a decode step: reduce each active row's argmax partials to a token,
// append it, apply the stop rules of q8_engine.rs:383-390, 444-448, and
// compact the active list in order.  One workgroup; rows <= kMaxRowsPerCall.
__global__ __launch_bounds__(1024) void k_finalize(FinalizeArgs f) {
  __shared__ int s_slot[kMaxRowsPerCall];
  __shared__ unsigned char s_keep[kMaxRowsPerCall];
  __shared__ int s_wsum[16];
  __shared__ int s_total;
  const int n = *f.n_active;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int r = wave; r < n; r += 16) {
    uint64_t best = 0;
    for (int p = lane; p < f.nparts; p += 64) {
      const uint64_t k = f.partials[(int64_t)r * f.nparts + p];
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) {
      const int slot = f.act[r];
      const int32_t tok = argmax_key_id(best);
      f.out_tok[f.out_base[slot] + f.step] = tok;
      f.count[slot] = (uint32_t)f.step + 1u;
      f.prev[slot] = tok;
      const bool fin = (tok == 0 && !(f.flags & 1u)) || (uint32_t)f.step + 1u >= f.limit[slot];
      s_slot[r] = slot;
      s_keep[r] = fin ? 0 : 1;
    }
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
    if (r < n && s_keep[r]) f.act[pos++] = s_slot[r];
  }
  if (tid == 0) *f.n_active = s_total;
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
  hipLaunchKernelGGL(k_quantize_rows, dim3((rows + 3) / 4), dim3(256), 0, s, x, ldx, rows,
                     rows_dev, cols, q, ldq, a, err);
  return hipGetLastError();
}

#define MH_PER_DISPATCH(PER_VALUE, CALL) \
  switch (PER_VALUE) {                   \
    case 4: CALL(4); break;              \
    case 6: CALL(6); break;              \
    case 8: CALL(8); break;              \
    case 12: CALL(12); break;            \
    case 16: CALL(16); break;            \
    default: return hipErrorInvalidValue; \
  }

hipError_t launch_residual_ln(const float* y, const float* r, const float* g, const float* b,
                              int rows, const int* rows_dev, int d, float* out, int8_t* q,
                              float* a, int* err, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (d % 64) return hipErrorInvalidValue;
  const dim3 grid((rows + 3) / 4), block(256);
#define MH_LN(P) \
  hipLaunchKernelGGL(k_residual_ln<P>, grid, block, 0, s, y, r, g, b, rows, rows_dev, out, q, a, err)
  MH_PER_DISPATCH(d / 64, MH_LN)
#undef MH_LN
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
  hipLaunchKernelGGL(k_finalize, dim3(1), dim3(1024), 0, s, f);
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
