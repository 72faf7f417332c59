// attention.hip — variable-length multi-head attention, one query row per
// workgroup and one 64-wide wavefront per head (head_dim = 64).
//
// Semantics of attention_into (tensor.rs:251-318): score_k = (q . k_k) * 1/8,
// softmax as max, exp(s - max), sum, multiply by 1/sum, then
// out = sum_k p_k v_k in key order.  Mapping onto the wave:
//   * scores: lane = key (keys lane, lane+64, ...), sequential 64-term dot
//     with q broadcast from SGPRs;
//   * softmax: wave max, canonical exp, lane partial sums + xor butterfly;
//   * PV: lane = output dim, keys accumulated in order (the reference order);
//     probabilities are broadcast from LDS.
// The score row never leaves the chip.  Sequences are packed (cu_seqlens), so
// there is no padding and no mask; keys beyond a row's count are never read.
// The three modes differ only in where a row's keys live: its own sequence
// (encoder self-attention / op-level varlen), the encoder output of its
// sequence (cross-attention at decode), or its per-sequence KV cache
// (decoder self-attention over steps 0..t).
#include "device_common.h"
#include "kernels.h"

namespace mh {
namespace {

template <typename T>
struct Io;
template <>
struct Io<float> {
  static __device__ __forceinline__ float at(const void* p, int64_t i) {
    return ((const float*)p)[i];
  }
  // 64 consecutive values starting at element i (16-byte aligned)
  static __device__ __forceinline__ void row64(const void* p, int64_t i, float* out) {
    const float4* v = (const float4*)((const float*)p + i);
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const float4 t = v[c];
      out[4 * c + 0] = t.x;
      out[4 * c + 1] = t.y;
      out[4 * c + 2] = t.z;
      out[4 * c + 3] = t.w;
    }
  }
};
template <>
struct Io<uint16_t> {
  static __device__ __forceinline__ float at(const void* p, int64_t i) {
    return bf16_to_f32(((const uint16_t*)p)[i]);
  }
  static __device__ __forceinline__ void row64(const void* p, int64_t i, float* out) {
    const uint4* v = (const uint4*)((const uint16_t*)p + i);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint4 t = v[c];
      const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        out[8 * c + 2 * u + 0] = __uint_as_float(w[u] << 16);
        out[8 * c + 2 * u + 1] = __uint_as_float(w[u] & 0xFFFF0000u);
      }
    }
  }
};

template <int CH, typename T>
__global__ __launch_bounds__(1024) void k_attention(AttnArgs a) {
  extern __shared__ float sP[];  // [heads][CH*64] probabilities
  __shared__ float sMax[16];
  const int r = blockIdx.x;
  const int n = a.rows_dev ? *a.rows_dev : a.rows;
  if (r >= n) return;
  const int h = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int D = a.heads * kHeadDim;

  int64_t key0;
  int nk;
  if (a.mode == ATT_SEQ) {
    const int sq = a.seq_of_row[r];
    key0 = a.cu[sq];
    nk = (int)(a.cu[sq + 1] - a.cu[sq]);
  } else if (a.mode == ATT_CROSS) {
    const int slot = a.act[r];
    key0 = a.cu[slot];
    nk = (int)(a.cu[slot + 1] - a.cu[slot]);
  } else {
    key0 = a.kv_base[a.act[r]];
    nk = a.step + 1;
  }
  // A key range longer than this variant holds would overrun the score
  // registers and the LDS row: flag it and attend over the first CH*64 keys.
  if (nk > CH * 64) {
    if (threadIdx.x == 0 && a.err) *a.err = 2;
    nk = CH * 64;
  }

  // q of this head, one element per lane, broadcast through SGPRs.
  const float qv = Io<T>::at(a.q, (int64_t)r * a.ldq + h * kHeadDim + lane);
  float qs[kHeadDim];
#pragma unroll
  for (int i = 0; i < kHeadDim; ++i)
    qs[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qv), i));

  const float scale = 1.0f / sqrtf((float)kHeadDim);
  float s[CH];
  float mloc = -INFINITY;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    s[c] = -INFINITY;
    const int j = c * 64 + lane;
    if (c * 64 < nk && j < nk) {
      float kr[kHeadDim];
      Io<T>::row64(a.k, (key0 + j) * a.ldkv + h * kHeadDim, kr);
      float dot = -0.0f;
#pragma unroll
      for (int i = 0; i < kHeadDim; ++i) dot = dot + qs[i] * kr[i];
      s[c] = dot * scale;
      mloc = fmaxf(mloc, s[c]);
    }
  }
  const float mx = wave_max(mloc);
  float part = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int j = c * 64 + lane;
    if (j < nk) {
      s[c] = canon_expf(s[c] - mx);
      part = part + s[c];
    }
  }
  const float inv = 1.0f / wave_sum_canon(part);
  float* ph = sP + h * (CH * 64);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int j = c * 64 + lane;
    if (j < nk) ph[j] = s[c] * inv;
  }
  __syncthreads();

  // out_d = sum_j v[j][d] * p_j, keys in order.
  const int64_t vbase = key0 * a.ldkv + h * kHeadDim + lane;
  float o = 0.0f;
  int j = 0;
  for (; j + 4 <= nk; j += 4) {
    const float v0 = Io<T>::at(a.v, vbase + (int64_t)(j + 0) * a.ldkv);
    const float v1 = Io<T>::at(a.v, vbase + (int64_t)(j + 1) * a.ldkv);
    const float v2 = Io<T>::at(a.v, vbase + (int64_t)(j + 2) * a.ldkv);
    const float v3 = Io<T>::at(a.v, vbase + (int64_t)(j + 3) * a.ldkv);
    o = o + v0 * ph[j + 0];
    o = o + v1 * ph[j + 1];
    o = o + v2 * ph[j + 2];
    o = o + v3 * ph[j + 3];
  }
  for (; j < nk; ++j) o = o + Io<T>::at(a.v, vbase + (int64_t)j * a.ldkv) * ph[j];

  if (a.out) a.out[(int64_t)r * a.ldo + h * kHeadDim + lane] = o;
  if (a.q8) {
    const bool bad = !isfinite(o);
    const float m = wave_max(fabsf(o));
    if (lane == 0) sMax[h] = m;
    __syncthreads();
    float absmax = 0.0f;
    for (int w = 0; w < a.heads; ++w) absmax = fmaxf(absmax, sMax[w]);
    const float sc = row_multiplier(absmax);
    a.q8[(int64_t)r * D + h * kHeadDim + lane] = (int8_t)quantize_one(o, sc);
    if (threadIdx.x == 0) a.qa[r] = sc;
    if (__any(bad) && lane == 0 && a.err) *a.err = 1;
  }
}

template <int CH>
hipError_t launch_ch(const AttnArgs& a, hipStream_t s) {
  const size_t lds = (size_t)a.heads * CH * 64 * sizeof(float);
  const dim3 grid(a.rows), block(a.heads * 64);
  if (a.bf16) {
    if (lds > 64 * 1024) {
      hipError_t e = hipFuncSetAttribute((const void*)k_attention<CH, uint16_t>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_attention<CH, uint16_t>), grid, block, lds, s, a);
  } else {
    if (lds > 64 * 1024) {
      hipError_t e = hipFuncSetAttribute((const void*)k_attention<CH, float>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((k_attention<CH, float>), grid, block, lds, s, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (a.heads <= 0 || a.heads > 16 || a.max_keys <= 0) return hipErrorInvalidValue;
  if (a.max_keys <= 128) return launch_ch<2>(a, s);
  if (a.max_keys <= 512) return launch_ch<8>(a, s);
  if (a.max_keys <= 1024) return launch_ch<16>(a, s);
  if (a.max_keys <= 4096 && a.heads <= 8) return launch_ch<64>(a, s);
  return hipErrorInvalidValue;
}

}  // namespace mh
