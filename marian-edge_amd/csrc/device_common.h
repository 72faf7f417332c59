// device_common.h — device helpers shared by the gfx950 kernels.
//
// Arithmetic contract (identical in the CPU oracle, bit for bit):
//  * fp32 sums over a row are "canonical": lane l of a 64-wide wavefront sums
//    elements l, l+64, l+128, ... in that order starting from 0.0f, then the
//    wave combines lane partials with an xor butterfly 32,16,8,4,2,1.
//  * exp is evaluated by canon_expf below (double precision Cody-Waite
//    reduction + degree-11 Taylor polynomial, rounded once to fp32).
//  * every other fp32 expression is evaluated in the reference's sequential
//    order with separate multiply and add (the library is built with
//    -ffp-contract=off, IEEE division and square root).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mh {

constexpr int kWave = 64;
constexpr int kHeadDim = 64;           // per-head width supported by the kernels
constexpr int kMaxPosition = 4096;     // marian-model manifest.rs:13
constexpr int kMaxRowsPerCall = 4096;  // engine batch ceiling (LDS scan size)

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum_canon(float p) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) p = p + __shfl_xor(p, off, kWave);
  return p;
}

__device__ __forceinline__ float wave_max(float p) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) p = fmaxf(p, __shfl_xor(p, off, kWave));
  return p;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int off) {
  const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  const uint32_t l2 = (uint32_t)__shfl_xor((int)lo, off, kWave);
  const uint32_t h2 = (uint32_t)__shfl_xor((int)hi, off, kWave);
  return ((uint64_t)h2 << 32) | l2;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = shfl_xor_u64(v, off);
    v = o > v ? o : v;
  }
  return v;
}

// exp(x) evaluated as: n = rint(x/ln2), r = x - n*ln2 (double), Horner
// polynomial sum_{k<=11} r^k/k! with separate multiplies and adds, scaled by
// 2^n and rounded once to fp32.  Matches the oracle's canon_expf exactly.
__device__ __forceinline__ float canon_expf(float xf) {
  if (!(xf == xf)) return xf;
  if (xf < -104.0f) return 0.0f;
  if (xf > 89.0f) return __int_as_float(0x7f800000);
  const double x = (double)xf;
  const double n = rint(x * 0x1.71547652b82fep+0);
  const double r = x - n * 0x1.62e42fefa39efp-1;
  double p = 0x1.ae64567f544e4p-26;
  p = p * r + 0x1.27e4fb7789f5cp-22;
  p = p * r + 0x1.71de3a556c734p-19;
  p = p * r + 0x1.a01a01a01a01ap-16;
  p = p * r + 0x1.a01a01a01a01ap-13;
  p = p * r + 0x1.6c16c16c16c17p-10;
  p = p * r + 0x1.1111111111111p-7;
  p = p * r + 0x1.5555555555555p-5;
  p = p * r + 0x1.5555555555555p-3;
  p = p * r + 0x1.0000000000000p-1;
  p = p * r + 1.0;
  p = p * r + 1.0;
  return (float)ldexp(p, (int)n);
}

// q = clamp(round_half_even(x * a), -127, 127)  (q8_gemm.rs:584-587)
__device__ __forceinline__ int quantize_one(float x, float a) {
  float v = rintf(x * a);
  v = fminf(fmaxf(v, -127.0f), 127.0f);
  return (int)v;
}

// Per-row activation multiplier: 127 / max|x| (1 for an all-zero row).
__device__ __forceinline__ float row_multiplier(float absmax) {
  return absmax > 0.0f ? 127.0f / absmax : 1.0f;
}

// y = acc * (1 / (a * w)) + b: one multiply, one divide, one multiply, one add
// (q8_gemm.rs:438-446).
__device__ __forceinline__ float dequant(int32_t acc, float a, float w, float b) {
  const float inv = 1.0f / (a * w);
  return (float)acc * inv + b;
}

// Orderable 64-bit key: larger logit wins, equal logits prefer the lower id
// (the reference's strict '>' scan in ascending id order).  0 = no candidate.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t id) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - id);
}
__device__ __forceinline__ int32_t argmax_key_id(uint64_t key) {
  return key == 0 ? 0 : (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu));
}

// Generation mask of the reference shortlist (shortlist.rs:169-176).
__device__ __forceinline__ bool generation_masked(uint32_t id) {
  return id == 1u || (id >= 7u && id <= 38u);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

}  // namespace mh
