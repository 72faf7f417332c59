// device_common.h — device helpers shared by the gfx950 kernels.
//
// Arithmetic contract: every fp32 value is produced by the same sequence of
// IEEE operations as the reference's x86 Q8 path, so results are identical
// bit for bit:
//  * sums follow the reference's order: LayerNorm's mean and variance and
//    attention's dot products are strictly sequential folds starting from
//    -0.0 (Rust's f32 Sum), the softmax denominator a sequential sum from 0.0;
//  * exp is the C library's expf (restated in ref_expf.h);
//  * every other expression is evaluated in the reference's order with
//    separate multiplies and adds (the library is built with
//    -ffp-contract=off, IEEE division and square root, fp32 denormals kept).
// Maxima (absmax, softmax max, argmax) are order independent and use wave
// reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ref_expf.h"

namespace mh {

// Native 4 x fp32 vector (HIP's float4 is a struct whose copies become memcpy,
// which keeps an array of them out of registers).
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kHeadDim = 64;           // per-head width supported by the kernels
constexpr int kMaxPosition = 4096;     // marian-model manifest.rs:13
constexpr int kMaxRowsPerCall = 4096;  // engine batch ceiling (LDS scan size)
constexpr float kLayerNormEpsilon = 1.0e-6f;  // tensor.rs:3

typedef int v4i __attribute__((ext_vector_type(4)));

// min(device row count, host bound) when the launch carries a device row
// count, else the host bound.  The count is read through a selected pointer
// (an absent count reads kNoRowCount), so no branch splits the kernel's
// prologue: a load behind a branch is waited for inside it, which would put
// a memory round trip between the loads issued before and after it.
static __device__ int kNoRowCount = 0x7fffffff;
__device__ __forceinline__ int bounded_rows(const int* rows_dev, int rows) {
  return min(*(rows_dev ? rows_dev : &kNoRowCount), rows);
}

// Requests every 64-byte line of the first BYTES bytes of the kernel's
// arguments in one batch of scalar loads at the start of the kernel.  The
// compiler loads an argument where it is first used, in several batches,
// and a scalar load's wait covers every scalar load in flight; with the
// lines already in the scalar cache, the later batches hit it instead of
// each waiting for a miss.
template <int BYTES>
__device__ __forceinline__ void touch_kernargs() {
  constexpr int kLines = (BYTES + 63) / 64;
  static_assert(kLines >= 1 && kLines <= 8, "one to eight lines");
  typedef const __attribute__((address_space(4))) uint32_t* karg_ptr;
  const karg_ptr k = (karg_ptr)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t t[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) t[i] = i < kLines ? k[16 * i] : 0u;
  asm volatile("" ::"s"(t[0]), "s"(t[1]), "s"(t[2]), "s"(t[3]), "s"(t[4]), "s"(t[5]), "s"(t[6]), "s"(t[7]));
}

// Value of lane (l ^ off) for lane l, for off = 1, 2 (DPP quad permutes),
// 4, 8, 16 (ds_swizzle lane swaps within 32) and 32 (v_permlane32_swap).
// Exactly the xor pairing of __shfl_xor, without the LDS crossbar.
template <int OFF>
__device__ __forceinline__ int xor_lane(int v) {
  if constexpr (OFF == 1) {
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (OFF == 2) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (OFF == 4 || OFF == 8 || OFF == 16) {
    return __builtin_amdgcn_ds_swizzle(v, (OFF << 10) | 0x1F);  // swizzle(SWAP, OFF)
  } else {
    static_assert(OFF == 32, "xor_lane offset");
    const auto sw = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (__lane_id() < 32) ? (int)sw[1] : (int)sw[0];
  }
}

template <int OFF>
__device__ __forceinline__ float xor_lane_f(float v) {
  return __int_as_float(xor_lane<OFF>(__float_as_int(v)));
}

template <int OFF>
__device__ __forceinline__ uint64_t xor_lane_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)xor_lane<OFF>((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)xor_lane<OFF>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Maximum over the wave; max is exact in any order, so the reduction uses
// VALU-only lane moves: DPP within each 16-lane row (quad swaps, rotations by
// 4 and 8), then the four row maxima are read out as scalars.  Every lane
// returns the same value.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float wave_max(float p) {
  p = fmaxf(p, __int_as_float(dpp_mov<0xB1>(__float_as_int(p))));   // quad_perm [1,0,3,2]
  p = fmaxf(p, __int_as_float(dpp_mov<0x4E>(__float_as_int(p))));   // quad_perm [2,3,0,1]
  p = fmaxf(p, __int_as_float(dpp_mov<0x124>(__float_as_int(p))));  // row_ror:4
  p = fmaxf(p, __int_as_float(dpp_mov<0x128>(__float_as_int(p))));  // row_ror:8
  const int b = __float_as_int(p);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Maximum over each 32-lane half of the wave (every lane returns its half's):
// the row maxima by DPP, then rows 0-1 and 2-3 paired by a lane swap.
__device__ __forceinline__ float half_wave_max(float p) {
  p = fmaxf(p, __int_as_float(dpp_mov<0xB1>(__float_as_int(p))));   // quad_perm [1,0,3,2]
  p = fmaxf(p, __int_as_float(dpp_mov<0x4E>(__float_as_int(p))));   // quad_perm [2,3,0,1]
  p = fmaxf(p, __int_as_float(dpp_mov<0x124>(__float_as_int(p))));  // row_ror:4
  p = fmaxf(p, __int_as_float(dpp_mov<0x128>(__float_as_int(p))));  // row_ror:8
  return fmaxf(p, xor_lane_f<16>(p));
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_mov_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)dpp_mov<CTRL>((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)dpp_mov<CTRL>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = umax64(v, dpp_mov_u64<0xB1>(v));
  v = umax64(v, dpp_mov_u64<0x4E>(v));
  v = umax64(v, dpp_mov_u64<0x124>(v));
  v = umax64(v, dpp_mov_u64<0x128>(v));
  uint64_t best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * r);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 16 * r);
    best = umax64(best, (hi << 32) | lo);
  }
  return best;
}

// Strictly sequential fp32 fold init + p[0] + p[1] + ... over N4 float4 in
// LDS (each lane its own p, or one shared p read as a broadcast).  Two
// buffers of NB float4 alternate: the next batch is read while the current
// one is added, so the dependent chain never waits on LDS.  The batch loop is
// kept rolled, which bounds the live registers (a fully unrolled fold lets
// the scheduler hoist every read and spill) and the code size.
template <int N4, int NB = 8>
__device__ __forceinline__ float seq_fold_lds(const float4* p, float init) {
  constexpr int NBATCH = N4 / NB;
  static_assert(N4 % (2 * NB) == 0, "pairs of batches");
  float4 A[NB], B[NB];
  float s = init;
#pragma unroll
  for (int b = 0; b < NB; ++b) A[b] = p[b];
#pragma unroll 1
  for (int k = 0; k < NBATCH - 2; k += 2) {
#pragma unroll
    for (int b = 0; b < NB; ++b) B[b] = p[(k + 1) * NB + b];
    __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the adds
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      s = s + A[b].x;
      s = s + A[b].y;
      s = s + A[b].z;
      s = s + A[b].w;
    }
    // A is consumed before it is reloaded: without this the compiler hoists
    // the reload into fresh registers and copies them back every iteration.
    asm volatile("" : "+v"(s)::"memory");
#pragma unroll
    for (int b = 0; b < NB; ++b) A[b] = p[(k + 2) * NB + b];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      s = s + B[b].x;
      s = s + B[b].y;
      s = s + B[b].z;
      s = s + B[b].w;
    }
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) B[b] = p[(NBATCH - 1) * NB + b];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    s = s + A[b].x;
    s = s + A[b].y;
    s = s + A[b].z;
    s = s + A[b].w;
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    s = s + B[b].x;
    s = s + B[b].y;
    s = s + B[b].z;
    s = s + B[b].w;
  }
  return s;
}

// ---- float keys ---------------------------------------------------------------
// The key of a float is its bit pattern with the magnitude bits of negative
// values flipped: a monotone, self-inverse map onto the 32-bit integers, with
// -0.0 just below +0.0, so consecutive floats have consecutive keys.
constexpr int kSpecChunk = 128;  // terms per chunk of the speculative folds

__device__ __forceinline__ int float_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (int)(b ^ ((uint32_t)((int)b >> 31) >> 1));
}
__device__ __forceinline__ float key_float(int k) {
  return __uint_as_float((uint32_t)k ^ ((uint32_t)(k >> 31) >> 1));
}

// All waves of the workgroup: this wave's LDS accesses complete, then the
// workgroup barrier.  Outstanding global loads are not waited for.
__device__ __forceinline__ void wg_lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Two wave sums at once (any order; every lane returns them): DPP within
// each 16-lane row, then the four row sums read out as scalars.
__device__ __forceinline__ void wave_sum2(float& a, float& b) {
  a += __int_as_float(dpp_mov<0xB1>(__float_as_int(a)));   // quad_perm [1,0,3,2]
  b += __int_as_float(dpp_mov<0xB1>(__float_as_int(b)));
  a += __int_as_float(dpp_mov<0x4E>(__float_as_int(a)));   // quad_perm [2,3,0,1]
  b += __int_as_float(dpp_mov<0x4E>(__float_as_int(b)));
  a += __int_as_float(dpp_mov<0x124>(__float_as_int(a)));  // row_ror:4
  b += __int_as_float(dpp_mov<0x124>(__float_as_int(b)));
  a += __int_as_float(dpp_mov<0x128>(__float_as_int(a)));  // row_ror:8
  b += __int_as_float(dpp_mov<0x128>(__float_as_int(b)));
  const int ia = __float_as_int(a), ib = __float_as_int(b);
  a = (__int_as_float(__builtin_amdgcn_readlane(ia, 0)) + __int_as_float(__builtin_amdgcn_readlane(ia, 16))) +
      (__int_as_float(__builtin_amdgcn_readlane(ia, 32)) + __int_as_float(__builtin_amdgcn_readlane(ia, 48)));
  b = (__int_as_float(__builtin_amdgcn_readlane(ib, 0)) + __int_as_float(__builtin_amdgcn_readlane(ib, 16))) +
      (__int_as_float(__builtin_amdgcn_readlane(ib, 32)) + __int_as_float(__builtin_amdgcn_readlane(ib, 48)));
}

// The same fold over the first nb (1 <= nb <= NBMAX, the same in every lane)
// batches of NB float4: straight-line code whose only branches are the exits
// after each batch.  The read-ahead past the end re-reads the last batch.
template <int NBMAX, int NB = 4, int LA = 1>
__device__ __forceinline__ float seq_fold_lds_upto(const float4* p, int nb, float init) {
  nb = __builtin_amdgcn_readfirstlane(nb);
  float4 buf[LA + 1][NB];
  float s = init;
#pragma unroll
  for (int k = 0; k < LA && k < NBMAX; ++k) {
    const int kn = min(k, nb - 1);
#pragma unroll
    for (int b = 0; b < NB; ++b) buf[k][b] = p[kn * NB + b];
  }
#pragma unroll
  for (int k = 0; k < NBMAX; ++k) {
    if (k + LA < NBMAX) {
      const int kn = min(k + LA, nb - 1);
#pragma unroll
      for (int b = 0; b < NB; ++b) buf[(k + LA) % (LA + 1)][b] = p[kn * NB + b];
    }
    __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the adds
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float4 v = buf[k % (LA + 1)][b];
      s = s + v.x;
      s = s + v.y;
      s = s + v.z;
      s = s + v.w;
    }
    asm volatile("" : "+v"(s)::"memory");  // this batch is consumed before its buffer is reloaded
    if (k + 1 >= nb) break;
  }
  return s;
}

// ---- speculative exact fold by one wave ---------------------------------------
// The sequential fold init + p[0] + ... + p[128 NC - 1] with a dependent chain
// of 128 additions instead of 128 NC: the values are cut into NC chunks of 128,
// stored in LDS 132 floats apart (chunk c at p + kSwStride c, so the lane
// groups' broadcast reads fall in different banks).  Lanes [0, kSwLead) fold
// chunk 0 from init; the kSwCand(NC) lanes of group c >= 1 fold chunk c from
// consecutive floats (by key) around est[c], an
// estimate of the prefix p[0] + ... + p[128c - 1].  Then the true start of
// each chunk (the end of the one before) picks its lane's chain end when it
// lies in the window, and otherwise chunk c is folded again from the true
// start.  Every step is the sequential fold's own float addition, so the
// result is exactly the sequential fold's; the estimates only decide how often
// a refold happens.  All lanes return the result.
constexpr int kSwStride = 132;
template <int NC>
constexpr int kSwCand = 63 / (NC - 1);  // chunk 0's start is known: its group needs one lane
template <int NC>
constexpr int kSwLead = 64 - (NC - 1) * kSwCand<NC>;

template <int NC>
__device__ __forceinline__ float spec_fold_wave(const float* p, const float (&est)[NC], float init,
                                                int lane) {
  static_assert(NC >= 2 && NC <= 4, "two to four chunks");
  constexpr int W = kSwCand<NC>, L0 = kSwLead<NC>;
  const int c = lane < L0 ? 0 : 1 + (lane - L0) / W;
  int base[NC];
#pragma unroll
  for (int k = 1; k < NC; ++k)
    base[k] = min(max(float_key(est[k]), INT32_MIN + W / 2), INT32_MAX - (W - 1) + W / 2) - W / 2;
  float st = init;
#pragma unroll
  for (int k = 1; k < NC; ++k)
    if (c == k) st = key_float(base[k] + (lane - L0 - (k - 1) * W));
  const float* pc = p + kSwStride * c;
  const int ek = float_key(seq_fold_lds<kSpecChunk / 4, 4>((const float4*)pc, st));
  int ks = __builtin_amdgcn_readfirstlane(ek);  // lane 0: the end of chunk 0
#pragma unroll
  for (int k = 1; k < NC; ++k) {
    const uint32_t d = (uint32_t)ks - (uint32_t)__builtin_amdgcn_readfirstlane(base[k]);
    if (d < (uint32_t)W) {
      ks = __builtin_amdgcn_readlane(ek, L0 + (k - 1) * W + (int)d);
    } else {  // the start lies outside the window: fold chunk k again from it
      const float s = seq_fold_lds<kSpecChunk / 4, 4>((const float4*)(p + kSwStride * k), key_float(ks));
      ks = __builtin_amdgcn_readfirstlane(float_key(s));
    }
  }
  return key_float(ks);
}

// LDS floats of one wave's LayerNorm row (room for the chunked layout).
template <int PER>
constexpr bool kLnSpec = PER == 4 || PER == 6 || PER == 8;
template <int PER>
constexpr int kLnRow = kLnSpec<PER> ? kSwStride * (PER / 2) : PER * 64;

// The sequential fold -0.0 + v[0] + v[1] + ... of a row held by one wave
// (lane l: elements l + 64j in v[j]) through its LDS row zr.  Rows of 256,
// 384 or 512 elements fold as 2, 3 or 4 speculative chunks (spec_fold_wave,
// the estimates being float sums of the chunks), others strictly in order.
template <int PER>
__device__ __forceinline__ float fold_row_wave(const float (&v)[PER], float* zr, int lane) {
  if constexpr (kLnSpec<PER>) {
    constexpr int NC = PER / 2;
#pragma unroll
    for (int j = 0; j < PER; ++j) zr[kSwStride * (j >> 1) + lane + 64 * (j & 1)] = v[j];
    // Prefix estimates: est[c] = sum of chunks 0 .. c-1.
    float cs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c + 1 < NC; ++c) cs[c] = v[2 * c] + v[2 * c + 1];
    wave_sum2(cs[0], cs[1]);
    if constexpr (NC == 4) wave_sum2(cs[2], cs[3]);
    float est[NC];
    est[0] = 0.0f;
#pragma unroll
    for (int c = 1; c < NC; ++c) est[c] = est[c - 1] + cs[c - 1];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the row is in LDS
    __builtin_amdgcn_wave_barrier();
    const float r = spec_fold_wave<NC>(zr, est, -0.0f, lane);
    __builtin_amdgcn_wave_barrier();
    return r;
  } else {
#pragma unroll
    for (int j = 0; j < PER; ++j) zr[lane + 64 * j] = v[j];
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    const float r = seq_fold_lds<PER * 16>((const float4*)zr, -0.0f);
    __builtin_amdgcn_wave_barrier();
    return r;
  }
}

// ---- the opt-in fast-reduction order (decoder only) -----------------------------
// With MARIAN_HIP_FLAG_FAST_REDUCTIONS the decoder's LayerNorm sums and
// softmax denominators are not the reference's left-to-right folds but a
// tree: 64 lane partials (lane l adds elements l, l + 64, l + 128, ... in
// order, from 0.0), then an xor butterfly over lane distances 32, 16, 8, 4, 2
// and 1 (lane l adds lane l ^ dist's value to its own; addition commutes, so
// every lane ends with the same sum).  One wave, no LDS.

// The partial p (this lane's in-order sum) combined over the wave.
__device__ __forceinline__ float tree_combine_wave(float p) {
  p = p + __shfl_xor(p, 32, 64);
  p = p + xor_lane_f<16>(p);
  p = p + xor_lane_f<8>(p);
  p = p + xor_lane_f<4>(p);
  p = p + xor_lane_f<2>(p);
  p = p + xor_lane_f<1>(p);
  return p;
}

// The tree sum of a row held by one wave (lane l: elements l + 64j in v[j]).
template <int PER>
__device__ __forceinline__ float tree_sum_wave(const float (&v)[PER]) {
  float p = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) p = p + v[j];
  return tree_combine_wave(p);
}

// LayerNorm of the row z (lane l holds elements l + 64j) by one wave with
// normalize_row's sequential folds (tensor.rs:372-385); zr is the wave's LDS
// row (kLnRow<PER> floats).  Returns the normalized row in o.  FAST: the two
// sums in the tree order above instead (zr unused).
template <int PER, bool FAST = false>
__device__ __forceinline__ void ln_wave(const float (&z)[PER], float* zr, const float (&gv)[PER],
                                        const float (&bv)[PER], int lane, float (&o)[PER]) {
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
#pragma unroll
  for (int j = 0; j < PER; ++j) o[j] = ((z[j] - mean) * inv) * gv[j] + bv[j];
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
__device__ __forceinline__ float dequant_scale(float a, float w) { return 1.0f / (a * w); }
__device__ __forceinline__ float dequant_apply(int32_t acc, float inv, float b) { return (float)acc * inv + b; }
__device__ __forceinline__ float dequant(int32_t acc, float a, float w, float b) {
  return dequant_apply(acc, dequant_scale(a, w), b);
}

// Weights in MFMA fragment order: for the 16-column tile t and the 64-wide
// k-step s of an int8 matrix W[N, K] (K-contiguous), lane l's B fragment
// W[16t + l % 16][64s + 16(l / 16) .. +16] is stored at byte
// ((t * K/64 + s) * 64 + l) * 16, so a wave's fragment load reads 1 KB
// contiguously (row-major fragments touch 16 rows x 64 bytes; measured 2-3x
// slower to issue).  Tiles past N hold zeros.
__device__ __forceinline__ v4i frag_load(const int8_t* Wf, int tile, int ksteps, int s, int lane) {
  return *(const v4i*)(Wf + (((int64_t)tile * ksteps + s) * 64 + lane) * 16);
}

// Orderable 64-bit key: larger logit wins, equal logits prefer the lower id
// (the reference's strict '>' scan in ascending id order).  0 = no candidate.
// The scan starts from -inf at the first candidate and never takes a NaN, so
// NaN ranks with -inf (a row of only -inf/NaN logits yields its first
// candidate); -0.0 equals +0.0 under '>', so it is folded into +0.0.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t id) {
  v = (v != v) ? -INFINITY : v + 0.0f;
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
