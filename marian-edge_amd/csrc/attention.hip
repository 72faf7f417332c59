// attention.hip — variable-length multi-head attention: one single-wave
// workgroup per (query row, head), head_dim 64 or 48 (the reference's 384-wide,
// 8-head production model).
//
// Semantics of attention_into (tensor.rs:251-318): score_k = (q . k_k) * 1/sqrt(dh),
// softmax as max, exp(s - max), sum, multiply by 1/sum, then
// out = sum_k p_k v_k in key order.  Mapping onto the wave:
//   * K and V rows arrive by coalesced 16-byte raw buffer loads and pass
//     through a per-head LDS tile;
//   * scores: lane = key (keys lane, lane+64, ...), sequential 64-term dot
//     with q read from LDS as broadcasts;
//   * softmax: wave max, the C library's expf (ref_expf.h) per key, then the
//     denominator summed over the keys in order through LDS;
//   * PV: lane = output dim, keys accumulated in order (the reference order);
//     probabilities are read from LDS as broadcasts, four keys at a time.
// The score row never leaves the chip.  Sequences are packed (cu_seqlens), so
// there is no padding and no mask; keys beyond a row's count are never read.
// The three modes differ only in where a row's keys live: its own sequence
// (encoder self-attention / op-level varlen), the encoder output of its
// sequence (cross-attention at decode), or its per-sequence KV cache
// (decoder self-attention over steps 0..t).
#include "device_common.h"
#include "kernels.h"
#include <hip/hip_ext.h>

namespace mh {
namespace {

template <typename T>
struct Io;
template <>
struct Io<float> {
  static __device__ __forceinline__ float at(const void* p, int64_t i) {
    return ((const float*)p)[i];
  }
};
template <>
struct Io<uint16_t> {
  static __device__ __forceinline__ float at(const void* p, int64_t i) {
    return bf16_to_f32(((const uint16_t*)p)[i]);
  }
};

// K and V rows of one 64-key chunk move through a per-head LDS tile: 16
// coalesced float4 loads (four 256-byte rows per instruction) into registers,
// then stored as [key][dim].  Keys past the row's last key reload that last
// key, so every load is in bounds and every value finite.
constexpr int kKRow = kHeadDim + 4;  // padded LDS row (floats), 16-byte aligned

// 2^(i/32) table of ref_expf, staged into LDS by each workgroup.
__constant__ uint64_t kExp2Tab[32] = {MH_EXP2_TABLE_32};

template <typename T>
__device__ __forceinline__ float4 load_row4(const void* p, int64_t off) {
  if constexpr (sizeof(T) == 4) {
    return *(const float4*)((const float*)p + off);
  } else {
    const uint2 w = *(const uint2*)((const uint16_t*)p + off);
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xFFFF0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xFFFF0000u));
  }
}

// One head's K or V rows of a row (or sequence) as a raw buffer resource
// whose range ends where key nk_ld would start: a raw buffer load whose
// offset lies at or past the range's end returns zeros (the hardware range
// check on the VGPR offset), so a chunk's loads need no clamped addresses,
// only one 32-bit byte offset each (a lane part plus a uniform part).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kRawBufferWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rows(const void* p, int64_t elem0, int64_t ld, int nk_ld) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)((const T*)p + elem0), (short)0,
                                           (int)((int64_t)nk_ld * ld * (int64_t)sizeof(T)), kRawBufferWord3);
}

template <typename T>
__device__ __forceinline__ float4 load_rows4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 4) {
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
  } else {
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xFFFF0000u),
                       __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xFFFF0000u));
  }
}

// Lane l loads dims 4*(l%16)..+3 of keys first + l/16 + 4i (i < 16): VOFF is
// the lane's byte offset of key l/16, LDB the bytes per key row.  Keys past
// the resource's range read as zeros (with head_dim 48 the lanes past dim 47
// reload dims 44-47 into tile columns that are never read).
#define MH_LOAD_CHUNK(T, R, VOFF, LDB, FIRST, OUT) \
  _Pragma("unroll") for (int i_ = 0; i_ < 16; ++i_) OUT[i_] = load_rows4<T>((R), (VOFF) + (uint32_t)((FIRST) + 4 * i_) * (LDB));
#define MH_STORE_CHUNK(TILE, LANE, IN)                                                         \
  _Pragma("unroll") for (int i_ = 0; i_ < 16; ++i_)                                            \
      *(float4*)((TILE) + (((LANE) >> 4) + 4 * i_) * kKRow + ((LANE)&15) * 4) = IN[i_];

// The decode key range of row r (read before the device row count; rows past
// it read clamped stale ranges and are discarded): its first cached row and
// its count (cross-attention: the row's own count; self-attention: step + 1).
// Both values are requested together and taken by one empty asm, so neither
// load waits behind the other; the count is read from a valid address in
// either mode.
__device__ __forceinline__ void decode_key_range(const AttnArgs& a, int r, int64_t& key0, int& nk) {
  const int* nkp = a.row_nk ? a.row_nk + r : &kNoRowCount;
  int64_t k0 = a.row_key0[r];
  int nkv = *nkp;
  asm("" : "+v"(k0), "+v"(nkv));
  nkv = __builtin_amdgcn_readfirstlane(nkv);  // uniform again
  k0 = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(k0 >> 32)) << 32) |
                 (uint32_t)__builtin_amdgcn_readfirstlane((int)k0));
  nk = max(a.mode == ATT_CROSS ? nkv : a.step + 1, 1);
  key0 = min(max(k0, (int64_t)0), a.max_row - 1);
}

// PRE (two chunks only): all four K/V chunks are requested up front, so a
// decode row waits for one memory round trip after its key range is known.
template <int CH, typename T, bool PRE, int DH>
__global__ __launch_bounds__(64) void k_attention(AttnArgs a) {
  static_assert(DH == 64 || DH == 48, "head widths");
  static_assert(!PRE || CH == 2, "up-front loads hold two chunks");
  __shared__ __attribute__((aligned(16))) float tile[64 * kKRow];  // one K or V chunk
  __shared__ __attribute__((aligned(16))) float sP[CH * 64];        // exponentials, then probabilities
  __shared__ __attribute__((aligned(16))) float sQ[64];             // the query, read as broadcasts
  __shared__ uint64_t sTab[32];
  const int h = blockIdx.x % a.heads, r = blockIdx.x / a.heads;  // r < a.rows, the host bound
  const int lane = threadIdx.x;
  const uint64_t tab_v = kExp2Tab[lane & 31];

  int64_t key0;
  int nk;
  if (a.mode == ATT_SEQ) {
    const int sq = a.seq_of_row[r];
    key0 = a.cu[sq];
    nk = (int)(a.cu[sq + 1] - a.cu[sq]);
  } else {
    decode_key_range(a, r, key0, nk);
  }
  // A key range longer than this variant holds would overrun the score
  // registers: attend over the first CH*64 keys (flagged below for live rows).
  const bool too_long = nk > CH * 64;
  if (too_long) nk = CH * 64;
  const int nch = (nk + 63) >> 6;
  const int64_t kbase = key0 * a.ldkv + h * DH;

  // Keys of a stale row may run past the buffer: its last readable key.
  const int nk_ld = a.mode == ATT_SEQ ? nk : (int)min((int64_t)nk, a.max_row - key0);
  const __amdgpu_buffer_rsrc_t rk = head_rows<T>(a.k, kbase, a.ldkv, nk_ld);
  const __amdgpu_buffer_rsrc_t rv = head_rows<T>(a.v, kbase, a.ldkv, nk_ld);
  const uint32_t ldb = (uint32_t)a.ldkv * (uint32_t)sizeof(T);
  const uint32_t voff = (uint32_t)(lane >> 4) * ldb + (uint32_t)min((lane & 15) * 4, DH - 4) * (uint32_t)sizeof(T);

  // q of this head, one element per lane (copied to LDS for broadcasts),
  // requested first and waited for before the chunk loop (below): a wait
  // for it inside the loop, after a chunk's conditional prefetch, would
  // have to drain every load in flight.
  const int qv = __float_as_int(Io<T>::at(a.q, (int64_t)r * a.ldq + h * DH + min(lane, DH - 1)));
  // Chunk 0's V rows are loaded now (used after the softmax), then K.
  float4 vreg[16], kreg[16], kreg1[PRE ? 16 : 1], vreg1[PRE ? 16 : 1];
  MH_LOAD_CHUNK(T, rv, voff, ldb, 0, vreg)
  MH_LOAD_CHUNK(T, rk, voff, ldb, 0, kreg)
  if constexpr (PRE) {
    if (nch > 1) {
      MH_LOAD_CHUNK(T, rk, voff, ldb, 64, kreg1)
      MH_LOAD_CHUNK(T, rv, voff, ldb, 64, vreg1)
    }
  }
  const int n = a.rows_dev ? *a.rows_dev : a.rows;
  if (r >= n) return;
  if (too_long && threadIdx.x == 0 && a.err) *a.err = 2;
  asm volatile("" ::"v"(qv));  // q has arrived (the K/V loads stay in flight)
  sQ[lane] = __int_as_float(qv);  // published by the first barrier below

  // Scores: lane = key within the chunk, DH-term dot in dimension order.  The
  // next chunk's K rows are loaded while this chunk's dot runs.
  const float scale = 1.0f / sqrtf((float)DH);
  if (lane < 32) sTab[lane] = tab_v;  // published by the first barrier below
  float s[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    s[c] = -INFINITY;
    if (c < nch) {
      if (c > 0) __syncthreads();  // the previous chunk's rows have been read
      if constexpr (PRE) {
        if (c == 0) {
          MH_STORE_CHUNK(tile, lane, kreg)
        } else {
          MH_STORE_CHUNK(tile, lane, kreg1)
        }
      } else {
        MH_STORE_CHUNK(tile, lane, kreg)
        if (c + 1 < nch) {
          MH_LOAD_CHUNK(T, rk, voff, ldb, (c + 1) * 64, kreg)
        }
      }
      __syncthreads();
      float dot = -0.0f;
#pragma unroll
      for (int i0 = 0; i0 < DH; i0 += 16) {
        float kr[16], qs[16];
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
          const float4 v = *(const float4*)(tile + lane * kKRow + i0 + i);
          const float4 q4 = *(const float4*)(sQ + i0 + i);
          kr[i] = v.x;
          kr[i + 1] = v.y;
          kr[i + 2] = v.z;
          kr[i + 3] = v.w;
          qs[i] = q4.x;
          qs[i + 1] = q4.y;
          qs[i + 2] = q4.z;
          qs[i + 3] = q4.w;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) dot = dot + qs[i] * kr[i];
      }
      if (c * 64 + lane < nk) s[c] = dot * scale;
    }
  }
  // V rows of chunk 1 go into the now free K registers (chunk c uses vreg
  // for even c, kreg for odd c).
  if (!PRE && nch > 1) {
    MH_LOAD_CHUNK(T, rv, voff, ldb, 64, kreg)
  }
  float mloc = -INFINITY;
#pragma unroll
  for (int c = 0; c < CH; ++c) mloc = fmaxf(mloc, s[c]);
  const float mx = wave_max(mloc);
#pragma unroll
  for (int c = 0; c < CH; ++c)
    s[c] = (c < nch && c * 64 + lane < nk) ? ref_expf(s[c] - mx, sTab) : 0.0f;
  // Denominator in key order from 0.0 (softmax_in_place): the exponentials
  // pass through LDS and every lane folds them sequentially.  Keys past
  // the last hold +0.0, which leaves the (non-negative) sum unchanged.
  // With a.fast (decode only) the denominator takes the fast-reduction tree
  // order instead: lane l's keys l, 64 + l, ... in order from 0.0, then the
  // xor butterfly (tree_combine_wave).
  float sum = 0.0f;
  if (a.fast) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
      if (c < nch) sum = sum + s[c];
    sum = tree_combine_wave(sum);
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c)
      if (c < nch) sP[c * 64 + lane] = s[c];
    __syncthreads();
    if constexpr (CH <= 8) {
      sum = seq_fold_lds_upto<CH * 4>((const float4*)sP, nch * 4, 0.0f);
    } else {  // long ranges: a rolled loop keeps the code small
#pragma unroll 4
      for (int j = 0; j < nch * 64; j += 4) {
        const float4 v = *(const float4*)(sP + j);
        sum = sum + v.x;
        sum = sum + v.y;
        sum = sum + v.z;
        sum = sum + v.w;
      }
    }
  }
  const float inv = 1.0f / sum;
  // The probabilities replace the exponentials in LDS (this wave's fold
  // reads were issued before these writes and LDS keeps a wave's order).
#pragma unroll
  for (int c = 0; c < CH; ++c)
    if (c < nch) sP[c * 64 + lane] = s[c] * inv;

  // out_d = sum_j v[j][d] * p_j in key order; p_j is read from LDS as a
  // broadcast, four keys at a time; keys past the last have p = 0 and zero
  // values (or stale ones: p * v = +-0), and adding +-0 to a sum that
  // started from +0.0 leaves it bit-identical to skipping them.
  float o = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (c < nch) {
      __syncthreads();  // the tile's previous contents have been read
      if constexpr (PRE) {
        if (c == 0) {
          MH_STORE_CHUNK(tile, lane, vreg)
        } else {
          MH_STORE_CHUNK(tile, lane, vreg1)
        }
      } else if (c & 1) {
        MH_STORE_CHUNK(tile, lane, kreg)
        if (c + 2 < nch) {
          MH_LOAD_CHUNK(T, rv, voff, ldb, (c + 2) * 64, kreg)
        }
      } else {
        MH_STORE_CHUNK(tile, lane, vreg)
        if (c + 2 < nch) {
          MH_LOAD_CHUNK(T, rv, voff, ldb, (c + 2) * 64, vreg)
        }
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 64; u += 4) {
        const float4 p4 = *(const float4*)(sP + c * 64 + u);
        o = o + tile[u * kKRow + lane] * p4.x;
        o = o + tile[(u + 1) * kKRow + lane] * p4.y;
        o = o + tile[(u + 2) * kKRow + lane] * p4.z;
        o = o + tile[(u + 3) * kKRow + lane] * p4.w;
      }
    }
  }

  if (lane < DH) a.out[(int64_t)r * a.ldo + h * DH + lane] = o;
  if (a.qout) {  // static multiplier of the next layer (elementwise)
    if (lane < DH) a.qout[(int64_t)r * a.ldqout + h * DH + lane] = (int8_t)quantize_one(o, a.qmult);
    if (lane == 0 && h == 0) a.qa[r] = a.qmult;
  }
  // |max| of this head's slice: the consumer derives the row's quantization
  // multiplier from the maxima of all heads.
  const bool bad = lane < DH && !isfinite(o);
  const float m = wave_max(lane < DH ? fabsf(o) : 0.0f);
  if (lane == 0 && a.amax) a.amax[(int64_t)r * a.heads + h] = m;
  if (__any(bad) && lane == 0 && a.err) *a.err = 1;
}


// ---------------------------------------------------------------------------
// Self-attention of packed sequences (ATT_SEQ) with keys shared by the queries
// of a tile: one workgroup of kTileQ waves per (query tile, head), a tile
// being up to kTileQ consecutive query rows of one sequence.  The sequence's
// K rows of this head are staged in LDS once and read by every wave (one
// query per wave), 64 keys at a time; then its V rows, likewise.  Per query the arithmetic is
// k_attention's: lane = key for the sequential 64-term dots, wave max, the
// restated expf, the denominator folded in key order from 0.0 through LDS,
// PV in key order with lane = dimension.  Sequences of up to kTileMaxKeys.
// A sequence of at most kPairKeys keys is one tile of all its queries, two per
// wave (its 64-lane chunk would leave half the score lanes idle): lanes 0-31
// take query 2w and lanes 32-63 query 2w + 1, each half computing its query's
// scores (lane = key), maximum, exponentials and key-order denominator, and
// each lane the PV sums of dimensions l % 32 and l % 32 + 32 of its half's
// query, both in key order.  The arithmetic per query is unchanged.
// ---------------------------------------------------------------------------
constexpr int kTileQ = 16;          // queries (waves) per workgroup
constexpr int kTileMaxKeys = 256;   // keys staged in LDS
constexpr int kPairKeys = 32;       // sequences up to this length: two queries per wave

// Tiles of a sequence of L queries: one tile of the whole sequence when it is
// short enough for two queries per wave, else tiles of kTileQ queries.
__device__ __forceinline__ int seq_tile_count(int L) {
  return L <= 0 ? 0 : (L <= kPairKeys ? 1 : (L + kTileQ - 1) / kTileQ);
}

__global__ __launch_bounds__(1024) void k_seq_tiles(const uint32_t* cu, int nseq, uint32_t* tiles,
                                                    int cap) {
  // tiles[0] = count; tiles[1 + 2i] = sequence, tiles[2 + 2i] = first query.
  __shared__ int s_wsum[16];
  __shared__ int s_base;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int per = (nseq + 1023) / 1024;
  const int s0 = tid * per, s1 = min(s0 + per, nseq);
  int cnt = 0;
  for (int q = s0; q < s1; ++q) cnt += seq_tile_count((int)(cu[q + 1] - cu[q]));
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
    s_base = run;
  }
  __syncthreads();
  int pos = s_wsum[wave] + incl - cnt;
  for (int q = s0; q < s1; ++q) {
    const int L = (int)(cu[q + 1] - cu[q]);
    const int step = L <= kPairKeys ? kPairKeys : kTileQ;
    for (int q0 = 0; q0 < L; q0 += step, ++pos) {
      if (pos < cap) {
        tiles[1 + 2 * pos] = (uint32_t)q;
        tiles[2 + 2 * pos] = (uint32_t)q0;
      }
    }
  }
  if (tid == 0) tiles[0] = (uint32_t)min(s_base, cap);
}

// Two workgroups per CU: at most 64 VGPRs (eight waves per SIMD).
template <typename T, int DH>
__global__ __launch_bounds__(kTileQ * 64) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_attn_tiles(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float stage[64 * kKRow];            // one 64-key chunk
  __shared__ __attribute__((aligned(16))) float sPall[kTileQ * kTileMaxKeys];  // per-wave probabilities
  __shared__ __attribute__((aligned(16))) float sQall[2 * kTileQ * kHeadDim];  // per-query query rows
  __shared__ uint64_t sTab[32];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int h = blockIdx.x % a.heads, ti = blockIdx.x / a.heads;
  if (ti >= (int)a.tiles[0]) return;  // uniform: the list is shorter than its bound
  const int sq = (int)a.tiles[1 + 2 * ti], q0 = (int)a.tiles[2 + 2 * ti];
  const int64_t key0 = a.cu[sq];
  const int L = (int)(a.cu[sq + 1] - key0);
  // A range past kTileMaxKeys is cut to it (and flagged).
  const int Lc = min(L, kTileMaxKeys);
  const int nch = (Lc + 63) >> 6;
  const int lpad = (Lc + 7) & ~7;
  float* sP = sPall + w * kTileMaxKeys;
  const int64_t base = key0 * a.ldkv + h * DH;
  if (tid < 32) sTab[tid] = kExp2Tab[tid];
  if (L > Lc && tid == 0 && a.err) *a.err = 2;
  const float scale = 1.0f / sqrtf((float)DH);

  // Chunk rows: thread t moves float4 t % 16 of key t / 16 of the chunk; keys
  // past the last are zero.  The next chunk is requested while this one is used.
  auto ld = [&](const void* src, int c) {
    const int key = c * 64 + (tid >> 4);
    return key < Lc ? load_row4<T>(src, base + (int64_t)key * a.ldkv + min((tid & 15) * 4, DH - 4))
                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  };
  float* srow = stage + (tid >> 4) * kKRow + (tid & 15) * 4;

  if (L <= kPairKeys) {  // the whole sequence, two queries per wave (q0 = 0)
    const int hf = lane >> 5, kl = lane & 31;
    const int qi = 2 * w + hf;  // this half's query
    const bool qlive = qi < L;
    *(float4*)srow = ld(a.k, 0);
    for (int i = tid; i < L * kHeadDim; i += kTileQ * 64) {
      const int q = i / kHeadDim, d = i % kHeadDim;
      if (d < DH) sQall[i] = Io<T>::at(a.q, (key0 + q) * a.ldq + h * DH + d);
    }
    const float4 vpre = ld(a.v, 0);
    __syncthreads();  // K rows, queries and the expf table are in LDS
    // Scores: lane = key, the DH-term dot in dimension order (the query read
    // from LDS, one address per half).
    float sc = -INFINITY;
    if (qlive) {
      const float* kr = stage + min(kl, Lc - 1) * kKRow;
      const float* sQ = sQall + qi * kHeadDim;
      float dot = -0.0f;
#pragma unroll
      for (int i = 0; i < DH; i += 4) {
        const float4 kk = *(const float4*)(kr + i);
        const float4 qq = *(const float4*)(sQ + i);
        dot = dot + qq.x * kk.x;
        dot = dot + qq.y * kk.y;
        dot = dot + qq.z * kk.z;
        dot = dot + qq.w * kk.w;
      }
      if (kl < Lc) sc = dot * scale;
    }
    const float mx = half_wave_max(sc);
    const float e = qlive && kl < Lc ? ref_expf(sc - mx, sTab) : 0.0f;
    // The half's exponentials in key order (+0.0 past the last key), folded
    // from 0.0 by each of its lanes; then p = e / sum.
    float* sPh = sP + hf * (kTileMaxKeys / 2);
    sPh[kl] = e;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes land
    __builtin_amdgcn_wave_barrier();
    const float inv = 1.0f / seq_fold_lds_upto<kPairKeys / 16>((const float4*)sPh, (Lc + 15) >> 4, 0.0f);
    __builtin_amdgcn_wave_barrier();
    sPh[kl] = e * inv;
    __syncthreads();  // every wave has read the K rows
    *(float4*)srow = vpre;
    __syncthreads();  // V rows (zero past the last key) and this wave's p are in LDS
    if (!qlive) return;
    // PV: dimensions kl and kl + 32 of the half's query, each a key-order sum
    // over batches of 8 keys (past the last key p is +0 and the rows are zero).
    const int nbat = __builtin_amdgcn_readfirstlane((Lc + 7) >> 3);  // 1..4
    const float* sv = stage + kl;
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int bt = 0; bt < kPairKeys / 8; ++bt) {
      float v0[8], v1[8];
      float4 pp[2];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v0[i] = sv[(bt * 8 + i) * kKRow];
        v1[i] = sv[(bt * 8 + i) * kKRow + 32];
      }
      pp[0] = *(const float4*)(sPh + bt * 8);
      pp[1] = *(const float4*)(sPh + bt * 8 + 4);
      const float pk[8] = {pp[0].x, pp[0].y, pp[0].z, pp[0].w, pp[1].x, pp[1].y, pp[1].z, pp[1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        o0 = o0 + v0[i] * pk[i];
        o1 = o1 + v1[i] * pk[i];
      }
      if (bt + 1 >= nbat) break;
    }
    const int64_t orow = key0 + qi;
    const bool d1 = kl + 32 < DH;  // kl < DH always (DH >= 48)
    a.out[orow * a.ldo + h * DH + kl] = o0;
    if (d1) a.out[orow * a.ldo + h * DH + kl + 32] = o1;
    if (a.qout) {
      a.qout[orow * a.ldqout + h * DH + kl] = (int8_t)quantize_one(o0, a.qmult);
      if (d1) a.qout[orow * a.ldqout + h * DH + kl + 32] = (int8_t)quantize_one(o1, a.qmult);
      if (kl == 0 && h == 0) a.qa[orow] = a.qmult;
    }
    const bool bad = !isfinite(o0) || (d1 && !isfinite(o1));
    if (__any(bad) && lane == 0 && a.err) *a.err = 1;
    return;
  }

  const int nq = min(kTileQ, L - q0);
  float4 pre = ld(a.k, 0);
  const bool live = w < nq;
  const int row = (int)key0 + q0 + w;
  const float* sQ = sQall + w * kHeadDim;
  if (live && lane < DH) sQall[w * kHeadDim + lane] = Io<T>::at(a.q, (int64_t)row * a.ldq + h * DH + lane);

  // Scores: lane = key of the chunk, DH-term dot in dimension order.
  float sc[kTileMaxKeys / 64];
#pragma unroll
  for (int c = 0; c < kTileMaxKeys / 64; ++c) {
    sc[c] = -INFINITY;
    if (c < nch) {
      if (c > 0) __syncthreads();  // every wave has read the previous chunk
      *(float4*)srow = pre;
      __syncthreads();
      pre = c + 1 < nch ? ld(a.k, c + 1) : ld(a.v, 0);
      if (live) {
        const float* kr = stage + min(lane, Lc - 1 - c * 64) * kKRow;
        // The query is read from LDS as broadcasts (published by the barrier above).
        float dot = -0.0f;
#pragma unroll
        for (int i = 0; i < DH; i += 4) {
          const float4 kk = *(const float4*)(kr + i);
          const float4 qq = *(const float4*)(sQ + i);
          dot = dot + qq.x * kk.x;
          dot = dot + qq.y * kk.y;
          dot = dot + qq.z * kk.z;
          dot = dot + qq.w * kk.w;
        }
        if (c * 64 + lane < Lc) sc[c] = dot * scale;
      }
    }
  }
  // Softmax of each live wave's query: max, expf, the denominator folded in
  // key order from 0.0 (entries past the last key are +0.0), then p = e / sum.
  if (live) {
    float mloc = -INFINITY;
#pragma unroll
    for (int c = 0; c < kTileMaxKeys / 64; ++c) mloc = fmaxf(mloc, sc[c]);
    const float mx = wave_max(mloc);
#pragma unroll
    for (int c = 0; c < kTileMaxKeys / 64; ++c) {
      if (c < nch) {
        sc[c] = c * 64 + lane < Lc ? ref_expf(sc[c] - mx, sTab) : 0.0f;
        sP[c * 64 + lane] = sc[c];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes land
    __builtin_amdgcn_wave_barrier();
    const float inv = 1.0f / seq_fold_lds_upto<kTileMaxKeys / 16>((const float4*)sP, (Lc + 15) >> 4, 0.0f);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < kTileMaxKeys / 64; ++c)
      if (c < nch) sP[c * 64 + lane] = sc[c] * inv;
  }

  // out_d = sum_k v_k[d] * p_k in key order, chunk by chunk, in batches of 8
  // keys read one batch ahead (past the last key p is +0 and the rows are
  // zero, so the added products are +0).
  float o = 0.0f;
#pragma unroll
  for (int c = 0; c < kTileMaxKeys / 64; ++c) {
    if (c < nch) {
      __syncthreads();  // every wave has read the previous chunk (and its probabilities are in LDS)
      *(float4*)srow = pre;
      __syncthreads();
      if (c + 1 < nch) pre = ld(a.v, c + 1);
      if (live) {
        // Straight-line batches of 8 keys with an exit after each: every read
        // has a constant offset, so no address register is rewritten while a
        // read into it is pending.  Reads stay inside the staged chunk.
        const int nbat = __builtin_amdgcn_readfirstlane(min(64, lpad - c * 64) >> 3);  // >= 1
        const float* sv = stage + lane;
        const float* pc = sP + c * 64;
        float v[2][8];
        float4 p[2][2];
        auto load8 = [&](int k0, float (&vv)[8], float4 (&pp)[2]) {
#pragma unroll
          for (int i = 0; i < 8; ++i) vv[i] = sv[(k0 + i) * kKRow];
          pp[0] = *(const float4*)(pc + k0);
          pp[1] = *(const float4*)(pc + k0 + 4);
        };
        load8(0, v[0], p[0]);
#pragma unroll
        for (int bt = 0; bt < 8; ++bt) {
          if (bt + 1 < 8) load8((bt + 1) * 8, v[(bt + 1) & 1], p[(bt + 1) & 1]);
          __builtin_amdgcn_sched_barrier(0);
          const float(&vv)[8] = v[bt & 1];
          const float4(&pp)[2] = p[bt & 1];
          o = o + vv[0] * pp[0].x;
          o = o + vv[1] * pp[0].y;
          o = o + vv[2] * pp[0].z;
          o = o + vv[3] * pp[0].w;
          o = o + vv[4] * pp[1].x;
          o = o + vv[5] * pp[1].y;
          o = o + vv[6] * pp[1].z;
          o = o + vv[7] * pp[1].w;
          asm volatile("" : "+v"(o)::"memory");  // this batch is consumed before its buffer is reloaded
          if (bt + 1 >= nbat) break;
        }
      }
    }
  }
  if (!live) return;
  if (lane < DH) a.out[(int64_t)row * a.ldo + h * DH + lane] = o;
  if (a.qout) {
    if (lane < DH) a.qout[(int64_t)row * a.ldqout + h * DH + lane] = (int8_t)quantize_one(o, a.qmult);
    if (lane == 0 && h == 0) a.qa[row] = a.qmult;
  }
  const bool bad = lane < DH && !isfinite(o);
  if (__any(bad) && lane == 0 && a.err) *a.err = 1;
}

// ---------------------------------------------------------------------------
// Decode attention over long key ranges (ATT_CROSS / ATT_SELF, 129 to 512
// keys): one workgroup of W = blockDim.x / 64 waves (3 to 8, the launch's key
// bound in 64-key chunks) per (row, head); wave w owns the keys
// [64w, 64w + 64) of the row.  Every wave requests its keys' K rows (lane =
// key, the head's 64 values in 16 float4) and V values (lane = dimension, one
// value per key) before anything else, so a row's whole key range is one
// memory round trip instead of one per 64-key chunk.  The arithmetic is
// k_attention's, in the reference order:
//   * scores: lane = key, the 64-term dot in dimension order from -0.0, the
//     query read from the wave's LDS copy as broadcasts;
//   * max over the workgroup (waves' maxima through LDS), the C library's
//     expf, the denominator folded in key order from 0.0 by wave 0 over the
//     exponentials in LDS (with FAST: the tree order, as in k_attention);
//   * PV: out_d = sum_k p_k v_k[d] in key order.  Each wave forms its keys'
//     products (lane = dimension, p read back from LDS as broadcasts), then the
//     running sums pass from wave to wave in key order through LDS, one
//     barrier per 64-key chunk, each wave adding its 64 products in order.
// Keys past the row's count have p = 0 (their values read as zeros through
// the buffer resource's range), so their products are +0 and leave the sums,
// which start from +0.0 and so are never -0.0, unchanged.
// The workgroup holds its waves through these dependent phases, so it pays
// where few (row, head) pairs leave the chip idle; with many, the one-wave
// kernel keeps more loads in flight per CU (launch_attention chooses).
// ---------------------------------------------------------------------------
constexpr int kLongWaves = 8;  // the most waves per workgroup
constexpr int kLongMaxKeys = 64 * kLongWaves;
constexpr int kLongMaxPairs = 512;  // (row, head) pairs up to which it runs

template <int DH, bool FAST>
__global__ __launch_bounds__(64 * kLongWaves) void k_attn_long(AttnArgs a) {
  static_assert(DH == 64 || DH == 48, "head widths");
  __shared__ __attribute__((aligned(16))) float sE[kLongMaxKeys];  // exponentials of the keys
  __shared__ float sO[64];                                          // the PV relay
  __shared__ __attribute__((aligned(16))) float sQw[kLongWaves][64];  // each wave's copy of the query
  __shared__ float sMax[kLongWaves];
  __shared__ float sInv;
  __shared__ uint64_t sTab[32];
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int nw = blockDim.x >> 6;  // 3..kLongWaves, set by the launch
  const int h = blockIdx.x % a.heads, r = blockIdx.x / a.heads;  // r < a.rows, the host bound
  const uint64_t tab_v = kExp2Tab[lane & 31];

  int64_t key0;
  int nk;
  decode_key_range(a, r, key0, nk);
  const bool too_long = nk > 64 * nw;
  if (too_long) nk = 64 * nw;
  const int nk_ld = (int)min((int64_t)nk, a.max_row - key0);  // readable rows
  const int nch = (nk + 63) >> 6;
  const int kc = 64 * w;         // this wave's first key
  const bool mine = kc < nk;     // uniform per wave
  const int64_t kbase = key0 * a.ldkv + h * DH;

  f4v kr[DH / 4];
  float vv[64];
  if (mine) {
    const int key = min(kc + lane, nk_ld - 1);
#pragma unroll
    for (int i = 0; i < DH / 4; ++i) kr[i] = *(const f4v*)((const float*)a.k + kbase + (int64_t)key * a.ldkv + 4 * i);
    // V: one raw buffer load per key, zeros past the readable keys.
    const __amdgpu_buffer_rsrc_t rv = head_rows<float>(a.v, kbase, a.ldkv, nk_ld);
    const uint32_t ldb = (uint32_t)a.ldkv * 4u, voff = (uint32_t)min(lane, DH - 1) * 4u;
#pragma unroll
    for (int j = 0; j < 64; ++j)
      vv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, voff + (uint32_t)(kc + j) * ldb, 0, 0));
  }
  const int qv = __float_as_int(((const float*)a.q)[(int64_t)r * a.ldq + h * DH + min(lane, DH - 1)]);
  const int n = a.rows_dev ? *a.rows_dev : a.rows;
  if (r >= n) return;  // the whole workgroup alike
  if (too_long && tid == 0 && a.err) *a.err = 2;
  if (tid < 32) sTab[tid] = tab_v;
  float* sQ = sQw[w];
  sQ[lane] = __int_as_float(qv);  // this wave's own copy: its reads below follow in LDS order

  // ---- scores and the row maximum ----
  const float scale = 1.0f / sqrtf((float)DH);
  const bool valid = mine && kc + lane < nk;
  float sc = -INFINITY;
  if (mine) {
    float dot = -0.0f;
#pragma unroll
    for (int i = 0; i < DH; i += 4) {  // the query read as LDS broadcasts
      const float4 q4 = *(const float4*)(sQ + i);
      dot = dot + q4.x * kr[i >> 2][0];
      dot = dot + q4.y * kr[i >> 2][1];
      dot = dot + q4.z * kr[i >> 2][2];
      dot = dot + q4.w * kr[i >> 2][3];
    }
    if (valid) sc = dot * scale;
  }
  const float wmax = wave_max(sc);
  if (lane == 0) sMax[w] = wmax;
  __syncthreads();  // also publishes sTab
  float mx = sMax[0];
  for (int i = 1; i < nw; ++i) mx = fmaxf(mx, sMax[i]);
  const float e = valid ? ref_expf(sc - mx, sTab) : 0.0f;
  if (mine) sE[kc + lane] = e;

  // ---- denominator (wave 0) ----
  __syncthreads();  // every exponential is in LDS
  if (w == 0) {
    float sum;
    if constexpr (FAST) {
      sum = 0.0f;  // lane l: keys l, 64 + l, ... in order from 0.0, then the butterfly
      for (int c = 0; c < nch; ++c) sum = sum + sE[64 * c + lane];
      sum = tree_combine_wave(sum);
    } else {
      // keys in order from 0.0, whole batches of 16 (zeros past the last key)
      sum = seq_fold_lds_upto<kLongMaxKeys / 16>((const float4*)sE, (nk + 15) >> 4, 0.0f);
    }
    if (lane == 0) sInv = 1.0f / sum;
  }
  __syncthreads();
  const float inv = sInv;

  // ---- PV: products, then the in-order relay across the waves ----
  float o = 0.0f;
  if (mine) {
    // p of key kc + lane replaces its exponential (wave 0's fold has read
    // them all: the barrier above), read back as LDS broadcasts.
    sE[kc + lane] = e * inv;
#pragma unroll
    for (int j = 0; j < 64; j += 4) {
      const float4 p4 = *(const float4*)(sE + kc + j);
      vv[j] = vv[j] * p4.x;
      vv[j + 1] = vv[j + 1] * p4.y;
      vv[j + 2] = vv[j + 2] * p4.z;
      vv[j + 3] = vv[j + 3] * p4.w;
    }
  }
  for (int c = 0; c < nch; ++c) {  // nch is uniform over the workgroup
    if (w == c) {
      o = c == 0 ? 0.0f : sO[lane];
#pragma unroll
      for (int j = 0; j < 64; ++j) o = o + vv[j];
      if (c + 1 < nch) sO[lane] = o;
    }
    if (c + 1 < nch) __syncthreads();
  }
  if (w != nch - 1) return;
  if (lane < DH) a.out[(int64_t)r * a.ldo + h * DH + lane] = o;
  const bool bad = lane < DH && !isfinite(o);
  const float m = wave_max(lane < DH ? fabsf(o) : 0.0f);
  if (lane == 0 && a.amax) a.amax[(int64_t)r * a.heads + h] = m;
  if (__any(bad) && lane == 0 && a.err) *a.err = 1;
}

// ev_start / ev_stop (optional) are recorded by the launch's own dispatch.
template <int CH, typename T, bool PRE>
hipError_t launch_t(const AttnArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  auto kern = a.head_dim == 48 ? k_attention<CH, T, PRE, 48> : k_attention<CH, T, PRE, 64>;
  if (ev0 || ev1)
    hipExtLaunchKernelGGL(kern, dim3(a.heads * a.rows), dim3(64), 0, s, ev0, ev1, 0, a);
  else
    hipLaunchKernelGGL(kern, dim3(a.heads * a.rows), dim3(64), 0, s, a);
  return hipGetLastError();
}

template <int CH, bool PRE = false>
hipError_t launch_ch(const AttnArgs& a, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  return a.bf16 ? launch_t<CH, uint16_t, PRE>(a, s, ev0, ev1) : launch_t<CH, float, PRE>(a, s, ev0, ev1);
}

template <int DH, bool FAST>
hipError_t launch_long(const AttnArgs& a, dim3 grid, dim3 block, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (ev0 || ev1)
    hipExtLaunchKernelGGL((k_attn_long<DH, FAST>), grid, block, 0, s, ev0, ev1, 0, a);
  else
    hipLaunchKernelGGL((k_attn_long<DH, FAST>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <typename T>
void launch_tiles(const AttnArgs& a, dim3 grid, dim3 block, hipStream_t s) {
  if (a.head_dim == 48)
    hipLaunchKernelGGL((k_attn_tiles<T, 48>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((k_attn_tiles<T, 64>), grid, block, 0, s, a);
}

}  // namespace

int seq_tiles_bound(int rows, int nseq) { return (rows + kTileQ - 1) / kTileQ + nseq; }

hipError_t launch_seq_tiles(const uint32_t* cu, int nseq, uint32_t* tiles, int cap, hipStream_t s) {
  if (nseq <= 0 || nseq > 16 * 1024 || cap <= 0 || !cu || !tiles) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_seq_tiles, dim3(1), dim3(1024), 0, s, cu, nseq, tiles, cap);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop) {
  if (a.rows <= 0) return hipSuccess;
  if (a.fast && a.mode == ATT_SEQ) return hipErrorInvalidValue;  // the encoder keeps the reference order
  if (a.heads <= 0 || a.heads > 16 || a.max_keys <= 0 || !a.out || (a.head_dim != 64 && a.head_dim != 48) ||
      (int64_t)a.rows * a.heads > 0x7fffffff)
    return hipErrorInvalidValue;
  if (a.qout && (!a.qa || a.ldqout < (int64_t)a.heads * a.head_dim || !(a.qmult > 0.0f) ||
                 !(a.qmult < __builtin_huge_valf())))
    return hipErrorInvalidValue;
  // Packed self-attention with a tile list: keys staged once per tile.
  if (a.mode == ATT_SEQ && a.tiles && a.tiles_cap > 0 && a.max_keys <= kTileMaxKeys) {
    if ((int64_t)a.tiles_cap * a.heads > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid(a.tiles_cap * a.heads), block(kTileQ * 64);
    if (a.bf16)
      launch_tiles<uint16_t>(a, grid, block, s);
    else
      launch_tiles<float>(a, grid, block, s);
    return hipGetLastError();
  }
  // Decode launches cover few rows: one round trip per row matters more
  // than occupancy.  Encoder launches keep the lighter register budget.
  hipEvent_t e0 = ev_start, e1 = ev_stop;
  // Up to 128 keys: with at most kLongMaxPairs (row, head) pairs, every chunk
  // requested up front (one round trip, one wave per SIMD); with more, the
  // one-chunk-ahead variant, whose two waves per SIMD keep more pairs going.
  if (a.max_keys <= 128)
    return a.mode == ATT_SEQ || a.rows * a.heads > kLongMaxPairs ? launch_ch<2>(a, s, e0, e1)
                                                                 : launch_ch<2, true>(a, s, e0, e1);
  if (a.max_keys <= kLongMaxKeys && a.mode != ATT_SEQ && !a.bf16 && !a.qout &&
      a.rows * a.heads <= kLongMaxPairs) {
    const dim3 grid(a.rows * a.heads), block(64 * ((a.max_keys + 63) / 64));
    if (a.head_dim == 64)
      return a.fast ? launch_long<64, true>(a, grid, block, s, e0, e1) : launch_long<64, false>(a, grid, block, s, e0, e1);
    return a.fast ? launch_long<48, true>(a, grid, block, s, e0, e1) : launch_long<48, false>(a, grid, block, s, e0, e1);
  }
  if (a.max_keys <= 512) return launch_ch<8>(a, s, e0, e1);
  if (a.max_keys <= 1024) return launch_ch<16>(a, s, e0, e1);
  if (a.max_keys <= 4096) return launch_ch<64>(a, s, e0, e1);
  return hipErrorInvalidValue;
}

}  // namespace mh
