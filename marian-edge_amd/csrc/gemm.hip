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

namespace mh {
namespace {

constexpr int kSkinnyRows = 64;     // rows per pass (A chunk in LDS)
constexpr int kSkinnyKChunk = 512;  // K per pass
constexpr int kSkinnyLds = kSkinnyKChunk + 16;  // padded LDS row (bytes)
constexpr int kSkinnyCols = 64;     // columns per workgroup (4 waves x 16)

constexpr int kTile = 128;
constexpr int kTileK = 64;
constexpr int kTileLds = kTileK + 16;  // padded LDS row (bytes)

__device__ __forceinline__ v4i zero4() { return v4i{0, 0, 0, 0}; }

// ---------------------------------------------------------------------------
// Skinny GEMM: one workgroup = 4 waves = 64 output columns.  The 16 columns of
// a wave are held as MFMA B fragments in registers for a whole K chunk, A
// streams through LDS 64 rows at a time, so each weight byte is read once per
// 64 rows (once per decode step for the usual M <= 64).
// ---------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256) void k_gemm_skinny(GemmArgs g, Epilogue e) {
  __shared__ __attribute__((aligned(16))) int8_t sA[kSkinnyRows * kSkinnyLds];
  __shared__ uint64_t sKey[4][kSkinnyRows];
  const int M = g.M_dev ? *g.M_dev : g.M;
  if (M <= 0) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ncol = blockIdx.x * kSkinnyCols + wave * 16 + (lane & 15);
  const bool col_ok = ncol < g.N;
  const int kq = (lane >> 4) * 16;

  for (int m0 = 0; m0 < M; m0 += kSkinnyRows) {
    v4i acc[4] = {zero4(), zero4(), zero4(), zero4()};
    for (int k0 = 0; k0 < g.K; k0 += kSkinnyKChunk) {
      const int kc = min(kSkinnyKChunk, g.K - k0);
      const int ksteps = kc >> 6;
      v4i bf[8];
      const int8_t* wrow = g.W + (int64_t)(col_ok ? ncol : 0) * g.K + k0 + kq;
#pragma unroll
      for (int s = 0; s < 8; ++s)
        bf[s] = (s < ksteps && col_ok) ? *(const v4i*)(wrow + s * 64) : zero4();
      __syncthreads();  // previous chunk's LDS reads are done
      const int cpr = kc >> 4;  // 16-byte chunks per row
      for (int c = tid; c < kSkinnyRows * cpr; c += 256) {
        const int row = c / cpr, cc = c - row * cpr;
        const int m = m0 + row;
        v4i v = zero4();
        if (m < M) v = *(const v4i*)(g.A + (int64_t)m * g.lda + k0 + cc * 16);
        *(v4i*)(sA + row * kSkinnyLds + cc * 16) = v;
      }
      __syncthreads();
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        if (m0 + ms * 16 < M) {
          const int8_t* arow = sA + (ms * 16 + (lane & 15)) * kSkinnyLds + kq;
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            if (s < ksteps) {
              const v4i af = *(const v4i*)(arow + s * 64);
              acc[ms] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[s], acc[ms], 0, 0, 0);
            }
          }
        }
      }
    }

    // Epilogue.  Lane l holds rows 4*(l/16)+r (r = 0..3) of column l%16.
    if (MODE == EPI_ARGMAX) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        if (m0 + ms * 16 < M) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + ms * 16 + (lane >> 4) * 4 + r;
            uint64_t key = 0;
            if (m < M && col_ok) {
              const float y = dequant(acc[ms][r], g.a[m], g.wmult[ncol], g.bias[ncol]);
              const bool masked = !(e.flags & 2u) && generation_masked((uint32_t)ncol);
              if (e.logits) e.logits[(int64_t)m * e.ldl + ncol] = masked ? -INFINITY : y;
              if (!masked && y == y) key = argmax_key(y, (uint32_t)ncol);
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
              const uint64_t o = shfl_xor_u64(key, off);
              key = o > key ? o : key;
            }
            if ((lane & 15) == 0) sKey[wave][ms * 16 + (lane >> 4) * 4 + r] = key;
          }
        }
      }
      __syncthreads();
      if (tid < kSkinnyRows && m0 + tid < M) {
        uint64_t best = sKey[0][tid];
#pragma unroll
        for (int w = 1; w < 4; ++w) best = sKey[w][tid] > best ? sKey[w][tid] : best;
        e.partials[(int64_t)(m0 + tid) * e.partial_ld + blockIdx.x] = best;
      }
    } else {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        if (m0 + ms * 16 < M) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + ms * 16 + (lane >> 4) * 4 + r;
            if (m < M && col_ok) {
              const int32_t iv = acc[ms][r];
              float y = dequant(iv, g.a[m], g.wmult[ncol], g.bias[ncol]);
              if (e.relu) y = y > 0.0f ? y : 0.0f;
              if (MODE == EPI_QKV_CACHE) {
                if (ncol < e.d) {
                  e.out[(int64_t)m * e.ldo + ncol] = y;
                } else {
                  const int64_t crow = e.kv_base[e.act[m]] + e.step;
                  if (ncol < 2 * e.d)
                    e.kcache[crow * e.d + (ncol - e.d)] = y;
                  else
                    e.vcache[crow * e.d + (ncol - 2 * e.d)] = y;
                }
              } else {
                if (e.out) e.out[(int64_t)m * e.ldo + ncol] = y;
                if (e.out_i32) e.out_i32[(int64_t)m * e.ldi + ncol] = iv;
              }
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Tile GEMM: 128x128 output tile per workgroup, 4 waves in a 2x2 grid each
// owning 64x64 (4x4 MFMA tiles), K in steps of 64 double-buffered through LDS
// (global -> registers -> LDS, next step's loads in flight during the MFMAs).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_gemm_tile(GemmArgs g, Epilogue e) {
  __shared__ __attribute__((aligned(16))) int8_t sA[2][kTile * kTileLds];
  __shared__ __attribute__((aligned(16))) int8_t sB[2][kTile * kTileLds];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
  const int M = g.M, N = g.N, K = g.K;

  v4i ra[2], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * 256, row = c >> 2, col = (c & 3) * 16;
      const int m = m0 + row, n = n0 + row;
      ra[i] = m < M ? *(const v4i*)(g.A + (int64_t)m * g.lda + k0 + col) : zero4();
      rb[i] = n < N ? *(const v4i*)(g.W + (int64_t)n * K + k0 + col) : zero4();
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * 256, row = c >> 2, col = (c & 3) * 16;
      *(v4i*)(sA[buf] + row * kTileLds + col) = ra[i];
      *(v4i*)(sB[buf] + row * kTileLds + col) = rb[i];
    }
  };

  v4i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = zero4();

  gload(0);
  lstore(0);
  __syncthreads();
  int cur = 0;
  const int kq = (lane >> 4) * 16;
  for (int k0 = 0; k0 < K; k0 += kTileK) {
    const bool more = k0 + kTileK < K;
    if (more) gload(k0 + kTileK);
    v4i af[4], bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *(const v4i*)(sA[cur] + (wm * 64 + i * 16 + (lane & 15)) * kTileLds + kq);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bfr[j] = *(const v4i*)(sB[cur] + (wn * 64 + j * 16 + (lane & 15)) * kTileLds + kq);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bfr[j], acc[i][j], 0, 0, 0);
    if (more) {
      lstore(cur ^ 1);
      __syncthreads();
      cur ^= 1;
    }
  }

#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + j * 16 + (lane & 15);
    if (n >= N) continue;
    const float wmul = g.wmult[n], bias = g.bias[n];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (m < M) {
          const int32_t iv = acc[i][j][r];
          float y = dequant(iv, g.a[m], wmul, bias);
          if (e.relu) y = y > 0.0f ? y : 0.0f;
          if (e.out) e.out[(int64_t)m * e.ldo + n] = y;
          if (e.out_i32) e.out_i32[(int64_t)m * e.ldi + n] = iv;
        }
      }
    }
  }
}

}  // namespace

int skinny_groups(int N) { return (N + kSkinnyCols - 1) / kSkinnyCols; }

hipError_t launch_gemm_skinny(const GemmArgs& g, int mode, const Epilogue& e, hipStream_t s) {
  if (g.K <= 0 || g.K % 64 || g.N <= 0) return hipErrorInvalidValue;
  if (!g.M_dev && g.M <= 0) return hipSuccess;
  const dim3 grid(skinny_groups(g.N)), block(256);
  switch (mode) {
    case EPI_STORE:
      hipLaunchKernelGGL(k_gemm_skinny<EPI_STORE>, grid, block, 0, s, g, e);
      break;
    case EPI_QKV_CACHE:
      hipLaunchKernelGGL(k_gemm_skinny<EPI_QKV_CACHE>, grid, block, 0, s, g, e);
      break;
    case EPI_ARGMAX:
      hipLaunchKernelGGL(k_gemm_skinny<EPI_ARGMAX>, grid, block, 0, s, g, e);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemm_tile(const GemmArgs& g, const Epilogue& e, hipStream_t s) {
  if (g.K <= 0 || g.K % 64 || g.N <= 0 || g.M_dev) return hipErrorInvalidValue;
  if (g.M <= 0) return hipSuccess;
  const dim3 grid((g.N + kTile - 1) / kTile, (g.M + kTile - 1) / kTile), block(256);
  hipLaunchKernelGGL(k_gemm_tile, grid, block, 0, s, g, e);
  return hipGetLastError();
}

hipError_t launch_gemm_store(const GemmArgs& g, const Epilogue& e, hipStream_t s) {
  if (g.M_dev || g.M <= kSkinnyRows) return launch_gemm_skinny(g, EPI_STORE, e, s);
  return launch_gemm_tile(g, e, s);
}

}  // namespace mh
