// oracle.cpp — CPU restatement of marian-cpu's Q8 greedy translation path.
//
// TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline).  The
// product library never links or calls this file.  See oracle.h for the list
// of reference functions each routine restates.
//
// Build: oracle/Makefile (gcc, -O3 -ffp-contract=off, no -ffast-math; AVX2
// routines are enabled per function so the rest of the file is baseline
// x86-64, like a default rustc build of the reference).

#include "oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

constexpr float kLayerNormEpsilon = 1.0e-6f;  // tensor.rs:3
constexpr uint32_t kMaximumPosition = 4096;   // marian-model manifest.rs:13

// ---------------------------------------------------------------------------
// Persistent worker pool (stands in for the reference's rayon pool).
// ---------------------------------------------------------------------------
class Pool {
 public:
  explicit Pool(int threads) : n_(std::max(1, threads)) {
    for (int i = 1; i < n_; ++i) workers_.emplace_back([this, i] { loop(i); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(m_);
      stop_ = true;
      ++generation_;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  int size() const { return n_; }
  // Runs fn(worker_index) on every worker including the caller.
  void run(const std::function<void(int)>& fn) {
    if (n_ == 1) {
      fn(0);
      return;
    }
    {
      std::lock_guard<std::mutex> g(m_);
      job_ = &fn;
      pending_ = n_ - 1;
      ++generation_;
    }
    cv_.notify_all();
    fn(0);
    std::unique_lock<std::mutex> lk(m_);
    done_cv_.wait(lk, [this] { return pending_ == 0; });
    job_ = nullptr;
  }

 private:
  void loop(int index) {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(int)>* job;
      {
        std::unique_lock<std::mutex> lk(m_);
        cv_.wait(lk, [&] { return generation_ != seen; });
        seen = generation_;
        if (stop_) return;
        job = job_;
      }
      (*job)(index);
      {
        std::lock_guard<std::mutex> g(m_);
        if (--pending_ == 0) done_cv_.notify_one();
      }
    }
  }
  int n_;
  std::vector<std::thread> workers_;
  std::mutex m_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int)>* job_ = nullptr;
  uint64_t generation_ = 0;
  int pending_ = 0;
  bool stop_ = false;
};

void parallel_for(Pool* pool, size_t n, const std::function<void(size_t, size_t)>& body) {
  if (!pool || pool->size() == 1 || n < 2) {
    body(0, n);
    return;
  }
  const int T = pool->size();
  pool->run([&](int w) {
    size_t lo = n * (size_t)w / (size_t)T, hi = n * (size_t)(w + 1) / (size_t)T;
    if (lo < hi) body(lo, hi);
  });
}

bool have_avx2() {
  static const bool v = __builtin_cpu_supports("avx2");
  return v;
}

// ---------------------------------------------------------------------------
// Elementary fp32 operations.
// ---------------------------------------------------------------------------

// Canonical exp: Cody-Waite reduction x = n*ln2 + r in double, Taylor series of
// degree 11 by Horner (mul then add, no fused ops), scaled by 2^n, rounded once
// to f32.  Every step is a basic IEEE operation, so the HIP kernels evaluate
// the identical sequence and get identical bits.  |relative error| < 1e-13
// before the final rounding.
float canon_expf(float xf) {
  if (!(xf == xf)) return xf;
  if (xf < -104.0f) return 0.0f;
  if (xf > 89.0f) return INFINITY;
  const double x = (double)xf;
  const double n = std::rint(x * 0x1.71547652b82fep+0);
  const double r = x - n * 0x1.62e42fefa39efp-1;
  double p = 0x1.ae64567f544e4p-26;  // 1/11!
  p = p * r + 0x1.27e4fb7789f5cp-22;  // 1/10!
  p = p * r + 0x1.71de3a556c734p-19;  // 1/9!
  p = p * r + 0x1.a01a01a01a01ap-16;  // 1/8!
  p = p * r + 0x1.a01a01a01a01ap-13;  // 1/7!
  p = p * r + 0x1.6c16c16c16c17p-10;  // 1/6!
  p = p * r + 0x1.1111111111111p-7;   // 1/5!
  p = p * r + 0x1.5555555555555p-5;   // 1/4!
  p = p * r + 0x1.5555555555555p-3;   // 1/3!
  p = p * r + 0x1.0000000000000p-1;   // 1/2!
  p = p * r + 1.0;
  p = p * r + 1.0;
  return (float)std::ldexp(p, (int)n);
}

// Canonical row sum: 64 lane partials over strided elements (lane l takes
// x[l], x[l+64], ... in that order), then an xor butterfly 32,16,8,4,2,1.
// This is the order a 64-wide wavefront produces when each lane owns the
// strided elements and the wave reduces with lane swaps.
float canon_sum(const float* x, size_t n) {
  float p[64];
  for (int l = 0; l < 64; ++l) {
    float s = 0.0f;
    for (size_t j = (size_t)l; j < n; j += 64) s = s + x[j];
    p[l] = s;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    float q[64];
    for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ off];
    std::memcpy(p, q, sizeof(p));
  }
  return p[0];
}

// Reference order: `iter().sum::<f32>()`, strictly left to right.
float seq_sum(const float* x, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; ++i) s = s + x[i];
  return s;
}

inline float row_sum(const float* x, size_t n, int order) {
  return order == ORACLE_ORDER_REFERENCE ? seq_sum(x, n) : canon_sum(x, n);
}

inline float exp_op(float x, int order) {
  return order == ORACLE_ORDER_CANONICAL ? canon_expf(x) : std::exp(x);
}

// The encoder's order: FAST_DECODER keeps the reference's there.
inline int encoder_order(int order) {
  return order == ORACLE_ORDER_FAST_DECODER ? ORACLE_ORDER_REFERENCE : order;
}

// Sequential fp32 dot (tensor.rs:479 on x86: map(a*b).sum()).
inline float dot_seq(const float* a, const float* b, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; ++i) s = s + a[i] * b[i];
  return s;
}

// ---------------------------------------------------------------------------
// Quantization (q8_gemm.rs:569-590 with the per-row dynamic multiplier).
// ---------------------------------------------------------------------------
inline int8_t quantize_one(float x, float a) {
  float v = std::nearbyint(x * a);  // round half to even (default mode)
  v = std::min(std::max(v, -127.0f), 127.0f);
  return (int8_t)v;
}

// Returns false on a non-finite value.
bool quantize_row(const float* x, size_t n, int8_t* q, float* a_out) {
  float m = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    if (!std::isfinite(x[i])) return false;
    m = std::max(m, std::fabs(x[i]));
  }
  const float a = m > 0.0f ? 127.0f / m : 1.0f;
  for (size_t i = 0; i < n; ++i) q[i] = quantize_one(x[i], a);
  *a_out = a;
  return true;
}

// ---------------------------------------------------------------------------
// Integer GEMMs.
// ---------------------------------------------------------------------------
__attribute__((target("avx2"))) int64_t hsum_epi32(__m256i v) {
  alignas(32) int32_t lanes[8];
  _mm256_store_si256((__m256i*)lanes, v);
  int64_t s = 0;
  for (int i = 0; i < 8; ++i) s += lanes[i];
  return s;
}

// Signed int8 x int8 dot, AVX2: sign-extend both to i16 and madd.
__attribute__((target("avx2"))) int64_t dot_i8_avx2(const int8_t* a, const int8_t* w, size_t n) {
  size_t i = 0;
  __m256i acc = _mm256_setzero_si256();
  for (; i + 16 <= n; i += 16) {
    __m256i av = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(a + i)));
    __m256i wv = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(w + i)));
    acc = _mm256_add_epi32(acc, _mm256_madd_epi16(av, wv));
  }
  int64_t s = hsum_epi32(acc);
  for (; i < n; ++i) s += (int64_t)a[i] * (int64_t)w[i];
  return s;
}

int64_t dot_i8_scalar(const int8_t* a, const int8_t* w, size_t n) {
  int64_t s = 0;
  for (size_t i = 0; i < n; ++i) s += (int64_t)a[i] * (int64_t)w[i];
  return s;
}

// Reference x86 kernel: q8_avx2.rs dot4_i64_avx2 (:294-358) and dot_i64_avx2
// (:246-290): u8 activations minus the zero point in i16, madd with widened
// i8 weights, i32 vector partials flushed to i64 every 16,384 blocks.
constexpr size_t kBlocksPerFlush = 16384;

__attribute__((target("avx2"))) int64_t dot_u8_avx2(const uint8_t* a, const int8_t* w, size_t n,
                                                    uint8_t zp) {
  size_t i = 0;
  int64_t total = 0;
  const __m256i z = _mm256_set1_epi16((int16_t)zp);
  while (i + 16 <= n) {
    const size_t blocks = std::min((n - i) / 16, kBlocksPerFlush);
    const size_t end = i + blocks * 16;
    __m256i acc = _mm256_setzero_si256();
    for (; i < end; i += 16) {
      __m256i av = _mm256_sub_epi16(
          _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(a + i))), z);
      __m256i wv = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(w + i)));
      acc = _mm256_add_epi32(acc, _mm256_madd_epi16(av, wv));
    }
    total += hsum_epi32(acc);
  }
  for (; i < n; ++i) total += ((int64_t)a[i] - (int64_t)zp) * (int64_t)w[i];
  return total;
}

__attribute__((target("avx2"))) void dot4_u8_avx2(const uint8_t* a, const int8_t* w4, size_t n,
                                                  uint8_t zp, int64_t out[4]) {
  size_t i = 0;
  int64_t totals[4] = {0, 0, 0, 0};
  const __m256i z = _mm256_set1_epi16((int16_t)zp);
  while (i + 16 <= n) {
    const size_t blocks = std::min((n - i) / 16, kBlocksPerFlush);
    const size_t end = i + blocks * 16;
    __m256i acc[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(),
                      _mm256_setzero_si256()};
    for (; i < end; i += 16) {
      __m256i av = _mm256_sub_epi16(
          _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(a + i))), z);
      for (int r = 0; r < 4; ++r) {
        __m256i wv =
            _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(w4 + (size_t)r * n + i)));
        acc[r] = _mm256_add_epi32(acc[r], _mm256_madd_epi16(av, wv));
      }
    }
    for (int r = 0; r < 4; ++r) totals[r] += hsum_epi32(acc[r]);
  }
  for (; i < n; ++i) {
    const int64_t av = (int64_t)a[i] - (int64_t)zp;
    for (int r = 0; r < 4; ++r) totals[r] += av * (int64_t)w4[(size_t)r * n + i];
  }
  for (int r = 0; r < 4; ++r) out[r] = totals[r];
}

bool fits_i32(int64_t v) { return v >= INT32_MIN && v <= INT32_MAX; }

// Exact i32 GEMM on signed int8 activations, rows split across the pool.
bool gemm_i8(Pool* pool, const int8_t* qa, size_t M, size_t K, const int8_t* qw, size_t N,
             int32_t* acc) {
  std::atomic<bool> ok{true};
  const bool avx2 = have_avx2();
  parallel_for(pool, M, [&](size_t lo, size_t hi) {
    for (size_t m = lo; m < hi; ++m) {
      const int8_t* a = qa + m * K;
      for (size_t n = 0; n < N; ++n) {
        const int64_t v = avx2 ? dot_i8_avx2(a, qw + n * K, K) : dot_i8_scalar(a, qw + n * K, K);
        if (!fits_i32(v)) ok = false;
        acc[m * N + n] = (int32_t)v;
      }
    }
  });
  return ok;
}

// Reference-schedule GEMM: q8_avx2.rs gemm_u8_i8_into (:125-229), including
// its row-parallel policy (rows > 1 && rows*N >= 8192).
bool gemm_u8_reference(Pool* pool, const uint8_t* a, size_t M, size_t K, const int8_t* w,
                       size_t N, uint8_t zp, int32_t* out) {
  std::atomic<bool> ok{true};
  auto row = [&](size_t m) {
    const uint8_t* ar = a + m * K;
    int32_t* orow = out + m * N;
    size_t c = 0;
    for (; c + 4 <= N; c += 4) {
      int64_t t[4];
      dot4_u8_avx2(ar, w + c * K, K, zp, t);
      for (int r = 0; r < 4; ++r) {
        if (!fits_i32(t[r])) ok = false;
        orow[c + r] = (int32_t)t[r];
      }
    }
    for (; c < N; ++c) {
      const int64_t t = dot_u8_avx2(ar, w + c * K, K, zp);
      if (!fits_i32(t)) ok = false;
      orow[c] = (int32_t)t;
    }
  };
  if (M > 1 && M * N >= 8192 && pool && pool->size() > 1) {
    parallel_for(pool, M, [&](size_t lo, size_t hi) {
      for (size_t m = lo; m < hi; ++m) row(m);
    });
  } else {
    for (size_t m = 0; m < M; ++m) row(m);
  }
  return ok;
}

// ---------------------------------------------------------------------------
// Linear layers.
// ---------------------------------------------------------------------------
struct Scratch {
  std::vector<int8_t> q;
  std::vector<uint8_t> qu;
  std::vector<float> a;
  std::vector<int32_t> acc;
};

void dequant(const int32_t* acc, const float* a, size_t M, const oracle_linear* lin, size_t N,
             bool relu, float* y) {
  for (size_t m = 0; m < M; ++m) {
    for (size_t n = 0; n < N; ++n) {
      const float inv = 1.0f / (a[m] * lin->mult[n]);
      float v = (float)acc[m * N + n] * inv + lin->bias[n];
      if (relu) v = v > 0.0f ? v : 0.0f;
      y[m * N + n] = v;
    }
  }
}

// Returns false on a non-finite activation or accumulator overflow.
bool linear(Pool* pool, Scratch& s, const float* x, size_t M, size_t K, const oracle_linear* lin,
            size_t N, bool relu, float* y) {
  s.q.resize(M * K);
  s.a.resize(M);
  s.acc.resize(M * N);
  for (size_t m = 0; m < M; ++m)
    if (!quantize_row(x + m * K, K, s.q.data() + m * K, &s.a[m])) return false;
  if (!gemm_i8(pool, s.q.data(), M, K, lin->weight, N, s.acc.data())) return false;
  dequant(s.acc.data(), s.a.data(), M, lin, N, relu, y);
  return true;
}

// Reference-schedule linear: u8 activations (q + 127) into the AVX2 kernel.
bool linear_reference(Pool* pool, Scratch& s, const float* x, size_t M, size_t K,
                      const oracle_linear* lin, size_t N, bool relu, float* y) {
  s.q.resize(M * K);
  s.qu.resize(M * K);
  s.a.resize(M);
  s.acc.resize(M * N);
  for (size_t m = 0; m < M; ++m)
    if (!quantize_row(x + m * K, K, s.q.data() + m * K, &s.a[m])) return false;
  for (size_t i = 0; i < M * K; ++i) s.qu[i] = (uint8_t)((int)s.q[i] + 127);
  if (!gemm_u8_reference(pool, s.qu.data(), M, K, lin->weight, N, 127, s.acc.data()))
    return false;
  dequant(s.acc.data(), s.a.data(), M, lin, N, relu, y);
  return true;
}

// ---------------------------------------------------------------------------
// LayerNorm (tensor.rs:132-155, 372-425), post-norm residual.
// ---------------------------------------------------------------------------
void residual_ln_row(const float* x, const float* r, const float* g, const float* b, size_t d,
                     int order, float* out, float* tmp) {
  for (size_t i = 0; i < d; ++i) tmp[i] = x[i] + r[i];
  const float mean = row_sum(tmp, d, order) / (float)d;
  std::vector<float> sq(d);
  for (size_t i = 0; i < d; ++i) {
    const float c = tmp[i] - mean;
    sq[i] = c * c;
  }
  const float var = row_sum(sq.data(), d, order) / (float)d;
  const float inv = 1.0f / std::sqrt(var + kLayerNormEpsilon);
  for (size_t i = 0; i < d; ++i) out[i] = ((tmp[i] - mean) * inv) * g[i] + b[i];
}

void residual_ln(const float* x, const float* r, const float* g, const float* b, size_t rows,
                 size_t d, int order, float* out) {
  std::vector<float> tmp(d);
  for (size_t m = 0; m < rows; ++m)
    residual_ln_row(x + m * d, r + m * d, g, b, d, order, out + m * d, tmp.data());
}

// ---------------------------------------------------------------------------
// Attention for one (query row, head) over `nk` keys (tensor.rs:251-318):
// score_k = dot(q, k_k) * (1/sqrt(dh)); softmax (max, exp(s - max), sum,
// multiply by 1/sum); out = sum_k p_k v_k accumulated in key order.
// ---------------------------------------------------------------------------
void attend_one(const float* q, const float* k, size_t ldk, const float* v, size_t ldv, size_t nk,
                size_t dh, float scale, int order, float* out, std::vector<float>& sc) {
  sc.resize(nk);
  for (size_t j = 0; j < nk; ++j) sc[j] = dot_seq(q, k + j * ldk, dh) * scale;
  float mx = -INFINITY;
  for (size_t j = 0; j < nk; ++j) mx = std::fmax(mx, sc[j]);
  for (size_t j = 0; j < nk; ++j) sc[j] = exp_op(sc[j] - mx, order);
  float sum;
  if (order == ORACLE_ORDER_REFERENCE) {
    sum = 0.0f;  // softmax_in_place starts its sum at 0.0
    for (size_t j = 0; j < nk; ++j) sum += sc[j];
  } else {
    sum = canon_sum(sc.data(), nk);
  }
  const float inv = 1.0f / sum;
  for (size_t j = 0; j < nk; ++j) sc[j] = sc[j] * inv;
  for (size_t i = 0; i < dh; ++i) out[i] = 0.0f;
  for (size_t j = 0; j < nk; ++j) {
    const float p = sc[j];
    const float* vr = v + j * ldv;
    for (size_t i = 0; i < dh; ++i) out[i] = out[i] + vr[i] * p;
  }
}

// ---------------------------------------------------------------------------
// Model helpers.
// ---------------------------------------------------------------------------
struct Geometry {
  size_t V, d, H, dh, F, Le, Ld;
  float emb_scale;
};

Geometry geometry(const oracle_model* m) {
  Geometry g;
  g.V = m->vocab;
  g.d = m->dim;
  g.H = m->heads;
  g.dh = m->dim / m->heads;
  g.F = m->ffn_dim;
  g.Le = m->encoder_layers;
  g.Ld = m->decoder_layers;
  g.emb_scale = std::sqrt((float)m->dim);  // q8_engine.rs:23 uses sqrt(384) as f32
  return g;
}

struct Positions {
  uint32_t dim = 0;
  std::vector<float> table;
};

const std::vector<float>& positions_for(uint32_t dim) {
  static std::mutex mu;
  static std::vector<Positions> cache;
  std::lock_guard<std::mutex> g(mu);
  for (auto& p : cache)
    if (p.dim == dim) return p.table;
  Positions p;
  p.dim = dim;
  p.table.resize((size_t)kMaximumPosition * dim);
  oracle_positions(dim, kMaximumPosition, p.table.data());
  cache.push_back(std::move(p));
  return cache.back().table;
}

// x = (q / mult) * sqrt(d) + pos  (q8_engine.rs:71, 599, 626).
void embed_row(const oracle_model* m, const Geometry& g, int32_t token, const float* pos,
               float* out) {
  const int8_t* e = m->embedding + (size_t)token * g.d;
  const float mult = m->embedding_mult[token];
  for (size_t i = 0; i < g.d; ++i) {
    const float v = (float)e[i] / mult;
    out[i] = v * g.emb_scale + pos[i];
  }
}

inline bool generation_masked(size_t id, uint32_t flags) {
  if (flags & ORACLE_FLAG_NO_GENERATION_MASK) return false;
  return id == 1 || (id >= 7 && id <= 38);  // shortlist.rs:169-176
}

struct Err {
  char* buf;
  size_t cap;
  int fail(int code, const char* fmt, ...) {
    if (buf && cap) {
      va_list ap;
      va_start(ap, fmt);
      vsnprintf(buf, cap, fmt, ap);
      va_end(ap);
    }
    return code;
  }
};

// Validation of the packed batch (q8_engine.rs:468-509, 1103-1119) and the
// per-row generation limit (q8_engine.rs:369-379).
int validate(const oracle_model* m, const int32_t* tokens, size_t n_tokens,
             const uint32_t* offsets, size_t n_offsets, const uint32_t* req,
             const oracle_limits* lim, std::vector<uint32_t>& limits, Err& e) {
  if (n_offsets < 2 || offsets[0] != 0 || offsets[n_offsets - 1] != n_tokens)
    return e.fail(-1, "invalid packed batch offsets");
  const size_t B = n_offsets - 1;
  if (lim->max_batch && B > lim->max_batch)
    return e.fail(-1, "batch contains %zu sentences; maximum is %u", B, lim->max_batch);
  size_t L = 0;
  for (size_t b = 0; b < B; ++b) {
    if (offsets[b + 1] <= offsets[b]) return e.fail(-1, "each input must contain at least one token");
    L = std::max<size_t>(L, offsets[b + 1] - offsets[b]);
  }
  if (lim->max_source_tokens && L > lim->max_source_tokens)
    return e.fail(-1, "source has %zu tokens; maximum is %u", L, lim->max_source_tokens);
  if (lim->max_padded_cells && (uint64_t)B * L * L > lim->max_padded_cells)
    return e.fail(-1, "padded attention work is %llu cells; maximum is %llu",
                  (unsigned long long)((uint64_t)B * L * L),
                  (unsigned long long)lim->max_padded_cells);
  if (L > kMaximumPosition) return e.fail(-1, "source longer than the position table");
  for (size_t i = 0; i < n_tokens; ++i)
    if (tokens[i] < 0 || (uint32_t)tokens[i] >= m->vocab)
      return e.fail(-1, "source token %d is outside vocabulary %u", tokens[i], m->vocab);
  const uint32_t maxpos = lim->max_position ? std::min(lim->max_position, kMaximumPosition)
                                            : kMaximumPosition;
  limits.resize(B);
  for (size_t b = 0; b < B; ++b) {
    uint64_t l = req[b];
    const uint64_t len = offsets[b + 1] - offsets[b];
    if (lim->max_length_factor) l = std::min<uint64_t>(l, len * lim->max_length_factor);
    if (lim->max_generation_steps) l = std::min<uint64_t>(l, lim->max_generation_steps);
    l = std::min<uint64_t>(l, maxpos);
    limits[b] = (uint32_t)l;
  }
  return 0;
}

// Encoder for one sentence of length L (rows independent of batch-mates).
bool encode_sentence(const oracle_model* m, const Geometry& g, const int32_t* tok, size_t L,
                     int order, Pool* pool, Scratch& s, std::vector<float>& x) {
  const auto& pos = positions_for(m->dim);
  const size_t d = g.d;
  x.resize(L * d);
  for (size_t i = 0; i < L; ++i) embed_row(m, g, tok[i], pos.data() + i * d, x.data() + i * d);
  std::vector<float> qkv(L * 3 * d), att(L * d), y(L * d), h(L * g.F), x2(L * d);
  const float scale = 1.0f / std::sqrt((float)g.dh);
  std::vector<float> sc;
  for (size_t l = 0; l < g.Le; ++l) {
    const oracle_encoder_layer& E = m->encoder[l];
    if (!linear(pool, s, x.data(), L, d, &E.qkv, 3 * d, false, qkv.data())) return false;
    for (size_t i = 0; i < L; ++i)
      for (size_t hd = 0; hd < g.H; ++hd)
        attend_one(qkv.data() + i * 3 * d + hd * g.dh, qkv.data() + d + hd * g.dh, 3 * d,
                   qkv.data() + 2 * d + hd * g.dh, 3 * d, L, g.dh, scale, order,
                   att.data() + i * d + hd * g.dh, sc);
    if (!linear(pool, s, att.data(), L, d, &E.out, d, false, y.data())) return false;
    residual_ln(y.data(), x.data(), E.ln1_scale, E.ln1_bias, L, d, order, x2.data());
    if (!linear(pool, s, x2.data(), L, d, &E.ffn1, g.F, true, h.data())) return false;
    if (!linear(pool, s, h.data(), L, g.F, &E.ffn2, d, false, y.data())) return false;
    residual_ln(y.data(), x2.data(), E.ln2_scale, E.ln2_bias, L, d, order, x.data());
  }
  return true;
}

// Output scoring for one row: quantize the state, exact int8 dot per vocab
// row, logit = acc * (1/(a*mult)) + bias, strict '>' argmax in ascending id
// order (q8_engine.rs:749-790), or over the candidate list in its order when
// one is given (no generation mask then).  Optionally stores every logit.
bool select_token(const oracle_model* m, const Geometry& g, const float* state, uint32_t flags,
                  int32_t* token, float* logits_out, const uint32_t* cands = nullptr,
                  size_t n_cands = 0) {
  std::vector<int8_t> q(g.d);
  float a;
  if (!quantize_row(state, g.d, q.data(), &a)) return false;
  const bool avx2 = have_avx2();
  int32_t best = -1;
  float best_v = -INFINITY;
  if (cands) {
    for (size_t i = 0; i < n_cands; ++i) {
      const size_t v = cands[i];
      const int64_t acc = avx2 ? dot_i8_avx2(q.data(), m->embedding + v * g.d, g.d)
                               : dot_i8_scalar(q.data(), m->embedding + v * g.d, g.d);
      const float logit = (float)acc * (1.0f / (a * m->embedding_mult[v])) + m->output_bias[v];
      if (best < 0) best = (int32_t)v;
      if (logit > best_v) {
        best_v = logit;
        best = (int32_t)v;
      }
    }
    *token = best;
    return true;
  }
  for (size_t v = 0; v < g.V; ++v) {
    const int64_t acc = avx2 ? dot_i8_avx2(q.data(), m->embedding + v * g.d, g.d)
                             : dot_i8_scalar(q.data(), m->embedding + v * g.d, g.d);
    const float inv = 1.0f / (a * m->embedding_mult[v]);
    const float logit = (float)acc * inv + m->output_bias[v];
    if (generation_masked(v, flags)) {
      if (logits_out) logits_out[v] = -INFINITY;
      continue;
    }
    if (logits_out) logits_out[v] = logit;
    if (best < 0) best = (int32_t)v;  // candidates[0] when nothing beats -inf
    if (logit > best_v) {
      best_v = logit;
      best = (int32_t)v;
    }
  }
  *token = best < 0 ? 0 : best;
  return true;
}

// Greedy decoding of one sentence given its encoder output.
bool decode_sentence(const oracle_model* m, const Geometry& g, const float* enc, size_t L,
                     uint32_t limit, uint32_t flags, int order, Pool* pool, Scratch& s,
                     std::vector<int32_t>& out, uint32_t stop_after, int64_t probe_step,
                     float* probe_logits, bool* probed, const uint32_t* cands = nullptr,
                     size_t n_cands = 0) {
  const auto& pos = positions_for(m->dim);
  const size_t d = g.d;
  std::vector<std::vector<float>> ckv(g.Ld, std::vector<float>(L * 2 * d));
  for (size_t l = 0; l < g.Ld; ++l)
    if (!linear(pool, s, enc, L, d, &m->decoder[l].cross_kv, 2 * d, false, ckv[l].data()))
      return false;
  std::vector<std::vector<float>> kc(g.Ld, std::vector<float>((size_t)limit * d)),
      vc(g.Ld, std::vector<float>((size_t)limit * d));
  std::vector<float> x(d), qkv(3 * d), att(d), y(d), x2(d), h(g.F), qc(d);
  const float scale = 1.0f / std::sqrt((float)g.dh);
  std::vector<float> sc;
  int32_t prev = -1;
  for (uint32_t t = 0; t < limit; ++t) {
    if (prev < 0) {
      std::memcpy(x.data(), pos.data() + (size_t)t * d, d * sizeof(float));
    } else {
      embed_row(m, g, prev, pos.data() + (size_t)t * d, x.data());
    }
    for (size_t l = 0; l < g.Ld; ++l) {
      const oracle_decoder_layer& D = m->decoder[l];
      if (!linear(pool, s, x.data(), 1, d, &D.self_qkv, 3 * d, false, qkv.data())) return false;
      std::memcpy(kc[l].data() + (size_t)t * d, qkv.data() + d, d * sizeof(float));
      std::memcpy(vc[l].data() + (size_t)t * d, qkv.data() + 2 * d, d * sizeof(float));
      for (size_t hd = 0; hd < g.H; ++hd)
        attend_one(qkv.data() + hd * g.dh, kc[l].data() + hd * g.dh, d, vc[l].data() + hd * g.dh,
                   d, (size_t)t + 1, g.dh, scale, order, att.data() + hd * g.dh, sc);
      if (!linear(pool, s, att.data(), 1, d, &D.self_out, d, false, y.data())) return false;
      residual_ln(y.data(), x.data(), D.ln1_scale, D.ln1_bias, 1, d, order, x2.data());
      if (!linear(pool, s, x2.data(), 1, d, &D.cross_q, d, false, qc.data())) return false;
      for (size_t hd = 0; hd < g.H; ++hd)
        attend_one(qc.data() + hd * g.dh, ckv[l].data() + hd * g.dh, 2 * d,
                   ckv[l].data() + d + hd * g.dh, 2 * d, L, g.dh, scale, order,
                   att.data() + hd * g.dh, sc);
      if (!linear(pool, s, att.data(), 1, d, &D.cross_out, d, false, y.data())) return false;
      residual_ln(y.data(), x2.data(), D.ln2_scale, D.ln2_bias, 1, d, order, x.data());
      if (!linear(pool, s, x.data(), 1, d, &D.ffn1, g.F, true, h.data())) return false;
      if (!linear(pool, s, h.data(), 1, g.F, &D.ffn2, d, false, y.data())) return false;
      residual_ln(y.data(), x.data(), D.ln3_scale, D.ln3_bias, 1, d, order, x2.data());
      x.swap(x2);
    }
    int32_t token;
    const bool want_logits = probe_logits && (int64_t)t == probe_step;
    if (!select_token(m, g, x.data(), flags, &token, want_logits ? probe_logits : nullptr, cands,
                      n_cands))
      return false;
    if (want_logits && probed) *probed = true;
    out.push_back(token);
    prev = token;
    if (stop_after && t + 1 == stop_after) break;
    if (token == 0 && !(flags & ORACLE_FLAG_IGNORE_EOS)) break;
  }
  return true;
}

int pack_output(const std::vector<std::vector<int32_t>>& gen, int32_t* out_tokens, size_t out_cap,
                uint32_t* out_offsets, size_t* out_len, Err& e) {
  size_t total = 0;
  for (auto& v : gen) total += v.size();
  if (out_len) *out_len = total;
  if (total > out_cap) return e.fail(-3, "output buffer holds %zu tokens; %zu needed", out_cap, total);
  size_t o = 0;
  out_offsets[0] = 0;
  for (size_t b = 0; b < gen.size(); ++b) {
    for (int32_t t : gen[b]) out_tokens[o++] = t;
    out_offsets[b + 1] = (uint32_t)o;
  }
  return 0;
}

// ---------------------------------------------------------------------------
// The Transformer-SSRU graph with static activation multipliers.
// ---------------------------------------------------------------------------
// Q8Linear::run_into (q8_gemm.rs:380-448): every element quantized with the
// tensor's act_mult (quantize_symmetric_u8_into :569-590, non-finite input is
// an error), exact GEMM, y = acc * (1 / (act_mult * weight_mult)) + bias, with
// 0.0 added where the layer has no bias (:444).
bool linear_static(Pool* pool, Scratch& s, const float* x, size_t M, size_t K,
                   const oracle_static_linear* lin, size_t N, bool relu, float* y) {
  s.q.resize(M * K);
  s.acc.resize(M * N);
  for (size_t i = 0; i < M * K; ++i) {
    if (!std::isfinite(x[i])) return false;
    s.q[i] = quantize_one(x[i], lin->act_mult);
  }
  if (!gemm_i8(pool, s.q.data(), M, K, lin->weight, N, s.acc.data())) return false;
  const float inv = 1.0f / (lin->act_mult * lin->weight_mult);
  for (size_t m = 0; m < M; ++m)
    for (size_t n = 0; n < N; ++n) {
      float v = (float)s.acc[m * N + n] * inv + (lin->bias ? lin->bias[n] : 0.0f);
      if (relu) v = v > 0.0f ? v : 0.0f;  // relu_in_place after the layer (q8_engine.rs:639)
      y[m * N + n] = v;
    }
  return true;
}

// Reference-schedule static linear (timed CPU baseline): the elements
// quantized with act_mult as u8 (q + 127, quantize_symmetric_u8_into
// q8_gemm.rs:569-590) into the AVX2 kernel (q8_avx2.rs:125-229), then the
// same dequantization as linear_static.
bool linear_static_reference(Pool* pool, Scratch& s, const float* x, size_t M, size_t K,
                             const oracle_static_linear* lin, size_t N, bool relu, float* y) {
  s.qu.resize(M * K);
  s.acc.resize(M * N);
  for (size_t i = 0; i < M * K; ++i) {
    if (!std::isfinite(x[i])) return false;
    s.qu[i] = (uint8_t)((int)quantize_one(x[i], lin->act_mult) + 127);
  }
  if (!gemm_u8_reference(pool, s.qu.data(), M, K, lin->weight, N, 127, s.acc.data())) return false;
  const float inv = 1.0f / (lin->act_mult * lin->weight_mult);
  for (size_t m = 0; m < M; ++m)
    for (size_t n = 0; n < N; ++n) {
      float v = (float)s.acc[m * N + n] * inv + (lin->bias ? lin->bias[n] : 0.0f);
      if (relu) v = v > 0.0f ? v : 0.0f;
      y[m * N + n] = v;
    }
  return true;
}

struct SsruGeometry {
  size_t Vs, Vt, d, H, dh, F, Le, Ld;
  float emb_scale;
};

SsruGeometry ssru_geometry(const oracle_ssru_model* m) {
  SsruGeometry g;
  g.Vs = m->source_vocab;
  g.Vt = m->target_vocab;
  g.d = m->dim;
  g.H = m->heads;
  g.dh = m->dim / m->heads;
  g.F = m->ffn_dim;
  g.Le = m->encoder_layers;
  g.Ld = m->decoder_layers;
  g.emb_scale = std::sqrt((float)m->dim);  // EMBEDDING_SCALE = sqrt(384) (q8_engine.rs:23)
  return g;
}

// Q8Embedding::row_into (q8_engine.rs:53-74) then x * EMBEDDING_SCALE + pos.
void embed_static(const int8_t* table, float mult, size_t d, float scale, int32_t token,
                  const float* pos, float* out) {
  const int8_t* e = table + (size_t)token * d;
  for (size_t i = 0; i < d; ++i) {
    const float v = (float)e[i] / mult;
    out[i] = v * scale + pos[i];
  }
}

// Attention of `rows` query rows over one sentence's keys, every head.
void attend_rows(const float* q, const float* k, const float* v, size_t rows, size_t nk,
                 const SsruGeometry& g, int order, float* out, std::vector<float>& sc) {
  const float scale = 1.0f / std::sqrt((float)g.dh);
  for (size_t i = 0; i < rows; ++i)
    for (size_t h = 0; h < g.H; ++h)
      attend_one(q + i * g.d + h * g.dh, k + h * g.dh, g.d, v + h * g.dh, g.d, nk, g.dh, scale,
                 order, out + i * g.d + h * g.dh, sc);
}

// encode (q8_engine.rs:511-558) for one sentence: Q, K and V each from their
// own layer and static multiplier.
bool encode_sentence_ssru(const oracle_ssru_model* m, const SsruGeometry& g, const int32_t* tok,
                          size_t L, int order, Pool* pool, Scratch& s, std::vector<float>& x) {
  const auto& pos = positions_for(m->dim);
  const size_t d = g.d;
  x.resize(L * d);
  for (size_t i = 0; i < L; ++i)
    embed_static(m->encoder_embedding, m->encoder_embedding_mult, d, g.emb_scale, tok[i],
                 pos.data() + i * d, x.data() + i * d);
  std::vector<float> q(L * d), k(L * d), v(L * d), att(L * d), y(L * d), h(L * g.F), x2(L * d);
  std::vector<float> sc;
  for (size_t l = 0; l < g.Le; ++l) {
    const oracle_ssru_encoder_layer& E = m->encoder[l];
    if (!linear_static(pool, s, x.data(), L, d, &E.wq, d, false, q.data()) ||
        !linear_static(pool, s, x.data(), L, d, &E.wk, d, false, k.data()) ||
        !linear_static(pool, s, x.data(), L, d, &E.wv, d, false, v.data()))
      return false;
    attend_rows(q.data(), k.data(), v.data(), L, L, g, order, att.data(), sc);
    if (!linear_static(pool, s, att.data(), L, d, &E.wo, d, false, y.data())) return false;
    residual_ln(y.data(), x.data(), E.attn_ln_scale, E.attn_ln_bias, L, d, order, x2.data());
    if (!linear_static(pool, s, x2.data(), L, d, &E.w1, g.F, true, h.data()) ||
        !linear_static(pool, s, h.data(), L, g.F, &E.w2, d, false, y.data()))
      return false;
    residual_ln(y.data(), x2.data(), E.ffn_ln_scale, E.ffn_ln_bias, L, d, order, x.data());
  }
  return true;
}

// select_token (q8_engine.rs:749-790) with the static output multiplier: the
// state quantized once, then a strict '>' scan from -inf over the candidates
// in order (cands == nullptr: every target id ascending, masked ids skipped).
bool select_static(const oracle_ssru_model* m, const SsruGeometry& g, const float* state,
                   uint32_t flags, const uint32_t* cands, size_t n_cands, int32_t* token,
                   float* logits_out) {
  std::vector<int8_t> q(g.d);
  for (size_t i = 0; i < g.d; ++i) {
    if (!std::isfinite(state[i])) return false;
    q[i] = quantize_one(state[i], m->output_act_mult);
  }
  const float inv = 1.0f / (m->output_act_mult * m->decoder_embedding_mult);
  const bool avx2 = have_avx2();
  auto logit_of = [&](size_t id) {
    const int8_t* w = m->decoder_embedding + id * g.d;
    const int64_t acc = avx2 ? dot_i8_avx2(q.data(), w, g.d) : dot_i8_scalar(q.data(), w, g.d);
    return (float)acc * inv + m->output_bias[id];
  };
  if (logits_out)
    for (size_t v = 0; v < g.Vt; ++v) logits_out[v] = -INFINITY;
  int32_t best = -1;
  float best_v = -INFINITY;
  const size_t n = cands ? n_cands : g.Vt;
  for (size_t i = 0; i < n; ++i) {
    const size_t id = cands ? cands[i] : i;
    if (!cands && generation_masked(id, flags)) continue;
    const float lg = logit_of(id);
    if (logits_out) logits_out[id] = lg;
    if (best < 0) best = (int32_t)id;  // candidates[0] when nothing beats -inf
    if (lg > best_v) {
      best_v = lg;
      best = (int32_t)id;
    }
  }
  *token = best < 0 ? 0 : best;
  return true;
}

// The greedy loop (q8_engine.rs:382-451) for one sentence with the SSRU
// decoder: per layer the SSRU sublayer (W and Wf on the layer input, the gate
// update and LayerNorm, :394-408), cross-attention over the sentence's
// encoder rows (:410-432) and the FFN.  The recurrent state starts at zero.
bool decode_sentence_ssru(const oracle_ssru_model* m, const SsruGeometry& g, const float* enc,
                          size_t L, uint32_t limit, uint32_t flags, int order, Pool* pool,
                          Scratch& s, const uint32_t* cands, size_t n_cands,
                          std::vector<int32_t>& out, int64_t probe_step, float* probe_logits,
                          bool* probed) {
  const auto& pos = positions_for(m->dim);
  const size_t d = g.d;
  std::vector<std::vector<float>> ck(g.Ld, std::vector<float>(L * d)),
      cv(g.Ld, std::vector<float>(L * d)), state(g.Ld, std::vector<float>(d, 0.0f));
  for (size_t l = 0; l < g.Ld; ++l)
    if (!linear_static(pool, s, enc, L, d, &m->decoder[l].wk, d, false, ck[l].data()) ||
        !linear_static(pool, s, enc, L, d, &m->decoder[l].wv, d, false, cv[l].data()))
      return false;
  std::vector<float> x(d), u(d), f(d), x1(d), qc(d), att(d), y(d), x2(d), h(g.F), sc;
  int32_t prev = -1;
  for (uint32_t t = 0; t < limit; ++t) {
    if (prev < 0)
      std::memcpy(x.data(), pos.data() + (size_t)t * d, d * sizeof(float));
    else
      embed_static(m->decoder_embedding, m->decoder_embedding_mult, d, g.emb_scale, prev,
                   pos.data() + (size_t)t * d, x.data());
    for (size_t l = 0; l < g.Ld; ++l) {
      const oracle_ssru_decoder_layer& D = m->decoder[l];
      if (!linear_static(pool, s, x.data(), 1, d, &D.ssru_w, d, false, u.data()) ||
          !linear_static(pool, s, x.data(), 1, d, &D.ssru_wf, d, false, f.data()))
        return false;
      oracle_ssru_layer_norm(u.data(), f.data(), state[l].data(), x.data(), D.ssru_ln_scale,
                             D.ssru_ln_bias, 1, d, order, x1.data());
      if (!linear_static(pool, s, x1.data(), 1, d, &D.wq, d, false, qc.data())) return false;
      attend_rows(qc.data(), ck[l].data(), cv[l].data(), 1, L, g, order, att.data(), sc);
      if (!linear_static(pool, s, att.data(), 1, d, &D.wo, d, false, y.data())) return false;
      residual_ln(y.data(), x1.data(), D.context_ln_scale, D.context_ln_bias, 1, d, order, x2.data());
      if (!linear_static(pool, s, x2.data(), 1, d, &D.w1, g.F, true, h.data()) ||
          !linear_static(pool, s, h.data(), 1, g.F, &D.w2, d, false, y.data()))
        return false;
      residual_ln(y.data(), x2.data(), D.ffn_ln_scale, D.ffn_ln_bias, 1, d, order, x.data());
    }
    int32_t token;
    const bool want = probe_logits && (int64_t)t == probe_step;
    if (!select_static(m, g, x.data(), flags, cands, n_cands, &token, want ? probe_logits : nullptr))
      return false;
    if (want && probed) *probed = true;
    out.push_back(token);
    prev = token;
    if (token == 0 && !(flags & ORACLE_FLAG_IGNORE_EOS)) break;
  }
  return true;
}

bool ssru_model_ok(const oracle_ssru_model* m) {
  return m && m->dim && m->heads && m->dim % m->heads == 0 && m->dim % 2 == 0 && m->dim >= 4 &&
         m->source_vocab > 0 && m->target_vocab > 0 && m->encoder_embedding &&
         m->decoder_embedding && m->output_bias && m->decoder_layers > 0 && m->decoder &&
         (m->encoder_layers == 0 || m->encoder);
}

bool model_ok(const oracle_model* m) {
  return m && m->dim && m->heads && m->dim % m->heads == 0 && m->dim % 2 == 0 && m->dim >= 4 &&
         m->vocab > 0 && m->embedding && m->embedding_mult && m->output_bias;
}

}  // namespace

// ===========================================================================
// C API
// ===========================================================================
extern "C" {

float oracle_expf(float x, int order) { return exp_op(x, order); }

#ifndef ORACLE_COMPILER
#define ORACLE_COMPILER "unknown"
#endif
const char* oracle_build_info(void) {
  return ORACLE_COMPILER ", -O3 -ffp-contract=off, AVX2 integer kernels (target attribute, no AVX-512)";
}

float oracle_row_sum(const float* x, size_t n, int order) { return row_sum(x, n, order); }

// position.rs:5-21: f_i = exp(-i * ln(10000) / (half-1)) in f32;
// pos[p][i] = sin(p*f_i), pos[p][half+i] = cos(p*f_i).
int oracle_positions(uint32_t dim, uint32_t count, float* out) {
  if (dim < 4 || dim % 2) return -1;
  const uint32_t half = dim / 2;
  const float ln10k = std::log(10000.0f);
  for (uint32_t p = 0; p < count; ++p) {
    for (uint32_t i = 0; i < half; ++i) {
      const float f = std::exp(-(float)i * ln10k / (float)(half - 1));
      const float arg = (float)p * f;
      out[(size_t)p * dim + i] = std::sin(arg);
      out[(size_t)p * dim + half + i] = std::cos(arg);
    }
  }
  return 0;
}

int oracle_quantize_rows(const float* x, size_t rows, size_t cols, int8_t* q, float* a) {
  for (size_t m = 0; m < rows; ++m)
    if (!quantize_row(x + m * cols, cols, q + m * cols, a + m)) return -1;
  return 0;
}

int oracle_quantize_static_u8(const float* x, size_t n, float mult, uint8_t* out) {
  if (!(std::isfinite(mult) && mult > 0.0f)) return -1;
  for (size_t i = 0; i < n; ++i) {
    if (!std::isfinite(x[i])) return -1;
    out[i] = (uint8_t)((int)quantize_one(x[i], mult) + 127);
  }
  return 0;
}

int oracle_gemm_i32(const int8_t* qa, size_t M, size_t K, const int8_t* qw, size_t N,
                    int32_t* acc, int threads) {
  Pool pool(threads);
  return gemm_i8(&pool, qa, M, K, qw, N, acc) ? 0 : -2;
}

int oracle_gemm_u8_i8_avx2(const uint8_t* a, size_t M, size_t K, const int8_t* w, size_t N,
                           uint8_t zero_point, int32_t* acc, int threads) {
  if (!have_avx2()) return -4;
  Pool pool(threads);
  return gemm_u8_reference(&pool, a, M, K, w, N, zero_point, acc) ? 0 : -2;
}

int32_t oracle_dot_u8_i8(const uint8_t* a, const int8_t* w, size_t n) {
  int32_t s = 0;
  for (size_t i = 0; i < n; ++i) s += ((int32_t)a[i] - 127) * (int32_t)w[i];
  return s;
}

int oracle_linear_forward(const float* x, size_t M, size_t K, const oracle_linear* lin, size_t N,
                          int relu, float* y, int32_t* acc, int8_t* qa, float* a, int threads) {
  Pool pool(threads);
  Scratch s;
  if (!linear(&pool, s, x, M, K, lin, N, relu != 0, y)) return -2;
  if (acc) std::memcpy(acc, s.acc.data(), M * N * sizeof(int32_t));
  if (qa) std::memcpy(qa, s.q.data(), M * K);
  if (a) std::memcpy(a, s.a.data(), M * sizeof(float));
  return 0;
}

// Q8Linear::run_into with the model's static activation multiplier
// (q8_gemm.rs:380-448, quantize_symmetric_u8_into :569-590): every row is
// quantized with act_mult, then the exact GEMM and dequant of the dynamic path.
int oracle_linear_forward_static(const float* x, size_t M, size_t K, const oracle_linear* lin,
                                 size_t N, float act_mult, int relu, float* y, int32_t* acc,
                                 int8_t* qa, int threads) {
  if (!(std::isfinite(act_mult) && act_mult > 0.0f)) return -1;
  std::vector<int8_t> q(M * K);
  for (size_t i = 0; i < M * K; ++i) {
    if (!std::isfinite(x[i])) return -1;  // :578-583 rejects non-finite input
    q[i] = quantize_one(x[i], act_mult);
  }
  std::vector<int32_t> ac(M * N);
  Pool pool(threads);
  if (!gemm_i8(&pool, q.data(), M, K, lin->weight, N, ac.data())) return -2;
  std::vector<float> a(M, act_mult);
  dequant(ac.data(), a.data(), M, lin, N, relu != 0, y);
  if (acc) std::memcpy(acc, ac.data(), M * N * sizeof(int32_t));
  if (qa) std::memcpy(qa, q.data(), M * K);
  return 0;
}

// ssru_update_layer_norm_into (tensor.rs:184-218): per element
// gate = 1 / (1 + exp(-f)), state = gate * state + (1 - gate) * cand; then
// out = normalize_row(relu(state) + residual) (relu_residual :718-724; the x86
// relu is _mm256_max_ps(x, 0), which gives +0.0 for NaN and -0.0).
int oracle_ssru_layer_norm(const float* cand, const float* forget, float* state,
                           const float* residual, const float* scale, const float* bias,
                           size_t rows, size_t d, int order, float* out) {
  if (!rows || !d) return 0;
  std::vector<float> z(d), zero(d, 0.0f);
  for (size_t m = 0; m < rows; ++m) {
    for (size_t i = 0; i < d; ++i) {
      const size_t k = m * d + i;
      const float gate = 1.0f / (1.0f + exp_op(-forget[k], order));
      const float next = gate * state[k] + (1.0f - gate) * cand[k];
      state[k] = next;
      z[i] = next > 0.0f ? next : 0.0f;
    }
    residual_ln(z.data(), residual + m * d, scale, bias, 1, d, order, out + m * d);
  }
  return 0;
}

// select_token over explicit candidate lists (q8_engine.rs:749-790): for row m
// and each candidate c in list order, logit = acc * (1/(xa[m]*mult[c])) +
// bias[c]; the strict '>' scan from -inf keeps the first maximum, and a row
// whose logits never exceed -inf keeps its first candidate.
int oracle_candidate_argmax(const int8_t* xq, const float* xa, size_t M, size_t K,
                            const int8_t* emb, const float* mult, const float* bias, size_t V,
                            const uint32_t* cand, const uint32_t* offs, int32_t* token,
                            float* logits) {
  for (size_t m = 0; m < M; ++m) {
    if (offs[m + 1] <= offs[m]) return -1;  // "cannot select from an empty candidate list"
    int32_t best = (int32_t)cand[offs[m]];
    float best_v = -INFINITY;
    for (uint32_t i = offs[m]; i < offs[m + 1]; ++i) {
      const uint32_t c = cand[i];
      if (c >= V) return -1;  // "output candidate exceeds vocabulary"
      const int64_t acc = dot_i8_scalar(xq + m * K, emb + (size_t)c * K, K);
      const float inv = 1.0f / (xa[m] * mult[c]);
      const float logit = (float)acc * inv + bias[c];
      if (logits) logits[i] = logit;
      if (logit > best_v) {
        best_v = logit;
        best = (int32_t)c;
      }
    }
    token[m] = best;
  }
  return 0;
}

int oracle_residual_layer_norm(const float* x, const float* r, const float* scale,
                               const float* bias, size_t rows, size_t d, int order, float* out) {
  residual_ln(x, r, scale, bias, rows, d, order, out);
  return 0;
}

int oracle_attention(const float* q, size_t ldq, const float* k, size_t ldk, const float* v,
                     size_t ldv, const uint32_t* cu_q, const uint32_t* cu_k, size_t batch,
                     size_t heads, size_t head_dim, int order, float* out, size_t ldo) {
  const float scale = 1.0f / std::sqrt((float)head_dim);
  std::vector<float> sc;
  for (size_t b = 0; b < batch; ++b) {
    const size_t nk = cu_k[b + 1] - cu_k[b];
    if (nk == 0) return -1;
    for (size_t i = cu_q[b]; i < cu_q[b + 1]; ++i)
      for (size_t h = 0; h < heads; ++h)
        attend_one(q + i * ldq + h * head_dim, k + (size_t)cu_k[b] * ldk + h * head_dim, ldk,
                   v + (size_t)cu_k[b] * ldv + h * head_dim, ldv, nk, head_dim, scale, order,
                   out + i * ldo + h * head_dim, sc);
  }
  return 0;
}

int oracle_translate(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                     const uint32_t* offsets, size_t n_offsets,
                     const uint32_t* max_output_tokens, const oracle_limits* limits,
                     uint32_t flags, int order, int threads, int32_t* out_tokens, size_t out_cap,
                     uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap) {
  return oracle_translate_probe(model, tokens, n_tokens, offsets, n_offsets, max_output_tokens,
                                limits, flags, order, threads, out_tokens, out_cap, out_offsets,
                                out_len, err, err_cap, UINT32_MAX, nullptr, nullptr, nullptr);
}

static int translate_impl(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                          const uint32_t* offsets, size_t n_offsets,
                          const uint32_t* max_output_tokens, const oracle_limits* limits,
                          uint32_t flags, int order, int threads, const uint32_t* cands,
                          const uint32_t* cand_offsets, int32_t* out_tokens, size_t out_cap,
                          uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap,
                          uint32_t probe_step, float* enc_out, float* logits_out,
                          uint8_t* active_out) {
  Err e{err, err_cap};
  if (!model_ok(model)) return e.fail(-2, "invalid model description");
  std::vector<uint32_t> lim;
  int rc = validate(model, tokens, n_tokens, offsets, n_offsets, max_output_tokens, limits, lim, e);
  if (rc) return rc;
  const Geometry g = geometry(model);
  const size_t B = n_offsets - 1;
  if (cands) {
    if (!cand_offsets || cand_offsets[0] != 0) return e.fail(-1, "invalid candidate offsets");
    for (size_t b = 0; b < B; ++b) {
      if (cand_offsets[b + 1] <= cand_offsets[b])
        return e.fail(-1, "cannot select from an empty candidate list");
      for (uint32_t i = cand_offsets[b]; i < cand_offsets[b + 1]; ++i)
        if (cands[i] >= g.V) return e.fail(-1, "output candidate %u exceeds vocabulary %zu", cands[i], g.V);
    }
  }
  std::vector<std::vector<int32_t>> gen(B);
  std::atomic<bool> ok{true};
  std::atomic<size_t> next{0};
  // Sentences are independent (batch invariance, q8_golden.rs:68-84), so the
  // checker runs one sentence per worker thread.
  const int T = std::max(1, threads);
  std::vector<std::thread> workers;
  auto work = [&] {
    Scratch s;
    std::vector<float> enc;
    for (;;) {
      const size_t b = next.fetch_add(1);
      if (b >= B) return;
      const size_t L = offsets[b + 1] - offsets[b];
      if (!encode_sentence(model, g, tokens + offsets[b], L, encoder_order(order), nullptr, s, enc)) {
        ok = false;
        continue;
      }
      if (enc_out) std::memcpy(enc_out + (size_t)offsets[b] * g.d, enc.data(), L * g.d * sizeof(float));
      bool probed = false;
      if (!decode_sentence(model, g, enc.data(), L, lim[b], flags, order, nullptr, s, gen[b], 0,
                           probe_step, logits_out ? logits_out + b * g.V : nullptr, &probed,
                           cands ? cands + cand_offsets[b] : nullptr,
                           cands ? cand_offsets[b + 1] - cand_offsets[b] : 0))
        ok = false;
      if (active_out) active_out[b] = probed ? 1 : 0;
    }
  };
  for (int i = 1; i < T; ++i) workers.emplace_back(work);
  work();
  for (auto& w : workers) w.join();
  if (!ok) return e.fail(-2, "non-finite activation or accumulator overflow");
  return pack_output(gen, out_tokens, out_cap, out_offsets, out_len, e);
}

int oracle_translate_probe(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                           const uint32_t* offsets, size_t n_offsets,
                           const uint32_t* max_output_tokens, const oracle_limits* limits,
                           uint32_t flags, int order, int threads, int32_t* out_tokens,
                           size_t out_cap, uint32_t* out_offsets, size_t* out_len, char* err,
                           size_t err_cap, uint32_t probe_step, float* enc_out,
                           float* logits_out, uint8_t* active_out) {
  return translate_impl(model, tokens, n_tokens, offsets, n_offsets, max_output_tokens, limits, flags,
                        order, threads, nullptr, nullptr, out_tokens, out_cap, out_offsets, out_len,
                        err, err_cap, probe_step, enc_out, logits_out, active_out);
}

int oracle_translate_shortlisted(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                                 const uint32_t* offsets, size_t n_offsets,
                                 const uint32_t* max_output_tokens, const oracle_limits* limits,
                                 uint32_t flags, int order, int threads, const uint32_t* candidates,
                                 const uint32_t* cand_offsets, int32_t* out_tokens, size_t out_cap,
                                 uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap) {
  if (!candidates) return Err{err, err_cap}.fail(-1, "candidate lists are required");
  return translate_impl(model, tokens, n_tokens, offsets, n_offsets, max_output_tokens, limits, flags,
                        order, threads, candidates, cand_offsets, out_tokens, out_cap, out_offsets,
                        out_len, err, err_cap, UINT32_MAX, nullptr, nullptr, nullptr);
}

int oracle_encode(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                  const uint32_t* offsets, size_t n_offsets, int order, int threads, float* out) {
  if (!model_ok(model) || n_offsets < 2 || offsets[n_offsets - 1] != n_tokens) return -1;
  const Geometry g = geometry(model);
  const size_t B = n_offsets - 1;
  std::atomic<bool> ok{true};
  std::atomic<size_t> next{0};
  auto work = [&] {
    Scratch s;
    std::vector<float> enc;
    for (;;) {
      const size_t b = next.fetch_add(1);
      if (b >= B) return;
      const size_t L = offsets[b + 1] - offsets[b];
      if (!encode_sentence(model, g, tokens + offsets[b], L, encoder_order(order), nullptr, s, enc)) ok = false;
      else std::memcpy(out + (size_t)offsets[b] * g.d, enc.data(), L * g.d * sizeof(float));
    }
  };
  std::vector<std::thread> workers;
  for (int i = 1; i < std::max(1, threads); ++i) workers.emplace_back(work);
  work();
  for (auto& w : workers) w.join();
  return ok ? 0 : -2;
}

int oracle_last_step_logits(const oracle_model* model, const int32_t* tokens, size_t n_tokens,
                            uint32_t steps, uint32_t flags, int order, float* logits) {
  if (!model_ok(model) || steps == 0 || n_tokens == 0) return -1;
  const Geometry g = geometry(model);
  Scratch s;
  std::vector<float> enc;
  std::vector<int32_t> out;
  if (!encode_sentence(model, g, tokens, n_tokens, encoder_order(order), nullptr, s, enc)) return -2;
  if (!decode_sentence(model, g, enc.data(), n_tokens, steps, flags | ORACLE_FLAG_IGNORE_EOS,
                       order, nullptr, s, out, steps, (int64_t)steps - 1, logits, nullptr))
    return -2;
  return 0;
}

// ---------------------------------------------------------------------------
// Reference-schedule execution (timed CPU baseline).  Mirrors
// Q8CpuEngine::translate_token_ids: pad to [batch x Lmax] with token 0
// (q8_engine.rs:511-524), run every encoder GEMM over all padded rows, mask
// keys by length, then decode all rows every step (q8_engine.rs:382-451) and
// score only unfinished rows with the scalar dot (q8_arm.rs:50-55).
// ---------------------------------------------------------------------------
int oracle_translate_reference_schedule(
    const oracle_model* model, const int32_t* tokens, size_t n_tokens, const uint32_t* offsets,
    size_t n_offsets, const uint32_t* max_output_tokens, const oracle_limits* limits,
    uint32_t flags, int order, int threads, int32_t* out_tokens, size_t out_cap,
    uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap) {
  Err e{err, err_cap};
  if (!model_ok(model)) return e.fail(-2, "invalid model description");
  std::vector<uint32_t> lim;
  int rc = validate(model, tokens, n_tokens, offsets, n_offsets, max_output_tokens, limits, lim, e);
  if (rc) return rc;
  if (!have_avx2()) return e.fail(-2, "the reference x86 schedule needs AVX2");
  const Geometry g = geometry(model);
  const size_t d = g.d, B = n_offsets - 1;
  Pool pool(threads);
  Scratch s;
  const auto& pos = positions_for(model->dim);
  std::vector<size_t> len(B);
  size_t Lmax = 0;
  for (size_t b = 0; b < B; ++b) {
    len[b] = offsets[b + 1] - offsets[b];
    Lmax = std::max(Lmax, len[b]);
  }
  const size_t R = B * Lmax;
  std::vector<float> x(R * d), qkv(R * 3 * d), att(R * d), y(R * d), h(R * g.F), x2(R * d);
  for (size_t b = 0; b < B; ++b)
    for (size_t i = 0; i < Lmax; ++i) {
      const int32_t t = i < len[b] ? tokens[offsets[b] + i] : 0;
      embed_row(model, g, t, pos.data() + i * d, x.data() + (b * Lmax + i) * d);
    }
  const float scale = 1.0f / std::sqrt((float)g.dh);
  std::vector<float> sc;
  auto fail = [&] { return e.fail(-2, "non-finite activation or accumulator overflow"); };
  for (size_t l = 0; l < g.Le; ++l) {
    const oracle_encoder_layer& E = model->encoder[l];
    if (!linear_reference(&pool, s, x.data(), R, d, &E.qkv, 3 * d, false, qkv.data())) return fail();
    for (size_t b = 0; b < B; ++b)
      for (size_t i = 0; i < Lmax; ++i)
        for (size_t hd = 0; hd < g.H; ++hd) {
          const size_t row = b * Lmax + i;
          attend_one(qkv.data() + row * 3 * d + hd * g.dh,
                     qkv.data() + b * Lmax * 3 * d + d + hd * g.dh, 3 * d,
                     qkv.data() + b * Lmax * 3 * d + 2 * d + hd * g.dh, 3 * d, len[b], g.dh,
                     scale, order, att.data() + row * d + hd * g.dh, sc);
        }
    if (!linear_reference(&pool, s, att.data(), R, d, &E.out, d, false, y.data())) return fail();
    residual_ln(y.data(), x.data(), E.ln1_scale, E.ln1_bias, R, d, order, x2.data());
    if (!linear_reference(&pool, s, x2.data(), R, d, &E.ffn1, g.F, true, h.data())) return fail();
    if (!linear_reference(&pool, s, h.data(), R, g.F, &E.ffn2, d, false, y.data())) return fail();
    residual_ln(y.data(), x2.data(), E.ln2_scale, E.ln2_bias, R, d, order, x.data());
  }
  std::vector<std::vector<float>> ckv(g.Ld, std::vector<float>(R * 2 * d));
  for (size_t l = 0; l < g.Ld; ++l)
    if (!linear_reference(&pool, s, x.data(), R, d, &model->decoder[l].cross_kv, 2 * d, false,
                          ckv[l].data()))
      return fail();

  uint32_t gen_limit = 0;
  for (uint32_t v : lim) gen_limit = std::max(gen_limit, v);
  std::vector<std::vector<float>> kc(g.Ld, std::vector<float>((size_t)B * gen_limit * d)),
      vc(g.Ld, std::vector<float>((size_t)B * gen_limit * d));
  std::vector<int32_t> prev(B, -1);
  std::vector<char> finished(B, 0);
  std::vector<std::vector<int32_t>> gen(B);
  std::vector<float> dx(B * d), dqkv(B * 3 * d), datt(B * d), dy(B * d), dx2(B * d),
      dh(B * g.F), dqc(B * d);
  std::vector<uint8_t> qu(d);
  for (uint32_t t = 0; t < gen_limit; ++t) {
    bool all = true;
    for (size_t b = 0; b < B; ++b) {
      if (!finished[b] && t >= lim[b]) finished[b] = 1;
      all = all && finished[b];
    }
    if (all) break;
    for (size_t b = 0; b < B; ++b) {
      if (prev[b] < 0)
        std::memcpy(dx.data() + b * d, pos.data() + (size_t)t * d, d * sizeof(float));
      else
        embed_row(model, g, prev[b], pos.data() + (size_t)t * d, dx.data() + b * d);
    }
    for (size_t l = 0; l < g.Ld; ++l) {
      const oracle_decoder_layer& D = model->decoder[l];
      if (!linear_reference(&pool, s, dx.data(), B, d, &D.self_qkv, 3 * d, false, dqkv.data()))
        return fail();
      for (size_t b = 0; b < B; ++b) {
        std::memcpy(kc[l].data() + ((size_t)b * gen_limit + t) * d, dqkv.data() + b * 3 * d + d,
                    d * sizeof(float));
        std::memcpy(vc[l].data() + ((size_t)b * gen_limit + t) * d,
                    dqkv.data() + b * 3 * d + 2 * d, d * sizeof(float));
        for (size_t hd = 0; hd < g.H; ++hd)
          attend_one(dqkv.data() + b * 3 * d + hd * g.dh,
                     kc[l].data() + (size_t)b * gen_limit * d + hd * g.dh, d,
                     vc[l].data() + (size_t)b * gen_limit * d + hd * g.dh, d, (size_t)t + 1, g.dh,
                     scale, order, datt.data() + b * d + hd * g.dh, sc);
      }
      if (!linear_reference(&pool, s, datt.data(), B, d, &D.self_out, d, false, dy.data()))
        return fail();
      residual_ln(dy.data(), dx.data(), D.ln1_scale, D.ln1_bias, B, d, order, dx2.data());
      if (!linear_reference(&pool, s, dx2.data(), B, d, &D.cross_q, d, false, dqc.data()))
        return fail();
      for (size_t b = 0; b < B; ++b)
        for (size_t hd = 0; hd < g.H; ++hd)
          attend_one(dqc.data() + b * d + hd * g.dh, ckv[l].data() + b * Lmax * 2 * d + hd * g.dh,
                     2 * d, ckv[l].data() + b * Lmax * 2 * d + d + hd * g.dh, 2 * d, len[b], g.dh,
                     scale, order, datt.data() + b * d + hd * g.dh, sc);
      if (!linear_reference(&pool, s, datt.data(), B, d, &D.cross_out, d, false, dy.data()))
        return fail();
      residual_ln(dy.data(), dx2.data(), D.ln2_scale, D.ln2_bias, B, d, order, dx.data());
      if (!linear_reference(&pool, s, dx.data(), B, d, &D.ffn1, g.F, true, dh.data())) return fail();
      if (!linear_reference(&pool, s, dh.data(), B, g.F, &D.ffn2, d, false, dy.data()))
        return fail();
      residual_ln(dy.data(), dx.data(), D.ln3_scale, D.ln3_bias, B, d, order, dx2.data());
      dx.swap(dx2);
    }
    for (size_t b = 0; b < B; ++b) {
      if (finished[b]) continue;
      // Scalar scoring as on x86 (q8_engine.rs:761-788, q8_arm.rs:50-55).
      std::vector<int8_t> q(d);
      float a;
      if (!quantize_row(dx.data() + b * d, d, q.data(), &a)) return fail();
      for (size_t i = 0; i < d; ++i) qu[i] = (uint8_t)((int)q[i] + 127);
      int32_t best = -1;
      float best_v = -INFINITY;
      for (size_t v = 0; v < g.V; ++v) {
        if (generation_masked(v, flags)) continue;
        if (best < 0) best = (int32_t)v;
        const int32_t acc = oracle_dot_u8_i8(qu.data(), model->embedding + v * d, d);
        const float logit = (float)acc * (1.0f / (a * model->embedding_mult[v])) +
                            model->output_bias[v];
        if (logit > best_v) {
          best_v = logit;
          best = (int32_t)v;
        }
      }
      const int32_t token = best < 0 ? 0 : best;
      prev[b] = token;
      gen[b].push_back(token);
      if (token == 0 && !(flags & ORACLE_FLAG_IGNORE_EOS)) finished[b] = 1;
    }
  }
  return pack_output(gen, out_tokens, out_cap, out_offsets, out_len, e);
}


int oracle_translate_ssru(const oracle_ssru_model* model, const int32_t* tokens, size_t n_tokens,
                          const uint32_t* offsets, size_t n_offsets,
                          const uint32_t* max_output_tokens, const oracle_limits* limits,
                          uint32_t flags, int order, int threads, const uint32_t* candidates,
                          const uint32_t* cand_offsets, int32_t* out_tokens, size_t out_cap,
                          uint32_t* out_offsets, size_t* out_len, char* err, size_t err_cap,
                          uint32_t probe_step, float* enc_out, float* logits_out,
                          uint8_t* active_out) {
  Err e{err, err_cap};
  if (!ssru_model_ok(model)) return e.fail(-2, "invalid model description");
  // validate_batch (q8_engine.rs:468-509) checks source ids against the
  // source vocabulary; the shared checks take it from a transformer view.
  oracle_model view{};
  view.vocab = model->source_vocab;
  std::vector<uint32_t> lim;
  int rc = validate(&view, tokens, n_tokens, offsets, n_offsets, max_output_tokens, limits, lim, e);
  if (rc) return rc;
  const SsruGeometry g = ssru_geometry(model);
  const size_t B = n_offsets - 1;
  if (candidates) {
    if (!cand_offsets || cand_offsets[0] != 0) return e.fail(-1, "invalid candidate offsets");
    for (size_t b = 0; b < B; ++b) {
      if (cand_offsets[b + 1] <= cand_offsets[b])
        return e.fail(-1, "cannot select from an empty candidate list");
      for (uint32_t i = cand_offsets[b]; i < cand_offsets[b + 1]; ++i)
        if (candidates[i] >= g.Vt)
          return e.fail(-1, "output candidate %u exceeds vocabulary %zu", candidates[i], g.Vt);
    }
  }
  std::vector<std::vector<int32_t>> gen(B);
  std::atomic<bool> ok{true};
  std::atomic<size_t> next{0};
  auto work = [&] {
    Scratch s;
    std::vector<float> enc;
    for (;;) {
      const size_t b = next.fetch_add(1);
      if (b >= B) return;
      const size_t L = offsets[b + 1] - offsets[b];
      if (!encode_sentence_ssru(model, g, tokens + offsets[b], L, encoder_order(order), nullptr, s, enc)) {
        ok = false;
        continue;
      }
      if (enc_out) std::memcpy(enc_out + (size_t)offsets[b] * g.d, enc.data(), L * g.d * sizeof(float));
      const uint32_t* c = candidates ? candidates + cand_offsets[b] : nullptr;
      const size_t nc = candidates ? cand_offsets[b + 1] - cand_offsets[b] : 0;
      bool probed = false;
      if (!decode_sentence_ssru(model, g, enc.data(), L, lim[b], flags, order, nullptr, s, c, nc,
                                gen[b], probe_step, logits_out ? logits_out + b * g.Vt : nullptr,
                                &probed))
        ok = false;
      if (active_out) active_out[b] = probed ? 1 : 0;
    }
  };
  std::vector<std::thread> workers;
  for (int i = 1; i < std::max(1, threads); ++i) workers.emplace_back(work);
  work();
  for (auto& w : workers) w.join();
  if (!ok) return e.fail(-2, "non-finite activation or accumulator overflow");
  return pack_output(gen, out_tokens, out_cap, out_offsets, out_len, e);
}

// ---------------------------------------------------------------------------
// The Transformer-SSRU graph on the reference schedule (timed CPU baseline).
// Mirrors Q8CpuEngine::translate_token_ids (q8_engine.rs:353-466): the batch
// padded to [batch x Lmax] with token 0 (encode, :511-558), every encoder and
// cross-projection GEMM over all padded rows, keys masked by length; then
// every row decoded at every step, finished or not (:382-436), and only the
// unfinished rows scored over their candidates with the scalar u8 x i8 dot
// (select_token, :749-790; q8_arm.rs:50-55).  Same tokens as
// oracle_translate_ssru.
// ---------------------------------------------------------------------------
int oracle_translate_ssru_reference_schedule(
    const oracle_ssru_model* model, const int32_t* tokens, size_t n_tokens, const uint32_t* offsets,
    size_t n_offsets, const uint32_t* max_output_tokens, const oracle_limits* limits, uint32_t flags,
    int order, int threads, const uint32_t* candidates, const uint32_t* cand_offsets,
    int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets, size_t* out_len, char* err,
    size_t err_cap) {
  Err e{err, err_cap};
  if (!ssru_model_ok(model)) return e.fail(-2, "invalid model description");
  oracle_model view{};
  view.vocab = model->source_vocab;
  std::vector<uint32_t> lim;
  int rc = validate(&view, tokens, n_tokens, offsets, n_offsets, max_output_tokens, limits, lim, e);
  if (rc) return rc;
  if (!have_avx2()) return e.fail(-2, "the reference x86 schedule needs AVX2");
  const SsruGeometry g = ssru_geometry(model);
  const size_t d = g.d, B = n_offsets - 1;
  if (candidates) {
    if (!cand_offsets || cand_offsets[0] != 0) return e.fail(-1, "invalid candidate offsets");
    for (size_t b = 0; b < B; ++b) {
      if (cand_offsets[b + 1] <= cand_offsets[b])
        return e.fail(-1, "cannot select from an empty candidate list");
      for (uint32_t i = cand_offsets[b]; i < cand_offsets[b + 1]; ++i)
        if (candidates[i] >= g.Vt)
          return e.fail(-1, "output candidate %u exceeds vocabulary %zu", candidates[i], g.Vt);
    }
  }
  Pool pool(threads);
  Scratch s;
  const auto& pos = positions_for(model->dim);
  std::vector<size_t> len(B);
  size_t Lmax = 0;
  for (size_t b = 0; b < B; ++b) {
    len[b] = offsets[b + 1] - offsets[b];
    Lmax = std::max(Lmax, len[b]);
  }
  const size_t R = B * Lmax;
  std::vector<float> x(R * d), q(R * d), k(R * d), v(R * d), att(R * d), y(R * d), h(R * g.F),
      x2(R * d), sc;
  for (size_t b = 0; b < B; ++b)
    for (size_t i = 0; i < Lmax; ++i) {
      const int32_t t = i < len[b] ? tokens[offsets[b] + i] : 0;
      embed_static(model->encoder_embedding, model->encoder_embedding_mult, d, g.emb_scale, t,
                   pos.data() + i * d, x.data() + (b * Lmax + i) * d);
    }
  auto fail = [&] { return e.fail(-2, "non-finite activation or accumulator overflow"); };
  for (size_t l = 0; l < g.Le; ++l) {
    const oracle_ssru_encoder_layer& E = model->encoder[l];
    if (!linear_static_reference(&pool, s, x.data(), R, d, &E.wq, d, false, q.data()) ||
        !linear_static_reference(&pool, s, x.data(), R, d, &E.wk, d, false, k.data()) ||
        !linear_static_reference(&pool, s, x.data(), R, d, &E.wv, d, false, v.data()))
      return fail();
    for (size_t b = 0; b < B; ++b)  // every padded query row, keys masked to the length
      attend_rows(q.data() + b * Lmax * d, k.data() + b * Lmax * d, v.data() + b * Lmax * d, Lmax,
                  len[b], g, order, att.data() + b * Lmax * d, sc);
    if (!linear_static_reference(&pool, s, att.data(), R, d, &E.wo, d, false, y.data())) return fail();
    residual_ln(y.data(), x.data(), E.attn_ln_scale, E.attn_ln_bias, R, d, order, x2.data());
    if (!linear_static_reference(&pool, s, x2.data(), R, d, &E.w1, g.F, true, h.data()) ||
        !linear_static_reference(&pool, s, h.data(), R, g.F, &E.w2, d, false, y.data()))
      return fail();
    residual_ln(y.data(), x2.data(), E.ffn_ln_scale, E.ffn_ln_bias, R, d, order, x.data());
  }
  std::vector<std::vector<float>> ck(g.Ld, std::vector<float>(R * d)), cv(g.Ld, std::vector<float>(R * d));
  for (size_t l = 0; l < g.Ld; ++l)
    if (!linear_static_reference(&pool, s, x.data(), R, d, &model->decoder[l].wk, d, false, ck[l].data()) ||
        !linear_static_reference(&pool, s, x.data(), R, d, &model->decoder[l].wv, d, false, cv[l].data()))
      return fail();

  uint32_t gen_limit = 0;
  for (uint32_t l : lim) gen_limit = std::max(gen_limit, l);
  std::vector<std::vector<float>> state(g.Ld, std::vector<float>(B * d, 0.0f));
  std::vector<int32_t> prev(B, -1);
  std::vector<char> finished(B, 0);
  std::vector<std::vector<int32_t>> gen(B);
  std::vector<float> dx(B * d), du(B * d), df(B * d), dx1(B * d), dq(B * d), datt(B * d), dy(B * d),
      dx2(B * d), dh(B * g.F);
  std::vector<uint8_t> qu(d);
  const float inv_out = 1.0f / (model->output_act_mult * model->decoder_embedding_mult);
  for (uint32_t t = 0; t < gen_limit; ++t) {
    bool all = true;
    for (size_t b = 0; b < B; ++b) {
      if (!finished[b] && t >= lim[b]) finished[b] = 1;
      all = all && finished[b];
    }
    if (all) break;
    for (size_t b = 0; b < B; ++b) {
      if (prev[b] < 0)
        std::memcpy(dx.data() + b * d, pos.data() + (size_t)t * d, d * sizeof(float));
      else
        embed_static(model->decoder_embedding, model->decoder_embedding_mult, d, g.emb_scale, prev[b],
                     pos.data() + (size_t)t * d, dx.data() + b * d);
    }
    for (size_t l = 0; l < g.Ld; ++l) {
      const oracle_ssru_decoder_layer& D = model->decoder[l];
      if (!linear_static_reference(&pool, s, dx.data(), B, d, &D.ssru_w, d, false, du.data()) ||
          !linear_static_reference(&pool, s, dx.data(), B, d, &D.ssru_wf, d, false, df.data()))
        return fail();
      oracle_ssru_layer_norm(du.data(), df.data(), state[l].data(), dx.data(), D.ssru_ln_scale,
                             D.ssru_ln_bias, B, d, order, dx1.data());
      if (!linear_static_reference(&pool, s, dx1.data(), B, d, &D.wq, d, false, dq.data())) return fail();
      for (size_t b = 0; b < B; ++b)
        attend_rows(dq.data() + b * d, ck[l].data() + b * Lmax * d, cv[l].data() + b * Lmax * d, 1,
                    len[b], g, order, datt.data() + b * d, sc);
      if (!linear_static_reference(&pool, s, datt.data(), B, d, &D.wo, d, false, dy.data())) return fail();
      residual_ln(dy.data(), dx1.data(), D.context_ln_scale, D.context_ln_bias, B, d, order, dx2.data());
      if (!linear_static_reference(&pool, s, dx2.data(), B, d, &D.w1, g.F, true, dh.data()) ||
          !linear_static_reference(&pool, s, dh.data(), B, g.F, &D.w2, d, false, dy.data()))
        return fail();
      residual_ln(dy.data(), dx2.data(), D.ffn_ln_scale, D.ffn_ln_bias, B, d, order, dx.data());
    }
    for (size_t b = 0; b < B; ++b) {
      if (finished[b]) continue;
      const float* st = dx.data() + b * d;
      for (size_t i = 0; i < d; ++i) {
        if (!std::isfinite(st[i])) return fail();
        qu[i] = (uint8_t)((int)quantize_one(st[i], model->output_act_mult) + 127);
      }
      const uint32_t* c = candidates ? candidates + cand_offsets[b] : nullptr;
      const size_t nc = candidates ? cand_offsets[b + 1] - cand_offsets[b] : g.Vt;
      int32_t best = -1;
      float best_v = -INFINITY;
      for (size_t i = 0; i < nc; ++i) {
        const size_t id = c ? c[i] : i;
        if (!c && generation_masked(id, flags)) continue;
        const int32_t acc = oracle_dot_u8_i8(qu.data(), model->decoder_embedding + id * d, d);
        const float lg = (float)acc * inv_out + model->output_bias[id];
        if (best < 0) best = (int32_t)id;
        if (lg > best_v) {
          best_v = lg;
          best = (int32_t)id;
        }
      }
      const int32_t token = best < 0 ? 0 : best;
      prev[b] = token;
      gen[b].push_back(token);
      if (token == 0 && !(flags & ORACLE_FLAG_IGNORE_EOS)) finished[b] = 1;
    }
  }
  return pack_output(gen, out_tokens, out_cap, out_offsets, out_len, e);
}

}  // extern "C"
