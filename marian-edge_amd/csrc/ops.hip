// ops.hip — op-level entry points (device pointers, caller's stream) and the
// device-memory helpers of marian_hip_util.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "../../include/marian_hip.h"
#include "../../include/marian_hip_util.h"
#include "device_common.h"
#include "kernels.h"

using namespace mh;

namespace {

thread_local std::string g_op_error;

int op_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MARIAN_HIP_OK;
  g_op_error = std::string(what) + ": " + hipGetErrorString(e);
  return e == hipErrorInvalidValue ? MARIAN_HIP_ERR_INVALID_INPUT : MARIAN_HIP_ERR_DEVICE;
}

// Library scratch for the op-level entry points that need intermediate
// buffers (quantized activations, argmax partials).  Grow-only, one set per
// (device, stream), so calls on different streams never share a buffer; a
// call's kernels run in its stream's order, so calls on one stream reuse the
// set safely.  A buffer that grows is freed once its stream has drained.
// Sets live until the process ends (a stream that is destroyed leaves its
// set behind).
struct OpScratch {
  void* p[4] = {nullptr, nullptr, nullptr, nullptr};
  size_t cap[4] = {0, 0, 0, 0};
};
std::mutex g_scratch_mu;
std::map<std::pair<int, uintptr_t>, OpScratch> g_scratch;

void* op_scratch(int which, size_t bytes, hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return nullptr;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  OpScratch& S = g_scratch[{dev, (uintptr_t)s}];
  if (S.cap[which] >= bytes && S.p[which]) return S.p[which];
  if (S.p[which]) {
    hipStreamSynchronize(s);  // the stream's earlier calls are done with it
    hipFree(S.p[which]);
    S.p[which] = nullptr;
    S.cap[which] = 0;
  }
  const size_t want = std::max<size_t>(bytes + bytes / 4, 4096);
  if (hipMalloc(&S.p[which], want) != hipSuccess) {
    S.p[which] = nullptr;
    return nullptr;
  }
  S.cap[which] = want;
  return S.p[which];
}

// Partial argmax keys of marian_hip_vocab_argmax_noalloc, one u64 per (row,
// 128-column vocabulary group): a fixed 1 MiB that each device holds for the
// life of the process.  In host code `scratch` is only a handle for
// hipGetSymbolAddress; kernels get the device address it returns.
constexpr size_t kNoAllocPartials = 131072;
static __device__ __align__(256) uint64_t scratch[kNoAllocPartials];

std::mutex g_noalloc_mu;
void* g_noalloc_ptr[64] = {};  // device address of `scratch` on each device

// Address of `scratch` on the current device, looked up on the first call
// with that device current and kept; nullptr if the lookup fails.
void* noalloc_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      op_status(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
      return nullptr;
    }
    g_noalloc_ptr[dev] = ptr;
  }
  return g_noalloc_ptr[dev];
}

// Vocabulary projection + argmax with the partial keys in `part` (M * nparts).
int vocab_argmax_into(const int8_t* xq, const float* xa, int64_t M, int64_t K, const int8_t* emb,
                      const float* emb_mult, const float* bias, int64_t V, uint32_t flags,
                      int32_t* token, float* logits, uint64_t* part, int nparts, hipStream_t s) {
  GemmArgs g;
  g.A = xq;
  g.a = xa;
  g.lda = K;
  g.M = (int)M;
  g.K = (int)K;
  g.W = emb;
  g.wmult = emb_mult;
  g.bias = bias;
  g.N = (int)V;
  Epilogue e;
  e.partials = part;
  e.partial_ld = nparts;
  e.logits = logits;
  e.ldl = V;
  e.flags = flags;
  int rc = op_status(launch_gemm_skinny(g, EPI_ARGMAX, e, s), "vocab_argmax gemm");
  if (rc) return rc;
  return op_status(launch_argmax_reduce(part, nparts, (int)M, token, s), "vocab_argmax reduce");
}

bool vocab_args_ok(const int8_t* xq, const float* xa, int64_t M, int64_t K, const int8_t* emb,
                   const float* emb_mult, const float* bias, int64_t V, const int32_t* token) {
  return xq && xa && emb && emb_mult && bias && token && M >= 0 && K > 0 && K % 64 == 0 &&
         K <= 512 && V > 0 && M <= INT32_MAX && V <= INT32_MAX;
}

}  // namespace

void mh::note_op_error(const char* msg) { g_op_error = msg ? msg : ""; }

extern "C" {

int marian_hip_quantize_rows(const float* x, int64_t rows, int64_t cols, int8_t* q, float* a,
                             int* err, void* stream) {
  if (!x || !q || !a || rows < 0 || cols <= 0 || rows > INT32_MAX || cols > INT32_MAX)
    return MARIAN_HIP_ERR_INVALID_INPUT;
  return op_status(launch_quantize_rows(x, cols, (int)rows, nullptr, (int)cols, q, cols, a, err,
                                        (hipStream_t)stream),
                   "quantize_rows");
}

int marian_hip_q8_linear(const float* x, const int8_t* xq, const float* xa, int64_t M, int64_t K,
                         const int8_t* w, const float* w_mult, const float* bias, int64_t N,
                         int relu, int32_t* out_i32, float* out_f32, int* err, void* stream) {
  if (M < 0 || K <= 0 || K % 64 || N <= 0 || !w || !w_mult || !bias || M > INT32_MAX ||
      N > INT32_MAX || K > INT32_MAX || (!x && (!xq || !xa)) || (!out_i32 && !out_f32))
    return MARIAN_HIP_ERR_INVALID_INPUT;
  if (M == 0) return MARIAN_HIP_OK;
  hipStream_t s = (hipStream_t)stream;
  if (x) {
    int8_t* q = (int8_t*)op_scratch(0, (size_t)M * K, s);
    float* a = (float*)op_scratch(1, (size_t)M * 4, s);
    if (!q || !a) return op_status(hipErrorOutOfMemory, "q8_linear scratch");
    int rc = op_status(launch_quantize_rows(x, K, (int)M, nullptr, (int)K, q, K, a, err, s),
                       "q8_linear quantize");
    if (rc) return rc;
    xq = q;
    xa = a;
  }
  GemmArgs g;
  g.A = xq;
  g.a = xa;
  g.lda = K;
  g.M = (int)M;
  g.K = (int)K;
  g.W = w;
  g.wmult = w_mult;
  g.bias = bias;
  g.N = (int)N;
  Epilogue e;
  e.out = out_f32;
  e.ldo = N;
  e.out_i32 = out_i32;
  e.ldi = N;
  e.relu = relu;
  return op_status(launch_gemm_store(g, e, s), "q8_linear gemm");
}

int marian_hip_q8_linear_static(const float* x, int64_t M, int64_t K, float act_mult,
                                const int8_t* w, const float* w_mult, const float* bias, int64_t N,
                                int relu, int32_t* out_i32, float* out_f32, int* err, void* stream) {
  if (!x || M < 0 || K <= 0 || K % 64 || N <= 0 || !w || !w_mult || !bias || M > INT32_MAX ||
      N > INT32_MAX || K > INT32_MAX || (!out_i32 && !out_f32) || !(act_mult > 0.0f) ||
      !std::isfinite(act_mult))
    return MARIAN_HIP_ERR_INVALID_INPUT;
  if (M == 0) return MARIAN_HIP_OK;
  hipStream_t s = (hipStream_t)stream;
  int8_t* q = (int8_t*)op_scratch(0, (size_t)M * K, s);
  float* a = (float*)op_scratch(1, (size_t)M * 4, s);
  if (!q || !a) return op_status(hipErrorOutOfMemory, "q8_linear_static scratch");
  int rc = op_status(launch_quantize_rows_static(x, K, (int)M, (int)K, act_mult, q, K, a, err, s),
                     "q8_linear_static quantize");
  if (rc) return rc;
  GemmArgs g;
  g.A = q;
  g.a = a;
  g.lda = K;
  g.M = (int)M;
  g.K = (int)K;
  g.W = w;
  g.wmult = w_mult;
  g.bias = bias;
  g.N = (int)N;
  Epilogue e;
  e.out = out_f32;
  e.ldo = N;
  e.out_i32 = out_i32;
  e.ldi = N;
  e.relu = relu;
  return op_status(launch_gemm_store(g, e, s), "q8_linear_static gemm");
}

int marian_hip_ssru_layer_norm(const float* cand, const float* forget, float* state,
                               const float* residual, const float* scale, const float* bias,
                               int64_t rows, int64_t dim, float* out, int8_t* q, float* a, int* err,
                               void* stream) {
  if (!cand || !forget || !state || !residual || !scale || !bias || !out || rows < 0 ||
      rows > INT32_MAX || dim <= 0 || dim % 64 || dim > 1024 || (q && !a))
    return MARIAN_HIP_ERR_INVALID_INPUT;
  return op_status(launch_ssru_ln(cand, forget, state, residual, scale, bias, (int)rows, (int)dim, out,
                                  q, a, err, (hipStream_t)stream),
                   "ssru_layer_norm");
}

int marian_hip_residual_layer_norm(const float* x, const float* r, const float* scale,
                                   const float* bias, int64_t rows, int64_t dim, float* out,
                                   int8_t* q, float* a, int* err, void* stream) {
  if (!x || !r || !scale || !bias || !out || rows < 0 || rows > INT32_MAX || dim % 64 ||
      dim <= 0 || dim > 1024 || (q && !a))
    return MARIAN_HIP_ERR_INVALID_INPUT;
  return op_status(launch_residual_ln(x, r, scale, bias, (int)rows, nullptr, (int)dim, out, q, a,
                                      err, (hipStream_t)stream),
                   "residual_layer_norm");
}

int marian_hip_attention(const void* q, int64_t ldq, const void* k, const void* v, int64_t ldkv,
                         const int32_t* seq_of_row, const uint32_t* cu_k, int64_t n_seqs,
                         int64_t rows, int64_t heads, int64_t head_dim, int64_t max_keys,
                         int in_bf16, float* out, int64_t ldo, void* stream) {
  if (!q || !k || !v || !seq_of_row || !cu_k || !out || rows < 0 || rows > INT32_MAX ||
      heads <= 0 || heads > 16 || (head_dim != 64 && head_dim != 48) || ldq % 8 || ldkv % 8 ||
      max_keys <= 0 || max_keys > 4096 || n_seqs < 0 || n_seqs > 16 * 1024)
    return MARIAN_HIP_ERR_INVALID_INPUT;
  AttnArgs a;
  a.mode = ATT_SEQ;
  a.q = q;
  a.ldq = ldq;
  a.k = k;
  a.v = v;
  a.ldkv = ldkv;
  a.bf16 = in_bf16 ? 1 : 0;
  a.heads = (int)heads;
  a.head_dim = (int)head_dim;
  a.rows = (int)rows;
  a.seq_of_row = seq_of_row;
  a.cu = cu_k;
  a.out = out;
  a.ldo = ldo;
  a.max_keys = (int)max_keys;
  if (n_seqs > 0 && rows > 0 && max_keys <= 256) {
    // Packed self-attention: the query-tile list first (library scratch).
    const int cap = seq_tiles_bound((int)rows, (int)n_seqs);
    uint32_t* tiles = (uint32_t*)op_scratch(3, (1 + 2 * (size_t)cap) * 4, (hipStream_t)stream);
    if (!tiles) return op_status(hipErrorOutOfMemory, "attention scratch");
    const int rc = op_status(launch_seq_tiles(cu_k, (int)n_seqs, tiles, cap, (hipStream_t)stream),
                             "attention tiles");
    if (rc != MARIAN_HIP_OK) return rc;
    a.tiles = tiles;
    a.tiles_cap = cap;
  }
  return op_status(launch_attention(a, (hipStream_t)stream), "attention");
}

int marian_hip_vocab_argmax(const int8_t* xq, const float* xa, int64_t M, int64_t K,
                            const int8_t* emb, const float* emb_mult, const float* bias, int64_t V,
                            uint32_t flags, int32_t* token, float* logits, void* stream) {
  if (!vocab_args_ok(xq, xa, M, K, emb, emb_mult, bias, V, token)) return MARIAN_HIP_ERR_INVALID_INPUT;
  if (M == 0) return MARIAN_HIP_OK;
  hipStream_t s = (hipStream_t)stream;
  const int nparts = argmax_groups((int)V, (int)K);
  uint64_t* part = (uint64_t*)op_scratch(2, (size_t)M * nparts * 8, s);
  if (!part) return op_status(hipErrorOutOfMemory, "vocab_argmax scratch");
  return vocab_argmax_into(xq, xa, M, K, emb, emb_mult, bias, V, flags, token, logits, part, nparts, s);
}

int marian_hip_candidate_argmax(const int8_t* xq, const float* xa, int64_t M, int64_t K,
                                const int8_t* emb, const float* emb_mult, const float* bias,
                                int64_t V, const uint32_t* cand, const uint32_t* cand_offsets,
                                int64_t max_cands, int32_t* token, float* logits, int* err,
                                void* stream) {
  if (!xq || !xa || !emb || !emb_mult || !bias || !cand || !cand_offsets || !token || M < 0 ||
      M > 65535 || K <= 0 || K % 64 || K > 4096 || V <= 0 || V > INT32_MAX || max_cands <= 0 ||
      max_cands > INT32_MAX / 2)
    return MARIAN_HIP_ERR_INVALID_INPUT;
  if (M == 0) return MARIAN_HIP_OK;
  hipStream_t s = (hipStream_t)stream;
  const int nparts = cand_groups((int)max_cands);
  uint64_t* part = (uint64_t*)op_scratch(2, (size_t)M * nparts * 8, s);
  if (!part) return op_status(hipErrorOutOfMemory, "candidate_argmax scratch");
  CandArgs c;
  c.xq = xq;
  c.xa = xa;
  c.M = (int)M;
  c.K = (int)K;
  c.V = (int)V;
  c.emb = emb;
  c.mult = emb_mult;
  c.bias = bias;
  c.cand = cand;
  c.off = cand_offsets;
  c.max_cands = (int)max_cands;
  c.partials = part;
  c.nparts = nparts;
  c.logits = logits;
  c.err = err;
  int rc = op_status(launch_cand_argmax(c, s), "candidate_argmax");
  if (rc) return rc;
  return op_status(launch_argmax_reduce(part, nparts, (int)M, token, s), "candidate_argmax reduce");
}

int marian_hip_vocab_argmax_noalloc(const int8_t* xq, const float* xa, int64_t M, int64_t K,
                                    const int8_t* emb, const float* emb_mult, const float* bias,
                                    int64_t V, uint32_t flags, int32_t* token, float* logits,
                                    void* stream) {
  if (!vocab_args_ok(xq, xa, M, K, emb, emb_mult, bias, V, token)) return MARIAN_HIP_ERR_INVALID_INPUT;
  if (M == 0) return MARIAN_HIP_OK;
  const int nparts = argmax_groups((int)V, (int)K);
  if ((uint64_t)M * (uint64_t)nparts > kNoAllocPartials) {
    char msg[160];
    snprintf(msg, sizeof msg, "vocab_argmax_noalloc: %lld rows x %d groups exceed the %zu partial keys",
             (long long)M, nparts, kNoAllocPartials);
    g_op_error = msg;
    return MARIAN_HIP_ERR_INVALID_INPUT;
  }
  uint64_t* part = (uint64_t*)noalloc_scratch();
  if (!part) return MARIAN_HIP_ERR_DEVICE;
  return vocab_argmax_into(xq, xa, M, K, emb, emb_mult, bias, V, flags, token, logits, part, nparts,
                           (hipStream_t)stream);
}

// ---- util ------------------------------------------------------------------
int marian_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int marian_hip_device_name(int device, char* buf, size_t cap) {
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return op_status(e, "hipGetDeviceProperties");
  char name[256] = {0};
  if (hipDeviceGetName(name, sizeof name, device) != hipSuccess || !name[0])
    snprintf(name, sizeof name, "%s", p.name);
  if (!name[0]) snprintf(name, sizeof name, "AMD GPU");  // no marketing name visible
  snprintf(buf, cap, "%s (%s)", name, p.gcnArchName);
  return MARIAN_HIP_OK;
}

int marian_hip_set_device(int device) { return op_status(hipSetDevice(device), "hipSetDevice"); }

void* marian_hip_device_alloc(size_t bytes) {
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, std::max<size_t>(bytes, 1));
  if (e != hipSuccess) {
    op_status(e, "hipMalloc");
    return nullptr;
  }
  return p;
}
int marian_hip_device_free(void* p) { return op_status(hipFree(p), "hipFree"); }
int marian_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return op_status(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy h2d");
}
int marian_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return op_status(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy d2h");
}
int marian_hip_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  return op_status(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice), "hipMemcpy d2d");
}
int marian_hip_memset(void* dst, int value, size_t bytes) {
  return op_status(hipMemset(dst, value, bytes), "hipMemset");
}
void* marian_hip_stream_create(void) {
  hipStream_t s = nullptr;
  if (op_status(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return nullptr;
  return s;
}
int marian_hip_stream_destroy(void* s) {
  return op_status(hipStreamDestroy((hipStream_t)s), "hipStreamDestroy");
}
int marian_hip_stream_sync(void* s) {
  return op_status(hipStreamSynchronize((hipStream_t)s), "hipStreamSynchronize");
}
int marian_hip_device_sync(void) { return op_status(hipDeviceSynchronize(), "hipDeviceSynchronize"); }
void* marian_hip_event_create(void) {
  hipEvent_t e = nullptr;
  if (op_status(hipEventCreate(&e), "hipEventCreate")) return nullptr;
  return e;
}
int marian_hip_event_destroy(void* e) { return op_status(hipEventDestroy((hipEvent_t)e), "hipEventDestroy"); }
int marian_hip_event_record(void* e, void* s) {
  return op_status(hipEventRecord((hipEvent_t)e, (hipStream_t)s), "hipEventRecord");
}
int marian_hip_event_sync(void* e) {
  return op_status(hipEventSynchronize((hipEvent_t)e), "hipEventSynchronize");
}
int marian_hip_event_elapsed(void* a, void* b, float* ms) {
  return op_status(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b), "hipEventElapsedTime");
}
const char* marian_hip_last_op_error(void) { return g_op_error.c_str(); }

#ifndef MARIAN_HIP_BUILD_ID
#define MARIAN_HIP_BUILD_ID "unknown"
#endif
const char* marian_hip_build_id(void) { return MARIAN_HIP_BUILD_ID; }

}  // extern "C"
