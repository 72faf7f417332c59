// engine.hip — the marian-hip engine: device-resident Q8 weights, a packed
// (padding-free) encoder, and a greedy decode loop whose active set is
// compacted on the device every step.
//
// Reference behaviour restated here: Q8CpuEngine::translate_token_ids
// (crates/marian-cpu/src/q8_engine.rs:353-466) with validate_batch (:468-509)
// and validate_work_shape (:1103-1119).  Differences in execution (not in
// results): sequences are packed by cu_seqlens instead of padded to the longest
// one, finished rows leave the active set instead of being recomputed, and the
// per-step token selection runs on the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/marian_hip.h"
#include "device_common.h"
#include "kernels.h"

using namespace mh;

namespace {

struct Lin {
  const int8_t* w = nullptr;   // [N, K], K-contiguous
  const int8_t* wf = nullptr;  // the same in MFMA fragment order (decode kernels)
  const float* mult = nullptr;
  const float* bias = nullptr;
  int N = 0, K = 0;
};
struct EncLayer {
  Lin qkv, out, ffn1, ffn2;
  const float *ln1_s, *ln1_b, *ln2_s, *ln2_b;
};
struct DecLayer {
  Lin self_qkv, self_out, cross_q, cross_kv, cross_out, ffn1, ffn2;
  const float *ln1_s, *ln1_b, *ln2_s, *ln2_b, *ln3_s, *ln3_b;
};

// The Transformer-SSRU graph (q8_engine.rs:76-114): dense layers with one
// static activation multiplier each.  Layers that read the same input are row
// blocks of one fused weight; when their multipliers agree (`shared`) one
// quantization and one GEMM serve them all.
struct SGroup {
  Lin all;  // [parts * n, K]
  int parts = 0, n = 0;
  float act[3] = {};
  bool shared = false;
  Lin part(int i) const {
    Lin l = all;
    l.N = n;
    l.w = all.w + (size_t)i * n * all.K;
    l.wf = all.wf ? all.wf + (size_t)i * (n / 16) * (all.K / 64) * 1024 : nullptr;
    l.mult = all.mult + (size_t)i * n;
    l.bias = all.bias + (size_t)i * n;
    return l;
  }
};
struct SEncLayer {
  SGroup qkv;  // Wq, Wk, Wv (q8_engine.rs:528-530)
  Lin o, w1, w2;
  float ao = 0, a1 = 0, a2 = 0;
  const float *ln1_s, *ln1_b, *ln2_s, *ln2_b;
};
struct SDecLayer {
  SGroup uf;   // SSRU W (candidate) and Wf (forget gate input), q8_engine.rs:394-395
  Lin q;       // context Wq
  SGroup kv;   // context Wk, Wv on the encoder output
  Lin o, w1, w2;
  float aq = 0, ao = 0, a1 = 0, a2 = 0;
  const float *ln0_s, *ln0_b, *ln1_s, *ln1_b, *ln2_s, *ln2_b;  // SSRU, context, FFN
};

// Host staging of every tensor the engine uploads: 256-byte aligned pieces of
// one buffer, copied to HBM once; each fix records which engine pointer gets
// which offset.
struct Packer {
  std::vector<char> host;
  struct Fix {
    size_t off;
    const void** dst;
  };
  std::vector<Fix> fixes;
  size_t reserve(size_t bytes, const void** dst) {
    const size_t off = (host.size() + 255) & ~size_t(255);
    host.resize(off + bytes);
    fixes.push_back({off, dst});
    return off;
  }
  void add(const void* src, size_t bytes, const void** dst) {
    const size_t off = reserve(bytes, dst);
    std::memcpy(host.data() + off, src, bytes);
  }
  // The decode kernels read their weights in MFMA fragment order: each
  // 16-column tile and 64-wide k-step is one contiguous 1 KB block, lane l's
  // 16 bytes W[16t + l % 16][64s + 16(l / 16) ..] at ((t * K/64 + s) * 64 + l) * 16.
  void add_frag(const int8_t* w, int N, int K, const int8_t** dst) {
    const int tiles = (N + 15) / 16, ks = K / 64;
    std::vector<int8_t> f((size_t)tiles * ks * 1024, 0);
    for (int t = 0; t < tiles; ++t)
      for (int st = 0; st < ks; ++st)
        for (int l = 0; l < 64; ++l) {
          const int n = 16 * t + (l & 15);
          if (n < N)
            std::memcpy(&f[(((size_t)t * ks + st) * 64 + l) * 16], w + (size_t)n * K + 64 * st + 16 * (l >> 4), 16);
        }
    add(f.data(), f.size(), (const void**)dst);
  }
};

// Records a model error for marian_hip_last_op_error and returns its code.
int model_fail(const char* fmt, ...) {
  char msg[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  note_op_error(msg);
  return MARIAN_HIP_ERR_MODEL;
}

// Grow-only device buffers reused across calls (the reference pools its
// scratch too, q8_engine.rs:733-747).
enum Buf {
  B_META, B_DMETA, B_X0, B_X1, B_XQ, B_XA, B_QKV, B_ATT, B_OQ, B_OA, B_Y, B_H, B_HQ, B_HA, B_CKV,
  B_KC, B_VC, B_DX0, B_DX1, B_DXQ, B_DXA, B_DQ, B_DATT, B_DAMAX, B_DY, B_DH, B_DHQ, B_DHA,
  B_PART, B_OUT, B_COUNT, B_HIST, B_TILES, B_STATE, B_DUF, B_COUNT_,
  // allocated only by marian_hip_translate_probe: the probed step's logits
  // and its active-row order
  B_PLOG = B_COUNT_, B_PSLOT, B_ALL_
};

// What marian_hip_translate_probe copies out besides the tokens.
struct Probe {
  uint32_t step = UINT32_MAX;
  float* enc = nullptr;      // [T, d]
  float* logits = nullptr;   // [B, V]
  uint8_t* active = nullptr; // [B]
};

// Load-time checks of one Q8 tensor (Q8Linear::new, q8_gemm.rs:96-110 with
// validate_quant_mult :592-600; the intgemm8 loader, legacy_q8.rs:384-395):
// no weight is -128 (symmetric range [-127, 127]) and every multiplier is
// finite and positive.  Returns the first problem, or nullptr.
const char* check_q8_tensor(const int8_t* w, const float* mult, size_t N, size_t K) {
  for (size_t n = 0; n < N; ++n)
    if (!(std::isfinite(mult[n]) && mult[n] > 0.0f)) return "weight multiplier is not finite and positive";
  const size_t total = N * K;
  for (size_t i = 0; i < total; ++i)
    if (w[i] == INT8_MIN) return "symmetric Q8 weights must be in [-127, 127]";
  return nullptr;
}

uint32_t host_positions(uint32_t dim, uint32_t count, float* out) {
  if (dim < 4 || dim % 2) return 1;
  const uint32_t half = dim / 2;
  volatile float ten_thousand = 10000.0f;  // evaluated by libm at run time
  const float ln10k = std::log((float)ten_thousand);
  for (uint32_t p = 0; p < count; ++p)
    for (uint32_t i = 0; i < half; ++i) {
      const float f = std::exp(-(float)i * ln10k / (float)(half - 1));
      const float arg = (float)p * f;
      out[(size_t)p * dim + i] = std::sin(arg);
      out[(size_t)p * dim + half + i] = std::cos(arg);
    }
  return 0;
}

}  // namespace

struct marian_hip_engine {
  int device = 0;
  hipStream_t stream = nullptr;
  // V: target vocabulary (scoring, decoder input); Vs: source vocabulary
  uint32_t V = 0, Vs = 0, d = 0, H = 0, F = 0, Le = 0, Ld = 0;
  float emb_scale = 1.0f;
  bool ssru = false;  // the Transformer-SSRU graph with static multipliers
  marian_hip_limits limits{};
  bool ready = true;
  uint32_t timing = 0;  // MARIAN_HIP_TIME_* flags
  std::string error;
  std::string device_name;

  void* weights = nullptr;
  Lin emb;      // decoder input embedding and tied output projection
  Lin src_emb;  // encoder input embedding (the same table in the transformer graph)
  std::vector<EncLayer> enc;
  std::vector<DecLayer> dec;
  std::vector<SEncLayer> senc;
  std::vector<SDecLayer> sdec;
  float out_act = 0.0f;  // static multiplier of the scored decoder state
  float* pos = nullptr;

  void* buf[B_ALL_] = {};
  size_t cap[B_ALL_] = {};
  int* err_flag = nullptr;
  int* pinned = nullptr;  // host-visible n_active polls
  hipEvent_t ev[6] = {};  // start, encoder end, decode end, two poll slots, results on host
  // Pinned host staging reused across calls (grow-only, like the device
  // buffers): the two metadata uploads and the readbacks (tokens, counts,
  // rows per step), so every copy is a DMA in the stream.
  enum Stage { H_META, H_DMETA, H_COUNT, H_GEN, H_HIST, H_ALL_ };
  char* hbuf[H_ALL_] = {};
  size_t hcap_[H_ALL_] = {};
  std::vector<int64_t> h_kv_base;
  std::vector<uint32_t> h_limit, h_remaining, h_ends;
  uint32_t allocs = 0;  // buffers (re)allocated by the current call
  // Kernel timing: start/stop event pairs of the timed launches and, per
  // launch, its kind (MARIAN_HIP_KERNEL_*), decode step and decoder layer.
  std::vector<hipEvent_t> kev;
  std::vector<uint32_t> kev_kind, kev_step, kev_layer;
  std::vector<float> kev_us;
  std::vector<hipEvent_t> step_ev;
  std::vector<uint32_t> step_rows;
  std::vector<float> step_ms;
  marian_hip_stats stats{};

  // Row capacities of the decode buffers (grow-only, with headroom): active
  // rows, KV-cache rows, encoder rows of the cross K/V, decode steps.
  size_t rcap = 0, ccap = 0, tcap = 0, hcap = 0;

  int fail(int code, const char* fmt, ...) {
    char msg[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    error = msg;
    if (code == MARIAN_HIP_ERR_DEVICE) ready = false;
    return code;
  }
  // A HIP error poisons the engine, except hipErrorInvalidValue from a launch
  // helper: that is a host-side shape rejection (nothing was launched), so
  // the stream is drained and the call fails as an inference error.
  int hip_fail(hipError_t e, const char* what) {
    if (e == hipErrorInvalidValue) {
      const hipError_t d = hipStreamSynchronize(stream);
      if (d == hipSuccess)
        return fail(MARIAN_HIP_ERR_INFERENCE, "%s: shape not supported by the kernels", what);
      e = d;
    }
    return fail(MARIAN_HIP_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
  }
  // Returns nullptr on failure (error recorded).
  void* get(Buf b, size_t bytes) {
    bytes = std::max<size_t>(bytes, 256);
    if (cap[b] >= bytes) return buf[b];
    if (buf[b]) {
      hipStreamSynchronize(stream);
      hipFree(buf[b]);
      buf[b] = nullptr;
      cap[b] = 0;
    }
    const size_t want = bytes + bytes / 4;
    if (hipMalloc(&buf[b], want) != hipSuccess) {
      buf[b] = nullptr;
      return nullptr;
    }
    ++allocs;
    cap[b] = want;
    return buf[b];
  }
  // Pinned host staging; every call ends with the stream drained, so an
  // outgrown buffer is idle when it is freed.  Returns nullptr on failure.
  char* host(Stage h, size_t bytes) {
    bytes = std::max<size_t>(bytes, 256);
    if (hcap_[h] >= bytes) return hbuf[h];
    if (hbuf[h]) {
      hipStreamSynchronize(stream);
      hipHostFree(hbuf[h]);
      hbuf[h] = nullptr;
      hcap_[h] = 0;
    }
    const size_t want = bytes + bytes / 4;
    if (hipHostMalloc((void**)&hbuf[h], want) != hipSuccess) {
      hbuf[h] = nullptr;
      return nullptr;
    }
    ++allocs;
    hcap_[h] = want;
    return hbuf[h];
  }
};

#define MH_HIP(expr)                                   \
  do {                                                 \
    hipError_t e_ = (expr);                            \
    if (e_ != hipSuccess) return E->hip_fail(e_, #expr); \
  } while (0)

extern "C" {

int marian_hip_positions(uint32_t dim, uint32_t count, float* out) {
  if (!out || host_positions(dim, count, out)) return MARIAN_HIP_ERR_INVALID_INPUT;
  return MARIAN_HIP_OK;
}

// Geometry every kernel of the path runs: 1-8 heads of width 64 or 48 (the
// reference's 384-wide production model) with d a multiple of 64 up to 512
// (the vocabulary kernel and the fp32-input projections hold K <= 512), FFN
// widths that are multiples of 64 up to 2048 (the skinny kernel's K), and at
// least one decoder layer (the decoder state the vocabulary projection
// scores).  Returns 0 or a model error with the reason noted.
static int check_geometry(uint32_t dim, uint32_t heads, uint32_t ffn, uint32_t dec_layers,
                          bool have_decoder) {
  if (!heads || heads > 8 || dim % heads || dim % 64 || dim > 512 ||
      (dim / heads != kHeadDim && dim / heads != 48))
    return model_fail("dim %u with %u heads: supported are 1-8 heads of width 64 or 48, dim a multiple of 64 up to 512",
                      dim, heads);
  if (!ffn || ffn % 64 || ffn > 2048)
    return model_fail("ffn_dim %u: supported are multiples of 64 up to 2048", ffn);
  if (!dec_layers || !have_decoder) return model_fail("the model needs at least one decoder layer");
  return 0;
}

static void apply_limits(marian_hip_engine* E, const marian_hip_limits* limits) {
  E->limits = limits ? *limits : marian_hip_limits{2, 256, 4096, 256, 256, 65536};
  if (E->limits.max_position > (uint32_t)kMaxPosition || E->limits.max_position == 0)
    E->limits.max_position = kMaxPosition;
}

// Whether every tensor the kernels read has a device address (each staged
// piece was bound to the engine's own pointer).
static bool tensors_placed(const marian_hip_engine* E) {
  auto lin = [](const Lin& l, bool frag) { return l.w && l.mult && l.bias && (!frag || l.wf); };
  bool ok = E->pos && lin(E->emb, true) && E->src_emb.w && E->src_emb.mult;
  for (const EncLayer& L : E->enc)
    ok = ok && lin(L.qkv, false) && lin(L.out, false) && lin(L.ffn1, false) && lin(L.ffn2, false) &&
         L.ln1_s && L.ln1_b && L.ln2_s && L.ln2_b;
  for (const DecLayer& L : E->dec)
    ok = ok && lin(L.self_qkv, true) && lin(L.self_out, true) && lin(L.cross_q, true) &&
         lin(L.cross_kv, false) && lin(L.cross_out, true) && lin(L.ffn1, true) && lin(L.ffn2, true) &&
         L.ln1_s && L.ln1_b && L.ln2_s && L.ln2_b && L.ln3_s && L.ln3_b;
  for (const SEncLayer& L : E->senc)
    ok = ok && lin(L.qkv.all, false) && lin(L.o, false) && lin(L.w1, false) && lin(L.w2, false) &&
         L.ln1_s && L.ln1_b && L.ln2_s && L.ln2_b;
  for (const SDecLayer& L : E->sdec)
    ok = ok && lin(L.uf.all, true) && lin(L.q, true) && lin(L.kv.all, false) && lin(L.o, true) &&
         lin(L.w1, true) && lin(L.w2, true) && L.ln0_s && L.ln0_b && L.ln1_s && L.ln1_b && L.ln2_s &&
         L.ln2_b;
  return ok;
}

// The model is valid: copy the staged weights to the device and create the
// engine's stream, flags and events.
static int engine_finish(marian_hip_engine* E, Packer& pk, int device, marian_hip_engine** out_engine) {
  auto cleanup_fail = [&](int code) {
    marian_hip_engine_destroy(E);
    return code;
  };
  std::vector<float> posv((size_t)kMaxPosition * E->d);
  host_positions(E->d, kMaxPosition, posv.data());
  pk.add(posv.data(), posv.size() * 4, (const void**)&E->pos);
  // Binds every staged piece at `base`.  First at a stand-in base that is
  // never dereferenced: a tensor the kernels read that no staged piece is
  // bound to is an error here, before the device is touched.
  auto bind = [&](const char* base) {
    for (const Packer::Fix& f : pk.fixes) *f.dst = base + f.off;
    if (!E->ssru) E->src_emb = E->emb;  // the transformer graph has one table
  };
  bind(reinterpret_cast<const char*>(uintptr_t(256)));
  if (!tensors_placed(E)) {
    marian_hip_engine_destroy(E);
    return model_fail("internal error: a model tensor has no device address");
  }

  if (hipSetDevice(device) != hipSuccess) return cleanup_fail(MARIAN_HIP_ERR_DEVICE);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
    char name[256] = {0};
    if (hipDeviceGetName(name, sizeof name, device) != hipSuccess || !name[0])
      std::snprintf(name, sizeof name, "%s", prop.name);
    if (!name[0]) std::snprintf(name, sizeof name, "AMD GPU");  // no marketing name visible
    E->device_name = std::string(name) + " (" + prop.gcnArchName + ")";
  }
  if (hipStreamCreateWithFlags(&E->stream, hipStreamNonBlocking) != hipSuccess)
    return cleanup_fail(MARIAN_HIP_ERR_DEVICE);

  if (hipMalloc(&E->weights, pk.host.size()) != hipSuccess) return cleanup_fail(MARIAN_HIP_ERR_DEVICE);
  if (hipMemcpy(E->weights, pk.host.data(), pk.host.size(), hipMemcpyHostToDevice) != hipSuccess)
    return cleanup_fail(MARIAN_HIP_ERR_DEVICE);
  bind((const char*)E->weights);

  if (hipMalloc(&E->err_flag, sizeof(int)) != hipSuccess) return cleanup_fail(MARIAN_HIP_ERR_DEVICE);
  if (hipHostMalloc((void**)&E->pinned, 64 * sizeof(int)) != hipSuccess)
    return cleanup_fail(MARIAN_HIP_ERR_DEVICE);
  for (auto& ev : E->ev)
    if (hipEventCreate(&ev) != hipSuccess) return cleanup_fail(MARIAN_HIP_ERR_DEVICE);
  *out_engine = E;
  return MARIAN_HIP_OK;
}

int marian_hip_engine_create(const marian_hip_model* m, const marian_hip_limits* limits,
                             int device, marian_hip_engine** out_engine) {
  if (!m || !out_engine) return MARIAN_HIP_ERR_INVALID_INPUT;
  *out_engine = nullptr;
  if (!m->embedding || !m->embedding_mult || !m->output_bias)
    return model_fail("embedding, its multipliers and the output bias are required");
  if (!m->vocab || m->vocab > (uint32_t)INT32_MAX) return model_fail("vocabulary size %u is not supported", m->vocab);
  if (int rc = check_geometry(m->dim, m->heads, m->ffn_dim, m->decoder_layers, m->decoder != nullptr)) return rc;
  if (m->encoder_layers && !m->encoder) return model_fail("encoder layers missing");
  auto* E = new marian_hip_engine();
  E->device = device;
  E->V = E->Vs = m->vocab;
  E->d = m->dim;
  E->H = m->heads;
  E->F = m->ffn_dim;
  E->Le = m->encoder_layers;
  E->Ld = m->decoder_layers;
  E->emb_scale = std::sqrt((float)m->dim);
  apply_limits(E, limits);

  Packer pk;
  const char* bad = nullptr;  // first tensor problem found
  auto add_lin = [&](const marian_hip_linear& l, int N, int K, Lin& out, bool frag = false) -> bool {
    if (!l.weight || !l.mult || !l.bias) {
      bad = "a linear layer is missing its weight, multipliers or bias";
      return false;
    }
    if ((bad = check_q8_tensor(l.weight, l.mult, (size_t)N, (size_t)K))) return false;
    out.N = N;
    out.K = K;
    pk.add(l.weight, (size_t)N * K, (const void**)&out.w);
    if (frag) pk.add_frag(l.weight, N, K, &out.wf);
    pk.add(l.mult, (size_t)N * 4, (const void**)&out.mult);
    pk.add(l.bias, (size_t)N * 4, (const void**)&out.bias);
    return true;
  };
  auto add_vec = [&](const float* v, size_t n, const float** dst) -> bool {
    if (!v) {
      bad = "a LayerNorm scale or bias is missing";
      return false;
    }
    pk.add(v, n * 4, (const void**)dst);
    return true;
  };
  const int d = (int)E->d, F = (int)E->F, V = (int)E->V;
  bool ok = true;
  if ((bad = check_q8_tensor(m->embedding, m->embedding_mult, (size_t)V, (size_t)d))) {
    marian_hip_engine_destroy(E);
    return model_fail("embedding: %s", bad);
  }
  E->emb.N = V;
  E->emb.K = d;
  pk.add(m->embedding, (size_t)V * d, (const void**)&E->emb.w);
  pk.add_frag(m->embedding, V, d, &E->emb.wf);
  pk.add(m->embedding_mult, (size_t)V * 4, (const void**)&E->emb.mult);
  pk.add(m->output_bias, (size_t)V * 4, (const void**)&E->emb.bias);
  E->enc.resize(E->Le);
  E->dec.resize(E->Ld);
  for (uint32_t l = 0; l < E->Le; ++l) {
    const marian_hip_encoder_layer& s = m->encoder[l];
    EncLayer& t = E->enc[l];
    ok = ok && add_lin(s.qkv, 3 * d, d, t.qkv) && add_lin(s.out, d, d, t.out) &&
         add_lin(s.ffn1, F, d, t.ffn1) && add_lin(s.ffn2, d, F, t.ffn2) &&
         add_vec(s.ln1_scale, d, &t.ln1_s) && add_vec(s.ln1_bias, d, &t.ln1_b) &&
         add_vec(s.ln2_scale, d, &t.ln2_s) && add_vec(s.ln2_bias, d, &t.ln2_b);
  }
  for (uint32_t l = 0; l < E->Ld; ++l) {
    const marian_hip_decoder_layer& s = m->decoder[l];
    DecLayer& t = E->dec[l];
    ok = ok && add_lin(s.self_qkv, 3 * d, d, t.self_qkv, true) &&
         add_lin(s.self_out, d, d, t.self_out, true) && add_lin(s.cross_q, d, d, t.cross_q, true) &&
         add_lin(s.cross_kv, 2 * d, d, t.cross_kv) && add_lin(s.cross_out, d, d, t.cross_out, true) &&
         add_lin(s.ffn1, F, d, t.ffn1, true) && add_lin(s.ffn2, d, F, t.ffn2, true) &&
         add_vec(s.ln1_scale, d, &t.ln1_s) && add_vec(s.ln1_bias, d, &t.ln1_b) &&
         add_vec(s.ln2_scale, d, &t.ln2_s) && add_vec(s.ln2_bias, d, &t.ln2_b) &&
         add_vec(s.ln3_scale, d, &t.ln3_s) && add_vec(s.ln3_bias, d, &t.ln3_b);
  }
  if (!ok) {
    marian_hip_engine_destroy(E);
    return model_fail("%s", bad ? bad : "invalid layer");
  }
  // The model is valid: only now is the device touched.
  return engine_finish(E, pk, device, out_engine);
}

int marian_hip_engine_create_ssru(const marian_hip_ssru_model* m, const marian_hip_limits* limits,
                                  int device, marian_hip_engine** out_engine) {
  if (!m || !out_engine) return MARIAN_HIP_ERR_INVALID_INPUT;
  *out_engine = nullptr;
  if (!m->encoder_embedding || !m->decoder_embedding || !m->output_bias)
    return model_fail("both embeddings and the output bias are required");
  if (!m->source_vocab || m->source_vocab > (uint32_t)INT32_MAX || !m->target_vocab ||
      m->target_vocab > (uint32_t)INT32_MAX)
    return model_fail("vocabulary sizes %u / %u are not supported", m->source_vocab, m->target_vocab);
  if (int rc = check_geometry(m->dim, m->heads, m->ffn_dim, m->decoder_layers, m->decoder != nullptr)) return rc;
  if (m->encoder_layers && !m->encoder) return model_fail("encoder layers missing");
  auto* E = new marian_hip_engine();
  E->ssru = true;
  E->device = device;
  E->V = m->target_vocab;
  E->Vs = m->source_vocab;
  E->d = m->dim;
  E->H = m->heads;
  E->F = m->ffn_dim;
  E->Le = m->encoder_layers;
  E->Ld = m->decoder_layers;
  E->emb_scale = std::sqrt((float)m->dim);  // EMBEDDING_SCALE = sqrt(384) (q8_engine.rs:23)
  apply_limits(E, limits);

  Packer pk;
  const char* bad = nullptr;
  const char* where = "";
  const int d = (int)E->d, F = (int)E->F;
  // A dense layer of the reference's per-tensor scheme: its multiplier and
  // bias expanded to one entry per output (the kernels' per-channel form; the
  // product 1 / (act * w) is the reference's inverse_scale, q8_gemm.rs:438),
  // 0.0 where it has no bias.
  auto check_static = [&](const marian_hip_static_linear& l, int N, int K, const char* name) -> bool {
    where = name;
    if (!l.weight) {
      bad = "a dense layer is missing its weight";
      return false;
    }
    if (!(std::isfinite(l.act_mult) && l.act_mult > 0.0f)) {
      bad = "activation multiplier is not finite and positive";
      return false;
    }
    std::vector<float> mult((size_t)N, l.weight_mult);
    return !(bad = check_q8_tensor(l.weight, mult.data(), (size_t)N, (size_t)K));
  };
  auto put = [&](const marian_hip_static_linear& l, int N, int K, size_t wofs, size_t vofs, Lin& all) {
    std::memcpy(pk.host.data() + wofs, l.weight, (size_t)N * K);
    float* mv = (float*)(pk.host.data() + vofs);
    std::fill(mv, mv + N, l.weight_mult);
    float* bv = (float*)(pk.host.data() + vofs + 4ull * all.N);
    if (l.bias) std::memcpy(bv, l.bias, 4ull * N);
    else std::fill(bv, bv + N, 0.0f);
  };
  // One or more layers reading the same input, as row blocks of one fused
  // weight [parts * N, K] (plus its fragment-order copy when `frag`).  The
  // staged pieces are bound to `all`, which must be the engine's own Lin: the
  // device addresses are written into it when the weights are uploaded.
  auto add_block = [&](std::initializer_list<const marian_hip_static_linear*> ls, int N, int K,
                       const char* name, Lin& all, float* act, bool& shared, bool frag) -> bool {
    for (const marian_hip_static_linear* l : ls)
      if (!check_static(*l, N, K, name)) return false;
    all.N = (int)ls.size() * N;
    all.K = K;
    const size_t wofs = pk.reserve((size_t)all.N * K, (const void**)&all.w);
    const size_t vofs = pk.reserve(8ull * all.N, (const void**)&all.mult);
    pk.fixes.push_back({vofs + 4ull * all.N, (const void**)&all.bias});
    int i = 0;
    shared = true;
    for (const marian_hip_static_linear* l : ls) {
      put(*l, N, K, wofs + (size_t)i * N * K, vofs + 4ull * i * N, all);
      act[i] = l->act_mult;
      shared = shared && l->act_mult == act[0];
      ++i;
    }
    if (frag) {  // from a copy: add_frag grows (and may move) the staging buffer
      const std::vector<int8_t> w((const int8_t*)pk.host.data() + wofs,
                                  (const int8_t*)pk.host.data() + wofs + (size_t)all.N * K);
      pk.add_frag(w.data(), all.N, K, &all.wf);
    }
    return true;
  };
  auto add_group = [&](std::initializer_list<const marian_hip_static_linear*> ls, int N, int K,
                       const char* name, SGroup& g, bool frag) -> bool {
    g.parts = (int)ls.size();
    g.n = N;
    return add_block(ls, N, K, name, g.all, g.act, g.shared, frag);
  };
  auto add_one = [&](const marian_hip_static_linear& l, int N, int K, const char* name, Lin& out,
                     float& act, bool frag) -> bool {
    bool single = true;
    return add_block({&l}, N, K, name, out, &act, single, frag);
  };
  auto add_vec = [&](const float* v, const float** dst, const char* name) -> bool {
    where = name;
    if (!v) {
      bad = "a LayerNorm scale or bias is missing";
      return false;
    }
    pk.add(v, 4ull * d, (const void**)dst);
    return true;
  };
  auto add_table = [&](const int8_t* w, float mult, int V, Lin& out, bool frag, const char* name) -> bool {
    where = name;
    std::vector<float> mv((size_t)V, mult);
    if ((bad = check_q8_tensor(w, mv.data(), (size_t)V, (size_t)d))) return false;
    out.N = V;
    out.K = d;
    pk.add(w, (size_t)V * d, (const void**)&out.w);
    if (frag) pk.add_frag(w, V, d, &out.wf);
    pk.add(mv.data(), 4ull * V, (const void**)&out.mult);
    return true;
  };
  bool ok = add_table(m->encoder_embedding, m->encoder_embedding_mult, (int)E->Vs, E->src_emb, false,
                      "encoder embedding") &&
            add_table(m->decoder_embedding, m->decoder_embedding_mult, (int)E->V, E->emb, true,
                      "decoder embedding");
  if (ok) {
    pk.add(m->output_bias, 4ull * E->V, (const void**)&E->emb.bias);
    where = "output multiplier";
    ok = std::isfinite(m->output_act_mult) && m->output_act_mult > 0.0f;
    if (!ok) bad = "activation multiplier is not finite and positive";
    E->out_act = m->output_act_mult;
  }
  E->senc.resize(E->Le);
  E->sdec.resize(E->Ld);
  for (uint32_t l = 0; ok && l < E->Le; ++l) {
    const marian_hip_ssru_encoder_layer& s = m->encoder[l];
    SEncLayer& t = E->senc[l];
    ok = add_group({&s.wq, &s.wk, &s.wv}, d, d, "encoder attention", t.qkv, false) &&
         add_one(s.wo, d, d, "encoder Wo", t.o, t.ao, false) &&
         add_vec(s.attn_ln_scale, &t.ln1_s, "encoder LayerNorm") &&
         add_vec(s.attn_ln_bias, &t.ln1_b, "encoder LayerNorm") &&
         add_one(s.w1, F, d, "encoder W1", t.w1, t.a1, false) &&
         add_one(s.w2, d, F, "encoder W2", t.w2, t.a2, false) &&
         add_vec(s.ffn_ln_scale, &t.ln2_s, "encoder LayerNorm") &&
         add_vec(s.ffn_ln_bias, &t.ln2_b, "encoder LayerNorm");
  }
  for (uint32_t l = 0; ok && l < E->Ld; ++l) {
    const marian_hip_ssru_decoder_layer& s = m->decoder[l];
    SDecLayer& t = E->sdec[l];
    ok = add_group({&s.ssru_w, &s.ssru_wf}, d, d, "SSRU", t.uf, true) &&
         add_vec(s.ssru_ln_scale, &t.ln0_s, "SSRU LayerNorm") &&
         add_vec(s.ssru_ln_bias, &t.ln0_b, "SSRU LayerNorm") &&
         add_one(s.wq, d, d, "context Wq", t.q, t.aq, true) &&
         add_group({&s.wk, &s.wv}, d, d, "context Wk/Wv", t.kv, false) &&
         add_one(s.wo, d, d, "context Wo", t.o, t.ao, true) &&
         add_vec(s.context_ln_scale, &t.ln1_s, "context LayerNorm") &&
         add_vec(s.context_ln_bias, &t.ln1_b, "context LayerNorm") &&
         add_one(s.w1, F, d, "decoder W1", t.w1, t.a1, true) &&
         add_one(s.w2, d, F, "decoder W2", t.w2, t.a2, true) &&
         add_vec(s.ffn_ln_scale, &t.ln2_s, "decoder LayerNorm") &&
         add_vec(s.ffn_ln_bias, &t.ln2_b, "decoder LayerNorm");
  }
  if (!ok) {
    marian_hip_engine_destroy(E);
    return model_fail("%s: %s", where, bad ? bad : "invalid layer");
  }
  return engine_finish(E, pk, device, out_engine);
}

void marian_hip_engine_destroy(marian_hip_engine* E) {
  if (!E) return;
  if (!E->stream && !E->weights) {  // rejected before the device was touched
    delete E;
    return;
  }
  hipSetDevice(E->device);
  if (E->stream) hipStreamSynchronize(E->stream);
  for (int b = 0; b < B_ALL_; ++b)
    if (E->buf[b]) hipFree(E->buf[b]);
  for (char* h : E->hbuf)
    if (h) hipHostFree(h);
  if (E->weights) hipFree(E->weights);
  if (E->err_flag) hipFree(E->err_flag);
  if (E->pinned) hipHostFree(E->pinned);
  for (auto& ev : E->ev)
    if (ev) hipEventDestroy(ev);
  for (auto& ev : E->kev) hipEventDestroy(ev);
  for (auto& ev : E->step_ev) hipEventDestroy(ev);
  if (E->stream) hipStreamDestroy(E->stream);
  delete E;
}

int marian_hip_is_ready(const marian_hip_engine* E) { return E && E->ready ? 1 : 0; }

const char* marian_hip_last_error(const marian_hip_engine* E) {
  return E ? E->error.c_str() : "null engine";
}

int marian_hip_info(const marian_hip_engine* E, char* buf, size_t cap) {
  if (!E || !buf || !cap) return MARIAN_HIP_ERR_INVALID_INPUT;
  const int n = snprintf(buf, cap,
                         "{\"name\":\"hip\",\"device\":\"%s\",\"model\":\"%s d=%u "
                         "heads=%u ffn=%u enc=%u dec=%u vocab=%u/%u\",\"precision\":\"%s\","
                         "\"attention\":\"varlen-fused\",\"supports_batching\":true}",
                         E->device_name.c_str(), E->ssru ? "transformer-ssru-q8" : "transformer-q8",
                         E->d, E->H, E->F, E->Le, E->Ld, E->Vs, E->V,
                         E->ssru ? "q8 static" : "q8");
  return (n < 0 || (size_t)n >= cap) ? MARIAN_HIP_ERR_BUFFER : MARIAN_HIP_OK;
}

int marian_hip_last_stats(const marian_hip_engine* E, marian_hip_stats* s) {
  if (!E || !s) return MARIAN_HIP_ERR_INVALID_INPUT;
  *s = E->stats;
  return MARIAN_HIP_OK;
}

int marian_hip_last_step_trace(const marian_hip_engine* E, uint32_t* active_rows,
                               float* step_end_ms, size_t cap, size_t* n_steps) {
  if (!E) return MARIAN_HIP_ERR_INVALID_INPUT;
  const size_t n = E->step_rows.size();
  if (n_steps) *n_steps = n;
  for (size_t i = 0; i < std::min(cap, n); ++i) {
    if (active_rows) active_rows[i] = E->step_rows[i];
    if (step_end_ms) step_end_ms[i] = i < E->step_ms.size() ? E->step_ms[i] : 0.0f;
  }
  return MARIAN_HIP_OK;
}

int marian_hip_last_kernel_trace(const marian_hip_engine* E, uint32_t* kind, uint32_t* step,
                                 uint32_t* layer, float* us, size_t cap, size_t* n) {
  if (!E) return MARIAN_HIP_ERR_INVALID_INPUT;
  const size_t m = E->kev_us.size();
  if (n) *n = m;
  for (size_t i = 0; i < std::min(cap, m); ++i) {
    if (kind) kind[i] = E->kev_kind[i];
    if (step) step[i] = E->kev_step[i];
    if (layer) layer[i] = E->kev_layer[i];
    if (us) us[i] = E->kev_us[i];
  }
  return MARIAN_HIP_OK;
}

int marian_hip_set_timing(marian_hip_engine* E, uint32_t flags) {
  if (!E || (flags & ~(uint32_t)(MARIAN_HIP_TIME_STEPS | MARIAN_HIP_TIME_KERNELS)))
    return MARIAN_HIP_ERR_INVALID_INPUT;
  E->timing = flags;
  return MARIAN_HIP_OK;
}

}  // extern "C"

namespace {

// Formats a message into `out` and returns `code`.
int fmt_msg(std::string& out, int code, const char* fmt, ...) {
  char msg[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  out = msg;
  return code;
}

// What the host checks of a packed batch establish about its shape.
struct BatchShape {
  size_t B = 0;       // sentences
  size_t Lmax = 0;    // longest source
  size_t n_cand = 0;  // candidate ids of a shortlisted call
  int max_cands = 0;  // longest candidate list
};

// The batch checks of the reference's engine, on the host before the device
// is touched: validate_batch (q8_engine.rs:468-509) and validate_work_shape
// (:1103-1119) with every cap a parameter (0: none), this engine's own batch
// ceiling, and, for a shortlisted call, the candidate lists (non-empty,
// strictly ascending as LexicalShortlist::candidates builds them,
// shortlist.rs:150-198, and inside the target vocabulary).  Returns
// MARIAN_HIP_OK, or MARIAN_HIP_ERR_INVALID_INPUT with the reason in `why`.
int check_batch(const marian_hip_limits& lim, uint32_t Vs, uint32_t V, const int32_t* tokens,
                size_t n_tokens, const uint32_t* offsets, size_t n_offsets, const uint32_t* cand,
                const uint32_t* cand_off, BatchShape& bs, std::string& why) {
  constexpr int BAD = MARIAN_HIP_ERR_INVALID_INPUT;
  if (!offsets || (n_tokens && !tokens)) return fmt_msg(why, BAD, "null input pointer");
  if (n_offsets < 2 || offsets[0] != 0 || offsets[n_offsets - 1] != n_tokens)
    return fmt_msg(why, BAD, "invalid packed batch offsets");
  const size_t B = n_offsets - 1;
  if (lim.max_batch && B > lim.max_batch)
    return fmt_msg(why, BAD, "batch contains %zu sentences; maximum is %u", B, lim.max_batch);
  if (B > (size_t)kMaxRowsPerCall)
    return fmt_msg(why, BAD, "batch contains %zu sentences; this engine handles %d per call", B,
                   kMaxRowsPerCall);
  size_t Lmax = 0;
  for (size_t b = 0; b < B; ++b) {
    if (offsets[b + 1] <= offsets[b]) return fmt_msg(why, BAD, "each input must contain at least one token");
    Lmax = std::max<size_t>(Lmax, offsets[b + 1] - offsets[b]);
  }
  if (lim.max_source_tokens && Lmax > lim.max_source_tokens)
    return fmt_msg(why, BAD, "source has %zu tokens; maximum is %u", Lmax, lim.max_source_tokens);
  if (lim.max_padded_cells && (uint64_t)B * Lmax * Lmax > lim.max_padded_cells)
    return fmt_msg(why, BAD, "padded attention work is %llu cells; maximum is %llu",
                   (unsigned long long)((uint64_t)B * Lmax * Lmax), (unsigned long long)lim.max_padded_cells);
  if (Lmax > (size_t)kMaxPosition) return fmt_msg(why, BAD, "source longer than the position table");
  for (size_t i = 0; i < n_tokens; ++i)
    if (tokens[i] < 0 || (uint32_t)tokens[i] >= Vs)
      return fmt_msg(why, BAD, "source token %d is outside vocabulary %u", tokens[i], Vs);
  bs = BatchShape();
  bs.B = B;
  bs.Lmax = Lmax;
  if (cand || cand_off) {  // select_token's candidates (q8_engine.rs:749-766)
    if (!cand || !cand_off || cand_off[0] != 0)
      return fmt_msg(why, BAD, "invalid candidate offsets");
    for (size_t b = 0; b < B; ++b) {
      if (cand_off[b + 1] <= cand_off[b]) return fmt_msg(why, BAD, "cannot select from an empty candidate list");
      const uint64_t n = cand_off[b + 1] - cand_off[b];
      bs.max_cands = std::max<int>(bs.max_cands, (int)std::min<uint64_t>(n, INT32_MAX));
      for (uint32_t i = cand_off[b]; i < cand_off[b + 1]; ++i) {
        if (cand[i] >= V) return fmt_msg(why, BAD, "output candidate %u exceeds vocabulary %u", cand[i], V);
        if (i > cand_off[b] && cand[i] <= cand[i - 1])
          return fmt_msg(why, BAD, "candidate list %zu is not strictly ascending at position %u", b,
                         i - cand_off[b]);
      }
    }
    bs.n_cand = cand_off[B];
  }
  return MARIAN_HIP_OK;
}

// The sizes one call's buffers are planned for.
struct CallShape {
  size_t B = 0, T = 0;     // sentences, source tokens
  size_t n_cand = 0;       // candidate ids (0: full-vocabulary scoring)
  bool cand = false;
  int nparts = 0;          // argmax partial keys per row
  uint64_t cache_rows = 1; // sum of the per-sentence generation limits
  uint32_t gen_limit = 0;  // longest generation
};

// Byte offsets of the two metadata uploads.  Encoder, per token: id, position
// in its sentence, sentence index; the cu offsets; the candidate lists.
// Decoder, per active row: its sequence, first KV-cache / output row, source
// range, previous token and generation limit; plus the device row count and
// step.
struct MetaLayout {
  size_t o_tok, o_pos, o_seq, o_cu, o_cand, o_coff, meta_bytes;
  size_t o_state, o_rslot, o_rkv0, o_rsrc0, o_rsrcn, o_rprev, o_rlim, dmeta_bytes;
};

// Device buffers of one call.
struct CallBufs {
  char *dmeta = nullptr, *ddec = nullptr;
  float *X0, *X1, *XA, *QKV, *ATT, *OA, *Y, *Hb, *HA, *CKV, *KC, *VC, *STATE, *DUF;
  int8_t *XQ, *OQ, *HQ, *DXQ, *DHQ;
  float *DX0, *DX1, *DXA, *DQ, *DATT, *DAMAX, *DY, *DH, *DHA;
  uint64_t* PART;
  int32_t* OUT;
  uint32_t *COUNT, *HIST, *TILES;
  int tiles_cap = 0;
};

// Grows the engine's capacities to `cs` (with headroom) and fetches every
// buffer a call of that shape uses.  Returns MARIAN_HIP_OK or a device error.
int plan_buffers(marian_hip_engine* E, const CallShape& cs, MetaLayout& L, CallBufs& b) {
  auto grow = [](size_t need, size_t cur) { return need <= cur ? cur : std::max(need, cur + cur / 2); };
  E->rcap = grow(cs.B, E->rcap);
  E->ccap = grow(std::max<uint64_t>(cs.cache_rows, 1), E->ccap);
  E->tcap = grow(std::max<size_t>(cs.T, 1), E->tcap);
  E->hcap = grow((size_t)cs.gen_limit + 1, E->hcap);
  const size_t R = E->rcap, CR = E->ccap, TR = E->tcap, T = cs.T, B = cs.B;
  const size_t d = E->d, F = E->F, H = E->H, LdA = std::max<uint32_t>(E->Ld, 1);

  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  size_t cur = 0;
  auto place = [&](size_t bytes) {
    const size_t o = cur;
    cur = align(cur + bytes);
    return o;
  };
  L.o_tok = place(4 * T);
  L.o_pos = place(4 * T);
  L.o_seq = place(4 * T);
  L.o_cu = place(4 * (B + 1));
  L.o_cand = place(4 * cs.n_cand);
  L.o_coff = place(cs.cand ? 4 * (B + 1) : 0);
  L.meta_bytes = cur;
  cur = 0;
  L.o_state = place(8);
  L.o_rslot = place(4 * R);
  L.o_rkv0 = place(8 * R);
  L.o_rsrc0 = place(8 * R);
  L.o_rsrcn = place(4 * R);
  L.o_rprev = place(4 * R);
  L.o_rlim = place(4 * R);
  L.dmeta_bytes = cur;

  b.dmeta = (char*)E->get(B_META, L.meta_bytes);
  b.ddec = (char*)E->get(B_DMETA, L.dmeta_bytes);
  b.X0 = (float*)E->get(B_X0, 4 * T * d);
  b.X1 = (float*)E->get(B_X1, 4 * T * d);
  b.XQ = (int8_t*)E->get(B_XQ, T * d);
  b.XA = (float*)E->get(B_XA, 4 * T);
  b.QKV = (float*)E->get(B_QKV, 12 * T * d);
  b.ATT = (float*)E->get(B_ATT, 4 * T * d);
  b.OQ = (int8_t*)E->get(B_OQ, T * d);
  b.OA = (float*)E->get(B_OA, 4 * T);
  b.Y = (float*)E->get(B_Y, 4 * T * d);
  b.Hb = (float*)E->get(B_H, 4 * T * F);
  b.HQ = (int8_t*)E->get(B_HQ, T * F);
  b.HA = (float*)E->get(B_HA, 4 * T);
  b.CKV = (float*)E->get(B_CKV, 8 * TR * d * LdA);
  // Self-attention caches (transformer graph); the SSRU graph keeps one
  // recurrent state row per sequence and layer instead (two buffers: step t
  // reads buffer t % 2 and writes the other, so every head of a row can read
  // the old state), and two projections per row for the SSRU's inputs.
  b.KC = (float*)E->get(B_KC, E->ssru ? 0 : 4 * CR * d * LdA);
  b.VC = (float*)E->get(B_VC, E->ssru ? 0 : 4 * CR * d * LdA);
  b.STATE = (float*)E->get(B_STATE, E->ssru ? 2 * 4 * R * d * LdA : 0);
  b.DUF = (float*)E->get(B_DUF, E->ssru ? 8 * R * d : 0);
  b.DX0 = (float*)E->get(B_DX0, 4 * R * d);
  b.DX1 = (float*)E->get(B_DX1, 4 * R * d);
  b.DXQ = (int8_t*)E->get(B_DXQ, R * d);
  b.DXA = (float*)E->get(B_DXA, 4 * R);
  b.DQ = (float*)E->get(B_DQ, 4 * R * d);
  b.DATT = (float*)E->get(B_DATT, 4 * R * d);
  b.DAMAX = (float*)E->get(B_DAMAX, 4 * R * H);
  b.DY = (float*)E->get(B_DY, 4 * R * d);
  b.DH = (float*)E->get(B_DH, 4 * R * F);
  b.DHQ = (int8_t*)E->get(B_DHQ, R * F);
  b.DHA = (float*)E->get(B_DHA, 4 * R);
  b.PART = (uint64_t*)E->get(B_PART, 8 * R * (size_t)cs.nparts);
  b.OUT = (int32_t*)E->get(B_OUT, 4 * CR);
  b.COUNT = (uint32_t*)E->get(B_COUNT, 4 * R);
  b.HIST = (uint32_t*)E->get(B_HIST, 4 * E->hcap);
  b.tiles_cap = seq_tiles_bound((int)T, (int)B);
  b.TILES = (uint32_t*)E->get(B_TILES, 4 * (1 + 2 * (size_t)b.tiles_cap));
  for (int i = 0; i < B_COUNT_; ++i)
    if (!E->buf[i]) return E->fail(MARIAN_HIP_ERR_DEVICE, "device allocation failed");
  if (!E->host(marian_hip_engine::H_META, L.meta_bytes) || !E->host(marian_hip_engine::H_DMETA, L.dmeta_bytes) ||
      !E->host(marian_hip_engine::H_COUNT, 4 * R) || !E->host(marian_hip_engine::H_GEN, 4 * CR) ||
      !E->host(marian_hip_engine::H_HIST, 4 * E->hcap))
    return E->fail(MARIAN_HIP_ERR_DEVICE, "pinned host allocation failed");
  return MARIAN_HIP_OK;
}

constexpr int kBlkMaxRows = 64;    // steps up to this many rows use attention blocks
constexpr int kLnFfnMaxRows = 32;  // ... and the LayerNorm + FFN up-projection block
constexpr int kFfnAfMaxRows = 8;   // ... and the FFN down-projection quantizing its fp32 rows
// Every kPoll-th decode step the finalizer also stores the new active count in
// a pinned host slot that the host polls.
constexpr uint32_t kPoll = 8;

// What one decode step launches, decided on the host: the row bound (grid
// sizes; rows at or past the device row count exit early), the path of each
// attention sublayer and the key bounds that pick kernel variants.
struct StepPlan {
  int rows, self_keys, cross_keys;
  bool blk_self, blk_cross, ln_ffn, ln_rows, ffn_af, vocab_ln;
};

#define MH_TRY(expr)                 \
  do {                               \
    const hipError_t e_ = (expr);    \
    if (e_ != hipSuccess) return e_; \
  } while (0)

// One translate call: the validated batch, its buffers, and the stages the
// call runs in order (upload, encoder, decode loop, readback).
struct Translation {
  marian_hip_engine* E;
  hipStream_t s = nullptr;
  // the call's arguments
  const int32_t* tokens = nullptr;
  size_t n_tokens = 0;
  const uint32_t* offsets = nullptr;
  const uint32_t* max_out = nullptr;
  uint32_t flags = 0;
  const uint32_t* cand = nullptr;  // host candidate lists (shortlisted calls)
  const uint32_t* cand_off = nullptr;
  Probe pr;
  BatchShape bs;
  // geometry and sizes
  int d = 0, F = 0, H = 0, T = 0, Bi = 0;
  size_t B = 0, R = 0, CR = 0, TR = 0;
  uint32_t LdA = 1;
  uint32_t gen_limit = 0;
  size_t cache_rows = 1;
  int n_active0 = 0, nparts = 0;
  bool tiled = false;
  bool fast = false;  // MARIAN_HIP_FLAG_FAST_REDUCTIONS: the decoder's sums in the tree order
  MetaLayout L{};
  CallBufs b{};
  // device views of the metadata
  int32_t *d_tok = nullptr, *d_pos = nullptr, *d_seq = nullptr;
  uint32_t* d_cu = nullptr;
  const uint32_t *d_cand = nullptr, *d_coff = nullptr;
  int* d_nact = nullptr;
  RowMeta rm;
  float* PLOG = nullptr;     // probe: the probed step's logits [R, V], active-row order
  int32_t* PSLOT = nullptr;  // probe: that step's row -> sequence map [R] and row count
  // decode loop
  int* host_active = nullptr;  // pinned host slot for this step's active count (poll steps)
  size_t n_timed = 0;
  uint32_t steps = 0, launched = 0;

  explicit Translation(marian_hip_engine* e) : E(e) {}

  int prepare();
  hipError_t upload();
  hipError_t encode();
  StepPlan make_plan(int rows, int self_keys, int cross_keys) const;
  hipError_t timer(uint32_t kind, uint32_t step, uint32_t layer, hipEvent_t* ev);
  hipError_t score(int rows, uint32_t t, RowPrologue& pend, float qmult = 0.0f);
  hipError_t emit_step(const StepPlan& P, uint32_t t);
  hipError_t emit_step_ssru(int rows, uint32_t t);
  hipError_t decode();
  int finish(int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets, size_t* out_len);
};

// Generation limits, buffer capacities and the host copies of the metadata.
int Translation::prepare() {
  const marian_hip_limits& lim = E->limits;
  const uint32_t maxpos = std::min<uint32_t>(lim.max_position, kMaxPosition);
  std::vector<uint32_t>& limit = E->h_limit;
  limit.assign(B, 0);
  uint64_t total_cap = 0;
  for (size_t i = 0; i < B; ++i) {  // q8_engine.rs:369-379, the caps as parameters
    uint64_t l = max_out[i];
    const uint64_t len = offsets[i + 1] - offsets[i];
    if (lim.max_length_factor) l = std::min<uint64_t>(l, len * lim.max_length_factor);
    if (lim.max_generation_steps) l = std::min<uint64_t>(l, lim.max_generation_steps);
    l = std::min<uint64_t>(l, maxpos);
    limit[i] = (uint32_t)l;
    gen_limit = std::max(gen_limit, limit[i]);
    total_cap += l;
  }
  cache_rows = std::max<uint64_t>(total_cap, 1);
  d = (int)E->d;
  F = (int)E->F;
  H = (int)E->H;
  T = (int)n_tokens;
  Bi = (int)B;
  LdA = std::max<uint32_t>(E->Ld, 1);
  nparts = cand ? cand_groups(bs.max_cands) : argmax_groups((int)E->V, (int)E->d);

  CallShape cs;
  cs.B = B;
  cs.T = (size_t)T;
  cs.n_cand = bs.n_cand;
  cs.cand = cand != nullptr;
  cs.nparts = nparts;
  cs.cache_rows = cache_rows;
  cs.gen_limit = gen_limit;
  if (int rc = plan_buffers(E, cs, L, b)) return rc;
  R = E->rcap;
  CR = E->ccap;
  TR = E->tcap;
  if (pr.logits) {
    PLOG = (float*)E->get(B_PLOG, 4ull * R * E->V);
    PSLOT = (int32_t*)E->get(B_PSLOT, 4ull * (R + 1));
    if (!PLOG || !PSLOT) return E->fail(MARIAN_HIP_ERR_DEVICE, "device allocation failed");
  }

  // Both uploads are written straight into the engine's pinned staging.
  char* meta = E->hbuf[marian_hip_engine::H_META];
  char* dmeta_h = E->hbuf[marian_hip_engine::H_DMETA];
  std::memset(meta, 0, L.meta_bytes);
  std::memset(dmeta_h, 0, L.dmeta_bytes);
  int32_t* positions = (int32_t*)(meta + L.o_pos);
  int32_t* seq_of_row = (int32_t*)(meta + L.o_seq);
  if (T) std::memcpy(meta + L.o_tok, tokens, 4 * (size_t)T);
  std::memcpy(meta + L.o_cu, offsets, 4 * (B + 1));
  if (cand) {
    std::memcpy(meta + L.o_cand, cand, 4 * bs.n_cand);
    std::memcpy(meta + L.o_coff, cand_off, 4 * (B + 1));
  }
  // Active rows: initially every sequence with a non-zero limit, in order;
  // the rest of the R rows padded with valid values.
  int32_t* r_slot = (int32_t*)(dmeta_h + L.o_rslot);
  int64_t* r_kv0 = (int64_t*)(dmeta_h + L.o_rkv0);
  int64_t* r_src0 = (int64_t*)(dmeta_h + L.o_rsrc0);
  int32_t* r_srcn = (int32_t*)(dmeta_h + L.o_rsrcn);
  int32_t* r_prev = (int32_t*)(dmeta_h + L.o_rprev);
  uint32_t* r_lim = (uint32_t*)(dmeta_h + L.o_rlim);
  for (size_t r = 0; r < R; ++r) {
    r_srcn[r] = 1;
    r_prev[r] = -1;
  }
  std::vector<int64_t>& kv_base = E->h_kv_base;
  kv_base.assign(B, 0);
  int64_t run = 0;
  n_active0 = 0;
  for (size_t i = 0; i < B; ++i) {
    for (uint32_t j = offsets[i]; j < offsets[i + 1]; ++j) {
      positions[j] = (int32_t)(j - offsets[i]);
      seq_of_row[j] = (int32_t)i;
    }
    kv_base[i] = run;
    run += limit[i];
    if (limit[i] > 0) {
      r_slot[n_active0] = (int32_t)i;
      r_kv0[n_active0] = kv_base[i];
      r_src0[n_active0] = offsets[i];
      r_srcn[n_active0] = (int32_t)(offsets[i + 1] - offsets[i]);
      r_lim[n_active0] = limit[i];
      ++n_active0;
    }
  }
  const int state0[2] = {n_active0, 0};  // device row count, decode step
  std::memcpy(dmeta_h + L.o_state, state0, 8);

  d_tok = (int32_t*)(b.dmeta + L.o_tok);
  d_pos = (int32_t*)(b.dmeta + L.o_pos);
  d_seq = (int32_t*)(b.dmeta + L.o_seq);
  d_cu = (uint32_t*)(b.dmeta + L.o_cu);
  d_cand = cand ? (const uint32_t*)(b.dmeta + L.o_cand) : nullptr;
  d_coff = cand ? (const uint32_t*)(b.dmeta + L.o_coff) : nullptr;
  d_nact = (int*)(b.ddec + L.o_state);
  rm.slot = (int*)(b.ddec + L.o_rslot);
  rm.kv0 = (int64_t*)(b.ddec + L.o_rkv0);
  rm.src0 = (int64_t*)(b.ddec + L.o_rsrc0);
  rm.srcn = (int32_t*)(b.ddec + L.o_rsrcn);
  rm.prev = (int32_t*)(b.ddec + L.o_rprev);
  rm.limit = (uint32_t*)(b.ddec + L.o_rlim);
  tiled = bs.Lmax <= 256;
  return MARIAN_HIP_OK;
}

// The packed-token upload opens the timed region (the device time runs from
// the upload of the packed batch to the generated tokens in host memory).
hipError_t Translation::upload() {
  MH_TRY(hipEventRecord(E->ev[0], s));
  MH_TRY(hipMemcpyAsync(b.dmeta, E->hbuf[marian_hip_engine::H_META], L.meta_bytes, hipMemcpyHostToDevice, s));
  MH_TRY(hipMemcpyAsync(b.ddec, E->hbuf[marian_hip_engine::H_DMETA], L.dmeta_bytes, hipMemcpyHostToDevice, s));
  MH_TRY(hipMemsetAsync(E->err_flag, 0, sizeof(int), s));
  MH_TRY(hipMemsetAsync(b.COUNT, 0, 4 * B, s));
  if (E->ssru) MH_TRY(hipMemsetAsync(b.STATE, 0, 4ull * R * d * LdA, s));  // step 0 reads zero states
  return hipSuccess;
}

// The encoder over the packed rows and each decoder layer's cross K/V
// (q8_engine.rs:511-574).
hipError_t Translation::encode() {
  // The SSRU graph quantizes every dense layer's input with that layer's
  // static multiplier: a LayerNorm or the embedding quantizes with the next
  // layer's (or group's shared) multiplier when there is exactly one, and a
  // separate pass runs per layer otherwise.
  const SGroup* qkv0 = E->ssru && E->Le ? &E->senc[0].qkv : nullptr;
  {
    EmbedArgs ea;
    ea.emb = E->src_emb.w;
    ea.emb_mult = E->src_emb.mult;
    ea.pos = E->pos;
    ea.scale = E->emb_scale;
    ea.d = d;
    ea.tokens = d_tok;
    ea.positions = d_pos;
    ea.rows = T;
    ea.x = b.X0;
    ea.xq = !E->ssru || (qkv0 && qkv0->shared) ? b.XQ : nullptr;
    ea.xa = b.XA;
    ea.qmult = qkv0 && qkv0->shared ? qkv0->act[0] : 0.0f;
    ea.err = E->err_flag;
    MH_TRY(launch_embed(ea, s));
  }
  // Query tiles of the packed sentences for the encoder's self-attention.
  if (tiled) MH_TRY(launch_seq_tiles(d_cu, Bi, b.TILES, b.tiles_cap, s));
  auto gemm = [&](const int8_t* A, const float* a, int M, const Lin& L, float* out, int relu,
                  int64_t ldo = 0, int8_t* q = nullptr, float* qa = nullptr, float qmult = 0.0f) {
    GemmArgs g;
    g.A = A;
    g.a = a;
    g.lda = L.K;
    g.M = M;
    g.K = L.K;
    g.W = L.w;
    g.wmult = L.mult;
    g.bias = L.bias;
    g.N = L.N;
    Epilogue e;
    e.out = out;
    e.ldo = ldo ? ldo : L.N;
    e.relu = relu;
    e.out_q = q;
    e.ldq = L.N;
    e.out_qa = qa;
    e.qmult = qmult;
    if (q) g.err = E->err_flag;
    return launch_gemm_store(g, e, s);
  };
  auto qstatic = [&](const float* x, int64_t ldx, int M, int K, float mult, int8_t* q, float* a,
                     const int* rows_dev) {
    return launch_quantize_rows_static(x, ldx, M, K, mult, q, K, a, E->err_flag, s, rows_dev);
  };
  // A group of static layers over the packed rows x (already quantized into
  // XQ when shared), written side by side into out (row stride parts * n).
  auto sgroup = [&](const SGroup& G, const float* x, float* out) -> hipError_t {
    if (G.shared) return gemm(b.XQ, b.XA, T, G.all, out, 0);
    for (int i = 0; i < G.parts; ++i) {
      hipError_t rc = qstatic(x, d, T, d, G.act[i], b.XQ, b.XA, nullptr);
      if (rc == hipSuccess) rc = gemm(b.XQ, b.XA, T, G.part(i), out + (size_t)i * G.n, 0, (int64_t)G.parts * G.n);
      if (rc != hipSuccess) return rc;
    }
    return hipSuccess;
  };
  // q / qa / qmult: the output also quantized with a static multiplier.
  auto enc_attention = [&](int8_t* q = nullptr, float* qa = nullptr, float qmult = 0.0f) {
    AttnArgs aa;
    aa.mode = ATT_SEQ;
    aa.q = b.QKV;
    aa.ldq = 3 * d;
    aa.k = b.QKV + d;
    aa.v = b.QKV + 2 * d;
    aa.ldkv = 3 * d;
    aa.heads = H;
    aa.head_dim = d / H;
    aa.rows = T;
    aa.seq_of_row = d_seq;
    aa.cu = d_cu;
    aa.max_keys = (int)bs.Lmax;
    if (tiled) {
      aa.tiles = b.TILES;
      aa.tiles_cap = b.tiles_cap;
    }
    aa.out = b.ATT;
    aa.ldo = d;
    aa.err = E->err_flag;
    aa.qout = q;
    aa.ldqout = d;
    aa.qa = qa;
    aa.qmult = qmult;
    return launch_attention(aa, s);
  };
  if (!E->ssru) {
    for (uint32_t l = 0; l < E->Le; ++l) {
      const EncLayer& L = E->enc[l];
      MH_TRY(gemm(b.XQ, b.XA, T, L.qkv, b.QKV, 0));
      MH_TRY(enc_attention());
      MH_TRY(launch_quantize_rows(b.ATT, d, T, nullptr, d, b.OQ, d, b.OA, E->err_flag, s));
      MH_TRY(gemm(b.OQ, b.OA, T, L.out, b.Y, 0));
      MH_TRY(launch_residual_ln(b.Y, b.X0, L.ln1_s, L.ln1_b, T, nullptr, d, b.X1, b.XQ, b.XA, E->err_flag, s));
      MH_TRY(gemm(b.XQ, b.XA, T, L.ffn1, b.Hb, 1));
      MH_TRY(launch_quantize_rows(b.Hb, F, T, nullptr, F, b.HQ, F, b.HA, E->err_flag, s));
      MH_TRY(gemm(b.HQ, b.HA, T, L.ffn2, b.Y, 0));
      MH_TRY(launch_residual_ln(b.Y, b.X1, L.ln2_s, L.ln2_b, T, nullptr, d, b.X0, b.XQ, b.XA, E->err_flag, s));
    }
    if (pr.enc) MH_TRY(hipMemcpyAsync(pr.enc, b.X0, 4ull * T * d, hipMemcpyDeviceToHost, s));
    for (uint32_t l = 0; l < E->Ld; ++l)
      MH_TRY(gemm(b.XQ, b.XA, T, E->dec[l].cross_kv, b.CKV + (size_t)l * TR * 2 * d, 0));
  } else {
    // encode (q8_engine.rs:526-558): Q, K and V from their own layers.
    for (uint32_t l = 0; l < E->Le; ++l) {
      const SEncLayer& L = E->senc[l];
      MH_TRY(sgroup(L.qkv, b.X0, b.QKV));
      // Static multipliers quantize elementwise, so the producers write the
      // next layer's int8 input themselves.
      MH_TRY(enc_attention(b.OQ, b.OA, L.ao));
      MH_TRY(gemm(b.OQ, b.OA, T, L.o, b.Y, 0));
      MH_TRY(launch_residual_ln(b.Y, b.X0, L.ln1_s, L.ln1_b, T, nullptr, d, b.X1, b.XQ, b.XA, E->err_flag, s,
                                L.a1));
      MH_TRY(gemm(b.XQ, b.XA, T, L.w1, nullptr, 1, 0, b.HQ, b.HA, L.a2));
      MH_TRY(gemm(b.HQ, b.HA, T, L.w2, b.Y, 0));
      const SGroup* nx = l + 1 < E->Le ? &E->senc[l + 1].qkv : nullptr;
      MH_TRY(launch_residual_ln(b.Y, b.X1, L.ln2_s, L.ln2_b, T, nullptr, d, b.X0, nx && nx->shared ? b.XQ : nullptr,
                                b.XA, E->err_flag, s, nx && nx->shared ? nx->act[0] : 0.0f));
    }
    if (pr.enc) MH_TRY(hipMemcpyAsync(pr.enc, b.X0, 4ull * T * d, hipMemcpyDeviceToHost, s));
    // Cross K/V (q8_engine.rs:560-567): Wk and Wv of each decoder layer side
    // by side, [T, 2d].
    for (uint32_t l = 0; l < E->Ld; ++l) {
      const SGroup& G = E->sdec[l].kv;
      if (G.shared) MH_TRY(qstatic(b.X0, d, T, d, G.act[0], b.XQ, b.XA, nullptr));
      MH_TRY(sgroup(G, b.X0, b.CKV + (size_t)l * TR * 2 * d));
    }
  }
  return hipSuccess;
}

StepPlan Translation::make_plan(int rows, int self_keys, int cross_keys) const {
  StepPlan P;
  P.rows = rows;
  P.self_keys = self_keys;
  P.cross_keys = cross_keys;
  P.blk_self = rows <= kBlkMaxRows && attn_block_supported(d, H, self_keys);
  P.blk_cross = rows <= kBlkMaxRows && attn_block_supported(d, H, cross_keys);
  P.ln_ffn = rows <= kLnFfnMaxRows && ln_gemm_block_supported(d, F);
  P.ln_rows = !P.ln_ffn && ln_gemm_rows_supported(d, F);
  P.ffn_af = rows <= kFfnAfMaxRows;
  P.vocab_ln = cand ? cand_ln_supported(d) : rows <= kVocabLnMaxRows && vocab_ln_supported(d);
  return P;
}

// With kernel timing on, a timed launch's own dispatch records a start and a
// stop event (ev[0], ev[1]); otherwise both stay null.  Each such launch costs
// several microseconds of extra device time.
hipError_t Translation::timer(uint32_t kind, uint32_t step, uint32_t layer, hipEvent_t* ev) {
  ev[0] = ev[1] = nullptr;
  if (!(E->timing & MARIAN_HIP_TIME_KERNELS)) return hipSuccess;
  while (E->kev.size() < 2 * (n_timed + 1)) {
    hipEvent_t x;
    MH_TRY(hipEventCreate(&x));
    E->kev.push_back(x);
  }
  ev[0] = E->kev[2 * n_timed];
  ev[1] = E->kev[2 * n_timed + 1];
  E->kev_kind.push_back(kind);
  E->kev_step.push_back(step);
  E->kev_layer.push_back(layer);
  ++n_timed;
  return hipSuccess;
}

// Token selection at the end of step t over the rows in DXQ / DXA (or the
// LayerNorm still pending in `pend`, built by the scoring kernel itself and
// quantized with qmult (> 0: static) or the row's own multiplier), then the
// stop rules and the compaction of the active set.  With candidates every row
// scores its sentence's list (select_token, q8_engine.rs:749-790); without,
// the whole vocabulary under the generation mask.
hipError_t Translation::score(int rows, uint32_t t, RowPrologue& pend, float qmult) {
  if (cand) {
    CandArgs c;
    c.xq = b.DXQ;
    c.xa = b.DXA;
    if (pend.kind == PRO_LN) {  // its fp32 output is not needed
      c.pro = pend;
      c.pro.out = nullptr;
      c.qmult = qmult;
      pend.kind = PRO_NONE;
    }
    c.M = rows;
    c.K = d;
    c.V = (int)E->V;
    c.emb = E->emb.w;
    c.mult = E->emb.mult;
    c.bias = E->emb.bias;
    c.cand = d_cand;
    c.off = d_coff;
    c.row_slot = rm.slot;
    c.rows_dev = d_nact;
    c.max_cands = bs.max_cands;
    c.partials = b.PART;
    c.nparts = nparts;
    c.err = E->err_flag;
    MH_TRY(launch_cand_argmax(c, s));
  } else {
    Epilogue e;
    e.partials = b.PART;
    e.partial_ld = nparts;
    e.flags = flags;
    GemmArgs g;
    g.A = b.DXQ;
    g.a = b.DXA;
    g.lda = d;
    g.M = rows;
    g.M_dev = d_nact;
    g.K = d;
    g.W = E->emb.w;
    g.Wf = E->emb.wf;
    g.wmult = E->emb.mult;
    g.bias = E->emb.bias;
    g.N = (int)E->V;
    if (pend.kind == PRO_LN) {  // rows built in the kernel: its fp32 output is not needed
      g.pro = pend;
      g.pro.out = nullptr;
      pend.kind = PRO_NONE;
    }
    const bool probed = PLOG && t == pr.step;
    if (probed) {  // this step's logits too (same kernel, extra stores)
      e.logits = PLOG;
      e.ldl = E->V;
    }
    hipEvent_t ev[2];
    MH_TRY(timer(MARIAN_HIP_KERNEL_VOCAB, t, 0, ev));
    MH_TRY(launch_vocab_argmax(g, e, s, ev[0], ev[1]));
    if (probed) {  // the active-row order before the finalizer compacts it
      MH_TRY(hipMemcpyAsync(PSLOT, rm.slot, 4ull * R, hipMemcpyDeviceToDevice, s));
      MH_TRY(hipMemcpyAsync(PSLOT + R, d_nact, sizeof(int32_t), hipMemcpyDeviceToDevice, s));
    }
  }
  FinalizeArgs f;
  f.partials = b.PART;
  f.nparts = nparts;
  f.rows = rm;
  f.n_active = d_nact;
  f.rows_ub = rows;
  f.err = E->err_flag;
  f.out_tok = b.OUT;
  f.count = b.COUNT;
  f.step = (int)t;
  f.flags = flags;
  f.active_hist = b.HIST;
  f.host_active = host_active;
  return launch_finalize(f, s);
}

// The launches of decode step t in the transformer graph (q8_engine.rs:382-451
// with the self-attention block of the BASELINE decoder layer).
hipError_t Translation::emit_step(const StepPlan& P, uint32_t t) {
  const int rows = P.rows;
  // When an attention block consumes a LayerNorm (or the decoder input
  // embedding), it builds its rows in its own prologue: no separate kernel,
  // and the LayerNorm's sequential folds overlap the block's weight and key
  // loads.  `pend` is the not yet materialised layer input; kind PRO_NONE
  // means it is in DXQ / DXA.
  RowPrologue pend;
  float* xres = b.DX0;  // the residual stream
  float* xalt = b.DX1;  // where the next LayerNorm writes it
  auto dgemm = [&](const int8_t* A, const float* a, const Lin& L, int mode, const Epilogue& e) {
    GemmArgs g;
    g.A = A;
    g.a = a;
    g.lda = L.K;
    g.M = rows;
    g.M_dev = d_nact;
    g.K = L.K;
    g.W = L.w;
    g.Wf = L.wf;
    g.wmult = L.mult;
    g.bias = L.bias;
    g.N = L.N;
    return launch_gemm_skinny(g, mode, e, s);
  };
  // Attention-output projection.  A is the fp32 attention output, quantized
  // while loading with the per-head maxima the attention kernel wrote; each
  // workgroup quantizes only its own 16 rows, so no row-quantization pass
  // runs in between.
  auto agemm = [&](const Lin& L, const Epilogue& e) -> hipError_t {
    GemmArgs g;
    g.Af = b.DATT;
    g.ldaf = d;
    g.Aamax = b.DAMAX;
    g.amax_parts = H;
    g.M = rows;
    g.M_dev = d_nact;
    g.K = L.K;
    g.W = L.w;
    g.Wf = L.wf;
    g.wmult = L.mult;
    g.bias = L.bias;
    g.N = L.N;
    return launch_gemm_skinny(g, EPI_STORE, e, s);
  };
  auto store_epi = [&](float* out, int ldo, int relu) {
    Epilogue e;
    e.out = out;
    e.ldo = ldo;
    e.relu = relu;
    return e;
  };
  auto xgemm = [&](const Lin& L, int mode, const Epilogue& e) -> hipError_t {
    return dgemm(b.DXQ, b.DXA, L, mode, e);
  };
  // A LayerNorm of y + xres: run now, or (defer) left pending for its
  // consumer, which builds the rows in its prologue.
  auto layer_norm = [&](const float* y, const float* gm, const float* bt, bool defer) -> hipError_t {
    hipError_t rc = hipSuccess;
    if (!defer) {
      rc = launch_residual_ln(y, xres, gm, bt, rows, d_nact, d, xalt, b.DXQ, b.DXA, E->err_flag, s, 0.0f,
                              fast);
    } else {
      pend = RowPrologue();
      pend.kind = PRO_LN;
      pend.y = y;
      pend.r = xres;
      pend.gamma = gm;
      pend.beta = bt;
      pend.out = xalt;
      pend.err = E->err_flag;
      pend.fast = fast;
    }
    std::swap(xres, xalt);
    return rc;
  };
  auto block = [&](int mode, uint32_t layer, const Lin& L, const float* k, const float* v,
                   int64_t ldkv, float* kc_out, float* vc_out, const int64_t* key0,
                   const int32_t* nk, int64_t max_row, int max_keys) -> hipError_t {
    hipEvent_t ev[2];
    MH_TRY(timer(mode == ATT_SELF ? MARIAN_HIP_KERNEL_SELF_BLOCK : MARIAN_HIP_KERNEL_CROSS_BLOCK, t,
                 layer, ev));
    BlockArgs ba;
    ba.mode = mode;
    ba.pro = pend;
    pend.kind = PRO_NONE;
    ba.rows = rows;
    ba.rows_dev = d_nact;
    ba.heads = (int)H;
    ba.W = L.wf;
    ba.wmult = L.mult;
    ba.bias = L.bias;
    ba.k = k;
    ba.v = v;
    ba.kc_out = kc_out;
    ba.vc_out = vc_out;
    ba.ldkv = ldkv;
    ba.row_key0 = key0;
    ba.row_nk = nk;
    ba.step = (int)t;
    ba.max_row = max_row;
    ba.max_keys = max_keys;
    ba.out = b.DATT;
    ba.ldo = d;
    ba.amax = b.DAMAX;
    ba.err = E->err_flag;
    ba.fast = fast;
    return launch_attn_block(ba, s, ev[0], ev[1]);
  };
  if (P.blk_self) {
    pend = RowPrologue();
    pend.kind = PRO_EMB;
    pend.emb = E->emb.w;
    pend.emb_mult = E->emb.mult;
    pend.pos = E->pos;
    pend.scale = E->emb_scale;
    pend.row_prev = rm.prev;
    pend.out = xres;
    pend.err = E->err_flag;
  } else {
    EmbedArgs ea;
    ea.emb = E->emb.w;
    ea.emb_mult = E->emb.mult;
    ea.pos = E->pos;
    ea.scale = E->emb_scale;
    ea.d = d;
    ea.row_prev = rm.prev;
    ea.step = (int)t;
    ea.rows = rows;
    ea.rows_dev = d_nact;
    ea.x = xres;
    ea.xq = b.DXQ;
    ea.xa = b.DXA;
    ea.err = E->err_flag;
    MH_TRY(launch_embed(ea, s));
  }
  for (uint32_t l = 0; l < E->Ld; ++l) {
    const DecLayer& L = E->dec[l];
    float* kc = b.KC + (size_t)l * CR * d;
    float* vc = b.VC + (size_t)l * CR * d;
    const float* ckv = b.CKV + (size_t)l * TR * 2 * d;
    // ---- self-attention over the row's cache ----
    if (P.blk_self) {
      MH_TRY(block(ATT_SELF, l, L.self_qkv, kc, vc, d, kc, vc, rm.kv0, nullptr, (int64_t)CR, P.self_keys));
    } else {
      Epilogue e;
      e.out = b.DQ;
      e.ldo = d;
      e.kcache = kc;
      e.vcache = vc;
      e.row_kv0 = rm.kv0;
      e.step = (int)t;
      e.d = d;
      MH_TRY(xgemm(L.self_qkv, EPI_QKV_CACHE, e));
      AttnArgs sa;
      sa.mode = ATT_SELF;
      sa.q = b.DQ;
      sa.ldq = d;
      sa.k = kc;
      sa.v = vc;
      sa.ldkv = d;
      sa.heads = H;
      sa.head_dim = d / H;
      sa.rows = rows;
      sa.rows_dev = d_nact;
      sa.row_key0 = rm.kv0;
      sa.max_row = (int64_t)CR;
      sa.step = (int)t;
      sa.max_keys = P.self_keys;
      sa.out = b.DATT;
      sa.ldo = d;
      sa.amax = b.DAMAX;
      sa.err = E->err_flag;
      sa.fast = fast;
      hipEvent_t ev[2];
      MH_TRY(timer(MARIAN_HIP_KERNEL_SELF_ATTN, t, l, ev));
      MH_TRY(launch_attention(sa, s, ev[0], ev[1]));
    }
    MH_TRY(agemm(L.self_out, store_epi(b.DY, d, 0)));
    MH_TRY(layer_norm(b.DY, L.ln1_s, L.ln1_b, P.blk_cross));
    // ---- cross-attention over the encoder output of the row's sentence ----
    if (P.blk_cross) {
      MH_TRY(block(ATT_CROSS, l, L.cross_q, ckv, ckv + d, 2 * (int64_t)d, nullptr, nullptr, rm.src0, rm.srcn,
                   (int64_t)TR, P.cross_keys));
    } else {
      MH_TRY(xgemm(L.cross_q, EPI_STORE, store_epi(b.DQ, d, 0)));
      AttnArgs ca;
      ca.mode = ATT_CROSS;
      ca.q = b.DQ;
      ca.ldq = d;
      ca.k = ckv;
      ca.v = ckv + d;
      ca.ldkv = 2 * d;
      ca.heads = H;
      ca.head_dim = d / H;
      ca.rows = rows;
      ca.rows_dev = d_nact;
      ca.row_key0 = rm.src0;
      ca.row_nk = rm.srcn;
      ca.max_row = (int64_t)TR;
      ca.max_keys = P.cross_keys;
      ca.out = b.DATT;
      ca.ldo = d;
      ca.amax = b.DAMAX;
      ca.err = E->err_flag;
      ca.fast = fast;
      hipEvent_t ev[2];
      MH_TRY(timer(MARIAN_HIP_KERNEL_CROSS_ATTN, t, l, ev));
      MH_TRY(launch_attention(ca, s, ev[0], ev[1]));
    }
    MH_TRY(agemm(L.cross_out, store_epi(b.DY, d, 0)));
    // ---- feed-forward; its LayerNorm inside the up-projection block ----
    MH_TRY(layer_norm(b.DY, L.ln2_s, L.ln2_b, P.ln_ffn || P.ln_rows));
    if (P.ln_rows) {  // more rows: eight rows per workgroup
      LnGemmRowsArgs lg;
      lg.y = pend.y;
      lg.r = pend.r;
      lg.gamma = pend.gamma;
      lg.beta = pend.beta;
      lg.x_out = pend.out;
      pend.kind = PRO_NONE;
      lg.rows = rows;
      lg.rows_dev = d_nact;
      lg.dyn = 1;
      lg.fast = fast;
      lg.part_n = F;
      lg.W = L.ffn1.wf;
      lg.wmult = L.ffn1.mult;
      lg.bias = L.ffn1.bias;
      lg.K = L.ffn1.K;
      lg.N = L.ffn1.N;
      lg.relu = 1;
      lg.out = b.DH;
      lg.ldo = F;
      lg.err = E->err_flag;
      MH_TRY(launch_ln_gemm_rows(lg, s));
    } else if (P.ln_ffn) {
      LnGemmArgs lg;
      lg.pro = pend;
      pend.kind = PRO_NONE;
      lg.rows = rows;
      lg.rows_dev = d_nact;
      lg.W = L.ffn1.wf;
      lg.wmult = L.ffn1.mult;
      lg.bias = L.ffn1.bias;
      lg.K = L.ffn1.K;
      lg.N = L.ffn1.N;
      lg.relu = 1;
      lg.out = b.DH;
      lg.ldo = F;
      lg.err = E->err_flag;
      MH_TRY(launch_ln_gemm_block(lg, s));
    } else {
      MH_TRY(xgemm(L.ffn1, EPI_STORE, store_epi(b.DH, F, 1)));
    }
    if (P.ffn_af) {
      // Few rows: the down-projection reads the fp32 hidden rows and finds
      // their maxima itself, in place of a row-quantization pass.
      GemmArgs g;
      g.Af = b.DH;
      g.ldaf = F;
      g.err = E->err_flag;
      g.M = rows;
      g.M_dev = d_nact;
      g.K = L.ffn2.K;
      g.W = L.ffn2.w;
      g.Wf = L.ffn2.wf;
      g.wmult = L.ffn2.mult;
      g.bias = L.ffn2.bias;
      g.N = L.ffn2.N;
      MH_TRY(launch_gemm_skinny(g, EPI_STORE, store_epi(b.DY, d, 0), s));
    } else {
      MH_TRY(launch_quantize_rows(b.DH, F, rows, d_nact, F, b.DHQ, F, b.DHA, E->err_flag, s));
      MH_TRY(dgemm(b.DHQ, b.DHA, L.ffn2, EPI_STORE, store_epi(b.DY, d, 0)));
    }
    // The last layer's LayerNorm goes into the vocabulary kernel's prologue
    // on steps with very few rows.
    MH_TRY(layer_norm(b.DY, L.ln3_s, L.ln3_b, l + 1 < E->Ld ? P.blk_self : P.vocab_ln));
  }
  return score(rows, t, pend);
}

// The launches of decode step t in the SSRU graph (q8_engine.rs:392-436): the
// decoder input, then per layer the SSRU sublayer (W and Wf on the layer
// input, gate, state update and LayerNorm), cross-attention over the row's
// sentence and the FFN, every dense layer's input quantized with that layer's
// static multiplier.
hipError_t Translation::emit_step_ssru(int rows, uint32_t t) {
  const bool ssru_blk = ssru_block_supported(d, H, (int)bs.Lmax);
  const bool ssru_lnf = ln_gemm_rows_supported(d, F) && ln_gemm_rows_supported(d, 2 * d);
  float* xres = b.DX0;
  float* xalt = b.DX1;
  auto dgemm = [&](const Lin& L, const int8_t* A, const float* a, float* out, int64_t ldo, int relu,
                   int8_t* q = nullptr, float* qa = nullptr, float qmult = 0.0f) {
    GemmArgs g;
    g.A = A;
    g.a = a;
    g.lda = L.K;
    g.M = rows;
    g.M_dev = d_nact;
    g.K = L.K;
    g.W = L.w;
    g.Wf = L.wf;
    g.wmult = L.mult;
    g.bias = L.bias;
    g.N = L.N;
    Epilogue e;
    e.out = out;
    e.ldo = ldo;
    e.relu = relu;
    e.out_q = q;
    e.ldq = L.N;
    e.out_qa = qa;
    e.qmult = qmult;
    if (q) g.err = E->err_flag;
    return launch_gemm_skinny(g, EPI_STORE, e, s);
  };
  auto qs = [&](const float* x, int K, float mult, int8_t* q, float* a) {
    return launch_quantize_rows_static(x, K, rows, K, mult, q, K, a, E->err_flag, s, d_nact);
  };
  const SGroup& uf0 = E->sdec[0].uf;
  // With the fused SSRU kernels the first layer's input kernel builds the
  // embedding itself.
  if (!ssru_blk) {
    EmbedArgs ea;
    ea.emb = E->emb.w;
    ea.emb_mult = E->emb.mult;
    ea.pos = E->pos;
    ea.scale = E->emb_scale;
    ea.d = d;
    ea.row_prev = rm.prev;
    ea.step = (int)t;
    ea.rows = rows;
    ea.rows_dev = d_nact;
    ea.x = xres;
    ea.xq = uf0.shared ? b.DXQ : nullptr;
    ea.xa = b.DXA;
    ea.qmult = uf0.shared ? uf0.act[0] : 0.0f;
    ea.err = E->err_flag;
    MH_TRY(launch_embed(ea, s));
  }
  // Residual LayerNorm + the linear that reads it, in one launch.
  // y == nullptr: y is the static linear Wy of the int8 rows DXQ (ya_mult).
  auto ln_gemm = [&](const float* y, const float* ln_s, const float* ln_b, const Lin& W, float a0, float a1,
                     int part_n, int relu, float* out, int8_t* q, float* qa, float qmult,
                     const Lin* Wy = nullptr, float ya_mult = 0.0f) {
    LnGemmRowsArgs lg;
    lg.y = y;
    if (!y) {
      lg.ya = b.DXQ;
      lg.ya_mult = ya_mult;
      lg.Wy = Wy->wf;
      lg.ymult = Wy->mult;
      lg.ybias = Wy->bias;
    }
    lg.r = xres;
    lg.gamma = ln_s;
    lg.beta = ln_b;
    lg.rows = rows;
    lg.rows_dev = d_nact;
    lg.x_out = xalt;
    lg.xq_mult[0] = a0;
    lg.xq_mult[1] = a1;
    lg.part_n = part_n;
    lg.W = W.wf;
    lg.wmult = W.mult;
    lg.bias = W.bias;
    lg.K = W.K;
    lg.N = W.N;
    lg.relu = relu;
    lg.out = out;
    lg.ldo = W.N;
    lg.out_q = q;
    lg.ldq = W.N;
    lg.qmult = qmult;
    lg.out_qa = qa;
    lg.err = E->err_flag;
    const hipError_t rc = launch_ln_gemm_rows(lg, s);
    std::swap(xres, xalt);
    return rc;
  };
  for (uint32_t l = 0; l < E->Ld; ++l) {
    const SDecLayer& L = E->sdec[l];
    float* st_in = b.STATE + ((size_t)(t & 1) * LdA + l) * R * d;
    float* st_out = b.STATE + ((size_t)((t + 1) & 1) * LdA + l) * R * d;
    const float* ckv = b.CKV + (size_t)l * TR * 2 * d;
    if (ssru_blk) {
      // ---- SSRU: the layer input, its candidate and forget-gate
      // projections and the state update (z = relu(state') + x in DUF) ----
      SsruInputArgs si;
      if (l == 0) {
        si.pro.kind = PRO_EMB;
        si.pro.emb = E->emb.w;
        si.pro.emb_mult = E->emb.mult;
        si.pro.pos = E->pos;
        si.pro.scale = E->emb_scale;
        si.pro.row_prev = rm.prev;
        si.step = (int)t;
      } else {  // the previous layer's last residual LayerNorm
        si.pro.kind = PRO_LN;
        si.pro.y = b.DY;
        si.pro.r = xres;
        si.pro.gamma = E->sdec[l - 1].ln2_s;
        si.pro.beta = E->sdec[l - 1].ln2_b;
      }
      si.rows = rows;
      si.rows_dev = d_nact;
      si.d = d;
      si.act_c = L.uf.act[0];
      si.act_f = L.uf.act[L.uf.shared ? 0 : 1];
      si.W = L.uf.all.wf;
      si.wmult = L.uf.all.mult;
      si.bias = L.uf.all.bias;
      si.state_in = st_in;
      si.state_out = st_out;
      si.state_row = rm.slot;
      si.state_rows = (int64_t)R;
      si.z = b.DUF;
      si.err = E->err_flag;
      MH_TRY(launch_ssru_input(si, s));
      // ---- SSRU LayerNorm, query projection and cross-attention ----
      SsruBlockArgs sb;
      sb.z = b.DUF;
      sb.gamma = L.ln0_s;
      sb.beta = L.ln0_b;
      sb.x_out = xalt;
      sb.xq_mult = L.aq;
      sb.Wq = L.q.wf;
      sb.wq_mult = L.q.mult;
      sb.wq_bias = L.q.bias;
      sb.k = ckv;
      sb.v = ckv + d;
      sb.ldkv = 2 * d;
      sb.row_key0 = rm.src0;
      sb.row_nk = rm.srcn;
      sb.max_row = (int64_t)TR;
      sb.max_keys = (int)bs.Lmax;
      sb.d = d;
      sb.heads = H;
      sb.rows = rows;
      sb.rows_dev = d_nact;
      sb.qout = b.DXQ;
      sb.ldqout = d;
      sb.qmult = L.ao;
      sb.qa = b.DXA;
      sb.err = E->err_flag;
      MH_TRY(launch_ssru_block(sb, s));
      std::swap(xres, xalt);
    } else {
      // ---- SSRU: candidate and forget-gate inputs side by side in DUF ----
      if (ssru_lnf && l > 0) {  // with the previous layer's last LayerNorm
        const SDecLayer& P = E->sdec[l - 1];
        MH_TRY(ln_gemm(b.DY, P.ln2_s, P.ln2_b, L.uf.all, L.uf.act[0], L.uf.act[L.uf.shared ? 0 : 1],
                       L.uf.shared ? 2 * d : d, 0, b.DUF, nullptr, nullptr, 0.0f));
      } else if (L.uf.shared) {
        MH_TRY(dgemm(L.uf.all, b.DXQ, b.DXA, b.DUF, 2 * d, 0));
      } else {
        for (int i = 0; i < 2; ++i) {
          MH_TRY(qs(xres, d, L.uf.act[i], b.DXQ, b.DXA));
          MH_TRY(dgemm(L.uf.part(i), b.DXQ, b.DXA, b.DUF + (size_t)i * d, 2 * d, 0));
        }
      }
      MH_TRY(launch_ssru_ln(b.DUF, b.DUF + d, st_in, xres, L.ln0_s, L.ln0_b, rows, d, xalt, b.DXQ, b.DXA,
                            E->err_flag, s, 2 * d, d_nact, rm.slot, L.aq, st_out));
      std::swap(xres, xalt);
      // ---- cross-attention over the row's sentence ----
      MH_TRY(dgemm(L.q, b.DXQ, b.DXA, b.DQ, d, 0));
      AttnArgs ca;
      ca.mode = ATT_CROSS;
      ca.q = b.DQ;
      ca.ldq = d;
      ca.k = ckv;
      ca.v = ckv + d;
      ca.ldkv = 2 * d;
      ca.heads = H;
      ca.head_dim = d / H;
      ca.rows = rows;
      ca.rows_dev = d_nact;
      ca.row_key0 = rm.src0;
      ca.row_nk = rm.srcn;
      ca.max_row = (int64_t)TR;
      ca.max_keys = (int)bs.Lmax;
      ca.out = b.DATT;
      ca.ldo = d;
      ca.err = E->err_flag;
      ca.qout = b.DXQ;  // quantized for Wo with its static multiplier
      ca.ldqout = d;
      ca.qa = b.DXA;
      ca.qmult = L.ao;
      MH_TRY(launch_attention(ca, s));
    }
    // ---- output projection, context LayerNorm, feed-forward (hidden
    // quantized for W2) ----
    if (ssru_lnf) {  // every workgroup projects its rows itself
      MH_TRY(ln_gemm(nullptr, L.ln1_s, L.ln1_b, L.w1, L.a1, L.a1, F, 1, nullptr, b.DHQ, b.DHA, L.a2, &L.o, L.ao));
    } else {
      MH_TRY(dgemm(L.o, b.DXQ, b.DXA, b.DY, d, 0));
      MH_TRY(launch_residual_ln(b.DY, xres, L.ln1_s, L.ln1_b, rows, d_nact, d, xalt, b.DXQ, b.DXA, E->err_flag,
                                s, L.a1));
      std::swap(xres, xalt);
      MH_TRY(dgemm(L.w1, b.DXQ, b.DXA, nullptr, F, 1, b.DHQ, b.DHA, L.a2));
    }
    MH_TRY(dgemm(L.w2, b.DHQ, b.DHA, b.DY, d, 0));
    // The next layer's SSRU projections build this LayerNorm themselves, and
    // so does the candidate scoring after the last layer.
    if ((ssru_blk || ssru_lnf) && l + 1 < E->Ld) continue;
    if (l + 1 == E->Ld && cand && cand_ln_supported(d)) {
      RowPrologue pend;
      pend.kind = PRO_LN;
      pend.y = b.DY;
      pend.r = xres;
      pend.gamma = L.ln2_s;
      pend.beta = L.ln2_b;
      pend.err = E->err_flag;
      return score(rows, t, pend, E->out_act);
    }
    // quantized for what reads it next: the next layer's SSRU inputs (when
    // they share a multiplier) or the output scoring
    const SGroup* nx = l + 1 < E->Ld ? &E->sdec[l + 1].uf : nullptr;
    const float qm = nx ? (nx->shared ? nx->act[0] : 0.0f) : E->out_act;
    MH_TRY(launch_residual_ln(b.DY, xres, L.ln2_s, L.ln2_b, rows, d_nact, d, xalt, qm > 0.0f ? b.DXQ : nullptr,
                              b.DXA, E->err_flag, s, qm));
    std::swap(xres, xalt);
  }
  RowPrologue none;
  return score(rows, t, none);
}

// The greedy decode loop with the device-side active set.  The host knows an
// upper bound on the active rows of every step (rows whose limit exceeds t);
// rows that end on EOS are seen through polling: on every kPoll-th step the
// finalizer also stores the new count in a pinned host slot, read once the
// event after that step has completed.  A slot starts at -1, and a count read
// late is an older, larger one: polling only ever stops the loop late, never
// early.
hipError_t Translation::decode() {
  E->kev_kind.clear();
  E->kev_step.clear();
  E->kev_layer.clear();
  E->kev_us.clear();
  if (E->timing & MARIAN_HIP_TIME_STEPS) {
    while (E->step_ev.size() < gen_limit) {
      hipEvent_t ev;
      MH_TRY(hipEventCreate(&ev));
      E->step_ev.push_back(ev);
    }
  }
  const std::vector<uint32_t>& limit = E->h_limit;
  std::vector<uint32_t>& remaining = E->h_remaining;  // rows with limit > t
  remaining.assign(gen_limit + 1, 0);
  for (size_t i = 0; i < B; ++i) remaining[0] += limit[i] > 0;
  {
    std::vector<uint32_t>& ends = E->h_ends;
    ends.assign(gen_limit + 1, 0);
    for (size_t i = 0; i < B; ++i) ends[limit[i]]++;
    for (uint32_t t = 1; t <= gen_limit; ++t) remaining[t] = remaining[t - 1] - ends[t];
  }
  int poll_slot = 0;
  uint32_t polls = 0;
  bool done = n_active0 == 0;
  E->pinned[0] = E->pinned[1] = -1;
  auto poll = [&]() -> hipError_t {
    // this step's count is on its way; look at the previous one if it has landed
    MH_TRY(hipEventRecord(E->ev[3 + poll_slot], s));
    const int other = poll_slot ^ 1;
    if (polls > 0 && hipEventQuery(E->ev[3 + other]) == hipSuccess && E->pinned[other] == 0) done = true;
    poll_slot = other;
    ++polls;
    return hipSuccess;
  };
  steps = 0;
  for (uint32_t t = 0; t < gen_limit && !done; ++t) {
    const int rows = (int)remaining[t];
    if (rows == 0) break;
    host_active = (t + 1) % kPoll == 0 ? E->pinned + poll_slot : nullptr;
    MH_TRY(E->ssru ? emit_step_ssru(rows, t) : emit_step(make_plan(rows, (int)t + 1, (int)bs.Lmax), t));
    if (E->timing & MARIAN_HIP_TIME_STEPS) MH_TRY(hipEventRecord(E->step_ev[t], s));
    ++steps;
    if ((t + 1) % kPoll == 0) MH_TRY(poll());
  }
  return hipEventRecord(E->ev[2], s);
}

// Results back to the host, the call's statistics, and the outputs in
// sequence order.
int Translation::finish(int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets, size_t* out_len) {
  uint32_t* count = (uint32_t*)E->hbuf[marian_hip_engine::H_COUNT];
  int32_t* gen = (int32_t*)E->hbuf[marian_hip_engine::H_GEN];
  uint32_t* hist = (uint32_t*)E->hbuf[marian_hip_engine::H_HIST];
  int* err_host = E->pinned + 2;  // pinned, like the other readbacks
  *err_host = 0;
  if (steps) MH_HIP(hipMemcpyAsync(hist, b.HIST, 4ull * steps, hipMemcpyDeviceToHost, s));
  MH_HIP(hipMemcpyAsync(count, b.COUNT, 4 * B, hipMemcpyDeviceToHost, s));
  MH_HIP(hipMemcpyAsync(gen, b.OUT, 4 * cache_rows, hipMemcpyDeviceToHost, s));
  MH_HIP(hipMemcpyAsync(err_host, E->err_flag, sizeof(int), hipMemcpyDeviceToHost, s));
  hipEvent_t ev_end = E->ev[5];
  MH_HIP(hipEventRecord(ev_end, s));
  MH_HIP(hipEventSynchronize(ev_end));
  // Steps launched after every row had finished (before the poll saw the
  // count reach zero) ran on no rows.
  launched = steps;
  while (steps > 0 && hist[steps - 1] == 0) --steps;
  E->step_rows.assign(hist, hist + steps);
  float ms_total = 0, ms_enc = 0, ms_dec = 0;
  hipEventElapsedTime(&ms_total, E->ev[0], ev_end);
  hipEventElapsedTime(&ms_enc, E->ev[0], E->ev[1]);
  hipEventElapsedTime(&ms_dec, E->ev[1], E->ev[2]);
  marian_hip_stats& st = E->stats;
  st.total_ms = ms_total;
  st.encoder_ms = ms_enc;
  st.decode_ms = ms_dec;
  st.decode_steps = steps;
  st.launched_steps = launched;
  st.max_active_rows = (uint32_t)n_active0;
  st.vocab_kernel_ms = 0;
  st.vocab_kernel_launches = 0;
  // Like the step trace, the launch trace ends with the last step that ran on rows.
  while (n_timed > 0 && E->kev_step[n_timed - 1] >= steps) --n_timed;
  E->kev_kind.resize(n_timed);
  E->kev_step.resize(n_timed);
  E->kev_layer.resize(n_timed);
  E->kev_us.assign(n_timed, 0.0f);
  for (size_t i = 0; i < n_timed; ++i) {
    float ms = 0;
    MH_HIP(hipEventElapsedTime(&ms, E->kev[2 * i], E->kev[2 * i + 1]));
    E->kev_us[i] = ms * 1000.0f;
    if (E->kev_kind[i] == MARIAN_HIP_KERNEL_VOCAB) {
      st.vocab_kernel_ms += ms;
      ++st.vocab_kernel_launches;
    }
  }
  E->step_ms.assign(steps, 0.0f);
  if (E->timing & MARIAN_HIP_TIME_STEPS)
    for (uint32_t i = 0; i < std::min(steps, launched); ++i)
      hipEventElapsedTime(&E->step_ms[i], E->ev[0], E->step_ev[i]);
  st.allocations = E->allocs;
  if (*err_host == 2) return E->fail(MARIAN_HIP_ERR_INFERENCE, "key range exceeds the attention kernel");
  if (*err_host == 3) return E->fail(MARIAN_HIP_ERR_INFERENCE, "active rows exceed the step bound");
  if (*err_host) return E->fail(MARIAN_HIP_ERR_INFERENCE, "activation is not finite");

  if (pr.active) std::memset(pr.active, 0, B);
  if (PLOG) {  // the probed step's rows, back in sequence order
    std::vector<int32_t> slot(R + 1);
    MH_HIP(hipMemcpy(slot.data(), PSLOT, 4ull * (R + 1), hipMemcpyDeviceToHost));
    const size_t n = (size_t)std::min<int64_t>(std::max(slot[R], 0), (int64_t)std::min(R, B));
    std::vector<float> lg(n * E->V);
    if (n) MH_HIP(hipMemcpy(lg.data(), PLOG, 4ull * n * E->V, hipMemcpyDeviceToHost));
    for (size_t r = 0; r < n; ++r) {
      const int32_t q = slot[r];
      if (q < 0 || (size_t)q >= B) continue;
      std::memcpy(pr.logits + (size_t)q * E->V, lg.data() + r * E->V, 4ull * E->V);
      if (pr.active) pr.active[q] = 1;
    }
  }

  size_t total = 0;
  for (size_t i = 0; i < B; ++i) total += count[i];
  st.generated_tokens = total;
  if (out_len) *out_len = total;
  if (total > out_cap || (total && !out_tokens))
    return E->fail(MARIAN_HIP_ERR_BUFFER, "output buffer holds %zu tokens; %zu needed", out_cap, total);
  size_t o = 0;
  out_offsets[0] = 0;
  const std::vector<int64_t>& kv_base = E->h_kv_base;
  for (size_t i = 0; i < B; ++i) {
    std::memcpy(out_tokens + o, gen + kv_base[i], 4ull * count[i]);
    o += count[i];
    out_offsets[i + 1] = (uint32_t)o;
  }
  return MARIAN_HIP_OK;
}

#undef MH_TRY

int translate(marian_hip_engine* E, const int32_t* tokens, size_t n_tokens, const uint32_t* offsets,
              size_t n_offsets, const uint32_t* max_output_tokens, uint32_t flags, const uint32_t* cand,
              const uint32_t* cand_off, int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets,
              size_t* out_len, const Probe& pr) {
  if (!E) return MARIAN_HIP_ERR_INVALID_INPUT;
  E->error.clear();
  if (!E->ready) return E->fail(MARIAN_HIP_ERR_NOT_READY, "engine is not ready after a device error");
  if (!max_output_tokens || !out_offsets) return E->fail(MARIAN_HIP_ERR_INVALID_INPUT, "null input pointer");
  if ((cand || cand_off) && pr.logits)
    return E->fail(MARIAN_HIP_ERR_INVALID_INPUT, "logits are probed without candidates only");
  Translation c(E);
  if (int rc = check_batch(E->limits, E->Vs, E->V, tokens, n_tokens, offsets, n_offsets, cand, cand_off, c.bs,
                           E->error))
    return rc;
  c.tokens = tokens;
  c.n_tokens = n_tokens;
  c.offsets = offsets;
  c.B = c.bs.B;
  c.max_out = max_output_tokens;
  c.flags = flags;
  c.cand = cand;
  c.cand_off = cand_off;
  c.pr = pr;
  c.fast = flags & MARIAN_HIP_FLAG_FAST_REDUCTIONS;
  if (c.fast && E->ssru)
    return E->fail(MARIAN_HIP_ERR_INVALID_INPUT, "fast reductions are implemented for the transformer graph only");

  const hipError_t he = hipSetDevice(E->device);
  if (he != hipSuccess) return E->hip_fail(he, "hipSetDevice");
  c.s = E->stream;
  E->stats = marian_hip_stats{};
  E->allocs = 0;
  if (int rc = c.prepare()) return rc;
  hipError_t e = c.upload();
  if (e != hipSuccess) return E->hip_fail(e, "batch upload");
  e = c.encode();
  if (e != hipSuccess) return E->hip_fail(e, "encoder");
  MH_HIP(hipEventRecord(E->ev[1], c.s));
  if (c.PSLOT) MH_HIP(hipMemsetAsync(c.PSLOT + c.R, 0, sizeof(int32_t), c.s));  // no rows unless the step runs
  e = c.decode();
  if (e != hipSuccess) return E->hip_fail(e, "decode step");
  return c.finish(out_tokens, out_cap, out_offsets, out_len);
}

}  // namespace

extern "C" {

int marian_hip_validate_batch(const marian_hip_limits* limits, uint32_t source_vocab, uint32_t target_vocab,
                              const int32_t* tokens, size_t n_tokens, const uint32_t* offsets,
                              size_t n_offsets, const uint32_t* candidates, const uint32_t* candidate_offsets,
                              char* msg, size_t msg_cap) {
  marian_hip_limits lim = limits ? *limits : marian_hip_limits{2, 256, 4096, 256, 256, 65536};
  BatchShape bs;
  std::string why;
  const int rc = check_batch(lim, source_vocab, target_vocab, tokens, n_tokens, offsets, n_offsets,
                             candidates, candidate_offsets, bs, why);
  if (msg && msg_cap) std::snprintf(msg, msg_cap, "%s", why.c_str());
  return rc;
}

int marian_hip_reserve(marian_hip_engine* E, const marian_hip_capacity* c) {
  if (!E || !c) return MARIAN_HIP_ERR_INVALID_INPUT;
  E->error.clear();
  if (!E->ready) return E->fail(MARIAN_HIP_ERR_NOT_READY, "engine is not ready after a device error");
  if (!c->sentences || c->sentences > (uint32_t)kMaxRowsPerCall)
    return E->fail(MARIAN_HIP_ERR_INVALID_INPUT, "capacity of %u sentences; this engine handles 1-%d per call",
                   c->sentences, kMaxRowsPerCall);
  const hipError_t he = hipSetDevice(E->device);
  if (he != hipSuccess) return E->hip_fail(he, "hipSetDevice");
  CallShape cs;
  cs.B = c->sentences;
  cs.T = std::max<uint32_t>(c->source_tokens, c->sentences);
  cs.cand = c->candidate_ids > 0;
  cs.n_cand = c->candidate_ids;
  const int full = argmax_groups((int)E->V, (int)E->d);
  cs.nparts = cs.cand ? std::max(full, cand_groups((int)std::min<uint32_t>(c->max_candidates, E->V))) : full;
  cs.cache_rows = std::max<uint64_t>(c->output_tokens, 1);
  cs.gen_limit = std::min<uint32_t>(c->steps, kMaxPosition);
  MetaLayout L;
  CallBufs b;
  E->allocs = 0;
  return plan_buffers(E, cs, L, b);
}

int marian_hip_warmup(marian_hip_engine* E) {
  // Q8CpuEngine::warmup (q8_engine.rs:349-351): one sentence [2, 0], at most
  // four output tokens; it runs every stage of the path once.
  const int32_t tokens[2] = {2, 0};
  const uint32_t offsets[2] = {0, 2};
  const uint32_t limit[1] = {4};
  int32_t out[4];
  uint32_t out_offsets[2];
  size_t n = 0;
  return translate(E, tokens, 2, offsets, 2, limit, 0, nullptr, nullptr, out, 4, out_offsets, &n, Probe());
}

int marian_hip_translate_token_ids(marian_hip_engine* E, const int32_t* tokens, size_t n_tokens,
                                   const uint32_t* offsets, size_t n_offsets,
                                   const uint32_t* max_output_tokens, uint32_t flags,
                                   int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets,
                                   size_t* out_len) {
  return translate(E, tokens, n_tokens, offsets, n_offsets, max_output_tokens, flags, nullptr, nullptr,
                   out_tokens, out_cap, out_offsets, out_len, Probe());
}

int marian_hip_translate_shortlisted(marian_hip_engine* E, const int32_t* tokens, size_t n_tokens,
                                     const uint32_t* offsets, size_t n_offsets,
                                     const uint32_t* max_output_tokens, uint32_t flags,
                                     const uint32_t* candidates, const uint32_t* candidate_offsets,
                                     int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets,
                                     size_t* out_len) {
  if (!E) return MARIAN_HIP_ERR_INVALID_INPUT;
  if (!candidates || !candidate_offsets) {
    E->error = "candidate lists are required";
    return MARIAN_HIP_ERR_INVALID_INPUT;
  }
  return translate(E, tokens, n_tokens, offsets, n_offsets, max_output_tokens, flags, candidates,
                   candidate_offsets, out_tokens, out_cap, out_offsets, out_len, Probe());
}

int marian_hip_translate_probe(marian_hip_engine* E, const int32_t* tokens, size_t n_tokens,
                               const uint32_t* offsets, size_t n_offsets,
                               const uint32_t* max_output_tokens, uint32_t flags,
                               int32_t* out_tokens, size_t out_cap, uint32_t* out_offsets,
                               size_t* out_len, uint32_t probe_step, float* enc_out,
                               float* logits_out, uint8_t* active_out) {
  if (!E) return MARIAN_HIP_ERR_INVALID_INPUT;
  if (active_out && !logits_out) return E->fail(MARIAN_HIP_ERR_INVALID_INPUT, "active_out needs logits_out");
  Probe pr;
  pr.step = probe_step;
  pr.enc = enc_out;
  pr.logits = logits_out;
  pr.active = active_out;
  return translate(E, tokens, n_tokens, offsets, n_offsets, max_output_tokens, flags, nullptr, nullptr,
                   out_tokens, out_cap, out_offsets, out_len, pr);
}

}  // extern "C"
