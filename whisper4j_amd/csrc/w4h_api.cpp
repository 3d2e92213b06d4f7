// Host runtime of whisper4j_amd: models, sessions, the decoder step and the kernel-level entry
// points of the C ABI (include/w4h.h).  Device work is launched through w4h_internal.h.

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "w4h_host.h"
#include "w4h_internal.h"

using w4h::LayerDev;
using w4h::StepParams;
using w4h::u64;

namespace w4h {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIPCHK(expr)                                                                                   \
  do {                                                                                                 \
    hipError_t e_ = (expr);                                                                            \
    if (e_ != hipSuccess) return fail(W4H_ERR_DEVICE, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

// ---------------------------------------------------------------------------------------------
// f16 helpers (IEEE binary16, round to nearest even)

float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    if (ax < 0x33000000u) return (uint16_t)sign;
    uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126 - e;
    uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = (((ax >> 23) - 112) << 10) | ((ax & 0x7fffffu) >> 13), rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}


// ---------------------------------------------------------------------------------------------
// device memory

struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  int alloc(size_t bytes) {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
    if (bytes == 0) return W4H_OK;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
      p = nullptr;
      return fail(W4H_ERR_OOM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    }
    n = bytes;
    return W4H_OK;
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// Page-locked host staging buffer (hipHostMalloc): per-step copies between the caller's arrays
// and the device go through these, so they are true asynchronous DMA copies.
struct PinnedBuf {
  void* p = nullptr;
  size_t n = 0;
  PinnedBuf() = default;
  PinnedBuf(const PinnedBuf&) = delete;
  PinnedBuf& operator=(const PinnedBuf&) = delete;
  ~PinnedBuf() {
    if (p) (void)hipHostFree(p);
  }
  int ensure(size_t bytes) {
    if (n >= bytes) return W4H_OK;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    n = 0;
    hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
      p = nullptr;
      return fail(W4H_ERR_OOM, "hipHostMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    }
    n = bytes;
    return W4H_OK;
  }
};

int upload(DevBuf& b, const void* src, size_t bytes) {
  int rc = b.alloc(bytes);
  if (rc) return rc;
  if (bytes) HIPCHK(hipMemcpy(b.p, src, bytes, hipMemcpyHostToDevice));
  return W4H_OK;
}

}  // namespace w4h

using namespace w4h;

struct w4h_model {
  int device = 0;
  w4h_dims dims{};
  int wq8 = 0;
  std::vector<std::unique_ptr<DevBuf>> bufs;
  std::vector<LayerDev> layers;
  DevBuf layers_dev;
  const void* emb = nullptr;
  const uint16_t* emb_s = nullptr;
  const float *pos = nullptr, *lnf_g = nullptr, *lnf_b = nullptr;
  std::atomic<int> refs{1};
  std::atomic<bool> closed{false};
};

namespace {

struct TensorTable {
  std::map<std::string, const w4h_tensor*> by_name;
  const w4h_tensor* get(const std::string& n) const {
    auto it = by_name.find(n);
    return it == by_name.end() ? nullptr : it->second;
  }
};

int64_t numel(const w4h_tensor* t) {
  int64_t n = 1;
  for (int i = 0; i < t->n_dims; i++) n *= t->ne[i];
  return n;
}

DevBuf* new_buf(w4h_model* m) {
  m->bufs.push_back(std::make_unique<DevBuf>());
  return m->bufs.back().get();
}

// 1-D f32 tensor (f16 accepted and widened).
int load_vec(w4h_model* m, const TensorTable& tt, const std::string& name, int n, const float** out,
             bool optional = false) {
  const w4h_tensor* t = tt.get(name);
  if (!t) {
    if (optional) {
      *out = nullptr;
      return W4H_OK;
    }
    return fail(W4H_ERR_NOT_FOUND, "missing tensor: %s", name.c_str());
  }
  if (numel(t) != n) return fail(W4H_ERR_SHAPE, "tensor %s has %lld elements, expected %d", name.c_str(), (long long)numel(t), n);
  std::vector<float> v(n);
  if (t->type == W4H_TYPE_F32) {
    memcpy(v.data(), t->data, sizeof(float) * n);
  } else if (t->type == W4H_TYPE_F16) {
    const uint16_t* h = static_cast<const uint16_t*>(t->data);
    for (int i = 0; i < n; i++) v[i] = half_to_float(h[i]);
  } else {
    return fail(W4H_ERR_FORMAT, "tensor %s: type %d not supported for a vector", name.c_str(), t->type);
  }
  DevBuf* b = new_buf(m);
  int rc = upload(*b, v.data(), sizeof(float) * n);
  if (rc) return rc;
  *out = b->as<float>();
  return W4H_OK;
}

// Stack 2-D matrices [rows_i][K] (GGML ne = [K, rows_i]) into one device matrix.
// f16 mode: halves [N][K] (f32 sources rounded to f16).  q8 mode: int8 [N][K] + f16 scales [N][K/32].
int load_mat(w4h_model* m, const TensorTable& tt, const std::vector<std::string>& names, const std::vector<int>& rows,
             int K, const void** w, const uint16_t** s) {
  int N = 0;
  for (int r : rows) N += r;
  std::vector<const w4h_tensor*> ts;
  for (size_t i = 0; i < names.size(); i++) {
    const w4h_tensor* t = tt.get(names[i]);
    if (!t) return fail(W4H_ERR_NOT_FOUND, "missing tensor: %s", names[i].c_str());
    if (t->n_dims != 2 || t->ne[0] != K || t->ne[1] != rows[i])
      return fail(W4H_ERR_SHAPE, "tensor %s: expected ne=[%d,%d], got n_dims=%d ne=[%lld,%lld]", names[i].c_str(), K, rows[i],
                  t->n_dims, (long long)t->ne[0], (long long)(t->n_dims > 1 ? t->ne[1] : 1));
    const bool q8 = t->type == W4H_TYPE_Q8_0;
    if (q8 != (m->wq8 != 0))
      return fail(W4H_ERR_FORMAT, "tensor %s: matrix type %d does not match the model's %s matrices", names[i].c_str(),
                  t->type, m->wq8 ? "q8_0" : "f16/f32");
    if (!q8 && t->type != W4H_TYPE_F16 && t->type != W4H_TYPE_F32)
      return fail(W4H_ERR_FORMAT, "tensor %s: unsupported type %d", names[i].c_str(), t->type);
    ts.push_back(t);
  }
  if (!m->wq8) {
    std::vector<uint16_t> h((size_t)N * K);
    size_t o = 0;
    for (size_t i = 0; i < ts.size(); i++) {
      const size_t n = (size_t)rows[i] * K;
      if (ts[i]->type == W4H_TYPE_F16) {
        memcpy(h.data() + o, ts[i]->data, n * 2);
      } else {
        const float* f = static_cast<const float*>(ts[i]->data);
        for (size_t j = 0; j < n; j++) h[o + j] = float_to_half(f[j]);
      }
      o += n;
    }
    DevBuf* b = new_buf(m);
    int rc = upload(*b, h.data(), h.size() * 2);
    if (rc) return rc;
    *w = b->p;
    *s = nullptr;
  } else {
    if (K % 32) return fail(W4H_ERR_SHAPE, "q8_0 matrix needs K %% 32 == 0 (K=%d)", K);
    std::vector<int8_t> q((size_t)N * K);
    std::vector<uint16_t> sc((size_t)N * (K / 32));
    size_t row = 0;
    for (size_t i = 0; i < ts.size(); i++) {
      const unsigned char* src = static_cast<const unsigned char*>(ts[i]->data);
      for (int r = 0; r < rows[i]; r++, row++)
        for (int b = 0; b < K / 32; b++) {
          const unsigned char* blk = src + ((size_t)r * (K / 32) + b) * 34;
          sc[row * (K / 32) + b] = (uint16_t)(blk[0] | (blk[1] << 8));
          memcpy(q.data() + row * K + (size_t)b * 32, blk + 2, 32);
        }
    }
    DevBuf* bw = new_buf(m);
    int rc = upload(*bw, q.data(), q.size());
    if (rc) return rc;
    DevBuf* bs = new_buf(m);
    rc = upload(*bs, sc.data(), sc.size() * 2);
    if (rc) return rc;
    *w = bw->p;
    *s = bs->as<uint16_t>();
  }
  return W4H_OK;
}

int build_model(w4h_model* m, const w4h_dims* dims, const w4h_tensor* tensors, int n_tensors) {
  TensorTable tt;
  for (int i = 0; i < n_tensors; i++) {
    if (!tensors[i].name) return fail(W4H_ERR_INVALID, "tensor %d has no name", i);
    tt.by_name[tensors[i].name] = &tensors[i];
  }
  const int d = dims->n_text_state, V = dims->n_vocab, C = dims->n_text_ctx, L = dims->n_text_layer;
  const w4h_tensor* te = tt.get("decoder.token_embedding.weight");
  if (!te) return fail(W4H_ERR_NOT_FOUND, "missing tensor: decoder.token_embedding.weight");
  m->wq8 = te->type == W4H_TYPE_Q8_0;
  int rc;
  if ((rc = load_mat(m, tt, {"decoder.token_embedding.weight"}, {V}, d, &m->emb, &m->emb_s))) return rc;
  if ((rc = load_vec(m, tt, "decoder.positional_embedding", C * d, &m->pos))) return rc;
  if ((rc = load_vec(m, tt, "decoder.ln.weight", d, &m->lnf_g))) return rc;
  if ((rc = load_vec(m, tt, "decoder.ln.bias", d, &m->lnf_b))) return rc;
  m->layers.resize(L);
  for (int i = 0; i < L; i++) {
    LayerDev& ld = m->layers[i];
    const std::string b = "decoder.blocks." + std::to_string(i) + ".";
    const void** ws[8] = {&ld.w_qkv, &ld.w_o, &ld.w_cq, &ld.w_co, &ld.w_1, &ld.w_2, &ld.w_ck, &ld.w_cv};
    const uint16_t** ss[8] = {&ld.s_qkv, &ld.s_o, &ld.s_cq, &ld.s_co, &ld.s_1, &ld.s_2, &ld.s_ck, &ld.s_cv};
    if ((rc = load_mat(m, tt, {b + "attn.query.weight", b + "attn.key.weight", b + "attn.value.weight"}, {d, d, d}, d, ws[0], ss[0])))
      return rc;
    if ((rc = load_mat(m, tt, {b + "attn.out.weight"}, {d}, d, ws[1], ss[1]))) return rc;
    if ((rc = load_mat(m, tt, {b + "cross_attn.query.weight"}, {d}, d, ws[2], ss[2]))) return rc;
    if ((rc = load_mat(m, tt, {b + "cross_attn.out.weight"}, {d}, d, ws[3], ss[3]))) return rc;
    if ((rc = load_mat(m, tt, {b + "mlp.0.weight"}, {4 * d}, d, ws[4], ss[4]))) return rc;
    if ((rc = load_mat(m, tt, {b + "mlp.2.weight"}, {d}, 4 * d, ws[5], ss[5]))) return rc;
    if ((rc = load_mat(m, tt, {b + "cross_attn.key.weight"}, {d}, d, ws[6], ss[6]))) return rc;
    if ((rc = load_mat(m, tt, {b + "cross_attn.value.weight"}, {d}, d, ws[7], ss[7]))) return rc;
    // QKV bias: query and value biases, key bias if the checkpoint has one (else zeros)
    {
      std::vector<float> bq(3 * d, 0.0f);
      const char* parts[3] = {"attn.query.bias", "attn.key.bias", "attn.value.bias"};
      for (int p = 0; p < 3; p++) {
        const w4h_tensor* t = tt.get(b + parts[p]);
        if (!t) {
          if (p == 1) continue;
          return fail(W4H_ERR_NOT_FOUND, "missing tensor: %s%s", b.c_str(), parts[p]);
        }
        if (numel(t) != d || (t->type != W4H_TYPE_F32 && t->type != W4H_TYPE_F16))
          return fail(W4H_ERR_SHAPE, "tensor %s%s: bad shape or type", b.c_str(), parts[p]);
        for (int j = 0; j < d; j++)
          bq[p * d + j] = t->type == W4H_TYPE_F32 ? static_cast<const float*>(t->data)[j]
                                                  : half_to_float(static_cast<const uint16_t*>(t->data)[j]);
      }
      DevBuf* bb = new_buf(m);
      if ((rc = upload(*bb, bq.data(), bq.size() * 4))) return rc;
      ld.b_qkv = bb->as<float>();
    }
    if ((rc = load_vec(m, tt, b + "attn.out.bias", d, &ld.b_o))) return rc;
    if ((rc = load_vec(m, tt, b + "cross_attn.query.bias", d, &ld.b_cq))) return rc;
    if ((rc = load_vec(m, tt, b + "cross_attn.out.bias", d, &ld.b_co))) return rc;
    if ((rc = load_vec(m, tt, b + "cross_attn.value.bias", d, &ld.b_cv))) return rc;
    if ((rc = load_vec(m, tt, b + "mlp.0.bias", 4 * d, &ld.b_1))) return rc;
    if ((rc = load_vec(m, tt, b + "mlp.2.bias", d, &ld.b_2))) return rc;
    if ((rc = load_vec(m, tt, b + "attn_ln.weight", d, &ld.ln1_g))) return rc;
    if ((rc = load_vec(m, tt, b + "attn_ln.bias", d, &ld.ln1_b))) return rc;
    if ((rc = load_vec(m, tt, b + "cross_attn_ln.weight", d, &ld.ln2_g))) return rc;
    if ((rc = load_vec(m, tt, b + "cross_attn_ln.bias", d, &ld.ln2_b))) return rc;
    if ((rc = load_vec(m, tt, b + "mlp_ln.weight", d, &ld.ln3_g))) return rc;
    if ((rc = load_vec(m, tt, b + "mlp_ln.bias", d, &ld.ln3_b))) return rc;
  }
  if ((rc = upload(m->layers_dev, m->layers.data(), sizeof(LayerDev) * L))) return rc;
  return W4H_OK;
}

int set_device(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(W4H_ERR_DEVICE, "no HIP device available");
  if (device < 0 || device >= n) return fail(W4H_ERR_INVALID, "device %d out of range (%d devices)", device, n);
  HIPCHK(hipSetDevice(device));
  return W4H_OK;
}

}  // namespace

void model_release(w4h_model* m) {
  if (m && m->refs.fetch_sub(1) == 1) {
    (void)hipSetDevice(m->device);
    delete m;
  }
}

extern "C" {

const char* w4h_last_error(void) { return g_err.c_str(); }

int w4h_device_count(int32_t* n) {
  if (!n) return fail(W4H_ERR_INVALID, "null argument");
  int c = 0;
  if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
  *n = c;
  return W4H_OK;
}

int w4h_model_create(const w4h_dims* dims, const w4h_tensor* tensors, int32_t n_tensors, int32_t device,
                     w4h_model** out) {
  if (!dims || !tensors || !out || n_tensors <= 0) return fail(W4H_ERR_INVALID, "null argument");
  *out = nullptr;
  const int d = dims->n_text_state;
  if (d <= 0 || d % 64 || dims->n_text_head * 64 != d)
    return fail(W4H_ERR_INVALID, "n_text_state (%d) must be 64 * n_text_head (%d)", d, dims->n_text_head);
  if (dims->n_vocab <= 0 || dims->n_text_ctx <= 0 || dims->n_text_layer <= 0 || dims->n_audio_ctx <= 0)
    return fail(W4H_ERR_INVALID, "dimensions must be positive");
  if (d > 1280 * 2) return fail(W4H_ERR_INVALID, "n_text_state %d above the supported 2560", d);
  int rc = set_device(device);
  if (rc) return rc;
  auto* m = new w4h_model();
  m->device = device;
  m->dims = *dims;
  rc = build_model(m, dims, tensors, n_tensors);
  if (rc) {
    delete m;
    return rc;
  }
  *out = m;
  return W4H_OK;
}

int w4h_model_dims(const w4h_model* m, w4h_dims* out) {
  if (!m || !out) return fail(W4H_ERR_INVALID, "null argument");
  *out = m->dims;
  return W4H_OK;
}

int w4h_model_destroy(w4h_model* m) {
  if (!m) return fail(W4H_ERR_INVALID, "null argument");
  if (m->closed.exchange(true)) return fail(W4H_ERR_CLOSED, "model already destroyed");
  model_release(m);
  return W4H_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// sessions

// Input area of a session: the device cancel word at offset 0, the error word at kErrOff (the kernels'
// abort check reads both with one 8-byte load), per-step inputs from offset 256.
constexpr size_t kErrOff = 4;

struct w4h_session {
  w4h_model* m = nullptr;
  int S = 1, X = 1, max_ctx = 0, grid = 0, ngroups = 2, ncs_max = 0, ncc = 0, chc = 0, rpw = 0, mw = 0;
  size_t rep_stride = 0, res_off = 0;
  int nres = 0;
  size_t item_bytes = 0;  // LDS bytes of one resident vocabulary item
  size_t lds = 0;
  hipStream_t stream = nullptr;
  DevBuf kvk, kvv, xk, xv, ll, out, forced, mask, logits, xa_tmp, trace, bias;
  DevBuf xa_hl;  // f16 (hi, lo) planes of an encoder output for the all-layer cross-K/V GEMM
  // Per-step inputs in one device area (error word, tokens, extra mask, slot table) filled by one
  // copy from its page-locked staging twin; forced rows and results are staged separately.
  DevBuf in;
  PinnedBuf h_in, h_forced, h_out;
  size_t o_toks = 0, o_mask2 = 0, o_slots = 0, in_bytes = 0;
  template <class T>
  T* in_at(size_t off) const {
    return reinterpret_cast<T*>(static_cast<char*>(in.p) + off);
  }
  u64 *qkv = nullptr, *sp = nullptr, *x1 = nullptr, *cq = nullptr, *cp = nullptr, *x2 = nullptr, *hm = nullptr,
      *x3 = nullptr, *lp = nullptr, *lpa = nullptr;
  int kv_len = 0;
  uint32_t next_tag = 1;
  int probe = -1;
  bool has_mask = false;
  bool bias_on = false;  // the fixed logit bias in `bias` is applied
  std::vector<int32_t> slots_host;
  bool slots_identity = true, slots_dirty = false;
  bool closed = false;
  // batched (wide) engine
  bool wide = false;
  int Rp = 0, nch = 0, chlen = 0, nsel = 0;
  WideGemm g_qkv{}, g_o{}, g_cq{}, g_co{}, g_1{}, g_2{}, g_v{};
  DevBuf wx, wact, whid, wpart, wcpart, wselp, wnext, wctl;
  WideGraph wgraph, wgraph_beam;
  DevBuf wbeam, wbsup;
  bool use_graph = true;
  bool no_fuse = false;  // whole-K GEMM step switched off (W4H_WIDE_FUSE=0)
  DevBuf xvt;            // V transposed [L][H][64][Ap] for the matrix-core cross-attention, or empty
  int Ap = 0;
  // device-sampled decodes (T > 0): sampler state, the step's logits rows, the static suppress mask
  DevBuf samp, samp_row, samp_sup;
  DevBuf samp_x, samp_io;  // in-launch sampling: exchange words; drawn tokens and log-probabilities
  // cancellation (w4h_session_cancel, callable from any thread): the host flag, and the device cancel
  // word (input area offset 0, before the error word) written on a stream of its own
  std::atomic<int> cancel{0};
  std::mutex cancel_mu;
  hipStream_t ctl = nullptr;
};

namespace w4h {

static StepParams base_params(w4h_session* s) {
  w4h_model* m = s->m;
  StepParams p{};
  p.layers = m->layers_dev.as<LayerDev>();
  p.L = m->dims.n_text_layer;
  p.d = m->dims.n_text_state;
  p.H = m->dims.n_text_head;
  p.V = m->dims.n_vocab;
  p.C = m->dims.n_text_ctx;
  p.A = m->dims.n_audio_ctx;
  p.wq8 = m->wq8;
  p.emb = m->emb;
  p.emb_s = m->emb_s;
  p.pos = m->pos;
  p.lnf_g = m->lnf_g;
  p.lnf_b = m->lnf_b;
  p.S = s->S;
  p.X = s->X;
  p.max_ctx = s->max_ctx;
  p.kv_k = s->kvk.as<uint16_t>();
  p.kv_v = s->kvv.as<uint16_t>();
  p.xk = s->xk.as<uint16_t>();
  p.xv = s->xv.as<uint16_t>();
  p.slots = s->slots_identity ? nullptr : s->in_at<int32_t>(s->o_slots);
  p.qkv = s->qkv;
  p.sp = s->sp;
  p.x1 = s->x1;
  p.cq = s->cq;
  p.cp = s->cp;
  p.x2 = s->x2;
  p.hm = s->hm;
  p.x3 = s->x3;
  p.lp = s->lp;
  p.lpa = s->lpa;
  p.ncs_max = s->ncs_max;
  p.ncc = s->ncc;
  p.chc = s->chc;
  p.mask = s->has_mask ? s->mask.as<uint32_t>() : nullptr;
  p.mw = s->mw;
  p.probe = s->probe;
  p.err = s->in_at<unsigned>(kErrOff);
  p.rows_per_wg = s->rpw;
  p.ngroups = s->ngroups;
  p.rep_stride = s->rep_stride;
  p.nres = s->nres;
  p.res_off = s->res_off;
  p.bias = s->bias_on ? s->bias.as<float>() : nullptr;
  return p;
}

static WideParams wide_params(w4h_session* s) {
  w4h_model* m = s->m;
  WideParams p{};
  p.layers = m->layers.data();
  p.L = m->dims.n_text_layer;
  p.d = m->dims.n_text_state;
  p.H = m->dims.n_text_head;
  p.V = m->dims.n_vocab;
  p.C = m->dims.n_text_ctx;
  p.A = m->dims.n_audio_ctx;
  p.wq8 = m->wq8;
  p.emb = m->emb;
  p.emb_s = m->emb_s;
  p.pos = m->pos;
  p.lnf_g = m->lnf_g;
  p.lnf_b = m->lnf_b;
  p.S = s->S;
  p.X = s->X;
  p.max_ctx = s->max_ctx;
  p.Rp = s->Rp;
  p.kv_k = s->kvk.as<uint16_t>();
  p.kv_v = s->kvv.as<uint16_t>();
  p.xk = s->xk.as<uint16_t>();
  p.xv = s->xv.as<uint16_t>();
  p.xvt = s->xvt.p ? s->xvt.as<uint16_t>() : nullptr;
  p.Ap = s->Ap;
  p.slots = s->slots_identity ? nullptr : s->in_at<int32_t>(s->o_slots);
  p.x = s->wx.as<float>();
  p.act = s->wact.as<float>();
  p.hid = s->whid.as<float>();
  p.part = s->wpart.as<float>();
  p.cpart = s->wcpart.as<float>();
  p.selp = s->wselp.as<float>();
  p.next_tok = s->wnext.as<int32_t>();
  p.ctl = s->wctl.as<WideCtl>();
  p.graph = s->use_graph ? &s->wgraph : nullptr;
  p.no_fuse = s->no_fuse ? 1 : 0;
  p.nch = s->nch;
  p.chlen = s->chlen;
  p.nsel = s->nsel;
  p.g_qkv = s->g_qkv;
  p.g_o = s->g_o;
  p.g_cq = s->g_cq;
  p.g_co = s->g_co;
  p.g_1 = s->g_1;
  p.g_2 = s->g_2;
  p.g_v = s->g_v;
  p.mask = s->has_mask ? s->mask.as<uint32_t>() : nullptr;
  p.mw = s->mw;
  p.probe = s->probe;
  p.bias = s->bias.as<float>();
  p.bias_on = s->bias_on ? 1 : 0;
  return p;
}

static int ensure(DevBuf& b, size_t bytes) {
  if (b.n >= bytes) return W4H_OK;
  return b.alloc(bytes);
}

// Copy the step results (and the error word) back through the page-locked staging buffer, wait for
// the stream, and hand them to the caller's arrays.
static int copy_back(w4h_session* s, int n_steps, w4h_step_out* out, float* logits, unsigned* herr) {
  const int V = s->m->dims.n_vocab;
  const size_t b_err = 256, b_out = out ? sizeof(w4h_step_out) * (size_t)n_steps * s->S : 0;
  const size_t b_lg = logits ? sizeof(float) * (size_t)n_steps * s->S * V : 0;
  int rc;
  if ((rc = s->h_out.ensure(b_err + b_out + b_lg))) return rc;
  char* hp = static_cast<char*>(s->h_out.p);
  if (herr) HIPCHK(hipMemcpyAsync(hp, s->in_at<char>(kErrOff), sizeof(unsigned), hipMemcpyDeviceToHost, s->stream));
  if (b_out) HIPCHK(hipMemcpyAsync(hp + b_err, s->out.p, b_out, hipMemcpyDeviceToHost, s->stream));
  if (b_lg) HIPCHK(hipMemcpyAsync(hp + b_err + b_out, s->logits.p, b_lg, hipMemcpyDeviceToHost, s->stream));
  HIPCHK(hipStreamSynchronize(s->stream));
  if (herr) memcpy(herr, hp, sizeof(unsigned));
  if (b_out) memcpy(out, hp + b_err, b_out);
  if (b_lg) memcpy(logits, hp + b_err + b_out, b_lg);
  return W4H_OK;
}

// LDS layout of a launch with the decode rules: the rules region takes the start of the resident
// vocabulary region, which gives up as many items as that needs.  Returns the launch's LDS bytes,
// or 0 when the rules region does not fit.
static size_t rules_layout(const w4h_session* s, int hist_cap, StepParams& p) {
  const size_t rb = rules_lds_bytes(hist_cap, s->rpw);
  p.rules_off = s->res_off;
  p.res_off = s->res_off + rb;
  const int drop = s->nres > 0 ? (int)std::min<size_t>((size_t)s->nres, (rb + s->item_bytes - 1) / s->item_bytes) : 0;
  p.nres = s->nres - drop;
  const size_t lds = std::max(s->lds, p.res_off + (size_t)p.nres * s->item_bytes);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, s->m->device) != hipSuccess || lds > (size_t)prop.sharedMemPerBlock) return 0;
  return lds;
}

// The persistent step kernel is a cooperative launch whose workgroups (one per compute unit) must all
// be resident at once; two of them on one device, from sessions driven on different threads, could
// each hold compute units the other waits for.  Its launches are serialized per device, from the
// launch until the results are back on the host.
static std::mutex& coop_lock(int device) {
  static std::mutex m[64];
  return m[device & 63];
}

// Whether the in-launch draw's scratch (the pairs, scan words) fits the step kernel's phase region,
// which ends where the resident vocabulary rows begin (the selection reduce sizes it larger).
static size_t sample_scratch_room(const w4h_session* s) {
  const size_t d = (size_t)s->m->dims.n_text_state;
  const size_t big0 = 8 + kMaxRows + (size_t)kResItems * kMaxRows * 8 + (size_t)s->S * 4 * d + (size_t)s->S * d;
  return s->res_off / sizeof(float) > big0 ? s->res_off / sizeof(float) - big0 : 0;
}
static bool sample_scratch_fits(const w4h_session* s) { return sample_scratch_room(s) >= (size_t)2 * s->grid + 48; }

// Launch n_steps steps; tokens/forced are host arrays.  Results (if out) are copied back.  With
// `rules` (one-row persistent sessions, greedy feedback, out required) the decode rules run on the
// device and the run ends after the step that selects rules->eot; *steps_done receives the number
// of steps run and the self-KV advances by that many.
int run_steps(w4h_session* s, const int32_t* tokens, const int32_t* forced, int n_steps, const uint32_t* extra_mask,
              int topk, w4h_step_out* out, float* logits, float* ms, uint64_t* trace = nullptr,
              const RulesRun* rules = nullptr, int* steps_done = nullptr, const SampleRun* samp = nullptr,
              SampleRunOut* sout = nullptr) {
  if (s->closed) return fail(W4H_ERR_CLOSED, "session destroyed");
  if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled");
  if (!tokens || n_steps <= 0) return fail(W4H_ERR_INVALID, "tokens and n_steps > 0 required");
  if (topk < 0 || topk > W4H_TOPK_MAX) return fail(W4H_ERR_INVALID, "topk %d outside [0, %d]", topk, W4H_TOPK_MAX);
  if (s->kv_len + n_steps > s->max_ctx)
    return fail(W4H_ERR_CAPACITY, "self-KV capacity %d exceeded (kv_len %d + %d steps)", s->max_ctx, s->kv_len, n_steps);
  const int V = s->m->dims.n_vocab;
  for (int i = 0; i < s->S; i++)
    if (tokens[i] < 0 || tokens[i] >= V) return fail(W4H_ERR_INVALID, "token %d out of range [0, %d)", tokens[i], V);
  if (forced)
    for (size_t i = 0; i < (size_t)(n_steps - 1) * s->S; i++)
      if (forced[i] < 0 || forced[i] >= V) return fail(W4H_ERR_INVALID, "forced token %d out of range", forced[i]);
  if ((uint64_t)s->next_tag + (uint64_t)n_steps >= 0xfffffff0ull) return fail(W4H_ERR_INVALID, "tag space exhausted; recreate the session");
  HIPCHK(hipSetDevice(s->m->device));
  int rc;
  // per-step inputs: one asynchronous copy of the leading part of the input area that changed
  char* hp = static_cast<char*>(s->h_in.p);
  *reinterpret_cast<unsigned*>(hp + kErrOff) = 0u;  // error word (the cancel word before it is not copied)
  memcpy(hp + s->o_toks, tokens, sizeof(int32_t) * s->S);
  if (extra_mask) memcpy(hp + s->o_mask2, extra_mask, sizeof(uint32_t) * (size_t)s->S * s->mw);
  if (s->slots_dirty) memcpy(hp + s->o_slots, s->slots_host.data(), sizeof(int32_t) * s->slots_host.size());
  const size_t in_len = s->slots_dirty ? s->in_bytes : (extra_mask ? s->o_slots : s->o_mask2);
  HIPCHK(hipMemcpyAsync(s->in_at<char>(kErrOff), hp + kErrOff, in_len - kErrOff, hipMemcpyHostToDevice, s->stream));
  s->slots_dirty = false;
  if (rules && (s->wide || s->S != 1 || forced || !out || trace || !steps_done || rules->nhist < 0 ||
                (rules->nhist > 0 && !rules->hist)))
    return fail(W4H_ERR_INVALID, "device decode rules need a one-row persistent session, greedy feedback and outputs");
  if (rules && rules->nhist > 0) {  // the history travels in the forced-token buffers (unused here)
    const size_t b_hist = sizeof(int32_t) * (size_t)rules->nhist;
    if ((rc = ensure(s->forced, b_hist)) || (rc = s->h_forced.ensure(b_hist))) return rc;
    memcpy(s->h_forced.p, rules->hist, b_hist);
    HIPCHK(hipMemcpyAsync(s->forced.p, s->h_forced.p, b_hist, hipMemcpyHostToDevice, s->stream));
  }
  if (forced && n_steps > 1) {
    const size_t b_forced = sizeof(int32_t) * (size_t)(n_steps - 1) * s->S;
    if ((rc = ensure(s->forced, b_forced)) || (rc = s->h_forced.ensure(b_forced))) return rc;
    memcpy(s->h_forced.p, forced, b_forced);
    HIPCHK(hipMemcpyAsync(s->forced.p, s->h_forced.p, b_forced, hipMemcpyHostToDevice, s->stream));
  }
  if (out && (rc = ensure(s->out, sizeof(w4h_step_out) * (size_t)n_steps * s->S))) return rc;
  if (logits && (rc = ensure(s->logits, sizeof(float) * (size_t)n_steps * s->S * V))) return rc;
  const size_t trace_n = (size_t)n_steps * (6 * s->m->dims.n_text_layer + 2) * 4 * s->grid;
  if (trace && (rc = ensure(s->trace, trace_n * sizeof(uint64_t)))) return rc;
  if (s->wide) {
    if (trace) return fail(W4H_ERR_INVALID, "phase traces are recorded by the persistent step kernel only");
    WideParams wp = wide_params(s);
    wp.nsteps = n_steps;
    wp.kv_len0 = s->kv_len;
    wp.tokens0 = s->in_at<int32_t>(s->o_toks);
    wp.forced = (forced && n_steps > 1) ? s->forced.as<int32_t>() : nullptr;
    wp.mask2 = extra_mask ? s->in_at<uint32_t>(s->o_mask2) : nullptr;
    wp.topk = topk;
    wp.out = out ? s->out.as<w4h_step_out>() : nullptr;
    wp.logits_out = logits ? s->logits.as<float>() : nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (ms) {
      HIPCHK(hipEventCreate(&e0));
      HIPCHK(hipEventCreate(&e1));
      HIPCHK(hipEventRecord(e0, s->stream));
    }
    hipError_t le = launch_wide(wp, s->stream);
    if (le != hipSuccess) return fail(W4H_ERR_DEVICE, "batched step launch failed: %s", hipGetErrorString(le));
    if (ms) HIPCHK(hipEventRecord(e1, s->stream));
    if ((rc = copy_back(s, n_steps, out, logits, nullptr))) return rc;
    if (ms) {
      HIPCHK(hipEventElapsedTime(ms, e0, e1));
      (void)hipEventDestroy(e0);
      (void)hipEventDestroy(e1);
    }
    s->kv_len += n_steps;
    if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled");
    return W4H_OK;
  }
  StepParams p = base_params(s);
  p.nsteps = n_steps;
  p.kv_len0 = s->kv_len;
  p.tag0 = s->next_tag;
  p.tokens0 = s->in_at<int32_t>(s->o_toks);
  p.forced = (forced && n_steps > 1) ? s->forced.as<int32_t>() : nullptr;
  p.mask2 = extra_mask ? s->in_at<uint32_t>(s->o_mask2) : nullptr;
  p.topk = topk;
  p.out = out ? s->out.as<w4h_step_out>() : nullptr;
  p.logits_out = logits ? s->logits.as<float>() : nullptr;
  p.trace = trace ? s->trace.as<unsigned long long>() : nullptr;
  size_t lds = s->lds;
  if (rules) {
    p.rules = 1;
    p.eot = rules->eot;
    p.tsb = rules->tsb;
    p.hist0 = rules->nhist > 0 ? s->forced.as<int32_t>() : nullptr;
    p.nhist0 = rules->nhist;
    p.hist_cap = rules->nhist + n_steps;
    if (!(lds = rules_layout(s, p.hist_cap, p))) return fail(W4H_ERR_INVALID, "no LDS left for the device decode rules");
  }
  if (samp) {
    if (!rules || !sout || !(samp->temperature > 0.0f)) return fail(W4H_ERR_INVALID, "in-launch sampling needs the decode rules");
    const int V = s->m->dims.n_vocab;
    if (s->grid > kThreads || (size_t)V > (size_t)s->grid * kThreads * kSampEpt)
      return fail(W4H_ERR_INVALID, "in-launch sampling needs grid <= %d and V <= grid * %d", kThreads, kThreads * kSampEpt);
    if (!sample_scratch_fits(s)) return fail(W4H_ERR_INVALID, "no LDS left for the in-launch sampler");
    const size_t xw = (size_t)s->grid * 6 + 2;
    if ((rc = ensure(s->samp_x, xw * sizeof(u64))) || (rc = ensure(s->samp_row, sizeof(float) * (size_t)V)) ||
        (rc = ensure(s->samp_io, (sizeof(int32_t) + sizeof(double)) * (size_t)n_steps)))
      return rc;
    HIPCHK(hipMemsetAsync(s->samp_x.p, 0, xw * sizeof(u64), s->stream));
    p.samp_t = samp->temperature;
    p.samp_rng = samp->rng;
    p.samp_x = s->samp_x.as<u64>();
    p.samp_lds = sample_scratch_room(s) >= (size_t)8 * s->grid + 56 ? 1 : 0;
    p.samp_row = s->samp_row.as<float>();
    p.samp_lp = s->samp_io.as<double>();
    p.samp_tok = reinterpret_cast<int32_t*>(p.samp_lp + n_steps);
  }
  std::unique_lock<std::mutex> coop(coop_lock(s->m->device));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (ms) {
    HIPCHK(hipEventCreate(&e0));
    HIPCHK(hipEventCreate(&e1));
    HIPCHK(hipEventRecord(e0, s->stream));
  }
  hipError_t le = launch_step(p, s->grid, lds, s->stream);
  if (le != hipSuccess) return fail(W4H_ERR_DEVICE, "decoder step launch failed: %s", hipGetErrorString(le));
  s->next_tag += (uint32_t)n_steps;
  if (ms) HIPCHK(hipEventRecord(e1, s->stream));
  unsigned herr = 0;
  if (trace) HIPCHK(hipMemcpyAsync(trace, s->trace.p, trace_n * sizeof(uint64_t), hipMemcpyDeviceToHost, s->stream));
  if ((rc = copy_back(s, n_steps, out, logits, &herr))) return rc;
  if (ms) {
    HIPCHK(hipEventElapsedTime(ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }
  if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled during the launch");
  if (herr) return fail(W4H_ERR_TIMEOUT, "a device-side wait expired during the step (code %u); step aborted", herr);
  int done = n_steps;
  if (samp) {
    // the drawn tokens end the run at the end token; the records' argmax does not
    std::vector<char> io((sizeof(int32_t) + sizeof(double)) * (size_t)n_steps);
    HIPCHK(hipMemcpy(io.data(), s->samp_io.p, io.size(), hipMemcpyDeviceToHost));
    const double* lp = reinterpret_cast<const double*>(io.data());
    const int32_t* tk = reinterpret_cast<const int32_t*>(lp + n_steps);
    for (int i = 0; i < n_steps; i++)
      if (tk[i] == rules->eot) {
        done = i + 1;
        break;
      }
    sout->steps = done;
    sout->ended = tk[done - 1] == rules->eot;
    sout->tokens.assign(tk, tk + done);
    sout->lps.assign(lp, lp + done);
  } else if (rules) {
    for (int i = 0; i < n_steps; i++)
      if (out[i].argmax == rules->eot) {
        done = i + 1;
        break;
      }
  }
  if (steps_done) *steps_done = done;
  s->kv_len += done;
  return W4H_OK;
}

// The per-step input area: [error word | tokens | extra mask | slot table], each 256-byte aligned,
// with its page-locked staging twin; zero error word and tokens, identity slot table.
static int init_inputs(w4h_session* s) {
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  s->o_toks = 256;
  s->o_mask2 = s->o_toks + al(sizeof(int32_t) * s->S);
  s->o_slots = s->o_mask2 + al(sizeof(uint32_t) * (size_t)s->S * s->mw);
  s->in_bytes = s->o_slots + al(sizeof(int32_t) * s->slots_host.size());
  int rc;
  if ((rc = s->in.alloc(s->in_bytes)) || (rc = s->h_in.ensure(s->in_bytes))) return rc;
  memset(s->h_in.p, 0, s->in_bytes);
  memcpy(static_cast<char*>(s->h_in.p) + s->o_slots, s->slots_host.data(), sizeof(int32_t) * s->slots_host.size());
  HIPCHK(hipMemcpy(s->in.p, s->h_in.p, s->in_bytes, hipMemcpyHostToDevice));
  return W4H_OK;
}

// Session set-up for the batched engine: KV cache, cross K/V, slot table, GEMM slicing and the
// work buffers (residual rows, GEMM input rows, GEMM partials, attention and selection partials).
int create_wide(std::unique_ptr<w4h_session>& s, const hipDeviceProp_t& prop, w4h_session** out) {
  w4h_model* m = s->m;
  const w4h_dims& D = m->dims;
  const int L = D.n_text_layer, d = D.n_text_state, H = D.n_text_head, A = D.n_audio_ctx, V = D.n_vocab;
  if (d % kWideKBlock != 0 || d > 2048 || H * kHeadDim != d)
    return fail(W4H_ERR_INVALID, "batched engine needs n_text_state a multiple of %d (<= 2048) and head size %d", kWideKBlock, kHeadDim);
  const int ncu = prop.multiProcessorCount;
  s->Rp = s->S <= 16 ? 16 : 32;
  // Sessions of at most 16 rows run whole-K GEMMs with the residual, LayerNorm and GELU steps
  // inside them; W4H_WIDE_FUSE=0 keeps the split-K GEMMs and separate kernels.
  if (const char* e = getenv("W4H_WIDE_FUSE")) s->no_fuse = atoi(e) == 0;
  // With those, rows sharing one encoder output run cross-attention on the matrix cores (scores
  // and values of up to 16 rows per key chunk as MFMA tiles), reading V transposed.
  const bool xattn = !s->no_fuse && wide_fused_ok(d, s->Rp) && s->X == 1;
  s->g_qkv = wide_plan(nullptr, nullptr, 3 * d, d, ncu);
  s->g_o = wide_plan(nullptr, nullptr, d, d, ncu);
  s->g_cq = s->g_o;
  s->g_co = s->g_o;
  s->g_1 = wide_plan(nullptr, nullptr, 4 * d, d, ncu);
  s->g_2 = wide_plan(nullptr, nullptr, d, 4 * d, ncu);
  s->g_v = wide_plan(m->emb, m->emb_s, V, d, ncu);
  size_t pmax = 0;
  for (const WideGemm* g : {&s->g_qkv, &s->g_o, &s->g_1, &s->g_2, &s->g_v})
    pmax = std::max(pmax, (size_t)g->ks * s->Rp * g->N);
  // cross-attention chunks: enough (encoder, head, chunk) workgroups for two per compute unit, but
  // no more than ceil(A / kWideKeysPerPass), the fewest that keep every chunk within one pass of the
  // kernel's key loop: more, shorter chunks only add partials to merge (small, 5 rows: 751 us per
  // step with 23 chunks of 66 keys, 731 with 12 of 125)
  const int ngroups = (s->X == s->S || xattn) ? 1 : (s->S + 7) / 8;
  int per_cu = 2;  // W4H_XWG overrides the cross-attention workgroups per compute unit (tuning)
  if (const char* e = getenv("W4H_XWG")) per_cu = std::max(1, std::min(16, atoi(e)));
  int nch = (per_cu * ncu + s->X * H * ngroups - 1) / (s->X * H * ngroups);
  nch = std::max(1, std::min(std::min(nch, (A + kWideKeysPerPass - 1) / kWideKeysPerPass), 64));  // k_w_cmerge: <= 64
  if (xattn) nch = std::max(nch, (A + kXattnKeys - 1) / kXattnKeys);  // its chunks hold at most kXattnKeys keys
  if (nch > 64) return fail(W4H_ERR_INVALID, "n_audio_ctx %d needs more than 64 cross-attention chunks", A);
  s->chlen = (A + nch - 1) / nch;
  if (xattn) s->chlen = (s->chlen + 31) / 32 * 32;  // whole 32-key wave slices (<= kXattnKeys)
  s->nch = (A + s->chlen - 1) / s->chlen;
  s->nsel = (V + kWideSelChunk - 1) / kWideSelChunk;
  int rc;
  const size_t kv_elems = (size_t)L * s->S * H * s->max_ctx * kHeadDim;
  if ((rc = s->kvk.alloc(kv_elems * 2)) || (rc = s->kvv.alloc(kv_elems * 2))) return rc;
  const size_t x_elems = (size_t)s->X * L * H * A * kHeadDim;
  if ((rc = s->xk.alloc(x_elems * 2)) || (rc = s->xv.alloc(x_elems * 2))) return rc;
  // device buffers are cleared on the session's own stream (not the legacy stream, which other
  // threads' sessions may be capturing beside)
  HIPCHK(hipStreamCreate(&s->stream));
  HIPCHK(hipMemsetAsync(s->xk.p, 0, x_elems * 2, s->stream));
  HIPCHK(hipMemsetAsync(s->xv.p, 0, x_elems * 2, s->stream));
  if (xattn) {
    // frames padded past the last 128-frame tile by one more chunk, all zero, so that a wave's
    // 32-key slice of the last chunk reads inside the rows
    s->Ap = (A + 127) / 128 * 128 + kXattnKeys;
    const size_t t_elems = (size_t)L * H * kHeadDim * s->Ap;
    if ((rc = s->xvt.alloc(t_elems * 2))) return rc;
    HIPCHK(hipMemsetAsync(s->xvt.p, 0, t_elems * 2, s->stream));
  }
  s->slots_host.resize((size_t)s->S * s->max_ctx);
  for (int r = 0; r < s->S; r++)
    for (int q = 0; q < s->max_ctx; q++) s->slots_host[(size_t)r * s->max_ctx + q] = r;
  if ((rc = init_inputs(s.get()))) return rc;
  if ((rc = s->wx.alloc(sizeof(float) * (size_t)s->S * d))) return rc;
  if ((rc = s->wact.alloc(sizeof(float) * (size_t)s->Rp * 4 * d))) return rc;
  HIPCHK(hipMemsetAsync(s->wact.p, 0, sizeof(float) * (size_t)s->Rp * 4 * d, s->stream));
  if ((rc = s->whid.alloc(sizeof(float) * (size_t)s->Rp * 4 * d))) return rc;
  HIPCHK(hipMemsetAsync(s->whid.p, 0, sizeof(float) * (size_t)s->Rp * 4 * d, s->stream));
  if ((rc = s->wpart.alloc(sizeof(float) * pmax))) return rc;
  if ((rc = s->wcpart.alloc(sizeof(float) * (size_t)s->S * H * s->nch * kPartWords))) return rc;
  if ((rc = s->wselp.alloc(sizeof(float) * (size_t)s->S * s->nsel * kSelWords))) return rc;
  if ((rc = s->wnext.alloc(sizeof(int32_t) * s->S))) return rc;
  if ((rc = s->wctl.alloc(sizeof(WideCtl)))) return rc;
  HIPCHK(hipMemsetAsync(s->wctl.p, 0, sizeof(WideCtl), s->stream));
  HIPCHK(wide_prepare(s->Rp, m->wq8));
  // One step is captured as a HIP graph and replayed per step; W4H_GRAPH=0 launches every kernel.
  if (const char* e = getenv("W4H_GRAPH")) s->use_graph = atoi(e) != 0;
  if ((rc = s->mask.alloc(sizeof(uint32_t) * (size_t)s->S * s->mw))) return rc;
  if ((rc = s->bias.alloc(sizeof(float) * (size_t)V))) return rc;
  // sampled-decode state, allocated up front: w4h_session_cancel writes its stop word from any thread
  if ((rc = s->samp.alloc(sizeof(SampleDev)))) return rc;
  HIPCHK(hipMemsetAsync(s->samp.p, 0, sizeof(SampleDev), s->stream));
  HIPCHK(hipStreamCreateWithFlags(&s->ctl, hipStreamNonBlocking));
  HIPCHK(hipStreamSynchronize(s->stream));
  m->refs.fetch_add(1);
  *out = s.release();
  return W4H_OK;
}

}  // namespace w4h

extern "C" {

int w4h_session_create(w4h_model* m, const w4h_session_desc* desc, w4h_session** out) {
  if (!m || !desc || !out) return fail(W4H_ERR_INVALID, "null argument");
  *out = nullptr;
  if (m->closed) return fail(W4H_ERR_CLOSED, "model destroyed");
  const w4h_dims& D = m->dims;
  if (desc->n_rows < 1 || desc->n_rows > kWideMaxRows)
    return fail(W4H_ERR_INVALID, "n_rows %d outside [1, %d]", desc->n_rows, kWideMaxRows);
  if (desc->n_encoders != 1 && desc->n_encoders != desc->n_rows)
    return fail(W4H_ERR_INVALID, "n_encoders must be 1 or n_rows");
  if (desc->max_ctx < 1 || desc->max_ctx > 8192) return fail(W4H_ERR_INVALID, "max_ctx %d outside [1, 8192]", desc->max_ctx);
  int rc = set_device(m->device);
  if (rc) return rc;
  auto s = std::make_unique<w4h_session>();
  s->m = m;
  s->S = desc->n_rows;
  s->X = desc->n_encoders;
  s->max_ctx = desc->max_ctx;
  const int L = D.n_text_layer, d = D.n_text_state, H = D.n_text_head, A = D.n_audio_ctx, V = D.n_vocab;
  s->ncs_max = (s->max_ctx + kSelfChunk - 1) / kSelfChunk + 1;  // cached-key chunks + the current key
  s->ncc = (A + kMaxChunk - 1) / kMaxChunk;
  s->chc = (A + s->ncc - 1) / s->ncc;
  s->mw = (V + 31) / 32;
  hipDeviceProp_t prop;
  HIPCHK(hipGetDeviceProperties(&prop, m->device));
  s->grid = prop.multiProcessorCount;
  // Engine: the persistent step kernel for few rows, the batched MFMA engine for more (measured on
  // MI355X: the batched engine is faster from 5 rows at d = 512 and from 3 rows at d = 768; the
  // persistent kernel holds at most kMaxRows).  W4H_ENGINE=wide or persistent overrides where both
  // apply.
  s->wide = s->S > kMaxRows || s->S >= 5 || (s->S >= 3 && d >= 768);
  if (const char* e = getenv("W4H_ENGINE")) {
    if (!strcmp(e, "wide")) s->wide = true;
    else if (!strcmp(e, "persistent") && s->S <= kMaxRows) s->wide = false;
  }
  if (s->wide) return create_wide(s, prop, out);
  // Phase groups (1, 2 or 4; see phase_group in the kernels); W4H_NGROUPS overrides the default below
  // for tuning.  A workgroup owns at most kResItems of the d/8 residual-row items.
  // One row with at most 4 MLP1 items per quarter workgroup (d <= 512 on 256 CUs): quarters.
  if (s->S == 1 && d / 2 <= s->grid) s->ngroups = 4;
  if (const char* e = getenv("W4H_NGROUPS")) {
    const int v = atoi(e);
    if (v == 1 || v == 2 || v == 4) s->ngroups = v;
  }
  while (s->ngroups > 1 && (s->grid < 2 * s->ngroups ||
                            (d / 8 + s->grid / s->ngroups - 1) / (s->grid / s->ngroups) > kResItems))
    s->ngroups /= 2;
  if ((d / 8 + s->grid - 1) / s->grid > kResItems)
    return fail(W4H_ERR_INVALID, "n_text_state %d needs more than %d compute units", d, d / (8 * kResItems));
  s->rpw = (((V + 7) / 8 + s->grid - 1) / s->grid) * 8;
  const size_t kv_elems = (size_t)L * s->S * H * s->max_ctx * kHeadDim;
  {
    // The step kernel reads its weights, self-KV and cross-KV through buffer resources with 32-bit
    // byte offsets, so each of those arrays must stay below 2 GiB.
    const size_t lim = 0x7fffffffu, xb = (size_t)s->X * L * H * A * kHeadDim * 2;
    const size_t wb = std::max((size_t)V * d, (size_t)4 * d * d) * 2;
    if (kv_elems * 2 > lim || xb > lim || wb > lim)
      return fail(W4H_ERR_INVALID,
                  "self-KV (%zu bytes), cross-KV (%zu bytes) or a weight matrix (%zu bytes) exceeds the step kernel's 2 GiB "
                  "addressing; use fewer rows or a smaller max_ctx",
                  kv_elems * 2, xb, wb);
  }
  StepParams probe_p{};
  probe_p.S = s->S;
  probe_p.d = d;
  probe_p.H = H;
  probe_p.wq8 = m->wq8;  // the one-row layout depends on the weight type
  probe_p.ncs_max = s->ncs_max;
  probe_p.ncc = s->ncc;
  probe_p.rows_per_wg = s->rpw;
  s->lds = step_lds_bytes(probe_p, s->grid);
  // One-row sessions keep the first vocabulary items of each workgroup's logits share resident in
  // the LDS left over by the step (step_rounds 16-byte chunks per thread and item, plus q8_0 scales).
  s->res_off = (s->lds + 15) & ~(size_t)15;
  if (s->S == 1) {
    const int dr = step_rounds(d, m->wq8);
    const size_t item_bytes = (size_t)dr * kThreads * 16 + (m->wq8 ? (size_t)dr * kThreads * 2 : 0);
    s->item_bytes = item_bytes;
    const size_t limit = (size_t)prop.sharedMemPerBlock;
    const size_t avail = limit > s->res_off + 1024 ? limit - s->res_off - 1024 : 0;
    const int nmine = ((V + 7) / 8 + s->grid - 1) / s->grid;
    // resident rows hold only the register rounds, so rows longer than those rounds are streamed
    const bool rows_fit = d <= (m->wq8 ? 512 : 256) * dr;
    s->nres = rows_fit ? (int)std::min<size_t>((size_t)nmine, avail / item_bytes) : 0;
    if (const char* e = getenv("W4H_NRES")) s->nres = std::max(0, std::min(s->nres, atoi(e)));
    s->lds = s->res_off + (size_t)s->nres * item_bytes;
  }
  if (s->lds > (size_t)prop.sharedMemPerBlock)
    return fail(W4H_ERR_INVALID, "n_rows %d x n_text_state %d needs %zu bytes of LDS per workgroup (max %zu)", s->S, d, s->lds,
                (size_t)prop.sharedMemPerBlock);
  if ((rc = s->kvk.alloc(kv_elems * 2)) || (rc = s->kvv.alloc(kv_elems * 2))) return rc;
  const size_t x_elems = (size_t)s->X * L * H * A * kHeadDim;
  if ((rc = s->xk.alloc(x_elems * 2)) || (rc = s->xv.alloc(x_elems * 2))) return rc;
  HIPCHK(hipStreamCreate(&s->stream));
  HIPCHK(hipMemsetAsync(s->xk.p, 0, x_elems * 2, s->stream));
  HIPCHK(hipMemsetAsync(s->xv.p, 0, x_elems * 2, s->stream));
  s->slots_host.resize((size_t)s->S * s->max_ctx);
  for (int r = 0; r < s->S; r++)
    for (int q = 0; q < s->max_ctx; q++) s->slots_host[(size_t)r * s->max_ctx + q] = r;
  if ((rc = init_inputs(s.get()))) return rc;
  // tagged exchange buffers, one allocation
  const size_t n_qkv = (size_t)L * s->S * 3 * d, n_sp = (size_t)L * s->ncs_max * s->S * H * kPartWords,
               n_vec = (size_t)L * s->S * d, n_cp = (size_t)L * s->ncc * s->S * H * kPartWords, n_hm = (size_t)L * s->S * 4 * d,
               n_lp = (size_t)s->grid * s->S * kSelWords, n_lpa = (size_t)s->grid * s->S * 2;
  const size_t total = n_qkv + n_sp + 4 * n_vec + n_cp + n_hm + n_lp + n_lpa;
  s->rep_stride = total;  // kRep replicas of the whole set, consecutive
  if ((rc = s->ll.alloc(total * kRep * sizeof(u64)))) return rc;
  u64* b = s->ll.as<u64>();
  s->qkv = b; b += n_qkv;
  s->sp = b; b += n_sp;
  s->x1 = b; b += n_vec;
  s->cq = b; b += n_vec;
  s->cp = b; b += n_cp;
  s->x2 = b; b += n_vec;
  s->hm = b; b += n_hm;
  s->x3 = b; b += n_vec;
  s->lp = b; b += n_lp;
  s->lpa = b;
  HIPCHK(launch_fill_u64(s->ll.as<u64>(), total * kRep, s->stream));
  if ((rc = s->mask.alloc(sizeof(uint32_t) * (size_t)s->S * s->mw))) return rc;
  if ((rc = s->bias.alloc(sizeof(float) * (size_t)V))) return rc;
  // sampled-decode state, allocated up front: w4h_session_cancel writes its stop word from any thread
  if ((rc = s->samp.alloc(sizeof(SampleDev)))) return rc;
  HIPCHK(hipMemsetAsync(s->samp.p, 0, sizeof(SampleDev), s->stream));
  HIPCHK(hipStreamCreateWithFlags(&s->ctl, hipStreamNonBlocking));
  HIPCHK(hipStreamSynchronize(s->stream));
  m->refs.fetch_add(1);
  *out = s.release();
  return W4H_OK;
}

int w4h_session_destroy(w4h_session* s) {
  if (!s) return fail(W4H_ERR_INVALID, "null argument");
  w4h_model* m = s->m;
  (void)hipSetDevice(m->device);
  if (s->stream) {
    (void)hipStreamSynchronize(s->stream);
    wide_graph_release(&s->wgraph);
    wide_graph_release(&s->wgraph_beam);
    (void)hipStreamDestroy(s->stream);
  }
  if (s->ctl) (void)hipStreamDestroy(s->ctl);
  delete s;
  model_release(m);
  return W4H_OK;
}

int w4h_session_cancel(w4h_session* s, int32_t on) {
  if (!s) return fail(W4H_ERR_INVALID, "null argument");
  std::lock_guard<std::mutex> lk(s->cancel_mu);
  HIPCHK(hipSetDevice(s->m->device));
  s->cancel.store(on ? 1 : 0);
  // The device words are written by the command processor of the control stream's queue (a stream
  // write, no copy kernel), so the write lands while the persistent kernel holds every compute unit:
  // the cancel word (read by the step kernel's waits and, with decode rules, once per step), and a
  // sampled decode's stop word, which makes every later launch of its chain return at once.
  HIPCHK(hipStreamWriteValue32(s->ctl, s->in.p, on ? 1u : 0u, 0));
  if (on && !s->wide) HIPCHK(hipStreamWriteValue32(s->ctl, &s->samp.as<SampleDev>()->stop, 1u, 0));
  HIPCHK(hipStreamSynchronize(s->ctl));
  return W4H_OK;
}

static int project_encoder(w4h_session* s, int32_t enc, const float* xa_dev) {
  const w4h_dims& D = s->m->dims;
  const size_t off = (size_t)enc * D.n_text_layer * D.n_text_head * D.n_audio_ctx * kHeadDim;
  const size_t sb = cross_kv_scratch_bytes(D.n_audio_ctx, D.n_text_state);
  void* scratch = nullptr;
  if (sb && !getenv("W4H_XKV_LAYERWISE")) {  // W4H_XKV_LAYERWISE: one GEMM per layer instead (comparison)
    const int rc = ensure(s->xa_hl, sb);
    if (rc) return rc;
    scratch = s->xa_hl.p;
  }
  // the transposed V copy exists only for one shared encoder (enc 0)
  HIPCHK(launch_cross_kv(s->m->layers_dev.as<LayerDev>(), D.n_text_layer, D.n_text_state, D.n_text_head, D.n_audio_ctx,
                         s->m->wq8, xa_dev, s->xk.as<uint16_t>() + off, s->xv.as<uint16_t>() + off,
                         s->xvt.p ? s->xvt.as<uint16_t>() : nullptr, s->Ap, scratch, s->stream));
  HIPCHK(hipStreamSynchronize(s->stream));
  return W4H_OK;
}

int w4h_session_set_encoder(w4h_session* s, int32_t enc, const float* xa) {
  if (!s || !xa) return fail(W4H_ERR_INVALID, "null argument");
  if (enc < 0 || enc >= s->X) return fail(W4H_ERR_INVALID, "encoder %d outside [0, %d)", enc, s->X);
  const w4h_dims& D = s->m->dims;
  HIPCHK(hipSetDevice(s->m->device));
  const size_t n = (size_t)D.n_audio_ctx * D.n_text_state;
  int rc = ensure(s->xa_tmp, n * sizeof(float));
  if (rc) return rc;
  HIPCHK(hipMemcpyAsync(s->xa_tmp.p, xa, n * sizeof(float), hipMemcpyHostToDevice, s->stream));
  return project_encoder(s, enc, s->xa_tmp.as<float>());
}

int w4h_session_set_encoder_device(w4h_session* s, int32_t enc, const float* xa_device) {
  if (!s || !xa_device) return fail(W4H_ERR_INVALID, "null argument");
  if (enc < 0 || enc >= s->X) return fail(W4H_ERR_INVALID, "encoder %d outside [0, %d)", enc, s->X);
  HIPCHK(hipSetDevice(s->m->device));
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, xa_device) != hipSuccess || attr.type != hipMemoryTypeDevice ||
      attr.device != s->m->device) {
    (void)hipGetLastError();
    return fail(W4H_ERR_INVALID, "xa_device is not device memory of device %d", s->m->device);
  }
  if (reinterpret_cast<uintptr_t>(xa_device) % 16 != 0) return fail(W4H_ERR_INVALID, "xa_device is not 16-byte aligned");
  return project_encoder(s, enc, xa_device);
}

int w4h_session_reset(w4h_session* s, int32_t kv_len) {
  if (!s) return fail(W4H_ERR_INVALID, "null argument");
  if (kv_len < 0 || kv_len > s->kv_len) return fail(W4H_ERR_INVALID, "kv_len %d outside [0, %d]", kv_len, s->kv_len);
  s->kv_len = kv_len;
  if (kv_len == 0 && !s->slots_identity) {
    for (int r = 0; r < s->S; r++)
      for (int q = 0; q < s->max_ctx; q++) s->slots_host[(size_t)r * s->max_ctx + q] = r;
    s->slots_identity = true;
    s->slots_dirty = true;
  }
  return W4H_OK;
}

int w4h_session_kv_len(const w4h_session* s, int32_t* kv_len) {
  if (!s || !kv_len) return fail(W4H_ERR_INVALID, "null argument");
  *kv_len = s->kv_len;
  return W4H_OK;
}

int w4h_session_set_suppress(w4h_session* s, const int32_t* ids, int32_t n) {
  if (!s || (n > 0 && !ids)) return fail(W4H_ERR_INVALID, "null argument");
  std::vector<uint32_t> bits((size_t)s->S * s->mw, 0u);
  const int V = s->m->dims.n_vocab;
  for (int i = 0; i < n; i++)
    if (ids[i] >= 0 && ids[i] < V)
      for (int r = 0; r < s->S; r++) bits[(size_t)r * s->mw + (ids[i] >> 5)] |= 1u << (ids[i] & 31);
  HIPCHK(hipSetDevice(s->m->device));
  HIPCHK(hipMemcpy(s->mask.p, bits.data(), bits.size() * 4, hipMemcpyHostToDevice));
  s->has_mask = n > 0;
  return W4H_OK;
}

int w4h_session_set_logit_bias(w4h_session* s, const float* bias) {
  if (!s) return fail(W4H_ERR_INVALID, "null argument");
  if (!bias) {
    s->bias_on = false;
    return W4H_OK;
  }
  HIPCHK(hipSetDevice(s->m->device));
  HIPCHK(hipMemcpy(s->bias.p, bias, sizeof(float) * (size_t)s->m->dims.n_vocab, hipMemcpyHostToDevice));
  s->bias_on = true;
  return W4H_OK;
}

int w4h_session_set_probe(w4h_session* s, int32_t token) {
  if (!s) return fail(W4H_ERR_INVALID, "null argument");
  s->probe = (token >= 0 && token < s->m->dims.n_vocab) ? token : -1;
  return W4H_OK;
}

int w4h_session_step(w4h_session* s, const int32_t* tokens, const uint32_t* extra_mask, int32_t topk, w4h_step_out* out,
                     float* logits) {
  if (!s) return fail(W4H_ERR_INVALID, "null argument");
  return run_steps(s, tokens, nullptr, 1, extra_mask, topk, out, logits, nullptr);
}

int w4h_session_run(w4h_session* s, const int32_t* tokens, const int32_t* forced, int32_t n_steps, int32_t topk,
                    w4h_step_out* out) {
  if (!s) return fail(W4H_ERR_INVALID, "null argument");
  return run_steps(s, tokens, forced, n_steps, nullptr, topk, out, nullptr, nullptr);
}

int w4h_session_reorder(w4h_session* s, const int32_t* parent) {
  if (!s || !parent) return fail(W4H_ERR_INVALID, "null argument");
  for (int r = 0; r < s->S; r++)
    if (parent[r] < 0 || parent[r] >= s->S) return fail(W4H_ERR_INVALID, "parent[%d]=%d outside [0, %d)", r, parent[r], s->S);
  std::vector<int32_t> old(s->slots_host);
  for (int r = 0; r < s->S; r++)
    memcpy(&s->slots_host[(size_t)r * s->max_ctx], &old[(size_t)parent[r] * s->max_ctx], sizeof(int32_t) * s->kv_len);
  bool ident = true;
  for (int r = 0; r < s->S && ident; r++)
    for (int q = 0; q < s->kv_len; q++)
      if (s->slots_host[(size_t)r * s->max_ctx + q] != r) {
        ident = false;
        break;
      }
  s->slots_identity = ident;
  s->slots_dirty = true;
  return W4H_OK;
}

int w4h_session_time_run(w4h_session* s, const int32_t* tokens, const int32_t* forced, int32_t n_steps, int32_t n_repeats,
                         float* ms_out, w4h_step_out* out) {
  if (!s || !ms_out || n_repeats < 1) return fail(W4H_ERR_INVALID, "bad argument");
  const int kv0 = s->kv_len;
  for (int r = 0; r < n_repeats; r++) {
    s->kv_len = kv0;
    int rc = run_steps(s, tokens, forced, n_steps, nullptr, 0, r + 1 == n_repeats ? out : nullptr, nullptr, &ms_out[r]);
    if (rc) {
      s->kv_len = kv0;
      return rc;
    }
  }
  s->kv_len = kv0;
  return W4H_OK;
}

int w4h_session_trace_run(w4h_session* s, const int32_t* tokens, const int32_t* forced, int32_t n_steps, uint64_t* trace,
                          int64_t trace_len, int32_t* n_workgroups) {
  if (!s || !trace || !n_workgroups) return fail(W4H_ERR_INVALID, "null argument");
  const int64_t need = (int64_t)n_steps * (6 * s->m->dims.n_text_layer + 2) * 4 * s->grid;
  *n_workgroups = s->grid;
  if (trace_len < need) return fail(W4H_ERR_INVALID, "trace needs %lld entries", (long long)need);
  const int kv0 = s->kv_len;
  int rc = run_steps(s, tokens, forced, n_steps, nullptr, 0, nullptr, nullptr, nullptr, trace);
  s->kv_len = kv0;
  return rc;
}

// ---------------------------------------------------------------------------------------------
// kernel-level entry points

static int op_prepare() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(W4H_ERR_DEVICE, "no HIP device available");
  return W4H_OK;
}

int w4h_op_linear(const void* w, int32_t w_type, int32_t n, int32_t k, const float* bias, const float* x, int32_t m,
                  float* y) {
  if (!w || !x || !y || n <= 0 || k <= 0 || m <= 0 || m > kMaxRows) return fail(W4H_ERR_INVALID, "bad argument");
  if (k % 32) return fail(W4H_ERR_SHAPE, "k must be a multiple of 32");
  if (w_type != W4H_TYPE_F16 && w_type != W4H_TYPE_Q8_0) return fail(W4H_ERR_INVALID, "w_type must be f16 or q8_0");
  int rc = op_prepare();
  if (rc) return rc;
  DevBuf dw, ds, db, dx, dy;
  if (w_type == W4H_TYPE_F16) {
    if ((rc = upload(dw, w, (size_t)n * k * 2))) return rc;
  } else {
    std::vector<int8_t> q((size_t)n * k);
    std::vector<uint16_t> sc((size_t)n * (k / 32));
    const unsigned char* src = static_cast<const unsigned char*>(w);
    for (int r = 0; r < n; r++)
      for (int b = 0; b < k / 32; b++) {
        const unsigned char* blk = src + ((size_t)r * (k / 32) + b) * 34;
        sc[(size_t)r * (k / 32) + b] = (uint16_t)(blk[0] | (blk[1] << 8));
        memcpy(q.data() + (size_t)r * k + b * 32, blk + 2, 32);
      }
    if ((rc = upload(dw, q.data(), q.size())) || (rc = upload(ds, sc.data(), sc.size() * 2))) return rc;
  }
  if (bias && (rc = upload(db, bias, (size_t)n * 4))) return rc;
  if ((rc = upload(dx, x, (size_t)m * k * 4)) || (rc = dy.alloc((size_t)m * n * 4))) return rc;
  HIPCHK(launch_op_linear(dw.p, ds.as<uint16_t>(), w_type == W4H_TYPE_Q8_0, n, k, bias ? db.as<float>() : nullptr,
                          dx.as<float>(), m, dy.as<float>(), nullptr));
  HIPCHK(hipMemcpy(y, dy.p, (size_t)m * n * 4, hipMemcpyDeviceToHost));
  return W4H_OK;
}

int w4h_op_layernorm(const float* x, int32_t rows, int32_t n, const float* gamma, const float* beta, float* y) {
  if (!x || !gamma || !beta || !y || rows <= 0 || n <= 0) return fail(W4H_ERR_INVALID, "bad argument");
  int rc = op_prepare();
  if (rc) return rc;
  DevBuf dx, dg, dbt, dy;
  if ((rc = upload(dx, x, (size_t)rows * n * 4)) || (rc = upload(dg, gamma, (size_t)n * 4)) ||
      (rc = upload(dbt, beta, (size_t)n * 4)) || (rc = dy.alloc((size_t)rows * n * 4)))
    return rc;
  HIPCHK(launch_op_layernorm(dx.as<float>(), rows, n, dg.as<float>(), dbt.as<float>(), dy.as<float>(), nullptr));
  HIPCHK(hipMemcpy(y, dy.p, (size_t)rows * n * 4, hipMemcpyDeviceToHost));
  return W4H_OK;
}

int w4h_op_gelu(const float* x, int32_t n, float* y) {
  if (!x || !y || n <= 0) return fail(W4H_ERR_INVALID, "bad argument");
  int rc = op_prepare();
  if (rc) return rc;
  DevBuf dx, dy;
  if ((rc = upload(dx, x, (size_t)n * 4)) || (rc = dy.alloc((size_t)n * 4))) return rc;
  HIPCHK(launch_op_gelu(dx.as<float>(), n, dy.as<float>(), nullptr));
  HIPCHK(hipMemcpy(y, dy.p, (size_t)n * 4, hipMemcpyDeviceToHost));
  return W4H_OK;
}

int w4h_op_attention(const float* q, const uint16_t* k, const uint16_t* v, int32_t n_heads, int32_t kv_len, float scale,
                     float* out) {
  if (!q || !k || !v || !out || n_heads <= 0 || kv_len <= 0 || kv_len > 8192) return fail(W4H_ERR_INVALID, "bad argument");
  int rc = op_prepare();
  if (rc) return rc;
  DevBuf dq, dk, dv, dout;
  const size_t kvn = (size_t)n_heads * kv_len * kHeadDim;
  if ((rc = upload(dq, q, (size_t)n_heads * kHeadDim * 4)) || (rc = upload(dk, k, kvn * 2)) || (rc = upload(dv, v, kvn * 2)) ||
      (rc = dout.alloc((size_t)n_heads * kHeadDim * 4)))
    return rc;
  HIPCHK(launch_op_attention(dq.as<float>(), dk.as<uint16_t>(), dv.as<uint16_t>(), n_heads, kv_len, scale, dout.as<float>(), nullptr));
  HIPCHK(hipMemcpy(out, dout.p, (size_t)n_heads * kHeadDim * 4, hipMemcpyDeviceToHost));
  return W4H_OK;
}

int w4h_op_select(const float* logits, int32_t rows, int32_t n, const uint32_t* mask, int32_t k, w4h_step_out* out) {
  if (!logits || !out || rows <= 0 || n <= 0 || k < 0 || k > W4H_TOPK_MAX) return fail(W4H_ERR_INVALID, "bad argument");
  int rc = op_prepare();
  if (rc) return rc;
  DevBuf dl, dm, dout;
  const size_t mw = (size_t)(n + 31) / 32;
  if ((rc = upload(dl, logits, (size_t)rows * n * 4))) return rc;
  if (mask && (rc = upload(dm, mask, (size_t)rows * mw * 4))) return rc;
  if ((rc = dout.alloc(sizeof(w4h_step_out) * rows))) return rc;
  HIPCHK(launch_op_select(dl.as<float>(), rows, n, mask ? dm.as<uint32_t>() : nullptr, k, dout.as<w4h_step_out>(), nullptr));
  HIPCHK(hipMemcpy(out, dout.p, sizeof(w4h_step_out) * rows, hipMemcpyDeviceToHost));
  return W4H_OK;
}

int w4h_op_sample(const float* logits, int32_t n, const uint32_t* suppress_mask, const int32_t* history,
                  int32_t n_history, int32_t eot, int32_t timestamp_begin, float temperature, uint64_t rng_state,
                  int32_t* token, double* logprob) {
  if (!logits || !token || !logprob || n <= 0 || n > kSampleMaxV || n_history < 0 || n_history >= kSampleHist ||
      (n_history > 0 && !history) || !(temperature > 0.0f))
    return fail(W4H_ERR_INVALID, "bad argument");
  int rc = op_prepare();
  if (rc) return rc;
  DevBuf dl, dm, dst;
  std::vector<char> hb(sizeof(SampleDev), 0);
  SampleDev* h = reinterpret_cast<SampleDev*>(hb.data());
  h->n = n_history;
  if (n_history > 0) std::copy(history, history + n_history, h->hist);
  if ((rc = upload(dl, logits, (size_t)n * 4))) return rc;
  if (suppress_mask && (rc = upload(dm, suppress_mask, (size_t)(n + 31) / 32 * 4))) return rc;
  if ((rc = upload(dst, hb.data(), hb.size()))) return rc;
  SampleParams sp{};
  sp.logits = dl.as<float>();
  sp.sup = suppress_mask ? dm.as<uint32_t>() : nullptr;
  sp.V = n;
  sp.eot = eot;
  sp.tsb = timestamp_begin > 0 ? timestamp_begin : 0;
  sp.rows = 1;
  sp.max_steps = 1;
  sp.temperature = temperature;
  sp.rng = rng_state;
  sp.st = dst.as<SampleDev>();
  sp.parts_out = sp.st->parts;
  sp.parts = sp.st->parts;
  sp.nparts = kSampleBlocks;
  sp.part_stride = 1;
  HIPCHK(launch_sample_mask(sp, nullptr));
  HIPCHK(launch_sample(sp, nullptr));
  HIPCHK(hipMemcpy(hb.data(), dst.p, hb.size(), hipMemcpyDeviceToHost));
  if (h->steps != 1) return fail(W4H_ERR_DEVICE, "sampling kernel did not run");
  *token = h->out_tok[0];
  *logprob = h->lp[0];
  return W4H_OK;
}

int w4h_op_select_noalloc(const float* logits, int32_t rows, int32_t n, const uint32_t* mask, int32_t k,
                          w4h_step_out* out, void* stream) {
  if (!logits || !out || rows <= 0 || n <= 0 || k < 0 || k > W4H_TOPK_MAX) return fail(W4H_ERR_INVALID, "bad argument");
  if (rows > W4H_SELECT_MAX_ROWS)
    return fail(W4H_ERR_INVALID, "rows %d exceeds the fixed selection scratch of %d rows", rows, W4H_SELECT_MAX_ROWS);
  if (select_lds_bytes(n) > (size_t)kSelectMaxLds) return fail(W4H_ERR_INVALID, "row length %d too long", n);
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  float* scratch = nullptr;
  HIPCHK(select_scratch(dev, &scratch));
  HIPCHK(launch_op_select_noalloc(logits, rows, n, mask, k, out, scratch, static_cast<hipStream_t>(stream)));
  return W4H_OK;
}

}  // extern "C"

namespace w4h {
int session_rows(const w4h_session* s) { return s->S; }
bool session_device_beam(const w4h_session* s) { return s->wide && s->S <= kBeamMax; }

bool session_device_rules(const w4h_session* s) {
  if (s->wide || s->S != 1) return false;
  if (const char* e = getenv("W4H_DEVICE_RULES"))
    if (!strcmp(e, "0")) return false;
  StepParams p{};  // room for the longest history a decode can reach
  return rules_layout(s, kMaxDecodeTokens + s->max_ctx, p) != 0;
}

int session_max_ctx(const w4h_session* s) { return s->max_ctx; }

int device_greedy_run(w4h_session* s, const RulesRun& r, int n_steps, const uint32_t* mask2, w4h_step_out* out,
                      int* steps_done) {
  if (!session_device_rules(s)) return fail(W4H_ERR_INVALID, "device decode rules need a one-row persistent session");
  if (r.nhist < 1 || !r.hist) return fail(W4H_ERR_INVALID, "device decode rules need the generated tokens");
  const int32_t tok = r.hist[r.nhist - 1];
  return run_steps(s, &tok, nullptr, n_steps, mask2, 1, out, nullptr, nullptr, nullptr, &r, steps_done);
}

// Sampled runs with the draw inside the step kernel (one launch per run) instead of a chain of one-step
// launches and sampling kernels: one-row persistent sessions.  W4H_SAMPLE_IN_LAUNCH=0 selects the chain;
// =2 takes the in-launch path without the eligibility checks, so that a session it does not fit fails
// (run_steps) instead of falling back (tests).
static bool sample_in_launch(const w4h_session* s) {
  if (const char* e = getenv("W4H_SAMPLE_IN_LAUNCH")) {
    if (!strcmp(e, "0")) return false;
    if (!strcmp(e, "2")) return true;
  }
  return session_device_rules(s) && s->grid <= kThreads &&
         (size_t)s->m->dims.n_vocab <= (size_t)s->grid * kThreads * kSampEpt && sample_scratch_fits(s);
}

bool session_device_sample(const w4h_session* s) {
  if (s->wide || s->S > kMaxRows || s->m->dims.n_vocab > kSampleMaxV) return false;
  if (const char* e = getenv("W4H_DEVICE_SAMPLE"))
    if (!strcmp(e, "0")) return false;
  return true;
}

// Sampled decode steps chained on the session stream: per step one launch of the step kernel (one
// step, raw logits of every row into samp_row), one of the masking kernel (the rules applied to row
// 0 in place) and one of the sampling kernel, which draws the token and leaves it as every row's
// next input.  After the end token
// the sampler sets the stop word and the remaining launches of the run return at once.  The host
// synchronises once per run.
int device_sampled_run(w4h_session* s, const SampleRun& r, int n_steps, const uint32_t* sup, SampleRunOut* out) {
  if (!session_device_sample(s)) return fail(W4H_ERR_INVALID, "device sampling needs a persistent session");
  if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled");
  if (r.nhist < 1 || !r.hist || r.nhist >= kSampleHist) return fail(W4H_ERR_INVALID, "device sampling needs the generated tokens");
  if (!(r.temperature > 0.0f)) return fail(W4H_ERR_INVALID, "device sampling needs a temperature above 0");
  if (n_steps < 1 || n_steps > kSampleHist) return fail(W4H_ERR_INVALID, "n_steps outside [1, %d]", kSampleHist);
  if (s->kv_len + n_steps > s->max_ctx)
    return fail(W4H_ERR_CAPACITY, "self-KV capacity %d exceeded (kv_len %d + %d steps)", s->max_ctx, s->kv_len, n_steps);
  if ((uint64_t)s->next_tag + (uint64_t)n_steps >= 0xfffffff0ull) return fail(W4H_ERR_INVALID, "tag space exhausted; recreate the session");
  const int V = s->m->dims.n_vocab;
  int rc;
  if (sample_in_launch(s)) {
    // The step kernel draws each token itself (phase_sample), kSampleLaunch steps per launch: between
    // launches the host sees a cancel (the device cancel word is a stream write, which waits while a
    // launch holds the queue it shares) at a cost of two launch gaps per kSampleLaunch tokens.  Each
    // launch continues the history and the generator (draw i of a launch after `done` draws is draw
    // done + i + 1 of the run: the state advances by done steps).
    constexpr int kSampleLaunch = 64;
    std::vector<int32_t> hist(r.hist, r.hist + r.nhist);
    std::vector<w4h_step_out> recs((size_t)std::min(kSampleLaunch, n_steps));
    out->steps = 0;
    out->ended = false;
    out->tokens.clear();
    out->lps.clear();
    while (out->steps < n_steps) {
      const int nc = std::min(kSampleLaunch, n_steps - out->steps);
      const RulesRun rr{hist.data(), (int)hist.size(), r.eot, r.tsb};
      SampleRun rc_run = r;
      rc_run.hist = hist.data();
      rc_run.nhist = (int)hist.size();
      rc_run.rng = r.rng + (uint64_t)out->steps * 0x9e3779b97f4a7c15ull;
      SampleRunOut so;
      int done = 0;
      const int32_t tok = hist.back();
      if ((rc = run_steps(s, &tok, nullptr, nc, sup, 0, recs.data(), nullptr, nullptr, nullptr, &rr, &done, &rc_run, &so)))
        return rc;
      out->steps += so.steps;
      out->tokens.insert(out->tokens.end(), so.tokens.begin(), so.tokens.end());
      out->lps.insert(out->lps.end(), so.lps.begin(), so.lps.end());
      if (so.ended) {
        out->ended = true;
        break;
      }
      hist.insert(hist.end(), so.tokens.begin(), so.tokens.end());
      if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled");
    }
    return W4H_OK;
  }
  HIPCHK(hipSetDevice(s->m->device));
  if ((rc = ensure(s->samp_row, sizeof(float) * (size_t)s->S * V)) || (rc = ensure(s->samp_sup, sizeof(uint32_t) * (size_t)s->mw)))
    return rc;
  std::vector<char> hb(sizeof(SampleDev), 0);
  SampleDev* h = reinterpret_cast<SampleDev*>(hb.data());
  h->n = r.nhist;
  std::copy(r.hist, r.hist + r.nhist, h->hist);
  for (int q = 0; q < s->S; q++) h->tok[q] = r.hist[r.nhist - 1];
  // error word (and the slot table, when a reorder changed it) as run_steps stages them
  char* hp = static_cast<char*>(s->h_in.p);
  *reinterpret_cast<unsigned*>(hp + kErrOff) = 0u;
  if (s->slots_dirty) memcpy(hp + s->o_slots, s->slots_host.data(), sizeof(int32_t) * s->slots_host.size());
  HIPCHK(hipMemcpyAsync(s->in_at<char>(kErrOff), hp + kErrOff, (s->slots_dirty ? s->in_bytes : kErrOff + sizeof(unsigned)) - kErrOff,
                        hipMemcpyHostToDevice, s->stream));
  s->slots_dirty = false;
  HIPCHK(hipMemcpyAsync(s->samp.p, hb.data(), offsetof(SampleDev, out_tok), hipMemcpyHostToDevice, s->stream));
  if (sup) HIPCHK(hipMemcpyAsync(s->samp_sup.p, sup, sizeof(uint32_t) * (size_t)s->mw, hipMemcpyHostToDevice, s->stream));
  // the state is in place before the chain starts, so a cancel's stop word cannot be overwritten by it
  HIPCHK(hipStreamSynchronize(s->stream));
  if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled");
  SampleDev* dst = s->samp.as<SampleDev>();
  SampleParams sp{};
  sp.logits = s->samp_row.as<float>();
  sp.sup = sup ? s->samp_sup.as<uint32_t>() : nullptr;
  sp.V = V;
  sp.eot = r.eot;
  sp.tsb = r.tsb;
  sp.rows = s->S;
  sp.max_steps = n_steps;
  sp.temperature = r.temperature;
  sp.rng = r.rng;
  sp.st = dst;
  sp.parts_out = dst->parts;
  sp.parts = dst->parts;
  sp.nparts = kSampleBlocks;
  sp.part_stride = 1;
  StepParams p = base_params(s);
  p.nsteps = 1;
  p.tokens0 = dst->tok;
  p.mask = nullptr;  // the sampler applies every mask to the raw row itself
  p.topk = 0;
  p.out = nullptr;
  p.logits_out = sp.logits;
  p.nres = 0;  // one step per launch: loading resident vocabulary rows would not pay
  p.stop = &dst->stop;
  {
    // Enqueued kSampleChunk steps at a time; between chunks the host reads the stop word (end token,
    // last step or cancel), so a decode that ends early leaves no launches to drain.
    constexpr int kSampleChunk = 32;
    std::unique_lock<std::mutex> coop(coop_lock(s->m->device));
    int i = 0;
    while (i < n_steps) {
      const int nc = std::min(kSampleChunk, n_steps - i);
      for (int j = 0; j < nc; j++, i++) {
        p.kv_len0 = s->kv_len + i;
        p.tag0 = s->next_tag++;
        hipError_t le = launch_step(p, s->grid, s->lds, s->stream);
        if (le != hipSuccess) return fail(W4H_ERR_DEVICE, "decoder step launch failed: %s", hipGetErrorString(le));
        if ((le = launch_sample_mask(sp, s->stream)) != hipSuccess || (le = launch_sample(sp, s->stream)) != hipSuccess)
          return fail(W4H_ERR_DEVICE, "sampling launch failed: %s", hipGetErrorString(le));
      }
      if (i >= n_steps) break;
      int32_t hdr[4];
      HIPCHK(hipMemcpyAsync(hdr, s->samp.p, sizeof(hdr), hipMemcpyDeviceToHost, s->stream));
      HIPCHK(hipStreamSynchronize(s->stream));
      if (hdr[2] || s->cancel.load()) break;  // SampleDev::stop
    }
    HIPCHK(hipMemcpyAsync(hb.data(), s->samp.p, sizeof(SampleDev), hipMemcpyDeviceToHost, s->stream));
    unsigned herr = 0;
    HIPCHK(hipMemcpyAsync(&herr, s->in_at<char>(kErrOff), sizeof(unsigned), hipMemcpyDeviceToHost, s->stream));
    HIPCHK(hipStreamSynchronize(s->stream));
    if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled during the sampled decode");
    if (herr) return fail(W4H_ERR_TIMEOUT, "a device-side wait expired during the step (code %u); step aborted", herr);
  }
  s->kv_len += h->steps;  // one step-kernel launch ran per sampled step
  out->steps = h->steps;
  out->ended = h->steps > 0 && h->out_tok[h->steps - 1] == r.eot;
  out->tokens.assign(h->out_tok, h->out_tok + h->steps);
  out->lps.assign(h->lp, h->lp + h->steps);
  return W4H_OK;
}

int device_beam_search(w4h_session* s, const BeamSearchIn& in, BeamSearchOut* out) {
  if (!s->wide || in.beam != s->S || in.beam > kBeamMax) return fail(W4H_ERR_INVALID, "device beam search needs a batched session");
  if (in.max_steps < 0 || in.max_steps >= kBeamTokMax) return fail(W4H_ERR_INVALID, "max_steps outside [0, %d)", kBeamTokMax);
  const int B = in.beam, V = s->m->dims.n_vocab;
  int rc;
  HIPCHK(hipSetDevice(s->m->device));
  if ((rc = ensure(s->wbeam, sizeof(BeamDev)))) return rc;
  if ((rc = ensure(s->wbsup, sizeof(int32_t) * (size_t)std::max(1, in.n_suppress)))) return rc;
  // initial state: one token per beam, nothing finished
  std::vector<char> hb(sizeof(BeamDev), 0);
  BeamDev* h = reinterpret_cast<BeamDev*>(hb.data());
  for (int b = 0; b < B; b++) {
    h->len[0][b] = 1;
    h->toks[0][b][0] = in.first_tokens[b];
    h->lps[b] = in.first_lps[b];
  }
  HIPCHK(hipMemcpy(s->wbeam.p, hb.data(), sizeof(BeamDev), hipMemcpyHostToDevice));
  if (in.n_suppress > 0)
    HIPCHK(hipMemcpy(s->wbsup.p, in.suppress, sizeof(int32_t) * in.n_suppress, hipMemcpyHostToDevice));
  // first run's inputs (tokens, mask, slot table) through the staging area
  char* hp = static_cast<char*>(s->h_in.p);
  *reinterpret_cast<unsigned*>(hp + kErrOff) = 0u;
  memcpy(hp + s->o_toks, in.first_tokens, sizeof(int32_t) * B);
  memcpy(hp + s->o_mask2, in.first_mask, sizeof(uint32_t) * (size_t)B * s->mw);
  memcpy(hp + s->o_slots, s->slots_host.data(), sizeof(int32_t) * s->slots_host.size());
  HIPCHK(hipMemcpyAsync(s->in_at<char>(kErrOff), hp + kErrOff, s->in_bytes - kErrOff, hipMemcpyHostToDevice, s->stream));
  s->slots_dirty = false;
  constexpr int kChunk = 32;  // steps per launch; the host checks for the end of the search between launches
  if ((rc = ensure(s->out, sizeof(w4h_step_out) * (size_t)kChunk * B))) return rc;
  int remaining = in.max_steps;
  bool first = true;
  while (remaining > 0) {
    // a launch takes at most the steps the self-KV still has room for; the search fails only when it
    // has not ended and no room is left (as the host loop, which checks one step at a time)
    const int n = std::min(std::min(kChunk, remaining), s->max_ctx - s->kv_len);
    if (n <= 0)
      return fail(W4H_ERR_CAPACITY, "self-KV capacity %d exceeded (kv_len %d, %d steps left)", s->max_ctx, s->kv_len, remaining);
    WideParams wp = wide_params(s);
    wp.nsteps = n;
    wp.kv_len0 = s->kv_len;
    wp.tokens0 = s->in_at<int32_t>(s->o_toks);
    wp.forced = nullptr;
    wp.mask2 = s->in_at<uint32_t>(s->o_mask2);
    wp.slots = s->in_at<int32_t>(s->o_slots);
    wp.topk = B + 1;
    wp.out = s->out.as<w4h_step_out>();
    wp.logits_out = nullptr;
    wp.beam_dev = s->wbeam.as<BeamDev>();
    wp.beam_sup = s->wbsup.as<int32_t>();
    wp.beam_nsup = in.n_suppress;
    wp.beam_eot = in.eot;
    wp.beam_tsb = in.timestamp_begin;
    wp.tok_dev = first ? 0 : 1;
    wp.graph = s->use_graph ? &s->wgraph_beam : nullptr;
    hipError_t le = launch_wide(wp, s->stream);
    if (le != hipSuccess) return fail(W4H_ERR_DEVICE, "beam step launch failed: %s", hipGetErrorString(le));
    WideCtl c{};
    HIPCHK(hipMemcpyAsync(&c, s->wctl.p, sizeof(WideCtl), hipMemcpyDeviceToHost, s->stream));
    HIPCHK(hipStreamSynchronize(s->stream));
    s->kv_len += c.i;  // steps that ran (each appended its KV row)
    remaining -= n;
    first = false;
    if (s->cancel.load()) return fail(W4H_ERR_CANCELLED, "session cancelled during the beam search");
    if (c.stop) break;
  }
  // results, and the slot table the device left behind
  HIPCHK(hipMemcpy(hb.data(), s->wbeam.p, sizeof(BeamDev), hipMemcpyDeviceToHost));
  HIPCHK(hipMemcpy(s->slots_host.data(), s->in_at<int32_t>(s->o_slots), sizeof(int32_t) * s->slots_host.size(),
                   hipMemcpyDeviceToHost));
  s->slots_identity = false;
  s->slots_dirty = false;
  out->fin.clear();
  out->fin_lp.clear();
  for (int f = 0; f < h->nfin; f++) {
    out->fin.emplace_back(h->fin_toks[f], h->fin_toks[f] + h->fin_len[f]);
    out->fin_lp.push_back(h->fin_lp[f]);
  }
  out->toks.assign(B, {});
  out->lps.assign(B, 0.0);
  for (int b = 0; b < B; b++) {
    out->toks[b].assign(h->toks[h->cur][b], h->toks[h->cur][b] + h->len[h->cur][b]);
    out->lps[b] = h->lps[b];
  }
  (void)V;
  return W4H_OK;
}
w4h_dims session_dims(const w4h_session* s) { return s->m->dims; }
}  // namespace w4h
