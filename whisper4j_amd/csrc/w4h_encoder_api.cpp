// Host side of the audio encoder (WhisperEncoder, main/nn/WhisperEncoder.java:27-76): weight upload
// and the forward sequence of encoder kernels (w4h_encoder.hip) on one stream.
//
// Device layout: activations [frames][channels] fp32; the conv1 input is the mel [n_mels][frames]
// copied time-major with a zero frame at each end; the conv1 output keeps the same two zero frames
// (rows 0 and 2T + 1 of x1p) so conv2 reads its windows without bounds checks.  Matrices [out][in]
// f16 (or q8_0 as int8 + f16 block scales), conv weights repacked [out][k][in] f16.

#include <hip/hip_runtime_api.h>

#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "w4h_encoder.h"
#include "w4h_host.h"

namespace w4h {
float half_to_float(uint16_t h);
uint16_t float_to_half(float f);
}  // namespace w4h

using namespace w4h;

#define HIPCHK(expr)                                                                                   \
  do {                                                                                                 \
    hipError_t e_ = (expr);                                                                            \
    if (e_ != hipSuccess) return fail(W4H_ERR_DEVICE, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

namespace {

struct Buf {
  void* p = nullptr;
  ~Buf() {
    if (p) (void)hipFree(p);
  }
};

struct EncLayer {
  const void *w_qkv = nullptr, *w_o = nullptr, *w_1 = nullptr, *w_2 = nullptr;
  const uint16_t *s_qkv = nullptr, *s_o = nullptr, *s_1 = nullptr, *s_2 = nullptr;
  const float *b_qkv = nullptr, *b_o = nullptr, *b_1 = nullptr, *b_2 = nullptr;
  const float *ln1_g = nullptr, *ln1_b = nullptr, *ln2_g = nullptr, *ln2_b = nullptr;
};

}  // namespace

struct w4h_encoder {
  int device = 0;
  w4h_encoder_dims dims{};
  int wq8 = 0;
  std::vector<std::unique_ptr<Buf>> bufs;
  const uint16_t *c1w = nullptr, *c2w = nullptr;
  const float *c1b = nullptr, *c2b = nullptr, *pos = nullptr, *lnp_g = nullptr, *lnp_b = nullptr;
  std::vector<EncLayer> layers;
  // working buffers
  float *melt = nullptr, *x1p = nullptr, *x = nullptr;
  // (hi, lo) f16 planes of the layer GEMMs' activation rows, [Mp][n] (rows past T stay zero)
  uint16_t *xnh = nullptr, *xnl = nullptr, *atth = nullptr, *attl = nullptr, *hidh = nullptr, *hidl = nullptr;
  float *mel_in = nullptr, *out = nullptr;  // staging for the host-memory entry point
  uint16_t* qkv = nullptr;
  int Tp = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;  // one forward at a time (the working buffers are shared)
  bool closed = false;
  ~w4h_encoder() {
    if (stream) (void)hipStreamDestroy(stream);
  }
};

namespace {

void* dev_alloc(w4h_encoder* e, size_t bytes, int* rc) {
  e->bufs.push_back(std::make_unique<Buf>());
  void* p = nullptr;
  if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) {
    *rc = fail(W4H_ERR_OOM, "hipMalloc(%zu) failed", bytes);
    return nullptr;
  }
  e->bufs.back()->p = p;
  if (hipMemset(p, 0, bytes ? bytes : 16) != hipSuccess) {
    *rc = fail(W4H_ERR_DEVICE, "hipMemset failed");
    return nullptr;
  }
  *rc = W4H_OK;
  return p;
}

int upload(w4h_encoder* e, const void* src, size_t bytes, void** dst) {
  int rc;
  void* p = dev_alloc(e, bytes, &rc);
  if (!p) return rc;
  HIPCHK(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
  *dst = p;
  return W4H_OK;
}

struct Table {
  std::map<std::string, const w4h_tensor*> m;
  const w4h_tensor* get(const std::string& n) const {
    auto it = m.find(n);
    return it == m.end() ? nullptr : it->second;
  }
};

int64_t numel(const w4h_tensor* t) {
  int64_t n = 1;
  for (int i = 0; i < t->n_dims; i++) n *= t->ne[i];
  return n;
}

int to_f32(const w4h_tensor* t, int64_t n, std::vector<float>& v) {
  v.resize((size_t)n);
  if (t->type == W4H_TYPE_F32) {
    memcpy(v.data(), t->data, (size_t)n * 4);
  } else if (t->type == W4H_TYPE_F16) {
    const uint16_t* h = static_cast<const uint16_t*>(t->data);
    for (int64_t i = 0; i < n; i++) v[(size_t)i] = half_to_float(h[i]);
  } else {
    return fail(W4H_ERR_FORMAT, "tensor %s: type %d not supported here", t->name, t->type);
  }
  return W4H_OK;
}

int load_vec(w4h_encoder* e, const Table& tt, const std::string& name, int64_t n, const float** out,
             bool optional_zero = false) {
  const w4h_tensor* t = tt.get(name);
  std::vector<float> v;
  if (!t) {
    if (!optional_zero) return fail(W4H_ERR_NOT_FOUND, "missing tensor: %s", name.c_str());
    v.assign((size_t)n, 0.0f);
  } else {
    if (numel(t) != n) return fail(W4H_ERR_SHAPE, "tensor %s has %lld elements, expected %lld", name.c_str(), (long long)numel(t), (long long)n);
    int rc = to_f32(t, n, v);
    if (rc) return rc;
  }
  void* p;
  int rc = upload(e, v.data(), v.size() * 4, &p);
  if (rc) return rc;
  *out = static_cast<const float*>(p);
  return W4H_OK;
}

// Matrices [rows_i][K] stacked into one device matrix: f16 [N][K] (f32 rounded to f16), or q8_0 as
// int8 [N][K] + f16 scales [N][K/32].
int load_mat(w4h_encoder* e, const Table& tt, const std::vector<std::string>& names, int rows, int K, const void** w,
             const uint16_t** s) {
  const int N = rows * (int)names.size();
  std::vector<const w4h_tensor*> ts;
  for (const auto& n : names) {
    const w4h_tensor* t = tt.get(n);
    if (!t) return fail(W4H_ERR_NOT_FOUND, "missing tensor: %s", n.c_str());
    if (t->n_dims != 2 || t->ne[0] != K || t->ne[1] != rows)
      return fail(W4H_ERR_SHAPE, "tensor %s: expected ne=[%d,%d]", n.c_str(), K, rows);
    if ((t->type == W4H_TYPE_Q8_0) != (e->wq8 != 0))
      return fail(W4H_ERR_FORMAT, "tensor %s: matrix type %d does not match the encoder's %s matrices", n.c_str(), t->type,
                  e->wq8 ? "q8_0" : "f16/f32");
    if (t->type != W4H_TYPE_Q8_0 && t->type != W4H_TYPE_F16 && t->type != W4H_TYPE_F32)
      return fail(W4H_ERR_FORMAT, "tensor %s: unsupported type %d", n.c_str(), t->type);
    ts.push_back(t);
  }
  int rc;
  void* p;
  if (!e->wq8) {
    std::vector<uint16_t> h((size_t)N * K);
    for (size_t i = 0; i < ts.size(); i++) {
      const size_t n = (size_t)rows * K, o = i * n;
      if (ts[i]->type == W4H_TYPE_F16) {
        memcpy(h.data() + o, ts[i]->data, n * 2);
      } else {
        const float* f = static_cast<const float*>(ts[i]->data);
        for (size_t j = 0; j < n; j++) h[o + j] = float_to_half(f[j]);
      }
    }
    if ((rc = upload(e, h.data(), h.size() * 2, &p))) return rc;
    *w = p;
    *s = nullptr;
    return W4H_OK;
  }
  if (K % 64) return fail(W4H_ERR_SHAPE, "q8_0 encoder matrix needs K %% 64 == 0 (K=%d)", K);
  std::vector<int8_t> q((size_t)N * K);
  std::vector<uint16_t> sc((size_t)N * (K / 32));
  size_t row = 0;
  for (size_t i = 0; i < ts.size(); i++) {
    const unsigned char* src = static_cast<const unsigned char*>(ts[i]->data);
    for (int r = 0; r < rows; r++, row++)
      for (int b = 0; b < K / 32; b++) {
        const unsigned char* blk = src + ((size_t)r * (K / 32) + b) * 34;
        sc[row * (K / 32) + b] = (uint16_t)(blk[0] | (blk[1] << 8));
        memcpy(q.data() + row * K + (size_t)b * 32, blk + 2, 32);
      }
  }
  if ((rc = upload(e, q.data(), q.size(), &p))) return rc;
  *w = p;
  if ((rc = upload(e, sc.data(), sc.size() * 2, &p))) return rc;
  *s = static_cast<const uint16_t*>(p);
  return W4H_OK;
}

// Conv1d weight (GGML ne = [3, in, out], i.e. [out][in][3]) -> [out][3][in] f16.
int load_conv(w4h_encoder* e, const Table& tt, const std::string& name, int out_ch, int in_ch, const uint16_t** w) {
  const w4h_tensor* t = tt.get(name);
  if (!t) return fail(W4H_ERR_NOT_FOUND, "missing tensor: %s", name.c_str());
  if (t->n_dims != 3 || t->ne[0] != 3 || t->ne[1] != in_ch || t->ne[2] != out_ch)
    return fail(W4H_ERR_SHAPE, "tensor %s: expected ne=[3,%d,%d]", name.c_str(), in_ch, out_ch);
  if (t->type != W4H_TYPE_F16 && t->type != W4H_TYPE_F32) return fail(W4H_ERR_FORMAT, "tensor %s: unsupported type %d", name.c_str(), t->type);
  std::vector<uint16_t> h((size_t)out_ch * 3 * in_ch);
  for (int o = 0; o < out_ch; o++)
    for (int i = 0; i < in_ch; i++)
      for (int k = 0; k < 3; k++) {
        const size_t src = ((size_t)o * in_ch + i) * 3 + k;
        const uint16_t v = t->type == W4H_TYPE_F16 ? static_cast<const uint16_t*>(t->data)[src]
                                                   : float_to_half(static_cast<const float*>(t->data)[src]);
        h[((size_t)o * 3 + k) * in_ch + i] = v;
      }
  void* p;
  int rc = upload(e, h.data(), h.size() * 2, &p);
  if (rc) return rc;
  *w = static_cast<const uint16_t*>(p);
  return W4H_OK;
}

int build(w4h_encoder* e, const w4h_tensor* tensors, int n) {
  Table tt;
  for (int i = 0; i < n; i++) {
    if (!tensors[i].name) return fail(W4H_ERR_INVALID, "tensor %d has no name", i);
    tt.m[tensors[i].name] = &tensors[i];
  }
  const w4h_encoder_dims& D = e->dims;
  const int d = D.n_audio_state, T = D.n_audio_ctx, nm = D.n_mels;
  const w4h_tensor* q0 = tt.get("encoder.blocks.0.attn.query.weight");
  e->wq8 = q0 && q0->type == W4H_TYPE_Q8_0;
  int rc;
  if ((rc = load_conv(e, tt, "encoder.conv1.weight", d, nm, &e->c1w))) return rc;
  if ((rc = load_conv(e, tt, "encoder.conv2.weight", d, d, &e->c2w))) return rc;
  if ((rc = load_vec(e, tt, "encoder.conv1.bias", d, &e->c1b))) return rc;
  if ((rc = load_vec(e, tt, "encoder.conv2.bias", d, &e->c2b))) return rc;
  if ((rc = load_vec(e, tt, "encoder.positional_embedding", (int64_t)T * d, &e->pos))) return rc;
  if ((rc = load_vec(e, tt, "encoder.ln_post.weight", d, &e->lnp_g))) return rc;
  if ((rc = load_vec(e, tt, "encoder.ln_post.bias", d, &e->lnp_b))) return rc;
  e->layers.resize(D.n_audio_layer);
  for (int l = 0; l < D.n_audio_layer; l++) {
    EncLayer& L = e->layers[l];
    const std::string b = "encoder.blocks." + std::to_string(l) + ".";
    if ((rc = load_mat(e, tt, {b + "attn.query.weight", b + "attn.key.weight", b + "attn.value.weight"}, d, d, &L.w_qkv, &L.s_qkv)))
      return rc;
    if ((rc = load_mat(e, tt, {b + "attn.out.weight"}, d, d, &L.w_o, &L.s_o))) return rc;
    if ((rc = load_mat(e, tt, {b + "mlp.0.weight"}, 4 * d, d, &L.w_1, &L.s_1))) return rc;
    if ((rc = load_mat(e, tt, {b + "mlp.2.weight"}, d, 4 * d, &L.w_2, &L.s_2))) return rc;
    {  // q | k | v biases; the key projection has none (a zero block)
      std::vector<float> bq((size_t)3 * d, 0.0f), v;
      const char* parts[3] = {"attn.query.bias", "attn.key.bias", "attn.value.bias"};
      for (int p = 0; p < 3; p++) {
        const w4h_tensor* t = tt.get(b + parts[p]);
        if (!t) {
          if (p == 1) continue;
          return fail(W4H_ERR_NOT_FOUND, "missing tensor: %s%s", b.c_str(), parts[p]);
        }
        if (numel(t) != d) return fail(W4H_ERR_SHAPE, "tensor %s%s: bad shape", b.c_str(), parts[p]);
        if ((rc = to_f32(t, d, v))) return rc;
        std::copy(v.begin(), v.end(), bq.begin() + (size_t)p * d);
      }
      void* p;
      if ((rc = upload(e, bq.data(), bq.size() * 4, &p))) return rc;
      L.b_qkv = static_cast<const float*>(p);
    }
    if ((rc = load_vec(e, tt, b + "attn.out.bias", d, &L.b_o))) return rc;
    if ((rc = load_vec(e, tt, b + "mlp.0.bias", 4 * d, &L.b_1))) return rc;
    if ((rc = load_vec(e, tt, b + "mlp.2.bias", d, &L.b_2))) return rc;
    if ((rc = load_vec(e, tt, b + "attn_ln.weight", d, &L.ln1_g))) return rc;
    if ((rc = load_vec(e, tt, b + "attn_ln.bias", d, &L.ln1_b))) return rc;
    if ((rc = load_vec(e, tt, b + "mlp_ln.weight", d, &L.ln2_g))) return rc;
    if ((rc = load_vec(e, tt, b + "mlp_ln.bias", d, &L.ln2_b))) return rc;
  }
  // working buffers (zeroed: the padding frames of x1p and of the attention planes stay zero)
  e->Tp = (T + kEncPad - 1) / kEncPad * kEncPad;
  const size_t F = (size_t)2 * T;
  if (!(e->melt = static_cast<float*>(dev_alloc(e, (F + 2) * nm * 4, &rc)))) return rc;
  if (!(e->x1p = static_cast<float*>(dev_alloc(e, (F + 2) * d * 4, &rc)))) return rc;
  if (!(e->x = static_cast<float*>(dev_alloc(e, (size_t)T * d * 4, &rc)))) return rc;
  const size_t Mp = (size_t)(T + kEncRowTile - 1) / kEncRowTile * kEncRowTile;
  uint16_t** planes[6] = {&e->xnh, &e->xnl, &e->atth, &e->attl, &e->hidh, &e->hidl};
  for (int i = 0; i < 6; ++i)
    if (!(*planes[i] = static_cast<uint16_t*>(dev_alloc(e, Mp * (i < 4 ? d : 4 * d) * 2, &rc)))) return rc;
  if (!(e->qkv = static_cast<uint16_t*>(dev_alloc(e, (size_t)6 * e->Tp * d * 2, &rc)))) return rc;
  if (!(e->mel_in = static_cast<float*>(dev_alloc(e, F * nm * 4, &rc)))) return rc;
  if (!(e->out = static_cast<float*>(dev_alloc(e, (size_t)T * d * 4, &rc)))) return rc;
  HIPCHK(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
  return W4H_OK;
}

int gemm(int epi, const float* a, int lda, int M, int N, int K, const void* w, const uint16_t* ws, const float* bias,
         float* out, int ldo, const float* add, uint16_t* qkv, int Tp, hipStream_t st) {
  EncGemm g{};
  g.a = a;
  g.lda = lda;
  g.M = M;
  g.N = N;
  g.K = K;
  g.w = w;
  g.ws = ws;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.add = add;
  g.qkv = qkv;
  g.Tp = Tp;
  HIPCHK(launch_enc_gemm(epi, g, st));
  return W4H_OK;
}

int gemm2(int epi, const uint16_t* ah, const uint16_t* al, int lda, int M, int N, int K, const void* w, const uint16_t* ws,
          const float* bias, float* out, uint16_t* oh, uint16_t* ol, int ldo, uint16_t* qkv, int Tp, hipStream_t st) {
  EncGemm2 g{};
  g.ah = ah;
  g.al = al;
  g.lda = lda;
  g.M = M;
  g.N = N;
  g.K = K;
  g.w = w;
  g.ws = ws;
  g.bias = bias;
  g.out = out;
  g.oh = oh;
  g.ol = ol;
  g.ldo = ldo;
  g.qkv = qkv;
  g.Tp = Tp;
  HIPCHK(launch_enc_gemm2(epi, g, st));
  return W4H_OK;
}

// The encoder forward on stream st: mel [n_mels][2T] (device) -> out [T][d] (device).
int forward(w4h_encoder* e, const float* mel, float* out, hipStream_t st) {
  const w4h_encoder_dims& D = e->dims;
  const int d = D.n_audio_state, T = D.n_audio_ctx, nm = D.n_mels, H = D.n_audio_head, F = 2 * T;
  int rc;
  HIPCHK(launch_enc_mel_t(mel, nm, F, e->melt, st));
  // conv1 + GELU into frames 1..F of x1p; conv2 (stride 2) + GELU + positional embedding into x
  if ((rc = gemm(kEpiGelu, e->melt, nm, F, d, 3 * nm, e->c1w, nullptr, e->c1b, e->x1p + d, d, nullptr, nullptr, 0, st)))
    return rc;
  if ((rc = gemm(kEpiGeluPos, e->x1p, 2 * d, T, d, 3 * d, e->c2w, nullptr, e->c2b, e->x, d, e->pos, nullptr, 0, st)))
    return rc;
  for (const EncLayer& L : e->layers) {
    HIPCHK(launch_enc_ln(e->x, T, d, L.ln1_g, L.ln1_b, nullptr, e->xnh, e->xnl, st));
    if ((rc = gemm2(kEpiQkv, e->xnh, e->xnl, d, T, 3 * d, d, L.w_qkv, L.s_qkv, L.b_qkv, nullptr, nullptr, nullptr, 0, e->qkv,
                    e->Tp, st)))
      return rc;
    HIPCHK(launch_enc_attn(e->qkv, T, e->Tp, H, e->atth, e->attl, st));
    if ((rc = gemm2(kEpiResid, e->atth, e->attl, d, T, d, d, L.w_o, L.s_o, L.b_o, e->x, nullptr, nullptr, d, nullptr, 0, st)))
      return rc;
    HIPCHK(launch_enc_ln(e->x, T, d, L.ln2_g, L.ln2_b, nullptr, e->xnh, e->xnl, st));
    if ((rc = gemm2(kEpiGeluPlanes, e->xnh, e->xnl, d, T, 4 * d, d, L.w_1, L.s_1, L.b_1, nullptr, e->hidh, e->hidl, 4 * d,
                    nullptr, 0, st)))
      return rc;
    if ((rc = gemm2(kEpiResid, e->hidh, e->hidl, 4 * d, T, d, 4 * d, L.w_2, L.s_2, L.b_2, e->x, nullptr, nullptr, d, nullptr, 0,
                    st)))
      return rc;
  }
  HIPCHK(launch_enc_ln(e->x, T, d, e->lnp_g, e->lnp_b, out, nullptr, nullptr, st));
  return W4H_OK;
}

}  // namespace

extern "C" {

int w4h_encoder_create(const w4h_encoder_dims* dims, const w4h_tensor* tensors, int32_t n_tensors, int32_t device,
                       w4h_encoder** out) {
  if (!dims || !tensors || !out || n_tensors <= 0) return fail(W4H_ERR_INVALID, "null argument");
  *out = nullptr;
  const int d = dims->n_audio_state;
  if (d <= 0 || d % 64 || dims->n_audio_head * 64 != d)
    return fail(W4H_ERR_INVALID, "n_audio_state (%d) must be 64 * n_audio_head (%d)", d, dims->n_audio_head);
  if (d > 64 * kEncLnPer) return fail(W4H_ERR_INVALID, "n_audio_state %d above the supported %d", d, 64 * kEncLnPer);
  if (dims->n_audio_ctx <= 0 || dims->n_audio_layer <= 0 || dims->n_mels <= 0 || dims->n_mels % 8 || dims->n_mels > 1024)
    return fail(W4H_ERR_INVALID, "n_audio_ctx and n_audio_layer must be positive, n_mels a multiple of 8 up to 1024");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(W4H_ERR_DEVICE, "no HIP device available");
  if (device < 0 || device >= n) return fail(W4H_ERR_INVALID, "device %d out of range (%d devices)", device, n);
  HIPCHK(hipSetDevice(device));
  auto* e = new w4h_encoder();
  e->device = device;
  e->dims = *dims;
  int rc = build(e, tensors, n_tensors);
  if (rc) {
    delete e;
    return rc;
  }
  *out = e;
  return W4H_OK;
}

int w4h_encoder_get_dims(const w4h_encoder* e, w4h_encoder_dims* out) {
  if (!e || !out) return fail(W4H_ERR_INVALID, "null argument");
  *out = e->dims;
  return W4H_OK;
}

int w4h_encoder_forward(w4h_encoder* e, const float* mel, float* out) {
  if (!e || !mel || !out) return fail(W4H_ERR_INVALID, "null argument");
  std::lock_guard<std::mutex> lk(e->mu);
  if (e->closed) return fail(W4H_ERR_CLOSED, "encoder destroyed");
  HIPCHK(hipSetDevice(e->device));
  const w4h_encoder_dims& D = e->dims;
  const size_t in_b = (size_t)D.n_mels * 2 * D.n_audio_ctx * 4, out_b = (size_t)D.n_audio_ctx * D.n_audio_state * 4;
  HIPCHK(hipMemcpyAsync(e->mel_in, mel, in_b, hipMemcpyHostToDevice, e->stream));
  int rc = forward(e, e->mel_in, e->out, e->stream);
  if (rc) return rc;
  HIPCHK(hipMemcpyAsync(out, e->out, out_b, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(hipStreamSynchronize(e->stream));
  return W4H_OK;
}

int w4h_encoder_forward_device(w4h_encoder* e, const float* mel_dev, float* out_dev, void* stream) {
  if (!e || !mel_dev || !out_dev) return fail(W4H_ERR_INVALID, "null argument");
  std::lock_guard<std::mutex> lk(e->mu);
  if (e->closed) return fail(W4H_ERR_CLOSED, "encoder destroyed");
  HIPCHK(hipSetDevice(e->device));
  hipStream_t st = stream ? static_cast<hipStream_t>(stream) : e->stream;
  int rc = forward(e, mel_dev, out_dev, st);
  if (rc) return rc;
  if (!stream) HIPCHK(hipStreamSynchronize(st));
  return W4H_OK;
}

int w4h_encoder_destroy(w4h_encoder* e) {
  if (!e) return fail(W4H_ERR_INVALID, "null argument");
  {
    std::lock_guard<std::mutex> lk(e->mu);
    if (e->closed) return fail(W4H_ERR_CLOSED, "encoder already destroyed");
    e->closed = true;
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
  }
  delete e;
  return W4H_OK;
}

}  // extern "C"
