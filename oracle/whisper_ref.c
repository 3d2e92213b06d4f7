/*
 * whisper_ref.c -- the oracle: CPU restatement of whisper4j's Linux text-decoder path.
 *
 * TEST INFRASTRUCTURE ONLY (see whisper_ref.h).  It is the parity reference for the HIP product and the
 * timed CPU baseline ("port"); nothing in whisper4j_amd/ links, loads or calls it.
 *
 * Build: gcc -O3 -march=x86-64-v3 -ffp-contract=off -fPIC -shared whisper_ref.c -lz -lm
 * (-ffp-contract=off is part of the contract: Java evaluates a*b+c as two roundings.)
 */
#include "whisper_ref.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <zlib.h>

/* ------------------------------------------------------------------------------------------ */
/* f16 <-> f32: Float.float16ToFloat / Float.floatToFloat16 (IEEE binary16, round-to-nearest-even) */

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do { man <<= 1; e++; } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf or NaN */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    uint32_t m = (ax >> 13) & 0x3ffu;
    return (uint16_t)(sign | 0x7c00u | (m ? m : 0x200u));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (ax < 0x38800000u) {                                      /* result is subnormal or zero */
    if (ax < 0x33000000u) return (uint16_t)sign;               /* < 2^-25 rounds to 0 */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - e; /* so that value = m * 2^-(shift+...)*/
    /* f = m * 2^(e-150); subnormal unit is 2^-24 -> q = m * 2^(e-150+24) = m >> (126-e) */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = (ax >> 23) - 127 + 15;
  uint32_t m = ax & 0x7fffffu;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------------------------------ */
/* GELU table: main/tensor/Tensor.java:493-501.  Same float expression tree, Math.tanh on the
 * widened argument, rounded back to float. */
void orc_gelu_table(float* table) {
  float s = (float)sqrt(2.0 / 3.14159265358979323846);
  for (int i = 0; i < 65536; i++) {
    float x = orc_f16_to_f32((uint16_t)i);
    float inner = s * (x + 0.044715f * x * x * x);
    table[i] = 0.5f * x * (1.0f + (float)tanh((double)inner));
  }
}

static float* g_gelu_table = NULL;
static const float* gelu_table(void) {
  if (!g_gelu_table) {
    float* t = (float*)malloc(65536 * sizeof(float));
    orc_gelu_table(t);
    g_gelu_table = t;
  }
  return g_gelu_table;
}

/* Tensor.geluInPlace: main/tensor/Tensor.java:524-538 */
void orc_gelu(float* x, int n) {
  const float* t = gelu_table();
  for (int i = 0; i < n; i++) x[i] = t[orc_f32_to_f16(x[i])];
}

/* ------------------------------------------------------------------------------------------ */
/* VectorSimdOps.dot: java26/.../VectorSimdOps.java:20-39.  acc = acc + a*b lane-wise over
 * loopBound(len); reduceLanes(ADD); scalar tail added in order. */
float orc_dot(const float* a, const float* b, int n) {
  float acc[ORC_LANES];
  for (int l = 0; l < ORC_LANES; l++) acc[l] = 0.0f;
  int bound = n - n % ORC_LANES;
  int i = 0;
  for (; i < bound; i += ORC_LANES)
    for (int l = 0; l < ORC_LANES; l++) acc[l] = acc[l] + a[i + l] * b[i + l];
  float sum = acc[0];
  for (int l = 1; l < ORC_LANES; l++) sum = sum + acc[l];
  for (; i < n; i++) sum = sum + a[i] * b[i];
  return sum;
}

/* Tensor.layerNorm: main/tensor/Tensor.java:592-619 (eps 1e-5 from main/nn/LayerNorm.java:16) */
void orc_layernorm(const float* x, int rows, int n, const float* g, const float* b, float eps, float* out) {
  for (int r = 0; r < rows; r++) {
    const float* row = x + (size_t)r * n;
    float* o = out + (size_t)r * n;
    float mean = 0.0f;
    for (int j = 0; j < n; j++) mean += row[j];
    mean /= (float)n;
    float variance = 0.0f;
    for (int j = 0; j < n; j++) {
      float d = row[j] - mean;
      variance += d * d;
    }
    float invStd = 1.0f / (float)sqrt((double)(variance / (float)n + eps));
    for (int j = 0; j < n; j++) o[j] = (row[j] - mean) * invStd * g[j] + b[j];
  }
}

/* Linear.forward = x.matmul(W^T) then bias addInPlace: main/nn/Linear.java:23-26.
 * M==1: Tensor.matmulVec -> matmulVecAccumulate (main/tensor/Tensor.java:383-398,
 * java26/.../VectorSimdOps.java:114-133): y_j = y_j + x_k * wt[k][j], k ascending, y zeroed.
 * M>1: Tensor.matmulTiled (main/tensor/Tensor.java:460-489): per element the same ascending-k
 * sum from 0 (tiles only reorder independent elements), so one loop order serves both.
 * Bias: Tensor.addInPlace broadcast (main/tensor/Tensor.java:251-263): y = y + b. */
void orc_linear(const float* x, int m, int k, const float* wt, int n, const float* bias, float* y) {
  for (int i = 0; i < m; i++) {
    float* yi = y + (size_t)i * n;
    const float* xi = x + (size_t)i * k;
    for (int j = 0; j < n; j++) yi[j] = 0.0f;
    for (int kk = 0; kk < k; kk++) {
      float xk = xi[kk];
      const float* w = wt + (size_t)kk * n;
      for (int j = 0; j < n; j++) yi[j] = yi[j] + xk * w[j];
    }
    if (bias)
      for (int j = 0; j < n; j++) yi[j] = yi[j] + bias[j];
  }
}

/* VectorSimdOps.fusedAttentionHead: java26/.../VectorSimdOps.java:137-203 (scores with the lane
 * dot, float max, (float)Math.exp, sequential float sum, p = e * (1/sum), out = out + p*v). */
void orc_attention_head(const float* q, const float* k, const float* v, int kv_len, int hd, float scale,
                        float* out) {
  float* scores = (float*)malloc(sizeof(float) * (size_t)(kv_len > 0 ? kv_len : 1));
  float maxScore = -INFINITY;
  for (int j = 0; j < kv_len; j++) {
    float s = orc_dot(q, k + (size_t)j * hd, hd) * scale;
    scores[j] = s;
    if (s > maxScore) maxScore = s;
  }
  float sum = 0.0f;
  for (int j = 0; j < kv_len; j++) {
    scores[j] = (float)exp((double)(scores[j] - maxScore));
    sum += scores[j];
  }
  float invSum = 1.0f / sum;
  for (int j = 0; j < kv_len; j++) scores[j] *= invSum;
  for (int d = 0; d < hd; d++) out[d] = 0.0f;
  for (int j = 0; j < kv_len; j++) {
    float sj = scores[j];
    const float* vr = v + (size_t)j * hd;
    for (int d = 0; d < hd; d++) out[d] = out[d] + sj * vr[d];
  }
  free(scores);
}

/* Tensor.softmax non-Accelerate path: main/tensor/Tensor.java:550-568 (max seeded with row[0]). */
void orc_softmax_rows(float* x, int rows, int n) {
  for (int r = 0; r < rows; r++) {
    float* row = x + (size_t)r * n;
    float max = row[0];
    for (int j = 1; j < n; j++)
      if (row[j] > max) max = row[j];
    float sum = 0.0f;
    for (int j = 0; j < n; j++) {
      row[j] = (float)exp((double)(row[j] - max));
      sum += row[j];
    }
    float invSum = 1.0f / sum;
    for (int j = 0; j < n; j++) row[j] *= invSum;
  }
}

/* WhisperDecoder.argmax: main/nn/WhisperDecoder.java:566-574 (first index of the maximum). */
int orc_argmax(const float* a, int n) {
  int best = 0;
  for (int i = 1; i < n; i++)
    if (a[i] > a[best]) best = i;
  return best;
}

/* WhisperDecoder.computeLogSoftmax: main/nn/WhisperDecoder.java:397-412. */
void orc_log_softmax(const float* logits, int n, float* out) {
  float max = -INFINITY;
  for (int i = 0; i < n; i++)
    if (logits[i] > max) max = logits[i];
  double logSum = 0;
  for (int i = 0; i < n; i++) logSum += exp((double)(logits[i] - max));
  float logSumF = (float)((double)max + log(logSum));
  for (int i = 0; i < n; i++) out[i] = logits[i] - logSumF;
}

/* WhisperDecoder.topkIndices: main/nn/WhisperDecoder.java:415-431 (insertion with strict >,
 * so ties keep the lower index; unfilled slots keep index 0). */
void orc_topk(const float* values, int n, int k, int32_t* idx) {
  float* top = (float*)malloc(sizeof(float) * (size_t)k);
  for (int i = 0; i < k; i++) { top[i] = -INFINITY; idx[i] = 0; }
  for (int i = 0; i < n; i++) {
    if (values[i] > top[k - 1]) {
      int pos = k - 1;
      while (pos > 0 && values[i] > top[pos - 1]) pos--;
      memmove(top + pos + 1, top + pos, sizeof(float) * (size_t)(k - 1 - pos));
      memmove(idx + pos + 1, idx + pos, sizeof(int32_t) * (size_t)(k - 1 - pos));
      top[pos] = values[i];
      idx[pos] = i;
    }
  }
  free(top);
}

/* WhisperDecoder.compressionRatio: main/nn/WhisperDecoder.java:628-647 (tokens as 2 LE bytes,
 * java.util.zip.Deflater defaults = zlib stream at the default level). */
float orc_compression_ratio(const int32_t* tokens, int n) {
  if (n == 0) return 0.0f;
  uLong len = (uLong)n * 2;
  unsigned char* bytes = (unsigned char*)malloc(len);
  for (int i = 0; i < n; i++) {
    bytes[2 * i] = (unsigned char)(tokens[i] & 0xff);
    bytes[2 * i + 1] = (unsigned char)((tokens[i] >> 8) & 0xff);
  }
  uLongf clen = compressBound(len);
  unsigned char* dst = (unsigned char*)malloc(clen);
  compress2(dst, &clen, bytes, len, Z_DEFAULT_COMPRESSION);
  free(bytes);
  free(dst);
  return (float)len / (float)(clen > 1 ? clen : 1);
}

/* GgmlLoader.dequantizeQ8_0: main/model/GgmlLoader.java:292-300 (34-byte blocks: f16 d, 32 int8). */
void orc_dequant_q8_0(const void* src, int64_t n, float* dst) {
  const unsigned char* p = (const unsigned char*)src;
  for (int64_t b = 0; b < n / 32; b++) {
    uint16_t hd = (uint16_t)(p[0] | (p[1] << 8));
    float scale = orc_f16_to_f32(hd);
    for (int j = 0; j < 32; j++) dst[b * 32 + j] = (float)(int8_t)p[2 + j] * scale;
    p += 34;
  }
}

/* ------------------------------------------------------------------------------------------ */
/* Model                                                                                        */

typedef struct {
  float *wt, *b; /* wt: [in][out] (Linear's transposed copy), b may be NULL */
  int in, out;
} orc_lin;

typedef struct {
  orc_lin q, k, v, o;
} orc_mha;

typedef struct {
  orc_mha attn, cross;
  float *attn_ln_g, *attn_ln_b, *cross_ln_g, *cross_ln_b, *mlp_ln_g, *mlp_ln_b;
  orc_lin mlp1, mlp2;
} orc_block;

struct orc_model {
  orc_dims d;
  float* tok_emb; /* [V][d] */
  float* pos_emb; /* [ctx][d] */
  float *ln_g, *ln_b;
  orc_block* blocks;
  float* logit_bias; /* [V] added to every logits row, or NULL */
};

static const orc_tensor* find_tensor(const orc_tensor* t, int n, const char* name) {
  for (int i = 0; i < n; i++)
    if (strcmp(t[i].name, name) == 0) return &t[i];
  return NULL;
}

/* GgmlLoader.dequantize (F32 slice, F16 exact widening, Q8_0): main/model/GgmlLoader.java:186-201, 224-238 */
static float* load_f32(const orc_tensor* tab, int ntab, const char* name, int64_t expect, char* err, int errlen) {
  const orc_tensor* t = find_tensor(tab, ntab, name);
  if (!t) {
    snprintf(err, errlen, "missing tensor: %s", name);
    return NULL;
  }
  int64_t numel = 1;
  for (int i = 0; i < t->n_dims; i++) numel *= t->ne[i];
  if (numel != expect) {
    snprintf(err, errlen, "tensor %s has %lld elements, expected %lld", name, (long long)numel, (long long)expect);
    return NULL;
  }
  float* out = (float*)malloc(sizeof(float) * (size_t)numel);
  if (t->type == ORC_TYPE_F32) {
    memcpy(out, t->data, sizeof(float) * (size_t)numel);
  } else if (t->type == ORC_TYPE_F16) {
    const uint16_t* h = (const uint16_t*)t->data;
    for (int64_t i = 0; i < numel; i++) out[i] = orc_f16_to_f32(h[i]);
  } else if (t->type == ORC_TYPE_Q8_0) {
    if (numel % 32) {
      snprintf(err, errlen, "tensor %s: q8_0 needs a multiple of 32 elements", name);
      free(out);
      return NULL;
    }
    orc_dequant_q8_0(t->data, numel, out);
  } else {
    snprintf(err, errlen, "tensor %s: unsupported type %d", name, t->type);
    free(out);
    return NULL;
  }
  return out;
}

/* Linear ctor: weight.transposeNative() (main/nn/Linear.java:16-19, main/tensor/Tensor.java:191-212) */
static int load_lin(orc_lin* l, const orc_tensor* tab, int ntab, const char* wname, const char* bname, int in,
                    int out, char* err, int errlen) {
  float* w = load_f32(tab, ntab, wname, (int64_t)in * out, err, errlen); /* [out][in] */
  if (!w) return -1;
  l->wt = (float*)malloc(sizeof(float) * (size_t)in * out);
  for (int r = 0; r < out; r++)
    for (int c = 0; c < in; c++) l->wt[(size_t)c * out + r] = w[(size_t)r * in + c];
  free(w);
  l->b = NULL;
  if (bname && find_tensor(tab, ntab, bname)) {
    l->b = load_f32(tab, ntab, bname, out, err, errlen);
    if (!l->b) return -1;
  }
  l->in = in;
  l->out = out;
  return 0;
}

static void free_lin(orc_lin* l) {
  free(l->wt);
  free(l->b);
}

void orc_model_destroy(orc_model* m) {
  if (!m) return;
  free(m->tok_emb);
  free(m->pos_emb);
  free(m->ln_g);
  free(m->ln_b);
  free(m->logit_bias);
  if (m->blocks) {
    for (int i = 0; i < m->d.n_text_layer; i++) {
      orc_block* b = &m->blocks[i];
      orc_lin* ls[] = {&b->attn.q, &b->attn.k, &b->attn.v, &b->attn.o, &b->cross.q, &b->cross.k,
                       &b->cross.v, &b->cross.o, &b->mlp1, &b->mlp2};
      for (size_t j = 0; j < sizeof(ls) / sizeof(ls[0]); j++) free_lin(ls[j]);
      free(b->attn_ln_g); free(b->attn_ln_b); free(b->cross_ln_g); free(b->cross_ln_b);
      free(b->mlp_ln_g); free(b->mlp_ln_b);
    }
    free(m->blocks);
  }
  free(m);
}

/* WhisperDecoder ctor + buildDecoderBlock + WhisperEncoder.buildMHA:
 * main/nn/WhisperDecoder.java:36-56, 658-669; main/nn/WhisperEncoder.java:98-105 (key bias optional). */
orc_model* orc_model_create(const orc_dims* dims, const orc_tensor* tab, int ntab, char* err, int errlen) {
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  m->d = *dims;
  int d = dims->n_text_state, V = dims->n_vocab, C = dims->n_text_ctx, L = dims->n_text_layer;
  char nb[256], bb[256];
  if (d % 64 != 0 || dims->n_text_head * 64 != d) {
    snprintf(err, errlen, "n_text_state %d must equal 64 * n_text_head %d", d, dims->n_text_head);
    goto fail;
  }
  if (!(m->tok_emb = load_f32(tab, ntab, "decoder.token_embedding.weight", (int64_t)V * d, err, errlen))) goto fail;
  if (!(m->pos_emb = load_f32(tab, ntab, "decoder.positional_embedding", (int64_t)C * d, err, errlen))) goto fail;
  if (!(m->ln_g = load_f32(tab, ntab, "decoder.ln.weight", d, err, errlen))) goto fail;
  if (!(m->ln_b = load_f32(tab, ntab, "decoder.ln.bias", d, err, errlen))) goto fail;
  m->blocks = (orc_block*)calloc((size_t)L, sizeof(orc_block));
  for (int i = 0; i < L; i++) {
    orc_block* b = &m->blocks[i];
    const char* mh[2] = {"attn", "cross_attn"};
    orc_mha* mp[2] = {&b->attn, &b->cross};
    for (int a = 0; a < 2; a++) {
      const char* pr[4] = {"query", "key", "value", "out"};
      orc_lin* lp[4] = {&mp[a]->q, &mp[a]->k, &mp[a]->v, &mp[a]->o};
      for (int j = 0; j < 4; j++) {
        snprintf(nb, sizeof nb, "decoder.blocks.%d.%s.%s.weight", i, mh[a], pr[j]);
        snprintf(bb, sizeof bb, "decoder.blocks.%d.%s.%s.bias", i, mh[a], pr[j]);
        if (j != 1 && !find_tensor(tab, ntab, bb)) {
          snprintf(err, errlen, "missing tensor: %s", bb);
          goto fail;
        }
        if (load_lin(lp[j], tab, ntab, nb, bb, d, d, err, errlen)) goto fail;
      }
    }
    const char* lnn[3] = {"attn_ln", "cross_attn_ln", "mlp_ln"};
    float** lg[3] = {&b->attn_ln_g, &b->cross_ln_g, &b->mlp_ln_g};
    float** lb[3] = {&b->attn_ln_b, &b->cross_ln_b, &b->mlp_ln_b};
    for (int j = 0; j < 3; j++) {
      snprintf(nb, sizeof nb, "decoder.blocks.%d.%s.weight", i, lnn[j]);
      if (!(*lg[j] = load_f32(tab, ntab, nb, d, err, errlen))) goto fail;
      snprintf(nb, sizeof nb, "decoder.blocks.%d.%s.bias", i, lnn[j]);
      if (!(*lb[j] = load_f32(tab, ntab, nb, d, err, errlen))) goto fail;
    }
    snprintf(nb, sizeof nb, "decoder.blocks.%d.mlp.0.weight", i);
    snprintf(bb, sizeof bb, "decoder.blocks.%d.mlp.0.bias", i);
    if (load_lin(&b->mlp1, tab, ntab, nb, bb, d, 4 * d, err, errlen)) goto fail;
    snprintf(nb, sizeof nb, "decoder.blocks.%d.mlp.2.weight", i);
    snprintf(bb, sizeof bb, "decoder.blocks.%d.mlp.2.bias", i);
    if (load_lin(&b->mlp2, tab, ntab, nb, bb, 4 * d, d, err, errlen)) goto fail;
  }
  return m;
fail:
  orc_model_destroy(m);
  return NULL;
}

/* A fixed logit bias (the beam workload's seeded bias; not part of the reference): added to the
 * raw logits of every row after the tied projection, before any rule or selection. */
void orc_model_set_logit_bias(orc_model* m, const float* bias) {
  free(m->logit_bias);
  m->logit_bias = NULL;
  if (bias) {
    m->logit_bias = (float*)malloc(sizeof(float) * (size_t)m->d.n_vocab);
    memcpy(m->logit_bias, bias, sizeof(float) * (size_t)m->d.n_vocab);
  }
}

/* ------------------------------------------------------------------------------------------ */
/* KV cache: the reference keeps a HashMap<String,Tensor> per decode call; appends allocate a new
 * (H, L+n, 64) tensor and copy (main/nn/MultiHeadAttention.java:140-164), beams copy the map so
 * tensors are shared (main/nn/WhisperDecoder.java:239-266, 342-361).  Here: refcounted tensors in
 * a refcounted per-call cache.                                                                 */

typedef struct {
  int refs;
  int h, len, hd;
  float* data; /* [h][len][hd] */
} orc_kv;

struct orc_cache {
  int refs;
  int n_layer;
  orc_kv** self_k;
  orc_kv** self_v;
  orc_kv** cross_k;
  orc_kv** cross_v;
};

static orc_kv* kv_new(int h, int len, int hd) {
  orc_kv* t = (orc_kv*)malloc(sizeof(orc_kv));
  t->refs = 1;
  t->h = h;
  t->len = len;
  t->hd = hd;
  t->data = (float*)malloc(sizeof(float) * (size_t)h * (size_t)(len > 0 ? len : 1) * hd);
  return t;
}
static void kv_unref(orc_kv* t) {
  if (t && --t->refs == 0) {
    free(t->data);
    free(t);
  }
}
static orc_kv* kv_ref(orc_kv* t) {
  if (t) t->refs++;
  return t;
}

orc_cache* orc_cache_create(const orc_model* m) {
  orc_cache* c = (orc_cache*)calloc(1, sizeof(orc_cache));
  c->refs = 1;
  c->n_layer = m->d.n_text_layer;
  c->self_k = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  c->self_v = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  c->cross_k = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  c->cross_v = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  return c;
}

void orc_cache_destroy(orc_cache* c) {
  if (!c || --c->refs > 0) return;
  for (int i = 0; i < c->n_layer; i++) {
    kv_unref(c->self_k[i]);
    kv_unref(c->self_v[i]);
    kv_unref(c->cross_k[i]);
    kv_unref(c->cross_v[i]);
  }
  free(c->self_k);
  free(c->self_v);
  free(c->cross_k);
  free(c->cross_v);
  free(c);
}

int orc_cache_len(const orc_cache* c) { return (c && c->self_k[0]) ? c->self_k[0]->len : 0; }

/* new map with the same entries (tensors shared) */
static orc_cache* cache_copy(const orc_cache* s) {
  orc_cache* c = (orc_cache*)calloc(1, sizeof(orc_cache));
  c->refs = 1;
  c->n_layer = s->n_layer;
  c->self_k = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  c->self_v = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  c->cross_k = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  c->cross_v = (orc_kv**)calloc((size_t)c->n_layer, sizeof(orc_kv*));
  for (int i = 0; i < c->n_layer; i++) {
    c->self_k[i] = kv_ref(s->self_k[i]);
    c->self_v[i] = kv_ref(s->self_v[i]);
    c->cross_k[i] = kv_ref(s->cross_k[i]);
    c->cross_v[i] = kv_ref(s->cross_v[i]);
  }
  return c;
}

/* (S, H*hd) -> (H, S, hd): Tensor.rearrangeToHeads main/tensor/Tensor.java:645-659 */
static void to_heads(const float* x, int s, int h, int hd, float* out) {
  for (int t = 0; t < s; t++)
    for (int i = 0; i < h; i++) memcpy(out + ((size_t)i * s + t) * hd, x + ((size_t)t * h + i) * hd, sizeof(float) * hd);
}

/* appendHeadsCache: main/nn/MultiHeadAttention.java:140-164 */
static orc_kv* kv_append(orc_kv* old, const float* heads, int n, int h, int hd) {
  int ol = old ? old->len : 0;
  orc_kv* t = kv_new(h, ol + n, hd);
  for (int i = 0; i < h; i++) {
    float* dst = t->data + (size_t)i * t->len * hd;
    if (ol) memcpy(dst, old->data + (size_t)i * ol * hd, sizeof(float) * (size_t)ol * hd);
    memcpy(dst + (size_t)ol * hd, heads + (size_t)i * n * hd, sizeof(float) * (size_t)n * hd);
  }
  return t;
}

/* MultiHeadAttention.forward: main/nn/MultiHeadAttention.java:37-96, with the fused M==1 branch
 * (:80-82, :110-132) and the unfused masked branch (:84-95). */
static void mha_forward(const orc_model* m, const orc_mha* a, const float* x, int n, const float* xa,
                        orc_cache* cache, int layer, int is_cross, float* out) {
  int d = m->d.n_text_state, H = m->d.n_text_head, hd = 64, A = m->d.n_audio_ctx;
  float scale = (float)(1.0 / sqrt((double)hd));
  float* q = (float*)malloc(sizeof(float) * (size_t)n * d);
  orc_linear(x, n, d, a->q.wt, d, a->q.b, q);
  orc_kv **kslot = is_cross ? &cache->cross_k[layer] : &cache->self_k[layer];
  orc_kv **vslot = is_cross ? &cache->cross_v[layer] : &cache->self_v[layer];
  orc_kv *kr, *vr;
  if (is_cross && *kslot) {
    kr = *kslot;
    vr = *vslot;
  } else if (!is_cross && *kslot) {
    float* nk = (float*)malloc(sizeof(float) * (size_t)n * d);
    float* nv = (float*)malloc(sizeof(float) * (size_t)n * d);
    float* hk = (float*)malloc(sizeof(float) * (size_t)n * d);
    float* hv = (float*)malloc(sizeof(float) * (size_t)n * d);
    orc_linear(x, n, d, a->k.wt, d, a->k.b, nk);
    orc_linear(x, n, d, a->v.wt, d, a->v.b, nv);
    to_heads(nk, n, H, hd, hk);
    to_heads(nv, n, H, hd, hv);
    orc_kv* ak = kv_append(*kslot, hk, n, H, hd);
    orc_kv* av = kv_append(*vslot, hv, n, H, hd);
    kv_unref(*kslot);
    kv_unref(*vslot);
    *kslot = ak;
    *vslot = av;
    kr = ak;
    vr = av;
    free(nk); free(nv); free(hk); free(hv);
  } else {
    const float* src = is_cross ? xa : x;
    int sl = is_cross ? A : n;
    float* k = (float*)malloc(sizeof(float) * (size_t)sl * d);
    float* v = (float*)malloc(sizeof(float) * (size_t)sl * d);
    orc_linear(src, sl, d, a->k.wt, d, a->k.b, k);
    orc_linear(src, sl, d, a->v.wt, d, a->v.b, v);
    kr = kv_new(H, sl, hd);
    vr = kv_new(H, sl, hd);
    to_heads(k, sl, H, hd, kr->data);
    to_heads(v, sl, H, hd, vr->data);
    free(k);
    free(v);
    *kslot = kr;
    *vslot = vr;
  }
  int kvLen = kr->len;
  float* merged = (float*)malloc(sizeof(float) * (size_t)n * d);
  if (n == 1) {
    for (int h = 0; h < H; h++)
      orc_attention_head(q + (size_t)h * hd, kr->data + (size_t)h * kvLen * hd, vr->data + (size_t)h * kvLen * hd,
                         kvLen, hd, scale, merged + (size_t)h * hd);
  } else {
    /* qr.matmulTransB(kr, scale) -> addMaskInPlace (no offset) -> softmax -> matmul(vr) */
    int C = m->d.n_text_ctx;
    float* w = (float*)malloc(sizeof(float) * (size_t)H * n * kvLen);
    float* qr = (float*)malloc(sizeof(float) * (size_t)n * d);
    to_heads(q, n, H, hd, qr);
    for (int h = 0; h < H; h++)
      for (int i = 0; i < n; i++)
        for (int j = 0; j < kvLen; j++)
          w[((size_t)h * n + i) * kvLen + j] =
              orc_dot(qr + ((size_t)h * n + i) * hd, kr->data + ((size_t)h * kvLen + j) * hd, hd) * scale;
    if (!is_cross) { /* mask passed only to self-attention (main/nn/ResidualAttentionBlock.java:46-47) */
      int aq = n < C ? n : C, ak = kvLen < C ? kvLen : C;
      for (int h = 0; h < H; h++)
        for (int i = 0; i < aq; i++)
          for (int j = 0; j < ak; j++) {
            float mv = j > i ? -INFINITY : 0.0f;
            w[((size_t)h * n + i) * kvLen + j] = w[((size_t)h * n + i) * kvLen + j] + mv;
          }
    }
    orc_softmax_rows(w, H * n, kvLen);
    for (int h = 0; h < H; h++)
      for (int i = 0; i < n; i++) {
        float* o = merged + (size_t)i * d + (size_t)h * hd; /* rearrangeFromHeads */
        for (int e = 0; e < hd; e++) o[e] = 0.0f;
        for (int j = 0; j < kvLen; j++) {
          float p = w[((size_t)h * n + i) * kvLen + j];
          const float* vv = vr->data + ((size_t)h * kvLen + j) * hd;
          for (int e = 0; e < hd; e++) o[e] = o[e] + p * vv[e];
        }
      }
    free(w);
    free(qr);
  }
  orc_linear(merged, n, d, a->o.wt, d, a->o.b, out);
  free(merged);
  free(q);
}

/* WhisperDecoder.forwardWithAttn: main/nn/WhisperDecoder.java:66-104;
 * ResidualAttentionBlock.forwardWithAttn: main/nn/ResidualAttentionBlock.java:42-60. */
int orc_forward(const orc_model* m, const int32_t* tokens, int n, const float* xa, orc_cache* cache,
                float* logits) {
  int d = m->d.n_text_state, C = m->d.n_text_ctx, V = m->d.n_vocab;
  int offset = 0;
  if (cache) {
    int inf = orc_cache_len(cache);
    offset = inf < C - n ? inf : C - n;
  }
  for (int t = 0; t < n; t++)
    if (tokens[t] < 0 || tokens[t] >= V) return -1;
  if (offset < 0 || offset + n > C) return -2;
  float* x = (float*)malloc(sizeof(float) * (size_t)n * d);
  float* h = (float*)malloc(sizeof(float) * (size_t)n * d);
  float* a = (float*)malloc(sizeof(float) * (size_t)n * d);
  float* f = (float*)malloc(sizeof(float) * (size_t)n * 4 * d);
  for (int t = 0; t < n; t++)
    for (int j = 0; j < d; j++)
      x[(size_t)t * d + j] = m->tok_emb[(size_t)tokens[t] * d + j] + m->pos_emb[(size_t)(offset + t) * d + j];
  orc_cache* tmp = cache ? NULL : orc_cache_create(m);
  orc_cache* c = cache ? cache : tmp;
  for (int l = 0; l < m->d.n_text_layer; l++) {
    const orc_block* b = &m->blocks[l];
    orc_layernorm(x, n, d, b->attn_ln_g, b->attn_ln_b, 1e-5f, h);
    if (!cache) { /* forward without a cache: fresh K/V each call */
      kv_unref(c->self_k[l]); kv_unref(c->self_v[l]);
      c->self_k[l] = c->self_v[l] = NULL;
    }
    mha_forward(m, &b->attn, h, n, NULL, c, l, 0, a);
    for (size_t i = 0; i < (size_t)n * d; i++) x[i] = a[i] + x[i];
    orc_layernorm(x, n, d, b->cross_ln_g, b->cross_ln_b, 1e-5f, h);
    mha_forward(m, &b->cross, h, n, xa, c, l, 1, a);
    for (size_t i = 0; i < (size_t)n * d; i++) x[i] = x[i] + a[i];
    orc_layernorm(x, n, d, b->mlp_ln_g, b->mlp_ln_b, 1e-5f, h);
    orc_linear(h, n, d, b->mlp1.wt, 4 * d, b->mlp1.b, f);
    orc_gelu(f, n * 4 * d);
    orc_linear(f, n, 4 * d, b->mlp2.wt, d, b->mlp2.b, a);
    for (size_t i = 0; i < (size_t)n * d; i++) x[i] = x[i] + a[i];
  }
  orc_layernorm(x, n, d, m->ln_g, m->ln_b, 1e-5f, h);
  /* x.matmulTransB(tokenEmbedding, 1f): main/tensor/Tensor.java:327-340 (M==1) and :357-371 */
  for (int t = 0; t < n; t++)
    for (int v = 0; v < V; v++)
      logits[(size_t)t * V + v] = orc_dot(h + (size_t)t * d, m->tok_emb + (size_t)v * d, d) * 1.0f;
  if (m->logit_bias)
    for (int t = 0; t < n; t++)
      for (int v = 0; v < V; v++) logits[(size_t)t * V + v] = logits[(size_t)t * V + v] + m->logit_bias[v];
  if (tmp) orc_cache_destroy(tmp);
  free(x); free(h); free(a); free(f);
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Logit rules and selection: main/nn/WhisperDecoder.java:442-626                               */

static float softmax_at(const float* l, int n, int index) { /* :600-612 */
  float max = -INFINITY;
  for (int i = 0; i < n; i++)
    if (l[i] > max) max = l[i];
  double sum = 0;
  for (int i = 0; i < n; i++) sum += exp((double)(l[i] - max));
  return (float)(exp((double)(l[index] - max)) / sum);
}

static double log_softmax_at(const float* l, int n, int index) { /* :614-626 */
  float max = -INFINITY;
  for (int i = 0; i < n; i++)
    if (l[i] > max) max = l[i];
  double logSum = 0;
  for (int i = 0; i < n; i++) logSum += exp((double)(l[i] - max));
  return (double)(l[index] - max) - log(logSum);
}

double orc_log_softmax_at(const float* l, int n, int index) { return log_softmax_at(l, n, index); }

/* suppressBlank :450-455 */
void orc_suppress_blank(float* l, int n, int eot) {
  l[eot] = -INFINITY;
  if (220 < n) l[220] = -INFINITY;
}

/* applySuppress :457-466 */
void orc_apply_suppress(float* l, const int32_t* s, int ns, int n) {
  if (!s) return;
  for (int i = 0; i < ns; i++)
    if (s[i] >= 0 && s[i] < n) l[s[i]] = -INFINITY;
}

/* applyNgramBlock :543-564 */
void orc_ngram_block(float* l, const int32_t* g, int cnt, int nn, int nvocab) {
  if (cnt < nn - 1) return;
  for (int i = 0; i <= cnt - nn; i++) {
    int match = 1;
    for (int j = 0; j < nn - 1; j++)
      if (g[i + j] != g[cnt - (nn - 1) + j]) { match = 0; break; }
    if (match) {
      int blocked = g[i + nn - 1];
      if (blocked >= 0 && blocked < nvocab) l[blocked] = -INFINITY;
    }
  }
}

/* applyRepetitionPenalty :472-476 */
static void repetition_penalty(float* l, const int32_t* g, int cnt, int nvocab) {
  orc_ngram_block(l, g, cnt, 3, nvocab);
  orc_ngram_block(l, g, cnt, 4, nvocab);
}

/* applyTimestampRules :484-541 */
void orc_timestamp_rules(float* l, const int32_t* g, int cnt, int tsb, int eot, int nvocab, int first) {
  if (tsb > 0 && tsb - 1 >= 0 && tsb - 1 < nvocab) l[tsb - 1] = -INFINITY;
  if (first) {
    for (int i = 0; i < tsb && i < nvocab; i++) l[i] = -INFINITY;
    int lastAllowed = tsb + 50;
    for (int i = lastAllowed + 1; i < nvocab; i++) l[i] = -INFINITY;
    return;
  }
  if (cnt == 0) return;
  int lastWasTs = g[cnt - 1] >= tsb;
  int penultimateWasTs = cnt < 2 || g[cnt - 2] >= tsb;
  if (lastWasTs) {
    if (penultimateWasTs) {
      for (int i = tsb; i < nvocab; i++) l[i] = -INFINITY;
    } else {
      for (int i = 0; i < eot && i < nvocab; i++) l[i] = -INFINITY;
    }
  }
  int lastTs = -1;
  for (int i = cnt - 1; i >= 0; i--)
    if (g[i] >= tsb) { lastTs = g[i]; break; }
  if (lastTs >= 0) {
    int blockUpTo = (lastWasTs && !penultimateWasTs) ? lastTs + 1 : lastTs;
    for (int i = tsb; i < blockUpTo && i < nvocab; i++) l[i] = -INFINITY;
  }
}

/* Math.random() replaced by a seeded SplitMix64 (Steele, Lea and Flood, "Fast splittable
 * pseudorandom number generators", OOPSLA 2014; the constants of Vigna's splitmix64.c) so runs
 * repeat; the reference's draw is unseeded.  The top 53 bits make a double in [0, 1). */
uint64_t orc_splitmix64_next(uint64_t* s) {
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

double orc_rng_uniform(uint64_t* s) { return (double)(orc_splitmix64_next(s) >> 11) * (1.0 / 9007199254740992.0); }

/* sample :576-598 with the uniform draw u given (mutates l: the reference overwrites the logits
 * with the unnormalised probabilities). */
int orc_sample_u(float* l, int n, float temperature, double u) {
  float max = -INFINITY;
  for (int i = 0; i < n; i++)
    if (l[i] > max) max = l[i];
  double sum = 0;
  for (int i = 0; i < n; i++) {
    double p = exp((double)((l[i] - max) / temperature));
    l[i] = (float)p;
    sum += p;
  }
  double r = u * sum;
  double cum = 0;
  for (int i = 0; i < n; i++) {
    cum += l[i];
    if (cum >= r) return i;
  }
  return n - 1;
}

/* needsFallback :435-440 */
int orc_needs_fallback(float compression_ratio, float avg_logprob, float no_speech_prob) {
  if (compression_ratio > 2.4f) return !(no_speech_prob > 0.6f && avg_logprob < -1.0f);
  return avg_logprob < -1.0f && !(no_speech_prob > 0.6f);
}

/* ------------------------------------------------------------------------------------------ */
/* Audio encoder: WhisperEncoder (main/nn/WhisperEncoder.java:27-76).                           */

typedef struct {
  orc_lin q, k, v, o, mlp1, mlp2;
  float *attn_ln_g, *attn_ln_b, *mlp_ln_g, *mlp_ln_b;
} orc_enc_block;

struct orc_encoder {
  orc_enc_dims d;
  float *c1w, *c1b, *c2w, *c2b; /* conv weights [out][in][3] */
  float* pos;                   /* [n_audio_ctx][d] */
  float *lnp_g, *lnp_b;
  orc_enc_block* blocks;
};

/* Conv1d.forward: im2col col[(ic * k + kk)][t] = in[ic][t * stride - pad + kk] (0 outside), then the
 * M>1 tiled matmul weightMatrix [out][in * k] . col (ascending-k sum from 0, main/tensor/Tensor.java:460-489)
 * and addBias rd[oc][t] += bias[oc] (main/nn/Conv1d.java:38-80). */
void orc_conv1d(const float* w, const float* bias, int out_ch, int in_ch, int ksize, int stride, int pad,
                const float* in, int len, float* out) {
  int out_len = (len + 2 * pad - ksize) / stride + 1;
  int rows = in_ch * ksize;
  float* col = (float*)malloc(sizeof(float) * (size_t)rows * out_len);
  for (int t = 0; t < out_len; t++) {
    int start = t * stride - pad;
    for (int ic = 0; ic < in_ch; ic++)
      for (int kk = 0; kk < ksize; kk++) {
        int idx = start + kk;
        col[(size_t)(ic * ksize + kk) * out_len + t] = (idx >= 0 && idx < len) ? in[(size_t)ic * len + idx] : 0.0f;
      }
  }
  for (int oc = 0; oc < out_ch; oc++) {
    float* o = out + (size_t)oc * out_len;
    const float* wr = w + (size_t)oc * rows;
    for (int t = 0; t < out_len; t++) {
      float sum = 0.0f;
      for (int j = 0; j < rows; j++) sum += wr[j] * col[(size_t)j * out_len + t];
      o[t] = sum;
    }
    if (bias)
      for (int t = 0; t < out_len; t++) o[t] += bias[oc];
  }
  free(col);
}

void orc_encoder_destroy(orc_encoder* e) {
  if (!e) return;
  free(e->c1w); free(e->c1b); free(e->c2w); free(e->c2b); free(e->pos); free(e->lnp_g); free(e->lnp_b);
  if (e->blocks) {
    for (int i = 0; i < e->d.n_audio_layer; i++) {
      orc_enc_block* b = &e->blocks[i];
      free_lin(&b->q); free_lin(&b->k); free_lin(&b->v); free_lin(&b->o); free_lin(&b->mlp1); free_lin(&b->mlp2);
      free(b->attn_ln_g); free(b->attn_ln_b); free(b->mlp_ln_g); free(b->mlp_ln_b);
    }
    free(e->blocks);
  }
  free(e);
}

/* WhisperEncoder(WeightStore, ModelDimensions): main/nn/WhisperEncoder.java:27-38, 86-105 */
orc_encoder* orc_encoder_create(const orc_enc_dims* dims, const orc_tensor* tab, int ntab, char* err, int errlen) {
  orc_encoder* e = (orc_encoder*)calloc(1, sizeof(orc_encoder));
  e->d = *dims;
  int d = dims->n_audio_state, nm = dims->n_mels, T = dims->n_audio_ctx;
  char nb[256], bb[256];
#define ELOAD(dst, name, n) do { if (!((dst) = load_f32(tab, ntab, (name), (n), err, errlen))) goto fail; } while (0)
  ELOAD(e->c1w, "encoder.conv1.weight", (int64_t)d * nm * 3);
  ELOAD(e->c1b, "encoder.conv1.bias", d);
  ELOAD(e->c2w, "encoder.conv2.weight", (int64_t)d * d * 3);
  ELOAD(e->c2b, "encoder.conv2.bias", d);
  ELOAD(e->pos, "encoder.positional_embedding", (int64_t)T * d);
  ELOAD(e->lnp_g, "encoder.ln_post.weight", d);
  ELOAD(e->lnp_b, "encoder.ln_post.bias", d);
  e->blocks = (orc_enc_block*)calloc((size_t)dims->n_audio_layer, sizeof(orc_enc_block));
  for (int i = 0; i < dims->n_audio_layer; i++) {
    orc_enc_block* b = &e->blocks[i];
    const char* pj[4] = {"query", "key", "value", "out"};
    orc_lin* lj[4] = {&b->q, &b->k, &b->v, &b->o};
    for (int j = 0; j < 4; j++) {
      snprintf(nb, sizeof nb, "encoder.blocks.%d.attn.%s.weight", i, pj[j]);
      snprintf(bb, sizeof bb, "encoder.blocks.%d.attn.%s.bias", i, pj[j]);
      if (load_lin(lj[j], tab, ntab, nb, bb, d, d, err, errlen)) goto fail;
    }
    snprintf(nb, sizeof nb, "encoder.blocks.%d.mlp.0.weight", i);
    snprintf(bb, sizeof bb, "encoder.blocks.%d.mlp.0.bias", i);
    if (load_lin(&b->mlp1, tab, ntab, nb, bb, d, 4 * d, err, errlen)) goto fail;
    snprintf(nb, sizeof nb, "encoder.blocks.%d.mlp.2.weight", i);
    snprintf(bb, sizeof bb, "encoder.blocks.%d.mlp.2.bias", i);
    if (load_lin(&b->mlp2, tab, ntab, nb, bb, 4 * d, d, err, errlen)) goto fail;
    snprintf(nb, sizeof nb, "encoder.blocks.%d.attn_ln.weight", i);
    ELOAD(b->attn_ln_g, nb, d);
    snprintf(nb, sizeof nb, "encoder.blocks.%d.attn_ln.bias", i);
    ELOAD(b->attn_ln_b, nb, d);
    snprintf(nb, sizeof nb, "encoder.blocks.%d.mlp_ln.weight", i);
    ELOAD(b->mlp_ln_g, nb, d);
    snprintf(nb, sizeof nb, "encoder.blocks.%d.mlp_ln.bias", i);
    ELOAD(b->mlp_ln_b, nb, d);
  }
#undef ELOAD
  return e;
fail:
  orc_encoder_destroy(e);
  return NULL;
}

/* WhisperEncoder.forward: conv1 + gelu, conv2 + gelu, transpose, + positional embedding, blocks
 * (ResidualAttentionBlock.forwardWithAttn with no mask, no cross-attention and no cache:
 * main/nn/ResidualAttentionBlock.java:42-60; MultiHeadAttention.forward qLen > 1 branch:
 * main/nn/MultiHeadAttention.java:84-95), ln_post. */
int orc_encoder_forward(const orc_encoder* e, const float* mel, float* out) {
  int d = e->d.n_audio_state, nm = e->d.n_mels, T = e->d.n_audio_ctx, H = e->d.n_audio_head, hd = 64;
  int F = 2 * T;
  float scale = (float)(1.0 / sqrt((double)hd));
  float* c1 = (float*)malloc(sizeof(float) * (size_t)d * F);
  float* c2 = (float*)malloc(sizeof(float) * (size_t)d * T);
  orc_conv1d(e->c1w, e->c1b, d, nm, 3, 1, 1, mel, F, c1);
  orc_gelu(c1, d * F);
  orc_conv1d(e->c2w, e->c2b, d, d, 3, 2, 1, c1, F, c2);
  orc_gelu(c2, d * T);
  float* x = (float*)malloc(sizeof(float) * (size_t)T * d);
  for (int t = 0; t < T; t++)
    for (int c = 0; c < d; c++) x[(size_t)t * d + c] = c2[(size_t)c * T + t] + e->pos[(size_t)t * d + c];
  free(c1);
  free(c2);
  float* xn = (float*)malloc(sizeof(float) * (size_t)T * d);
  float* q = (float*)malloc(sizeof(float) * (size_t)T * d);
  float* k = (float*)malloc(sizeof(float) * (size_t)T * d);
  float* v = (float*)malloc(sizeof(float) * (size_t)T * d);
  float* qh = (float*)malloc(sizeof(float) * (size_t)T * hd);
  float* kh = (float*)malloc(sizeof(float) * (size_t)T * hd);
  float* vh = (float*)malloc(sizeof(float) * (size_t)T * hd);
  float* w = (float*)malloc(sizeof(float) * (size_t)T * T);
  float* merged = (float*)malloc(sizeof(float) * (size_t)T * d);
  float* o = (float*)malloc(sizeof(float) * (size_t)T * d);
  float* hbuf = (float*)malloc(sizeof(float) * (size_t)T * 4 * d);
  for (int l = 0; l < e->d.n_audio_layer; l++) {
    const orc_enc_block* b = &e->blocks[l];
    orc_layernorm(x, T, d, b->attn_ln_g, b->attn_ln_b, 1e-5f, xn);
    orc_linear(xn, T, d, b->q.wt, d, b->q.b, q);
    orc_linear(xn, T, d, b->k.wt, d, b->k.b, k);
    orc_linear(xn, T, d, b->v.wt, d, b->v.b, v);
    for (int h = 0; h < H; h++) {
      for (int t = 0; t < T; t++)
        for (int c = 0; c < hd; c++) {
          qh[(size_t)t * hd + c] = q[(size_t)t * d + h * hd + c];
          kh[(size_t)t * hd + c] = k[(size_t)t * d + h * hd + c];
          vh[(size_t)t * hd + c] = v[(size_t)t * d + h * hd + c];
        }
      /* qr.matmulTransB(kr, scale): lane dot times scale; softmax rows; attnWeights.matmul(vr) */
      for (int i = 0; i < T; i++)
        for (int j = 0; j < T; j++) w[(size_t)i * T + j] = orc_dot(qh + (size_t)i * hd, kh + (size_t)j * hd, hd) * scale;
      orc_softmax_rows(w, T, T);
      for (int i = 0; i < T; i++) {
        float* mo = merged + (size_t)i * d + h * hd;
        for (int c = 0; c < hd; c++) mo[c] = 0.0f;
        for (int j = 0; j < T; j++) {
          float p = w[(size_t)i * T + j];
          const float* vv = vh + (size_t)j * hd;
          for (int c = 0; c < hd; c++) mo[c] = mo[c] + p * vv[c];
        }
      }
    }
    orc_linear(merged, T, d, b->o.wt, d, b->o.b, o);
    for (size_t i = 0; i < (size_t)T * d; i++) x[i] = o[i] + x[i]; /* attnOut.addInPlace(x) */
    orc_layernorm(x, T, d, b->mlp_ln_g, b->mlp_ln_b, 1e-5f, xn);
    orc_linear(xn, T, d, b->mlp1.wt, 4 * d, b->mlp1.b, hbuf);
    orc_gelu(hbuf, T * 4 * d);
    orc_linear(hbuf, T, 4 * d, b->mlp2.wt, d, b->mlp2.b, o);
    for (size_t i = 0; i < (size_t)T * d; i++) x[i] = x[i] + o[i]; /* result.addInPlace(mlpOut) */
  }
  orc_layernorm(x, T, d, e->lnp_g, e->lnp_b, 1e-5f, out);
  free(x); free(xn); free(q); free(k); free(v); free(qh); free(kh); free(vh); free(w); free(merged); free(o); free(hbuf);
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Decode drivers over a logits source.  The model-backed source below runs orc_forward with one
 * KV cache per hypothesis; tests drive the same drivers from hand-built logit tables.           */

/* WhisperDecoder.decode: main/nn/WhisperDecoder.java:161-204 */
int orc_greedy_drive(const orc_ops* ops, int V, int eot, int max_tokens, const int32_t* suppress, int n_suppress,
                     int no_speech, float temperature, int ts_begin, uint64_t seed, orc_result* out) {
  if (max_tokens > 1024 || max_tokens < 0) return -3;
  int32_t generated[1024];
  int genCount = 0;
  double sumLogprob = 0;
  float noSpeechProb = 0;
  uint64_t rng = seed;
  float* first = (float*)malloc(sizeof(float) * (size_t)V);
  float* last = (float*)malloc(sizeof(float) * (size_t)V);
  int rc = 0;
  for (int step = 0; step < max_tokens; step++) {
    rc = step == 0 ? ops->prefill(ops->ctx, first, last) : ops->step(ops->ctx, 0, generated[genCount - 1], last);
    if (rc) break;
    if (step == 0) {
      /* collectNoSpeechProb reads logits row 0 (:442-448) */
      noSpeechProb = (no_speech < 0 || no_speech >= V) ? 0.0f : softmax_at(first, V, no_speech);
      orc_suppress_blank(last, V, eot);
    }
    orc_apply_suppress(last, suppress, n_suppress, V);
    repetition_penalty(last, generated, genCount, V);
    if (ts_begin > 0) orc_timestamp_rules(last, generated, genCount, ts_begin, eot, V, step == 0);
    int best = temperature == 0.0f ? orc_argmax(last, V) : orc_sample_u(last, V, temperature, orc_rng_uniform(&rng));
    sumLogprob += log_softmax_at(last, V, best);
    if (best == eot) break;
    generated[genCount++] = best;
  }
  free(first);
  free(last);
  if (rc) return rc;
  out->n_tokens = genCount;
  memcpy(out->tokens, generated, sizeof(int32_t) * (size_t)genCount);
  out->avg_logprob = genCount > 0 ? (float)(sumLogprob / genCount) : 0.0f;
  out->compression_ratio = orc_compression_ratio(generated, genCount);
  out->no_speech_prob = noSpeechProb;
  out->temperature = temperature;
  return 0;
}

typedef struct {
  double score;
  int beam, tok;
} cand_t;

/* WhisperDecoder.decodeBeam: main/nn/WhisperDecoder.java:214-394 */
int orc_beam_drive(const orc_ops* ops, int V, int eot, int max_tokens, const int32_t* suppress, int n_suppress,
                   int no_speech, int ts_begin, int beam, orc_result* out, double* gaps) {
  if (max_tokens > 1024 || max_tokens < 1 || beam < 1 || beam > 16) return -3;
  int32_t(*toks)[1024] = calloc((size_t)beam, sizeof(*toks));
  int* lens = (int*)calloc((size_t)beam, sizeof(int));
  double* lps = (double*)calloc((size_t)beam, sizeof(double));
  int maxfin = beam + 1;
  int32_t(*fin_t)[1024] = calloc((size_t)maxfin, sizeof(*fin_t));
  int* fin_len = (int*)calloc((size_t)maxfin, sizeof(int));
  double* fin_lp = (double*)calloc((size_t)maxfin, sizeof(double));
  int nfin = 0;
  float* first = (float*)malloc(sizeof(float) * (size_t)V);
  float* logits = (float*)malloc(sizeof(float) * (size_t)V);
  float* lp = (float*)malloc(sizeof(float) * (size_t)V);
  int32_t* top = (int32_t*)malloc(sizeof(int32_t) * (size_t)(beam + 1));
  cand_t* cands = (cand_t*)malloc(sizeof(cand_t) * (size_t)beam * (beam + 1));
  int32_t(*ntoks)[1024] = calloc((size_t)beam, sizeof(*ntoks));
  int* nlens = (int*)calloc((size_t)beam, sizeof(int));
  double* nlps = (double*)calloc((size_t)beam, sizeof(double));
  int32_t* src = (int32_t*)calloc((size_t)beam, sizeof(int32_t));
  float noSpeechProb = 0.0f;
  if (gaps)
    for (int i = 0; i < max_tokens; i++) gaps[i] = INFINITY;
  int rc = ops->prefill(ops->ctx, first, logits);
  if (rc) goto done;
  noSpeechProb = (no_speech < 0 || no_speech >= V) ? 0.0f : softmax_at(first, V, no_speech);
  orc_suppress_blank(logits, V, eot);
  orc_apply_suppress(logits, suppress, n_suppress, V);
  orc_log_softmax(logits, V, lp);
  orc_topk(lp, V, beam, top);
  for (int b = 0; b < beam; b++) {
    toks[b][0] = top[b];
    lens[b] = 1;
    lps[b] = (double)lp[top[b]];
    src[b] = 0; /* every beam starts from the prompt's cache (:260-266) */
  }
  if ((rc = ops->rearrange(ops->ctx, src, beam, beam))) goto done;
  for (int step = 1; step < max_tokens; step++) {
    int nc = 0;
    for (int b = 0; b < beam; b++) {
      if (toks[b][lens[b] - 1] == eot) continue;
      if ((rc = ops->step(ops->ctx, b, toks[b][lens[b] - 1], logits))) goto done;
      orc_apply_suppress(logits, suppress, n_suppress, V);
      repetition_penalty(logits, toks[b], lens[b], V);
      if (ts_begin > 0) orc_timestamp_rules(logits, toks[b], lens[b], ts_begin, eot, V, 0);
      orc_log_softmax(logits, V, lp);
      orc_topk(lp, V, beam + 1, top);
      for (int k = 0; k < beam + 1; k++) {
        cands[nc].score = lps[b] + (double)lp[top[k]];
        cands[nc].beam = b;
        cands[nc].tok = top[k];
        nc++;
      }
    }
    if (nc == 0) break;
    /* candidates.sort(descending): stable insertion sort on double scores (List.sort is stable) */
    for (int i = 1; i < nc; i++) {
      cand_t c = cands[i];
      int j = i - 1;
      while (j >= 0 && cands[j].score < c.score) {
        cands[j + 1] = cands[j];
        j--;
      }
      cands[j + 1] = c;
    }
    int saved = 0;
    for (int ci = 0; ci < nc; ci++) {
      int sb = cands[ci].beam, tok = cands[ci].tok;
      double score = cands[ci].score;
      /* decision margin of this step: the last hypothesis kept against the first non-end candidate
       * left out (test instrumentation, not part of the reference's algorithm) */
      if (gaps && tok != eot && saved == beam && gaps[step] == INFINITY) gaps[step] = nlps[beam - 1] - score;
      if (tok == eot) {
        memcpy(fin_t[nfin], toks[sb], sizeof(int32_t) * (size_t)lens[sb]);
        fin_len[nfin] = lens[sb];
        fin_lp[nfin] = score;
        nfin++;
        if (nfin >= beam) break;
        continue;
      }
      if (saved >= beam) continue;
      memcpy(ntoks[saved], toks[sb], sizeof(int32_t) * (size_t)lens[sb]);
      ntoks[saved][lens[sb]] = tok;
      nlens[saved] = lens[sb] + 1;
      nlps[saved] = score;
      src[saved] = sb;
      saved++;
    }
    if (saved == 0 || nfin >= beam) break;
    for (int b = saved; b < beam; b++) { /* leftover beams continue new beam 0 (:356-361) */
      memcpy(ntoks[b], ntoks[0], sizeof(int32_t) * (size_t)nlens[0]);
      nlens[b] = nlens[0];
      nlps[b] = nlps[0];
      src[b] = -1;
    }
    if ((rc = ops->rearrange(ops->ctx, src, saved, beam))) goto done;
    memcpy(toks, ntoks, sizeof(*toks) * (size_t)beam);
    memcpy(lens, nlens, sizeof(int) * (size_t)beam);
    memcpy(lps, nlps, sizeof(double) * (size_t)beam);
  }
  for (int b = 0; b < beam && nfin < beam; b++) { /* unfinished beams fill the list (:370-377) */
    memcpy(fin_t[nfin], toks[b], sizeof(int32_t) * (size_t)lens[b]);
    fin_len[nfin] = lens[b];
    fin_lp[nfin] = lps[b];
    nfin++;
  }
  {
    int bestIdx = 0;
    double bestScore = -INFINITY, second = -INFINITY;
    for (int i = 0; i < nfin; i++) { /* MaximumLikelihoodRanker (:379-388) */
      double score = fin_lp[i] / (double)(fin_len[i] > 1 ? fin_len[i] : 1);
      if (score > bestScore) {
        second = bestScore;
        bestScore = score;
        bestIdx = i;
      } else if (score > second) {
        second = score;
      }
    }
    if (gaps) gaps[0] = bestScore - second; /* margin of the final pick */
    out->n_tokens = fin_len[bestIdx];
    memcpy(out->tokens, fin_t[bestIdx], sizeof(int32_t) * (size_t)fin_len[bestIdx]);
    out->avg_logprob = fin_len[bestIdx] > 0 ? (float)(fin_lp[bestIdx] / fin_len[bestIdx]) : 0.0f;
    out->compression_ratio = orc_compression_ratio(out->tokens, out->n_tokens);
    out->no_speech_prob = noSpeechProb;
    out->temperature = 0.0f;
  }
done:
  free(toks); free(lens); free(lps); free(fin_t); free(fin_len); free(fin_lp);
  free(first); free(logits); free(lp); free(top); free(cands);
  free(ntoks); free(nlens); free(nlps); free(src);
  return rc;
}

/* decodeWithFallback's loop (main/nn/WhisperDecoder.java:119-149) as a state machine: feed the
 * result decoded at temps[i]; returns 1 when the loop ends (result in *best), 0 to continue with
 * temps[i + 1]. */
static const float kTemps[6] = {0.0f, 0.2f, 0.4f, 0.6f, 0.8f, 1.0f};
static int fallback_feed(const orc_result* cur, float t, orc_result* best, int* have) {
  if (!orc_needs_fallback(cur->compression_ratio, cur->avg_logprob, cur->no_speech_prob)) {
    *best = *cur;
    return 1;
  }
  if (!*have || cur->avg_logprob > best->avg_logprob) {
    *best = *cur;
    *have = 1;
  }
  if (t == 0.0f && cur->compression_ratio <= 2.4f) return 1;
  if (t > 0.0f && cur->avg_logprob < best->avg_logprob - 1.0f) return 1;
  return 0;
}

/* The fallback choice over results already decoded at 0, 0.2, .., 1.0: index of the result
 * decodeWithFallback returns, and in *n_used how many decodes it would have run. */
int orc_fallback_pick(const orc_result* per_temp, int* n_used) {
  orc_result best;
  int have = 0, i = 0, pick = -1;
  for (; i < 6; i++) {
    if (fallback_feed(&per_temp[i], kTemps[i], &best, &have)) {
      i++;
      break;
    }
  }
  for (int j = 0; j < 6; j++)
    if (memcmp(&per_temp[j], &best, sizeof best) == 0) { pick = j; break; }
  if (n_used) *n_used = i;
  return pick;
}

/* ---- the model-backed logits source ---- */
typedef struct {
  const orc_model* m;
  const float* xa;
  const int32_t* prompt;
  int n_prompt, n;
  orc_cache** caches; /* [n] */
  float* rows;        /* [n_prompt][V] */
} model_src;

static int ms_prefill(void* ctx, float* first, float* last) {
  model_src* s = (model_src*)ctx;
  int V = s->m->d.n_vocab;
  int rc = orc_forward(s->m, s->prompt, s->n_prompt, s->xa, s->caches[0], s->rows);
  if (rc) return rc;
  memcpy(first, s->rows, sizeof(float) * (size_t)V);
  memcpy(last, s->rows + (size_t)(s->n_prompt - 1) * V, sizeof(float) * (size_t)V);
  return 0;
}

static int ms_step(void* ctx, int b, int32_t token, float* out) {
  model_src* s = (model_src*)ctx;
  return orc_forward(s->m, &token, 1, s->xa, s->caches[b], out);
}

/* Beam cache rearrangement (:342-361): hypothesis b continues src[b]'s map (the same map when
 * src[b] == b, a copy sharing the tensors otherwise); src[b] < 0 aliases new hypothesis 0's map. */
static int ms_rearrange(void* ctx, const int32_t* src, int saved, int beam) {
  model_src* s = (model_src*)ctx;
  orc_cache** nc = (orc_cache**)calloc((size_t)beam, sizeof(orc_cache*));
  for (int b = 0; b < saved; b++) {
    if (src[b] == b) {
      nc[b] = s->caches[b];
      s->caches[b]->refs++;
    } else {
      nc[b] = cache_copy(s->caches[src[b]]);
    }
  }
  for (int b = saved; b < beam; b++) {
    nc[b] = nc[0];
    nc[0]->refs++;
  }
  for (int b = 0; b < beam; b++) orc_cache_destroy(s->caches[b]);
  free(s->caches);
  s->caches = nc;
  return 0;
}

static void ms_init(model_src* s, orc_ops* ops, const orc_model* m, const float* xa, const int32_t* prompt,
                    int n_prompt, int n) {
  s->m = m;
  s->xa = xa;
  s->prompt = prompt;
  s->n_prompt = n_prompt;
  s->n = n;
  s->caches = (orc_cache**)calloc((size_t)n, sizeof(orc_cache*));
  s->caches[0] = orc_cache_create(m);
  for (int b = 1; b < n; b++) { /* every map starts empty (:223-229) */
    s->caches[b] = orc_cache_create(m);
  }
  s->rows = (float*)malloc(sizeof(float) * (size_t)(n_prompt > 0 ? n_prompt : 1) * m->d.n_vocab);
  ops->ctx = s;
  ops->prefill = ms_prefill;
  ops->step = ms_step;
  ops->rearrange = ms_rearrange;
}

static void ms_free(model_src* s) {
  for (int b = 0; b < s->n; b++) orc_cache_destroy(s->caches[b]);
  free(s->caches);
  free(s->rows);
}

int orc_decode(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot, int max_tokens,
               const int32_t* suppress, int n_suppress, int no_speech, float temperature, int ts_begin,
               uint64_t seed, orc_result* out) {
  if (n_prompt < 1) return -3;
  model_src s;
  orc_ops ops;
  ms_init(&s, &ops, m, xa, prompt, n_prompt, 1);
  int rc = orc_greedy_drive(&ops, m->d.n_vocab, eot, max_tokens, suppress, n_suppress, no_speech, temperature,
                            ts_begin, seed, out);
  ms_free(&s);
  return rc;
}

int orc_decode_beam(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot,
                    int max_tokens, const int32_t* suppress, int n_suppress, int no_speech, int ts_begin, int beam,
                    orc_result* out) {
  if (n_prompt < 1 || beam < 1 || beam > 16) return -3;
  model_src s;
  orc_ops ops;
  ms_init(&s, &ops, m, xa, prompt, n_prompt, beam);
  int rc = orc_beam_drive(&ops, m->d.n_vocab, eot, max_tokens, suppress, n_suppress, no_speech, ts_begin, beam, out,
                          NULL);
  ms_free(&s);
  return rc;
}

int orc_decode_beam_gaps(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot,
                         int max_tokens, const int32_t* suppress, int n_suppress, int no_speech, int ts_begin, int beam,
                         orc_result* out, double* gaps) {
  if (n_prompt < 1 || beam < 1 || beam > 16) return -3;
  model_src s;
  orc_ops ops;
  ms_init(&s, &ops, m, xa, prompt, n_prompt, beam);
  int rc = orc_beam_drive(&ops, m->d.n_vocab, eot, max_tokens, suppress, n_suppress, no_speech, ts_begin, beam, out,
                          gaps);
  ms_free(&s);
  return rc;
}

/* WhisperDecoder.decodeWithFallback: main/nn/WhisperDecoder.java:119-149 (the sampling draws of
 * temperature i use seed + i). */
int orc_decode_with_fallback(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot,
                             int max_tokens, const int32_t* suppress, int n_suppress, int no_speech, int ts_begin,
                             int beam, uint64_t seed, orc_result* out) {
  orc_result cur, best;
  int have = 0;
  for (int i = 0; i < 6; i++) {
    float t = kTemps[i];
    int rc = (beam > 1 && t == 0.0f)
                 ? orc_decode_beam(m, xa, prompt, n_prompt, eot, max_tokens, suppress, n_suppress, no_speech, ts_begin,
                                   beam, &cur)
                 : orc_decode(m, xa, prompt, n_prompt, eot, max_tokens, suppress, n_suppress, no_speech, t, ts_begin,
                              seed + (uint64_t)i, &cur);
    if (rc) return rc;
    if (fallback_feed(&cur, t, &best, &have)) break;
  }
  *out = best;
  return 0;
}
/* Teacher-forced greedy sweep (the workload of the parity tests and the CPU baseline). */
int orc_forced(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, const int32_t* forced,
               int n_steps, int32_t* argmax_out, float* max_out, float* second_out, float* lse_out,
               float* logits_out) {
  int V = m->d.n_vocab;
  orc_cache* cache = orc_cache_create(m);
  float* logits = (float*)malloc(sizeof(float) * (size_t)(n_prompt > 1 ? n_prompt : 1) * V);
  int rc = 0;
  for (int r = 0; r <= n_steps; r++) {
    const int32_t* tk = r == 0 ? prompt : &forced[r - 1];
    int n = r == 0 ? n_prompt : 1;
    if ((rc = orc_forward(m, tk, n, xa, cache, logits))) break;
    const float* row = logits + (size_t)(n - 1) * V;
    int am = orc_argmax(row, V);
    float mx = row[am], sec = -INFINITY;
    double s = 0;
    for (int i = 0; i < V; i++) {
      if (i != am && row[i] > sec) sec = row[i];
      s += exp((double)(row[i] - mx));
    }
    if (argmax_out) argmax_out[r] = am;
    if (max_out) max_out[r] = mx;
    if (second_out) second_out[r] = sec;
    if (lse_out) lse_out[r] = (float)((double)mx + log(s));
    if (logits_out) memcpy(logits_out + (size_t)r * V, row, sizeof(float) * (size_t)V);
  }
  free(logits);
  orc_cache_destroy(cache);
  return rc;
}
