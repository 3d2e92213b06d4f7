// Device code of whisper4j_amd for gfx950 (CDNA4, wave64).
//
// The decoder step runs as ONE persistent cooperative kernel (k_step) per launch, covering one or
// more token steps.  Work inside a step is a chain of phases per layer
//     QKV -> self-attention -> out-proj -> cross-q -> cross-attention -> cross-out -> MLP1 -> MLP2
// then the logits phase and a selection reduction.  Workgroups hand results to the next phase
// through "tagged" 64-bit words: the low 32 bits hold an fp32 value, the high 32 bits the step tag.
// A consumer polls the words it needs with agent-scope loads until every tag matches, so a hop
// costs one write-through store plus one polled load, with no grid barrier, no counter atomics and
// no cache-wide fence on the data path.  Each workgroup issues the weight loads of its next work
// item before it starts polling, so weight streaming overlaps the hop latency.  Every wait is
// bounded: on expiry the workgroup raises an error flag and all workgroups leave the kernel.
//
// The same __device__ building blocks (GEMV over 8 rows, LayerNorm, attention chunk, selection)
// back the standalone op kernels used by the kernel-level entry points.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>

#include "w4h_internal.h"

namespace w4h {

#define DEV __device__ __forceinline__

constexpr unsigned kSpinLimit = 1u << 20;  // polls before a wait is declared expired (~1 s)
constexpr int PFR = 8;  // 16-byte weight chunks per lane kept in registers (prefetched) per item
constexpr int PFL = 8;  // the same for the logits phase (rows of the tied embedding)
constexpr int KPT_SELF = kSelfChunk / 32;   // keys per thread, self-attention chunk
constexpr int KPT_CROSS = kMaxChunk / 32;   // keys per thread, cross-attention chunk
constexpr int kPollBatch = 8;  // tagged words each thread loads before checking tags
constexpr int kRedBlock = 64;   // selection partials merged per block by the output workgroup

// ------------------------------------------------------------------------------------------------
// small helpers

DEV float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
DEV uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }
DEV float2 h2x2(uint32_t u) {
  __half2 h;
  __builtin_memcpy(&h, &u, 4);
  return __half22float2(h);
}

DEV u64 ll_ld(const u64* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void ll_st(u64* p, float v, uint32_t tag) {
  __hip_atomic_store(p, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV bool aborted(const unsigned* err) {
  return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
DEV void raise_err(unsigned* err, unsigned code) {
  __hip_atomic_fetch_or(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
// (value, index) maximum; equal values keep the lower index.  NaN never wins.
DEV void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(v, o);
    int oi = __shfl_xor(i, o);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// Sum over the workgroup; every thread receives the result.  scratch: 4 floats of LDS.
DEV float wg_sum(float v, float* scratch) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

// ------------------------------------------------------------------------------------------------
// tagged-word polling

// Poll words [0, n0) of src0 and [0, n1) of src1 until every word carries `tag`, then copy the
// values into dst0 / dst1 (LDS).  Returns false (uniformly across the workgroup) when the wait
// expired or another workgroup aborted.
DEV bool ll_poll2(const u64* src0, int n0, float* dst0, const u64* src1, int n1, float* dst1, uint32_t tag,
                  unsigned* err) {
  const int total = n0 + n1;
  bool fail = false;
  for (int base = 0; base < total && !fail; base += kThreads * kPollBatch) {
    u64 v[kPollBatch];
#pragma unroll
    for (int u = 0; u < kPollBatch; ++u) {
      const int i = base + u * kThreads + (int)threadIdx.x;
      v[u] = i < n0 ? ll_ld(src0 + i) : (i < total ? ll_ld(src1 + (i - n0)) : ((u64)tag << 32));
    }
    unsigned spins = 0;
    while (true) {
      bool ok = true;
#pragma unroll
      for (int u = 0; u < kPollBatch; ++u)
        if ((uint32_t)(v[u] >> 32) != tag) {
          const int i = base + u * kThreads + (int)threadIdx.x;
          ok = false;
          v[u] = i < n0 ? ll_ld(src0 + i) : ll_ld(src1 + (i - n0));
        }
      if (ok) break;
      ++spins;
      if (spins > kSpinLimit) {
        raise_err(err, 1u);
        fail = true;
        break;
      }
      if ((spins & 63u) == 0 && aborted(err)) {
        fail = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!fail) {
#pragma unroll
      for (int u = 0; u < kPollBatch; ++u) {
        const int i = base + u * kThreads + (int)threadIdx.x;
        if (i < n0)
          dst0[i] = __uint_as_float((uint32_t)v[u]);
        else if (i < total)
          dst1[i - n0] = __uint_as_float((uint32_t)v[u]);
      }
    }
  }
  return !__syncthreads_or(fail);
}

DEV bool ll_poll1(const u64* src, int n, float* dst, uint32_t tag, unsigned* err) {
  return ll_poll2(src, n, dst, nullptr, 0, nullptr, tag, err);
}

// ------------------------------------------------------------------------------------------------
// GEMV over one item of 8 weight rows, for up to SM activation rows held in LDS.
//
// Lane layout (256 threads): wave w, lane l -> weight row r0 + (l >> 3), slot (w << 3) | (l & 7).
// A row is cut into 16-byte chunks (8 halves for f16, 16 int8 for q8_0); slot j takes chunks
// j, j+32, j+64, ...  Eight adjacent lanes therefore read 128 contiguous bytes of one row.
// Partial dots are reduced over the 8 lanes with xor-shuffles and over the 4 waves through LDS.

template <int R>
struct WRegs {
  uint4 w[R];
  uint16_t s[R];
};

template <int R, int WQ8>
DEV void gemv_prefetch(const void* W, const uint16_t* Ws, int N, int K, int r0, WRegs<R>& wr) {
  const int tid = threadIdx.x, lane = tid & 63, row = lane >> 3, slot = ((tid >> 6) << 3) | (lane & 7);
  const int gr = r0 + row;
  if (gr >= N) return;
  if (!WQ8) {
    const int nch = K >> 3;
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(W) + (size_t)gr * K);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int c = slot + 32 * r;
      if (c < nch) wr.w[r] = src[c];
    }
  } else {
    const int nch = K >> 4;
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const int8_t*>(W) + (size_t)gr * K);
    const uint16_t* ss = Ws + (size_t)gr * (K >> 5);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int c = slot + 32 * r;
      if (c < nch) {
        wr.w[r] = src[c];
        wr.s[r] = ss[c >> 1];
      }
    }
  }
}

DEV float dot8_f16(const uint4& w, const float* x) {
  const float4 a = *reinterpret_cast<const float4*>(x);
  const float4 b = *reinterpret_cast<const float4*>(x + 4);
  float2 w0 = h2x2(w.x), w1 = h2x2(w.y), w2 = h2x2(w.z), w3 = h2x2(w.w);
  float s = w0.x * a.x;
  s = fmaf(w0.y, a.y, s);
  s = fmaf(w1.x, a.z, s);
  s = fmaf(w1.y, a.w, s);
  s = fmaf(w2.x, b.x, s);
  s = fmaf(w2.y, b.y, s);
  s = fmaf(w3.x, b.z, s);
  s = fmaf(w3.y, b.w, s);
  return s;
}

DEV float dot16_q8(const uint4& w, const float* x) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 a = *reinterpret_cast<const float4*>(x + 4 * k);
    s = fmaf((float)(int8_t)(u[k] & 0xff), a.x, s);
    s = fmaf((float)(int8_t)((u[k] >> 8) & 0xff), a.y, s);
    s = fmaf((float)(int8_t)((u[k] >> 16) & 0xff), a.z, s);
    s = fmaf((float)(int8_t)(u[k] >> 24), a.w, s);
  }
  return s;
}

// out[s*8 + r] = sum_k W[r0 + r][k] * x[s*K + k] for s < S (LDS in, LDS out).  Chunks of the
// prefetched rounds come from registers; later rounds of long rows are loaded here.
template <int R, int WQ8, int SM>
DEV void gemv_compute(const WRegs<R>& wr, const void* W, const uint16_t* Ws, int N, int K, int r0, int S,
                      const float* x, float* red, float* out) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, row = lane >> 3, sub = lane & 7;
  const int slot = (w << 3) | sub;
  const int gr = r0 + row;
  float acc[SM];
#pragma unroll
  for (int s = 0; s < SM; ++s) acc[s] = 0.f;
  if (gr < N) {
    if (!WQ8) {
      const int nch = K >> 3;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int c = slot + 32 * r;
        if (c < nch) {
#pragma unroll
          for (int s = 0; s < SM; ++s)
            if (s < S) acc[s] += dot8_f16(wr.w[r], x + s * K + c * 8);
        }
      }
      const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(W) + (size_t)gr * K);
      for (int c = slot + 32 * R; c < nch; c += 32 * 4) {
        uint4 t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c + 32 * u < nch) t[u] = src[c + 32 * u];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c + 32 * u < nch) {
#pragma unroll
            for (int s = 0; s < SM; ++s)
              if (s < S) acc[s] += dot8_f16(t[u], x + s * K + (c + 32 * u) * 8);
          }
      }
    } else {
      const int nch = K >> 4;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int c = slot + 32 * r;
        if (c < nch) {
          const float sc = h2f(wr.s[r]);
#pragma unroll
          for (int s = 0; s < SM; ++s)
            if (s < S) acc[s] = fmaf(sc, dot16_q8(wr.w[r], x + s * K + c * 16), acc[s]);
        }
      }
      const uint4* src = reinterpret_cast<const uint4*>(static_cast<const int8_t*>(W) + (size_t)gr * K);
      const uint16_t* ss = Ws + (size_t)gr * (K >> 5);
      for (int c = slot + 32 * R; c < nch; c += 32 * 4) {
        uint4 t[4];
        uint16_t ts[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c + 32 * u < nch) {
            t[u] = src[c + 32 * u];
            ts[u] = ss[(c + 32 * u) >> 1];
          }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c + 32 * u < nch) {
            const float sc = h2f(ts[u]);
#pragma unroll
            for (int s = 0; s < SM; ++s)
              if (s < S) acc[s] = fmaf(sc, dot16_q8(t[u], x + s * K + (c + 32 * u) * 16), acc[s]);
          }
      }
    }
  }
#pragma unroll
  for (int s = 0; s < SM; ++s) {
    acc[s] += __shfl_xor(acc[s], 1);
    acc[s] += __shfl_xor(acc[s], 2);
    acc[s] += __shfl_xor(acc[s], 4);
  }
  if (sub == 0) {
#pragma unroll
    for (int s = 0; s < SM; ++s)
      if (s < S) red[((w << 3) + row) * SM + s] = acc[s];
  }
  __syncthreads();
  if (tid < 8 * S) {
    const int s = tid >> 3, rr = tid & 7;
    out[s * 8 + rr] = (red[rr * SM + s] + red[(8 + rr) * SM + s]) + (red[(16 + rr) * SM + s] + red[(24 + rr) * SM + s]);
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------
// LayerNorm over S rows of d (LDS in, LDS out), eps 1e-5, two passes.

DEV void wg_layernorm(const float* x, float* y, int S, int d, const float* g, const float* b, float* scratch) {
  for (int s = 0; s < S; ++s) {
    const float* xs = x + s * d;
    float a = 0.f;
    for (int i = threadIdx.x; i < d; i += kThreads) a += xs[i];
    const float mean = wg_sum(a, scratch) / (float)d;
    float v = 0.f;
    for (int i = threadIdx.x; i < d; i += kThreads) {
      float t = xs[i] - mean;
      v = fmaf(t, t, v);
    }
    const float var = wg_sum(v, scratch) / (float)d;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    for (int i = threadIdx.x; i < d; i += kThreads) y[s * d + i] = (xs[i] - mean) * inv * g[i] + b[i];
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------
// Attention of ns query rows over one chunk of keys.
//
// Keys [0, n) are f16 rows of 64 halves at kb + off(j) / vb + off(j).  When kx != null one more key
// (index n) is the current token's fp32 key/value in LDS (one query row).  Scores and the AV
// product use 8 lanes per key row (16 bytes each); 32 key groups per workgroup.
// Result: pm[s] = max score, pl[s] = sum exp(score - max), acc[s*64 + e] = sum p * v.

template <int KPT>
struct KVRegs {
  uint4 k[KPT];
  uint4 v[KPT];
};

template <int KPT, class Off>
DEV void attn_prefetch(const uint16_t* kb, const uint16_t* vb, Off off, int n, KVRegs<KPT>& r) {
  const int sub = threadIdx.x & 7, kg = threadIdx.x >> 3;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    int j = kg + 32 * i;
    if (j < n) {
      size_t o = off(j) + (size_t)sub * 8;
      r.k[i] = *reinterpret_cast<const uint4*>(kb + o);
      r.v[i] = *reinterpret_cast<const uint4*>(vb + o);
    }
  }
}

template <int KPT, int SM>
DEV void attn_compute(const KVRegs<KPT>& r, int n, int ns, const float* q, const float* kx, const float* vx,
                      float scale, float* sc, int scs, float* red, float* pm, float* pl, float* acc_out) {
  const int tid = threadIdx.x, sub = tid & 7, kg = tid >> 3, w = tid >> 6, lane = tid & 63;
  // scores
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int j = kg + 32 * i;
    float part[SM];
#pragma unroll
    for (int s = 0; s < SM; ++s) part[s] = 0.f;
    if (j < n) {
#pragma unroll
      for (int s = 0; s < SM; ++s)
        if (s < ns) part[s] = dot8_f16(r.k[i], q + s * kHeadDim + sub * 8);
    }
#pragma unroll
    for (int s = 0; s < SM; ++s) {
      part[s] += __shfl_xor(part[s], 1);
      part[s] += __shfl_xor(part[s], 2);
      part[s] += __shfl_xor(part[s], 4);
    }
    if (sub == 0 && j < n) {
#pragma unroll
      for (int s = 0; s < SM; ++s)
        if (s < ns) sc[s * scs + j] = part[s] * scale;
    }
  }
  if (kx != nullptr && w == 0) {
    for (int s = 0; s < ns; ++s) {
      float t = wave_sum(q[s * kHeadDim + lane] * kx[lane]);
      if (lane == 0) sc[s * scs + n] = t * scale;
    }
  }
  __syncthreads();
  const int nt = n + (kx != nullptr ? 1 : 0);
  // softmax statistics, one wave per query row
  for (int s = w; s < ns; s += 4) {
    float m = -INFINITY;
    for (int j = lane; j < nt; j += 64) m = fmaxf(m, sc[s * scs + j]);
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < nt; j += 64) {
      float e = __expf(sc[s * scs + j] - m);
      sc[s * scs + j] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      pm[s] = m;
      pl[s] = l;
    }
  }
  __syncthreads();
  // AV
  float a[SM][8];
#pragma unroll
  for (int s = 0; s < SM; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) a[s][e] = 0.f;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int j = kg + 32 * i;
    if (j < n) {
      float2 v0 = h2x2(r.v[i].x), v1 = h2x2(r.v[i].y), v2 = h2x2(r.v[i].z), v3 = h2x2(r.v[i].w);
#pragma unroll
      for (int s = 0; s < SM; ++s)
        if (s < ns) {
          const float p = sc[s * scs + j];
          a[s][0] = fmaf(p, v0.x, a[s][0]);
          a[s][1] = fmaf(p, v0.y, a[s][1]);
          a[s][2] = fmaf(p, v1.x, a[s][2]);
          a[s][3] = fmaf(p, v1.y, a[s][3]);
          a[s][4] = fmaf(p, v2.x, a[s][4]);
          a[s][5] = fmaf(p, v2.y, a[s][5]);
          a[s][6] = fmaf(p, v3.x, a[s][6]);
          a[s][7] = fmaf(p, v3.y, a[s][7]);
        }
    }
  }
#pragma unroll
  for (int s = 0; s < SM; ++s)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[s][e] += __shfl_xor(a[s][e], 8);
      a[s][e] += __shfl_xor(a[s][e], 16);
      a[s][e] += __shfl_xor(a[s][e], 32);
    }
  if (lane < 8) {
#pragma unroll
    for (int s = 0; s < SM; ++s)
      if (s < ns)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[(w * SM + s) * kHeadDim + sub * 8 + e] = a[s][e];
  }
  __syncthreads();
  for (int i = tid; i < ns * kHeadDim; i += kThreads) {
    const int s = i >> 6, e = i & 63;
    float o = (red[(0 * SM + s) * kHeadDim + e] + red[(1 * SM + s) * kHeadDim + e]) +
              (red[(2 * SM + s) * kHeadDim + e] + red[(3 * SM + s) * kHeadDim + e]);
    if (kx != nullptr) o = fmaf(sc[s * scs + n], vx[e], o);
    acc_out[i] = o;
  }
  __syncthreads();
}

// Merge attention partials: part[(c * nrow + row) * kPartWords + w] for c < nc -> o[row*64 + e].
DEV void attn_merge(const float* part, int nc, int nrow, float* o) {
  for (int i = threadIdx.x; i < nrow * kHeadDim; i += kThreads) {
    const int row = i >> 6, e = i & 63;
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, part[(c * nrow + row) * kPartWords]);
    float Lsum = 0.f, acc = 0.f;
    for (int c = 0; c < nc; ++c) {
      const float* pp = part + (c * nrow + row) * kPartWords;
      const float f = __expf(pp[0] - M);
      Lsum = fmaf(pp[1], f, Lsum);
      acc = fmaf(pp[2 + e], f, acc);
    }
    o[i] = acc / Lsum;
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------
// Selection.  A workgroup partial over its rows (lg masked, rw raw logits, idx global ids) is
// kSelWords floats: [max, argmax, sumexp(masked - max), raw max, raw sumexp, probe, topk values[8],
// topk ids[8]].  Ties go to the lower vocabulary id everywhere.

DEV void sel_partial(const float* lg, const float* rw, const int* idx, int n, int probe, int topk, float* rec) {
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY, rv = -INFINITY, pv = -INFINITY;
  int bi = 0x7fffffff;
  for (int j = lane; j < n; j += 64) {
    const float v = lg[j];
    const int id = idx[j];
    if (v > bv || (v == bv && id < bi)) {
      bv = v;
      bi = id;
    }
    rv = fmaxf(rv, rw[j]);
    if (id == probe) pv = rw[j];
  }
  wave_argmax(bv, bi);
  rv = wave_max(rv);
  pv = wave_max(pv);
  float se = 0.f, re = 0.f;
  for (int j = lane; j < n; j += 64) {
    if (bv > -INFINITY) se += __expf(lg[j] - bv);
    if (rv > -INFINITY) re += __expf(rw[j] - rv);
  }
  se = wave_sum(se);
  re = wave_sum(re);
  float tv[W4H_TOPK_MAX];
  int ti[W4H_TOPK_MAX];
  for (int k = 0; k < W4H_TOPK_MAX; ++k) {
    tv[k] = -INFINITY;
    ti[k] = 0x7fffffff;
  }
  for (int k = 0; k < topk; ++k) {
    float cv = -INFINITY;
    int ci = 0x7fffffff;
    for (int j = lane; j < n; j += 64) {
      const float v = lg[j];
      const int id = idx[j];
      bool taken = false;
      for (int q = 0; q < k; ++q) taken |= (ti[q] == id);
      if (!taken && v > -INFINITY && (v > cv || (v == cv && id < ci))) {
        cv = v;
        ci = id;
      }
    }
    wave_argmax(cv, ci);
    tv[k] = cv;
    ti[k] = ci;
  }
  if (lane == 0) {
    rec[0] = bv;
    rec[1] = __int_as_float(bi);
    rec[2] = se;
    rec[3] = rv;
    rec[4] = re;
    rec[5] = pv;
    for (int k = 0; k < W4H_TOPK_MAX; ++k) {
      rec[6 + k] = tv[k];
      rec[6 + W4H_TOPK_MAX + k] = __int_as_float(ti[k]);
    }
  }
}

// Argmax over n (max, index) pairs at `stride` floats apart, one wave; every lane gets the result.
DEV int sel_argmax(const float* recs, int n, int stride) {
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int g = lane; g < n; g += 64) {
    const float v = recs[(size_t)g * stride];
    const int id = __float_as_int(recs[(size_t)g * stride + 1]);
    if (v > bv || (v == bv && id < bi)) {
      bv = v;
      bi = id;
    }
  }
  wave_argmax(bv, bi);
  return bi;
}

// Merge n selection partials (stride floats apart) into one partial of the same layout, one wave.
DEV void sel_merge(const float* recs, int n, int stride, int topk, float* out_rec) {
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY, rv = -INFINITY, pv = -INFINITY;
  int bi = 0x7fffffff;
  for (int g = lane; g < n; g += 64) {
    const float* r = recs + (size_t)g * stride;
    const int id = __float_as_int(r[1]);
    if (r[0] > bv || (r[0] == bv && id < bi)) {
      bv = r[0];
      bi = id;
    }
    rv = fmaxf(rv, r[3]);
    pv = fmaxf(pv, r[5]);
  }
  wave_argmax(bv, bi);
  rv = wave_max(rv);
  pv = wave_max(pv);
  float se = 0.f, re = 0.f;
  for (int g = lane; g < n; g += 64) {
    const float* r = recs + (size_t)g * stride;
    if (r[0] > -INFINITY) se += r[2] * __expf(r[0] - bv);
    if (r[3] > -INFINITY) re += r[4] * __expf(r[3] - rv);
  }
  se = wave_sum(se);
  re = wave_sum(re);
  float tv[W4H_TOPK_MAX];
  int ti[W4H_TOPK_MAX];
  for (int k = 0; k < W4H_TOPK_MAX; ++k) {
    tv[k] = -INFINITY;
    ti[k] = 0x7fffffff;
  }
  for (int k = 0; k < topk; ++k) {
    float cv = -INFINITY;
    int ci = 0x7fffffff;
    for (int c = lane; c < n * W4H_TOPK_MAX; c += 64) {
      const int g = c / W4H_TOPK_MAX, q = c % W4H_TOPK_MAX;
      const float v = recs[(size_t)g * stride + 6 + q];
      const int id = __float_as_int(recs[(size_t)g * stride + 6 + W4H_TOPK_MAX + q]);
      bool taken = false;
      for (int p = 0; p < k; ++p) taken |= (ti[p] == id);
      if (!taken && v > -INFINITY && (v > cv || (v == cv && id < ci))) {
        cv = v;
        ci = id;
      }
    }
    wave_argmax(cv, ci);
    tv[k] = cv;
    ti[k] = ci;
  }
  if (lane == 0) {
    out_rec[0] = bv;
    out_rec[1] = __int_as_float(bi);
    out_rec[2] = se;
    out_rec[3] = rv;
    out_rec[4] = re;
    out_rec[5] = pv;
    for (int k = 0; k < W4H_TOPK_MAX; ++k) {
      out_rec[6 + k] = tv[k];
      out_rec[6 + W4H_TOPK_MAX + k] = __int_as_float(ti[k]);
    }
  }
}

DEV void rec_to_out(const float* r, int topk, w4h_step_out* out) {
  const int bi = __float_as_int(r[1]);
  out->argmax = (bi == 0x7fffffff) ? 0 : bi;
  out->max_logit = r[0];
  out->logsumexp = r[0] + logf(r[2]);
  out->probe_logit = r[5] > -INFINITY ? r[5] : 0.f;
  out->raw_logsumexp = r[3] + logf(r[4]);
  for (int k = 0; k < W4H_TOPK_MAX; ++k) {
    const bool ok = k < topk && r[6 + k] > -INFINITY;
    out->topk_ids[k] = ok ? __float_as_int(r[6 + W4H_TOPK_MAX + k]) : 0;
    out->topk_logits[k] = ok ? r[6 + k] : -INFINITY;
  }
}

DEV bool masked(const uint32_t* m, int mw, int s, int v) {
  return m != nullptr && ((m[(size_t)s * mw + (v >> 5)] >> (v & 31)) & 1u);
}

// ------------------------------------------------------------------------------------------------
// The persistent decoder-step kernel.

struct Lds {
  float* xin;   // [S][4d]   polled activations
  float* xn;    // [S][d]    LayerNorm output / merged attention output
  float* red;   // [32][SM]
  float* gout;  // [SM][8]
  float* scr;   // [8]
  int* toks;    // [kMaxRows] tokens of the current step
  float* big;   // phase scratch
};

// First work item of workgroup g for a phase with `off` rotation, G workgroups.
DEV int first_item(int g, int off, int G) { return (g - off % G + G) % G; }

struct StepCtx {
  uint32_t tag;
  int st, kv, pe, ncs;
};

#define NOINL __device__ __noinline__

// x of layer 0 = token embedding + positional embedding (exact dequant, one rounding)
template <int WQ8>
DEV void embed(const StepParams& p, const Lds& m, const StepCtx& c, float* dst) {
  const int d = p.d;
  for (int s = 0; s < p.S; ++s) {
    const int tk = m.toks[s];
    for (int j = threadIdx.x; j < d; j += kThreads) {
      float e;
      if (!WQ8) {
        e = h2f(static_cast<const uint16_t*>(p.emb)[(size_t)tk * d + j]);
      } else {
        e = (float)static_cast<const int8_t*>(p.emb)[(size_t)tk * d + j] * h2f(p.emb_s[(size_t)tk * (d >> 5) + (j >> 5)]);
      }
      dst[s * d + j] = e + p.pos[(size_t)c.pe * d + j];
    }
  }
  __syncthreads();
}

// LN1 + QKV; k and v are also appended to the self-KV cache at position c.kv.
template <int SM, int WQ8>
NOINL bool phase_qkv(const StepParams& p, Lds m, StepCtx c, int l, int rot) {
  const int G = gridDim.x, tid = threadIdx.x, S = p.S, d = p.d, H = p.H, d3 = 3 * d;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d3 + 7) / 8;
  const int it0 = first_item(blockIdx.x, rot, G);
  if (it0 >= nitems) return true;
  WRegs<PFR> wr;
  gemv_prefetch<PFR, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, it0 * 8, wr);
  if (l == 0) {
    embed<WQ8>(p, m, c, m.xin);
  } else {
    if (!ll_poll1(p.x3 + (size_t)(l - 1) * S * d, S * d, m.xin, c.tag, p.err)) return false;
  }
  wg_layernorm(m.xin, m.xn, S, d, lw.ln1_g, lw.ln1_b, m.scr);
  for (int it = it0; it < nitems; it += G) {
    if (it != it0) gemv_prefetch<PFR, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, it * 8, wr);
    gemv_compute<PFR, WQ8, SM>(wr, lw.w_qkv, lw.s_qkv, d3, d, it * 8, S, m.xn, m.red, m.gout);
    if (tid < 8 * S) {
      const int s = tid >> 3, row = it * 8 + (tid & 7);
      if (row < d3) {
        const float y = m.gout[tid] + lw.b_qkv[row];
        const int part = row / d, e = row - part * d, h = e >> 6;
        if (part > 0) {
          uint16_t* dstkv = part == 1 ? p.kv_k : p.kv_v;
          dstkv[((((size_t)l * S + s) * H + h) * p.max_ctx + c.kv) * kHeadDim + (e & 63)] = f2h(y);
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        }
        ll_st(p.qkv + (((size_t)l * S + s) * H + h) * 3 * kHeadDim + part * kHeadDim + (e & 63), y, c.tag);
      }
    }
  }
  return true;
}

// Self-attention: one item per (row, head, chunk of kSelfChunk keys); the current token's key and
// value come from the tagged QKV words, earlier keys from the f16 cache.
NOINL bool phase_self_attn(const StepParams& p, Lds m, StepCtx c, int l, int rot) {
  const int G = gridDim.x, tid = threadIdx.x, S = p.S, H = p.H;
  const int nitems = S * H * c.ncs;
  for (int it = first_item(blockIdx.x, rot, G); it < nitems; it += G) {
    const int ch = it % c.ncs, sh = it / c.ncs, h = sh % H, s = sh / H;
    const int k0 = ch * kSelfChunk;
    const int k1 = min(k0 + kSelfChunk, c.kv + 1);
    const int ncache = min(k1, c.kv) - k0;
    const bool cur = (k1 == c.kv + 1);
    const int32_t* slots = p.slots ? p.slots + (size_t)s * p.max_ctx : nullptr;
    const size_t lb = (size_t)l * S;
    const int H_ = H, mc = p.max_ctx;
    auto off = [=](int j) -> size_t {
      const int pos = k0 + j;
      const int slot = slots ? slots[pos] : s;
      return (((lb + slot) * H_ + h) * mc + pos) * kHeadDim;
    };
    KVRegs<KPT_SELF> kr;
    attn_prefetch<KPT_SELF>(p.kv_k, p.kv_v, off, ncache, kr);
    float* q = m.big;  // q, k_cur, v_cur contiguous: [3][64]
    float* kx = q + kHeadDim;
    float* vx = kx + kHeadDim;
    float* pmv = vx + kHeadDim;
    float* plv = pmv + 8;
    float* acc = plv + 8;
    float* sc = acc + kHeadDim;
    float* red = sc + kSelfChunk + 4;
    const u64* qb = p.qkv + (((size_t)l * S + s) * H + h) * 3 * kHeadDim;
    if (!ll_poll1(qb, cur ? 3 * kHeadDim : kHeadDim, q, c.tag, p.err)) return false;
    attn_compute<KPT_SELF, 1>(kr, ncache, 1, q, cur ? kx : nullptr, vx, 0.125f, sc, kSelfChunk + 4, red, pmv, plv, acc);
    u64* dst = p.sp + ((((size_t)l * p.ncs_max + ch) * S + s) * H + h) * kPartWords;
    for (int i = tid; i < kPartWords; i += kThreads) ll_st(dst + i, i == 0 ? pmv[0] : (i == 1 ? plv[0] : acc[i - 2]), c.tag);
  }
  return true;
}

// Merge attention partials, out-projection, bias and residual:  xout = xres + (Wo . o + b).
template <int SM, int WQ8>
NOINL bool phase_out(const StepParams& p, Lds m, StepCtx c, int l, int rot, bool cross) {
  const int G = gridDim.x, tid = threadIdx.x, S = p.S, d = p.d, H = p.H;
  const LayerDev& lw = p.layers[l];
  const void* W = cross ? lw.w_co : lw.w_o;
  const uint16_t* Ws = cross ? lw.s_co : lw.s_o;
  const float* bias = cross ? lw.b_co : lw.b_o;
  const int nitems = (d + 7) / 8;
  const int it0 = first_item(blockIdx.x, rot, G);
  if (it0 >= nitems) return true;
  WRegs<PFR> wr;
  gemv_prefetch<PFR, WQ8>(W, Ws, d, d, it0 * 8, wr);
  float* part = m.big;
  const int nc = cross ? p.ncc : c.ncs;
  const u64* psrc = cross ? p.cp + (size_t)l * p.ncc * S * H * kPartWords : p.sp + (size_t)l * p.ncs_max * S * H * kPartWords;
  // residual input: x1 for the cross block, the layer input for the self block (layer 0: embedding)
  const u64* rsrc = cross ? p.x1 + (size_t)l * S * d : p.x3 + (size_t)(l > 0 ? l - 1 : 0) * S * d;
  const int rn = (cross || l > 0) ? S * d : 0;
  if (!ll_poll2(psrc, nc * S * H * kPartWords, part, rsrc, rn, m.xin, c.tag, p.err)) return false;
  if (rn == 0) embed<WQ8>(p, m, c, m.xin);
  attn_merge(part, nc, S * H, m.xn);
  u64* xout = (cross ? p.x2 : p.x1) + (size_t)l * S * d;
  for (int it = it0; it < nitems; it += G) {
    if (it != it0) gemv_prefetch<PFR, WQ8>(W, Ws, d, d, it * 8, wr);
    gemv_compute<PFR, WQ8, SM>(wr, W, Ws, d, d, it * 8, S, m.xn, m.red, m.gout);
    if (tid < 8 * S) {
      const int s = tid >> 3, row = it * 8 + (tid & 7);
      if (row < d) ll_st(xout + (size_t)s * d + row, m.xin[s * d + row] + (m.gout[tid] + bias[row]), c.tag);
    }
  }
  return true;
}

// LN2 + cross q, published head-major [H][S][64] so a head's rows are contiguous.
template <int SM, int WQ8>
NOINL bool phase_cq(const StepParams& p, Lds m, StepCtx c, int l, int rot) {
  const int G = gridDim.x, tid = threadIdx.x, S = p.S, d = p.d, H = p.H;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d + 7) / 8;
  const int it0 = first_item(blockIdx.x, rot, G);
  if (it0 >= nitems) return true;
  WRegs<PFR> wr;
  gemv_prefetch<PFR, WQ8>(lw.w_cq, lw.s_cq, d, d, it0 * 8, wr);
  if (!ll_poll1(p.x1 + (size_t)l * S * d, S * d, m.xin, c.tag, p.err)) return false;
  wg_layernorm(m.xin, m.xn, S, d, lw.ln2_g, lw.ln2_b, m.scr);
  for (int it = it0; it < nitems; it += G) {
    if (it != it0) gemv_prefetch<PFR, WQ8>(lw.w_cq, lw.s_cq, d, d, it * 8, wr);
    gemv_compute<PFR, WQ8, SM>(wr, lw.w_cq, lw.s_cq, d, d, it * 8, S, m.xn, m.red, m.gout);
    if (tid < 8 * S) {
      const int s = tid >> 3, row = it * 8 + (tid & 7);
      if (row < d)
        ll_st(p.cq + (((size_t)l * H + (row >> 6)) * S + s) * kHeadDim + (row & 63), m.gout[tid] + lw.b_cq[row], c.tag);
    }
  }
  return true;
}

// Cross-attention: one item per (encoder group, head, key chunk); rows sharing an encoder output
// are processed together so the chunk's K/V is read once.
template <int SM>
NOINL bool phase_cross_attn(const StepParams& p, Lds m, StepCtx c, int l, int rot) {
  const int G = gridDim.x, tid = threadIdx.x, S = p.S, H = p.H, L = p.L;
  const int ngrp = p.X == 1 ? 1 : S;
  const int ns = p.X == 1 ? S : 1;
  const int nitems = ngrp * H * p.ncc;
  for (int it = first_item(blockIdx.x, rot, G); it < nitems; it += G) {
    const int ch = it % p.ncc, gh = it / p.ncc, h = gh % H, grp = gh / H;
    const int k0 = ch * p.chc;
    const int n = min(p.chc, p.A - k0);
    const size_t base = ((((size_t)grp * L + l) * H + h) * p.A + k0) * kHeadDim;
    auto off = [=](int j) -> size_t { return base + (size_t)j * kHeadDim; };
    KVRegs<KPT_CROSS> kr;
    attn_prefetch<KPT_CROSS>(p.xk, p.xv, off, n, kr);
    float* q = m.big;                     // [ns][64]
    float* pmv = q + SM * kHeadDim;       // [8]
    float* plv = pmv + 8;                 // [8]
    float* acc = plv + 8;                 // [ns][64]
    float* red = acc + SM * kHeadDim;     // [4][SM][64]
    float* sc = red + 4 * SM * kHeadDim;  // [ns][kMaxChunk + 4]
    const u64* qsrc = p.cq + (((size_t)l * H + h) * S + (p.X == 1 ? 0 : grp)) * kHeadDim;
    if (!ll_poll1(qsrc, ns * kHeadDim, q, c.tag, p.err)) return false;
    attn_compute<KPT_CROSS, SM>(kr, n, ns, q, nullptr, nullptr, 0.125f, sc, kMaxChunk + 4, red, pmv, plv, acc);
    for (int i = tid; i < ns * kPartWords; i += kThreads) {
      const int s = i / kPartWords, w = i - s * kPartWords;
      const int row = p.X == 1 ? s : grp;
      u64* dst = p.cp + ((((size_t)l * p.ncc + ch) * S + row) * H + h) * kPartWords;
      ll_st(dst + w, w == 0 ? pmv[s] : (w == 1 ? plv[s] : acc[s * kHeadDim + w - 2]), c.tag);
    }
  }
  return true;
}

// LN3 + MLP1 + GELU table lookup.
template <int SM, int WQ8>
NOINL bool phase_mlp1(const StepParams& p, Lds m, StepCtx c, int l, int rot) {
  const int G = gridDim.x, tid = threadIdx.x, S = p.S, d = p.d, d4 = 4 * d;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d4 + 7) / 8;
  const int it0 = first_item(blockIdx.x, rot, G);
  if (it0 >= nitems) return true;
  WRegs<PFR> wr;
  gemv_prefetch<PFR, WQ8>(lw.w_1, lw.s_1, d4, d, it0 * 8, wr);
  if (!ll_poll1(p.x2 + (size_t)l * S * d, S * d, m.xin, c.tag, p.err)) return false;
  wg_layernorm(m.xin, m.xn, S, d, lw.ln3_g, lw.ln3_b, m.scr);
  for (int it = it0; it < nitems; it += G) {
    if (it != it0) gemv_prefetch<PFR, WQ8>(lw.w_1, lw.s_1, d4, d, it * 8, wr);
    gemv_compute<PFR, WQ8, SM>(wr, lw.w_1, lw.s_1, d4, d, it * 8, S, m.xn, m.red, m.gout);
    if (tid < 8 * S) {
      const int s = tid >> 3, row = it * 8 + (tid & 7);
      if (row < d4) ll_st(p.hm + ((size_t)l * S + s) * d4 + row, p.gelu[f2h(m.gout[tid] + lw.b_1[row])], c.tag);
    }
  }
  return true;
}

// MLP2 + bias + residual.
template <int SM, int WQ8>
NOINL bool phase_mlp2(const StepParams& p, Lds m, StepCtx c, int l, int rot) {
  const int G = gridDim.x, tid = threadIdx.x, S = p.S, d = p.d, d4 = 4 * d;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d + 7) / 8;
  const int it0 = first_item(blockIdx.x, rot, G);
  if (it0 >= nitems) return true;
  WRegs<PFR> wr;
  gemv_prefetch<PFR, WQ8>(lw.w_2, lw.s_2, d, d4, it0 * 8, wr);
  if (!ll_poll2(p.hm + (size_t)l * S * d4, S * d4, m.xin, p.x2 + (size_t)l * S * d, S * d, m.xn, c.tag, p.err))
    return false;
  for (int it = it0; it < nitems; it += G) {
    if (it != it0) gemv_prefetch<PFR, WQ8>(lw.w_2, lw.s_2, d, d4, it * 8, wr);
    gemv_compute<PFR, WQ8, SM>(wr, lw.w_2, lw.s_2, d, d4, it * 8, S, m.xin, m.red, m.gout);
    if (tid < 8 * S) {
      const int s = tid >> 3, row = it * 8 + (tid & 7);
      if (row < d) ll_st(p.x3 + ((size_t)l * S + s) * d + row, m.xn[s * d + row] + (m.gout[tid] + lw.b_2[row]), c.tag);
    }
  }
  return true;
}

// Final LN + tied-embedding logits over this workgroup's 8-row vocabulary groups, masks, and
// the workgroup's selection partial (full record and a (max, argmax) pair).
template <int SM, int WQ8>
NOINL bool phase_logits(const StepParams& p, Lds m, StepCtx c) {
  const int G = gridDim.x, g = blockIdx.x, tid = threadIdx.x, S = p.S, d = p.d, V = p.V;
  const int nitems = (V + 7) / 8;
  const int rpw = p.rows_per_wg;
  float* lg = m.big;                                  // [S][rpw] masked
  float* rw = lg + S * rpw;                           // [S][rpw] raw
  int* lidx = reinterpret_cast<int*>(rw + S * rpw);   // [rpw]
  float* rec = reinterpret_cast<float*>(lidx + rpw);  // [S][kSelWords]
  WRegs<PFL> wa, wb;
  if (g < nitems) gemv_prefetch<PFL, WQ8>(p.emb, p.emb_s, V, d, g * 8, wa);
  if (!ll_poll1(p.x3 + (size_t)(p.L - 1) * S * d, S * d, m.xin, c.tag, p.err)) return false;
  wg_layernorm(m.xin, m.xn, S, d, p.lnf_g, p.lnf_b, m.scr);
  int nl = 0;
  for (int it = g; it < nitems; it += G) {
    const int nx = it + G;
    if (nx < nitems) gemv_prefetch<PFL, WQ8>(p.emb, p.emb_s, V, d, nx * 8, wb);
    gemv_compute<PFL, WQ8, SM>(wa, p.emb, p.emb_s, V, d, it * 8, S, m.xn, m.red, m.gout);
    if (tid < 8 * S) {
      const int s = tid >> 3, rr = tid & 7, row = it * 8 + rr, li = nl + rr;
      if (row < V) {
        const float v = m.gout[tid];
        rw[s * rpw + li] = v;
        lg[s * rpw + li] = (masked(p.mask, p.mw, s, row) || masked(p.mask2, p.mw, s, row)) ? -INFINITY : v;
        if (s == 0) lidx[li] = row;
        if (p.logits_out) p.logits_out[((size_t)c.st * S + s) * V + row] = v;
      }
    }
    nl += min(8, V - it * 8);
    wa = wb;
  }
  __syncthreads();
  for (int s = tid >> 6; s < S; s += 4)
    sel_partial(lg + s * rpw, rw + s * rpw, lidx, nl, p.probe, p.topk, rec + s * kSelWords);
  __syncthreads();
  for (int i = tid; i < S * kSelWords; i += kThreads) ll_st(p.lp + (size_t)g * S * kSelWords + i, rec[i], c.tag);
  for (int i = tid; i < 2 * S; i += kThreads) ll_st(p.lpa + (size_t)g * S * 2 + i, rec[(i >> 1) * kSelWords + (i & 1)], c.tag);
  return true;
}

// Selection reduction.  Every workgroup reduces the (max, argmax) pairs to get the next token;
// the last workgroup also merges the full partials (blocks of kRedBlock workgroups) into the
// step outputs.
NOINL bool phase_reduce(const StepParams& p, Lds m, StepCtx c) {
  const int G = gridDim.x, g = blockIdx.x, tid = threadIdx.x, S = p.S;
  float* pairs = m.big;  // [G][S][2]
  if (!ll_poll1(p.lpa, G * S * 2, pairs, c.tag, p.err)) return false;
  const bool last_step = c.st + 1 == p.nsteps;
  for (int s = tid >> 6; s < S; s += 4) {
    const int am = sel_argmax(pairs + 2 * s, G, 2 * S);
    if ((tid & 63) == 0 && !last_step)
      m.toks[s] = p.forced ? p.forced[(size_t)c.st * S + s] : (am == 0x7fffffff ? 0 : am);
  }
  __syncthreads();
  if (g == G - 1 && p.out != nullptr) {
    const int nblk = (G + kRedBlock - 1) / kRedBlock;
    float* blk = m.big;                                     // [kRedBlock][S][kSelWords]
    float* brec = blk + (size_t)kRedBlock * S * kSelWords;  // [nblk][S][kSelWords]
    for (int b = 0; b < nblk; ++b) {
      const int g0 = b * kRedBlock, ng = min(kRedBlock, G - g0);
      if (!ll_poll1(p.lp + (size_t)g0 * S * kSelWords, ng * S * kSelWords, blk, c.tag, p.err)) return false;
      for (int s = tid >> 6; s < S; s += 4)
        sel_merge(blk + s * kSelWords, ng, S * kSelWords, p.topk, brec + ((size_t)b * S + s) * kSelWords);
      __syncthreads();
    }
    float* fin = brec + (size_t)nblk * S * kSelWords;  // [S][kSelWords]
    for (int s = tid >> 6; s < S; s += 4) sel_merge(brec + s * kSelWords, nblk, S * kSelWords, p.topk, fin + s * kSelWords);
    __syncthreads();
    if (tid < S) rec_to_out(fin + tid * kSelWords, p.topk, p.out + (size_t)c.st * S + tid);
    __syncthreads();
  }
  return true;
}

template <int SM, int WQ8>
__global__ void __launch_bounds__(kThreads, 1) k_step(StepParams p) {
  extern __shared__ float lds_raw[];
  const int tid = threadIdx.x, S = p.S, d = p.d;
  Lds m;
  m.xin = lds_raw;
  m.xn = m.xin + S * 4 * d;
  m.red = m.xn + S * d;
  m.gout = m.red + 32 * SM;
  m.scr = m.gout + 8 * SM;
  m.toks = reinterpret_cast<int*>(m.scr + 8);
  m.big = m.scr + 8 + kMaxRows;
  if (tid < S) m.toks[tid] = p.tokens0[tid];
  __syncthreads();
  for (int st = 0; st < p.nsteps; ++st) {
    StepCtx c;
    c.tag = p.tag0 + (uint32_t)st;
    c.st = st;
    c.kv = p.kv_len0 + st;                         // keys already cached; this token is key c.kv
    c.pe = c.kv < p.C - 1 ? c.kv : p.C - 1;        // positional row (clamped as the reference)
    c.ncs = (c.kv + 1 + kSelfChunk - 1) / kSelfChunk;
    int rot = 0;
    for (int l = 0; l < p.L; ++l) {
      if (!phase_qkv<SM, WQ8>(p, m, c, l, rot)) return;
      rot += 37;
      if (!phase_self_attn(p, m, c, l, rot)) return;
      rot += 37;
      if (!phase_out<SM, WQ8>(p, m, c, l, rot, false)) return;
      rot += 37;
      if (!phase_cq<SM, WQ8>(p, m, c, l, rot)) return;
      rot += 37;
      if (!phase_cross_attn<SM>(p, m, c, l, rot)) return;
      rot += 37;
      if (!phase_out<SM, WQ8>(p, m, c, l, rot, true)) return;
      rot += 37;
      if (!phase_mlp1<SM, WQ8>(p, m, c, l, rot)) return;
      rot += 37;
      if (!phase_mlp2<SM, WQ8>(p, m, c, l, rot)) return;
      rot += 37;
    }
    if (!phase_logits<SM, WQ8>(p, m, c)) return;
    if (!phase_reduce(p, m, c)) return;
  }
}

// ------------------------------------------------------------------------------------------------
// Cross-attention K/V projection: out[h][t][e] = f16(sum_k xa[t][k] * W[h*64+e][k] (+ b)), per layer.
// 64x64 output tiles, k-tiles of 32, 4x4 outputs per thread (fp32 FMA).

template <int WQ8>
__global__ void __launch_bounds__(kThreads) k_cross_kv(const LayerDev* layers, int d, int H, int A, const float* xa,
                                                      uint16_t* xk, uint16_t* xv) {
  __shared__ float As[32][64 + 4];  // [k][t]
  __shared__ float Bs[32][64 + 4];  // [k][n]
  const int t0 = blockIdx.x * 64, n0 = blockIdx.y * 64;
  const int l = blockIdx.z >> 1, isv = blockIdx.z & 1;
  const LayerDev& lw = layers[l];
  const void* W = isv ? lw.w_cv : lw.w_ck;
  const uint16_t* Ws = isv ? lw.s_cv : lw.s_ck;
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < d; k0 += 32) {
    for (int i = tid; i < 64 * 32; i += kThreads) {
      const int r = i >> 5, kk = i & 31;
      const int t = t0 + r;
      As[kk][r] = t < A ? xa[(size_t)t * d + k0 + kk] : 0.f;
      const int n = n0 + r;
      float wv;
      if (!WQ8) {
        wv = h2f(static_cast<const uint16_t*>(W)[(size_t)n * d + k0 + kk]);
      } else {
        wv = (float)static_cast<const int8_t*>(W)[(size_t)n * d + k0 + kk] * h2f(Ws[(size_t)n * (d >> 5) + ((k0 + kk) >> 5)]);
      }
      Bs[kk][r] = wv;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = As[kk][ty * 4 + i];
        b[i] = Bs[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  uint16_t* out = (isv ? xv : xk) + (size_t)l * H * A * kHeadDim;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + ty * 4 + i;
    if (t >= A) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      float v = acc[i][j];
      if (isv && lw.b_cv) v += lw.b_cv[n];
      out[((size_t)(n >> 6) * A + t) * kHeadDim + (n & 63)] = f2h(v);
    }
  }
}

__global__ void k_fill_u64(u64* p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0ull;
}

// ------------------------------------------------------------------------------------------------
// Standalone op kernels (plain global memory in and out).

template <int WQ8>
__global__ void __launch_bounds__(kThreads) k_op_linear(const void* W, const uint16_t* Ws, int N, int K,
                                                       const float* bias, const float* x, int M, float* y) {
  extern __shared__ float sm[];
  float* xs = sm;               // [M][K]
  float* red = xs + M * K;      // [32][8]
  float* out = red + 32 * 8;    // [8][8]
  for (int i = threadIdx.x; i < M * K; i += kThreads) xs[i] = x[i];
  __syncthreads();
  const int it = blockIdx.x;
  WRegs<PFR> wr;
  gemv_prefetch<PFR, WQ8>(W, Ws, N, K, it * 8, wr);
  gemv_compute<PFR, WQ8, kMaxRows>(wr, W, Ws, N, K, it * 8, M, xs, red, out);
  if (threadIdx.x < 8 * M) {
    const int s = threadIdx.x >> 3, row = it * 8 + (threadIdx.x & 7);
    if (row < N) y[(size_t)s * N + row] = out[threadIdx.x] + (bias ? bias[row] : 0.f);
  }
}

__global__ void __launch_bounds__(kThreads) k_op_layernorm(const float* x, int rows, int n, const float* g,
                                                          const float* b, float* y) {
  extern __shared__ float sm[];
  float* xs = sm;
  float* ys = xs + n;
  float* scr = ys + n;
  const int r = blockIdx.x;
  for (int i = threadIdx.x; i < n; i += kThreads) xs[i] = x[(size_t)r * n + i];
  __syncthreads();
  wg_layernorm(xs, ys, 1, n, g, b, scr);
  for (int i = threadIdx.x; i < n; i += kThreads) y[(size_t)r * n + i] = ys[i];
}

__global__ void k_op_gelu(const float* x, int n, const float* table, float* y) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = table[f2h(x[i])];
}

// One workgroup per head; the keys are processed in chunks of kSelfChunk and merged exactly as the
// decoder step merges its self-attention partials.
__global__ void __launch_bounds__(kThreads) k_op_attention(const float* q, const uint16_t* k, const uint16_t* v,
                                                          int kv_len, float scale, float* out) {
  extern __shared__ float sm[];
  const int h = blockIdx.x;
  const int nc = (kv_len + kSelfChunk - 1) / kSelfChunk;
  float* qs = sm;                           // [64]
  float* pmv = qs + kHeadDim;               // [8]
  float* plv = pmv + 8;
  float* acc = plv + 8;                     // [64]
  float* sc = acc + kHeadDim;               // [kSelfChunk + 4]
  float* red = sc + kSelfChunk + 4;         // [4][1][64]
  float* part = red + 4 * kHeadDim;         // [nc][kPartWords]
  for (int i = threadIdx.x; i < kHeadDim; i += kThreads) qs[i] = q[h * kHeadDim + i];
  __syncthreads();
  const uint16_t* kb = k + (size_t)h * kv_len * kHeadDim;
  const uint16_t* vb = v + (size_t)h * kv_len * kHeadDim;
  for (int c = 0; c < nc; ++c) {
    const int k0 = c * kSelfChunk, n = min(kSelfChunk, kv_len - k0);
    auto off = [&](int j) -> size_t { return (size_t)(k0 + j) * kHeadDim; };
    KVRegs<KPT_SELF> kr;
    attn_prefetch<KPT_SELF>(kb, vb, off, n, kr);
    attn_compute<KPT_SELF, 1>(kr, n, 1, qs, nullptr, nullptr, scale, sc, kSelfChunk + 4, red, pmv, plv, acc);
    for (int i = threadIdx.x; i < kPartWords; i += kThreads)
      part[c * kPartWords + i] = i == 0 ? pmv[0] : (i == 1 ? plv[0] : acc[i - 2]);
    __syncthreads();
  }
  attn_merge(part, nc, 1, acc);
  for (int i = threadIdx.x; i < kHeadDim; i += kThreads) out[h * kHeadDim + i] = acc[i];
}

// Selection over rows of logits: grid (G, rows); workgroup (g, r) takes 8-row groups g, g+G, ...
// of row r and writes one partial; k_op_select_final merges them.
__global__ void __launch_bounds__(kThreads) k_op_select_part(const float* logits, int n, const uint32_t* mask, int mw,
                                                            int k, int rpw, float* parts) {
  extern __shared__ float sm[];
  const int G = gridDim.x, g = blockIdx.x, r = blockIdx.y;
  float* lg = sm;
  float* rw = lg + rpw;
  int* idx = reinterpret_cast<int*>(rw + rpw);
  float* rec = reinterpret_cast<float*>(idx + rpw);
  int nl = 0;
  for (int it = g; it * 8 < n; it += G) {
    if (threadIdx.x < 8) {
      const int row = it * 8 + threadIdx.x;
      if (row < n) {
        const float v = logits[(size_t)r * n + row];
        rw[nl + threadIdx.x] = v;
        lg[nl + threadIdx.x] = masked(mask, mw, r, row) ? -INFINITY : v;
        idx[nl + threadIdx.x] = row;
      }
    }
    nl += min(8, n - it * 8);
  }
  __syncthreads();
  if (threadIdx.x < 64) sel_partial(lg, rw, idx, nl, -1, k, rec);
  __syncthreads();
  for (int i = threadIdx.x; i < kSelWords; i += kThreads) parts[((size_t)r * G + g) * kSelWords + i] = rec[i];
}

__global__ void __launch_bounds__(64) k_op_select_final(const float* parts, int G, int k, w4h_step_out* out) {
  __shared__ float rec[kSelWords];
  const int r = blockIdx.x;
  sel_merge(parts + (size_t)r * G * kSelWords, G, kSelWords, k, rec);
  __syncthreads();
  if (threadIdx.x == 0) rec_to_out(rec, k, out + r);
}

// ------------------------------------------------------------------------------------------------
// launchers

size_t step_lds_bytes(const StepParams& p, int grid) {
  const int S = p.S, d = p.d, SM = S > 1 ? kMaxRows : 1;
  size_t fixed = (size_t)S * 4 * d + (size_t)S * d + 32 * SM + 8 * SM + 8 + kMaxRows;
  const size_t self_attn = 3 * kHeadDim + 16 + kHeadDim + kSelfChunk + 4 + 4 * kHeadDim;
  const size_t cross_attn = SM * kHeadDim + 16 + SM * kHeadDim + 4 * SM * kHeadDim + (size_t)SM * (kMaxChunk + 4);
  const size_t merge_self = (size_t)p.ncs_max * S * p.H * kPartWords;
  const size_t merge_cross = (size_t)p.ncc * S * p.H * kPartWords;
  const size_t logits = (size_t)2 * S * p.rows_per_wg + p.rows_per_wg + (size_t)S * kSelWords;
  const int nblk = (grid + kRedBlock - 1) / kRedBlock;
  size_t reduce = (size_t)(kRedBlock + nblk + 1) * S * kSelWords;
  if ((size_t)grid * S * 2 > reduce) reduce = (size_t)grid * S * 2;
  size_t big = self_attn;
  big = big > cross_attn ? big : cross_attn;
  big = big > merge_self ? big : merge_self;
  big = big > merge_cross ? big : merge_cross;
  big = big > logits ? big : logits;
  big = big > reduce ? big : reduce;
  return (fixed + big) * sizeof(float);
}

int step_max_grid(size_t lds_bytes) {
  hipDeviceProp_t prop;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  if (lds_bytes > (size_t)prop.sharedMemPerBlock) return 0;
  return prop.multiProcessorCount;  // one workgroup per CU (launch_bounds(256, 1), <= 160 KB LDS)
}

template <int SM, int WQ8>
static hipError_t launch_step_t(const StepParams& p, int grid, size_t lds, hipStream_t st) {
  hipError_t e = hipFuncSetAttribute((const void*)k_step<SM, WQ8>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  StepParams pp = p;
  void* args[] = {&pp};
  return hipLaunchCooperativeKernel((const void*)k_step<SM, WQ8>, dim3(grid), dim3(kThreads), args, (unsigned)lds, st);
}

#ifndef W4H_STEP_VARIANTS
#define W4H_STEP_VARIANTS 15
#endif
hipError_t launch_step(const StepParams& p, int grid, size_t lds, hipStream_t st) {
#if W4H_STEP_VARIANTS & 1
  if (p.S == 1 && !p.wq8) return launch_step_t<1, 0>(p, grid, lds, st);
#endif
#if W4H_STEP_VARIANTS & 2
  if (p.S == 1 && p.wq8) return launch_step_t<1, 1>(p, grid, lds, st);
#endif
#if W4H_STEP_VARIANTS & 4
  if (p.S > 1 && !p.wq8) return launch_step_t<kMaxRows, 0>(p, grid, lds, st);
#endif
#if W4H_STEP_VARIANTS & 8
  if (p.S > 1 && p.wq8) return launch_step_t<kMaxRows, 1>(p, grid, lds, st);
#endif
  return hipErrorInvalidValue;
}

hipError_t launch_cross_kv(const LayerDev* layers_dev, int L, int d, int H, int A, int wq8, const float* xa,
                           uint16_t* xk, uint16_t* xv, hipStream_t st) {
  dim3 grid((A + 63) / 64, d / 64, 2 * L);
  if (wq8)
    hipLaunchKernelGGL(k_cross_kv<1>, grid, dim3(kThreads), 0, st, layers_dev, d, H, A, xa, xk, xv);
  else
    hipLaunchKernelGGL(k_cross_kv<0>, grid, dim3(kThreads), 0, st, layers_dev, d, H, A, xa, xk, xv);
  return hipGetLastError();
}

hipError_t launch_fill_u64(u64* p, size_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_u64, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

hipError_t launch_op_linear(const void* w, const uint16_t* ws, int wq8, int n, int k, const float* bias, const float* x,
                            int m, float* y, hipStream_t st) {
  size_t lds = ((size_t)m * k + 32 * 8 + 64) * sizeof(float);
  dim3 grid((n + 7) / 8);
  hipError_t e;
  if (wq8) {
    e = hipFuncSetAttribute((const void*)k_op_linear<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_op_linear<1>, grid, dim3(kThreads), lds, st, w, ws, n, k, bias, x, m, y);
  } else {
    e = hipFuncSetAttribute((const void*)k_op_linear<0>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_op_linear<0>, grid, dim3(kThreads), lds, st, w, ws, n, k, bias, x, m, y);
  }
  return hipGetLastError();
}

hipError_t launch_op_layernorm(const float* x, int rows, int n, const float* g, const float* b, float* y,
                               hipStream_t st) {
  size_t lds = ((size_t)2 * n + 8) * sizeof(float);
  hipError_t e = hipFuncSetAttribute((const void*)k_op_layernorm, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_op_layernorm, dim3(rows), dim3(kThreads), lds, st, x, rows, n, g, b, y);
  return hipGetLastError();
}

hipError_t launch_op_gelu(const float* x, int n, const float* table, float* y, hipStream_t st) {
  hipLaunchKernelGGL(k_op_gelu, dim3((n + 255) / 256), dim3(256), 0, st, x, n, table, y);
  return hipGetLastError();
}

hipError_t launch_op_attention(const float* q, const uint16_t* k, const uint16_t* v, int nh, int kv_len, float scale,
                               float* out, hipStream_t st) {
  const int nc = (kv_len + kSelfChunk - 1) / kSelfChunk;
  size_t lds = ((size_t)kHeadDim + 16 + kHeadDim + kSelfChunk + 4 + 4 * kHeadDim + (size_t)nc * kPartWords) * sizeof(float);
  hipError_t e = hipFuncSetAttribute((const void*)k_op_attention, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_op_attention, dim3(nh), dim3(kThreads), lds, st, q, k, v, kv_len, scale, out);
  return hipGetLastError();
}

hipError_t launch_op_select(const float* logits, int rows, int n, const uint32_t* mask, int k, w4h_step_out* out,
                            hipStream_t st) {
  const int G = 64;
  const int rpw = (((n + 7) / 8 + G - 1) / G) * 8;
  float* parts = nullptr;
  hipError_t e = hipMallocAsync((void**)&parts, (size_t)rows * G * kSelWords * sizeof(float), st);
  if (e != hipSuccess) return e;
  size_t lds = ((size_t)3 * rpw + kSelWords) * sizeof(float);
  e = hipFuncSetAttribute((const void*)k_op_select_part, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_op_select_part, dim3(G, rows), dim3(kThreads), lds, st, logits, n, mask, (n + 31) / 32, k, rpw,
                       parts);
    hipLaunchKernelGGL(k_op_select_final, dim3(rows), dim3(64), 0, st, parts, G, k, out);
    e = hipGetLastError();
  }
  hipError_t e2 = hipFreeAsync(parts, st);
  return e != hipSuccess ? e : e2;
}

}  // namespace w4h
