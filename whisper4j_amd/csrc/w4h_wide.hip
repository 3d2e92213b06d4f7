// Batched ("wide") decoder step for gfx950: the rows of a session (beam hypotheses or independent
// streams, up to 32) advance one token per step through a sequence of ordinary kernels, and every
// projection is an MFMA GEMM over all rows at once (v_mfma_f32_16x16x32_f16).
//
// Per layer:  resid+LN1 -> QKV GEMM -> self-attention (KV append) -> out GEMM -> resid+LN2 ->
//             cross-q GEMM -> cross-attention chunks -> chunk merge -> cross-out GEMM -> resid+LN3 ->
//             MLP1 GEMM -> GELU -> MLP2 GEMM
// then resid+final LN -> tied logits GEMM -> selection partials -> selection merge (+ next token).
//
// Numerics.  Activations are fp32.  A GEMM stages its activation slice in LDS as two f16 parts,
// hi = f16(a) and lo = f16(a - hi), and runs every MFMA twice (hi and lo) against the same f16
// weight fragment, so products carry ~22 bits of the activation and accumulate in fp32.  q8_0
// weights enter the MFMA as their exact int8 values and one MFMA step covers exactly one 32-element
// block, whose f16 scale is applied to the step's fp32 result.  The self-KV cache is f16, as in the
// persistent step kernel; the current token's key and value are used in fp32.
//
// Output layout of a GEMM: partial sums per k slice, out[slice][row][N]; consumers (attention,
// residual, GELU, selection) add the slices, so no GEMM needs a cross-workgroup reduction.

#include "w4h_kernels.h"

namespace w4h {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int int2v __attribute__((ext_vector_type(2)));

constexpr int kPadH = 8;  // halves of padding per LDS activation row (16 bytes: spreads banks)

DEV half8 as_half8(uint4 u) {
  half8 h;
  __builtin_memcpy(&h, &u, 16);
  return h;
}

// 8 int8 values (two dwords) to 8 exact f16 values.
DEV half8 i8x8_to_h8(uint2 u) {
  half8 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = (_Float16)(float)(int8_t)((u.x >> (8 * j)) & 0xff);
    h[4 + j] = (_Float16)(float)(int8_t)((u.y >> (8 * j)) & 0xff);
  }
  return h;
}

// ------------------------------------------------------------------------------------------------
// GEMM: grid (ceil(N / 64), slices), 256 threads.  Wave w of workgroup (nb, ks) owns output columns
// nb*64 + w*16 + [0, 16) and the k range of slice ks.  Lane i holds weight row n = base + i%16 and,
// for MFMA step b of block kb, the 8 k values kb*128 + 32b + 8(i/16) + [0, 8): 16 bytes (f16) or 8
// bytes (int8) per load, 64 contiguous bytes per row per step.  Every weight fragment of the slice
// is loaded into registers before the activation slice is staged, so the stream of weight bytes
// overlaps the staging.  act rows >= S are staged as zeros.

template <int MT, int WQ8, int KB>
__global__ __launch_bounds__(256) void k_w_gemm(const void* __restrict__ w, const uint16_t* __restrict__ ws, int N, int K,
                                                const float* __restrict__ act, int lda, int S, float* __restrict__ out) {
  extern __shared__ __align__(16) uint16_t lds_h[];
  constexpr int Rp = MT * 16;
  constexpr int kslice = KB * kWideKBlock;
  constexpr int rs = kslice + kPadH;  // halves per LDS row
  uint16_t* hi = lds_h;
  uint16_t* lo = lds_h + Rp * rs;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g4 = lane >> 4, c16 = lane & 15;
  const int n = blockIdx.x * kWideCols + wv * 16 + c16;
  const int k0 = blockIdx.y * kslice;
  const int nkb = min(kslice, K - k0) / kWideKBlock;
  const int nr = min(n, N - 1);

  // 1. weight fragments of the whole slice
  half8 bf[KB][4];
  uint2 bq[KB][4];
  float sc[KB][4];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int k = k0 + kb * kWideKBlock + 32 * b + 8 * g4;
      if (kb < nkb) {
        if (!WQ8) {
          bf[kb][b] = as_half8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + (size_t)nr * K + k));
        } else {
          bq[kb][b] = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(w) + (size_t)nr * K + k);
          sc[kb][b] = h2f(ws[(size_t)nr * (K >> 5) + (k >> 5)]);
        }
      }
    }
  }

  // 2. activation slice -> LDS (hi, lo); 8 consecutive k per task
  constexpr int tasks_per_row = kslice / 8;
  for (int t = tid; t < Rp * tasks_per_row; t += 256) {
    const int r = t / tasks_per_row, c8 = t - r * tasks_per_row;
    const int k = k0 + c8 * 8;
    float v[8];
    if (r < S && k < K) {
      const float4 a0 = *reinterpret_cast<const float4*>(act + (size_t)r * lda + k);
      const float4 a1 = *reinterpret_cast<const float4*>(act + (size_t)r * lda + k + 4);
      v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
      v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.f;
    }
    half8 h, l;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h[j] = (_Float16)v[j];
      l[j] = (_Float16)(v[j] - (float)h[j]);
    }
    *reinterpret_cast<half8*>(hi + r * rs + c8 * 8) = h;
    *reinterpret_cast<half8*>(lo + r * rs + c8 * 8) = l;
  }
  lds_barrier();

  // 3. MFMA over the slice
  floatx4 acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    if (kb < nkb) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int kk = kb * kWideKBlock + 32 * b + 8 * g4;
        const half8 B = WQ8 ? i8x8_to_h8(bq[kb][b]) : bf[kb][b];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const half8 ah = *reinterpret_cast<const half8*>(hi + (m * 16 + c16) * rs + kk);
          const half8 al = *reinterpret_cast<const half8*>(lo + (m * 16 + c16) * rs + kk);
          if (!WQ8) {
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, B, acc[m], 0, 0, 0);
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, B, acc[m], 0, 0, 0);
          } else {
            floatx4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, B, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, B, t, 0, 0, 0);
            acc[m] += t * sc[kb][b];
          }
        }
      }
    }
  }

  // 4. partial sums of this slice: lane holds rows 4(i/16) + [0, 4) of each 16-row tile, column n
  if (n < N) {
    float* o = out + (size_t)blockIdx.y * Rp * N + n;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) o[(size_t)(m * 16 + 4 * g4 + j) * N] = acc[m][j];
  }
}

// Sum of the slices of a GEMM output at (row, col).
DEV float slice_sum(const float* p, int ks, size_t sstride, size_t idx) {
  float v = 0.f;
  for (int j = 0; j < ks; ++j) v += p[j * sstride + idx];
  return v;
}

// ------------------------------------------------------------------------------------------------
// Residual update + LayerNorm, one workgroup per row.  Mode 0: x = token embedding + positional
// row t.  Mode 1: x += bias + sum of the GEMM slices.  Then act[row] = LN(x) (when g != null).
// LN: two passes, eps 1e-5, as nn/LayerNorm.java:5-31.

constexpr int kWideVec = 8;  // d <= 8 * 256

template <int WQ8>
__global__ __launch_bounds__(256) void k_w_resid(int mode, const float* __restrict__ P, int ks, size_t sstride, const float* __restrict__ bias,
                                                 const void* __restrict__ emb, const uint16_t* __restrict__ emb_s,
                                                 const float* __restrict__ pos, int t, const int32_t* __restrict__ toks,
                                                 float* __restrict__ x, int d, const float* __restrict__ g,
                                                 const float* __restrict__ b, float* __restrict__ act, int lda) {
  __shared__ float red[8];
  const int s = blockIdx.x, tid = threadIdx.x;
  float v[kWideVec];
  float sum = 0.f;
  const int tk = mode == 0 ? toks[s] : 0;
#pragma unroll
  for (int i = 0; i < kWideVec; ++i) {
    const int j = tid + 256 * i;
    v[i] = 0.f;
    if (j < d) {
      float xv;
      if (mode == 0) {
        float e;
        if (!WQ8) e = h2f(static_cast<const uint16_t*>(emb)[(size_t)tk * d + j]);
        else e = (float)static_cast<const int8_t*>(emb)[(size_t)tk * d + j] * h2f(emb_s[(size_t)tk * (d >> 5) + (j >> 5)]);
        xv = e + pos[(size_t)t * d + j];
      } else {
        xv = x[(size_t)s * d + j] + (bias[j] + slice_sum(P, ks, sstride, (size_t)s * d + j));
      }
      x[(size_t)s * d + j] = xv;
      v[i] = xv;
      sum += xv;
    }
  }
  if (g == nullptr) return;
  sum = wave_sum(sum);
  if ((tid & 63) == 0) red[tid >> 6] = sum;
  __syncthreads();
  const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kWideVec; ++i)
    if (tid + 256 * i < d) q = fmaf(v[i] - mean, v[i] - mean, q);
  q = wave_sum(q);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = q;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[4] + red[5] + red[6] + red[7]) / (float)d + 1e-5f);
#pragma unroll
  for (int i = 0; i < kWideVec; ++i) {
    const int j = tid + 256 * i;
    if (j < d) act[(size_t)s * lda + j] = (v[i] - mean) * inv * g[j] + b[j];
  }
}

// ------------------------------------------------------------------------------------------------
// Self-attention of one (row, head): q, k, v = bias + GEMM slices; k, v appended to the cache at
// position t (f16); softmax over the t cached keys (row s reads position j from slot slots[s][j])
// plus the current key (fp32); output -> act[s][h*64, +64).  8 lanes per key, 16 bytes each.

__global__ __launch_bounds__(256) void k_w_self(const float* __restrict__ P, int ks, size_t sstride, int N, const float* __restrict__ bqkv,
                                                int d, int H, int l, int S, int max_ctx, int t, uint16_t* __restrict__ kvk,
                                                uint16_t* __restrict__ kvv, const int32_t* __restrict__ slots,
                                                float* __restrict__ act, int lda) {
  extern __shared__ float sc[];  // [t + 1] scores, then probabilities
  __shared__ float q[64], kc[64], vc[64], red[4 * 64], stat[8];
  const int s = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const size_t head_base = ((size_t)l * S * H) * max_ctx * kHeadDim;  // layer l
  if (tid < 192) {
    const int part = tid >> 6, e = tid & 63;
    const int col = part * d + h * kHeadDim + e;
    const float v = bqkv[col] + slice_sum(P, ks, sstride, (size_t)s * N + col);
    if (part == 0) q[e] = v;
    else if (part == 1) kc[e] = v;
    else vc[e] = v;
    if (part > 0) {
      const size_t row = head_base + (((size_t)s * H + h) * max_ctx + t) * kHeadDim + e;
      (part == 1 ? kvk : kvv)[row] = f2h(v);
    }
  }
  __syncthreads();
  const int kg = tid >> 3, dc = tid & 7;
  float qd[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qd[e] = q[dc * 8 + e];
  const int32_t* srow = slots ? slots + (size_t)s * max_ctx : nullptr;
  for (int j0 = 0; j0 < t; j0 += 32) {
    const int j = j0 + kg;
    float dot = 0.f;
    if (j < t) {
      const int slot = srow ? srow[j] : s;
      const uint4 u = *reinterpret_cast<const uint4*>(kvk + head_base + (((size_t)slot * H + h) * max_ctx + j) * kHeadDim + dc * 8);
      const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float2 f = h2x2(uw[e]);
        dot = fmaf(qd[2 * e], f.x, dot);
        dot = fmaf(qd[2 * e + 1], f.y, dot);
      }
    }
    dot = sum8(dot);
    if (dc == 0 && j < t) sc[j] = dot * 0.125f;
  }
  if (wv == 0) {
    const float cur = wave_sum(q[lane] * kc[lane]);
    if (lane == 0) sc[t] = cur * 0.125f;
  }
  __syncthreads();
  const int n = t + 1;
  float mx = -INFINITY;
  for (int j = tid; j < n; j += 256) mx = fmaxf(mx, sc[j]);
  mx = wave_max(mx);
  if (lane == 0) stat[wv] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(stat[0], stat[1]), fmaxf(stat[2], stat[3]));
  float se = 0.f;
  for (int j = tid; j < n; j += 256) {
    const float p = __expf(sc[j] - mx);
    sc[j] = p;
    se += p;
  }
  se = wave_sum(se);
  if (lane == 0) stat[4 + wv] = se;
  __syncthreads();
  const float tot = stat[4] + stat[5] + stat[6] + stat[7];
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;
  for (int j = kg; j < n; j += 32) {
    const float p = sc[j];
    if (j < t) {
      const int slot = srow ? srow[j] : s;
      const uint4 u = *reinterpret_cast<const uint4*>(kvv + head_base + (((size_t)slot * H + h) * max_ctx + j) * kHeadDim + dc * 8);
      const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float2 f = h2x2(uw[e]);
        o[2 * e] = fmaf(p, f.x, o[2 * e]);
        o[2 * e + 1] = fmaf(p, f.y, o[2 * e + 1]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = fmaf(p, vc[dc * 8 + e], o[e]);
    }
  }
  // sum over the 8 key groups of a wave (lane bits 3..5), then over the 4 waves
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] += __shfl_xor(o[e], 8);
    o[e] += __shfl_xor(o[e], 16);
    o[e] += __shfl_xor(o[e], 32);
  }
  if (lane < 8)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wv * 64 + lane * 8 + e] = o[e];
  __syncthreads();
  if (tid < 64) {
    const float v = red[tid] + red[64 + tid] + red[128 + tid] + red[192 + tid];
    act[(size_t)s * lda + h * kHeadDim + tid] = v / tot;
  }
}

// ------------------------------------------------------------------------------------------------
// Cross-attention chunk partials.  Workgroup (e, h, z): encoder e, head h, key chunk z % nch, row
// group z / nch (up to RG rows that read encoder e: the one row e when every row has its own
// encoder, else rows of the shared encoder).  Keys are scored for every row of the group, so a
// shared encoder's K/V chunk is read once per group.  Partial (m, l, acc[64]) per row.

template <int RG>
__global__ __launch_bounds__(256) void k_w_cross(const float* __restrict__ P, int ks, size_t sstride, int d, const float* __restrict__ bcq,
                                                 int H, int A, int l, int L, int S, int X, int chlen, int nch,
                                                 const uint16_t* __restrict__ xk, const uint16_t* __restrict__ xv,
                                                 float* __restrict__ cpart) {
  extern __shared__ float scs[];  // [RG][chlen]
  __shared__ float q[RG * 64], red[4 * RG * 64], rm[RG], rl[RG];
  const int e = blockIdx.x, h = blockIdx.y, c = blockIdx.z % nch, rg = blockIdx.z / nch;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  int r0, nr;
  if (X == S) {
    r0 = e;
    nr = 1;
  } else {
    r0 = rg * RG;
    nr = min(RG, S - r0);
  }
  for (int i = tid; i < nr * 64; i += 256) {
    const int r = i >> 6, k = i & 63;
    const int col = h * kHeadDim + k;
    q[i] = (bcq[col] + slice_sum(P, ks, sstride, (size_t)(r0 + r) * d + col)) * 0.125f;
  }
  __syncthreads();
  const int j0 = c * chlen, j1 = min(A, j0 + chlen), n = j1 - j0;
  const size_t base = ((((size_t)e * L + l) * H + h) * A) * kHeadDim;
  const int kg = tid >> 3, dc = tid & 7;
  for (int jj = 0; jj < n; jj += 32) {
    const int j = jj + kg;
    float kd[8];
    if (j < n) {
      const uint4 u = *reinterpret_cast<const uint4*>(xk + base + (size_t)(j0 + j) * kHeadDim + dc * 8);
      const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        const float2 f = h2x2(uw[q2]);
        kd[2 * q2] = f.x;
        kd[2 * q2 + 1] = f.y;
      }
    } else {
#pragma unroll
      for (int q2 = 0; q2 < 8; ++q2) kd[q2] = 0.f;
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      if (r < nr) {
        float dot = 0.f;
#pragma unroll
        for (int q2 = 0; q2 < 8; ++q2) dot = fmaf(q[r * 64 + dc * 8 + q2], kd[q2], dot);
        dot = sum8(dot);
        if (dc == 0 && j < n) scs[r * chlen + j] = dot;
      }
    }
  }
  __syncthreads();
  for (int r = wv; r < nr; r += 4) {
    float mx = -INFINITY;
    for (int j = lane; j < n; j += 64) mx = fmaxf(mx, scs[r * chlen + j]);
    mx = wave_max(mx);
    float se = 0.f;
    for (int j = lane; j < n; j += 64) {
      const float p = __expf(scs[r * chlen + j] - mx);
      scs[r * chlen + j] = p;
      se += p;
    }
    se = wave_sum(se);
    if (lane == 0) {
      rm[r] = mx;
      rl[r] = se;
    }
  }
  __syncthreads();
  float o[RG][8];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int q2 = 0; q2 < 8; ++q2) o[r][q2] = 0.f;
  for (int j = kg; j < n; j += 32) {
    const uint4 u = *reinterpret_cast<const uint4*>(xv + base + (size_t)(j0 + j) * kHeadDim + dc * 8);
    const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
    float vd[8];
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2) {
      const float2 f = h2x2(uw[q2]);
      vd[2 * q2] = f.x;
      vd[2 * q2 + 1] = f.y;
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      if (r < nr) {
        const float p = scs[r * chlen + j];
#pragma unroll
        for (int q2 = 0; q2 < 8; ++q2) o[r][q2] = fmaf(p, vd[q2], o[r][q2]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    if (r < nr) {
#pragma unroll
      for (int q2 = 0; q2 < 8; ++q2) {
        float v = o[r][q2];
        v += __shfl_xor(v, 8);
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        o[r][q2] = v;
      }
      if (lane < 8)
#pragma unroll
        for (int q2 = 0; q2 < 8; ++q2) red[(wv * RG + r) * 64 + lane * 8 + q2] = o[r][q2];
    }
  }
  __syncthreads();
  for (int i = tid; i < nr * 64; i += 256) {
    const int r = i >> 6, k = i & 63;
    const float v = red[(0 * RG + r) * 64 + k] + red[(1 * RG + r) * 64 + k] + red[(2 * RG + r) * 64 + k] +
                    red[(3 * RG + r) * 64 + k];
    float* dst = cpart + (((size_t)(r0 + r) * H + h) * nch + c) * kPartWords;
    dst[2 + k] = v;
    if (k == 0) {
      dst[0] = rm[r];
      dst[1] = rl[r];
    }
  }
}

// Merge the chunk partials of (row, head) into act[row][h*64, +64).  64 threads.
__global__ __launch_bounds__(64) void k_w_cmerge(const float* __restrict__ cpart, int H, int nch, float* __restrict__ act, int lda) {
  const int s = blockIdx.x, h = blockIdx.y, k = threadIdx.x;
  const float* p = cpart + ((size_t)s * H + h) * nch * kPartWords;
  float M = -INFINITY;
  for (int c = 0; c < nch; ++c) M = fmaxf(M, p[c * kPartWords]);
  float Lsum = 0.f, o = 0.f;
  for (int c = 0; c < nch; ++c) {
    const float f = __expf(p[c * kPartWords] - M);
    Lsum = fmaf(f, p[c * kPartWords + 1], Lsum);
    o = fmaf(f, p[c * kPartWords + 2 + k], o);
  }
  act[(size_t)s * lda + h * kHeadDim + k] = o / Lsum;
}

// act[r][k] = GELU(bias[k] + sum of the MLP1 slices), r < S, k < n.
__global__ __launch_bounds__(256) void k_w_gelu(const float* __restrict__ P, int ks, size_t sstride, const float* __restrict__ bias, int S,
                                                int n, float* __restrict__ act, int lda) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= S * n) return;
  const int r = i / n, k = i - r * n;
  act[(size_t)r * lda + k] = gelu_f16(bias[k] + slice_sum(P, ks, sstride, (size_t)r * n + k));
}

// ------------------------------------------------------------------------------------------------
// Selection.  Workgroup (s, b): 4 waves, wave w reduces entries [(4b + w) * 512, +512) of row s's
// logits (sum of the logits GEMM slices) to one selection partial; the raw logits are copied out
// when requested.  Then one wave per row merges the partials into the step result and the next
// token (argmax, first index of the maximum).

__global__ __launch_bounds__(256) void k_w_select(const float* __restrict__ P, int ks, size_t sstride, int V, const uint32_t* mask,
                                                  const uint32_t* mask2, int mw, int probe, int topk, float* __restrict__ selp,
                                                  int nsel, float* __restrict__ logits_out) {
  __shared__ float lg[4][kWideSelChunk], rw[4][kWideSelChunk];
  __shared__ int idx[4][kWideSelChunk];
  const int s = blockIdx.x, wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int part = blockIdx.y * 4 + wv;
  const int v0 = part * kWideSelChunk;
  const int nl = max(0, min(kWideSelChunk, V - v0));
  for (int j = lane; j < nl; j += 64) {
    const int v = v0 + j;
    const float x = slice_sum(P, ks, sstride, (size_t)s * V + v);
    rw[wv][j] = x;
    lg[wv][j] = (masked(mask, mw, s, v) || masked(mask2, mw, s, v)) ? -INFINITY : x;
    idx[wv][j] = v;
    if (logits_out) logits_out[(size_t)s * V + v] = x;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
  if (part < nsel) sel_partial(lg[wv], rw[wv], idx[wv], nl, probe, topk, selp + ((size_t)s * nsel + part) * kSelWords);
}

__global__ __launch_bounds__(64) void k_w_selmerge(const float* __restrict__ selp, int nsel, int topk, w4h_step_out* out,
                                                   int32_t* __restrict__ next_tok) {
  __shared__ float rec[kSelWords];
  const int s = blockIdx.x;
  sel_merge(selp + (size_t)s * nsel * kSelWords, nsel, kSelWords, topk, rec);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
  if (threadIdx.x == 0) {
    const int bi = __float_as_int(rec[1]);
    next_tok[s] = (bi == 0x7fffffff) ? 0 : bi;
    if (out) rec_to_out(rec, topk, out + s);
  }
}

// ------------------------------------------------------------------------------------------------
// host side

WideGemm wide_plan(const void* w, const uint16_t* ws, int N, int K, int n_cu) {
  WideGemm g{};
  g.w = w;
  g.ws = ws;
  g.N = N;
  g.K = K;
  const int kbt = K / kWideKBlock;
  const int nblk = (N + kWideCols - 1) / kWideCols;
  // largest slice (fewest partial sums) that still gives every compute unit two workgroups
  int kb = 4;
  while (kb > 1 && nblk * ((kbt + kb - 1) / kb) < 2 * n_cu) --kb;
  g.kb = kb;
  g.ks = (kbt + kb - 1) / kb;
  return g;
}

template <int MT, int WQ8, int KB>
static hipError_t gemm_kb(const WideGemm& g, const float* act, int lda, int S, float* out, hipStream_t st) {
  const dim3 grid((g.N + kWideCols - 1) / kWideCols, g.ks);
  const size_t lds = (size_t)2 * MT * 16 * (KB * kWideKBlock + kPadH) * sizeof(uint16_t);
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_w_gemm<MT, WQ8, KB>), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((k_w_gemm<MT, WQ8, KB>), grid, dim3(256), lds, st, g.w, g.ws, g.N, g.K, act, lda, S, out);
  return hipGetLastError();
}

template <int MT, int WQ8>
static hipError_t gemm_mt(const WideGemm& g, const float* act, int lda, int S, float* out, hipStream_t st) {
  switch (g.kb) {
    case 1: return gemm_kb<MT, WQ8, 1>(g, act, lda, S, out, st);
    case 2: return gemm_kb<MT, WQ8, 2>(g, act, lda, S, out, st);
    case 3: return gemm_kb<MT, WQ8, 3>(g, act, lda, S, out, st);
    default: return gemm_kb<MT, WQ8, 4>(g, act, lda, S, out, st);
  }
}

static hipError_t gemm(const WideParams& p, const WideGemm& g, float* out, hipStream_t st) {
  const int lda = 4 * p.d;
  if (p.Rp == 16) return p.wq8 ? gemm_mt<1, 1>(g, p.act, lda, p.S, out, st) : gemm_mt<1, 0>(g, p.act, lda, p.S, out, st);
  return p.wq8 ? gemm_mt<2, 1>(g, p.act, lda, p.S, out, st) : gemm_mt<2, 0>(g, p.act, lda, p.S, out, st);
}

static size_t sstride(const WideParams& p, const WideGemm& g) { return (size_t)p.Rp * g.N; }

static hipError_t resid(const WideParams& p, int mode, const float* P, const WideGemm* g, const float* bias, int t,
                        const int32_t* toks, const float* lg, const float* lb, hipStream_t st) {
  const int lda = 4 * p.d;
  const int ks = g ? g->ks : 0;
  const size_t ss = g ? sstride(p, *g) : 0;
  if (p.wq8)
    hipLaunchKernelGGL(k_w_resid<1>, dim3(p.S), dim3(256), 0, st, mode, P, ks, ss, bias, p.emb, p.emb_s, p.pos, t, toks, p.x, p.d, lg, lb,
                       p.act, lda);
  else
    hipLaunchKernelGGL(k_w_resid<0>, dim3(p.S), dim3(256), 0, st, mode, P, ks, ss, bias, p.emb, p.emb_s, p.pos, t, toks, p.x, p.d, lg, lb,
                       p.act, lda);
  return hipGetLastError();
}

#define WCHK(x)                          \
  do {                                   \
    const hipError_t e_ = (x);           \
    if (e_ != hipSuccess) return e_;     \
  } while (0)

hipError_t launch_wide(const WideParams& p, hipStream_t st) {
  const int d = p.d, H = p.H, lda = 4 * d;
  const int rg_rows = (p.X == p.S) ? 1 : 8;
  const int ngroups = (p.X == p.S) ? 1 : (p.S + 7) / 8;
  const size_t cross_lds = (size_t)rg_rows * p.chlen * sizeof(float);
  for (int i = 0; i < p.nsteps; ++i) {
    const int t = p.kv_len0 + i;
    const int pe = t < p.C - 1 ? t : p.C - 1;  // positional row, clamped as the reference
    const int32_t* toks = i == 0 ? p.tokens0 : (p.forced ? p.forced + (size_t)(i - 1) * p.S : p.next_tok);
    for (int l = 0; l < p.L; ++l) {
      const LayerDev& lw = p.layers[l];
      if (l == 0) {
        WCHK(resid(p, 0, nullptr, nullptr, nullptr, pe, toks, lw.ln1_g, lw.ln1_b, st));
      } else {
        WCHK(resid(p, 1, p.pb, &p.g_2, p.layers[l - 1].b_2, t, toks, lw.ln1_g, lw.ln1_b, st));
      }
      WideGemm g = p.g_qkv;
      g.w = lw.w_qkv;
      g.ws = lw.s_qkv;
      WCHK(gemm(p, g, p.pa, st));
      hipLaunchKernelGGL(k_w_self, dim3(p.S, H), dim3(256), (size_t)(t + 1) * sizeof(float), st, p.pa, g.ks, sstride(p, g), 3 * d,
                         lw.b_qkv, d, H, l, p.S, p.max_ctx, t, p.kv_k, p.kv_v, p.slots, p.act, lda);
      WCHK(hipGetLastError());
      g = p.g_o;
      g.w = lw.w_o;
      g.ws = lw.s_o;
      WCHK(gemm(p, g, p.pa, st));
      WCHK(resid(p, 1, p.pa, &g, lw.b_o, t, toks, lw.ln2_g, lw.ln2_b, st));
      g = p.g_cq;
      g.w = lw.w_cq;
      g.ws = lw.s_cq;
      WCHK(gemm(p, g, p.pa, st));
      if (rg_rows == 1)
        hipLaunchKernelGGL(k_w_cross<1>, dim3(p.X, H, p.nch * ngroups), dim3(256), cross_lds, st, p.pa, g.ks, sstride(p, g), d, lw.b_cq, H,
                           p.A, l, p.L, p.S, p.X, p.chlen, p.nch, p.xk, p.xv, p.cpart);
      else
        hipLaunchKernelGGL(k_w_cross<8>, dim3(p.X, H, p.nch * ngroups), dim3(256), cross_lds, st, p.pa, g.ks, sstride(p, g), d, lw.b_cq, H,
                           p.A, l, p.L, p.S, p.X, p.chlen, p.nch, p.xk, p.xv, p.cpart);
      WCHK(hipGetLastError());
      hipLaunchKernelGGL(k_w_cmerge, dim3(p.S, H), dim3(64), 0, st, p.cpart, H, p.nch, p.act, lda);
      WCHK(hipGetLastError());
      g = p.g_co;
      g.w = lw.w_co;
      g.ws = lw.s_co;
      WCHK(gemm(p, g, p.pa, st));
      WCHK(resid(p, 1, p.pa, &g, lw.b_co, t, toks, lw.ln3_g, lw.ln3_b, st));
      g = p.g_1;
      g.w = lw.w_1;
      g.ws = lw.s_1;
      WCHK(gemm(p, g, p.pa, st));
      hipLaunchKernelGGL(k_w_gelu, dim3((p.S * 4 * d + 255) / 256), dim3(256), 0, st, p.pa, g.ks, sstride(p, g), lw.b_1, p.S, 4 * d, p.act,
                         lda);
      WCHK(hipGetLastError());
      g = p.g_2;
      g.w = lw.w_2;
      g.ws = lw.s_2;
      WCHK(gemm(p, g, p.pb, st));
    }
    WCHK(resid(p, 1, p.pb, &p.g_2, p.layers[p.L - 1].b_2, t, toks, p.lnf_g, p.lnf_b, st));
    WCHK(gemm(p, p.g_v, p.pa, st));
    const int nblk = (p.nsel + 3) / 4;
    hipLaunchKernelGGL(k_w_select, dim3(p.S, nblk), dim3(256), 0, st, p.pa, p.g_v.ks, sstride(p, p.g_v), p.V, p.mask, p.mask2, p.mw,
                       p.probe, p.topk, p.selp, p.nsel, p.logits_out ? p.logits_out + (size_t)i * p.S * p.V : nullptr);
    WCHK(hipGetLastError());
    hipLaunchKernelGGL(k_w_selmerge, dim3(p.S), dim3(64), 0, st, p.selp, p.nsel, p.topk, p.out ? p.out + (size_t)i * p.S : nullptr,
                       p.next_tok);
    WCHK(hipGetLastError());
  }
  return hipSuccess;
}

}  // namespace w4h
