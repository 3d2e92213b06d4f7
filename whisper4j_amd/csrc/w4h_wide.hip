// Batched ("wide") decoder step for gfx950: the rows of a session (beam hypotheses or independent
// streams, up to 32) advance one token per step through a sequence of ordinary kernels, and every
// projection is an MFMA GEMM over all rows at once (v_mfma_f32_16x16x32_f16).
//
// Per layer:  residual + LN1 -> QKV GEMM -> self-attention (KV append) -> out GEMM -> residual + LN2 ->
//             cross-q GEMM -> cross-attention chunks -> chunk merge -> cross-out GEMM -> residual + LN3
//             -> MLP1 GEMM -> GELU -> MLP2 GEMM
// then residual + final LN -> tied logits GEMM -> selection partials -> selection merge (+ next token).
//
// Numerics.  Activations are fp32.  A GEMM stages its activation slice in LDS as two f16 parts,
// hi = f16(a) and lo = f16(a - hi), and runs every MFMA twice (hi and lo) against the same f16
// weight fragment, so products carry ~22 bits of the activation and accumulate in fp32.  q8_0
// weights enter the MFMA as their exact int8 values and one MFMA step covers exactly one 32-element
// block, whose f16 scale is applied to the step's fp32 result.  The self-KV cache is f16, as in the
// persistent step kernel; the current token's key and value are used in fp32.
//
// Split-K.  A GEMM splits K into slices (one workgroup per 64 output columns and slice) and stores
// one partial sum per slice, out[slice][row][N]; the next kernel, which reads every value anyway,
// adds the slices in slice order together with the bias (and residual, GELU), so a GEMM ends with
// its stores and no workgroup waits for another.

#include "w4h_mfma.h"

namespace w4h {

struct GemmArgs {
  const void* w;         // [N][K] f16, or int8 with f16 scales [N][K/32] in ws
  const uint16_t* ws;
  int N, K;
  const float* act;      // [Rp][lda] fp32 rows (rows >= S read as zero)
  int lda, S;
  float* part;           // [slices][Rp][N] partial sums (rows < S written)
  const WideCtl* ctl;    // a stopped run (ended beam search) stores nothing
};

// Sum of the ks slices of a GEMM output at p[j * ss + idx], added in slice order: B slices' loads in
// flight at a time, with clamped (branch-free) addresses.  Kernels with one output value per thread
// take every slice in one round trip (B = kWideMaxSlices); the selection, which loops over many
// values per lane, takes four at a time.
template <int B>
DEV float slice_sum(const float* p, int ks, size_t ss, size_t idx) {
  if (ks == 1) return p[idx];  // whole-K GEMM output (uniform branch)
  float v = 0.f;
  for (int j = 0; j < ks; j += B) {
    float t[B];
#pragma unroll
    for (int u = 0; u < B; ++u) t[u] = p[(size_t)min(j + u, ks - 1) * ss + idx];
#pragma unroll
    for (int u = 0; u < B; ++u) v += j + u < ks ? t[u] : 0.f;
  }
  return v;
}

// ------------------------------------------------------------------------------------------------
// GEMM: grid (ceil(N / (16 NW)), ks), 256 threads = 4 waves as NW column groups x KW = 4/NW k parts.
// Workgroup (nb, kz) owns columns nb*16*NW + [0, 16 NW) and the k range of slice kz
// (KW*KB*128 values); wave w takes column group w % NW and k part w / NW (KB blocks of 128).  Lane
// i holds weight row n = base + i%16 and, for MFMA step b of block kb, the 8 k values
// kb*128 + 32b + 8(i/16) + [0, 8): 16 bytes (f16) or 8 bytes (int8) per load, 64 contiguous bytes per
// row per step.  Every weight fragment of the wave's part is loaded into registers before the
// activation slice is staged, so the stream of weight bytes overlaps the staging.  The k parts of a
// column group are added through LDS in k order.

template <int MT, int WQ8, int KB, int NW>
__global__ __launch_bounds__(256) void k_w_gemm(GemmArgs a) {
  extern __shared__ __align__(16) uint16_t lds_h[];
  // an ended beam search: nothing is stored (the flag is read with the other loads, used at the end)
  const int stopped = a.ctl->stop;
  constexpr int KW = 4 / NW;
  constexpr int Rp = MT * 16;
  constexpr int CB = 16 * NW;                // columns per column block
  constexpr int kpart = KB * kWideKBlock;    // k per wave
  constexpr int kslice = KW * kpart;         // k per workgroup
  constexpr int rs = kslice + kPadH;         // halves per LDS row
  uint16_t* hi = lds_h;
  uint16_t* lo = lds_h + Rp * rs;
  const int N = a.N, K = a.K;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g4 = lane >> 4, c16 = lane & 15;
  const int cg = wv % NW, kw = wv / NW;
  const int k0 = blockIdx.y * kslice;        // workgroup's first k
  const int kp0 = k0 + kw * kpart;           // wave's first k
  const int nkb = max(0, min(kpart, K - kp0)) / kWideKBlock;
  const int n = blockIdx.x * CB + cg * 16 + c16;
  const int nr = min(n, N - 1);

  // 1. activation slice into registers first (L2 hits), so that waiting for it does not wait for
  //    the weight loads issued after it; 8 consecutive k per task
  constexpr int tasks_per_row = kslice / 8;
  constexpr int TPT = Rp * tasks_per_row / 256;  // tasks per thread
  //    Every load is unconditional (rows and k clamped, out-of-range values zeroed when staged), so
  //    the compiler can count the loads in flight and wait only for the ones it consumes.
  float4 av[TPT][2];
#pragma unroll
  for (int q = 0; q < TPT; ++q) {
    const int t = tid + 256 * q;
    const int r = t / tasks_per_row, c8 = t - r * tasks_per_row;
    const int rc = min(r, a.S - 1), kc = min(k0 + c8 * 8, K - 8);
    av[q][0] = *reinterpret_cast<const float4*>(a.act + (size_t)rc * a.lda + kc);
    av[q][1] = *reinterpret_cast<const float4*>(a.act + (size_t)rc * a.lda + kc + 4);
  }

  // 2. weight fragments of the wave's k part; blocks past K (the last slice) load the row's last 16
  //    bytes again and are skipped by the MFMA loop.  The activation loads are issued first and the
  //    weights after them, so that staging the activations waits for its own loads only.
  half8 bf[KB][4];
  uint2 bq[KB][4];
  float sc[KB][4];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int k = min(kp0 + kb * kWideKBlock + 32 * b + 8 * g4, K - 8);
      if (!WQ8) {
        bf[kb][b] = as_half8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.w) + (size_t)nr * K + k));
      } else {
        bq[kb][b] = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(a.w) + (size_t)nr * K + k);
        sc[kb][b] = h2f(a.ws[(size_t)nr * (K >> 5) + (k >> 5)]);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // activation slice -> LDS as (hi, lo) f16 parts
#pragma unroll
  for (int q = 0; q < TPT; ++q) {
    const int t = tid + 256 * q;
    const int r = t / tasks_per_row, c8 = t - r * tasks_per_row;
    const bool in = r < a.S && k0 + c8 * 8 < K;
    float v[8] = {av[q][0].x, av[q][0].y, av[q][0].z, av[q][0].w, av[q][1].x, av[q][1].y, av[q][1].z, av[q][1].w};
    half8 h, l;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = in ? v[j] : 0.f;
      h[j] = (_Float16)v[j];
      l[j] = (_Float16)(v[j] - (float)h[j]);
    }
    *reinterpret_cast<half8*>(hi + r * rs + c8 * 8) = h;
    *reinterpret_cast<half8*>(lo + r * rs + c8 * 8) = l;
  }
  lds_barrier();

  // 3. MFMA over the wave's k part
  {
    floatx4 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (kb < nkb) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int kk = kw * kpart + kb * kWideKBlock + 32 * b + 8 * g4;
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
    // 4. k parts of a column group added in k order through LDS (after the staged slice)
    if constexpr (KW > 1) {
      float* red = reinterpret_cast<float*>(lds_h + 2 * Rp * rs);  // [KW-1][NW][MT*4][64]
      lds_barrier();
      if (kw > 0)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int j = 0; j < 4; ++j) red[(((kw - 1) * NW + cg) * MT * 4 + m * 4 + j) * 64 + lane] = acc[m][j];
      lds_barrier();
      if (kw == 0)
#pragma unroll
        for (int q = 1; q < KW; ++q)
#pragma unroll
          for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[m][j] += red[(((q - 1) * NW + cg) * MT * 4 + m * 4 + j) * 64 + lane];
    }
    // 5. partial sums of this slice: lane holds rows 4(i/16) + [0, 4) of each 16-row tile, column n
    if (!stopped && kw == 0 && n < N) {
      float* o = a.part + (size_t)blockIdx.y * Rp * N + n;
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (m * 16 + 4 * g4 + j < a.S) o[(size_t)(m * 16 + 4 * g4 + j) * N] = acc[m][j];
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Residual update + LayerNorm, one workgroup per row.  EMB = 1: x = token embedding + positional
// row (layer 0).  EMB = 2: x as it is (the whole-K GEMMs updated it).  EMB = 0: x += bias + the
// slices of the last GEMM (out-projection, cross-out or MLP2).  Then act[row] = LN(x[row]), two
// passes, eps 1e-5, as nn/LayerNorm.java:5-31.

constexpr int kWideVec = 8;  // d <= 8 * 256

// NV = ceil(d / 256) elements per thread (template, so no dead element slots).  The residual row
// is loaded first, then every slice of every element at once with clamped (branch-free) addresses.
template <int WQ8, int EMB, int NV>
__global__ __launch_bounds__(256) void k_w_resid(const WideCtl* __restrict__ ctl, const int32_t* __restrict__ tokens0,
                                                 const int32_t* __restrict__ forced, const int32_t* __restrict__ next_tok, int S, int C,
                                                 const void* __restrict__ emb, const uint16_t* __restrict__ emb_s,
                                                 const float* __restrict__ pos, const float* __restrict__ P, int ks, size_t ss,
                                                 const float* __restrict__ bias, float* __restrict__ x, int d,
                                                 const float* __restrict__ g, const float* __restrict__ b, float* __restrict__ act,
                                                 int lda) {
  __shared__ float red[8];
  const int stopped = ctl->stop;  // ended beam search: read with the other loads, checked before storing
  const int s = blockIdx.x, tid = threadIdx.x;
  float v[NV];
  if (EMB == 1) {
    // token of this step: the run's first tokens, the forced row, or the last step's argmax;
    // positional row clamped as the reference
    const int i0 = ctl->i, t = ctl->kv_len0 + i0;
    const int pe = t < C - 1 ? t : C - 1;
    const int tk = (i0 == 0 && !ctl->tok_dev) ? tokens0[s]
                                              : (ctl->forced_on ? forced[(size_t)(i0 - 1) * S + s] : next_tok[s]);
    // every load unconditional (clamped j), so they are all in flight together
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int j = min(tid + 256 * i, d - 1);
      float e;
      if (!WQ8) e = h2f(static_cast<const uint16_t*>(emb)[(size_t)tk * d + j]);
      else e = (float)static_cast<const int8_t*>(emb)[(size_t)tk * d + j] * h2f(emb_s[(size_t)tk * (d >> 5) + (j >> 5)]);
      const float pv = pos[(size_t)pe * d + j];
      v[i] = tid + 256 * i < d ? e + pv : 0.f;
    }
  } else if (EMB == 2) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int j = min(tid + 256 * i, d - 1);
      const float xr = x[(size_t)s * d + j];
      v[i] = tid + 256 * i < d ? xr : 0.f;
    }
  } else {
    float xr[NV], bs[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int j = min(tid + 256 * i, d - 1);
      xr[i] = x[(size_t)s * d + j];
      bs[i] = bias[j];
    }
    // slices added in slice order; kWideMaxSlices of every element in flight at once
    float acc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = 0.f;
    for (int z = 0; z < ks; z += kWideMaxSlices) {
      float t[NV][kWideMaxSlices];
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int u = 0; u < kWideMaxSlices; ++u) {
          const int j = min(tid + 256 * i, d - 1), zz = min(z + u, ks - 1);
          t[i][u] = P[(size_t)zz * ss + (size_t)s * d + j];
        }
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int u = 0; u < kWideMaxSlices; ++u) acc[i] += z + u < ks ? t[i][u] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = tid + 256 * i < d ? xr[i] + (bs[i] + acc[i]) : 0.f;
  }
  if (stopped) return;
  if (EMB != 2)
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (tid + 256 * i < d) x[(size_t)s * d + tid + 256 * i] = v[i];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) sum += v[i];
  sum = wave_sum(sum);
  if ((tid & 63) == 0) red[tid >> 6] = sum;
  __syncthreads();
  const float mean = (red[0] + red[1] + red[2] + red[3]) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (tid + 256 * i < d) q = fmaf(v[i] - mean, v[i] - mean, q);
  q = wave_sum(q);
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = q;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[4] + red[5] + red[6] + red[7]) / (float)d + 1e-5f);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int j = tid + 256 * i;
    if (j < d) act[(size_t)s * lda + j] = (v[i] - mean) * inv * g[j] + b[j];
  }
}

// act[r][k] = GELU(bias[k] + the slices of the MLP1 GEMM), r < S, k < n.
__global__ __launch_bounds__(256) void k_w_gelu(const WideCtl* __restrict__ ctl, const float* __restrict__ P, int ks, size_t ss,
                                                const float* __restrict__ bias, int S, int n, float* __restrict__ act, int lda) {
  const int stopped = ctl->stop;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= S * n) return;
  const int r = i / n, k = i - r * n;
  const float v = gelu_f16(bias[k] + slice_sum<kWideMaxSlices>(P, ks, ss, (size_t)r * n + k));
  if (!stopped) act[(size_t)r * lda + k] = v;
}

// ------------------------------------------------------------------------------------------------
// Whole-K GEMM for sessions of at most 16 rows (one MFMA row tile).  A workgroup owns 16 output
// columns and all of K, split over its W waves (KS MFMA steps of 32 k per wave), so it ends with
// finished sums and applies the step that consumes them itself; no split-K partials, and no
// separate residual+LayerNorm or GELU kernel:
//   PRO = kProLn   input rows are the residual stream x; the workgroup forms each row's LayerNorm
//                  (two passes, eps 1e-5, nn/LayerNorm.java:5-31) from the fragments its waves hold,
//                  which cover every element of every row, and normalises them before the MFMA.
//   PRO = kProRaw  input rows enter as they are (attention outputs, MLP hidden rows).
//   EPI = kFEpiRaw    out[r][n] = sum (the attention kernels add the bias as they read q, k, v)
//   EPI = kFEpiResid  out[r][n] = out[r][n] + (bias[n] + sum)   (the residual update of x)
//   EPI = kFEpiGelu   out[r][n] = GELU(bias[n] + sum)            (MLP hidden row, f16 table value)
// Every lane loads its A fragments (row lane % 16, 8 consecutive k per step) from memory straight
// into registers, then its weight fragments: one memory round trip, the activation loads first so
// that the statistics wait only for them.  Lanes of padding rows (>= S) load nothing (their
// fragments are zero; the loads sit in a branch those lanes skip).  The LayerNorm
// gain and bias pass through LDS (one copy per workgroup).  The waves' sums are added in wave
// order through LDS, and wave j applies the epilogue to component j of every lane's 4 rows.

enum { kProRaw = 0, kProLn = 1 };
enum { kFEpiRaw = 0, kFEpiResid = 1, kFEpiGelu = 2 };

struct FusedArgs {
  const void* w;          // [N][K] f16, or int8 with f16 scales [N][K/32] in ws
  const uint16_t* ws;
  int N, K;
  const float* in;        // [S][lda] input rows
  int lda, S;
  const float *g, *b;     // LayerNorm gain and bias [K] (kProLn)
  const float* bias;      // [N] (kFEpiResid, kFEpiGelu)
  float* out;             // [S][ldo]
  int ldo;
  const WideCtl* ctl;     // a stopped run (ended beam search) stores nothing
};

template <int WQ8, int W, int KS, int PRO, int EPI>
__global__ __launch_bounds__(64 * W) void k_w_fgemm(FusedArgs a) {
  static_assert(W >= 4, "the epilogue takes one row component per wave");
  constexpr int KL = PRO == kProLn ? W * KS * 32 : 4;  // LayerNorm gain / bias entries in LDS
  __shared__ float s_st[2][W][16];
  __shared__ __attribute__((aligned(16))) float s_g[KL], s_b[KL];
  __shared__ floatx4 s_acc[W][64];
  const int stopped = a.ctl->stop;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g4 = lane >> 4, c16 = lane & 15;
  const int n = blockIdx.x * 16 + c16;
  const int kw0 = wv * KS * 32 + 8 * g4;  // the lane's first k
  const int S = a.S;
  const bool live = c16 < S;

  // 1. loads: LayerNorm gain / bias (bound for LDS), A fragments, weights, then the epilogue's
  //    bias and residual values.  Every load is unconditional, so that each consumer waits only
  //    for the loads issued before its own.
  constexpr int NG = PRO == kProLn ? (KL / 4 + 64 * W - 1) / (64 * W) : 1;
  float4 gq[NG], bq4[NG];
  if constexpr (PRO == kProLn) {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int i = min(tid + 64 * W * j, KL / 4 - 1);
      gq[j] = reinterpret_cast<const float4*>(a.g)[i];
      bq4[j] = reinterpret_cast<const float4*>(a.b)[i];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  float4 av[KS][2];
  if (live) {
    const float* src = a.in + (size_t)c16 * a.lda + kw0;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      av[s][0] = *reinterpret_cast<const float4*>(src + 32 * s);
      av[s][1] = *reinterpret_cast<const float4*>(src + 32 * s + 4);
    }
  } else {
#pragma unroll
    for (int s = 0; s < KS; ++s) av[s][0] = av[s][1] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 bf[KS];
  uint2 bq[KS];
  float sc[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int k = kw0 + 32 * s;
    if (!WQ8) {
      bf[s] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.w) + (size_t)n * a.K + k);
    } else {
      bq[s] = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(a.w) + (size_t)n * a.K + k);
      sc[s] = h2f(a.ws[(size_t)n * (a.K >> 5) + (k >> 5)]);
    }
  }
  const int er = 4 * g4 + (wv & 3);  // epilogue row of this lane (waves 0-3)
  float bb = 0.f, xo = 0.f;
  if constexpr (EPI != kFEpiRaw) bb = a.bias[n];
  if constexpr (EPI == kFEpiResid) {
    if (wv < 4) xo = a.out[(size_t)min(er, S - 1) * a.ldo + n];
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PRO == kProLn) {
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const int i = tid + 64 * W * j;
      if (i < KL / 4) {
        reinterpret_cast<float4*>(s_g)[i] = gq[j];
        reinterpret_cast<float4*>(s_b)[i] = bq4[j];
      }
    }
  }

  float v[KS][8];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const float t[8] = {av[s][0].x, av[s][0].y, av[s][0].z, av[s][0].w, av[s][1].x, av[s][1].y, av[s][1].z, av[s][1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[s][e] = t[e];
  }

  // 2. LayerNorm of the fragments: row sums over the lane's values, the 4 lanes of the row in the
  //    wave, then the waves in wave order
  if constexpr (PRO == kProLn) {
    float s1 = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) s1 += v[s][e];
    s1 += __shfl_xor(s1, 16);
    s1 += __shfl_xor(s1, 32);
    if (lane < 16) s_st[0][wv][lane] = s1;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) tot += s_st[0][w][c16];
    const float mean = tot / (float)a.K;
    float s2 = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) s2 = fmaf(v[s][e] - mean, v[s][e] - mean, s2);
    s2 += __shfl_xor(s2, 16);
    s2 += __shfl_xor(s2, 32);
    if (lane < 16) s_st[1][wv][lane] = s2;
    __syncthreads();
    float tq = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) tq += s_st[1][w][c16];
    const float inv = 1.0f / sqrtf(tq / (float)a.K + 1e-5f);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = kw0 + 32 * s;
      const float4 g0 = *reinterpret_cast<const float4*>(&s_g[k]), g1 = *reinterpret_cast<const float4*>(&s_g[k + 4]);
      const float4 b0 = *reinterpret_cast<const float4*>(&s_b[k]), b1 = *reinterpret_cast<const float4*>(&s_b[k + 4]);
      const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      const float be[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) v[s][e] = live ? (v[s][e] - mean) * inv * gg[e] + be[e] : 0.f;
    }
  }

  // 3. MFMA over the wave's k range, each step as (hi, lo) f16 parts against one weight fragment
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    half8 ah, al;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ah[e] = (_Float16)v[s][e];
      al[e] = (_Float16)(v[s][e] - (float)ah[e]);
    }
    const half8 B = WQ8 ? i8x8_to_h8(bq[s]) : as_half8(bf[s]);
    if (!WQ8) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, B, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, B, acc, 0, 0, 0);
    } else {
      floatx4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, B, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, B, t, 0, 0, 0);
      acc += t * sc[s];
    }
  }

  // 4. waves' sums in wave order; wave j (< 4) finishes component j of every lane: row
  //    4 (lane / 16) + j, column n
  s_acc[wv][lane] = acc;
  __syncthreads();
  if (wv >= 4 || stopped || er >= S) return;
  const float* sa = reinterpret_cast<const float*>(&s_acc[0][0]);
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < W; ++w) t += sa[(w * 64 + lane) * 4 + wv];
  float o;
  if constexpr (EPI == kFEpiRaw) o = t;
  else if constexpr (EPI == kFEpiResid) o = xo + (bb + t);
  else o = gelu_f16(bb + t);
  a.out[(size_t)er * a.ldo + n] = o;
}

// ------------------------------------------------------------------------------------------------
// Self-attention of one (row, head): q, k, v = bias + the QKV GEMM slices; k, v appended to the
// cache at position t (f16); softmax over the t cached keys (row s reads position j from slot
// slots[s][j]) plus the current key (fp32); output -> act[s][h*64, +64).  8 lanes per key, 16 bytes
// each.  The cached keys and values of the first kSelfBlock positions are loaded before q is
// formed (they do not depend on it), so one memory round trip covers them; longer contexts loop.

constexpr int kKeysInFlight = 4;   // keys per lane group in flight (cross-attention loops)
static_assert(32 * kKeysInFlight == kWideKeysPerPass, "one key-loop pass: 32 lane groups x kKeysInFlight");
constexpr int kSelfKF = 16;        // keys per lane group loaded up front (self-attention)
constexpr int kSelfBlock = 32 * kSelfKF;

DEV float dot8h(const float* qd, uint4 u) {
  const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
  float dot = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float2 fv = h2x2(uw[e]);
    dot = fmaf(qd[2 * e], fv.x, dot);
    dot = fmaf(qd[2 * e + 1], fv.y, dot);
  }
  return dot;
}

DEV void axpy8h(float p, uint4 u, float* o) {
  const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float2 fv = h2x2(uw[e]);
    o[2 * e] = fmaf(p, fv.x, o[2 * e]);
    o[2 * e + 1] = fmaf(p, fv.y, o[2 * e + 1]);
  }
}

__global__ __launch_bounds__(256) void k_w_self(const WideCtl* __restrict__ ctl, const float* __restrict__ P, int ks, size_t ss,
                                                const float* __restrict__ bqkv, int d, int H, int l, int S, int max_ctx,
                                                uint16_t* __restrict__ kvk, uint16_t* __restrict__ kvv,
                                                const int32_t* __restrict__ slot_table, float* __restrict__ act, int lda) {
  extern __shared__ float sc[];  // [t + 1] scores, then probabilities
  __shared__ float q[64], kc[64], vc[64], red[4 * 64], stat[8];
  const int s = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int kg = tid >> 3, dc = tid & 7;
  // the slot-table entries of the first block, loaded with the control block (not after it)
  int slot0[kSelfKF];
  if (slot_table)
#pragma unroll
    for (int f = 0; f < kSelfKF; ++f) slot0[f] = slot_table[(size_t)s * max_ctx + min(32 * f + kg, max_ctx - 1)];
  if (ctl->stop) return;
  const int t = ctl->kv_len0 + ctl->i;  // position of the current token
  const int32_t* srow = ctl->slots_on ? slot_table + (size_t)s * max_ctx : nullptr;
  const size_t head_base = ((size_t)l * S * H) * max_ctx * kHeadDim;  // layer l
  auto kv_off = [&](int j) -> size_t {
    const int slot = srow ? srow[j] : s;
    return head_base + (((size_t)slot * H + h) * max_ctx + j) * kHeadDim + dc * 8;
  };
  // cached keys and values of the first block, before q exists
  uint4 kr[kSelfKF], vr[kSelfKF];
#pragma unroll
  for (int f = 0; f < kSelfKF; ++f) {
    const int j = 32 * f + kg;
    if (j < t) {
      const int slot = srow ? slot0[f] : s;
      const size_t o = head_base + (((size_t)slot * H + h) * max_ctx + j) * kHeadDim + dc * 8;
      kr[f] = *reinterpret_cast<const uint4*>(kvk + o);
      vr[f] = *reinterpret_cast<const uint4*>(kvv + o);
    } else {
      kr[f] = make_uint4(0, 0, 0, 0);
      vr[f] = kr[f];
    }
  }
  if (tid < 192) {
    const int part = tid >> 6, e = tid & 63;
    const int col = part * d + h * kHeadDim + e;
    const float v = bqkv[col] + slice_sum<kWideMaxSlices>(P, ks, ss, (size_t)s * 3 * d + col);
    if (part == 0) q[e] = v;
    else if (part == 1) kc[e] = v;
    else vc[e] = v;
    if (part > 0) {
      const size_t row = head_base + (((size_t)s * H + h) * max_ctx + t) * kHeadDim + e;
      (part == 1 ? kvk : kvv)[row] = f2h(v);
    }
  }
  __syncthreads();
  float qd[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qd[e] = q[dc * 8 + e];
#pragma unroll
  for (int f = 0; f < kSelfKF; ++f) {
    if (32 * f >= t) break;  // uniform: the first block's key groups that hold positions
    const int j = 32 * f + kg;
    const float dot = sum8(dot8h(qd, kr[f]));
    if (dc == 0 && j < t) sc[j] = dot * 0.125f;
  }
  for (int j0 = kSelfBlock; j0 < t; j0 += 32 * kKeysInFlight) {  // positions past the first block
    uint4 u[kKeysInFlight];
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = j0 + 32 * f + kg;
      u[f] = j < t ? *reinterpret_cast<const uint4*>(kvk + kv_off(j)) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = j0 + 32 * f + kg;
      const float dot = sum8(dot8h(qd, u[f]));
      if (dc == 0 && j < t) sc[j] = dot * 0.125f;
    }
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
#pragma unroll
  for (int f = 0; f < kSelfKF; ++f) {
    if (32 * f >= t) break;
    const int j = 32 * f + kg;
    axpy8h(j < t ? sc[j] : 0.f, vr[f], o);
  }
  for (int j0 = kSelfBlock; j0 < t; j0 += 32 * kKeysInFlight) {
    uint4 u[kKeysInFlight];
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = j0 + 32 * f + kg;
      u[f] = j < t ? *reinterpret_cast<const uint4*>(kvv + kv_off(j)) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = j0 + 32 * f + kg;
      axpy8h(j < t ? sc[j] : 0.f, u[f], o);
    }
  }
  if (kg == 0) {
    const float p = sc[t];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = fmaf(p, vc[dc * 8 + e], o[e]);
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
// shared encoder's K/V chunk is read once per group.  Partial (m, l, acc[64]) per row, or, with a
// single chunk, the normalised output written to act directly.

template <int RG>
__global__ __launch_bounds__(256) void k_w_cross(const WideCtl* __restrict__ ctl, const float* __restrict__ P, int ks, size_t ss,
                                                 const float* __restrict__ bcq, int d,
                                                 int H, int A, int l, int L, int S, int X, int chlen, int nch,
                                                 const uint16_t* __restrict__ xk,
                                                 const uint16_t* __restrict__ xv, float* __restrict__ cpart,
                                                 float* __restrict__ act, int lda) {
  extern __shared__ float scs[];  // [RG][chlen]
  __shared__ float q[RG * 64], red[4 * RG * 64], rm[RG], rl[RG];
  const int stopped = ctl->stop;  // checked before the stores
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
  const int j0 = c * chlen, j1 = min(A, j0 + chlen), n = j1 - j0;
  const uint16_t* kb = xk + ((((size_t)e * L + l) * H + h) * A + j0) * kHeadDim;
  const uint16_t* vb = xv + ((((size_t)e * L + l) * H + h) * A + j0) * kHeadDim;
  const int kg = tid >> 3, dc = tid & 7;
  // keys and values of the chunk's first 32 * kKeysInFlight positions, before the query exists
  uint4 u0[kKeysInFlight], v0[kKeysInFlight];
#pragma unroll
  for (int f = 0; f < kKeysInFlight; ++f) {
    const int j = 32 * f + kg;
    u0[f] = j < n ? *reinterpret_cast<const uint4*>(kb + (size_t)j * kHeadDim + dc * 8) : make_uint4(0, 0, 0, 0);
    v0[f] = j < n ? *reinterpret_cast<const uint4*>(vb + (size_t)j * kHeadDim + dc * 8) : make_uint4(0, 0, 0, 0);
  }
  for (int i = tid; i < nr * 64; i += 256) {
    const int r = i >> 6, k = i & 63;
    const int col = h * kHeadDim + k;
    q[i] = (bcq[col] + slice_sum<kWideMaxSlices>(P, ks, ss, (size_t)(r0 + r) * d + col)) * 0.125f;
  }
  __syncthreads();
  for (int jj = 0; jj < n; jj += 32 * kKeysInFlight) {
    uint4 u[kKeysInFlight];
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = jj + 32 * f + kg;
      u[f] = jj == 0 ? u0[f] : (j < n ? *reinterpret_cast<const uint4*>(kb + (size_t)j * kHeadDim + dc * 8) : make_uint4(0, 0, 0, 0));
    }
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = jj + 32 * f + kg;
      float kd[8];
      const uint32_t uw[4] = {u[f].x, u[f].y, u[f].z, u[f].w};
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        const float2 fv = h2x2(uw[q2]);
        kd[2 * q2] = fv.x;
        kd[2 * q2 + 1] = fv.y;
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
  for (int jj = 0; jj < n; jj += 32 * kKeysInFlight) {
    uint4 u[kKeysInFlight];
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = jj + 32 * f + kg;
      u[f] = jj == 0 ? v0[f] : (j < n ? *reinterpret_cast<const uint4*>(vb + (size_t)j * kHeadDim + dc * 8) : make_uint4(0, 0, 0, 0));
    }
#pragma unroll
    for (int f = 0; f < kKeysInFlight; ++f) {
      const int j = jj + 32 * f + kg;
      float vd[8];
      const uint32_t uw[4] = {u[f].x, u[f].y, u[f].z, u[f].w};
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        const float2 fv = h2x2(uw[q2]);
        vd[2 * q2] = fv.x;
        vd[2 * q2 + 1] = fv.y;
      }
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        if (r < nr) {
          const float p = j < n ? scs[r * chlen + j] : 0.f;
#pragma unroll
          for (int q2 = 0; q2 < 8; ++q2) o[r][q2] = fmaf(p, vd[q2], o[r][q2]);
        }
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
  if (stopped) return;
  for (int i = tid; i < nr * 64; i += 256) {
    const int r = i >> 6, k = i & 63;
    const float v = red[(0 * RG + r) * 64 + k] + red[(1 * RG + r) * 64 + k] + red[(2 * RG + r) * 64 + k] +
                    red[(3 * RG + r) * 64 + k];
    if (nch == 1) {  // one chunk: the normalised output goes straight to the out-projection's input
      act[(size_t)(r0 + r) * lda + h * kHeadDim + k] = v / rl[r];
      continue;
    }
    float* dst = cpart + (((size_t)(r0 + r) * H + h) * nch + c) * kPartWords;
    dst[2 + k] = v;
    if (k == 0) {
      dst[0] = rm[r];
      dst[1] = rl[r];
    }
  }
}

// Merge the chunk partials of (row, head) into act[row][h*64, +64).  64 threads; lane c holds chunk
// c's (max, sum) (nch <= 64), then every lane adds its output element over the chunks in chunk order
// with eight loads in flight.
__global__ __launch_bounds__(64) void k_w_cmerge(const WideCtl* __restrict__ ctl, const float* __restrict__ cpart, int H, int nch,
                                                  float* __restrict__ act, int lda) {
  const int stopped = ctl->stop;  // checked before the store
  const int s = blockIdx.x, h = blockIdx.y, k = threadIdx.x;
  const float* p = cpart + ((size_t)s * H + h) * nch * kPartWords;
  const float mc = k < nch ? p[k * kPartWords] : -INFINITY;
  const float lc = k < nch ? p[k * kPartWords + 1] : 0.f;
  const float M = wave_max(mc);
  const float f = k < nch ? __expf(mc - M) : 0.f;
  const float Lsum = wave_sum(f * lc);
  float o = 0.f;
  for (int c0 = 0; c0 < nch; c0 += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = c0 + u < nch ? p[(c0 + u) * kPartWords + 2 + k] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) o = fmaf(__shfl(f, c0 + u), t[u], o);
  }
  if (!stopped) act[(size_t)s * lda + h * kHeadDim + k] = o / Lsum;
}

// ------------------------------------------------------------------------------------------------
// Cross-attention on the matrix cores for rows that share one encoder output (beam hypotheses; at
// most 16 rows).  Workgroup (h, c): head h, key chunk c of at most kXattnKeys keys; wave w takes
// 32 keys of it.  Scores are computed transposed, S^T = K . q^T (A = key rows, f16; B = the rows'
// queries as (hi, lo) f16 parts), so a lane ends with 8 keys of one row: {g4 + [0, 4)} of each
// 16-key tile (g4 = 4 (lane / 16)), row lane % 16.  After the chunk's row maximum (waves combined
// through LDS) the probabilities stay in registers as the B operand of O^T = V^T . P^T, with the
// keys of one 32-key MFMA step taken in that order; A = V^T rows (one head dimension over the same
// keys) read from the transposed V copy.  The waves' O^T tiles are added through LDS.  Output:
// the chunk partial (max, sum, acc[64]) per row for k_w_cmerge, or, with one chunk, the
// normalised row straight into act.

__global__ __launch_bounds__(256) void k_w_xattn(const WideCtl* __restrict__ ctl, const float* __restrict__ P, int ks, size_t ss,
                                                 const float* __restrict__ bcq, int d, int H, int A, int Ap, int l, int S,
                                                 int chlen, int nch, const uint16_t* __restrict__ xk,
                                                 const uint16_t* __restrict__ xvt, float* __restrict__ cpart,
                                                 float* __restrict__ act, int lda) {
  __shared__ float s_m[4][16], s_l[4][16];
  __shared__ floatx4 s_o[4][4][64];
  const int stopped = ctl->stop;  // checked before the stores
  const int h = blockIdx.x, c = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, g4 = 4 * g, c16 = lane & 15;
  const int j0 = c * chlen, j1 = min(A, j0 + chlen);
  const int kw = j0 + 32 * wv;  // the wave's first key
  const uint16_t* kb = xk + ((size_t)l * H + h) * A * kHeadDim;
  const uint16_t* vt = xvt + ((size_t)l * H + h) * kHeadDim * Ap;

  // loads: key fragments (A of S^T: key kw + 16 t + c16, clamped to the last frame; dims
  // 8 g + 32 q), V^T fragments (A of O^T: dim 16 nd + c16, keys kw + g4 + [0, 4) and
  // kw + 16 + g4 + [0, 4); the copy is zero past A and long enough for every chunk's 128 keys),
  // then the query of row c16 (bias + slices, dims 8 g + 32 q + [0, 8)) scaled by 1/8
  uint4 kf[2][2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int q = 0; q < 2; ++q)
      kf[t][q] = *reinterpret_cast<const uint4*>(kb + (size_t)min(kw + 16 * t + c16, A - 1) * kHeadDim + 8 * g + 32 * q);
  uint2 vf[4][2];
#pragma unroll
  for (int nd = 0; nd < 4; ++nd)
#pragma unroll
    for (int u = 0; u < 2; ++u)
      vf[nd][u] = *reinterpret_cast<const uint2*>(vt + (size_t)(16 * nd + c16) * Ap + kw + 16 * u + g4);
  const int row = min(c16, S - 1);
  half8 qh[2], ql[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int col = h * kHeadDim + 8 * g + 32 * q;
    float qv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = bcq[col + e];
    for (int z = 0; z < ks; ++z) {
      const float4 a0 = *reinterpret_cast<const float4*>(P + z * ss + (size_t)row * d + col);
      const float4 a1 = *reinterpret_cast<const float4*>(P + z * ss + (size_t)row * d + col + 4);
      const float t8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[e] += t8[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = c16 < S ? qv[e] * 0.125f : 0.f;
      qh[q][e] = (_Float16)v;
      ql[q][e] = (_Float16)(v - (float)qh[q][e]);
    }
  }

  // S^T tiles: keys kw + 16 t + g4 + e of row c16
  floatx4 sc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    sc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const half8 K = as_half8(kf[t][q]);
      sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(K, qh[q], sc[t], 0, 0, 0);
      sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(K, ql[q], sc[t], 0, 0, 0);
    }
  }
  // chunk maximum of row c16: the lane's 8 keys, lanes ^16 and ^32, then the waves
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (kw + 16 * t + g4 + e >= j1) sc[t][e] = -INFINITY;
      mx = fmaxf(mx, sc[t][e]);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  if (lane < 16) s_m[wv][lane] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_m[0][c16], s_m[1][c16]), fmaxf(s_m[2][c16], s_m[3][c16]));
  float ls = 0.f;
  half8 ph, pl;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float pv = __expf(sc[t][e] - M);
      ls += pv;
      const _Float16 hi = (_Float16)pv;
      ph[4 * t + e] = hi;
      pl[4 * t + e] = (_Float16)(pv - (float)hi);
    }
  ls += __shfl_xor(ls, 16);
  ls += __shfl_xor(ls, 32);
  if (lane < 16) s_l[wv][lane] = ls;
  // O^T tiles over the wave's 32 keys: dims 16 nd + g4 + e of row c16
#pragma unroll
  for (int nd = 0; nd < 4; ++nd) {
    half8 V;
    __builtin_memcpy(&V, &vf[nd][0], 8);
    __builtin_memcpy(reinterpret_cast<char*>(&V) + 8, &vf[nd][1], 8);
    floatx4 o = __builtin_amdgcn_mfma_f32_16x16x32_f16(V, ph, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    o = __builtin_amdgcn_mfma_f32_16x16x32_f16(V, pl, o, 0, 0, 0);
    s_o[wv][nd][lane] = o;
  }
  __syncthreads();
  // wave w adds dim tile w over the waves (wave order) and stores rows < S
  if (stopped || c16 >= S) return;
  const float L = (s_l[0][c16] + s_l[1][c16]) + (s_l[2][c16] + s_l[3][c16]);
  floatx4 o = s_o[0][wv][lane];
#pragma unroll
  for (int w = 1; w < 4; ++w) o += s_o[w][wv][lane];
  const int dim = 16 * wv + g4;
  if (nch == 1) {
    const float inv = 1.f / L;
    *reinterpret_cast<float4*>(act + (size_t)c16 * lda + h * kHeadDim + dim) = make_float4(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
    return;
  }
  float* dst = cpart + (((size_t)c16 * H + h) * nch + c) * kPartWords;  // 8-byte aligned
#pragma unroll
  for (int e = 0; e < 4; ++e) dst[2 + dim + e] = o[e];
  if (wv == 0 && g == 0) {
    dst[0] = M;
    dst[1] = L;
  }
}

// ------------------------------------------------------------------------------------------------
// Selection.  Workgroup (s, b): 4 waves, wave w reduces entries [(4b + w) * 512, +512) of row s's
// logits to one selection partial; the raw logits are copied out when requested.  Then one wave
// per row merges the partials into the step result and the next token (argmax, first index of the
// maximum).

__global__ __launch_bounds__(256) void k_w_select(const WideCtl* __restrict__ ctl, const float* __restrict__ P, int ks, size_t ss,
                                                  int S, int V,
                                                  const uint32_t* mask_buf, const uint32_t* mask2_buf, int mw,
                                                  const float* __restrict__ bias_buf,
                                                  float* __restrict__ selp, int nsel, float* __restrict__ logits_buf) {
  __shared__ float lg[4][kWideSelChunk], rw[4][kWideSelChunk];
  __shared__ int idx[4][kWideSelChunk];
  if (ctl->stop) return;
  const int s = blockIdx.x, wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t* mask = ctl->mask_on ? mask_buf : nullptr;
  const uint32_t* mask2 = ctl->mask2_on ? mask2_buf : nullptr;
  const int probe = ctl->probe, topk = ctl->topk;
  float* logits_out = ctl->logits_on ? logits_buf + (size_t)ctl->i * S * V : nullptr;
  const float* bias = ctl->bias_on ? bias_buf : nullptr;
  const int part = blockIdx.y * 4 + wv;
  const int v0 = part * kWideSelChunk;
  const int nl = max(0, min(kWideSelChunk, V - v0));
  if (nl > 0 && ks <= 4) {
    // every load of the lane's kSelPer entries (slices, bias, mask words) issued before any is used;
    // indices clamped to the chunk's last entry, the stores guarded
    constexpr int kSelPer = kWideSelChunk / 64;
    float t[kSelPer][4], bv[kSelPer];
    uint32_t m1[kSelPer], m2[kSelPer];
#pragma unroll
    for (int u = 0; u < kSelPer; ++u) {
      const int v = v0 + min(lane + 64 * u, nl - 1);
#pragma unroll
      for (int z = 0; z < 4; ++z) t[u][z] = P[(size_t)min(z, ks - 1) * ss + (size_t)s * V + v];
      bv[u] = bias ? bias[v] : 0.f;
      m1[u] = mask ? mask[(size_t)s * mw + (v >> 5)] : 0u;
      m2[u] = mask2 ? mask2[(size_t)s * mw + (v >> 5)] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kSelPer; ++u) {
      const int j = lane + 64 * u;
      if (j >= nl) continue;
      const int v = v0 + j;
      float acc = 0.f;
#pragma unroll
      for (int z = 0; z < 4; ++z) acc += z < ks ? t[u][z] : 0.f;
      const float x = acc + bv[u];
      rw[wv][j] = x;
      lg[wv][j] = (((m1[u] | m2[u]) >> (v & 31)) & 1u) ? -INFINITY : x;
      idx[wv][j] = v;
      if (logits_out) logits_out[(size_t)s * V + v] = x;
    }
  } else {
    for (int j = lane; j < nl; j += 64) {
      const int v = v0 + j;
      const float x = slice_sum<4>(P, ks, ss, (size_t)s * V + v) + (bias ? bias[v] : 0.f);
      rw[wv][j] = x;
      lg[wv][j] = (masked(mask, mw, s, v) || masked(mask2, mw, s, v)) ? -INFINITY : x;
      idx[wv][j] = v;
      if (logits_out) logits_out[(size_t)s * V + v] = x;
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
  if (part < nsel) sel_partial(lg[wv], rw[wv], idx[wv], nl, probe, topk, selp + ((size_t)s * nsel + part) * kSelWords);
}

// sel_merge for at most 128 partials: a lane's two records are loaded whole before any is used
// (the same operations in the same order, so the same result).
DEV void sel_merge_128(const float* recs, int n, int topk, float* out_rec) {
  const int lane = threadIdx.x & 63;
  float r[2][kSelWords];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float* src = recs + (size_t)min(lane + 64 * h, n - 1) * kSelWords;
#pragma unroll
    for (int w = 0; w < kSelWords; ++w) r[h][w] = src[w];
  }
  float bv = -INFINITY, rv = -INFINITY, pv = -INFINITY;
  int bi = 0x7fffffff;
  TopList tl;
  top_init(tl);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (lane + 64 * h >= n) continue;
    const int id = __float_as_int(r[h][1]);
    if (r[h][0] > bv || (r[h][0] == bv && id < bi)) {
      bv = r[h][0];
      bi = id;
    }
    rv = fmaxf(rv, r[h][3]);
    pv = fmaxf(pv, r[h][5]);
#pragma unroll
    for (int q = 0; q < W4H_TOPK_MAX; ++q)
      if (q < topk) top_insert(tl, r[h][6 + q], __float_as_int(r[h][6 + W4H_TOPK_MAX + q]));
  }
  wave_argmax(bv, bi);
  rv = wave_max(rv);
  pv = wave_max(pv);
  float se = 0.f, re = 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (lane + 64 * h >= n) continue;
    if (r[h][0] > -INFINITY) se += r[h][2] * __expf(r[h][0] - bv);
    if (r[h][3] > -INFINITY) re += r[h][4] * __expf(r[h][3] - rv);
  }
  se = wave_sum(se);
  re = wave_sum(re);
  float tv[W4H_TOPK_MAX];
  int ti[W4H_TOPK_MAX];
  top_pop(tl, topk, tv, ti);
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

__global__ __launch_bounds__(64) void k_w_selmerge(WideCtl* __restrict__ ctl, const float* __restrict__ selp, int S, int nsel,
                                                   w4h_step_out* out_buf, int32_t* __restrict__ next_tok) {
  __shared__ float rec[kSelWords];
  if (ctl->stop) return;
  const int s = blockIdx.x;
  const int topk = ctl->topk, i = ctl->i;
  if (nsel <= 128) sel_merge_128(selp + (size_t)s * nsel * kSelWords, nsel, topk, rec);
  else sel_merge(selp + (size_t)s * nsel * kSelWords, nsel, kSelWords, topk, rec);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
  if (threadIdx.x == 0) {
    const int bi = __float_as_int(rec[1]);
    next_tok[s] = (bi == 0x7fffffff) ? 0 : bi;
    if (ctl->out_on) rec_to_out(rec, topk, out_buf + (size_t)i * S + s);
    // the last row of the step to finish advances the step index (every row has read it)
    const unsigned prev = __hip_atomic_fetch_add(&ctl->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (unsigned)(S - 1)) {
      __hip_atomic_store(&ctl->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ctl->i, i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}


// ------------------------------------------------------------------------------------------------
// One step of beam search on the device (WhisperDecoder.decodeBeam, main/nn/WhisperDecoder.java:
// 278-394, the same steps as the host driver): candidates (beam b, rank k) of the live beams score
// lps[b] + (topk_logit - logsumexp); a stable descending sort; end tokens go to the finished list
// (until beam_size are finished), the first beam_size others become the new beams, leftover beams
// continue from the first; the slot table is regathered from the parents; the next step's tokens
// and suppression mask (suppress list, 3- and 4-gram repeats, timestamp rules) are written.  When
// the search ends (nothing saved, or enough finished) the beams are left as they were and ctl->stop
// makes the later steps of the run return at once.  One workgroup.

constexpr int kBeamCand = kBeamMax * (kBeamMax + 1);
constexpr int kSlotChunk = 1024;
constexpr int kBeamSupLds = 512;  // suppress-list entries held in LDS

// Dynamic LDS of k_w_beam: the slot-table chunk, then reused for the next step's masks.
inline size_t beam_lds_bytes(int B, int mw) {
  const size_t a = sizeof(int32_t) * (size_t)kBeamMax * kSlotChunk, b = sizeof(uint32_t) * (size_t)B * mw;
  return a > b ? a : b;
}

__global__ __launch_bounds__(256) void k_w_beam(WideCtl* __restrict__ ctl, BeamDev* __restrict__ bd, const w4h_step_out* out_buf,
                                                int B, int eot, int tsb, const int32_t* __restrict__ sup, int nsup, int V, int mw,
                                                uint32_t* __restrict__ mask2, int32_t* __restrict__ slots, int max_ctx,
                                                int32_t* __restrict__ next_tok) {
  extern __shared__ int32_t dyn[];  // slot chunk [kBeamMax][kSlotChunk], later masks [B][mw]
  __shared__ int stoks[kBeamMax][kBeamTokMax];
  __shared__ int slen[kBeamMax];
  __shared__ double slps[kBeamMax];
  __shared__ float stl[kBeamCand], slse[kBeamMax];
  __shared__ int sti[kBeamCand];
  __shared__ double csc[kBeamCand];
  __shared__ int clive[kBeamCand], order[kBeamCand];
  __shared__ int psrc[kBeamMax], ptok[kBeamMax], fsrc[kBeamMax];
  __shared__ double plp[kBeamMax], fsc[kBeamMax];
  __shared__ int s_nf0, s_nf, s_done, s_cur, s_maxlen;
  __shared__ int ssup[kBeamSupLds];
  if (ctl->stop) return;
  const int tid = threadIdx.x;
  for (int q = tid; q < min(nsup, kBeamSupLds); q += 256) ssup[q] = sup[q];  // read once, used per row below
  const int step = ctl->i - 1;             // the selection merge of this step has advanced the index
  const int kv = ctl->kv_len0 + step + 1;  // KV length after this step
  const int nc = B * (B + 1);
  // 1. beam state and this step's records into LDS
  if (tid == 0) {
    s_cur = bd->cur;
    s_nf0 = bd->nfin;
  }
  if (tid < B) {
    const w4h_step_out& o = out_buf[(size_t)step * B + tid];
    slse[tid] = o.logsumexp;
    slps[tid] = bd->lps[tid];
  }
  if (tid < nc) {
    const int b = tid / (B + 1), k = tid - b * (B + 1);
    const w4h_step_out& o = out_buf[(size_t)step * B + b];
    stl[tid] = o.topk_logits[k];
    sti[tid] = o.topk_ids[k];
  }
  __syncthreads();
  const int cur = s_cur, nxt = cur ^ 1;
  if (tid < B) slen[tid] = bd->len[cur][tid];
  __syncthreads();
  if (tid == 0) {
    int m = 0;
    for (int b = 0; b < B; ++b) m = max(m, slen[b]);
    s_maxlen = m;
  }
  __syncthreads();
  for (int e = tid; e < B * s_maxlen; e += 256) {
    const int b = e / s_maxlen, q = e - b * s_maxlen;
    if (q < slen[b]) stoks[b][q] = bd->toks[cur][b][q];
  }
  __syncthreads();
  // 2. candidates in the host driver's order (beam-major, then rank) and their stable sort
  if (tid < nc) {
    const int b = tid / (B + 1);
    const bool ok = stl[tid] > -INFINITY;
    const float lp = ok ? stl[tid] - slse[b] : -INFINITY;
    csc[tid] = slps[b] + (double)lp;
    if (!ok) sti[tid] = 0;
    clive[tid] = stoks[b][slen[b] - 1] != eot;
  }
  __syncthreads();
  if (tid < nc && clive[tid]) {
    int rank = 0;
#pragma unroll 8
    for (int c = 0; c < nc; ++c)
      if (clive[c] && (csc[c] > csc[tid] || (csc[c] == csc[tid] && c < tid))) ++rank;
    order[rank] = tid;
  }
  __syncthreads();
  // The walk over the sorted candidates (end tokens to the finished list until it holds B, stopping
  // there; the first B others become the new beams), done by wave 0 at once, lane q taking sorted
  // position q (nc <= 56 < 64): the counts of end tokens and of others before each position come
  // from ballots.
  if (tid < 64) {
    const int q = tid;
    const u64 lt = (1ull << q) - 1ull;
    const int nlive = __popcll(__ballot(q < nc && clive[q]));
    const bool act = q < nlive;
    const int c = act ? order[q] : 0, b = c / (B + 1);
    const bool is_eot = act && sti[c] == eot;
    const u64 eotm = __ballot(is_eot);
    const int e_before = __popcll(eotm & lt);
    // the walk stops at the first end token that fills the finished list (inclusive)
    const u64 brk = __ballot(is_eot && s_nf0 + e_before + 1 >= B);
    const int qstop = brk ? __ffsll((long long)brk) - 1 : 64;
    const bool proc = act && q <= qstop;
    if (proc && is_eot) {
      fsrc[s_nf0 + e_before] = b;
      fsc[s_nf0 + e_before] = csc[c];
    }
    const u64 keep = __ballot(proc && !is_eot);
    const int n_before = __popcll(keep & lt);
    if (proc && !is_eot && n_before < B) {
      psrc[n_before] = b;
      ptok[n_before] = sti[c];
      plp[n_before] = csc[c];
    }
    const int saved = min(B, __popcll(keep));
    const int nf = s_nf0 + __popcll(eotm & __ballot(proc));
    // leftover beams continue from the first saved one (the lane at n_before == 0)
    const int first = keep ? __ffsll((long long)keep) - 1 : 0;
    const int f_b = __shfl(b, first), f_tok = __shfl(act ? sti[c] : 0, first);
    const double f_lp = __shfl(act ? csc[c] : 0.0, first);
    if (saved > 0 && q >= saved && q < B) {
      psrc[q] = f_b;
      ptok[q] = f_tok;
      plp[q] = f_lp;
    }
    if (q == 0) {
      s_nf = nf;
      s_done = (nlive == 0 || saved == 0 || nf >= B) ? 1 : 0;
    }
  }
  __syncthreads();
  // 3. finished entries of this step: the source beam's tokens (without the end token)
  for (int f = s_nf0; f < s_nf; ++f) {
    const int b = fsrc[f];
    for (int q = tid; q < slen[b]; q += 256) bd->fin_toks[f][q] = stoks[b][q];
  }
  if (tid == 0) {
    for (int f = s_nf0; f < s_nf; ++f) {
      bd->fin_len[f] = slen[fsrc[f]];
      bd->fin_lp[f] = fsc[f];
    }
    bd->nfin = s_nf;
  }
  if (s_done) {
    if (tid == 0) {
      bd->done = 1;
      __hip_atomic_store(&ctl->stop, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  // 4. new beams
  for (int e = tid; e < B * (s_maxlen + 1); e += 256) {
    const int j = e / (s_maxlen + 1), q = e - j * (s_maxlen + 1);
    const int b = psrc[j], lb = slen[b];
    if (q < lb) bd->toks[nxt][j][q] = stoks[b][q];
    else if (q == lb) bd->toks[nxt][j][q] = ptok[j];
  }
  if (tid < B) {
    bd->len[nxt][tid] = slen[psrc[tid]] + 1;
    bd->lps[tid] = plp[tid];
    next_tok[tid] = ptok[tid];
  }
  // 5. slot table: row j continues parent psrc[j] over positions [0, kv)
  for (int p0 = 0; p0 < kv; p0 += kSlotChunk) {
    const int np = min(kSlotChunk, kv - p0);
    for (int e = tid; e < B * np; e += 256) {
      const int r = e / np, q = e - r * np;
      dyn[r * kSlotChunk + q] = slots[(size_t)r * max_ctx + p0 + q];
    }
    __syncthreads();
    for (int e = tid; e < B * np; e += 256) {
      const int r = e / np, q = e - r * np;
      slots[(size_t)r * max_ctx + p0 + q] = dyn[psrc[r] * kSlotChunk + q];
    }
    __syncthreads();
  }
  // 6. next step's suppression mask per beam, built in LDS: suppress list, 3- and 4-gram repeats of
  //    the new history (a match of the last n-1 tokens at i blocks the token after it), timestamp
  //    rules (not the first step)
  uint32_t* msk = reinterpret_cast<uint32_t*>(dyn);
  for (int e = tid; e < B * mw; e += 256) msk[e] = 0u;
  __syncthreads();
  auto set = [&](int j, int t) {
    if (t >= 0 && t < V) atomicOr(msk + (size_t)j * mw + (t >> 5), 1u << (t & 31));
  };
  // tokens [lo, hi) of row j, one word per thread and step (bits of [lo, hi) within each word)
  auto set_range = [&](int j, int lo, int hi) {
    lo = max(lo, 0);
    hi = min(hi, V);
    if (lo >= hi) return;
    for (int w = (lo >> 5) + tid; w <= ((hi - 1) >> 5); w += 256) {
      const int a = max(lo - 32 * w, 0), e = min(hi - 32 * w, 32);  // bits [a, e) of word w
      const uint32_t bits = (e >= 32 ? 0xffffffffu : ((1u << e) - 1u)) & ~((1u << a) - 1u);
      atomicOr(msk + (size_t)j * mw + w, bits);
    }
  };
  __shared__ int s_lastq;
  for (int j = 0; j < B; ++j) {
    const int b = psrc[j], cnt = slen[b] + 1;
    auto g = [&](int q) { return q < cnt - 1 ? stoks[b][q] : ptok[j]; };
    for (int q = tid; q < nsup; q += 256) set(j, q < kBeamSupLds ? ssup[q] : sup[q]);
    for (int nn = 3; nn <= 4; ++nn)
      for (int i = tid; i <= cnt - nn; i += 256) {
        bool match = true;
        for (int q = 0; q < nn - 1; ++q) match &= g(i + q) == g(cnt - (nn - 1) + q);
        if (match) set(j, g(i + nn - 1));
      }
    if (tsb > 0) {
      if (tid == 0) set(j, tsb - 1);
      const bool last_ts = g(cnt - 1) >= tsb;
      const bool pen_ts = cnt < 2 || g(cnt - 2) >= tsb;
      // the last timestamp of the history: the largest position holding one, found in parallel
      if (tid == 0) s_lastq = -1;
      __syncthreads();
      int qmax = -1;
      for (int q = tid; q < cnt; q += 256)
        if (g(q) >= tsb) qmax = q;
      if (qmax >= 0) atomicMax(&s_lastq, qmax);
      __syncthreads();
      const int lastTs = s_lastq >= 0 ? g(s_lastq) : -1;
      __syncthreads();  // s_lastq is reset for the next beam only after every thread has read it
      int lo1 = 0, hi1 = 0, lo2 = 0, hi2 = 0;
      if (last_ts) {
        if (pen_ts) {
          lo1 = tsb;
          hi1 = V;
        } else {
          lo1 = 0;
          hi1 = eot;
        }
      }
      if (lastTs >= 0) {
        lo2 = tsb;
        hi2 = (last_ts && !pen_ts) ? lastTs + 1 : lastTs;
      }
      set_range(j, lo1, hi1);
      set_range(j, lo2, hi2);
    }
  }
  __syncthreads();
  for (int e = tid; e < B * mw; e += 256) mask2[e] = msk[e];
  if (tid == 0) bd->cur = nxt;
}

// Control block of a run (one thread).
__global__ void k_w_setctl(WideCtl* ctl, WideCtl v) {
  if (threadIdx.x == 0) *ctl = v;
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
  // Workgroups of 64 columns (4 waves of 16).  Slices of kb blocks of 128: the longest slice that
  // still gives every compute unit two workgroups, but no more than kWideMaxSlices slices (each
  // consumer adds every slice).
  int kb = 4;
  while (kb > 1 && nblk * ((kbt + kb - 1) / kb) < 2 * n_cu) --kb;
  while (kb < 4 && (kbt + kb - 1) / kb > kWideMaxSlices) ++kb;
  g.nw = 4;
  g.kb = kb;
  g.ks = (kbt + kb - 1) / kb;
  return g;
}

template <int MT, int KB, int NW>
constexpr size_t gemm_lds() {
  return (size_t)2 * MT * 16 * ((4 / NW) * KB * kWideKBlock + kPadH) * sizeof(uint16_t) +
         (size_t)(4 / NW - 1) * NW * MT * 4 * 64 * sizeof(float);
}

template <int MT, int WQ8, int KB, int NW>
static hipError_t gemm_attr() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&k_w_gemm<MT, WQ8, KB, NW>), hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)gemm_lds<MT, KB, NW>());
}

template <int MT, int WQ8, int KB, int NW>
static hipError_t gemm_launch(const GemmArgs& a, int ks, hipStream_t st) {
  const dim3 grid((a.N + 16 * NW - 1) / (16 * NW), ks);
  constexpr size_t lds = gemm_lds<MT, KB, NW>();
  hipLaunchKernelGGL((k_w_gemm<MT, WQ8, KB, NW>), grid, dim3(256), lds, st, a);
  return hipGetLastError();
}

template <int MT, int WQ8>
static hipError_t gemm_mt(int kb, const GemmArgs& a, int ks, hipStream_t st) {
  switch (kb) {
    case 1: return gemm_launch<MT, WQ8, 1, 4>(a, ks, st);
    case 2: return gemm_launch<MT, WQ8, 2, 4>(a, ks, st);
    case 3: return gemm_launch<MT, WQ8, 3, 4>(a, ks, st);
    default: return gemm_launch<MT, WQ8, 4, 4>(a, ks, st);
  }
}

// One GEMM of the step: act rows (row stride 4d) times the weights -> partial sums in p.part.
static hipError_t gemm(const WideParams& p, const WideGemm& g, const void* w, const uint16_t* ws, const float* act, hipStream_t st) {
  GemmArgs a{};
  a.w = w;
  a.ws = ws;
  a.N = g.N;
  a.K = g.K;
  a.act = act;
  a.lda = 4 * p.d;
  a.S = p.S;
  a.part = p.part;
  a.ctl = p.ctl;
  if (p.Rp == 16) return p.wq8 ? gemm_mt<1, 1>(g.kb, a, g.ks, st) : gemm_mt<1, 0>(g.kb, a, g.ks, st);
  return p.wq8 ? gemm_mt<2, 1>(g.kb, a, g.ks, st) : gemm_mt<2, 0>(g.kb, a, g.ks, st);
}

static size_t sstride(const WideParams& p, const WideGemm& g) { return (size_t)p.Rp * g.N; }

template <int WQ8, int NV>
static hipError_t resid_nv(const WideParams& p, int mode, int ks, size_t ss, const float* bias, const float* lg, const float* lb,
                           hipStream_t st) {
  const int lda = 4 * p.d;
  const dim3 grid(p.S), blk(256);
  if (mode == 1)
    hipLaunchKernelGGL((k_w_resid<WQ8, 1, NV>), grid, blk, 0, st, p.ctl, p.tokens0, p.forced, p.next_tok, p.S, p.C, p.emb, p.emb_s, p.pos,
                       p.part, ks, ss, bias, p.x, p.d, lg, lb, p.act, lda);
  else if (mode == 2)
    hipLaunchKernelGGL((k_w_resid<WQ8, 2, NV>), grid, blk, 0, st, p.ctl, p.tokens0, p.forced, p.next_tok, p.S, p.C, p.emb, p.emb_s, p.pos,
                       p.part, ks, ss, bias, p.x, p.d, lg, lb, p.act, lda);
  else
    hipLaunchKernelGGL((k_w_resid<WQ8, 0, NV>), grid, blk, 0, st, p.ctl, p.tokens0, p.forced, p.next_tok, p.S, p.C, p.emb, p.emb_s, p.pos,
                       p.part, ks, ss, bias, p.x, p.d, lg, lb, p.act, lda);
  return hipGetLastError();
}

template <int WQ8>
static hipError_t resid_wq(const WideParams& p, int mode, int ks, size_t ss, const float* bias, const float* lg, const float* lb,
                           hipStream_t st) {
  switch ((p.d + 255) / 256) {
    case 1:
    case 2: return resid_nv<WQ8, 2>(p, mode, ks, ss, bias, lg, lb, st);
    case 3: return resid_nv<WQ8, 3>(p, mode, ks, ss, bias, lg, lb, st);
    case 4: return resid_nv<WQ8, 4>(p, mode, ks, ss, bias, lg, lb, st);
    case 5: return resid_nv<WQ8, 5>(p, mode, ks, ss, bias, lg, lb, st);
    default: return resid_nv<WQ8, kWideVec>(p, mode, ks, ss, bias, lg, lb, st);
  }
}

// Residual update (or layer-0 embedding when g_prev is null) + LayerNorm (lg, lb) -> act.
static hipError_t resid(const WideParams& p, const WideGemm* g_prev, const float* bias, const float* lg, const float* lb,
                        hipStream_t st) {
  const int ks = g_prev ? g_prev->ks : 0;
  const size_t ss = g_prev ? sstride(p, *g_prev) : 0;
  return p.wq8 ? resid_wq<1>(p, g_prev ? 0 : 1, ks, ss, bias, lg, lb, st) : resid_wq<0>(p, g_prev ? 0 : 1, ks, ss, bias, lg, lb, st);
}

// LayerNorm (lg, lb) of x as it is -> act.
static hipError_t ln_only(const WideParams& p, const float* lg, const float* lb, hipStream_t st) {
  return p.wq8 ? resid_wq<1>(p, 2, 0, 0, nullptr, lg, lb, st) : resid_wq<0>(p, 2, 0, 0, nullptr, lg, lb, st);
}

// Whole-K GEMMs (sessions of at most 16 rows).  Four waves over K = d (KS = d / 128 steps each),
// sixteen over K = 4d (MLP2, KS = d / 128).
bool wide_fused_ok(int d, int Rp) { return Rp == 16 && (d == 384 || d == 512 || d == 768 || d == 1024); }

template <int WQ8, int W, int KS, int PRO, int EPI>
static hipError_t fgemm_launch(const FusedArgs& a, hipStream_t st) {
  if (a.K != W * KS * 32 || a.N % 16 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL((k_w_fgemm<WQ8, W, KS, PRO, EPI>), dim3(a.N / 16), dim3(64 * W), 0, st, a);
  return hipGetLastError();
}

template <int WQ8, int PRO, int EPI>
static hipError_t fgemm_d(const FusedArgs& a, hipStream_t st) {
  switch (a.K) {
    case 384: return fgemm_launch<WQ8, 4, 3, PRO, EPI>(a, st);
    case 512: return fgemm_launch<WQ8, 4, 4, PRO, EPI>(a, st);
    case 768: return fgemm_launch<WQ8, 4, 6, PRO, EPI>(a, st);
    case 1024: return fgemm_launch<WQ8, 4, 8, PRO, EPI>(a, st);
    default: return hipErrorInvalidValue;
  }
}

template <int WQ8>
static hipError_t fgemm_4d(const FusedArgs& a, hipStream_t st) {
  switch (a.K) {
    case 4 * 384: return fgemm_launch<WQ8, 16, 3, kProRaw, kFEpiResid>(a, st);
    case 4 * 512: return fgemm_launch<WQ8, 16, 4, kProRaw, kFEpiResid>(a, st);
    case 4 * 768: return fgemm_launch<WQ8, 16, 6, kProRaw, kFEpiResid>(a, st);
    case 4 * 1024: return fgemm_launch<WQ8, 16, 8, kProRaw, kFEpiResid>(a, st);
    default: return hipErrorInvalidValue;
  }
}

// One whole-K GEMM of the step: in rows [S][lda] (LayerNorm lg/lb first when given) times the
// weights [N][K] -> out [S][ldo] through the epilogue.
static hipError_t fgemm(const WideParams& p, const void* w, const uint16_t* ws, int N, int K, const float* in, int lda,
                        const float* lg, const float* lb, int epi, const float* bias, float* out, int ldo, hipStream_t st) {
  FusedArgs a{};
  a.w = w;
  a.ws = ws;
  a.N = N;
  a.K = K;
  a.in = in;
  a.lda = lda;
  a.S = p.S;
  a.g = lg;
  a.b = lb;
  a.bias = bias;
  a.out = out;
  a.ldo = ldo;
  a.ctl = p.ctl;
  if (K == 4 * p.d) return epi == kFEpiResid && !lg ? (p.wq8 ? fgemm_4d<1>(a, st) : fgemm_4d<0>(a, st)) : hipErrorInvalidValue;
  if (lg && epi == kFEpiRaw) return p.wq8 ? fgemm_d<1, kProLn, kFEpiRaw>(a, st) : fgemm_d<0, kProLn, kFEpiRaw>(a, st);
  if (lg && epi == kFEpiGelu) return p.wq8 ? fgemm_d<1, kProLn, kFEpiGelu>(a, st) : fgemm_d<0, kProLn, kFEpiGelu>(a, st);
  if (!lg && epi == kFEpiResid) return p.wq8 ? fgemm_d<1, kProRaw, kFEpiResid>(a, st) : fgemm_d<0, kProRaw, kFEpiResid>(a, st);
  return hipErrorInvalidValue;
}

#define WCHK(x)                          \
  do {                                   \
    const hipError_t e_ = (x);           \
    if (e_ != hipSuccess) return e_;     \
  } while (0)

template <int MT, int WQ8>
static hipError_t prepare_mt() {
  WCHK((gemm_attr<MT, WQ8, 1, 4>()));
  WCHK((gemm_attr<MT, WQ8, 2, 4>()));
  WCHK((gemm_attr<MT, WQ8, 3, 4>()));
  return gemm_attr<MT, WQ8, 4, 4>();
}

hipError_t wide_prepare(int Rp, int wq8) {
  WCHK(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_w_beam), hipFuncAttributeMaxDynamicSharedMemorySize,
                           (int)beam_lds_bytes(kBeamMax, 4096)));
  if (Rp == 16) return wq8 ? prepare_mt<1, 1>() : prepare_mt<1, 0>();
  return wq8 ? prepare_mt<2, 1>() : prepare_mt<2, 0>();
}

// Cross-attention of layer l (chunk partials, then their merge when there is more than one chunk)
// reading the query from q (ks slices of stride ss).
static hipError_t cross(const WideParams& p, int l, const float* q, int ks, size_t ss, hipStream_t st) {
  const LayerDev& lw = p.layers[l];
  const int d = p.d, H = p.H, lda = 4 * d;
  if (p.xvt) {
    // one shared encoder, one row tile, chunks of whole 32-key wave slices (8-byte aligned V^T
    // reads) within the transposed copy's rows
    if (p.X != 1 || p.S > 16 || p.chlen > kXattnKeys || p.chlen % 32 != 0 || (p.nch - 1) * p.chlen + kXattnKeys > p.Ap ||
        p.Ap % 128 != 0)
      return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_w_xattn, dim3(H, p.nch), dim3(256), 0, st, p.ctl, q, ks, ss, lw.b_cq, d, H, p.A, p.Ap, l, p.S,
                       p.chlen, p.nch, p.xk, p.xvt, p.cpart, p.act, lda);
    WCHK(hipGetLastError());
    if (p.nch > 1) {
      hipLaunchKernelGGL(k_w_cmerge, dim3(p.S, H), dim3(64), 0, st, p.ctl, p.cpart, H, p.nch, p.act, lda);
      WCHK(hipGetLastError());
    }
    return hipSuccess;
  }
  const int rg_rows = (p.X == p.S) ? 1 : 8;
  const int ngroups = (p.X == p.S) ? 1 : (p.S + 7) / 8;
  const size_t cross_lds = (size_t)rg_rows * p.chlen * sizeof(float);
  if (rg_rows == 1)
    hipLaunchKernelGGL(k_w_cross<1>, dim3(p.X, H, p.nch * ngroups), dim3(256), cross_lds, st, p.ctl, q, ks, ss,
                       lw.b_cq, d, H, p.A, l, p.L, p.S, p.X, p.chlen, p.nch, p.xk, p.xv, p.cpart, p.act, lda);
  else
    hipLaunchKernelGGL(k_w_cross<8>, dim3(p.X, H, p.nch * ngroups), dim3(256), cross_lds, st, p.ctl, q, ks, ss,
                       lw.b_cq, d, H, p.A, l, p.L, p.S, p.X, p.chlen, p.nch, p.xk, p.xv, p.cpart, p.act, lda);
  WCHK(hipGetLastError());
  if (p.nch > 1) {
    hipLaunchKernelGGL(k_w_cmerge, dim3(p.S, H), dim3(64), 0, st, p.ctl, p.cpart, H, p.nch, p.act, lda);
    WCHK(hipGetLastError());
  }
  return hipSuccess;
}

// Logits GEMM, selection and (device beam search) the beam step, after the final LayerNorm.
static hipError_t enqueue_head(const WideParams& p, hipStream_t st) {
  WCHK(gemm(p, p.g_v, p.emb, p.emb_s, p.act, st));
  const int nblk = (p.nsel + 3) / 4;
  hipLaunchKernelGGL(k_w_select, dim3(p.S, nblk), dim3(256), 0, st, p.ctl, p.part, p.g_v.ks, sstride(p, p.g_v), p.S, p.V, p.mask,
                     p.mask2, p.mw, p.bias, p.selp, p.nsel, p.logits_out);
  WCHK(hipGetLastError());
  hipLaunchKernelGGL(k_w_selmerge, dim3(p.S), dim3(64), 0, st, p.ctl, p.selp, p.S, p.nsel, p.out, p.next_tok);
  WCHK(hipGetLastError());
  if (p.beam_dev) {
    hipLaunchKernelGGL(k_w_beam, dim3(1), dim3(256), beam_lds_bytes(p.S, p.mw), st, p.ctl, p.beam_dev, p.out, p.S, p.beam_eot,
                       p.beam_tsb, p.beam_sup,
                       p.beam_nsup, p.V, p.mw, const_cast<uint32_t*>(p.mask2), const_cast<int32_t*>(p.slots), p.max_ctx, p.next_tok);
    WCHK(hipGetLastError());
  }
  return hipSuccess;
}

// The kernels of one step with whole-K GEMMs (at most 16 rows): 8 or 9 per layer, the residual
// updates, LayerNorms and GELU inside the GEMMs.
static hipError_t enqueue_step_fused(const WideParams& p, hipStream_t st) {
  const int d = p.d, H = p.H, lda = 4 * d;
  const size_t self_lds = (size_t)(p.max_ctx + 1) * sizeof(float);
  WCHK(resid(p, nullptr, nullptr, p.layers[0].ln1_g, p.layers[0].ln1_b, st));  // x = embedding + position
  for (int l = 0; l < p.L; ++l) {
    const LayerDev& lw = p.layers[l];
    WCHK(fgemm(p, lw.w_qkv, lw.s_qkv, 3 * d, d, p.x, d, lw.ln1_g, lw.ln1_b, kFEpiRaw, nullptr, p.part, 3 * d, st));
    hipLaunchKernelGGL(k_w_self, dim3(p.S, H), dim3(256), self_lds, st, p.ctl, p.part, 1, (size_t)0, lw.b_qkv, d, H,
                       l, p.S, p.max_ctx, p.kv_k, p.kv_v, p.slots, p.act, lda);
    WCHK(hipGetLastError());
    WCHK(fgemm(p, lw.w_o, lw.s_o, d, d, p.act, lda, nullptr, nullptr, kFEpiResid, lw.b_o, p.x, d, st));
    WCHK(fgemm(p, lw.w_cq, lw.s_cq, d, d, p.x, d, lw.ln2_g, lw.ln2_b, kFEpiRaw, nullptr, p.part, d, st));
    WCHK(cross(p, l, p.part, 1, 0, st));
    WCHK(fgemm(p, lw.w_co, lw.s_co, d, d, p.act, lda, nullptr, nullptr, kFEpiResid, lw.b_co, p.x, d, st));
    WCHK(fgemm(p, lw.w_1, lw.s_1, 4 * d, d, p.x, d, lw.ln3_g, lw.ln3_b, kFEpiGelu, lw.b_1, p.hid, lda, st));
    WCHK(fgemm(p, lw.w_2, lw.s_2, d, 4 * d, p.hid, lda, nullptr, nullptr, kFEpiResid, lw.b_2, p.x, d, st));
  }
  WCHK(ln_only(p, p.lnf_g, p.lnf_b, st));
  WCHK(enqueue_head(p, st));
  return hipGetLastError();
}

// The kernels of one step; every per-step value comes from the control block.
static hipError_t enqueue_step(const WideParams& p, hipStream_t st) {
  if (wide_fused_ok(p.d, p.Rp) && !p.no_fuse) return enqueue_step_fused(p, st);
  const int d = p.d, H = p.H, lda = 4 * d;
  const size_t self_lds = (size_t)(p.max_ctx + 1) * sizeof(float);
  for (int l = 0; l < p.L; ++l) {
    const LayerDev& lw = p.layers[l];
    if (l == 0) WCHK(resid(p, nullptr, nullptr, lw.ln1_g, lw.ln1_b, st));
    else WCHK(resid(p, &p.g_2, p.layers[l - 1].b_2, lw.ln1_g, lw.ln1_b, st));
    WCHK(gemm(p, p.g_qkv, lw.w_qkv, lw.s_qkv, p.act, st));
    hipLaunchKernelGGL(k_w_self, dim3(p.S, H), dim3(256), self_lds, st, p.ctl, p.part, p.g_qkv.ks, sstride(p, p.g_qkv), lw.b_qkv, d, H,
                       l, p.S, p.max_ctx, p.kv_k, p.kv_v, p.slots, p.act, lda);
    WCHK(hipGetLastError());
    WCHK(gemm(p, p.g_o, lw.w_o, lw.s_o, p.act, st));
    WCHK(resid(p, &p.g_o, lw.b_o, lw.ln2_g, lw.ln2_b, st));
    WCHK(gemm(p, p.g_cq, lw.w_cq, lw.s_cq, p.act, st));
    WCHK(cross(p, l, p.part, p.g_cq.ks, sstride(p, p.g_cq), st));
    WCHK(gemm(p, p.g_co, lw.w_co, lw.s_co, p.act, st));
    WCHK(resid(p, &p.g_co, lw.b_co, lw.ln3_g, lw.ln3_b, st));
    WCHK(gemm(p, p.g_1, lw.w_1, lw.s_1, p.act, st));
    hipLaunchKernelGGL(k_w_gelu, dim3((p.S * 4 * d + 255) / 256), dim3(256), 0, st, p.ctl, p.part, p.g_1.ks, sstride(p, p.g_1), lw.b_1, p.S,
                       4 * d, p.hid, lda);
    WCHK(hipGetLastError());
    WCHK(gemm(p, p.g_2, lw.w_2, lw.s_2, p.hid, st));
  }
  WCHK(resid(p, &p.g_2, p.layers[p.L - 1].b_2, p.lnf_g, p.lnf_b, st));
  WCHK(enqueue_head(p, st));
  return hipGetLastError();
}

void wide_graph_release(WideGraph* g) {
  if (g && g->exec) {
    (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(g->exec));
    g->exec = nullptr;
  }
}

hipError_t launch_wide(const WideParams& p, hipStream_t st) {
  WideCtl c{};
  c.i = 0;
  c.kv_len0 = p.kv_len0;
  c.forced_on = p.forced != nullptr;
  c.out_on = p.out != nullptr;
  c.logits_on = p.logits_out != nullptr;
  c.mask_on = p.mask != nullptr;
  c.mask2_on = p.mask2 != nullptr;
  c.slots_on = p.slots != nullptr;
  c.bias_on = p.bias_on;
  c.topk = p.topk;
  c.probe = p.probe;
  c.done = 0;
  c.tok_dev = p.tok_dev;
  c.stop = 0;
  hipLaunchKernelGGL(k_w_setctl, dim3(1), dim3(64), 0, st, p.ctl, c);
  WCHK(hipGetLastError());
  if (!p.graph) {
    for (int i = 0; i < p.nsteps; ++i) WCHK(enqueue_step(p, st));
    return hipSuccess;
  }
  // Buffers a step reads or writes that may be (re)allocated between runs: the captured step is
  // valid while they stay where they were.
  const void* key[8] = {p.tokens0, p.forced, p.out, p.logits_out, p.mask2, p.mask, p.slots, p.ctl};
  // and the beam-search arguments baked into the captured beam kernel (compared exactly)
  const uintptr_t bkey[6] = {(uintptr_t)p.beam_dev, (uintptr_t)p.beam_sup, (uintptr_t)p.beam_nsup, (uintptr_t)p.beam_eot,
                             (uintptr_t)p.beam_tsb, (uintptr_t)1};
  bool same = p.graph->exec != nullptr;
  for (int k = 0; k < 8 && same; ++k) same = key[k] == nullptr || key[k] == p.graph->key[k];
  for (int k = 0; k < 6 && same; ++k) same = bkey[k] == p.graph->bkey[k];
  if (!same) {
    // capture with every optional buffer present in the key, so later runs that leave some out
    // (null: switched off in the control block) replay the same graph
    WideParams q = p;
    for (int k = 0; k < 8; ++k)
      if (key[k] == nullptr) key[k] = p.graph->key[k];
    q.tokens0 = static_cast<const int32_t*>(key[0]);
    q.forced = static_cast<const int32_t*>(key[1]);
    q.out = static_cast<w4h_step_out*>(const_cast<void*>(key[2]));
    q.logits_out = static_cast<float*>(const_cast<void*>(key[3]));
    q.mask2 = static_cast<const uint32_t*>(key[4]);
    q.mask = static_cast<const uint32_t*>(key[5]);
    q.slots = static_cast<const int32_t*>(key[6]);
    wide_graph_release(p.graph);
    // Captured on a stream of its own that does not synchronize with the legacy stream, in this
    // thread's capture mode: other threads may keep using the legacy stream (memsets, copies of
    // their sessions) while the capture is open.  Capturing runs nothing, so the step needs no
    // ordering with st here; every replay is launched on st.
    hipStream_t cs = nullptr;
    WCHK(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
    hipGraph_t graph = nullptr;
    hipError_t be = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
    const hipError_t ce = be == hipSuccess ? enqueue_step(q, cs) : be;
    const hipError_t ee = be == hipSuccess ? hipStreamEndCapture(cs, &graph) : be;
    (void)hipStreamDestroy(cs);
    WCHK(ce);
    WCHK(ee);
    hipGraphExec_t exec = nullptr;
    const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    WCHK(ie);
    p.graph->exec = exec;
    for (int k = 0; k < 8; ++k) p.graph->key[k] = key[k];
    for (int k = 0; k < 6; ++k) p.graph->bkey[k] = bkey[k];
  }
  for (int i = 0; i < p.nsteps; ++i) WCHK(hipGraphLaunch(static_cast<hipGraphExec_t>(p.graph->exec), st));
  return hipSuccess;
}

}  // namespace w4h
