// Device temperature sampling for decodes at T > 0 (WhisperDecoder.sample and the log-probability
// the decode loop adds for the sampled token, main/nn/WhisperDecoder.java:176-195, 576-598,
// 614-626).  In a sampled decode the step kernel runs one step per launch and leaves the raw logits
// row in device memory; the masking kernel applies the rules that depend on the generated tokens,
// and the sampling kernel draws the token and leaves it as the next launch's input, so a sampled
// decode needs no logits row on the host and no host round trip per token.
//
// Arithmetic follows the reference's: x = (l - max) / T in float, p = exp((double) x) rounded to
// float for the cumulative weights, the total from the unrounded double p, r = u * total, the first
// index whose cumulative weight reaches r (the last index when none does).  The log-probability is
// taken over the row the sampling rewrote (the reference's logSoftmax runs on the weights):
// (p_k - 1) - log(sum exp(p_i - 1)), the row maximum being exactly 1.  Sums run as per-thread
// sequential sums combined by trees and scans instead of one sequential loop, which changes them
// only in the last bits of a double.

#include "w4h_kernels.h"

namespace w4h {

// Exclusive scan over the block (256 threads) of per-thread doubles, in thread order; *total gets the
// block sum.  red: 4 doubles of LDS.
DEV double block_scan_excl(double v, double* red, double* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const double inc = wave_scan_d(v);
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  double t = 0.0, pre = __shfl_up(inc, 1);
  pre = lane == 0 ? 0.0 : pre;
  for (int w = 0; w < 4; ++w) {
    pre += w < wave ? red[w] : 0.0;
    t += red[w];
  }
  *total = t;
  __syncthreads();
  return pre;
}

// Loads this thread's kSamplePer entries of the row (entries past V read as -inf).
DEV void load_entries(const float* row, int i0, int V, float (&v)[kSamplePer]) {
  if (i0 + kSamplePer - 1 < V) {
    const float4 q = *reinterpret_cast<const float4*>(row + i0);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
#pragma unroll
    for (int e = 0; e < kSamplePer; ++e) v[e] = i0 + e < V ? row[i0 + e] : -INFINITY;
  }
}

// The decode rules that depend on the generated tokens (st->hist): the suppress bitmask, applyNgramBlock for n = 3
// and 4 (:472-476, 543-564) and applyTimestampRules after the first step (:484-541) set entries of
// the block's range to -inf in place; the block's maximum goes to parts_out[b].
__global__ void __launch_bounds__(kThreads) k_sample_mask(SampleParams p) {
  __shared__ int hist[kSampleHist];
  __shared__ uint32_t bits[kSampleSpan / 32];
  __shared__ int ts_w[4];
  __shared__ float fmax_w[4];
  __shared__ int rng_lo[4], rng_hi[4], nrng;
  const SampleDev* st = p.st;
  if (st->stop) return;  // the decode has ended (uniform)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x;
  const int n = st->n, V = p.V, tsb = p.tsb, lo = b * kSampleSpan;
  for (int i = tid; i < kSampleSpan / 32; i += kThreads) {
    const int w = lo / 32 + i;
    bits[i] = (p.sup && w < (V + 31) / 32) ? p.sup[w] : 0u;
  }
  for (int i = tid; i < n; i += kThreads) hist[i] = st->hist[i];
  __syncthreads();
  const int l1 = n >= 1 ? hist[n - 1] : -1, l2 = n >= 2 ? hist[n - 2] : -1, l3 = n >= 3 ? hist[n - 3] : -1;
  int last_ts = -1;
  for (int i = tid; i < n; i += kThreads) {
    if (tsb > 0 && hist[i] >= tsb) last_ts = i;
    int t = -1;
    if (i <= n - 3 && hist[i] == l2 && hist[i + 1] == l1) t = hist[i + 2];
    if (t >= lo && t < lo + kSampleSpan && t < V) atomicOr(&bits[(t - lo) >> 5], 1u << (t & 31));
    t = -1;
    if (i <= n - 4 && hist[i] == l3 && hist[i + 1] == l2 && hist[i + 2] == l1) t = hist[i + 3];
    if (t >= lo && t < lo + kSampleSpan && t < V) atomicOr(&bits[(t - lo) >> 5], 1u << (t & 31));
  }
  last_ts = -wave_min_i(-last_ts);
  if (lane == 0) ts_w[wave] = last_ts;
  __syncthreads();
  if (tid == 0) {
    int k = 0;
    if (tsb > 0) {
      rng_lo[k] = tsb - 1;
      rng_hi[k++] = tsb;
      if (n > 0) {
        const int lt = max(max(ts_w[0], ts_w[1]), max(ts_w[2], ts_w[3]));
        const bool last_was = hist[n - 1] >= tsb, pen_was = n < 2 || hist[n - 2] >= tsb;
        if (last_was) {
          rng_lo[k] = pen_was ? tsb : 0;
          rng_hi[k++] = pen_was ? V : p.eot;
        }
        if (lt >= 0) {
          rng_lo[k] = tsb;
          rng_hi[k++] = (last_was && !pen_was) ? hist[lt] + 1 : hist[lt];
        }
      }
    }
    nrng = k;
  }
  __syncthreads();
  const int i0 = lo + tid * kSamplePer, nr = nrng;
  float v[kSamplePer];
  load_entries(p.logits, i0, V, v);
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < kSamplePer; ++e) {
    const int t = i0 + e;
    bool m = t >= V || ((bits[(t - lo) >> 5] >> (t & 31)) & 1u);
    for (int k = 0; k < nr; ++k) m = m || (t >= rng_lo[k] && t < rng_hi[k]);
    v[e] = m ? -INFINITY : v[e];
    mx = fmaxf(mx, v[e]);
    if (t < V) p.logits[t] = v[e];
  }
  mx = wave_max(mx);
  if (lane == 0) fmax_w[wave] = mx;
  __syncthreads();
  if (tid == 0) p.parts_out[b] = (u64)__float_as_uint(fmaxf(fmaxf(fmax_w[0], fmax_w[1]), fmaxf(fmax_w[2], fmax_w[3])));
}

__global__ void __launch_bounds__(kThreads) k_sample(SampleParams p) {
  __shared__ float fmax_w[4];
  __shared__ double dred[3][4];
  __shared__ int last, pick;
  __shared__ float pick_pf;
  __shared__ double s_r, s_se, s_pre;
  __shared__ int s_blk;
  SampleDev* st = p.st;
  if (st->stop) return;  // the decode has ended: the later steps of the run do nothing (uniform)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x;
  const int V = p.V, i0 = b * kSampleSpan + tid * kSamplePer;
  // the row maximum from the maxima of its parts
  float mx = -INFINITY;
  for (int k = tid; k < p.nparts; k += kThreads) mx = fmaxf(mx, __uint_as_float((unsigned)p.parts[(size_t)k * p.part_stride]));
  mx = wave_max(mx);
  if (lane == 0) fmax_w[wave] = mx;
  if (tid == 0) pick = 0x7fffffff;
  __syncthreads();
  const float M = fmaxf(fmaxf(fmax_w[0], fmax_w[1]), fmaxf(fmax_w[2], fmax_w[3]));
  // weights p = exp((l - M) / T) (float quotient widened, exp in double), pf = (float) p over the row
  float* row = p.logits;
  float v[kSamplePer];
  load_entries(row, i0, V, v);
  const float T = p.temperature;
  double sd = 0.0, sf = 0.0, se = 0.0;
  float w[kSamplePer];
#pragma unroll
  for (int e = 0; e < kSamplePer; ++e) {
    const bool in = i0 + e < V;
    const double ex = exp((double)((v[e] - M) / T));
    w[e] = in ? (float)ex : 0.f;
    sd += in ? ex : 0.0;
    sf += (double)w[e];
    se += in ? exp((double)(w[e] - 1.0f)) : 0.0;
  }
  if (i0 + kSamplePer - 1 < V) {
    *reinterpret_cast<float4*>(row + i0) = make_float4(w[0], w[1], w[2], w[3]);
  } else {
#pragma unroll
    for (int e = 0; e < kSamplePer; ++e)
      if (i0 + e < V) row[i0 + e] = w[e];
  }
  sd = wave_sum_d(sd);
  sf = wave_sum_d(sf);
  se = wave_sum_d(se);
  if (lane == 0) {
    dred[0][wave] = sd;
    dred[1][wave] = sf;
    dred[2][wave] = se;
  }
  __syncthreads();
  if (tid < 3) st->bsum[b][tid] = ((dred[tid][0] + dred[tid][1]) + dred[tid][2]) + dred[tid][3];
  // the last block to finish draws the token: every thread's weight stores and the block sums are
  // made visible at device scope before the arrival is counted
  __threadfence();
  __syncthreads();
  if (tid == 0) last = atomicAdd(&st->done, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  __threadfence();
  // totals and block prefixes in vocabulary order (lane k of wave 0 takes block k), the draw, then
  // the first index whose cumulative weight reaches r, from the block where the block sums cross it
  if (wave == 0) {
    const bool in = lane < (int)gridDim.x;
    const double bsd = in ? ld_agent(&st->bsum[lane][0]) : 0.0;
    const double bsf = in ? ld_agent(&st->bsum[lane][1]) : 0.0;
    const double bse = in ? ld_agent(&st->bsum[lane][2]) : 0.0;
    const double SD = wave_sum_d(bsd), SE = wave_sum_d(bse);
    const double inc = wave_scan_d(bsf);
    double exc = __shfl_up(inc, 1);
    exc = lane == 0 ? 0.0 : exc;
    const double r = splitmix_uniform(p.rng, st->steps + 1) * SD;
    const unsigned long long hit = __ballot(in && inc >= r);
    const int blk = hit ? __ffsll((long long)hit) - 1 : (int)gridDim.x;
    const double pre = __shfl(exc, blk < 64 ? blk : 0);
    if (lane == 0) {
      s_r = r;
      s_se = SE;
      s_pre = blk < (int)gridDim.x ? pre : 0.0;
      s_blk = blk;
    }
  }
  __syncthreads();
  const double r = s_r;
  double pre = s_pre;
  for (int blk = s_blk; blk < (int)gridDim.x; ++blk) {
    const int j0 = blk * kSampleSpan + tid * kSamplePer;
    float q[kSamplePer];
    double ts = 0.0;
#pragma unroll
    for (int e = 0; e < kSamplePer; ++e) {
      q[e] = j0 + e < V ? __hip_atomic_load(row + j0 + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      ts += (double)q[e];
    }
    double btot;
    double c = pre + block_scan_excl(ts, &dred[0][0], &btot);
    int cand = 0x7fffffff;
    float cpf = 0.f;
#pragma unroll
    for (int e = 0; e < kSamplePer; ++e) {
      c += (double)q[e];
      const bool h = cand == 0x7fffffff && j0 + e < V && c >= r;
      cand = h ? j0 + e : cand;
      cpf = h ? q[e] : cpf;
    }
    if (cand != 0x7fffffff) atomicMin(&pick, cand);
    __syncthreads();
    if (cand != 0x7fffffff && cand == pick) pick_pf = cpf;
    __syncthreads();
    if (pick != 0x7fffffff) break;
    pre += btot;
  }
  if (tid == 0) {
    int tok = pick;
    float pf = pick_pf;
    if (tok == 0x7fffffff) {  // no cumulative weight reached r: the reference returns the last index
      tok = V - 1;
      pf = __hip_atomic_load(row + V - 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int k = st->steps, n = st->n;
    st->out_tok[k] = tok;
    st->lp[k] = (double)(pf - 1.0f) - log(s_se);
    st->steps = k + 1;
    st->done = 0u;  // every block has arrived: ready for the next launch
    if (tok == p.eot) {
      st->stop = 1;
    } else {
      st->hist[n] = tok;
      st->n = n + 1;
      for (int q = 0; q < p.rows; ++q) st->tok[q] = tok;
      if (k + 1 >= p.max_steps || n + 1 >= kSampleHist) st->stop = 1;
    }
  }
}

hipError_t launch_sample_mask(const SampleParams& p, hipStream_t st) {
  hipLaunchKernelGGL(k_sample_mask, dim3(kSampleBlocks), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_sample(const SampleParams& p, hipStream_t st) {
  hipLaunchKernelGGL(k_sample, dim3(kSampleBlocks), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace w4h
