#pragma once
// Device code of whisper4j_amd for gfx950 (CDNA4, wave64): building blocks, phases and the
// persistent step kernel template, included by the step translation units (w4h_step_*.hip) and by
// w4h_device.hip (cross-K/V projection, op kernels, launchers).
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
constexpr int KPT_SELF = kSelfChunk / 32;   // keys per thread, self-attention chunk
constexpr int KPT_CROSS = kMaxChunk / 32;   // keys per thread, cross-attention chunk
constexpr int kPollBatch = 8;   // tagged words a polling lane keeps in flight (sparse waits)
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

// Raw buffer loads: the descriptor carries the buffer size, and the hardware returns zero for any
// access past it, so disabled lanes load from kOOB instead of branching around the load.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOB = 0x80000000u;  // beyond every buffer this library creates (< 2 GiB)
DEV __amdgpu_buffer_rsrc_t brsrc(const void* base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)(bytes > 0x7fffffffu ? 0x7fffffffu : bytes),
                                           0x00020000);
}
DEV uint4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
DEV uint16_t bld2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// Self-KV rows: written with device-coherent (sc1, write-through) stores and read back with sc1
// loads by other workgroups at later steps of the same launch.  kv_drain() waits until this
// wave's stores have completed before it publishes anything that comes after them.
DEV void kv_store(uint16_t* base, size_t bytes, size_t elem, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, brsrc(base, bytes), (int)(elem * 2), 0, 16);
}
DEV void kv_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0), expcnt and lgkmcnt untouched */ }

DEV u64 ll_ld(const u64* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Publish one tagged word to every replica of an exchange buffer (replica r sits rs words after
// replica r - 1).  Consumers poll the replica of their own workgroup (blockIdx % kRep), which
// spreads the polling load of ~100 consumer workgroups over kRep copies of each word.
DEV void ll_st(u64* p, float v, uint32_t tag, size_t rs) {
  const u64 w = ((u64)tag << 32) | (u64)__float_as_uint(v);
#pragma unroll
  for (int r = 0; r < kRep; ++r) __hip_atomic_store(p + r * rs, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The error word and, just before it (8-byte aligned), the session's cancel word, which the host
// may set while a launch runs: one 8-byte load covers both.
DEV bool aborted(const unsigned* err) {
  return __hip_atomic_load(reinterpret_cast<const unsigned long long*>(err - 1), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT) != 0ull;
}
DEV void raise_err(unsigned* err, unsigned code) {
  __hip_atomic_fetch_or(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// DPP lane moves (gfx9 dpp_ctrl encodings): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141 (lane i <-> 7-i within 8), row_mirror = 0x140 (i <-> 15-i within 16),
// row_ror:8 = 0x128, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROWMASK = 0xF, bool BC = true>
DEV float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xF, BC));
}
// Sum over each aligned group of 8 lanes; every lane of the group gets it.
DEV float sum8(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v;
}
// Sum over each row of 16 lanes.
DEV float sum16(float v) {
  v = sum8(v);
  v += dpp<0x140>(v);
  return v;
}
DEV float wave_sum(float v) {
  v = sum16(v);
  // rows -> lane 63: row_bcast:15 adds row r's lane 15 into row r+1, row_bcast:31 lane 31 into rows 2-3
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
DEV float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), 0x142, 0xA, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), 0x143, 0xC, 0xF, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
DEV int wave_min_i(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, true));
  v = min(v, __builtin_amdgcn_update_dpp(0x7fffffff, v, 0x142, 0xA, 0xF, false));
  v = min(v, __builtin_amdgcn_update_dpp(0x7fffffff, v, 0x143, 0xC, 0xF, false));
  return __builtin_amdgcn_readlane(v, 63);
}

// (value, index) maximum over the wave; equal values keep the lower index, NaN never wins.  Two
// DPP reductions: the maximum value, then the lowest index that holds it.  Every lane gets both.
DEV void wave_argmax(float& v, int& i) {
  const float m = wave_max(v);
  i = wave_min_i(v == m ? i : 0x7fffffff);
  v = m;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations (lgkmcnt), not for
// its global loads and stores, so weight and key/value prefetches stay in flight across it.  No
// phase needs global memory written by one wave to be read by another wave of the same workgroup
// (workgroups exchange data only through tagged words), so every barrier in the step is this one.
DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The k-th SplitMix64 output after `state` (k >= 1) as a double in [0, 1): the draw the host decode
// loop's generator returns on its k-th call.
DEV double splitmix_uniform(uint64_t state, int k) {
  uint64_t z = state + (uint64_t)k * 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  z ^= z >> 31;
  return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

DEV double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Inclusive scan over the wave's lanes, in lane order.
DEV double wave_scan_d(double v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double u = __shfl_up(v, o);
    if (lane >= o) v += u;
  }
  return v;
}

DEV double ld_agent(const double* p) {
  return __longlong_as_double((long long)__hip_atomic_load(reinterpret_cast<const unsigned long long*>(p),
                                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// OR of `pred` over the workgroup through LDS (LDS-only barriers); the second barrier keeps the
// vote words from being rewritten by a later call before every wave has read them.
DEV bool wg_any(bool pred) {
  __shared__ int votes[4];
  const bool any = __any(pred);
  if ((threadIdx.x & 63) == 0) votes[threadIdx.x >> 6] = any ? 1 : 0;
  lds_barrier();
  const bool r = (votes[0] | votes[1] | votes[2] | votes[3]) != 0;
  lds_barrier();
  return r;
}

// Sum over the workgroup; every thread receives the result.  scratch: 4 floats of LDS.
DEV float wg_sum(float v, float* scratch) {
  v = wave_sum(v);
  lds_barrier();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  lds_barrier();
  return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

// ------------------------------------------------------------------------------------------------
// tagged-word polling

// Poll words [0, n0) of src0 and [0, n1) of src1 until every word carries `tag`, then copy the
// values into dst0 / dst1 (LDS).  Each thread keeps PB words in flight per round (a round covers
// PB * kThreads words).  Returns false (uniformly across the workgroup) when the wait expired or
// another workgroup aborted.
template <int PB>
DEV bool ll_poll2(const u64* src0, int n0, float* dst0, const u64* src1, int n1, float* dst1, uint32_t tag,
                  unsigned* err) {
  const int total = n0 + n1;
  bool fail = false;
  for (int base = 0; base < total && !fail; base += kThreads * PB) {
    u64 v[PB];
#pragma unroll
    for (int u = 0; u < PB; ++u) {
      const int i = base + u * kThreads + (int)threadIdx.x;
      v[u] = i < n0 ? ll_ld(src0 + i) : (i < total ? ll_ld(src1 + (i - n0)) : ((u64)tag << 32));
    }
    unsigned spins = 0;
    while (true) {
      bool ok = true;
#pragma unroll
      for (int u = 0; u < PB; ++u)
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
      for (int u = 0; u < PB; ++u) {
        const int i = base + u * kThreads + (int)threadIdx.x;
        if (i < n0)
          dst0[i] = __uint_as_float((uint32_t)v[u]);
        else if (i < total)
          dst1[i - n0] = __uint_as_float((uint32_t)v[u]);
      }
    }
  }
  return !wg_any(fail);
}

template <int PB>
DEV bool ll_poll1(const u64* src, int n, float* dst, uint32_t tag, unsigned* err) {
  return ll_poll2<PB>(src, n, dst, nullptr, 0, nullptr, tag, err);
}

// Cheap readiness wait before a full read: one wave polls the words k*stride + off1 (and + off2
// when off2 >= 0) for k < nrec with a short sleep between rounds.  These are the last words each
// producer writes, so the full read that follows normally finds every tag in place on its first
// round (it still verifies every word).  Keeps the number of polling loads in flight low.
DEV bool ll_wait_sparse(const u64* src, int nrec, int stride, int off1, int off2, uint32_t tag, unsigned* err) {
  bool fail = false;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int per = off2 >= 0 ? 2 : 1;
    const int total = nrec * per;
    for (int base = 0; base < total && !fail; base += 64 * kPollBatch) {
      unsigned spins = 0;
      while (true) {
        bool ok = true;
#pragma unroll
        for (int u = 0; u < kPollBatch; ++u) {
          const int i = base + u * 64 + lane;
          if (i < total) {
            const int k = i / per, w = (per == 2 && (i & 1)) ? off2 : off1;
            ok &= (uint32_t)(ll_ld(src + (size_t)k * stride + w) >> 32) == tag;
          }
        }
        if (__all(ok)) break;
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
        __builtin_amdgcn_s_sleep(2);
      }
    }
  }
  return !wg_any(fail);
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
  const bool rok = gr < N;
  if (!WQ8) {
    const int nch = K >> 3;
    const auto rs = brsrc(W, (size_t)N * K * 2);
    const uint32_t base = (uint32_t)gr * (uint32_t)K * 2u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = slot + 32 * r;
      wr.w[r] = bld16(rs, (rok && c < nch) ? base + (uint32_t)c * 16u : kOOB);
    }
  } else {
    const int nch = K >> 4;
    const auto rs = brsrc(W, (size_t)N * K);
    const auto ss = brsrc(Ws, (size_t)N * (K >> 5) * 2);
    const uint32_t base = (uint32_t)gr * (uint32_t)K, sbase = (uint32_t)gr * (uint32_t)(K >> 5) * 2u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = slot + 32 * r;
      const bool ok = rok && c < nch;
      wr.w[r] = bld16(rs, ok ? base + (uint32_t)c * 16u : kOOB);
      wr.s[r] = bld2(ss, ok ? sbase + (uint32_t)(c >> 1) * 2u : kOOB);
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

// Chunks of a row beyond the R prefetched rounds: loaded here, four rounds at a time, with a
// round count that is uniform across the wave (disabled lanes load zeros).
template <int R, int WQ8, int SM>
DEV void stream_rest(const void* W, const uint16_t* Ws, int N, int K, int gr, int slot, int S, const float* x,
                     float (&acc)[SM]) {
  const int nch = WQ8 ? (K >> 4) : (K >> 3);
  const int extra = nch - 32 * R;  // chunks not prefetched (per row)
  if (extra <= 0) return;
  const auto rs = brsrc(W, (size_t)N * K * (WQ8 ? 1 : 2));
  const auto ss = brsrc(Ws, WQ8 ? (size_t)N * (K >> 5) * 2 : 0);
  const uint32_t base = (uint32_t)gr * (uint32_t)K * (WQ8 ? 1u : 2u);
  const uint32_t sbase = (uint32_t)gr * (uint32_t)(K >> 5) * 2u;
  for (int c0 = 32 * R; c0 < nch; c0 += 32 * 4) {
    uint4 t[4];
    uint16_t ts[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + slot + 32 * u;
      t[u] = bld16(rs, c < nch ? base + (uint32_t)c * 16u : kOOB);
      if (WQ8) ts[u] = bld2(ss, c < nch ? sbase + (uint32_t)(c >> 1) * 2u : kOOB);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + slot + 32 * u;
      if (c < nch) {
#pragma unroll
        for (int s = 0; s < SM; ++s)
          if (s < S) {
            if (WQ8)
              acc[s] = fmaf(h2f(ts[u]), dot16_q8(t[u], x + s * K + c * 16), acc[s]);
            else
              acc[s] += dot8_f16(t[u], x + s * K + c * 8);
          }
      }
    }
  }
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
      stream_rest<R, 0, SM>(W, Ws, N, K, gr, slot, S, x, acc);
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
      stream_rest<R, 1, SM>(W, Ws, N, K, gr, slot, S, x, acc);
    }
  }
#pragma unroll
  for (int s = 0; s < SM; ++s) acc[s] = sum8(acc[s]);
  if (sub == 0) {
#pragma unroll
    for (int s = 0; s < SM; ++s)
      if (s < S) red[((w << 3) + row) * SM + s] = acc[s];
  }
  lds_barrier();
  if (tid < 8 * S) {
    const int s = tid >> 3, rr = tid & 7;
    out[s * 8 + rr] = (red[rr * SM + s] + red[(8 + rr) * SM + s]) + (red[(16 + rr) * SM + s] + red[(24 + rr) * SM + s]);
  }
  lds_barrier();
}

// Batched GEMV: NB items of 8 rows (item i covers rows (it0 + i * istr) * 8 .. + 8, i < nit) with
// one cross-wave reduction for the whole batch.  Same lane layout as above.
template <int R, int NB>
struct WBatch {
  uint4 w[NB][R];
  uint16_t s[NB][R];
};

template <int R, int NB, int WQ8>
DEV void gemvb_prefetch(const void* W, const uint16_t* Ws, int N, int K, int it0, int istr, int nit,
                        WBatch<R, NB>& wb) {
  const int tid = threadIdx.x, lane = tid & 63, row = lane >> 3, slot = ((tid >> 6) << 3) | (lane & 7);
  const int nch = WQ8 ? (K >> 4) : (K >> 3);
  const auto rs = brsrc(W, (size_t)N * K * (WQ8 ? 1 : 2));
  const auto ss = brsrc(Ws, WQ8 ? (size_t)N * (K >> 5) * 2 : 0);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int gr = (it0 + i * istr) * 8 + row;
    const bool rok = i < nit && gr < N;
    const uint32_t base = (uint32_t)gr * (uint32_t)K * (WQ8 ? 1u : 2u);
    const uint32_t sbase = (uint32_t)gr * (uint32_t)(K >> 5) * 2u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = slot + 32 * r;
      const bool ok = rok && c < nch;
      wb.w[i][r] = bld16(rs, ok ? base + (uint32_t)c * 16u : kOOB);
      if (WQ8) wb.s[i][r] = bld2(ss, ok ? sbase + (uint32_t)(c >> 1) * 2u : kOOB);
    }
  }
}

// One row of an item: dot of the lane's chunks (prefetched rounds, then streamed ones).
template <int R, int WQ8, int SM>
DEV void row_dots(const uint4 (&w)[R], const uint16_t (&sc)[R], const void* W, const uint16_t* Ws, int N, int gr,
                  int K, int slot, int S, const float* x, float (&acc)[SM]) {
  const int nch = WQ8 ? (K >> 4) : (K >> 3);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c = slot + 32 * r;
    if (c < nch) {
#pragma unroll
      for (int s = 0; s < SM; ++s)
        if (s < S) {
          if (WQ8)
            acc[s] = fmaf(h2f(sc[r]), dot16_q8(w[r], x + s * K + c * 16), acc[s]);
          else
            acc[s] += dot8_f16(w[r], x + s * K + c * 8);
        }
    }
  }
  stream_rest<R, WQ8, SM>(W, Ws, N, K, gr, slot, S, x, acc);
}

// out[(i * SM + s) * 8 + r] = sum_k W[(it0 + i * istr) * 8 + r][k] * x[s * K + k]
// red: LDS [NB][32][SM], out: LDS [NB][SM][8].
template <int R, int NB, int WQ8, int SM>
DEV void gemvb_compute(const WBatch<R, NB>& wb, const void* W, const uint16_t* Ws, int N, int K, int it0, int istr,
                       int nit, int S, const float* x, float* red, float* out) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, row = lane >> 3, sub = lane & 7;
  const int slot = (w << 3) | sub;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    if (i < nit) {
      float acc[SM];
#pragma unroll
      for (int s = 0; s < SM; ++s) acc[s] = 0.f;
      const int gr = (it0 + i * istr) * 8 + row;
      if (gr < N) row_dots<R, WQ8, SM>(wb.w[i], wb.s[i], W, Ws, N, gr, K, slot, S, x, acc);
#pragma unroll
      for (int s = 0; s < SM; ++s) acc[s] = sum8(acc[s]);
      if (sub == 0) {
#pragma unroll
        for (int s = 0; s < SM; ++s)
          if (s < S) red[(i * 32 + (w << 3) + row) * SM + s] = acc[s];
      }
    }
  }
  lds_barrier();
  for (int idx = tid; idx < nit * S * 8; idx += kThreads) {
    const int i = idx / (S * 8), rem = idx - i * S * 8, s = rem >> 3, rr = rem & 7;
    const float* rp = red + i * 32 * SM;
    out[(i * SM + s) * 8 + rr] = (rp[rr * SM + s] + rp[(8 + rr) * SM + s]) + (rp[(16 + rr) * SM + s] + rp[(24 + rr) * SM + s]);
  }
  lds_barrier();
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
  lds_barrier();
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

// AUX 16 (sc1) makes the loads coherent at device scope: used for the self-KV cache, whose rows
// are appended by other workgroups earlier in the same launch.
template <int KPT, int AUX, class Off>
DEV void attn_prefetch(const uint16_t* kb, const uint16_t* vb, size_t kv_bytes, Off off, int n, KVRegs<KPT>& r) {
  const int sub = threadIdx.x & 7, kg = threadIdx.x >> 3;
  const auto rk = brsrc(kb, kv_bytes), rv = brsrc(vb, kv_bytes);
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int j = kg + 32 * i;
    const uint32_t o = j < n ? (uint32_t)((off(j) + (size_t)sub * 8) * 2) : kOOB;
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rk, (int)o, 0, AUX);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)o, 0, AUX);
    r.k[i] = make_uint4(a.x, a.y, a.z, a.w);
    r.v[i] = make_uint4(b.x, b.y, b.z, b.w);
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
    for (int s = 0; s < SM; ++s) part[s] = sum8(part[s]);
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
  lds_barrier();
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
  lds_barrier();
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
    for (int e = 0; e < 8; ++e) a[s][e] += dpp<0x128>(a[s][e]);  // + lane ^ 8
  // lanes 0..7 of each 16-lane row now hold the row's partial: 4 rows x 4 waves -> LDS
  if ((lane & 15) < 8) {
    const int rw = w * 4 + (lane >> 4);
#pragma unroll
    for (int s = 0; s < SM; ++s)
      if (s < ns)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[(rw * SM + s) * kHeadDim + sub * 8 + e] = a[s][e];
  }
  lds_barrier();
  for (int i = tid; i < ns * kHeadDim; i += kThreads) {
    const int s = i >> 6, e = i & 63;
    float o = 0.f;
#pragma unroll
    for (int rw = 0; rw < 16; ++rw) o += red[(rw * SM + s) * kHeadDim + e];
    if (kx != nullptr) o = fmaf(sc[s * scs + n], vx[e], o);
    acc_out[i] = o;
  }
  lds_barrier();
}

// Merge attention partials: part[(c * nrow + row) * kPartWords + w] for c < nc -> o[row*64 + e].
// With nc <= kMergeChunks, PAD = true reads every chunk slot below kMergeChunks, in range or not (the
// caller's partial area holds kMergeChunks chunks), so the reads need no per-chunk address select;
// PAD = false re-reads the last chunk for the slots past it.  Slots at or past nc are left out of
// the sums either way.
template <bool PAD>
DEV void attn_merge(const float* part, int nc, int nrow, float* o) {
  constexpr int CM = kMergeChunks;  // chunks merged from registers: every partial read before the sums
  if (nc <= CM) {
    const int cs = nrow * kPartWords;
    for (int i = threadIdx.x; i < nrow * kHeadDim; i += kThreads) {
      const int row = i >> 6, e = i & 63;
      const float* pp = part + row * kPartWords;
      float mv[CM], lv[CM], av[CM];
#pragma unroll
      for (int c = 0; c < CM; ++c) {
        const float* pc = PAD ? pp + c * cs : part + (min(c, nc - 1) * nrow + row) * kPartWords;
        mv[c] = pc[0];
        lv[c] = pc[1];
        av[c] = pc[2 + e];
      }
      float M = -INFINITY;
#pragma unroll
      for (int c = 0; c < CM; ++c) M = fmaxf(M, PAD && c >= nc ? -INFINITY : mv[c]);  // re-reads leave M alone
      float Lsum = 0.f, acc = 0.f;
#pragma unroll
      for (int c = 0; c < CM; ++c) {
        if (c < nc) {  // same chunks, same order as below
          const float f = __expf(mv[c] - M);
          Lsum = fmaf(lv[c], f, Lsum);
          acc = fmaf(av[c], f, acc);
        }
      }
      o[i] = acc / Lsum;
    }
    lds_barrier();
    return;
  }
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
  lds_barrier();
}

constexpr int kVecRegs = 10;  // elements of a d-vector per thread (d <= 2560)
constexpr int kNB = 8;        // items per GEMV batch (64 rows)


// A d-vector parameter (LayerNorm gamma/beta, positional row) held in registers: thread t keeps
// elements t + kThreads * i.  Loaded before a phase polls its inputs, so no parameter load sits
// between the inputs' arrival and the phase's results.
struct VecRegs {
  float v[kVecRegs];
};
DEV void vec_prefetch(const float* src, int d, VecRegs& r) {
  const auto rs = brsrc(src, (size_t)d * 4);
#pragma unroll
  for (int i = 0; i < kVecRegs; ++i) {
    const int j = threadIdx.x + kThreads * i;
    r.v[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, j < d ? j * 4 : (int)kOOB, 0, 0));
  }
}

// ------------------------------------------------------------------------------------------------
// Single-row (S = 1) paths, written as straight-line code: a lane's activation chunks are loaded
// from LDS into registers once and reused by every 8-row group of the batch, out-of-range chunks
// are zeroed by selects instead of branches (their weights are zero as well: buffer loads past the
// end of a matrix return 0), and the only barrier is the one before the cross-wave reduction.

// Activation chunks of a lane in the GEMV lane layout: round r holds x[(slot + 32 r) * CE + e],
// e < CE, with CE = 8 (f16 weights: 8 halves per 16-byte chunk) or 16 (q8_0: 16 int8).
template <int R, int WQ8>
struct XR {
  float v[R][WQ8 ? 16 : 8];
};

// Chunks at or past K are zeroed.  With q8_0 weights every round reads x + (slot + 32 r) * CE, in
// range or not, so that the R addresses are one base plus constant offsets: the q8_0 kernel is at
// its register limit and otherwise spills the per-round addresses.  Those reads span 32 * R * CE
// floats from x, which the step kernel's LDS sizing keeps inside the allocation (step_lds_bytes).
// The f16 kernels read chunk 0 for the rounds past K.
template <int R, int WQ8>
DEV void xr_load(const float* x, int K, XR<R, WQ8>& X) {
  constexpr int CE = WQ8 ? 16 : 8;
  const int slot = ((threadIdx.x >> 6) << 3) | (threadIdx.x & 7);
  const float* base = x + slot * CE;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool ok = (slot + 32 * r + 1) * CE <= K;
    const float4* src = reinterpret_cast<const float4*>(WQ8 ? base + 32 * CE * r : x + (ok ? (slot + 32 * r) * CE : 0));
#pragma unroll
    for (int q = 0; q < CE / 4; ++q) {
      const float4 t = src[q];
      X.v[r][4 * q + 0] = ok ? t.x : 0.f;
      X.v[r][4 * q + 1] = ok ? t.y : 0.f;
      X.v[r][4 * q + 2] = ok ? t.z : 0.f;
      X.v[r][4 * q + 3] = ok ? t.w : 0.f;
    }
  }
}

DEV float dot8_fx(const uint4& w, const float* x) {
  const float2 w0 = h2x2(w.x), w1 = h2x2(w.y), w2 = h2x2(w.z), w3 = h2x2(w.w);
  float s = w0.x * x[0];
  s = fmaf(w0.y, x[1], s);
  s = fmaf(w1.x, x[2], s);
  s = fmaf(w1.y, x[3], s);
  s = fmaf(w2.x, x[4], s);
  s = fmaf(w2.y, x[5], s);
  s = fmaf(w3.x, x[6], s);
  s = fmaf(w3.y, x[7], s);
  return s;
}

DEV float dot16_qx(const uint4& w, const float* x) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    s = fmaf((float)(int8_t)(u[k] & 0xff), x[4 * k + 0], s);
    s = fmaf((float)(int8_t)((u[k] >> 8) & 0xff), x[4 * k + 1], s);
    s = fmaf((float)(int8_t)((u[k] >> 16) & 0xff), x[4 * k + 2], s);
    s = fmaf((float)(int8_t)(u[k] >> 24), x[4 * k + 3], s);
  }
  return s;
}

// Partial dots of the NB items of a prefetched batch against the lane's activation chunks, reduced
// over the 8 lanes of a row and written as red[i * 32 + wave * 8 + row] (LDS).  Chunks beyond the R
// prefetched rounds (K > 32 R CE) are streamed here against x (LDS).  The caller puts an
// lds_barrier() between this and gemv_out().
template <int R, int NB, int WQ8>
DEV void gemv_rx(const WBatch<R, NB>& wb, const XR<R, WQ8>& X, const void* W, const uint16_t* Ws, int N, int K, int it0,
                 int istr, const float* x, float* red) {
  constexpr int CE = WQ8 ? 16 : 8;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, row = lane >> 3;
  const int slot = (w << 3) | (lane & 7);
  float acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    float a = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (!WQ8)
        a += dot8_fx(wb.w[i][r], X.v[r]);
      else
        a = fmaf(h2f(wb.s[i][r]), dot16_qx(wb.w[i][r], X.v[r]), a);
    }
    acc[i] = a;
  }
  if (K > 32 * R * CE) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      float t[1] = {0.f};
      stream_rest<R, WQ8, 1>(W, Ws, N, K, (it0 + i * istr) * 8 + row, slot, 1, x, t);
      acc[i] += t[0];
    }
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) acc[i] = sum8(acc[i]);
  if ((lane & 7) == 0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) red[i * 32 + (w << 3) + row] = acc[i];
  }
}

// Output rr of item i of the last gemv_rx (after the barrier).
DEV float gemv_out(const float* red, int i, int rr) {
  const float* p = red + i * 32 + rr;
  return (p[0] + p[8]) + (p[16] + p[24]);
}
// All 8 outputs of item i (o[rr] = gemv_out(red, i, rr), same sums): the item's 32 partials are
// contiguous and read as eight 16-byte words at once.
DEV void gemv_out8(const float* red, int i, float (&o)[8]) {
  float4 q[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) q[k] = reinterpret_cast<const float4*>(red + i * 32)[k];
  const float* p = reinterpret_cast<const float*>(q);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (p[e] + p[8 + e]) + (p[16 + e] + p[24 + e]);
}

// gemv_rx for items whose weight chunks sit in LDS in register-image order
// (wl[(i * R + r) * kThreads + thread], scales alike).  Items i >= nit (nit >= 1) recompute item
// nit - 1 and their sums are not used: without a branch per item every LDS read of the batch is
// issued at once and the items' FMA chains interleave.
template <int R, int NB, int WQ8>
DEV void gemv_lds(const uint4* wl, const uint16_t* sl, int nit, const XR<R, WQ8>& X, float* red) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, row = lane >> 3;
  uint4 wv[NB][R];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r) wv[i][r] = wl[(min(i, nit - 1) * R + r) * kThreads + tid];
  float acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int ic = min(i, nit - 1);
    float a = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (!WQ8)
        a += dot8_fx(wv[i][r], X.v[r]);
      else
        a = fmaf(h2f(sl[(ic * R + r) * kThreads + tid]), dot16_qx(wv[i][r], X.v[r]), a);
    }
    acc[i] = sum8(a);
  }
  if ((lane & 7) == 0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) red[i * 32 + (w << 3) + row] = acc[i];
  }
}

// Load this workgroup's first nres vocabulary items (items g, g + G, ...) into LDS in the register
// image of the logits GEMV (DR 16-byte chunks per lane and row), eight items per batch of loads.
template <int WQ8, int DR>
DEV void load_resident_vocab(const StepParams& p, uint4* ew, uint16_t* es, int nres) {
  const int G = gridDim.x, g = blockIdx.x, tid = threadIdx.x;
  for (int b = 0; b < nres; b += kNB) {
    WBatch<DR, kNB> wb;
    gemvb_prefetch<DR, kNB, WQ8>(p.emb, p.emb_s, p.V, p.d, g + b * G, G, min(kNB, nres - b), wb);
#pragma unroll
    for (int i = 0; i < kNB; ++i)
      if (b + i < nres) {
#pragma unroll
        for (int r = 0; r < DR; ++r) {
          ew[((b + i) * DR + r) * kThreads + tid] = wb.w[i][r];
          if (WQ8) es[((b + i) * DR + r) * kThreads + tid] = wb.s[i][r];
        }
      }
  }
  lds_barrier();
}

// Multi-row GEMV: rows s < S of x (LDS, row stride K) against the NB items of a prefetched batch.
// Weight chunks are read from registers once per round and applied to every row; a row's
// activation chunk is loaded from LDS once per round and applied to every item.  Result layout
// red[((i * 32) + wave * 8 + row) * SM + s], read back with gemv_outm() after a barrier.
template <int SM, int R, int NB, int WQ8>
DEV void gemv_rxm(const WBatch<R, NB>& wb, const float* x, int S, int K, const void* W, const uint16_t* Ws, int N,
                  int it0, int istr, float* red) {
  constexpr int CE = WQ8 ? 16 : 8;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, row = lane >> 3;
  const int slot = (w << 3) | (lane & 7);
  float acc[NB][SM];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int s = 0; s < SM; ++s) acc[i][s] = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c = slot + 32 * r;
    const bool ok = (c + 1) * CE <= K;
#pragma unroll
    for (int s = 0; s < SM; ++s) {
      if (s < S) {
        float xv[CE];
        const float4* src = reinterpret_cast<const float4*>(x + (size_t)s * K + (ok ? c * CE : 0));
#pragma unroll
        for (int q = 0; q < CE / 4; ++q) {
          const float4 t = src[q];
          xv[4 * q + 0] = ok ? t.x : 0.f;
          xv[4 * q + 1] = ok ? t.y : 0.f;
          xv[4 * q + 2] = ok ? t.z : 0.f;
          xv[4 * q + 3] = ok ? t.w : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
          if (!WQ8)
            acc[i][s] += dot8_fx(wb.w[i][r], xv);
          else
            acc[i][s] = fmaf(h2f(wb.s[i][r]), dot16_qx(wb.w[i][r], xv), acc[i][s]);
        }
      }
    }
  }
  if (K > 32 * R * CE) {
#pragma unroll
    for (int i = 0; i < NB; ++i) stream_rest<R, WQ8, SM>(W, Ws, N, K, (it0 + i * istr) * 8 + row, slot, S, x, acc[i]);
  }
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int s = 0; s < SM; ++s) acc[i][s] = sum8(acc[i][s]);
  if ((lane & 7) == 0) {
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int s = 0; s < SM; ++s)
        if (s < S) red[((i * 32) + (w << 3) + row) * SM + s] = acc[i][s];
  }
}

// Output rr of item i, row s of the last gemv_rxm (after the barrier).
template <int SM>
DEV float gemv_outm(const float* red, int i, int rr, int s) {
  const float* q = red + (i * 32 + rr) * SM + s;
  return (q[0] + q[8 * SM]) + (q[16 * SM] + q[24 * SM]);
}

// Per-wave LayerNorm statistics of x[0, d) (LDS), two passes, eps 1e-5; no barrier.  Lane l reads
// x[4 l + 256 k, +4) for k < NI (d <= 256 * NI); reads past d are clamped to 0 and masked by a
// select, so the loads issue back to back.
template <int NI>
DEV void ln_stats(const float* x, int d, float& mean, float& inv) {
  const int lane = threadIdx.x & 63;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const int i = lane * 4 + 256 * k;
    const float4 t = *reinterpret_cast<const float4*>(x + (i < d ? i : 0));
    s += i < d ? (t.x + t.y) + (t.z + t.w) : 0.f;
  }
  mean = wave_sum(s) / (float)d;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const int i = lane * 4 + 256 * k;
    const float4 t = *reinterpret_cast<const float4*>(x + (i < d ? i : 0));
    const float a = t.x - mean, b = t.y - mean, c = t.z - mean, e = t.w - mean;
    const float q = fmaf(a, a, fmaf(b, b, fmaf(c, c, e * e)));
    v += i < d ? q : 0.f;
  }
  inv = 1.0f / sqrtf(wave_sum(v) / (float)d + 1e-5f);
}

// Iterations of ln_stats for a kernel instance: two for the d <= 512 f16 instance, enough for the
// widest supported row otherwise.
template <int WQ8, int DR>
constexpr int ln_iters() { return (WQ8 || DR > 2) ? kVecRegs : 2; }

// LayerNorm of one row x[0, d) into y (LDS) with gamma/beta in registers (VecRegs layout); every
// wave computes the statistics itself, so the only barrier is the one that publishes y.
template <int NI>
DEV void ln_row(const float* x, float* y, int d, const VecRegs& g, const VecRegs& b) {
  float mean, inv;
  ln_stats<NI>(x, d, mean, inv);
  // every element read first (clamped index, no branch per element), so the LDS reads overlap;
  // NI * 256 >= d, so NI elements per thread cover the row
  float xv[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) xv[i] = x[min((int)threadIdx.x + kThreads * i, d - 1)];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int j = threadIdx.x + kThreads * i;
    if (j < d) y[j] = (xv[i] - mean) * inv * g.v[i] + b.v[i];
  }
  lds_barrier();
}

// Attention of one query row over n keys held in registers (8 lanes per key; key j = kg + 32 i,
// kg = thread / 8), with the lane's query chunk Q = q[sub * 8, +8) in registers.  Each wave forms
// its own softmax partial over its keys; the four partials are merged through LDS (wpart, 4 x 66
// floats) after one barrier.  Threads 0..63 return acc[thread] of the merged partial (m, l, acc)
// and m, l.
template <int KPT>
DEV void attn_rx(const KVRegs<KPT>& r, int n, const float (&Q)[8], float scale, float* wpart, float& m_out,
                 float& l_out, float& acc_out) {
  const int tid = threadIdx.x, kg = tid >> 3, sub = tid & 7, w = tid >> 6, lane = tid & 63;
  float sc[KPT];
  float mloc = -INFINITY;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const float t = sum8(dot8_fx(r.k[i], Q)) * scale;
    sc[i] = (kg + 32 * i) < n ? t : -INFINITY;
    mloc = fmaxf(mloc, sc[i]);
  }
  const float mw = wave_max(mloc);
  float ls = 0.f, a[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = 0.f;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const float pr = sc[i] > -INFINITY ? __expf(sc[i] - mw) : 0.f;
    ls += pr;
    const float2 v0 = h2x2(r.v[i].x), v1 = h2x2(r.v[i].y), v2 = h2x2(r.v[i].z), v3 = h2x2(r.v[i].w);
    a[0] = fmaf(pr, v0.x, a[0]);
    a[1] = fmaf(pr, v0.y, a[1]);
    a[2] = fmaf(pr, v1.x, a[2]);
    a[3] = fmaf(pr, v1.y, a[3]);
    a[4] = fmaf(pr, v2.x, a[4]);
    a[5] = fmaf(pr, v2.y, a[5]);
    a[6] = fmaf(pr, v3.x, a[6]);
    a[7] = fmaf(pr, v3.y, a[7]);
  }
  const float lw = wave_sum(sub == 0 ? ls : 0.f);
  // sum over the 8 key groups of the wave (lanes sub + 8 g)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] += dpp<0x128>(a[e]);  // lane ^ 8 (row_ror:8 within 16 lanes)
    a[e] += __shfl_xor(a[e], 16);
    a[e] += __shfl_xor(a[e], 32);
  }
  if (lane < 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) wpart[w * kPartWords + 2 + sub * 8 + e] = a[e];
    if (lane == 0) {
      wpart[w * kPartWords] = mw;
      wpart[w * kPartWords + 1] = lw;
    }
  }
  lds_barrier();
  if (tid < 64) {
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < 4; ++q) M = fmaxf(M, wpart[q * kPartWords]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float mq = wpart[q * kPartWords];
      const float f = mq > -INFINITY ? __expf(mq - M) : 0.f;
      L = fmaf(wpart[q * kPartWords + 1], f, L);
      A = fmaf(wpart[q * kPartWords + 2 + tid], f, A);
    }
    m_out = M;
    l_out = L;
    acc_out = A;
  }
}

// ------------------------------------------------------------------------------------------------
// Selection.  A workgroup partial over its rows (lg masked, rw raw logits, idx global ids) is
// kSelWords floats: [max, argmax, sumexp(masked - max), raw max, raw sumexp, probe, topk values[8],
// topk ids[8]].  Ties go to the lower vocabulary id everywhere.

// Top-k helpers: every lane keeps its own best W4H_TOPK_MAX (value descending, lower id on ties) in
// registers; the wave then pops the best lane head k times.  Entries at -inf never enter.
struct TopList {
  float v[W4H_TOPK_MAX];
  int i[W4H_TOPK_MAX];
};

DEV void top_init(TopList& t) {
#pragma unroll
  for (int k = 0; k < W4H_TOPK_MAX; ++k) {
    t.v[k] = -INFINITY;
    t.i[k] = 0x7fffffff;
  }
}

DEV bool top_better(float v, int id, float w, int jd) { return v > w || (v == w && id < jd); }

// Insert (v, id) into the lane's sorted list (no-op unless it beats the last entry).
DEV void top_insert(TopList& t, float v, int id) {
  if (!(v > -INFINITY) || !top_better(v, id, t.v[W4H_TOPK_MAX - 1], t.i[W4H_TOPK_MAX - 1])) return;
#pragma unroll
  for (int k = W4H_TOPK_MAX - 1; k > 0; --k) {
    const bool shift = top_better(v, id, t.v[k - 1], t.i[k - 1]);
    const bool here = !shift && top_better(v, id, t.v[k], t.i[k]);
    if (shift) {
      t.v[k] = t.v[k - 1];
      t.i[k] = t.i[k - 1];
    } else if (here) {
      t.v[k] = v;
      t.i[k] = id;
    }
  }
  if (top_better(v, id, t.v[0], t.i[0])) {
    t.v[0] = v;
    t.i[0] = id;
  }
}

// k rounds: the wave's best lane head is taken and that lane advances.  tv/ti (every lane) get the
// wave's top k in order.
DEV void top_pop(TopList& t, int topk, float* tv, int* ti) {
  int head = 0;
  for (int k = 0; k < W4H_TOPK_MAX; ++k) {
    tv[k] = -INFINITY;
    ti[k] = 0x7fffffff;
  }
  for (int k = 0; k < topk; ++k) {
    float hv = -INFINITY;
    int hi = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < W4H_TOPK_MAX; ++q)
      if (q == head) {
        hv = t.v[q];
        hi = t.i[q];
      }
    float bv = hv;
    int bi = hi;
    wave_argmax(bv, bi);
    tv[k] = bv;
    ti[k] = bv > -INFINITY ? bi : 0x7fffffff;
    if (bv > -INFINITY && hi == bi && hv == bv) ++head;
  }
}

DEV void sel_partial(const float* lg, const float* rw, const int* idx, int n, int probe, int topk, float* rec) {
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY, rv = -INFINITY, pv = -INFINITY;
  int bi = 0x7fffffff;
  TopList tl;
  top_init(tl);
  for (int j = lane; j < n; j += 64) {
    const float v = lg[j];
    const int id = idx[j];
    if (v > bv || (v == bv && id < bi)) {
      bv = v;
      bi = id;
    }
    rv = fmaxf(rv, rw[j]);
    if (id == probe) pv = rw[j];
    if (topk > 0) top_insert(tl, v, id);
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
  top_pop(tl, topk, tv, ti);
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
// The partials cover disjoint vocabulary ranges, so their top-k lists hold distinct ids.
DEV void sel_merge(const float* recs, int n, int stride, int topk, float* out_rec) {
  const int lane = threadIdx.x & 63;
  float bv = -INFINITY, rv = -INFINITY, pv = -INFINITY;
  int bi = 0x7fffffff;
  TopList tl;
  top_init(tl);
  for (int g = lane; g < n; g += 64) {
    const float* r = recs + (size_t)g * stride;
    const int id = __float_as_int(r[1]);
    if (r[0] > bv || (r[0] == bv && id < bi)) {
      bv = r[0];
      bi = id;
    }
    rv = fmaxf(rv, r[3]);
    pv = fmaxf(pv, r[5]);
    for (int q = 0; q < topk; ++q) top_insert(tl, r[6 + q], __float_as_int(r[6 + W4H_TOPK_MAX + q]));
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
  float* xin;   // [S][4d]        polled activations
  float* xn;    // [S][d]         LayerNorm output / merged attention output
  float* scr;   // [8]
  int* toks;    // [kMaxRows]     tokens of the current step
  float* res;   // [kResItems][S][8] residual rows of this workgroup's d-row items
  float* big;   // phase scratch
  uint4* ew;    // [nres][DR][kThreads] resident vocabulary rows (S = 1), GEMV register image
  uint16_t* es; // [nres][DR][kThreads] their q8_0 scales
  int* hist;        // decode rules: [hist_cap] generated tokens
  uint32_t* rbits;  // decode rules: [(rows_per_wg + 31) / 32] rows of this workgroup masked this step
  int* rrng;        // decode rules: range count, then [lo, hi) token ranges masked this step
};

// LayerNorm of S rows of d (LDS in, LDS out) with gamma/beta in registers; two passes, eps 1e-5.
DEV void wg_layernorm_r(const float* x, float* y, int S, int d, const VecRegs& g, const VecRegs& b, float* scratch) {
  for (int s = 0; s < S; ++s) {
    const float* xs = x + s * d;
    float xv[kVecRegs];
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < kVecRegs; ++i) {
      const int j = threadIdx.x + kThreads * i;
      xv[i] = j < d ? xs[j] : 0.f;
      a += xv[i];
    }
    const float mean = wg_sum(a, scratch) / (float)d;
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kVecRegs; ++i) {
      const int j = threadIdx.x + kThreads * i;
      if (j < d) {
        const float t = xv[i] - mean;
        v = fmaf(t, t, v);
      }
    }
    const float var = wg_sum(v, scratch + 4) / (float)d;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < kVecRegs; ++i) {
      const int j = threadIdx.x + kThreads * i;
      if (j < d) y[s * d + j] = (xv[i] - mean) * inv * g.v[i] + b.v[i];
    }
  }
  lds_barrier();
}

// Workgroup group of a phase.  Consecutive phases run on different groups, so a workgroup has idle
// phases in which the weights, key/value rows and parameters of its next phase arrive, while fewer
// workgroups poll any one exchange buffer.  The out-projection, cross-out and MLP2 phases (odd
// phase numbers) always share one group, which keeps the residual rows in its workgroups' LDS.
//   ngroups 1: every phase on the whole grid;
//   ngroups 2: phase q on half q % 2;
//   ngroups 4: quarters: self-attention on quarter 0, the residual phases on quarter 1,
//              cross-attention on quarter 2, MLP1 on quarter 3.
struct Grp {
  int base, size;
};
DEV Grp phase_group(int q, int G, int ng) {
  const int sz = G / ng;
  if (ng == 4) {
    const int k = q % 6;
    const int grp = (k & 1) ? 1 : (k == 0 ? 0 : (k == 2 ? 2 : 3));
    return Grp{grp * sz, sz};
  }
  return Grp{(q % ng) * sz, sz};
}
// First item of this workgroup in the group (items i, i + size, ...), or a value past any item count.
DEV int grp_first(Grp gr) {
  const int g = blockIdx.x;
  return (g >= gr.base && g < gr.base + gr.size) ? g - gr.base : 0x7fffffff;
}

// This workgroup's replica of an exchange buffer.
DEV const u64* rep(const StepParams& p, const u64* b) { return b + (size_t)(blockIdx.x % kRep) * p.rep_stride; }

struct StepCtx {
  uint32_t tag;
  int st, kv, pe, ph, nph;
};

// Diagnostics: sub-phase timestamps (0 start, 1 inputs arrived, 2 computed, 3 end).
#define STAMP(sub)                                                                                            \
  do {                                                                                                        \
    if (p.trace != nullptr && threadIdx.x == 0)                                                               \
      p.trace[(((size_t)c.st * c.nph + c.ph) * 4 + (sub)) * gridDim.x + blockIdx.x] = wall_clock64();         \
  } while (0)

// x of layer 0 = token embedding + positional embedding (exact dequant, one rounding); the
// positional row was prefetched into registers.
template <int WQ8>
DEV void embed_r(const StepParams& p, const Lds& m, const VecRegs& pe, float* dst) {
  const int d = p.d;
  for (int s = 0; s < p.S; ++s) {
    const int tk = m.toks[s];
#pragma unroll
    for (int i = 0; i < kVecRegs; ++i) {
      const int j = threadIdx.x + kThreads * i;
      if (j < d) {
        float e;
        if (!WQ8) {
          e = h2f(static_cast<const uint16_t*>(p.emb)[(size_t)tk * d + j]);
        } else {
          e = (float)static_cast<const int8_t*>(p.emb)[(size_t)tk * d + j] * h2f(p.emb_s[(size_t)tk * (d >> 5) + (j >> 5)]);
        }
        dst[s * d + j] = e + pe.v[i];
      }
    }
  }
  lds_barrier();
}

// GELU of the f16-rounded input, as the reference's 65 536-entry table defines it
// (main/tensor/Tensor.java:493-501, 524-538): x = f32(f16(v)),
//   y = fl(fl(0.5 x) * fl(1 + (float)tanh((double) fl(s * fl(x + fl(fl(fl(0.044715 x) x) x))))))
// with s = (float)sqrt(2/pi), every float operation rounded on its own (contraction off) and tanh
// taken in double.  Computed instead of looked up, so no table load waits on the GEMV result.
DEV float gelu_f16(float v) {
#pragma clang fp contract(off)
  const float x = h2f(f2h(v));
  const float s = (float)sqrt(2.0 / 3.14159265358979323846);
  const float c = ((0.044715f * x) * x) * x;
  const float inner = s * (x + c);
  // tanh in double as (e^{2z} - 1) / (e^{2z} + 1) from expm1 (a few double ulps), then rounded
  // to float: equal to the correctly rounded double tanh rounded to float on every f16 input.
  const double z = (double)inner;
  double t;
  if (fabs(z) > 20.0) {
    t = z > 0.0 ? 1.0 : -1.0;
  } else {
    const double e = expm1(2.0 * z);
    t = e / (e + 2.0);
  }
  return (0.5f * x) * (1.0f + (float)t);
}

// ------------------------------------------------------------------------------------------------
// Phases.  SM is the row capacity of the kernel instance (1: greedy decode of one stream; 8: beams or
// streams, S <= 8 rows at run time).  Every phase is built on the straight-line blocks above:
// weights (and key/value chunks) are prefetched into registers before the poll, a lane's
// activation chunks are read from LDS once per round and applied to every weight row it holds, and
// the only barriers are the cross-wave reductions.

// Bias chunk of a lane for a 64-row head block: o[e] = b[base + (thread % 8) * 8 + e].
DEV void bias8(const float* b, int base, float (&o)[8]) {
  const float4* q = reinterpret_cast<const float4*>(b + base + (threadIdx.x & 7) * 8);
  const float4 a = q[0], c = q[1];
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = c.x; o[5] = c.y; o[6] = c.z; o[7] = c.w;
}

// Self-attention with the q/k/v projection folded in.  Per (row s, head h) the items are:
//   j <  nold : cached-key chunk j (keys [j*C, min((j+1)*C, kv)));  projects q_h, attends, writes a
//               partial (m, l, acc[64]) to chunk slot j;
//   j == nold : projects q_h and k_h, appends k_h to the cache, writes the current key's score as
//               (m = q.k * scale, l = 1) into chunk slot nold;
//   j == nold+1: projects v_h, appends it to the cache, writes it as acc[64] of chunk slot nold.
// All items depend only on the layer input, so the projection costs no extra hand-over.  The
// appended rows are read only by later steps; the logits phase drains every workgroup's stores
// before it publishes, which orders them before any later step reads the cache.
template <int SM, int WQ8, int DR>
DEV bool phase_self(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = DR;
  const int tid = threadIdx.x, S = p.S, d = p.d, H = p.H, d3 = 3 * d, sub = tid & 7;
  const LayerDev& lw = p.layers[l];
  const int nold = (c.kv + kSelfChunk - 1) / kSelfChunk;
  const int per = nold + 2;
  const int nitems = S * H * per;
  int it = grp_first(gr);
  if (it >= nitems) return true;
  STAMP(0);
  VecRegs g1, b1, pe;
  vec_prefetch(lw.ln1_g, d, g1);
  vec_prefetch(lw.ln1_b, d, b1);
  if (l == 0) vec_prefetch(p.pos + (size_t)c.pe * d, d, pe);
  const size_t kv_bytes = (size_t)p.L * S * H * p.max_ctx * kHeadDim * 2;
  const int mc = p.max_ctx;
  bool have_x = false;
  auto ensure_x = [&]() -> bool {
    if (have_x) return true;
    if (l == 0) {
      embed_r<WQ8>(p, m, pe, m.xin);
    } else if (!ll_poll1<8>(rep(p, p.x3 + (size_t)(l - 1) * S * d), S * d, m.xin, c.tag, p.err)) {
      return false;
    }
    STAMP(1);
    for (int s = 0; s < S; ++s) ln_row<ln_iters<WQ8, DR>()>(m.xin + s * d, m.xn + s * d, d, g1, b1);
    have_x = true;
    return true;
  };
  float* red = m.big;         // [8][32]
  float* red2 = red + 256;    // [8][32]
  float* wpart = red2 + 256;  // [4][kPartWords]
  for (; it < nitems; it += gr.size) {
    const int j = it % per, sh = it / per, h = sh % H, s = sh / H;
    const int kind = j < nold ? 0 : (j == nold ? 1 : 2);
    const int rowA = (kind == 2 ? 2 * d : 0) + h * kHeadDim;  // q rows, or v rows for the value item
    const int rowB = d + h * kHeadDim;                         // k rows
    u64* dst = p.sp + ((((size_t)l * p.ncs_max + (kind == 0 ? j : nold)) * S + s) * H + h) * kPartWords;
    const float* xs = m.xn + s * d;
    if (kind == 0) {
      // cached keys: q projection + attention over this chunk
      WBatch<R, kNB> wa;
      gemvb_prefetch<R, kNB, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, rowA >> 3, 1, kNB, wa);
      float bq[8];
      bias8(lw.b_qkv, rowA, bq);
      const int k0 = j * kSelfChunk;
      const int n = min(kSelfChunk, c.kv - k0);
      const int32_t* slots = p.slots ? p.slots + (size_t)s * mc : nullptr;
      const size_t lb = (size_t)l * S;
      auto off = [=](int jj) -> size_t {
        const int pos = k0 + jj;
        const int slot = slots ? slots[pos] : s;
        return (((lb + slot) * H + h) * mc + pos) * kHeadDim;
      };
      KVRegs<KPT_SELF> kr;
      attn_prefetch<KPT_SELF, 16>(p.kv_k, p.kv_v, kv_bytes, off, n, kr);
      if (!ensure_x()) return false;
      gemv_rxm<1, R, kNB, WQ8>(wa, xs, 1, d, lw.w_qkv, lw.s_qkv, d3, rowA >> 3, 1, red);
      lds_barrier();
      float Q[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) Q[e] = gemv_outm<1>(red, sub, e, 0) + bq[e];
      float M, Ls, A;
      attn_rx<KPT_SELF>(kr, n, Q, 0.125f, wpart, M, Ls, A);
      STAMP(2);
      if (tid < 64) {
        ll_st(dst + 2 + tid, A, c.tag, p.rep_stride);
        if (tid == 0) {
          ll_st(dst + 0, M, c.tag, p.rep_stride);
          ll_st(dst + 1, Ls, c.tag, p.rep_stride);
        }
      }
    } else {
      // the current token: (q, k) score and k append, or v append
      WBatch<R, kNB> wa, wb;
      gemvb_prefetch<R, kNB, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, rowA >> 3, 1, kNB, wa);
      if (kind == 1) gemvb_prefetch<R, kNB, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, rowB >> 3, 1, kNB, wb);
      const float ba = tid < kHeadDim ? lw.b_qkv[rowA + tid] : 0.f;
      const float bb = (kind == 1 && tid < kHeadDim) ? lw.b_qkv[rowB + tid] : 0.f;
      if (!ensure_x()) return false;
      gemv_rxm<1, R, kNB, WQ8>(wa, xs, 1, d, lw.w_qkv, lw.s_qkv, d3, rowA >> 3, 1, red);
      if (kind == 1) gemv_rxm<1, R, kNB, WQ8>(wb, xs, 1, d, lw.w_qkv, lw.s_qkv, d3, rowB >> 3, 1, red2);
      lds_barrier();
      STAMP(2);
      const size_t kvrow = ((((size_t)l * S + s) * H + h) * mc + c.kv) * kHeadDim;
      if (tid < 64) {
        const float va = gemv_outm<1>(red, tid >> 3, tid & 7, 0) + ba;
        if (kind == 1) {
          const float vb = gemv_outm<1>(red2, tid >> 3, tid & 7, 0) + bb;
          const float t = wave_sum(va * vb);
          if (tid == 0) {
            ll_st(dst + 0, t * 0.125f, c.tag, p.rep_stride);
            ll_st(dst + 1, 1.0f, c.tag, p.rep_stride);
          }
          kv_store(p.kv_k, kv_bytes, kvrow + tid, f2h(vb));
        } else {
          ll_st(dst + 2 + tid, va, c.tag, p.rep_stride);
          kv_store(p.kv_v, kv_bytes, kvrow + tid, f2h(va));
        }
      }
    }
    lds_barrier();
  }
  return true;
}

// Residual rows.  The out-projection, cross-out and MLP2 phases all produce d rows in 8-row
// items, run on the same workgroup group and give item i to the same workgroup, so each workgroup
// adds the residual to exactly the rows it produced in the previous such phase: those rows stay
// in LDS (m.res[(item * S + s) * 8 + r]) and the residual stream is never polled.  Layer 0's
// self block starts from the embedding of the workgroup's rows.
template <int WQ8>
DEV float resid_embed(const StepParams& p, const Lds& m, int s, int row, float pos) {
  const int tk = m.toks[s], d = p.d;
  float e;
  if (!WQ8) {
    e = h2f(static_cast<const uint16_t*>(p.emb)[(size_t)tk * d + row]);
  } else {
    e = (float)static_cast<const int8_t*>(p.emb)[(size_t)tk * d + row] * h2f(p.emb_s[(size_t)tk * (d >> 5) + (row >> 5)]);
  }
  return e + pos;
}

// Merge attention partials, out-projection, bias and residual (the workgroup's own rows):
// xout = xres + (Wo . o + b).
template <int SM, int WQ8, int DR>
DEV bool phase_out(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr, bool cross) {
  constexpr int R = DR;
  const int tid = threadIdx.x, S = p.S, d = p.d, H = p.H;
  const LayerDev& lw = p.layers[l];
  const void* W = cross ? lw.w_co : lw.w_o;
  const uint16_t* Ws = cross ? lw.s_co : lw.s_o;
  const float* bias = cross ? lw.b_co : lw.b_o;
  const int nitems = (d + 7) / 8;
  const int it0 = grp_first(gr);
  if (it0 >= nitems) return true;
  STAMP(0);
  const int nmine = (nitems - it0 + gr.size - 1) / gr.size;
  WBatch<R, 1> wr;
  gemvb_prefetch<R, 1, WQ8>(W, Ws, d, d, it0, gr.size, 1, wr);
  const bool emb_res = !cross && l == 0;
  const bool mine = tid < S * 8;  // thread -> (row s = tid / 8, row-in-item tid % 8)
  auto row_of = [&](int b) -> int { return (it0 + b * gr.size) * 8 + (tid & 7); };
  float bv = 0.f, pv = 0.f;
  if (mine && row_of(0) < d) {
    bv = bias[row_of(0)];
    if (emb_res) pv = p.pos[(size_t)c.pe * d + row_of(0)];
  }
  // partials, merged attention output and reduction buffers: one row in the phase scratch; several
  // rows from the start of the per-phase region (the phase needs no activation buffer)
  const size_t mp = (size_t)(p.ncs_max > p.ncc ? p.ncs_max : p.ncc) * S * H * kPartWords;
  float* part = SM == 1 ? m.big : m.xin;
  float* o = SM == 1 ? m.xn : part + mp;
  float* red = SM == 1 ? part + mp : o + S * d;  // [2][32 * SM]
  const int nc = cross ? p.ncc : (c.kv + kSelfChunk - 1) / kSelfChunk + 1;
  const u64* psrc = cross ? p.cp + (size_t)l * p.ncc * S * H * kPartWords : p.sp + (size_t)l * p.ncs_max * S * H * kPartWords;
  if (!ll_poll1<16>(rep(p, psrc), nc * S * H * kPartWords, part, c.tag, p.err)) return false;
  STAMP(1);
  attn_merge<false>(part, nc, S * H, o);
  u64* xout = (cross ? p.x2 : p.x1) + (size_t)l * S * d;
  for (int b = 0; b < nmine; ++b) {
    if (b > 0) {
      gemvb_prefetch<R, 1, WQ8>(W, Ws, d, d, it0 + b * gr.size, gr.size, 1, wr);
      if (mine && row_of(b) < d) {
        bv = bias[row_of(b)];
        if (emb_res) pv = p.pos[(size_t)c.pe * d + row_of(b)];
      }
    }
    float* rb = red + (b & 1) * 32 * SM;
    gemv_rxm<SM, R, 1, WQ8>(wr, o, S, d, W, Ws, d, it0 + b * gr.size, gr.size, rb);
    lds_barrier();
    if (mine) {
      const int s = tid >> 3, rr = tid & 7, row = row_of(b);
      if (row < d) {
        float* rs = m.res + (b * S + s) * 8 + rr;
        const float xr = emb_res ? resid_embed<WQ8>(p, m, s, row, pv) : *rs;
        const float y = xr + (gemv_outm<SM>(rb, 0, rr, s) + bv);
        *rs = y;
        ll_st(xout + (size_t)s * d + row, y, c.tag, p.rep_stride);
      }
    }
    STAMP(2);
  }
  return true;
}

// Cross-attention with the q projection folded in: one item per (encoder group, head, key chunk);
// the item projects q_h for its rows from LN2(x1), then attends over its chunk of encoder keys.
// Rows sharing an encoder output (beams) are processed together so the chunk's K/V is read once.
template <int SM, int WQ8, int DR>
DEV bool phase_cross(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = DR;
  const int tid = threadIdx.x, S = p.S, d = p.d, H = p.H, L = p.L, sub = tid & 7;
  const LayerDev& lw = p.layers[l];
  const int ngrp = p.X == 1 ? 1 : S;
  const int ns = p.X == 1 ? S : 1;
  const int nitems = ngrp * H * p.ncc;
  int it = grp_first(gr);
  if (it >= nitems) return true;
  STAMP(0);
  VecRegs g2, b2;
  vec_prefetch(lw.ln2_g, d, g2);
  vec_prefetch(lw.ln2_b, d, b2);
  bool have_x = false;
  float* red = m.big;             // [8][32][SM]
  float* wpart = red + 256 * SM;  // [4][kPartWords]
  for (; it < nitems; it += gr.size) {
    const int ch = it % p.ncc, gh = it / p.ncc, h = gh % H, grp = gh / H;
    const int k0 = ch * p.chc;
    const int n = min(p.chc, p.A - k0);
    const size_t base = ((((size_t)grp * L + l) * H + h) * p.A + k0) * kHeadDim;
    auto off = [=](int j) -> size_t { return base + (size_t)j * kHeadDim; };
    WBatch<R, kNB> wq;
    gemvb_prefetch<R, kNB, WQ8>(lw.w_cq, lw.s_cq, d, d, (h * kHeadDim) >> 3, 1, kNB, wq);
    float bq[8];
    bias8(lw.b_cq, h * kHeadDim, bq);
    KVRegs<KPT_CROSS> kr;
    attn_prefetch<KPT_CROSS, 0>(p.xk, p.xv, (size_t)p.X * L * H * p.A * kHeadDim * 2, off, n, kr);
    if (!have_x) {
      if (!ll_poll1<8>(rep(p, p.x1 + (size_t)l * S * d), S * d, m.xin, c.tag, p.err)) return false;
      STAMP(1);
      for (int s = 0; s < S; ++s) ln_row<ln_iters<WQ8, DR>()>(m.xin + s * d, m.xn + s * d, d, g2, b2);
      have_x = true;
    }
    const float* xs = m.xn + (p.X == 1 ? 0 : grp) * d;
    if (ns == 1)
      gemv_rxm<1, R, kNB, WQ8>(wq, xs, 1, d, lw.w_cq, lw.s_cq, d, (h * kHeadDim) >> 3, 1, red);
    else
      gemv_rxm<SM, R, kNB, WQ8>(wq, xs, ns, d, lw.w_cq, lw.s_cq, d, (h * kHeadDim) >> 3, 1, red);
    lds_barrier();
    for (int q = 0; q < ns; ++q) {
      float Q[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) Q[e] = (ns == 1 ? gemv_outm<1>(red, sub, e, 0) : gemv_outm<SM>(red, sub, e, q)) + bq[e];
      float M, Ls, A;
      attn_rx<KPT_CROSS>(kr, n, Q, 0.125f, wpart, M, Ls, A);
      STAMP(2);
      const int row = p.X == 1 ? q : grp;
      u64* dst = p.cp + ((((size_t)l * p.ncc + ch) * S + row) * H + h) * kPartWords;
      if (tid < 64) {
        ll_st(dst + 2 + tid, A, c.tag, p.rep_stride);
        if (tid == 0) {
          ll_st(dst + 0, M, c.tag, p.rep_stride);
          ll_st(dst + 1, Ls, c.tag, p.rep_stride);
        }
      }
      lds_barrier();
    }
  }
  return true;
}

// LN3 + MLP1 + GELU.
template <int SM, int WQ8, int DR>
DEV bool phase_mlp1(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = DR, NBM = 4;
  const int tid = threadIdx.x, S = p.S, d = p.d, d4 = 4 * d;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d4 + 7) / 8;
  const int it0 = grp_first(gr);
  if (it0 >= nitems) return true;
  STAMP(0);
  const int nmine = (nitems - it0 + gr.size - 1) / gr.size;
  WBatch<R, NBM> wr;
  gemvb_prefetch<R, NBM, WQ8>(lw.w_1, lw.s_1, d4, d, it0, gr.size, min(NBM, nmine), wr);
  // thread -> (item tid / (S * 8), row s, row-in-item tid % 8)
  auto row_of = [&](int b) -> int { return (it0 + (b + tid / (S * 8)) * gr.size) * 8 + (tid & 7); };
  auto bias_of = [&](int b) -> float {
    const int nit = min(NBM, nmine - b), row = row_of(b);
    return (tid < nit * S * 8 && row < d4) ? lw.b_1[row] : 0.f;
  };
  float bv = bias_of(0);
  VecRegs g3, b3;
  vec_prefetch(lw.ln3_g, d, g3);
  vec_prefetch(lw.ln3_b, d, b3);
  float* red = m.big;  // [2][NBM * 32 * SM]
  if (!ll_poll1<8>(rep(p, p.x2 + (size_t)l * S * d), S * d, m.xin, c.tag, p.err)) return false;
  STAMP(1);
  for (int s = 0; s < S; ++s) ln_row<ln_iters<WQ8, DR>()>(m.xin + s * d, m.xn + s * d, d, g3, b3);
  for (int b = 0, k = 0; b < nmine; b += NBM, ++k) {
    const int nit = min(NBM, nmine - b);
    if (b > 0) {
      gemvb_prefetch<R, NBM, WQ8>(lw.w_1, lw.s_1, d4, d, it0 + b * gr.size, gr.size, nit, wr);
      bv = bias_of(b);
    }
    float* rb = red + (k & 1) * NBM * 32 * SM;
    gemv_rxm<SM, R, NBM, WQ8>(wr, m.xn, S, d, lw.w_1, lw.s_1, d4, it0 + b * gr.size, gr.size, rb);
    lds_barrier();
    if (tid < nit * S * 8) {
      const int i = tid / (S * 8), s = (tid - i * S * 8) >> 3, rr = tid & 7;
      const int row = row_of(b);
      if (row < d4)
        ll_st(p.hm + ((size_t)l * S + s) * d4 + row, gelu_f16(gemv_outm<SM>(rb, i, rr, s) + bv), c.tag, p.rep_stride);
    }
    STAMP(2);
  }
  return true;
}

// MLP2 + bias + residual (the workgroup's own x2 rows, kept in LDS by the cross-out phase).
template <int SM, int WQ8, int DR>
DEV bool phase_mlp2(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = 4 * DR;
  const int tid = threadIdx.x, S = p.S, d = p.d, d4 = 4 * d;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d + 7) / 8;
  const int it0 = grp_first(gr);
  if (it0 >= nitems) return true;
  STAMP(0);
  const int nmine = (nitems - it0 + gr.size - 1) / gr.size;
  WBatch<R, 1> wr;
  gemvb_prefetch<R, 1, WQ8>(lw.w_2, lw.s_2, d, d4, it0, gr.size, 1, wr);
  const bool mine = tid < S * 8;
  auto row_of = [&](int b) -> int { return (it0 + b * gr.size) * 8 + (tid & 7); };
  float bv = (mine && row_of(0) < d) ? lw.b_2[row_of(0)] : 0.f;
  float* red = m.big;  // [2][32 * SM]
  if (!ll_poll1<16>(rep(p, p.hm + (size_t)l * S * d4), S * d4, m.xin, c.tag, p.err)) return false;
  STAMP(1);
  for (int b = 0; b < nmine; ++b) {
    if (b > 0) {
      gemvb_prefetch<R, 1, WQ8>(lw.w_2, lw.s_2, d, d4, it0 + b * gr.size, gr.size, 1, wr);
      bv = (mine && row_of(b) < d) ? lw.b_2[row_of(b)] : 0.f;
    }
    float* rb = red + (b & 1) * 32 * SM;
    gemv_rxm<SM, R, 1, WQ8>(wr, m.xin, S, d4, lw.w_2, lw.s_2, d, it0 + b * gr.size, gr.size, rb);
    lds_barrier();
    if (mine) {
      const int s = tid >> 3, rr = tid & 7, row = row_of(b);
      if (row < d) {
        float* rs = m.res + (b * S + s) * 8 + rr;
        const float y = *rs + (gemv_outm<SM>(rb, 0, rr, s) + bv);
        *rs = y;
        ll_st(p.x3 + ((size_t)l * S + s) * d + row, y, c.tag, p.rep_stride);
      }
    }
    STAMP(2);
  }
  return true;
}

// Final LN + tied-embedding logits over this workgroup's 8-row vocabulary items (items g, g+G, ...)
// + masks + the workgroup's selection partial per row (a full record and a (max, argmax) pair).
// The session's fixed logit bias (the beam workload's seeded bias) added to this workgroup's
// masked and raw rows before selection; when logits_out is requested the biased raw rows overwrite
// the unbiased ones the GEMV wrote there.
DEV void add_bias_rows(const StepParams& p, float* lg, float* rw, const int* lidx, int nl, int S, int rpw, int st) {
  for (int e = threadIdx.x; e < S * nl; e += kThreads) {
    const int s = e / nl, j = e - s * nl, row = lidx[j];
    if (row < 0) continue;
    const float b = p.bias[row];
    lg[s * rpw + j] += b;
    rw[s * rpw + j] += b;
    if (p.logits_out) p.logits_out[((size_t)st * S + s) * p.V + row] = rw[s * rpw + j];
  }
  lds_barrier();
}

// One-row sessions keep the first nres items resident in LDS; the rest are streamed, two batches
// in flight before the poll.
template <int SM, int WQ8, int DR>
DEV bool phase_logits(const StepParams& p, const Lds& m, const StepCtx& c) {
  // several rows: every item streamed (one-row sessions run phase_logits1, which keeps part of the
  // vocabulary resident in LDS)
  static_assert(SM > 1, "one-row sessions use phase_logits1");
  constexpr int R = DR, NBL = 4;
  const int G = gridDim.x, g = blockIdx.x, tid = threadIdx.x, S = p.S, d = p.d, V = p.V;
  const int nitems = (V + 7) / 8;
  const int nmine = g < nitems ? (nitems - g + G - 1) / G : 0;
  const int nr = 0;
  const int nst = nmine - nr;
  const int nb = (nst + NBL - 1) / NBL;
  const int rpw = p.rows_per_wg;
  float* lg = m.big;                                  // [S][rpw] masked
  float* rw = lg + S * rpw;                           // [S][rpw] raw
  int* lidx = reinterpret_cast<int*>(rw + S * rpw);   // [rpw]
  float* rec = reinterpret_cast<float*>(lidx + rpw);  // [S][kSelWords]
  float* red = rec + S * kSelWords;                   // [2][NBL * 32 * SM]
  WBatch<R, NBL> wa, wb;
  STAMP(0);
  if (nb > 0) gemvb_prefetch<R, NBL, WQ8>(p.emb, p.emb_s, V, d, g + nr * G, G, min(NBL, nst), wa);
  if (nb > 1) gemvb_prefetch<R, NBL, WQ8>(p.emb, p.emb_s, V, d, g + (nr + NBL) * G, G, min(NBL, nst - NBL), wb);
  VecRegs gf, bf;
  vec_prefetch(p.lnf_g, d, gf);
  vec_prefetch(p.lnf_b, d, bf);
  if (!ll_poll1<8>(rep(p, p.x3 + (size_t)(p.L - 1) * S * d), S * d, m.xin, c.tag, p.err)) return false;
  STAMP(1);
  for (int s = 0; s < S; ++s) ln_row<ln_iters<WQ8, DR>()>(m.xin + s * d, m.xn + s * d, d, gf, bf);
  int nbat = 0;  // batches done (alternates the reduction buffers)
  // outputs of a batch of nit items starting at local item i0
  auto emit = [&](const float* rb, int i0, int nit) {
    if (tid < nit * S * 8) {
      const int i = tid / (S * 8), s = (tid - i * S * 8) >> 3, rr = tid & 7;
      const int row = (g + (i0 + i) * G) * 8 + rr, li = (i0 + i) * 8 + rr;
      if (row < V) {
        const float v = gemv_outm<SM>(rb, i, rr, s);
        rw[s * rpw + li] = v;
        lg[s * rpw + li] = (masked(p.mask, p.mw, s, row) || masked(p.mask2, p.mw, s, row)) ? -INFINITY : v;
        if (s == 0) lidx[li] = row;
        if (p.logits_out) p.logits_out[((size_t)c.st * S + s) * V + row] = v;
      } else if (s == 0) {
        lidx[li] = -1;
      }
    }
  };
  auto batch = [&](const WBatch<R, NBL>& w, int b) {
    const int nit = min(NBL, nst - b * NBL);
    float* rb = red + (nbat & 1) * NBL * 32 * SM;
    ++nbat;
    gemv_rxm<SM, R, NBL, WQ8>(w, m.xn, S, d, p.emb, p.emb_s, V, g + (nr + b * NBL) * G, G, rb);
    lds_barrier();
    emit(rb, nr + b * NBL, nit);
  };
  for (int b = 0; b < nb; b += 2) {
    if (b > 0 && b + 1 < nb) gemvb_prefetch<R, NBL, WQ8>(p.emb, p.emb_s, V, d, g + (nr + (b + 1) * NBL) * G, G, min(NBL, nst - (b + 1) * NBL), wb);
    batch(wa, b);
    if (b + 1 < nb) {
      if (b + 2 < nb) gemvb_prefetch<R, NBL, WQ8>(p.emb, p.emb_s, V, d, g + (nr + (b + 2) * NBL) * G, G, min(NBL, nst - (b + 2) * NBL), wa);
      batch(wb, b + 1);
    }
  }
  lds_barrier();
  STAMP(2);
  int nl = nmine * 8;
  if (nmine > 0) {
    const int last_row0 = (g + (nmine - 1) * G) * 8;
    nl = (nmine - 1) * 8 + min(8, V - last_row0);
  }
  if (__builtin_expect(p.bias != nullptr, 0)) add_bias_rows(p, lg, rw, lidx, nl, S, rpw, c.st);
  for (int s = tid >> 6; s < S; s += 4)
    sel_partial(lg + s * rpw, rw + s * rpw, lidx, nl, p.probe, p.topk, rec + s * kSelWords);
  lds_barrier();
  // Self-KV rows this workgroup appended in this step are complete before its partial is visible:
  // every workgroup of the next step's phases waits (directly or through other phases) on the
  // selection, which waits on every workgroup's partial.
  kv_drain();
  for (int i = tid; i < S * kSelWords; i += kThreads) ll_st(p.lp + (size_t)g * S * kSelWords + i, rec[i], c.tag, p.rep_stride);
  for (int i = tid; i < 2 * S; i += kThreads)
    ll_st(p.lpa + (size_t)g * S * 2 + i, rec[(i >> 1) * kSelWords + (i & 1)], c.tag, p.rep_stride);
  return true;
}

// Selection reduction.  Every workgroup that runs a phase reading the next token reduces the
// (max, argmax) pairs; one workgroup also merges the full partials (blocks of kRedBlock
// workgroups) into the step outputs.
// Exclusive scan over the workgroup's threads (in thread order) of per-thread doubles; *total gets
// the sum.  red: 4 doubles of LDS.  LDS-only barriers (global loads in flight stay in flight).
DEV double wg_scan_excl_d(double v, double* red, double* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const double inc = wave_scan_d(v);
  if (lane == 63) red[wave] = inc;
  lds_barrier();
  double pre = __shfl_up(inc, 1);
  pre = lane == 0 ? 0.0 : pre;
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    pre += w < wave ? red[w] : 0.0;
    t += red[w];
  }
  *total = t;
  lds_barrier();
  return pre;
}

// Thread k < n waits for the W tagged words src[W k .. W k + W) and takes their values in v; the
// same bounded wait as ll_poll2 (spin limit, cancel word).  Every thread of the workgroup calls it.
template <int W>
DEV bool ll_poll_regs(const u64* src, int n, float (&v)[W], uint32_t tag, unsigned* err) {
  const int k = threadIdx.x;
  bool fail = false;
  if (k < n) {
    u64 w[W];
#pragma unroll
    for (int u = 0; u < W; ++u) w[u] = ll_ld(src + (size_t)W * k + u);
    unsigned spins = 0;
    while (true) {
      bool ok = true;
#pragma unroll
      for (int u = 0; u < W; ++u)
        if ((uint32_t)(w[u] >> 32) != tag) {
          ok = false;
          w[u] = ll_ld(src + (size_t)W * k + u);
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
#pragma unroll
    for (int u = 0; u < W; ++u) v[u] = __uint_as_float((uint32_t)w[u]);
  } else {
#pragma unroll
    for (int u = 0; u < W; ++u) v[u] = 0.f;
  }
  return !wg_any(fail);
}

// A double as two tagged words, low half at p, high half at p + stride.
DEV void ll_st_d(u64* p, size_t stride, double v, uint32_t tag) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  ll_st(p, __uint_as_float((uint32_t)b), tag, 0);
  ll_st(p + stride, __uint_as_float((uint32_t)(b >> 32)), tag, 0);
}
DEV double words_d(const float* w) {
  return __longlong_as_double((long long)(((unsigned long long)__float_as_uint(w[1]) << 32) | __float_as_uint(w[0])));
}

// Temperature sampling of the step's token by the whole grid, inside the launch (one row, decode
// rules on): WhisperDecoder.sample and the log-probability the decode loop takes of the drawn token
// (main/nn/WhisperDecoder.java:186-187, 576-598, 614-626).  The logits phase stored the masked row in
// p.samp_row (device-coherent) before publishing each workgroup's (maximum, index) pair.  Workgroup g
// owns the contiguous range [g * per, (g + 1) * per) of the row, thread t of it ept consecutive entries:
//   1. M = the row maximum, from the pairs;
//   2. p = exp((double)((l - M) / T)) (the float quotient widened), pf = (float) p; the range's sums of
//      p, pf and exp(pf - 1) in double, published as tagged words;
//   3. every workgroup: the totals in workgroup order, r = u * sum p (u: draw st + 1 of the SplitMix64
//      generator after p.samp_rng), and the first range whose cumulative pf sum reaches r (the last
//      range when none does);
//   4. that range's workgroup finds, in vocabulary order, the first entry whose cumulative weight
//      reaches r (continuing into the following ranges when its own sum fell short by rounding; the
//      last index when none does) and publishes it with its pf;
//   5. every workgroup takes the token; workgroup 0 records it with (pf - 1) - log(sum exp(pf - 1))
//      (the reference's logSoftmax over the rewritten row, whose maximum is exactly 1).
// The sums combine per-thread sequential sums by scans over threads and workgroups: they differ from
// one sequential loop in the last bits of a double.  Compiled only into the step kernel instances
// for sampled runs (SAMP = 1), so the greedy instances keep their registers.
DEV bool phase_sample(const StepParams& p, const Lds& m, const StepCtx& c) {
  const int G = gridDim.x, g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, V = p.V;
  // LDS: the pairs [G][2] (then the token words), 16 doubles and 8 ints of scan scratch (within the
  // phase region, which the selection reduce already sizes to at least 2 G + 48 floats), then, with
  // p.samp_lds, the grid's sums [G][6]
  float* pairs = m.big;
  double* dsc = reinterpret_cast<double*>((reinterpret_cast<uintptr_t>(m.big + 2 * G) + 7) & ~(uintptr_t)7);
  int* isc = reinterpret_cast<int*>(dsc + 16);
  const int per = (V + G - 1) / G, ept = (per + kThreads - 1) / kThreads;
  const float T = p.samp_t;
  u64* sx = p.samp_x;
  // 1. the row maximum
  if (!ll_poll1<8>(rep(p, p.lpa), G * 2, pairs, c.tag, p.err)) return false;
  float mx = -INFINITY;
  for (int k = tid; k < G; k += kThreads) mx = fmaxf(mx, pairs[2 * k]);
  mx = wave_max(mx);
  if (lane == 0) dsc[wave] = mx;
  lds_barrier();
  const float M = fmaxf(fmaxf((float)dsc[0], (float)dsc[1]), fmaxf((float)dsc[2], (float)dsc[3]));
  // 2. this workgroup's range: weights and sums
  const int lo = g * per, hi = min(V, lo + per), j0 = lo + tid * ept;
  float w[kSampEpt];
  double sd = 0.0, sf = 0.0, se = 0.0;
#pragma unroll
  for (int e = 0; e < kSampEpt; ++e) {
    const int j = j0 + e;
    const bool in = e < ept && j < hi;
    const float v = in ? __hip_atomic_load(p.samp_row + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
    const double ex = in ? exp((double)((v - M) / T)) : 0.0;
    w[e] = in ? (float)ex : 0.f;
    sd += ex;
    sf += (double)w[e];
    se += in ? exp((double)(w[e] - 1.0f)) : 0.0;
  }
  double tsf;
  const double pre_t = wg_scan_excl_d(sf, dsc + 4, &tsf);  // this thread's entries' prefix within the range
  const double tsd = wave_sum_d(sd), tse = wave_sum_d(se);
  if (lane == 0) {
    dsc[8 + wave] = tsd;
    dsc[12 + wave] = tse;
  }
  lds_barrier();
  if (tid == 0) {  // workgroup g's six words together (fewer workgroups writing one line)
    ll_st_d(sx + (size_t)g * 6, 1, ((dsc[8] + dsc[9]) + dsc[10]) + dsc[11], c.tag);
    ll_st_d(sx + (size_t)g * 6 + 2, 1, tsf, c.tag);
    ll_st_d(sx + (size_t)g * 6 + 4, 1, ((dsc[12] + dsc[13]) + dsc[14]) + dsc[15], c.tag);
  }
  // 3. every workgroup: totals, the draw, the crossing range (thread k < G takes workgroup k)
  // thread k < G takes workgroup k's sums: polled into LDS in bulk where the phase region has room
  // for them, else each thread polls its six words into registers
  const bool gin = tid < G;
  float sw[6];
  if (p.samp_lds) {
    float* sums = reinterpret_cast<float*>(isc + 8);  // [G][6]
    if (!ll_poll1<8>(sx, G * 6, sums, c.tag, p.err)) return false;
#pragma unroll
    for (int u = 0; u < 6; ++u) sw[u] = gin ? sums[6 * tid + u] : 0.f;
  } else {
    if (!ll_poll_regs<6>(sx, G, sw, c.tag, p.err)) return false;
  }
  const double gsd = gin ? words_d(sw) : 0.0;
  const double gsf = gin ? words_d(sw + 2) : 0.0;
  const double gse = gin ? words_d(sw + 4) : 0.0;
  double SD, SF, SE;
  (void)wg_scan_excl_d(gsd, dsc + 4, &SD);
  const double gpre = wg_scan_excl_d(gsf, dsc + 4, &SF);
  (void)wg_scan_excl_d(gse, dsc + 4, &SE);
  const double r = splitmix_uniform(p.samp_rng, c.st + 1) * SD;
  const int hitg = gin && gpre + gsf >= r ? tid : 0x7fffffff;
  const int wh = wave_min_i(hitg);
  if (lane == 0) isc[wave] = wh;
  lds_barrier();
  int gs = min(min(isc[0], isc[1]), min(isc[2], isc[3]));
  if (gs == 0x7fffffff) gs = G - 1;  // no range reaches r: the last one's scan ends at the last index
  const double gs_pre = __shfl(gpre, gs & 63);  // the crossing range's prefix (wave gs / 64 holds it)
  lds_barrier();
  if (wave == (gs >> 6) && lane == 0) dsc[0] = gs_pre;
  lds_barrier();
  // 4. the crossing range's workgroup: the first entry whose cumulative weight reaches r
  if (g == gs) {
    double cum = dsc[0];
    int tok = 0x7fffffff;
    float tpf = 0.f;
    for (int rg = gs; rg < G; ++rg) {
      float q[kSampEpt];
      double ts = 0.0;
      const int rlo = rg * per, rhi = min(V, rlo + per), r0 = rlo + tid * ept;
      if (rg == gs) {
#pragma unroll
        for (int e = 0; e < kSampEpt; ++e) q[e] = w[e];
        ts = sf;
      } else {
        // past the crossing range (rounding): its weights again from the row
#pragma unroll
        for (int e = 0; e < kSampEpt; ++e) {
          const int j = r0 + e;
          const bool in = e < ept && j < rhi;
          const float v = in ? __hip_atomic_load(p.samp_row + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
          q[e] = in ? (float)exp((double)((v - M) / T)) : 0.f;
          ts += (double)q[e];
        }
      }
      double rtot;
      double cc = cum + (rg == gs ? pre_t : wg_scan_excl_d(ts, dsc + 4, &rtot));
      if (rg == gs) rtot = tsf;
      int cand = 0x7fffffff;
      float cpf = 0.f;
#pragma unroll
      for (int e = 0; e < kSampEpt; ++e) {
        cc += (double)q[e];
        const bool h = cand == 0x7fffffff && e < ept && r0 + e < rhi && cc >= r;
        cand = h ? r0 + e : cand;
        cpf = h ? q[e] : cpf;
      }
      const int wc = wave_min_i(cand);
      if (lane == 0) isc[wave] = wc;
      lds_barrier();
      const int best = min(min(isc[0], isc[1]), min(isc[2], isc[3]));
      lds_barrier();
      if (best != 0x7fffffff) {
        tok = best;
        if (cand == best) dsc[1] = (double)cpf;
        lds_barrier();
        tpf = (float)dsc[1];
        break;
      }
      cum += rtot;
    }
    if (tok == 0x7fffffff) {  // no cumulative weight reached r: the last index
      tok = V - 1;
      tpf = (float)exp((double)((__hip_atomic_load(p.samp_row + V - 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - M) / T));
    }
    if (tid == 0) {
      ll_st(sx + (size_t)G * 6, __int_as_float(tok), c.tag, 0);
      ll_st(sx + (size_t)G * 6 + 1, tpf, c.tag, 0);
    }
  }
  // 5. every workgroup: the token
  float* tw = pairs;  // [2] (the pairs were read in step 1)
  if (!ll_poll1<8>(sx + (size_t)G * 6, 2, tw, c.tag, p.err)) return false;
  const int tok = __float_as_int(tw[0]);
  if (tid == 0) {
    m.toks[0] = tok;
    m.hist[p.nhist0 + c.st] = tok;
    if (g == 0) {
      p.samp_tok[c.st] = tok;
      p.samp_lp[c.st] = (double)(tw[1] - 1.0f) - log(SE);
    }
  }
  lds_barrier();
  return true;
}

template <int SAMP>
DEV bool phase_reduce(const StepParams& p, const Lds& m, const StepCtx& c) {
  const int G = gridDim.x, g = blockIdx.x, tid = threadIdx.x, S = p.S, ng = p.ngroups;
  const bool last_step = c.st + 1 == p.nsteps;
  // Only the workgroups of the first two phases of the next step (layer 0 self-attention and
  // out-projection, which embed the next token) need the token; the output writer needs the
  // records.  Everyone else goes straight to its next phase, whose inputs depend on these.
  // The output writer is the grid's last workgroup: the first phases of the next step give their
  // items to the first workgroups of their groups, so the merge stays off the next step's path.
  const Grp g0 = phase_group(0, G, ng), g1 = phase_group(1, G, ng);
  const int writer = G - 1;
  // A workgroup of those groups that has no item in them at the next step skips the wait (the item
  // counts are the phases' own: self-attention S * H * (cached chunks + 2), out-projection d / 8).
  // With decode rules every workgroup keeps the token history, so every workgroup needs the token.
  const int kvn = c.kv + 1;
  const int self_items = S * p.H * ((kvn + kSelfChunk - 1) / kSelfChunk + 2), out_items = (p.d + 7) / 8;
  const bool need_tok = !last_step && !SAMP && (p.rules || (g >= g0.base && g < g0.base + g0.size && g - g0.base < self_items) ||
                                       (g >= g1.base && g < g1.base + g1.size && g - g1.base < out_items));
  const bool is_writer = g == writer && p.out != nullptr;
  if constexpr (SAMP) {
    // every workgroup takes part in the draw (the last step's token is an output too); the writer
    // then records the step as usual
    if (!phase_sample(p, m, c)) return false;
    if (!is_writer) return true;
  }
  if (!need_tok && !is_writer) return true;
  float* pairs = m.big;  // [G][S][2]
  STAMP(0);
  if (need_tok) {
    if (!ll_poll1<8>(rep(p, p.lpa), G * S * 2, pairs, c.tag, p.err)) return false;
  }
  STAMP(1);
  if (need_tok) {
    for (int s = tid >> 6; s < S; s += 4) {
      const int am = sel_argmax(pairs + 2 * s, G, 2 * S);
      if ((tid & 63) == 0) m.toks[s] = p.forced ? p.forced[(size_t)c.st * S + s] : (am == 0x7fffffff ? 0 : am);
    }
    lds_barrier();
    if (p.rules && tid == 0) m.hist[p.nhist0 + c.st] = m.toks[0];
  }
  if (is_writer) {
    const int nblk = (G + kRedBlock - 1) / kRedBlock;
    float* blk = m.big;                                     // [kRedBlock][S][kSelWords]
    float* brec = blk + (size_t)kRedBlock * S * kSelWords;  // [nblk][S][kSelWords]
    for (int b = 0; b < nblk; ++b) {
      const int gb = b * kRedBlock, ngb = min(kRedBlock, G - gb);
      if (!ll_wait_sparse(rep(p, p.lp + (size_t)gb * S * kSelWords), ngb, S * kSelWords, S * kSelWords - 1, -1, c.tag, p.err)) return false;
      if (!ll_poll1<8>(rep(p, p.lp + (size_t)gb * S * kSelWords), ngb * S * kSelWords, blk, c.tag, p.err)) return false;
      for (int s = tid >> 6; s < S; s += 4)
        sel_merge(blk + s * kSelWords, ngb, S * kSelWords, p.topk, brec + ((size_t)b * S + s) * kSelWords);
      lds_barrier();
    }
    float* fin = brec + (size_t)nblk * S * kSelWords;  // [S][kSelWords]
    for (int s = tid >> 6; s < S; s += 4) sel_merge(brec + s * kSelWords, nblk, S * kSelWords, p.topk, fin + s * kSelWords);
    lds_barrier();
    if (tid < S) rec_to_out(fin + tid * kSelWords, p.topk, p.out + (size_t)c.st * S + tid);
    lds_barrier();
  }
  return true;
}

// ------------------------------------------------------------------------------------------------
// One-row phases (SM = 1: greedy decode of one stream).  Same items, exchange buffers and
// publication order as the phases above, specialised for one row: a lane's activation chunks stay
// in registers across both projections of an item, and the logits read part of the vocabulary
// from LDS.

template <int WQ8, int DR>
DEV bool phase_self1(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = DR;
  const int tid = threadIdx.x, d = p.d, H = p.H, d3 = 3 * d, sub = tid & 7;
  const LayerDev& lw = p.layers[l];
  const int nold = (c.kv + kSelfChunk - 1) / kSelfChunk;
  const int per = nold + 2;
  const int nitems = H * per;
  int it = grp_first(gr);
  if (it >= nitems) return true;
  STAMP(0);
  VecRegs g1, b1, pe;
  vec_prefetch(lw.ln1_g, d, g1);
  vec_prefetch(lw.ln1_b, d, b1);
  if (l == 0) vec_prefetch(p.pos + (size_t)c.pe * d, d, pe);
  const size_t kv_bytes = (size_t)p.L * H * p.max_ctx * kHeadDim * 2;
  const int mc = p.max_ctx;
  bool have_x = false;
  auto ensure_x = [&]() -> bool {
    if (have_x) return true;
    if (l == 0) {
      embed_r<WQ8>(p, m, pe, m.xin);
    } else if (!ll_poll1<8>(rep(p, p.x3 + (size_t)(l - 1) * d), d, m.xin, c.tag, p.err)) {
      return false;
    }
    STAMP(1);
    ln_row<ln_iters<WQ8, DR>()>(m.xin, m.xn, d, g1, b1);
    have_x = true;
    return true;
  };
  float* red = m.big;         // [8][32]
  float* red2 = red + 256;    // [8][32]
  float* wpart = red2 + 256;  // [4][kPartWords]
  for (; it < nitems; it += gr.size) {
    const int j = it % per, h = it / per;
    const int kind = j < nold ? 0 : (j == nold ? 1 : 2);
    const int rowA = (kind == 2 ? 2 * d : 0) + h * kHeadDim;  // q rows, or v rows for the value item
    const int rowB = d + h * kHeadDim;                         // k rows
    u64* dst = p.sp + (((size_t)l * p.ncs_max + (kind == 0 ? j : nold)) * H + h) * kPartWords;
    if (kind == 0) {
      // cached keys: q projection + attention over this chunk
      WBatch<R, kNB> wa;
      gemvb_prefetch<R, kNB, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, rowA >> 3, 1, kNB, wa);
      float bq[8];
      bias8(lw.b_qkv, rowA, bq);
      const int k0 = j * kSelfChunk;
      const int n = min(kSelfChunk, c.kv - k0);
      const int32_t* slots = p.slots;
      const size_t lb = (size_t)l;
      auto off = [=](int jj) -> size_t {
        const int pos = k0 + jj;
        const int slot = slots ? slots[pos] : 0;
        return (((lb + slot) * H + h) * mc + pos) * kHeadDim;
      };
      KVRegs<KPT_SELF> kr;
      attn_prefetch<KPT_SELF, 16>(p.kv_k, p.kv_v, kv_bytes, off, n, kr);
      if (!ensure_x()) return false;
      XR<R, WQ8> X;
      xr_load<R, WQ8>(m.xn, d, X);
      gemv_rx<R, kNB, WQ8>(wa, X, lw.w_qkv, lw.s_qkv, d3, d, rowA >> 3, 1, m.xn, red);
      lds_barrier();
      float Q[8];
      {
        float qv[8];
        gemv_out8(red, sub, qv);
#pragma unroll
        for (int e = 0; e < 8; ++e) Q[e] = qv[e] + bq[e];
      }
      float M, Ls, A;
      attn_rx<KPT_SELF>(kr, n, Q, 0.125f, wpart, M, Ls, A);
      STAMP(2);
      if (tid < 64) {
        ll_st(dst + 2 + tid, A, c.tag, p.rep_stride);
        if (tid == 0) {
          ll_st(dst + 0, M, c.tag, p.rep_stride);
          ll_st(dst + 1, Ls, c.tag, p.rep_stride);
        }
      }
    } else {
      // the current token: (q, k) score and k append, or v append
      WBatch<R, kNB> wa, wb;
      gemvb_prefetch<R, kNB, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, rowA >> 3, 1, kNB, wa);
      if (kind == 1) gemvb_prefetch<R, kNB, WQ8>(lw.w_qkv, lw.s_qkv, d3, d, rowB >> 3, 1, kNB, wb);
      const float ba = tid < kHeadDim ? lw.b_qkv[rowA + tid] : 0.f;
      const float bb = (kind == 1 && tid < kHeadDim) ? lw.b_qkv[rowB + tid] : 0.f;
      if (!ensure_x()) return false;
      XR<R, WQ8> X;
      xr_load<R, WQ8>(m.xn, d, X);
      gemv_rx<R, kNB, WQ8>(wa, X, lw.w_qkv, lw.s_qkv, d3, d, rowA >> 3, 1, m.xn, red);
      if (kind == 1) gemv_rx<R, kNB, WQ8>(wb, X, lw.w_qkv, lw.s_qkv, d3, d, rowB >> 3, 1, m.xn, red2);
      lds_barrier();
      STAMP(2);
      const size_t kvrow = (((size_t)l * H + h) * mc + c.kv) * kHeadDim;
      if (tid < 64) {
        const float va = gemv_out(red, tid >> 3, tid & 7) + ba;
        if (kind == 1) {
          const float vb = gemv_out(red2, tid >> 3, tid & 7) + bb;
          const float t = wave_sum(va * vb);
          if (tid == 0) {
            ll_st(dst + 0, t * 0.125f, c.tag, p.rep_stride);
            ll_st(dst + 1, 1.0f, c.tag, p.rep_stride);
          }
          kv_store(p.kv_k, kv_bytes, kvrow + tid, f2h(vb));
        } else {
          ll_st(dst + 2 + tid, va, c.tag, p.rep_stride);
          kv_store(p.kv_v, kv_bytes, kvrow + tid, f2h(va));
        }
      }
    }
    lds_barrier();
  }
  return true;
}

template <int WQ8, int DR>
DEV bool phase_cross1(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = DR;
  const int tid = threadIdx.x, d = p.d, H = p.H, L = p.L, sub = tid & 7;
  const LayerDev& lw = p.layers[l];
  const int nitems = H * p.ncc;
  int it = grp_first(gr);
  if (it >= nitems) return true;
  STAMP(0);
  VecRegs g2, b2;
  vec_prefetch(lw.ln2_g, d, g2);
  vec_prefetch(lw.ln2_b, d, b2);
  bool have_x = false;
  float* red = m.big;        // [8][32]
  float* wpart = red + 256;  // [4][kPartWords]
  for (; it < nitems; it += gr.size) {
    const int ch = it % p.ncc, h = it / p.ncc;
    const int k0 = ch * p.chc;
    const int n = min(p.chc, p.A - k0);
    const size_t base = ((((size_t)l) * H + h) * p.A + k0) * kHeadDim;
    auto off = [=](int j) -> size_t { return base + (size_t)j * kHeadDim; };
    WBatch<R, kNB> wq;
    gemvb_prefetch<R, kNB, WQ8>(lw.w_cq, lw.s_cq, d, d, (h * kHeadDim) >> 3, 1, kNB, wq);
    float bq[8];
    bias8(lw.b_cq, h * kHeadDim, bq);
    KVRegs<KPT_CROSS> kr;
    attn_prefetch<KPT_CROSS, 0>(p.xk, p.xv, (size_t)L * H * p.A * kHeadDim * 2, off, n, kr);
    if (!have_x) {
      if (!ll_poll1<8>(rep(p, p.x1 + (size_t)l * d), d, m.xin, c.tag, p.err)) return false;
      STAMP(1);
      ln_row<ln_iters<WQ8, DR>()>(m.xin, m.xn, d, g2, b2);
      have_x = true;
    }
    XR<R, WQ8> X;
    xr_load<R, WQ8>(m.xn, d, X);
    gemv_rx<R, kNB, WQ8>(wq, X, lw.w_cq, lw.s_cq, d, d, (h * kHeadDim) >> 3, 1, m.xn, red);
    lds_barrier();
    float Q[8];
    {
      float qv[8];
      gemv_out8(red, sub, qv);
#pragma unroll
      for (int e = 0; e < 8; ++e) Q[e] = qv[e] + bq[e];
    }
    float M, Ls, A;
    attn_rx<KPT_CROSS>(kr, n, Q, 0.125f, wpart, M, Ls, A);
    STAMP(2);
    u64* dst = p.cp + (((size_t)l * p.ncc + ch) * H + h) * kPartWords;
    if (tid < 64) {
      ll_st(dst + 2 + tid, A, c.tag, p.rep_stride);
      if (tid == 0) {
        ll_st(dst + 0, M, c.tag, p.rep_stride);
        ll_st(dst + 1, Ls, c.tag, p.rep_stride);
      }
    }
    lds_barrier();
  }
  return true;
}

// Merge attention partials, out-projection, bias and residual (the workgroup's own rows).
template <int WQ8, int DR>
DEV bool phase_out1(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr, bool cross) {
  constexpr int R = DR;
  const int tid = threadIdx.x, d = p.d, H = p.H;
  const LayerDev& lw = p.layers[l];
  const void* W = cross ? lw.w_co : lw.w_o;
  const uint16_t* Ws = cross ? lw.s_co : lw.s_o;
  const float* bias = cross ? lw.b_co : lw.b_o;
  const int nitems = (d + 7) / 8;
  const int it0 = grp_first(gr);
  if (it0 >= nitems) return true;
  STAMP(0);
  const int nmine = (nitems - it0 + gr.size - 1) / gr.size;
  WBatch<R, 1> wr;
  gemvb_prefetch<R, 1, WQ8>(W, Ws, d, d, it0, gr.size, 1, wr);
  const bool emb_res = !cross && l == 0;
  auto row_of = [&](int b) -> int { return (it0 + b * gr.size) * 8 + (tid & 7); };
  float bv = 0.f, pv = 0.f;
  if (tid < 8 && row_of(0) < d) {
    bv = bias[row_of(0)];
    if (emb_res) pv = p.pos[(size_t)c.pe * d + row_of(0)];
  }
  float* part = m.big;  // [merge_chunks_1(p)][H][kPartWords]
  float* red = part + (size_t)merge_chunks_1(p) * H * kPartWords;  // [2][256]
  const int nc = cross ? p.ncc : (c.kv + kSelfChunk - 1) / kSelfChunk + 1;
  const u64* psrc = cross ? p.cp + (size_t)l * p.ncc * H * kPartWords : p.sp + (size_t)l * p.ncs_max * H * kPartWords;
  if (!ll_poll1<16>(rep(p, psrc), nc * H * kPartWords, part, c.tag, p.err)) return false;
  STAMP(1);
  attn_merge<WQ8 != 0>(part, nc, H, m.xn);  // q8_0: the padded reads keep the kernel from spilling
  XR<R, WQ8> X;
  xr_load<R, WQ8>(m.xn, d, X);
  u64* xout = (cross ? p.x2 : p.x1) + (size_t)l * d;
  for (int b = 0; b < nmine; ++b) {
    if (b > 0) {
      gemvb_prefetch<R, 1, WQ8>(W, Ws, d, d, it0 + b * gr.size, gr.size, 1, wr);
      if (tid < 8 && row_of(b) < d) {
        bv = bias[row_of(b)];
        if (emb_res) pv = p.pos[(size_t)c.pe * d + row_of(b)];
      }
    }
    float* rb = red + (b & 1) * 256;
    gemv_rx<R, 1, WQ8>(wr, X, W, Ws, d, d, it0 + b * gr.size, gr.size, m.xn, rb);
    lds_barrier();
    if (tid < 8) {
      const int row = row_of(b);
      if (row < d) {
        float* rs = m.res + b * 8 + tid;
        const float xr = emb_res ? resid_embed<WQ8>(p, m, 0, row, pv) : *rs;
        const float y = xr + (gemv_out(rb, 0, tid) + bv);
        *rs = y;
        ll_st(xout + row, y, c.tag, p.rep_stride);
      }
    }
    STAMP(2);
  }
  return true;
}

// LN3 + MLP1 + GELU.
template <int WQ8, int DR>
DEV bool phase_mlp1_1(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = DR, NBM = 4;
  const int tid = threadIdx.x, d = p.d, d4 = 4 * d;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d4 + 7) / 8;
  const int it0 = grp_first(gr);
  if (it0 >= nitems) return true;
  STAMP(0);
  const int nmine = (nitems - it0 + gr.size - 1) / gr.size;
  WBatch<R, NBM> wr;
  gemvb_prefetch<R, NBM, WQ8>(lw.w_1, lw.s_1, d4, d, it0, gr.size, min(NBM, nmine), wr);
  auto row_of = [&](int b) -> int { return (it0 + (b + (tid >> 3)) * gr.size) * 8 + (tid & 7); };
  auto bias_of = [&](int b) -> float {
    const int nit = min(NBM, nmine - b), row = row_of(b);
    return (tid < nit * 8 && row < d4) ? lw.b_1[row] : 0.f;
  };
  float bv = bias_of(0);
  VecRegs g3, b3;
  vec_prefetch(lw.ln3_g, d, g3);
  vec_prefetch(lw.ln3_b, d, b3);
  float* red = m.big;  // [2][NBM * 32]
  if (!ll_poll1<8>(rep(p, p.x2 + (size_t)l * d), d, m.xin, c.tag, p.err)) return false;
  STAMP(1);
  ln_row<ln_iters<WQ8, DR>()>(m.xin, m.xn, d, g3, b3);
  XR<R, WQ8> X;
  xr_load<R, WQ8>(m.xn, d, X);
  for (int b = 0, k = 0; b < nmine; b += NBM, ++k) {
    const int nit = min(NBM, nmine - b);
    if (b > 0) {
      gemvb_prefetch<R, NBM, WQ8>(lw.w_1, lw.s_1, d4, d, it0 + b * gr.size, gr.size, nit, wr);
      bv = bias_of(b);
    }
    float* rb = red + (k & 1) * NBM * 32;
    gemv_rx<R, NBM, WQ8>(wr, X, lw.w_1, lw.s_1, d4, d, it0 + b * gr.size, gr.size, m.xn, rb);
    lds_barrier();
    if (tid < nit * 8) {
      const int row = row_of(b);
      if (row < d4) ll_st(p.hm + (size_t)l * d4 + row, gelu_f16(gemv_out(rb, tid >> 3, tid & 7) + bv), c.tag, p.rep_stride);
    }
    STAMP(2);
  }
  return true;
}

// MLP2 + bias + residual (the workgroup's own x2 rows, kept in LDS by the cross-out phase).
template <int WQ8, int DR>
DEV bool phase_mlp2_1(const StepParams& p, const Lds& m, const StepCtx& c, int l, Grp gr) {
  constexpr int R = 4 * DR;
  const int tid = threadIdx.x, d = p.d, d4 = 4 * d;
  const LayerDev& lw = p.layers[l];
  const int nitems = (d + 7) / 8;
  const int it0 = grp_first(gr);
  if (it0 >= nitems) return true;
  STAMP(0);
  const int nmine = (nitems - it0 + gr.size - 1) / gr.size;
  WBatch<R, 1> wr;
  gemvb_prefetch<R, 1, WQ8>(lw.w_2, lw.s_2, d, d4, it0, gr.size, 1, wr);
  auto row_of = [&](int b) -> int { return (it0 + b * gr.size) * 8 + (tid & 7); };
  float bv = (tid < 8 && row_of(0) < d) ? lw.b_2[row_of(0)] : 0.f;
  float* red = m.big;  // [2][256]
  if (!ll_poll1<16>(rep(p, p.hm + (size_t)l * d4), d4, m.xin, c.tag, p.err)) return false;
  STAMP(1);
  XR<R, WQ8> X;
  xr_load<R, WQ8>(m.xin, d4, X);
  for (int b = 0; b < nmine; ++b) {
    if (b > 0) {
      gemvb_prefetch<R, 1, WQ8>(lw.w_2, lw.s_2, d, d4, it0 + b * gr.size, gr.size, 1, wr);
      bv = (tid < 8 && row_of(b) < d) ? lw.b_2[row_of(b)] : 0.f;
    }
    float* rb = red + (b & 1) * 256;
    gemv_rx<R, 1, WQ8>(wr, X, lw.w_2, lw.s_2, d, d4, it0 + b * gr.size, gr.size, m.xin, rb);
    lds_barrier();
    if (tid < 8) {
      const int row = row_of(b);
      if (row < d) {
        float* rs = m.res + b * 8 + tid;
        const float y = *rs + (gemv_out(rb, 0, tid) + bv);
        *rs = y;
        ll_st(p.x3 + (size_t)l * d + row, y, c.tag, p.rep_stride);
      }
    }
    STAMP(2);
  }
  return true;
}

// Final LN + tied-embedding logits + masks + the workgroup's selection partial (one row).
// Decode rules of one greedy step from the n generated tokens in m.hist (WhisperDecoder
// applyRepetitionPenalty / applyNgramBlock, main/nn/WhisperDecoder.java:472-476, 543-564, and
// applyTimestampRules for every step after the first, :484-541): a token that would complete a
// 3-gram or 4-gram already in the history is masked, marked in m.rbits when it is one of this
// workgroup's logits rows (item (row / 8) = g + i * G is local row i * 8 + row % 8); the
// timestamp rules become at most four [lo, hi) ranges in m.rrng.  Runs before the logits poll.
DEV void rules_prepare(const StepParams& p, const Lds& m, int n, int rpw) {
  const int tid = threadIdx.x, G = gridDim.x, g = blockIdx.x, V = p.V, tsb = p.tsb;
  const int* h = m.hist;
  for (int i = tid; i < (rpw + 31) / 32; i += kThreads) m.rbits[i] = 0u;
  lds_barrier();
  const int l1 = n >= 1 ? h[n - 1] : -1, l2 = n >= 2 ? h[n - 2] : -1, l3 = n >= 3 ? h[n - 3] : -1;
  auto mark = [&](int t) {
    if (t < 0 || t >= V) return;
    const int item = t >> 3;
    if (item < g || (item - g) % G != 0) return;
    const int li = ((item - g) / G) * 8 + (t & 7);
    atomicOr(&m.rbits[li >> 5], 1u << (li & 31));
  };
  int last_ts = -1;  // index of the last timestamp token
  for (int i = tid; i < n; i += kThreads) {
    if (tsb > 0 && h[i] >= tsb) last_ts = i;
    if (i <= n - 3 && h[i] == l2 && h[i + 1] == l1) mark(h[i + 2]);
    if (i <= n - 4 && h[i] == l3 && h[i + 1] == l2 && h[i + 2] == l1) mark(h[i + 3]);
  }
  last_ts = -wave_min_i(-last_ts);
  int* red = m.rrng + 5;  // the pair slots double as the four waves' maxima before they are written
  lds_barrier();
  if ((tid & 63) == 0) red[tid >> 6] = last_ts;
  lds_barrier();
  if (tid == 0) {
    const int lt = max(max(red[0], red[1]), max(red[2], red[3]));
    int r[8], nr = 0;
    if (tsb > 0) {
      r[nr++] = tsb - 1;
      r[nr++] = tsb;
      if (n > 0) {
        const bool last_was = h[n - 1] >= tsb, pen_was = n < 2 || h[n - 2] >= tsb;
        if (last_was) {
          r[nr++] = pen_was ? tsb : 0;
          r[nr++] = pen_was ? V : p.eot;
        }
        if (lt >= 0) {
          r[nr++] = tsb;
          r[nr++] = (last_was && !pen_was) ? h[lt] + 1 : h[lt];
        }
      }
    }
    m.rrng[0] = nr / 2;
    for (int k = 0; k < nr; ++k) m.rrng[1 + k] = r[k];
  }
  lds_barrier();
}

DEV bool rule_masked(const StepParams& p, const Lds& m, int row, int li) {
  if (!p.rules) return false;
  if ((m.rbits[li >> 5] >> (li & 31)) & 1u) return true;
  const int nr = m.rrng[0];
  for (int k = 0; k < nr; ++k)
    if (row >= m.rrng[1 + 2 * k] && row < m.rrng[2 + 2 * k]) return true;
  return false;
}

template <int WQ8, int DR, int SAMP>
DEV bool phase_logits1(const StepParams& p, const Lds& m, const StepCtx& c) {
  constexpr int R = DR;
  const int G = gridDim.x, g = blockIdx.x, tid = threadIdx.x, d = p.d, V = p.V;
  const int nitems = (V + 7) / 8;
  const int nmine = g < nitems ? (nitems - g + G - 1) / G : 0;
  const int nr = min(p.nres, nmine);                // items resident in LDS
  const int nst = nmine - nr;                       // items streamed from memory
  const int nb = (nst + kNB - 1) / kNB;
  const int rpw = p.rows_per_wg;
  float* lg = m.big;                                  // [rpw] masked
  float* rw = lg + rpw;                               // [rpw] raw
  int* lidx = reinterpret_cast<int*>(rw + rpw);       // [rpw]
  float* rec = reinterpret_cast<float*>(lidx + rpw);  // [kSelWords]
  float* red = rec + kSelWords;                       // [2][256]
  WBatch<R, kNB> wa, wb;
  STAMP(0);
  // streamed item k (0-based among the streamed ones) is item nr + k of this workgroup; the first
  // two batches are in flight before the poll
  if (nb > 0) gemvb_prefetch<R, kNB, WQ8>(p.emb, p.emb_s, V, d, g + nr * G, G, min(kNB, nst), wa);
  if (nb > 1) gemvb_prefetch<R, kNB, WQ8>(p.emb, p.emb_s, V, d, g + (nr + kNB) * G, G, min(kNB, nst - kNB), wb);
  VecRegs gf, bf;
  vec_prefetch(p.lnf_g, d, gf);
  vec_prefetch(p.lnf_b, d, bf);
  if (!ll_poll1<8>(rep(p, p.x3 + (size_t)(p.L - 1) * d), d, m.xin, c.tag, p.err)) return false;
  STAMP(1);
  ln_row<ln_iters<WQ8, DR>()>(m.xin, m.xn, d, gf, bf);
  XR<R, WQ8> X;
  xr_load<R, WQ8>(m.xn, d, X);
  int nbat = 0;  // batches done (alternates the reduction buffers)
  // outputs of a batch of nit items starting at local item i0
  auto emit = [&](const float* rb, int i0, int nit) {
    if (tid < nit * 8) {
      const int i = tid >> 3, rr = tid & 7;
      const int row = (g + (i0 + i) * G) * 8 + rr, li = (i0 + i) * 8 + rr;
      if (row < V) {
        const float v = gemv_out(rb, i, rr);
        rw[li] = v;
        lg[li] = (masked(p.mask, p.mw, 0, row) || masked(p.mask2, p.mw, 0, row) || rule_masked(p, m, row, li)) ? -INFINITY : v;
        lidx[li] = row;
        if (p.logits_out) p.logits_out[(size_t)c.st * V + row] = v;
      } else {
        lidx[li] = -1;
      }
    }
  };
  for (int b = 0; b < nr; b += kNB, ++nbat) {
    const int nit = min(kNB, nr - b);
    float* rb = red + (nbat & 1) * 256;
    gemv_lds<R, kNB, WQ8>(m.ew + (size_t)b * R * kThreads, m.es + (size_t)b * R * kThreads, nit, X, rb);
    lds_barrier();
    emit(rb, b, nit);
  }
  auto batch = [&](const WBatch<R, kNB>& w, int b) {
    const int nit = min(kNB, nst - b * kNB);
    float* rb = red + (nbat & 1) * 256;
    ++nbat;
    gemv_rx<R, kNB, WQ8>(w, X, p.emb, p.emb_s, V, d, g + (nr + b * kNB) * G, G, m.xn, rb);
    lds_barrier();
    emit(rb, nr + b * kNB, nit);
  };
  for (int b = 0; b < nb; b += 2) {
    if (b > 0 && b + 1 < nb) gemvb_prefetch<R, kNB, WQ8>(p.emb, p.emb_s, V, d, g + (nr + (b + 1) * kNB) * G, G, min(kNB, nst - (b + 1) * kNB), wb);
    batch(wa, b);
    if (b + 1 < nb) {
      if (b + 2 < nb) gemvb_prefetch<R, kNB, WQ8>(p.emb, p.emb_s, V, d, g + (nr + (b + 2) * kNB) * G, G, min(kNB, nst - (b + 2) * kNB), wa);
      batch(wb, b + 1);
    }
  }
  lds_barrier();
  STAMP(2);
  int nl = nmine * 8;
  if (nmine > 0) {
    const int last_row0 = (g + (nmine - 1) * G) * 8;
    nl = (nmine - 1) * 8 + min(8, V - last_row0);
  }
  if (__builtin_expect(p.bias != nullptr, 0)) add_bias_rows(p, lg, rw, lidx, nl, 1, rpw, c.st);
  if constexpr (SAMP) {
    // in-launch sampling: the masked row goes to memory with device-coherent stores, complete in
    // every wave before the pair that tells the other workgroups it is there
    lds_barrier();
    for (int li = tid; li < nl; li += kThreads)
      if (lidx[li] >= 0) __hip_atomic_store(p.samp_row + lidx[li], lg[li], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    kv_drain();
    lds_barrier();
  }
  if (tid < 64) {
    // The (max, argmax) pair goes out first: the next step waits on it, while the full record
    // (log-sum-exp, top-k, probe) only feeds the step outputs.  Same order and ties as sel_partial.
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int j = tid; j < nl; j += 64) {
      const float v = lg[j];
      const int id = lidx[j];
      if (v > bv || (v == bv && id < bi)) {
        bv = v;
        bi = id;
      }
    }
    wave_argmax(bv, bi);
    // this wave appended the step's self-KV rows: they are complete before the pair is visible
    kv_drain();
    if (tid < 2) ll_st(p.lpa + (size_t)g * 2 + tid, tid == 0 ? bv : __int_as_float(bi), c.tag, p.rep_stride);
    sel_partial(lg, rw, lidx, nl, p.probe, p.topk, rec);
  }
  lds_barrier();
  for (int i = tid; i < kSelWords; i += kThreads) ll_st(p.lp + (size_t)g * kSelWords + i, rec[i], c.tag, p.rep_stride);
  return true;
}

template <int SM, int WQ8, int DR, int SAMP>
__global__ void __launch_bounds__(kThreads, 1) k_step(StepParams p) {
  extern __shared__ float lds_raw[];
  // a chained sampled decode that has ended: nothing left to compute (uniform across the grid)
  if (__builtin_expect(p.stop != nullptr, 0) && *p.stop) return;
  const int tid = threadIdx.x, S = p.S, d = p.d;
  Lds m;
  // persistent: scratch words, tokens, residual rows; then the per-phase region
  m.scr = lds_raw;
  m.toks = reinterpret_cast<int*>(m.scr + 8);
  m.res = m.scr + 8 + kMaxRows;
  m.xin = m.res + kResItems * kMaxRows * 8;
  m.xn = m.xin + S * 4 * d;
  m.big = m.xn + S * d;
  m.ew = reinterpret_cast<uint4*>(reinterpret_cast<char*>(lds_raw) + p.res_off);
  m.es = reinterpret_cast<uint16_t*>(m.ew + (size_t)p.nres * DR * kThreads);
  m.hist = reinterpret_cast<int*>(reinterpret_cast<char*>(lds_raw) + p.rules_off);
  m.rbits = reinterpret_cast<uint32_t*>(m.hist + p.hist_cap);
  m.rrng = reinterpret_cast<int*>(m.rbits + (p.rows_per_wg + 31) / 32);
  if (tid < S) m.toks[tid] = p.tokens0[tid];
  if (p.rules)
    for (int i = tid; i < p.nhist0; i += kThreads) m.hist[i] = p.hist0[i];
  if constexpr (SM == 1) {
    if (p.nres > 0) {
      const int nitems = (p.V + 7) / 8, G = gridDim.x;
      const int nmine = blockIdx.x < nitems ? (nitems - blockIdx.x + G - 1) / G : 0;
      load_resident_vocab<WQ8, DR>(p, m.ew, m.es, min(p.nres, nmine));
    }
  }
  lds_barrier();
  const int nph = 6 * p.L + 2;
  const int G = gridDim.x, ng = p.ngroups;
  for (int st = 0; st < p.nsteps; ++st) {
    StepCtx c;
    c.tag = p.tag0 + (uint32_t)st;
    c.st = st;
    c.kv = p.kv_len0 + st;                   // keys already cached; this token is key c.kv
    c.pe = c.kv < p.C - 1 ? c.kv : p.C - 1;  // positional row (clamped as the reference)
    c.nph = nph;
    c.ph = 0;
    for (int l = 0; l < p.L; ++l) {
      const int q = 6 * l;
      if constexpr (SM == 1) {
        if (!phase_self1<WQ8, DR>(p, m, c, l, phase_group(q, G, ng))) return;
        STAMP(3);
        ++c.ph;
        // Decode rules for this step's logits, prepared where the workgroup waits anyway: the
        // group of layer 0's out-projection waits there for the self-attention, the other group
        // waits for the out-projection before its cross-attention.
        const bool in_g1 = grp_first(phase_group(1, G, ng)) != 0x7fffffff;
        if (l == 0 && p.rules && in_g1) rules_prepare(p, m, p.nhist0 + st, p.rows_per_wg);
        if (!phase_out1<WQ8, DR>(p, m, c, l, phase_group(q + 1, G, ng), false)) return;
        STAMP(3);
        ++c.ph;
        if (l == 0 && p.rules && !in_g1) rules_prepare(p, m, p.nhist0 + st, p.rows_per_wg);
        if (!phase_cross1<WQ8, DR>(p, m, c, l, phase_group(q + 2, G, ng))) return;
        STAMP(3);
        ++c.ph;
        if (!phase_out1<WQ8, DR>(p, m, c, l, phase_group(q + 3, G, ng), true)) return;
        STAMP(3);
        ++c.ph;
        if (!phase_mlp1_1<WQ8, DR>(p, m, c, l, phase_group(q + 4, G, ng))) return;
        STAMP(3);
        ++c.ph;
        if (!phase_mlp2_1<WQ8, DR>(p, m, c, l, phase_group(q + 5, G, ng))) return;
        STAMP(3);
        ++c.ph;
        continue;
      }
      if (!phase_self<SM, WQ8, DR>(p, m, c, l, phase_group(q, G, ng))) return;
      STAMP(3);
      ++c.ph;
      if (!phase_out<SM, WQ8, DR>(p, m, c, l, phase_group(q + 1, G, ng), false)) return;
      STAMP(3);
      ++c.ph;
      if (!phase_cross<SM, WQ8, DR>(p, m, c, l, phase_group(q + 2, G, ng))) return;
      STAMP(3);
      ++c.ph;
      if (!phase_out<SM, WQ8, DR>(p, m, c, l, phase_group(q + 3, G, ng), true)) return;
      STAMP(3);
      ++c.ph;
      if (!phase_mlp1<SM, WQ8, DR>(p, m, c, l, phase_group(q + 4, G, ng))) return;
      STAMP(3);
      ++c.ph;
      if (!phase_mlp2<SM, WQ8, DR>(p, m, c, l, phase_group(q + 5, G, ng))) return;
      STAMP(3);
      ++c.ph;
    }
    if constexpr (SM == 1) {
      if (!phase_logits1<WQ8, DR, SAMP>(p, m, c)) return;
    } else {
      if (!phase_logits<SM, WQ8, DR>(p, m, c)) return;
    }
    STAMP(3);
    ++c.ph;
    // a decode with the rules on runs to its end token in this launch: it also ends on a cancel
    // (the word is read before the selection wait, which hides its latency); workgroups that leave
    // a step early make the others' next waits see the cancel word and leave as well
    const bool cancel = p.rules && aborted(p.err);
    if (!phase_reduce<SAMP>(p, m, c)) return;
    STAMP(3);
    ++c.ph;
    // every workgroup saw the same token (all reduce the same pairs): the run ends together
    if (p.rules && st + 1 < p.nsteps && (m.toks[0] == p.eot || cancel)) break;
  }
  kv_drain();
}

// Cooperative launch of one step-kernel instance (grid = one workgroup per CU).
template <int SM, int WQ8, int DR, int SAMP = 0>
static hipError_t launch_step_t(const StepParams& p, int grid, size_t lds, hipStream_t st) {
  hipError_t e = hipFuncSetAttribute((const void*)k_step<SM, WQ8, DR, SAMP>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  StepParams pp = p;
  void* args[] = {&pp};
  return hipLaunchCooperativeKernel((const void*)k_step<SM, WQ8, DR, SAMP>, dim3(grid), dim3(kThreads), args, (unsigned)lds, st);
}

}  // namespace w4h
