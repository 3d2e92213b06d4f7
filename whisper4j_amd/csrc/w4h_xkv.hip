// Cross-attention K/V projection for gfx950: for every layer, K = xa . Wk^T and V = xa . Wv^T + bv
// over the encoder frames (MultiHeadAttention.forward, cross branch,
// main/nn/MultiHeadAttention.java:65-75; the key projection has no bias), computed once per encoder
// output and stored f16 per head, [layer][head][frame][64], for the decode steps to stream.
//
// One MFMA GEMM per (layer, K or V) matrix: a workgroup owns 128 frames x 64 output columns (one
// head) and walks k in stages of 64.  The encoder output is fp32; like the decode GEMMs, each value
// enters the MFMA as two f16 parts, hi = f16(x) and lo = f16(x - hi), against the same weight
// fragment (~22 bits of x per product, fp32 accumulation).  q8_0 weights enter as exact int8
// values, one 32-element block per MFMA step, and the block's f16 scale multiplies that step's
// fp32 result.  Each stage is loaded into registers while the previous one runs on the matrix
// cores, then split into hi/lo and written to LDS; results leave through LDS as 16-byte rows.
// Sessions whose rows share one encoder output also get V transposed, [layer][head][64][Ap]
// (frames past A zero), the layout their matrix-core cross-attention reads.

#include "w4h_mfma.h"

namespace w4h {

constexpr int kXkvBM = 128;              // frames per workgroup (32 per wave)
constexpr int kXkvBK = 64;               // k per stage (two MFMA steps)
constexpr int kXkvLd = kXkvBK + kPadH;   // LDS row pitch in halves (144 bytes)

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

template <int WQ8>
__global__ __launch_bounds__(256) void k_cross_kv(const LayerDev* __restrict__ layers, int d, int H, int A,
                                                 const float* __restrict__ xa, uint16_t* __restrict__ xk,
                                                 uint16_t* __restrict__ xv, uint16_t* __restrict__ xvt, int Ap) {
  __shared__ __attribute__((aligned(16))) _Float16 s_ah[kXkvBM * kXkvLd];
  __shared__ __attribute__((aligned(16))) _Float16 s_al[kXkvBM * kXkvLd];
  __shared__ __attribute__((aligned(16))) _Float16 s_b[64 * kXkvLd];
  __shared__ float s_sc[64][2];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int t0 = blockIdx.x * kXkvBM, h = blockIdx.y;
  const int l = blockIdx.z >> 1, isv = blockIdx.z & 1;
  const LayerDev& lw = layers[l];
  const void* W = isv ? lw.w_cv : lw.w_ck;
  const uint16_t* Ws = isv ? lw.s_cv : lw.s_ck;
  const size_t wrow0 = (size_t)h * kHeadDim;  // weight row of this head's first output column

  // Stage registers.  Frames: 128 x 64 fp32 = 2048 float4, 8 per thread (float4 c = j * 256 + tid is
  // frame c >> 4, k 4 * (c & 15)); frames past A read frame A - 1 and their results are dropped.
  // f16 weights: 64 rows x 64 halves, 2 x 16 bytes per thread (row c >> 3, k 8 * (c & 7)).  q8_0:
  // 64 rows x 64 int8, 16 bytes per thread (row tid >> 2, k 16 * (tid & 3)), and the scales of
  // (row tid >> 1, block tid & 1) for the first 128 threads.
  float4 ra[8];
  uint4 rb[2];
  uint4 rq;
  uint16_t rs = 0;
  auto load = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = j * 256 + tid;
      const int f = min(t0 + (c >> 4), A - 1);
      ra[j] = *reinterpret_cast<const float4*>(xa + (size_t)f * d + k0 + 4 * (c & 15));
    }
    if (!WQ8) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = j * 256 + tid;
        rb[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(W) + (wrow0 + (c >> 3)) * d + k0 + 8 * (c & 7));
      }
    } else {
      rq = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(W) + (wrow0 + (tid >> 2)) * d + k0 + 16 * (tid & 3));
      if (tid < 128) rs = Ws[(wrow0 + (tid >> 1)) * (size_t)(d >> 5) + (k0 >> 5) + (tid & 1)];
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = j * 256 + tid;
      const int o = (c >> 4) * kXkvLd + 4 * (c & 15);
      const float v[4] = {ra[j].x, ra[j].y, ra[j].z, ra[j].w};
      half4 hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = (_Float16)v[e];
        lo[e] = (_Float16)(v[e] - (float)hi[e]);
      }
      *reinterpret_cast<half4*>(&s_ah[o]) = hi;
      *reinterpret_cast<half4*>(&s_al[o]) = lo;
    }
    if (!WQ8) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = j * 256 + tid;
        *reinterpret_cast<uint4*>(&s_b[(c >> 3) * kXkvLd + 8 * (c & 7)]) = rb[j];
      }
    } else {
      const int o = (tid >> 2) * kXkvLd + 16 * (tid & 3);
      *reinterpret_cast<half8*>(&s_b[o]) = i8x8_to_h8(make_uint2(rq.x, rq.y));
      *reinterpret_cast<half8*>(&s_b[o + 8]) = i8x8_to_h8(make_uint2(rq.z, rq.w));
      if (tid < 128) s_sc[tid >> 1][tid & 1] = h2f(rs);
    }
  };

  floatx4 acc[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};

  load(0);
  for (int k0 = 0; k0 < d; k0 += kXkvBK) {
    lds_barrier();  // every wave has read the previous stage
    stash();
    lds_barrier();
    if (k0 + kXkvBK < d) load(k0 + kXkvBK);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kk = ks * 32 + 8 * (lane >> 4);
      half8 bfr[4];
      float sc[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        bfr[nt] = *reinterpret_cast<const half8*>(&s_b[(nt * 16 + (lane & 15)) * kXkvLd + kk]);
        sc[nt] = WQ8 ? s_sc[nt * 16 + (lane & 15)][ks] : 1.f;
      }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int r = wv * 32 + mt * 16 + (lane & 15);
        const half8 ah = *reinterpret_cast<const half8*>(&s_ah[r * kXkvLd + kk]);
        const half8 al = *reinterpret_cast<const half8*>(&s_al[r * kXkvLd + kk]);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          if (!WQ8) {
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bfr[nt], acc[mt][nt], 0, 0, 0);
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bfr[nt], acc[mt][nt], 0, 0, 0);
          } else {
            floatx4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bfr[nt], floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bfr[nt], t, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][nt][e] = fmaf(sc[nt], t[e], acc[mt][nt][e]);
          }
        }
      }
    }
  }

  // Bias, f16, through LDS (the hi tile) into whole 128-byte output rows.
  lds_barrier();
  const float* bias = isv ? lw.b_cv : nullptr;
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int c = nt * 16 + (lane & 15);
    const float b = bias ? bias[wrow0 + c] : 0.f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = wv * 32 + mt * 16 + 4 * (lane >> 4) + e;
        s_ah[r * kXkvLd + c] = (_Float16)(acc[mt][nt][e] + b);
      }
  }
  lds_barrier();
  uint16_t* out = (isv ? xv : xk) + ((size_t)l * H + h) * A * kHeadDim;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = j * 256 + tid;
    const int r = c >> 3;
    if (t0 + r < A)
      *reinterpret_cast<uint4*>(out + (size_t)(t0 + r) * kHeadDim + 8 * (c & 7)) =
          *reinterpret_cast<const uint4*>(&s_ah[r * kXkvLd + 8 * (c & 7)]);
  }
  if (isv && xvt) {
    // transposed: task c = (dim c >> 4, frames 8 (c & 15) + [0, 8)), one 16-byte row piece each
    uint16_t* ot = xvt + ((size_t)l * H + h) * kHeadDim * Ap;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = j * 256 + tid;
      const int dm = c >> 4, f0 = 8 * (c & 15);
      uint16_t e[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const _Float16 v = s_ah[(f0 + q) * kXkvLd + dm];
        e[q] = t0 + f0 + q < A ? __builtin_bit_cast(uint16_t, v) : (uint16_t)0;
      }
      *reinterpret_cast<uint4*>(ot + (size_t)dm * Ap + t0 + f0) =
          make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16, e[4] | (uint32_t)e[5] << 16,
                     e[6] | (uint32_t)e[7] << 16);
    }
  }
}

hipError_t launch_cross_kv(const LayerDev* layers_dev, int L, int d, int H, int A, int wq8, const float* xa,
                           uint16_t* xk, uint16_t* xv, uint16_t* xvt, int Ap, hipStream_t st) {
  if (d != H * kHeadDim || d % kXkvBK != 0 || A < 1 || L < 1) return hipErrorInvalidValue;
  // every frame tile of the transposed copy lies inside its rows
  if (xvt && (Ap % 8 != 0 || Ap < (A + kXkvBM - 1) / kXkvBM * kXkvBM)) return hipErrorInvalidValue;
  const dim3 grid((A + kXkvBM - 1) / kXkvBM, H, 2 * L);
  if (wq8)
    hipLaunchKernelGGL(k_cross_kv<1>, grid, dim3(256), 0, st, layers_dev, d, H, A, xa, xk, xv, xvt, Ap);
  else
    hipLaunchKernelGGL(k_cross_kv<0>, grid, dim3(256), 0, st, layers_dev, d, H, A, xa, xk, xv, xvt, Ap);
  return hipGetLastError();
}

}  // namespace w4h
