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

// ------------------------------------------------------------------------------------------------
// The same projection for every layer at once, as one GEMM: C[frame][n] = xa[frame] . W_n, n over
// the 2 L d output columns (layer l, K then V, d each).  The encoder output is split once into f16
// (hi, lo) planes [Mp][d] (k_xa_split, rows past A zero), so the GEMM stages f16 tiles without
// converting them again for every column block.  A workgroup owns 128 frames x 128 columns (two
// heads of one layer's K or V), 4 waves of 64 x 64 (4 x 4 MFMA tiles each); k in stages of 64, the
// next stage loaded into registers while the current one runs on the matrix cores.  Workgroups
// are ordered so that the column blocks of one XCD are contiguous: the weight tiles a workgroup
// reads stay in that XCD's L2 for the other frame blocks.

constexpr int kX2BM = 128, kX2BN = 128, kX2BK = 64;
constexpr int kX2Ld = kX2BK + kPadH;  // LDS row pitch in halves

__global__ __launch_bounds__(256) void k_xa_split(const float* __restrict__ xa, int A, int d, int Mp,
                                                  _Float16* __restrict__ xh, _Float16* __restrict__ xl) {
  const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= (size_t)Mp * d) return;
  const size_t r = i / d;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (r < (size_t)A) v = *reinterpret_cast<const float4*>(xa + i);
  const float f[4] = {v.x, v.y, v.z, v.w};
  half4 h, l;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = (_Float16)f[e];
    l[e] = (_Float16)(f[e] - (float)h[e]);
  }
  *reinterpret_cast<half4*>(xh + i) = h;
  *reinterpret_cast<half4*>(xl + i) = l;
}

template <int WQ8>
__global__ __launch_bounds__(256) void k_cross_kv2(const LayerDev* __restrict__ layers, int d, int H, int A, int Mt, int Nt,
                                                   const _Float16* __restrict__ xh, const _Float16* __restrict__ xl,
                                                   uint16_t* __restrict__ xk, uint16_t* __restrict__ xv,
                                                   uint16_t* __restrict__ xvt, int Ap) {
  __shared__ __attribute__((aligned(16))) _Float16 s_a[2 * kX2BM * kX2Ld];  // hi plane, then lo plane
  __shared__ __attribute__((aligned(16))) _Float16 s_b[kX2BN * kX2Ld];
  _Float16* s_ah = s_a;
  _Float16* s_al = s_a + kX2BM * kX2Ld;
  __shared__ float s_sc[kX2BN][2];
  // tile of this workgroup: XCD (id % 8) takes the contiguous run [xcd * per, +per) of the
  // column-major tile order (consecutive tiles share their column block)
  const int total = Mt * Nt, per = (total + 7) / 8;
  const int T = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (T >= total) return;
  const int nt = T / Mt, mt = T % Mt;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g = lane >> 4, c16 = lane & 15;
  const int wm = wv >> 1, wn = wv & 1;
  const int m0 = mt * kX2BM;
  const int n0 = nt * kX2BN;                 // column in [0, 2 L d)
  const int l = n0 / (2 * d), isv = (n0 % (2 * d)) / d, c0 = n0 % d;  // c0: first output column of the matrix
  const LayerDev& lw = layers[l];
  const void* W = isv ? lw.w_cv : lw.w_ck;
  const uint16_t* Ws = isv ? lw.s_cv : lw.s_ck;

  // stage registers (named, not arrays: arrays captured by helper lambdas went to scratch): A
  // planes 128 x 64 halves = 1024 x 16 bytes each, 4 per thread (row c >> 3, k 8 (c & 7)); f16
  // weights 128 x 64 halves, 4 per thread; q8_0 128 x 64 bytes, 2 per thread (row c >> 2,
  // k 16 (c & 3)) and the scales of (row tid >> 1, block tid & 1)
  uint4 ah0, ah1, ah2, ah3, al0, al1, al2, al3, b0, b1, b2, b3;
  uint16_t rs = 0;
  const int ar = tid >> 3, ak = 8 * (tid & 7);                 // A / f16 B task of j = 0 (rows + 32 j)
  const int qr = tid >> 2, qk = 16 * (tid & 3);                // q8_0 B task of j = 0 (rows + 64 j)
  const _Float16* xhp = xh + (size_t)(m0 + ar) * d + ak;
  const _Float16* xlp = xl + (size_t)(m0 + ar) * d + ak;
  const size_t rstep = (size_t)32 * d;
#define X2_LOAD(K0)                                                                                                   \
  do {                                                                                                              \
    ah0 = *reinterpret_cast<const uint4*>(xhp + (K0));                                                              \
    ah1 = *reinterpret_cast<const uint4*>(xhp + rstep + (K0));                                                      \
    ah2 = *reinterpret_cast<const uint4*>(xhp + 2 * rstep + (K0));                                                  \
    ah3 = *reinterpret_cast<const uint4*>(xhp + 3 * rstep + (K0));                                                  \
    al0 = *reinterpret_cast<const uint4*>(xlp + (K0));                                                              \
    al1 = *reinterpret_cast<const uint4*>(xlp + rstep + (K0));                                                      \
    al2 = *reinterpret_cast<const uint4*>(xlp + 2 * rstep + (K0));                                                  \
    al3 = *reinterpret_cast<const uint4*>(xlp + 3 * rstep + (K0));                                                  \
    if (!WQ8) {                                                                                                     \
      const uint16_t* wp = static_cast<const uint16_t*>(W) + (size_t)(c0 + ar) * d + ak + (K0);                     \
      b0 = *reinterpret_cast<const uint4*>(wp);                                                                     \
      b1 = *reinterpret_cast<const uint4*>(wp + rstep);                                                             \
      b2 = *reinterpret_cast<const uint4*>(wp + 2 * rstep);                                                         \
      b3 = *reinterpret_cast<const uint4*>(wp + 3 * rstep);                                                         \
    } else {                                                                                                        \
      const int8_t* wp = static_cast<const int8_t*>(W) + (size_t)(c0 + qr) * d + qk + (K0);                         \
      b0 = *reinterpret_cast<const uint4*>(wp);                                                                     \
      b1 = *reinterpret_cast<const uint4*>(wp + 2 * rstep);                                                         \
      rs = Ws[(size_t)(c0 + (tid >> 1)) * (d >> 5) + ((K0) >> 5) + (tid & 1)];                                      \
    }                                                                                                               \
  } while (0)
  const int ao = ar * kX2Ld + ak, astep = 32 * kX2Ld;
  auto stash = [&]() {
    *reinterpret_cast<uint4*>(&s_ah[ao]) = ah0;
    *reinterpret_cast<uint4*>(&s_ah[ao + astep]) = ah1;
    *reinterpret_cast<uint4*>(&s_ah[ao + 2 * astep]) = ah2;
    *reinterpret_cast<uint4*>(&s_ah[ao + 3 * astep]) = ah3;
    *reinterpret_cast<uint4*>(&s_al[ao]) = al0;
    *reinterpret_cast<uint4*>(&s_al[ao + astep]) = al1;
    *reinterpret_cast<uint4*>(&s_al[ao + 2 * astep]) = al2;
    *reinterpret_cast<uint4*>(&s_al[ao + 3 * astep]) = al3;
    if (!WQ8) {
      *reinterpret_cast<uint4*>(&s_b[ao]) = b0;
      *reinterpret_cast<uint4*>(&s_b[ao + astep]) = b1;
      *reinterpret_cast<uint4*>(&s_b[ao + 2 * astep]) = b2;
      *reinterpret_cast<uint4*>(&s_b[ao + 3 * astep]) = b3;
    } else {
      const int o = qr * kX2Ld + qk;
      *reinterpret_cast<half8*>(&s_b[o]) = i8x8_to_h8(make_uint2(b0.x, b0.y));
      *reinterpret_cast<half8*>(&s_b[o + 8]) = i8x8_to_h8(make_uint2(b0.z, b0.w));
      *reinterpret_cast<half8*>(&s_b[o + 64 * kX2Ld]) = i8x8_to_h8(make_uint2(b1.x, b1.y));
      *reinterpret_cast<half8*>(&s_b[o + 64 * kX2Ld + 8]) = i8x8_to_h8(make_uint2(b1.z, b1.w));
      s_sc[tid >> 1][tid & 1] = h2f(rs);
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  X2_LOAD(0);
  for (int k0 = 0; k0 < d; k0 += kX2BK) {
    lds_barrier();  // every wave has read the previous stage
    stash();
    lds_barrier();
    if (k0 + kX2BK < d) X2_LOAD(k0 + kX2BK);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kk = ks * 32 + 8 * g;
      half8 bfr[4];
      float sc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = wn * 64 + j * 16 + c16;
        bfr[j] = *reinterpret_cast<const half8*>(&s_b[col * kX2Ld + kk]);
        sc[j] = WQ8 ? s_sc[col][ks] : 1.f;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wm * 64 + i * 16 + c16;
        const half8 ah = *reinterpret_cast<const half8*>(&s_ah[r * kX2Ld + kk]);
        const half8 al = *reinterpret_cast<const half8*>(&s_al[r * kX2Ld + kk]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!WQ8) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bfr[j], acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bfr[j], acc[i][j], 0, 0, 0);
          } else {
            floatx4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bfr[j], floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bfr[j], t, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(sc[j], t[e], acc[i][j][e]);
          }
        }
      }
    }
  }

  // bias (V), f16, through LDS (the hi planes, 128 x 136 halves) into whole 128-byte rows per head
  constexpr int kOld = kX2BN + kPadH;
  static_assert(kX2BM * kOld <= 2 * kX2BM * kX2Ld, "output tile fits the A planes");
  _Float16* so = s_a;
  lds_barrier();
  const float* bias = isv ? lw.b_cv : nullptr;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = wn * 64 + j * 16 + c16;
    const float b = bias ? bias[c0 + col] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = wm * 64 + i * 16 + 4 * g + e;
        so[r * kOld + col] = (_Float16)(acc[i][j][e] + b);
      }
  }
  lds_barrier();
  const int h0 = c0 / kHeadDim;
  uint16_t* out = isv ? xv : xk;
  // rows (frame, head): task c = (row c >> 4, head (c >> 3) & 1, 16-byte piece c & 7)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = j * 256 + tid;
    const int r = c >> 4, hh = (c >> 3) & 1, pc = c & 7;
    if (m0 + r < A)
      *reinterpret_cast<uint4*>(out + (((size_t)l * H + h0 + hh) * A + m0 + r) * kHeadDim + 8 * pc) =
          *reinterpret_cast<const uint4*>(&so[r * kOld + hh * kHeadDim + 8 * pc]);
  }
  if (isv && xvt) {
    // transposed: task c = (column c >> 4, frames 8 (c & 15) + [0, 8)), frames past A zero
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = j * 256 + tid;
      const int col = c >> 4, f0 = 8 * (c & 15);
      uint16_t e[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const _Float16 v = so[(f0 + q) * kOld + col];
        e[q] = m0 + f0 + q < A ? __builtin_bit_cast(uint16_t, v) : (uint16_t)0;
      }
      const int hh = col / kHeadDim, dm = col % kHeadDim;
      *reinterpret_cast<uint4*>(xvt + (((size_t)l * H + h0 + hh) * kHeadDim + dm) * Ap + m0 + f0) =
          make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16, e[4] | (uint32_t)e[5] << 16,
                     e[6] | (uint32_t)e[7] << 16);
    }
  }
}

size_t cross_kv_scratch_bytes(int A, int d) { return d % kX2BN == 0 ? (size_t)2 * ((A + kX2BM - 1) / kX2BM * kX2BM) * d * 2 : 0; }

hipError_t launch_cross_kv(const LayerDev* layers_dev, int L, int d, int H, int A, int wq8, const float* xa,
                           uint16_t* xk, uint16_t* xv, uint16_t* xvt, int Ap, void* scratch, hipStream_t st) {
  if (d != H * kHeadDim || d % kXkvBK != 0 || A < 1 || L < 1) return hipErrorInvalidValue;
  if (scratch && d % kX2BN == 0) {
    // all layers as one GEMM over f16 (hi, lo) planes of the encoder output
    const int Mp = (A + kX2BM - 1) / kX2BM * kX2BM;
    if (xvt && (Ap % 8 != 0 || Ap < Mp)) return hipErrorInvalidValue;
    _Float16* xh = static_cast<_Float16*>(scratch);
    _Float16* xl = xh + (size_t)Mp * d;
    const size_t n4 = (size_t)Mp * d / 4;
    hipLaunchKernelGGL(k_xa_split, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, xa, A, d, Mp, xh, xl);
    const int Mt = Mp / kX2BM, Nt = 2 * L * d / kX2BN;
    const int grid = (Mt * Nt + 7) / 8 * 8;
    if (wq8)
      hipLaunchKernelGGL(k_cross_kv2<1>, dim3(grid), dim3(256), 0, st, layers_dev, d, H, A, Mt, Nt, xh, xl, xk, xv, xvt, Ap);
    else
      hipLaunchKernelGGL(k_cross_kv2<0>, dim3(grid), dim3(256), 0, st, layers_dev, d, H, A, Mt, Nt, xh, xl, xk, xv, xvt, Ap);
    return hipGetLastError();
  }
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
