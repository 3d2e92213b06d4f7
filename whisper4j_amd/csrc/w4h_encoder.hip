// Audio encoder for gfx950 (WhisperEncoder.forward, main/nn/WhisperEncoder.java:42-76): conv1 (k 3,
// pad 1) + GELU, conv2 (k 3, stride 2, pad 1) + GELU, + positional embedding, N pre-LN blocks of
// unmasked self-attention over the frames and a GELU MLP (main/nn/ResidualAttentionBlock.java:42-60),
// then ln_post.  Activations live in HBM as [frames][channels] fp32 rows.
//
// Every product runs on the matrix cores (v_mfma_f32_16x16x32_f16, fp32 accumulation) with fp32
// operands entering as f16 hi/lo pairs, hi = f16(x), lo = f16(x - hi):
//   - projections and convolutions: weight (f16, or q8_0 as exact int8 with the block scale applied
//     per 32-k step) x activation (hi, lo): two products per pair, ~22 bits of the activation;
//   - attention: both operands are activations, so q.k and p.v take three products each
//     (hi.hi + hi.lo + lo.hi), ~22 bits of each operand.
// The convolutions are implicit GEMMs: the input is kept time-major with one zero row of padding
// at each end, so output frame t reads the 3 input frames it covers as ONE contiguous row of
// 3 x channels values (stride 1: row t of the padded input; stride 2: row 2t), and the GEMM takes
// rows at a stride smaller than their length.  The weights are repacked at load from [out][in][k]
// to [out][k][in] to match.

#include "w4h_mfma.h"
#include "w4h_encoder.h"

namespace w4h {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;              // accelerator complex dies of an MI355X, each with its own L2
constexpr int kEncBN = 64;            // GEMM columns per workgroup: 4 MFMA column tiles per wave
constexpr int kEncBK = 64;            // k per stage: two MFMA k steps
constexpr int kEncLd = kEncBK + kPadH;  // LDS pitch in halves (144 bytes)

// C = A . W^T + bias over [M][N], with the epilogue EPI:
//   kEpiStore: out = C;  kEpiGelu: out = gelu(C);  kEpiResid: out = add + C (add may alias out);
//   kEpiGeluPos: out = gelu(C) + add (the positional embedding, [M][N]);
//   kEpiQkv: C's columns are q | k | v of H heads; each goes out as f16 hi/lo planes
//   (q pre-multiplied by 0.125, the exact 1/sqrt(64) of the scores): q, k as [H][Tp][64],
//   v transposed as [H][64][Tp] (the attention kernel's operand layouts).
// Each wave owns MT x 16 rows x 64 columns (a workgroup 64 MT rows).  Its activation rows go from
// memory straight into MFMA operand registers (lane: row lane & 15, 8 consecutive k per k step)
// and are split into hi/lo there; only the weight tile, shared by the four waves, is staged in LDS.
// Both are loaded one stage ahead.  MT = 1: two 16-row tiles per wave (half the weight reads per
// product, half the workgroups) measured slower on the widest GEMM (turbo MLP1: 109 against 103 us).
template <int EPI, int WQ8>
__global__ __launch_bounds__(256) void k_enc_gemm(EncGemm g) {
  constexpr int MT = 1;
  constexpr int kEncBM = 64 * MT;
  __shared__ __attribute__((aligned(16))) _Float16 s_b[kEncBN * kEncLd];
  __shared__ float s_sc[kEncBN][2];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int M = g.M, N = g.N, K = g.K;
  // XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs (id % 8), each with
  // its own L2.  XCD x takes the consecutive tiles [x * per, (x + 1) * per) in row-block-major order,
  // so the column tiles of one row block run on one XCD and read its activation rows from that L2.
  const int ncb = (N + kEncBN - 1) / kEncBN, ntiles = ((M + kEncBM - 1) / kEncBM) * ncb;
  const int per = (ntiles + kXcds - 1) / kXcds;
  const int tile = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (tile >= ntiles) return;
  const int m0 = (tile / ncb) * kEncBM, n0 = (tile % ncb) * kEncBN;
  // activation operand of m tile mt: row (clamped; rows past M are dropped) m0 + wv * 16 MT + 16 mt +
  // (lane & 15), k = k0 + 32 ks + 8 (lane >> 4) + [0, 8)
  const float* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    arow[mt] = g.a + (size_t)min(m0 + wv * 16 * MT + 16 * mt + (lane & 15), M - 1) * g.lda + 8 * (lane >> 4);
  float4 ra[MT][4];  // [mt][ks][half]
  // f16 W: 64 x 64 halves, 2 x 16 bytes per thread (row c >> 3, k 8 * (c & 7)); q8_0 W: 64 x 64 int8,
  // 16 bytes per thread (row tid >> 2, k 16 * (tid & 3)) and the scales (row tid >> 1, block tid & 1)
  uint4 rb[2];
  uint4 rq;
  uint16_t rs = 0;
  auto load = [&](int k0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int k = k0 + 32 * ks + 8 * (lane >> 4);
        const bool in = k < K;  // K % 8 == 0: a lane's 8 values are all in range or all out
        ra[mt][2 * ks] = in ? *reinterpret_cast<const float4*>(arow[mt] + k0 + 32 * ks) : make_float4(0.f, 0.f, 0.f, 0.f);
        ra[mt][2 * ks + 1] = in ? *reinterpret_cast<const float4*>(arow[mt] + k0 + 32 * ks + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    if (!WQ8) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = j * 256 + tid;
        const int r = min(n0 + (c >> 3), N - 1), k = k0 + 8 * (c & 7);
        rb[j] = k < K ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(g.w) + (size_t)r * K + k)
                      : make_uint4(0u, 0u, 0u, 0u);
      }
    } else {
      const int r = min(n0 + (tid >> 2), N - 1);
      rq = *reinterpret_cast<const uint4*>(static_cast<const int8_t*>(g.w) + (size_t)r * K + k0 + 16 * (tid & 3));
      if (tid < 128) rs = g.ws[(size_t)min(n0 + (tid >> 1), N - 1) * (K >> 5) + (k0 >> 5) + (tid & 1)];
    }
  };
  auto stash = [&]() {
    if (!WQ8) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = j * 256 + tid;
        *reinterpret_cast<uint4*>(&s_b[(c >> 3) * kEncLd + 8 * (c & 7)]) = rb[j];
      }
    } else {
      const int o = (tid >> 2) * kEncLd + 16 * (tid & 3);
      *reinterpret_cast<half8*>(&s_b[o]) = i8x8_to_h8(make_uint2(rq.x, rq.y));
      *reinterpret_cast<half8*>(&s_b[o + 8]) = i8x8_to_h8(make_uint2(rq.z, rq.w));
      if (tid < 128) s_sc[tid >> 1][tid & 1] = h2f(rs);
    }
  };

  floatx4 acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = floatx4{0.f, 0.f, 0.f, 0.f};

  load(0);
  for (int k0 = 0; k0 < K; k0 += kEncBK) {
    lds_barrier();  // every wave has read the previous weight tile
    stash();
    // this stage's activation operand, split into hi/lo (registers of the loads just consumed)
    half8 ah[MT][2], al[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float v[8] = {ra[mt][2 * ks].x, ra[mt][2 * ks].y, ra[mt][2 * ks].z, ra[mt][2 * ks].w,
                            ra[mt][2 * ks + 1].x, ra[mt][2 * ks + 1].y, ra[mt][2 * ks + 1].z, ra[mt][2 * ks + 1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ah[mt][ks][e] = (_Float16)v[e];
          al[mt][ks][e] = (_Float16)(v[e] - (float)ah[mt][ks][e]);
        }
      }
    lds_barrier();
    load(min(k0 + kEncBK, ((K - 1) / kEncBK) * kEncBK));  // the last stage again at the end
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kk = ks * 32 + 8 * (lane >> 4);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const half8 bfr = *reinterpret_cast<const half8*>(&s_b[(nt * 16 + (lane & 15)) * kEncLd + kk]);
        const float sc = WQ8 ? s_sc[nt * 16 + (lane & 15)][ks] : 1.f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (!WQ8) {
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt][ks], bfr, acc[mt][nt], 0, 0, 0);
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt][ks], bfr, acc[mt][nt], 0, 0, 0);
          } else {
            floatx4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt][ks], bfr, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt][ks], bfr, t, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][nt][e] = fmaf(sc, t[e], acc[mt][nt][e]);
          }
        }
      }
    }
  }

  // Epilogue: lane holds rows wv * 16 MT + 16 mt + 4 * (lane >> 4) + e of column nt * 16 + (lane & 15).
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = n0 + nt * 16 + (lane & 15);
    if (n >= N) continue;
    const float b = g.bias ? g.bias[n] : 0.f;
#pragma unroll
    for (int me = 0; me < 4 * MT; ++me) {
      const int mt = me >> 2, e = me & 3;
      const int m = m0 + wv * 16 * MT + 16 * mt + 4 * (lane >> 4) + e;
      if (m >= M) continue;
      const float c = acc[mt][nt][e] + b;
      if constexpr (EPI == kEpiStore) {
        g.out[(size_t)m * g.ldo + n] = c;
      } else if constexpr (EPI == kEpiGelu) {
        g.out[(size_t)m * g.ldo + n] = gelu_f16(c);
      } else if constexpr (EPI == kEpiResid) {
        g.out[(size_t)m * g.ldo + n] = g.add[(size_t)m * g.ldo + n] + c;
      } else if constexpr (EPI == kEpiGeluPos) {
        g.out[(size_t)m * g.ldo + n] = gelu_f16(c) + g.add[(size_t)m * N + n];
      } else {  // kEpiQkv
        const int d = N / 3, part = n / d, h = (n - part * d) >> 6, ei = n & 63;
        const float v = part == 0 ? c * 0.125f : c;
        const _Float16 hi = (_Float16)v, lo = (_Float16)(v - (float)hi);
        const size_t plane = (size_t)(d >> 6) * g.Tp * kHeadDim;  // halves per (part, hi|lo) plane
        const size_t idx = part == 2 ? ((size_t)h * kHeadDim + ei) * g.Tp + m : ((size_t)h * g.Tp + m) * kHeadDim + ei;
        _Float16* q16 = reinterpret_cast<_Float16*>(g.qkv);
        q16[(size_t)(part * 2) * plane + idx] = hi;
        q16[(size_t)(part * 2 + 1) * plane + idx] = lo;
      }
    }
  }
}

// The per-layer GEMMs, with activation rows that their producers (LayerNorm, attention, the MLP1
// epilogue) wrote as f16 (hi, lo) planes: no conversion in the GEMM, and BM x BN workgroup tiles
// (4 waves of BM/2 x BN/2: BM/32 x BN/32 MFMA tiles each) staged through LDS, k in stages of 64, the next
// stage in registers while the current one runs on the matrix cores.  Workgroups are ordered so
// that an XCD takes a contiguous run of the column-major tile order: its weight tiles stay in its
// L2 across the row blocks.  Two f16 products per (hi, lo) pair, fp32 accumulation; q8_0 weights
// as exact int8 with the block scale per 32-k step.
constexpr int kE2BK = 64;
constexpr int kE2Ld = kE2BK + kPadH;

template <int EPI, int WQ8, int BM, int BN>
__global__ __launch_bounds__(256) void k_enc_gemm2(EncGemm2 g) {
  constexpr int NT = BN / 32;  // MFMA column tiles per wave
  constexpr int MT = BM / 32;  // MFMA row tiles per wave
  __shared__ __attribute__((aligned(16))) _Float16 s_a[2 * BM * kE2Ld];  // hi plane, then lo plane
  __shared__ __attribute__((aligned(16))) _Float16 s_b[BN * kE2Ld];
  __shared__ float s_sc[BN][2];
  _Float16* s_ah = s_a;
  _Float16* s_al = s_a + BM * kE2Ld;
  const int M = g.M, N = g.N, K = g.K;
  const int Mt = (M + BM - 1) / BM, Nt = N / BN, total = Mt * Nt, per = (total + kXcds - 1) / kXcds;
  const int T = (blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (T >= total) return;
  const int m0 = (T % Mt) * BM, n0 = (T / Mt) * BN;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, gq = lane >> 4, c16 = lane & 15;
  const int wm = wv >> 1, wn = wv & 1;

  // stage registers: A planes 128 x 64 halves (4 x 16 bytes per thread and plane: rows ar + 32 j,
  // k ak); f16 weights BN x 64 (BN / 32 per thread, rows ar + 32 j); q8_0 BN x 64 bytes (BN / 64 per
  // thread: rows qr + 64 j, k qk) and the scales of (row tid >> 1, block tid & 1), tid < 2 BN
  const int ar = tid >> 3, ak = 8 * (tid & 7), qr = tid >> 2, qk = 16 * (tid & 3);
  const _Float16* ahp = reinterpret_cast<const _Float16*>(g.ah) + (size_t)(m0 + ar) * g.lda + ak;
  const _Float16* alp = reinterpret_cast<const _Float16*>(g.al) + (size_t)(m0 + ar) * g.lda + ak;
  const size_t astep = (size_t)32 * g.lda;
  uint4 a0_0, a1_0, a2_0, a3_0, l0_0, l1_0, l2_0, l3_0, b0_0, b1_0, b2_0, b3_0;
  uint16_t rs_0 = 0;
#define E2_LOAD(X, K0)                                                                                                \
  do {                                                                                                              \
    a0_##X = *reinterpret_cast<const uint4*>(ahp + (K0));                                                           \
    a1_##X = *reinterpret_cast<const uint4*>(ahp + astep + (K0));                                                   \
    if (BM == 128) {                                                                                                \
      a2_##X = *reinterpret_cast<const uint4*>(ahp + 2 * astep + (K0));                                             \
      a3_##X = *reinterpret_cast<const uint4*>(ahp + 3 * astep + (K0));                                             \
    }                                                                                                               \
    l0_##X = *reinterpret_cast<const uint4*>(alp + (K0));                                                           \
    l1_##X = *reinterpret_cast<const uint4*>(alp + astep + (K0));                                                   \
    if (BM == 128) {                                                                                                \
      l2_##X = *reinterpret_cast<const uint4*>(alp + 2 * astep + (K0));                                             \
      l3_##X = *reinterpret_cast<const uint4*>(alp + 3 * astep + (K0));                                             \
    }                                                                                                               \
    if (!WQ8) {                                                                                                     \
      const uint16_t* wp = static_cast<const uint16_t*>(g.w) + (size_t)(n0 + ar) * K + ak + (K0);                    \
      b0_##X = *reinterpret_cast<const uint4*>(wp);                                                                 \
      b1_##X = *reinterpret_cast<const uint4*>(wp + (size_t)32 * K);                                                \
      if (BN == 128) {                                                                                              \
        b2_##X = *reinterpret_cast<const uint4*>(wp + (size_t)64 * K);                                              \
        b3_##X = *reinterpret_cast<const uint4*>(wp + (size_t)96 * K);                                              \
      }                                                                                                             \
    } else {                                                                                                        \
      const int8_t* wp = static_cast<const int8_t*>(g.w) + (size_t)(n0 + qr) * K + qk + (K0);                        \
      b0_##X = *reinterpret_cast<const uint4*>(wp);                                                                 \
      if (BN == 128) b1_##X = *reinterpret_cast<const uint4*>(wp + (size_t)64 * K);                                 \
      if (tid < 2 * BN) rs_##X = g.ws[(size_t)(n0 + (tid >> 1)) * (K >> 5) + ((K0) >> 5) + (tid & 1)];              \
    }                                                                                                               \
  } while (0)
  const int ao = ar * kE2Ld + ak, ls = 32 * kE2Ld;
#define E2_STASH(X)                                                                                                   \
  do {                                                                                                              \
    *reinterpret_cast<uint4*>(&s_ah[ao]) = a0_##X;                                                                  \
    *reinterpret_cast<uint4*>(&s_ah[ao + ls]) = a1_##X;                                                             \
    if (BM == 128) {                                                                                                \
      *reinterpret_cast<uint4*>(&s_ah[ao + 2 * ls]) = a2_##X;                                                       \
      *reinterpret_cast<uint4*>(&s_ah[ao + 3 * ls]) = a3_##X;                                                       \
    }                                                                                                               \
    *reinterpret_cast<uint4*>(&s_al[ao]) = l0_##X;                                                                  \
    *reinterpret_cast<uint4*>(&s_al[ao + ls]) = l1_##X;                                                             \
    if (BM == 128) {                                                                                                \
      *reinterpret_cast<uint4*>(&s_al[ao + 2 * ls]) = l2_##X;                                                       \
      *reinterpret_cast<uint4*>(&s_al[ao + 3 * ls]) = l3_##X;                                                       \
    }                                                                                                               \
    if (!WQ8) {                                                                                                     \
      *reinterpret_cast<uint4*>(&s_b[ao]) = b0_##X;                                                                 \
      *reinterpret_cast<uint4*>(&s_b[ao + ls]) = b1_##X;                                                            \
      if (BN == 128) {                                                                                              \
        *reinterpret_cast<uint4*>(&s_b[ao + 2 * ls]) = b2_##X;                                                      \
        *reinterpret_cast<uint4*>(&s_b[ao + 3 * ls]) = b3_##X;                                                      \
      }                                                                                                             \
    } else {                                                                                                        \
      const int o = qr * kE2Ld + qk;                                                                                \
      *reinterpret_cast<half8*>(&s_b[o]) = i8x8_to_h8(make_uint2(b0_##X.x, b0_##X.y));                              \
      *reinterpret_cast<half8*>(&s_b[o + 8]) = i8x8_to_h8(make_uint2(b0_##X.z, b0_##X.w));                          \
      if (BN == 128) {                                                                                              \
        *reinterpret_cast<half8*>(&s_b[o + 64 * kE2Ld]) = i8x8_to_h8(make_uint2(b1_##X.x, b1_##X.y));               \
        *reinterpret_cast<half8*>(&s_b[o + 64 * kE2Ld + 8]) = i8x8_to_h8(make_uint2(b1_##X.z, b1_##X.w));           \
      }                                                                                                             \
      if (tid < 2 * BN) s_sc[tid >> 1][tid & 1] = h2f(rs_##X);                                                      \
    }                                                                                                               \
  } while (0)

  floatx4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&]() {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kk = ks * 32 + 8 * gq;
      half8 bfr[NT];
      float sc[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int col = wn * (BN / 2) + j * 16 + c16;
        bfr[j] = *reinterpret_cast<const half8*>(&s_b[col * kE2Ld + kk]);
        sc[j] = WQ8 ? s_sc[col][ks] : 1.f;
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int r = wm * (BM / 2) + i * 16 + c16;
        const half8 ah = *reinterpret_cast<const half8*>(&s_ah[r * kE2Ld + kk]);
        const half8 al = *reinterpret_cast<const half8*>(&s_al[r * kE2Ld + kk]);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
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
  };
  // the next stage's loads are issued while the current one runs
  E2_LOAD(0, 0);
  for (int k0 = 0; k0 < K; k0 += kE2BK) {
    lds_barrier();  // every wave has read the previous stage
    E2_STASH(0);
    lds_barrier();
    if (k0 + kE2BK < K) E2_LOAD(0, k0 + kE2BK);
    compute();
  }
#undef E2_LOAD
#undef E2_STASH

  // epilogue: lane holds rows wm * BM / 2 + 16 i + 4 gq + e of column wn * BN / 2 + 16 j + c16
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int n = n0 + wn * (BN / 2) + j * 16 + c16;
    const float b = g.bias ? g.bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * (BM / 2) + 16 * i + 4 * gq + e;
        if (m >= M) continue;
        const float c = acc[i][j][e] + b;
        if constexpr (EPI == kEpiResid) {
          g.out[(size_t)m * g.ldo + n] += c;
        } else if constexpr (EPI == kEpiGeluPlanes) {
          const float v = gelu_f16(c);
          const _Float16 hi = (_Float16)v;
          reinterpret_cast<_Float16*>(g.oh)[(size_t)m * g.ldo + n] = hi;
          reinterpret_cast<_Float16*>(g.ol)[(size_t)m * g.ldo + n] = (_Float16)(v - (float)hi);
        } else {  // kEpiQkv
          const int d = N / 3, part = n / d, h = (n - part * d) >> 6, ei = n & 63;
          const float v = part == 0 ? c * 0.125f : c;
          const _Float16 hi = (_Float16)v, lo = (_Float16)(v - (float)hi);
          const size_t plane = (size_t)(d >> 6) * g.Tp * kHeadDim;
          const size_t idx = part == 2 ? ((size_t)h * kHeadDim + ei) * g.Tp + m : ((size_t)h * g.Tp + m) * kHeadDim + ei;
          _Float16* q16 = reinterpret_cast<_Float16*>(g.qkv);
          q16[(size_t)(part * 2) * plane + idx] = hi;
          q16[(size_t)(part * 2 + 1) * plane + idx] = lo;
        }
      }
  }
}

// Attention of every frame over every frame for one head (no mask), flash style: a workgroup owns
// 64 query rows (16 per wave) and walks the keys in blocks of 64 (K and V staged in LDS, double
// buffered), with an online softmax in fp32.  Products are taken transposed, S^T = K . Q^T and
// O^T = V^T . P^T, so that the softmax weights come out of the first product (lane: query lane & 15,
// keys 16 nt + 4 (lane >> 4) + [0, 4)) already where the second needs its B operand: the 32 keys of
// one k step are taken in the order {4g + [0,4), 16 + 4g + [0,4)} for lane group g (any order of k
// gives the same sum, V^T is read in the same order).  q.k and p.v each take three f16 products
// (hi.hi + hi.lo + lo.hi).  The operand planes hold Tp frames (a multiple of 64, the frames past T
// zero), so every block load is in range and aligned; keys past T are masked to -inf.
// out[t][h * 64 + e].
constexpr int kAttBQ = 64, kAttBK = 64, kAttLd = 64 + kPadH;

__global__ __launch_bounds__(256) void k_enc_attn(const _Float16* __restrict__ qkv, int T, int Tp, int H, _Float16* __restrict__ oh,
                                                  _Float16* __restrict__ ol) {
  __shared__ __attribute__((aligned(16))) _Float16 s_k[2][2][kAttBK * kAttLd];    // [buffer][hi|lo][key][dim]
  __shared__ __attribute__((aligned(16))) _Float16 s_v[2][2][kHeadDim * kAttLd];  // [buffer][hi|lo][dim][key]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, g4 = 4 * (lane >> 4), c16 = lane & 15;
  const int q0 = blockIdx.x * kAttBQ, h = blockIdx.y;
  const size_t plane = (size_t)H * Tp * kHeadDim;
  const _Float16* Qh = qkv + (size_t)h * Tp * kHeadDim;
  const _Float16* Ql = Qh + plane;
  const _Float16* Kh = qkv + 2 * plane + (size_t)h * Tp * kHeadDim;
  const _Float16* Kl = Kh + plane;
  const _Float16* Vh = qkv + 4 * plane + (size_t)h * kHeadDim * Tp;
  const _Float16* Vl = Vh + plane;
  // this lane's query operand (B of S^T: column = query lane & 15, dims 8 * (lane >> 4) + 32 ks)
  const int qr = q0 + wv * 16 + c16;
  half8 qh[2], ql[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    qh[ks] = *reinterpret_cast<const half8*>(Qh + (size_t)qr * kHeadDim + 32 * ks + 8 * (lane >> 4));
    ql[ks] = *reinterpret_cast<const half8*>(Ql + (size_t)qr * kHeadDim + 32 * ks + 8 * (lane >> 4));
  }
  // key / value block loads: 64 x 64 halves per plane = 512 x 16 bytes, 2 per thread per plane
  // (key or dim tid >> 3 and 32 + that, 8 halves at 8 * (tid & 7)), held in named registers
  const int lr = tid >> 3, lc = 8 * (tid & 7);
  uint4 k0h, k0l, k1h, k1l, v0h, v0l, v1h, v1l;
  auto load = [&](int k0) {
    const size_t ka = (size_t)(k0 + lr) * kHeadDim + lc, kb = ka + (size_t)32 * kHeadDim;
    k0h = *reinterpret_cast<const uint4*>(Kh + ka);
    k0l = *reinterpret_cast<const uint4*>(Kl + ka);
    k1h = *reinterpret_cast<const uint4*>(Kh + kb);
    k1l = *reinterpret_cast<const uint4*>(Kl + kb);
    const size_t va = (size_t)lr * Tp + k0 + lc, vb = va + (size_t)32 * Tp;
    v0h = *reinterpret_cast<const uint4*>(Vh + va);
    v0l = *reinterpret_cast<const uint4*>(Vl + va);
    v1h = *reinterpret_cast<const uint4*>(Vh + vb);
    v1l = *reinterpret_cast<const uint4*>(Vl + vb);
  };
  auto stash = [&](int buf) {
    const int o0 = lr * kAttLd + lc, o1 = o0 + 32 * kAttLd;
    *reinterpret_cast<uint4*>(&s_k[buf][0][o0]) = k0h;
    *reinterpret_cast<uint4*>(&s_k[buf][1][o0]) = k0l;
    *reinterpret_cast<uint4*>(&s_k[buf][0][o1]) = k1h;
    *reinterpret_cast<uint4*>(&s_k[buf][1][o1]) = k1l;
    *reinterpret_cast<uint4*>(&s_v[buf][0][o0]) = v0h;
    *reinterpret_cast<uint4*>(&s_v[buf][1][o0]) = v0l;
    *reinterpret_cast<uint4*>(&s_v[buf][0][o1]) = v1h;
    *reinterpret_cast<uint4*>(&s_v[buf][1][o1]) = v1l;
  };
  floatx4 o[4];  // O^T: dims 16 nd + g4 + e of query c16
#pragma unroll
  for (int nd = 0; nd < 4; ++nd) o[nd] = floatx4{0.f, 0.f, 0.f, 0.f};
  float mrow = -INFINITY, lrow = 0.f;  // of this lane's query
  load(0);
  stash(0);
  load(min(kAttBK, Tp - kAttBK));
  lds_barrier();
  int buf = 0;
  for (int k0 = 0; k0 < T; k0 += kAttBK, buf ^= 1) {  // k0 + 64 <= Tp
    // the next block goes to the other buffer, which every wave finished reading before the last
    // barrier; then the loads of the block after it (the last one again at the end: every load is
    // in range and unconditional)
    stash(buf ^ 1);
    load(min(k0 + 2 * kAttBK, Tp - kAttBK));
    const _Float16* sk0 = s_k[buf][0];
    const _Float16* sk1 = s_k[buf][1];
    const _Float16* sv0 = s_v[buf][0];
    const _Float16* sv1 = s_v[buf][1];
    floatx4 s[4];  // S^T: keys 16 nt + g4 + e of query c16
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      s[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int off = (nt * 16 + c16) * kAttLd + 32 * ks + 8 * (lane >> 4);
        const half8 kh = *reinterpret_cast<const half8*>(sk0 + off);
        const half8 kl = *reinterpret_cast<const half8*>(sk1 + off);
        s[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[ks], s[nt], 0, 0, 0);
        s[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[ks], s[nt], 0, 0, 0);
        s[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[ks], s[nt], 0, 0, 0);
      }
    }
    // online softmax for this lane's query: its 16 keys here, the other 48 in lanes ^16, ^32, ^48
    float mb = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (k0 + nt * 16 + g4 + e >= T) s[nt][e] = -INFINITY;
        mb = fmaxf(mb, s[nt][e]);
      }
    mb = fmaxf(mb, __shfl_xor(mb, 16));
    mb = fmaxf(mb, __shfl_xor(mb, 32));
    const float mn = fmaxf(mrow, mb);
    const float alpha = __expf(mrow - mn);
    mrow = mn;
    float ls = 0.f;
    half8 ph[2], pl[2];  // B of O^T for k step ks: keys {32 ks + g4 + [0,4), 32 ks + 16 + g4 + [0,4)}
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pv = __expf(s[nt][e] - mn);
        ls += pv;
        const _Float16 hi = (_Float16)pv;
        ph[nt >> 1][4 * (nt & 1) + e] = hi;
        pl[nt >> 1][4 * (nt & 1) + e] = (_Float16)(pv - (float)hi);
      }
    ls += __shfl_xor(ls, 16);
    ls += __shfl_xor(ls, 32);
    lrow = lrow * alpha + ls;
#pragma unroll
    for (int nd = 0; nd < 4; ++nd)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[nd][e] *= alpha;
    // O^T += V^T . P^T: A = V^T rows (dims 16 nd + c16) over the same key order
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int nd = 0; nd < 4; ++nd) {
        const int off = (nd * 16 + c16) * kAttLd + 32 * ks + g4;
        half8 vh, vl;
        const half4 a0 = *reinterpret_cast<const half4*>(sv0 + off), a1 = *reinterpret_cast<const half4*>(sv0 + off + 16);
        const half4 b0 = *reinterpret_cast<const half4*>(sv1 + off), b1 = *reinterpret_cast<const half4*>(sv1 + off + 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vh[e] = a0[e];
          vh[4 + e] = a1[e];
          vl[e] = b0[e];
          vl[4 + e] = b1[e];
        }
        o[nd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph[ks], o[nd], 0, 0, 0);
        o[nd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph[ks], o[nd], 0, 0, 0);
        o[nd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl[ks], o[nd], 0, 0, 0);
      }
    }
    lds_barrier();  // this buffer is read; the other one is written
  }
  const int t = q0 + wv * 16 + c16;
  if (t < T) {
    const float inv = 1.f / lrow;
    const size_t base = (size_t)t * H * kHeadDim + h * kHeadDim;
#pragma unroll
    for (int nd = 0; nd < 4; ++nd) {
      half4 hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = o[nd][e] * inv;
        hi[e] = (_Float16)v;
        lo[e] = (_Float16)(v - (float)hi[e]);
      }
      *reinterpret_cast<half4*>(oh + base + nd * 16 + g4) = hi;
      *reinterpret_cast<half4*>(ol + base + nd * 16 + g4) = lo;
    }
  }
}

// LayerNorm of rows of n (eps 1e-5), one wave per row, two passes in fp32 (main/tensor/Tensor.java:592-619).
__global__ __launch_bounds__(256) void k_enc_ln(const float* __restrict__ x, int rows, int n, const float* __restrict__ gam,
                                                const float* __restrict__ bet, float* __restrict__ y, _Float16* __restrict__ yh,
                                                _Float16* __restrict__ yl) {
  const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* xr = x + (size_t)r * n;
  float v[kEncLnPer];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kEncLnPer; ++i) {
    const int j = lane + 64 * i;
    v[i] = j < n ? xr[j] : 0.f;
    s += v[i];
  }
  s = wave_sum(s);
  const float mean = s / (float)n;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kEncLnPer; ++i) {
    const int j = lane + 64 * i;
    const float dd = j < n ? v[i] - mean : 0.f;
    q += dd * dd;
  }
  q = wave_sum(q);
  const float inv = 1.f / sqrtf(q / (float)n + 1e-5f);
#pragma unroll
  for (int i = 0; i < kEncLnPer; ++i) {
    const int j = lane + 64 * i;
    if (j >= n) continue;
    const float o = (v[i] - mean) * inv * gam[j] + bet[j];
    if (y) {
      y[(size_t)r * n + j] = o;
    } else {
      const _Float16 hi = (_Float16)o;
      yh[(size_t)r * n + j] = hi;
      yl[(size_t)r * n + j] = (_Float16)(o - (float)hi);
    }
  }
}

// Time-major copy of the mel input with a zero frame at each end: dst[r][c] = mel[c][r - 1] for
// 1 <= r <= frames, 0 for r = 0 and r = frames + 1.
__global__ void k_enc_mel_t(const float* __restrict__ mel, int n_mels, int frames, float* __restrict__ dst) {
  const int r = blockIdx.x, c = threadIdx.x;
  if (c >= n_mels) return;
  dst[(size_t)r * n_mels + c] = (r >= 1 && r <= frames) ? mel[(size_t)c * frames + r - 1] : 0.f;
}

template <int EPI>
static hipError_t gemm_t(const EncGemm& g, hipStream_t st) {
  const int ntiles = ((g.M + 63) / 64) * ((g.N + kEncBN - 1) / kEncBN);
  const dim3 grid(((ntiles + kXcds - 1) / kXcds) * kXcds);
  if (g.ws)
    hipLaunchKernelGGL((k_enc_gemm<EPI, 1>), grid, dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((k_enc_gemm<EPI, 0>), grid, dim3(256), 0, st, g);
  return hipGetLastError();
}

hipError_t launch_enc_gemm(int epi, const EncGemm& g, hipStream_t st) {
  if (g.M < 1 || g.N < 1 || g.K < 1 || g.K % 8 || g.lda % 4 || (g.ws && g.K % 64)) return hipErrorInvalidValue;
  if (epi == kEpiQkv && (g.N % 192 || g.Tp < g.M || g.Tp % kEncPad)) return hipErrorInvalidValue;
  switch (epi) {
    case kEpiStore: return gemm_t<kEpiStore>(g, st);
    case kEpiGelu: return gemm_t<kEpiGelu>(g, st);
    case kEpiResid: return gemm_t<kEpiResid>(g, st);
    case kEpiGeluPos: return gemm_t<kEpiGeluPos>(g, st);
    case kEpiQkv: return gemm_t<kEpiQkv>(g, st);
    default: return hipErrorInvalidValue;
  }
}

template <int EPI, int BM, int BN>
static hipError_t gemm2_t(const EncGemm2& g, hipStream_t st) {
  const int total = ((g.M + BM - 1) / BM) * (g.N / BN);
  const dim3 grid(((total + kXcds - 1) / kXcds) * kXcds);
  if (g.ws)
    hipLaunchKernelGGL((k_enc_gemm2<EPI, 1, BM, BN>), grid, dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((k_enc_gemm2<EPI, 0, BM, BN>), grid, dim3(256), 0, st, g);
  return hipGetLastError();
}

// Workgroup tile: the largest of 128 x 128, 128 x 64 and 64 x 64 that gives at least min_wg
// workgroups (default 512, two per compute unit), else 64 x 64.  W4H_ENC_MINWG overrides it.
template <int EPI>
static hipError_t gemm2_bn(const EncGemm2& g, hipStream_t st) {
  static const int min_wg = [] {
    const char* e = getenv("W4H_ENC_MINWG");
    return e ? atoi(e) : 512;
  }();
  const int m128 = (g.M + 127) / 128, m64 = (g.M + 63) / 64;
  if (g.N % 128 == 0 && m128 * (g.N / 128) >= min_wg) return gemm2_t<EPI, 128, 128>(g, st);
  if (m128 * (g.N / 64) >= min_wg) return gemm2_t<EPI, 128, 64>(g, st);
  (void)m64;
  return gemm2_t<EPI, 64, 64>(g, st);
}

hipError_t launch_enc_gemm2(int epi, const EncGemm2& g, hipStream_t st) {
  if (g.M < 1 || g.N % 64 || g.K % kE2BK || g.lda % 8 || g.K > g.lda) return hipErrorInvalidValue;
  if (epi == kEpiQkv && (g.N % 192 || g.Tp < g.M || g.Tp % kEncPad)) return hipErrorInvalidValue;
  switch (epi) {
    case kEpiResid: return gemm2_bn<kEpiResid>(g, st);
    case kEpiQkv: return gemm2_bn<kEpiQkv>(g, st);
    case kEpiGeluPlanes: return gemm2_bn<kEpiGeluPlanes>(g, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_enc_attn(const uint16_t* qkv, int T, int Tp, int H, uint16_t* oh, uint16_t* ol, hipStream_t st) {
  if (T < 1 || Tp < T || Tp % kEncPad) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_enc_attn, dim3((T + kAttBQ - 1) / kAttBQ, H), dim3(256), 0, st,
                     reinterpret_cast<const _Float16*>(qkv), T, Tp, H, reinterpret_cast<_Float16*>(oh), reinterpret_cast<_Float16*>(ol));
  return hipGetLastError();
}

hipError_t launch_enc_ln(const float* x, int rows, int n, const float* g, const float* b, float* y, uint16_t* yh, uint16_t* yl,
                         hipStream_t st) {
  if (n > 64 * kEncLnPer || (!y && (!yh || !yl))) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_enc_ln, dim3((rows + 3) / 4), dim3(256), 0, st, x, rows, n, g, b, y, reinterpret_cast<_Float16*>(yh),
                     reinterpret_cast<_Float16*>(yl));
  return hipGetLastError();
}

hipError_t launch_enc_mel_t(const float* mel, int n_mels, int frames, float* dst, hipStream_t st) {
  if (n_mels > 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_enc_mel_t, dim3(frames + 2), dim3((n_mels + 63) & ~63), 0, st, mel, n_mels, frames, dst);
  return hipGetLastError();
}

}  // namespace w4h
