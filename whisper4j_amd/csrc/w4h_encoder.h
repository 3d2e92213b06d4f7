// Interface between the encoder's host code (w4h_encoder_api.cpp) and its kernels (w4h_encoder.hip).
// Not part of the public C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace w4h {

enum EncEpi { kEpiStore = 0, kEpiGelu = 1, kEpiResid = 2, kEpiGeluPos = 3, kEpiQkv = 4, kEpiGeluPlanes = 5 };

constexpr int kEncLnPer = 20;  // LayerNorm row elements per lane (rows up to 1280)
constexpr int kEncPad = 64;    // frame count padding of the attention operand planes

// One encoder GEMM: C[M][N] = A . W^T + bias, A rows at a + m * lda (K contiguous fp32 values;
// lda < K is allowed: the convolutions' overlapping windows), W [N][K] f16, or int8 with f16 block
// scales [N][K / 32] in ws.
struct EncGemm {
  const float* a;
  int lda, M, N, K;
  const void* w;
  const uint16_t* ws;
  const float* bias;   // [N] or null
  float* out;          // [M][ldo] fp32 (every epilogue but kEpiQkv)
  int ldo;
  const float* add;    // kEpiResid: [M][ldo] (may be out); kEpiGeluPos: [M][N]
  uint16_t* qkv;       // kEpiQkv: six f16 planes (q hi, q lo, k hi, k lo, v hi, v lo) of
                       // H * Tp * 64 halves; q, k [H][Tp][64], v [H][64][Tp]
  int Tp;              // kEpiQkv: frames rounded up to kEncPad
};

hipError_t launch_enc_gemm(int epi, const EncGemm& g, hipStream_t st);

// A GEMM of a layer whose activation rows arrive as f16 (hi, lo) planes: C[M][N] = A . W^T + bias
// with A = ah + al, rows [Mp][lda] halves (Mp = M rounded up to 128, the padding rows finite),
// N a multiple of 64, K of 64.  Epilogues kEpiResid (out [M][ldo] fp32 += C), kEpiQkv (as above)
// and kEpiGeluPlanes (GELU(C) as hi / lo planes oh, ol [M][ldo]).
struct EncGemm2 {
  const uint16_t *ah, *al;
  int lda, M, N, K;
  const void* w;
  const uint16_t* ws;
  const float* bias;
  float* out;
  int ldo;
  uint16_t *oh, *ol;
  uint16_t* qkv;
  int Tp;
};
hipError_t launch_enc_gemm2(int epi, const EncGemm2& g, hipStream_t st);
constexpr int kEncRowTile = 128;  // row padding of the (hi, lo) activation planes
// Attention of T frames over themselves for H heads from the kEpiQkv planes; out [T][H * 64] as
// (hi, lo) f16 planes oh, ol.
hipError_t launch_enc_attn(const uint16_t* qkv, int T, int Tp, int H, uint16_t* oh, uint16_t* ol, hipStream_t st);
// LayerNorm rows -> y fp32, or (y null) -> (hi, lo) f16 planes yh, yl.
hipError_t launch_enc_ln(const float* x, int rows, int n, const float* g, const float* b, float* y, uint16_t* yh, uint16_t* yl,
                         hipStream_t st);
// mel [n_mels][frames] -> [frames + 2][n_mels] time-major with a zero frame at each end.
hipError_t launch_enc_mel_t(const float* mel, int n_mels, int frames, float* dst, hipStream_t st);

}  // namespace w4h
