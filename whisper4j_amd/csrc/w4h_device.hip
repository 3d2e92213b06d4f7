// Device code of whisper4j_amd for gfx950 outside the step kernels: the op kernels behind the
// kernel-level entry points and their launchers.

#include <mutex>

#include "w4h_kernels.h"

namespace w4h {

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
  lds_barrier();
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
  lds_barrier();
  wg_layernorm(xs, ys, 1, n, g, b, scr);
  for (int i = threadIdx.x; i < n; i += kThreads) y[(size_t)r * n + i] = ys[i];
}

__global__ void k_op_gelu(const float* x, int n, float* y) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = gelu_f16(x[i]);
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
  float* red = sc + kSelfChunk + 4;         // [16][1][64]
  float* part = red + 16 * kHeadDim;        // [nc][kPartWords]
  for (int i = threadIdx.x; i < kHeadDim; i += kThreads) qs[i] = q[h * kHeadDim + i];
  lds_barrier();
  const uint16_t* kb = k + (size_t)h * kv_len * kHeadDim;
  const uint16_t* vb = v + (size_t)h * kv_len * kHeadDim;
  for (int c = 0; c < nc; ++c) {
    const int k0 = c * kSelfChunk, n = min(kSelfChunk, kv_len - k0);
    auto off = [&](int j) -> size_t { return (size_t)(k0 + j) * kHeadDim; };
    KVRegs<KPT_SELF> kr;
    attn_prefetch<KPT_SELF, 0>(kb, vb, (size_t)kv_len * kHeadDim * 2, off, n, kr);
    attn_compute<KPT_SELF, 1>(kr, n, 1, qs, nullptr, nullptr, scale, sc, kSelfChunk + 4, red, pmv, plv, acc);
    for (int i = threadIdx.x; i < kPartWords; i += kThreads)
      part[c * kPartWords + i] = i == 0 ? pmv[0] : (i == 1 ? plv[0] : acc[i - 2]);
    lds_barrier();
  }
  attn_merge<false>(part, nc, 1, acc);
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
  lds_barrier();
  if (threadIdx.x < 64) sel_partial(lg, rw, idx, nl, -1, k, rec);
  lds_barrier();
  for (int i = threadIdx.x; i < kSelWords; i += kThreads) parts[((size_t)r * G + g) * kSelWords + i] = rec[i];
}

__global__ void __launch_bounds__(64) k_op_select_final(const float* parts, int G, int k, w4h_step_out* out) {
  __shared__ float rec[kSelWords];
  const int r = blockIdx.x;
  sel_merge(parts + (size_t)r * G * kSelWords, G, kSelWords, k, rec);
  lds_barrier();
  if (threadIdx.x == 0) rec_to_out(rec, k, out + r);
}

// ------------------------------------------------------------------------------------------------
// launchers

size_t step_lds_bytes(const StepParams& p, int grid) {
  // in floats: persistent words, then the per-phase region [xin S*4d][xn S*d][big]
  const int S = p.S, d = p.d, SM = S > 1 ? kMaxRows : 1;
  const size_t persistent = 8 + kMaxRows + kResItems * kMaxRows * 8;
  const size_t fixed = (size_t)S * 4 * d + (size_t)S * d;
  const size_t mp = (size_t)(p.ncs_max > p.ncc ? p.ncs_max : p.ncc) * S * p.H * kPartWords;
  const size_t self_attn = 512 + 4 * kPartWords;                   // two reductions + wave partials
  const size_t cross_attn = (size_t)kNB * 32 * SM + 4 * kPartWords;  // reduction + wave partials
  const size_t mlp1 = (size_t)2 * 4 * 32 * SM;
  const size_t mlp2 = SM == 1 ? 512 : (size_t)2 * 32 * SM;  // phase_mlp2_1 uses two 256-float buffers
  const size_t nbl = SM == 1 ? kNB : 4;
  const size_t logits = (size_t)2 * S * p.rows_per_wg + p.rows_per_wg + (size_t)S * kSelWords + 2 * nbl * 32 * SM;
  const int nblk = (grid + kRedBlock - 1) / kRedBlock;
  size_t reduce = (size_t)(kRedBlock + nblk + 1) * S * kSelWords;
  if ((size_t)grid * S * 2 > reduce) reduce = (size_t)grid * S * 2;
  // out phases: one row keeps partials + reductions in big; several rows put partials, merged
  // output and reductions at the start of the region
  // phase_out1: partials (room for merge_chunks_1 chunks) + two 256-float reductions
  const size_t out_one = S == 1 ? (size_t)merge_chunks_1(p) * p.H * kPartWords + 512 : 0;
  const size_t out_rows = S == 1 ? 0 : mp + (size_t)S * d + 2 * 32 * SM;
  size_t big = self_attn;
  big = big > cross_attn ? big : cross_attn;
  big = big > mlp1 ? big : mlp1;
  big = big > mlp2 ? big : mlp2;
  big = big > logits ? big : logits;
  big = big > reduce ? big : reduce;
  big = big > out_one ? big : out_one;
  size_t region = fixed + big > out_rows ? fixed + big : out_rows;
  if (S == 1 && p.wq8) {
    // One-row q8_0 GEMV activation loads (xr_load) read a fixed span from xin (4d inputs of the
    // second MLP matrix: 4 * DR rounds) and from xn (d inputs: DR rounds), past K when K is shorter.
    const size_t ce = 16, dr = (size_t)step_rounds(d, p.wq8);
    const size_t span_xin = 32 * 4 * dr * ce, span_xn = (size_t)4 * d + 32 * dr * ce;
    if (region < span_xin) region = span_xin;
    if (region < span_xn) region = span_xn;
  }
  return (persistent + region) * sizeof(float);
}

int step_max_grid(size_t lds_bytes) {
  hipDeviceProp_t prop;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  if (lds_bytes > (size_t)prop.sharedMemPerBlock) return 0;
  return prop.multiProcessorCount;  // one workgroup per CU (launch_bounds(256, 1), <= 160 KB LDS)
}

// Step kernel variants live in their own translation units (w4h_step_*.hip), compiled in parallel.
hipError_t launch_step_1_f16_r2(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_1_f16_r2_s(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_1_f16_r3_s(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_1_q8_r2_s(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_1_f16_r3(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_1_q8_r2(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_8_f16_r2(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_8_f16_r3(const StepParams& p, int grid, size_t lds, hipStream_t st);
hipError_t launch_step_8_q8_r2(const StepParams& p, int grid, size_t lds, hipStream_t st);

hipError_t launch_step(const StepParams& p, int grid, size_t lds, hipStream_t st) {
  const int dr = step_rounds(p.d, p.wq8);
  if (p.S == 1 && p.samp_t > 0.f) {
    if (p.wq8) return launch_step_1_q8_r2_s(p, grid, lds, st);
    return dr == 2 ? launch_step_1_f16_r2_s(p, grid, lds, st) : launch_step_1_f16_r3_s(p, grid, lds, st);
  }
  if (p.samp_t > 0.f) return hipErrorInvalidValue;  // in-launch sampling draws for one row
  if (p.S == 1) {
    if (p.wq8) return launch_step_1_q8_r2(p, grid, lds, st);
    return dr == 2 ? launch_step_1_f16_r2(p, grid, lds, st) : launch_step_1_f16_r3(p, grid, lds, st);
  }
  if (p.wq8) return launch_step_8_q8_r2(p, grid, lds, st);
  return dr == 2 ? launch_step_8_f16_r2(p, grid, lds, st) : launch_step_8_f16_r3(p, grid, lds, st);
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

hipError_t launch_op_gelu(const float* x, int n, float* y, hipStream_t st) {
  hipLaunchKernelGGL(k_op_gelu, dim3((n + 255) / 256), dim3(256), 0, st, x, n, y);
  return hipGetLastError();
}

hipError_t launch_op_attention(const float* q, const uint16_t* k, const uint16_t* v, int nh, int kv_len, float scale,
                               float* out, hipStream_t st) {
  const int nc = (kv_len + kSelfChunk - 1) / kSelfChunk;
  size_t lds = ((size_t)kHeadDim + 16 + kHeadDim + kSelfChunk + 4 + 16 * kHeadDim + (size_t)nc * kPartWords) * sizeof(float);
  hipError_t e = hipFuncSetAttribute((const void*)k_op_attention, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_op_attention, dim3(nh), dim3(kThreads), lds, st, q, k, v, kv_len, scale, out);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Selection without allocation (w4h_op_select_noalloc): the partials live in a fixed device array of
// this file, kSelScratchRows rows of kSelParts partials.  Its address is resolved per device once, with
// that device current; host code only ever uses the resolved pointer (the array's name on the host
// side is a stand-in, not a device address).

constexpr int kSelParts = 64;  // partials (workgroups) per row, as launch_op_select
constexpr int kSelScratchRows = W4H_SELECT_MAX_ROWS;
static __device__ __align__(256) float scratch[(size_t)kSelScratchRows * kSelParts * kSelWords];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
float* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];
}  // namespace

hipError_t select_scratch(int device, float** ptr) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(g_scratch_once[device], [device]() {
    int prev = 0;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess) e = hipSetDevice(device);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    // the partial kernel may need more than the default LDS for long rows
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)k_op_select_part, hipFuncAttributeMaxDynamicSharedMemorySize, kSelectMaxLds);
    if (prev != device) (void)hipSetDevice(prev);
    g_scratch_ptr[device] = e == hipSuccess ? static_cast<float*>(p) : nullptr;
    g_scratch_err[device] = e;
  });
  *ptr = g_scratch_ptr[device];
  return g_scratch_err[device];
}

size_t select_lds_bytes(int n) {
  const size_t rpw = (size_t)(((n + 7) / 8 + kSelParts - 1) / kSelParts) * 8;
  return (3 * rpw + kSelWords) * sizeof(float);
}

hipError_t launch_op_select_noalloc(const float* logits, int rows, int n, const uint32_t* mask, int k, w4h_step_out* out,
                                    float* scratch_ptr, hipStream_t st) {
  const int rpw = (((n + 7) / 8 + kSelParts - 1) / kSelParts) * 8;
  hipLaunchKernelGGL(k_op_select_part, dim3(kSelParts, rows), dim3(kThreads), select_lds_bytes(n), st, logits, n, mask,
                     (n + 31) / 32, k, rpw, scratch_ptr);
  hipLaunchKernelGGL(k_op_select_final, dim3(rows), dim3(64), 0, st, scratch_ptr, kSelParts, k, out);
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
  // one limit for every caller of the partial kernel (the allocation-free entry point shares it)
  e = lds <= (size_t)kSelectMaxLds ? hipFuncSetAttribute((const void*)k_op_select_part,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, kSelectMaxLds)
                                   : hipErrorInvalidValue;
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
