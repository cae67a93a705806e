// CDNA4 (gfx950) kernels of the training step. Wave64 throughout; reductions use cross-lane
// shuffles within a wave and LDS across waves; matrix contractions use the f32 MFMA
// (v_mfma_f32_16x16x4f32). Built with -ffp-contract=off: every f32 expression rounds as written,
// and fused multiply-adds appear only where a kernel calls __builtin_fmaf.
#include "kernels.h"

#include <algorithm>
#include <stdexcept>
#include <string>

namespace msx::hk {

namespace {
typedef float v4f __attribute__((ext_vector_type(4)));

[[noreturn]] void bad(const std::string& what) { throw std::runtime_error("kernel launch refused: " + what); }

inline unsigned blocks_for(int64_t n, int per) { return unsigned((n + per - 1) / per); }

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// The GELU of interpreter.rs:1539-1587 in device arithmetic: the nearest f32 constants, the same
// operation order, the device expf.
__device__ __forceinline__ float d_gelu_twice_inner(float x) {
  const float scale = 0.797884560802865f, cubic = 0.044715f;
  return 2.0f * scale * (x + cubic * x * x * x);
}
__device__ __forceinline__ float d_logistic(float v) { return 1.0f / (1.0f + expf(0.0f - v)); }
__device__ __forceinline__ float d_gelu(float x) { return x * d_logistic(d_gelu_twice_inner(x)); }
__device__ __forceinline__ float d_gelu_grad(float x, float g) {
  const float scale = 0.797884560802865f, cubic = 0.044715f;
  float v = d_gelu_twice_inner(x);
  float s = d_logistic(v), r = d_logistic(0.0f - v);
  float slope = scale * (1.0f + 3.0f * cubic * x * x);
  return (s + 2.0f * (s * x) * r * slope) * g;
}

// Philox4x32-10 word 0 (train/init.rs:91-109), on the device for the dropout masks.
__device__ __forceinline__ uint32_t philox_w0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                              uint32_t k1) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    if (round > 0) { k0 += W0; k1 += W1; }
    uint32_t hi0 = __umulhi(M0, c0), lo0 = M0 * c0, hi1 = __umulhi(M1, c2), lo1 = M1 * c2;
    uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
  }
  return c0;
}
}  // namespace

// ---------------------------------------------------------------------------------------------
// Elementwise.
__global__ void k_elementwise(int op, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ o,
                              int64_t n, int as, int bs) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (; i < n; i += stride) {
    float x = a[as ? 0 : i];
    float r;
    switch (op) {
      case EW_ADD: r = x + b[bs ? 0 : i]; break;
      case EW_SUB: r = x - b[bs ? 0 : i]; break;
      case EW_MUL: r = x * b[bs ? 0 : i]; break;
      case EW_DIV: r = x / b[bs ? 0 : i]; break;
      case EW_RELU: r = x > 0.0f ? x : 0.0f; break;
      case EW_RELU_GRAD: r = x > 0.0f ? b[i] : 0.0f; break;
      case EW_GELU: r = d_gelu(x); break;
      case EW_GELU_GRAD: r = d_gelu_grad(x, b[i]); break;
      case EW_SQRT: r = sqrtf(x); break;
      default: r = x; break;
    }
    o[i] = r;
  }
}

void elementwise(hipStream_t s, int op, const float* a, const float* b, float* o, int64_t n, bool as, bool bs) {
  if (n <= 0) return;
  unsigned grid = std::min<unsigned>(blocks_for(n, 256), 8192);
  hipLaunchKernelGGL(k_elementwise, dim3(grid), dim3(256), 0, s, op, a, b, o, n, int(as), int(bs));
}

void copy(hipStream_t s, const float* a, float* o, int64_t n) { elementwise(s, EW_COPY, a, nullptr, o, n, false, false); }

__global__ void k_fill_from(const float* __restrict__ v, float* __restrict__ o, int64_t n) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  float x = v[0];
  for (; i < n; i += int64_t(gridDim.x) * blockDim.x) o[i] = x;
}
void fill_from(hipStream_t s, const float* v, float* o, int64_t n) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_fill_from, dim3(std::min<unsigned>(blocks_for(n, 256), 8192)), dim3(256), 0, s, v, o, n);
}

__global__ void k_fill_zero(uint32_t* __restrict__ o, int64_t words) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t stride = int64_t(gridDim.x) * blockDim.x;
  // Four words a thread per pass where they fit: 16-byte stores.
  int64_t quads = words / 4;
  uint4* o4 = reinterpret_cast<uint4*>(o);
  for (int64_t q = i; q < quads; q += stride) o4[q] = make_uint4(0, 0, 0, 0);
  for (int64_t w = quads * 4 + i; w < words; w += stride) o[w] = 0;
}
void fill_zero(hipStream_t s, void* o, int64_t bytes) {
  if (bytes <= 0) return;
  if (bytes % 4 || reinterpret_cast<uintptr_t>(o) % 16) bad("fill_zero needs 16-byte aligned whole words");
  int64_t words = bytes / 4;
  hipLaunchKernelGGL(k_fill_zero, dim3(std::min<unsigned>(blocks_for(words / 4 + 1, 256), 8192)), dim3(256), 0, s,
                     static_cast<uint32_t*>(o), words);
}

// ---------------------------------------------------------------------------------------------
// GEMM on the f32 MFMA: a 64x64 output tile per 256-thread block, each wave a 32x32 quarter as
// 2x2 MFMA 16x16x4 tiles, K staged through LDS 16 at a time. Operands may be read transposed in
// place. Split-K writes each slice's partial to the workspace; a second kernel sums the slices in
// ascending order, so the result is deterministic.
namespace {
constexpr int BM = 64, BN = 64, BK = 16;
}

template <bool TA, bool TB>
__global__ __launch_bounds__(256) void k_gemm(const float* __restrict__ A, const float* __restrict__ B,
                                              float* __restrict__ C, const float* __restrict__ bias, int64_t M,
                                              int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                                              int64_t kchunk, float* __restrict__ ws) {
  __shared__ float As[BK][BM + 4];
  __shared__ float Bs[BK][BN + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = int64_t(blockIdx.y) * BM, n0 = int64_t(blockIdx.x) * BN;
  const int64_t kbeg = int64_t(blockIdx.z) * kchunk;
  const int64_t kend = K < kbeg + kchunk ? K : kbeg + kchunk;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  v4f acc00 = {0, 0, 0, 0}, acc01 = acc00, acc10 = acc00, acc11 = acc00;
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
#pragma unroll
    for (int e0 = 0; e0 < BM * BK; e0 += 256) {
      int e = e0 + tid;
      int i, kk;
      if (!TA) { i = e / BK; kk = e % BK; } else { kk = e / BM; i = e % BM; }
      int64_t gi = m0 + i, gk = k0 + kk;
      float v = 0.0f;
      if (gi < M && gk < kend) v = TA ? A[gk * lda + gi] : A[gi * lda + gk];
      As[kk][i] = v;
    }
#pragma unroll
    for (int e0 = 0; e0 < BK * BN; e0 += 256) {
      int e = e0 + tid;
      int j, kk;
      if (!TB) { kk = e / BN; j = e % BN; } else { j = e / BK; kk = e % BK; }
      int64_t gj = n0 + j, gk = k0 + kk;
      float v = 0.0f;
      if (gj < N && gk < kend) v = TB ? B[gj * ldb + gk] : B[gk * ldb + gj];
      Bs[kk][j] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      const int kr = kk + (lane >> 4), c = lane & 15;
      float a0 = As[kr][wm + c], a1 = As[kr][wm + 16 + c];
      float b0 = Bs[kr][wn + c], b1 = Bs[kr][wn + 16 + c];
      acc00 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc00, 0, 0, 0);
      acc01 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc01, 0, 0, 0);
      acc10 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc10, 0, 0, 0);
      acc11 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc11, 0, 0, 0);
    }
    __syncthreads();
  }
  const v4f* accs[4] = {&acc00, &acc01, &acc10, &acc11};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int si = t >> 1, sj = t & 1;
    const int64_t col = n0 + wn + sj * 16 + (lane & 15);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = m0 + wm + si * 16 + 4 * (lane >> 4) + r;
      if (row < M && col < N) {
        float v = (*accs[t])[r];
        if (ws) ws[int64_t(blockIdx.z) * M * N + row * N + col] = v;
        else C[row * ldc + col] = bias ? v + bias[col] : v;
      }
    }
  }
}

__global__ void k_splitk_reduce(const float* __restrict__ ws, float* __restrict__ C, const float* __restrict__ bias,
                                int64_t M, int64_t N, int64_t ldc, int splits) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t mn = M * N;
  for (; i < mn; i += int64_t(gridDim.x) * blockDim.x) {
    float acc = ws[i];
    for (int z = 1; z < splits; ++z) acc = acc + ws[int64_t(z) * mn + i];
    int64_t row = i / N, col = i % N;
    C[row * ldc + col] = bias ? acc + bias[col] : acc;
  }
}

int gemm_split_for(int64_t m, int64_t n, int64_t k) {
  int64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  if (tiles >= 512 || k < 256) return 1;
  int64_t want = (1024 + tiles - 1) / tiles;
  int64_t most = k / 128;
  int64_t split = std::max<int64_t>(1, std::min(want, most));
  int64_t chunk = ((k + split - 1) / split + BK - 1) / BK * BK;
  return int((k + chunk - 1) / chunk);
}

void gemm(hipStream_t s, const GemmArgs& g) {
  if (g.m <= 0 || g.n <= 0) return;
  if (g.k <= 0) bad("gemm with k = 0");
  int split = gemm_split_for(g.m, g.n, g.k);
  int64_t chunk = ((g.k + split - 1) / split + BK - 1) / BK * BK;
  split = int((g.k + chunk - 1) / chunk);
  float* ws = nullptr;
  if (split > 1) {
    if (!g.workspace || g.workspace_floats < int64_t(split) * g.m * g.n) bad("gemm split-K workspace too small");
    ws = g.workspace;
  }
  dim3 grid(unsigned((g.n + BN - 1) / BN), unsigned((g.m + BM - 1) / BM), unsigned(split));
  if (grid.y > 65535) bad("gemm M too large");
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, g.a, g.b, g.c, split > 1 ? nullptr : g.bias, g.m, g.n, g.k,
                       g.lda, g.ldb, g.ldc, chunk, ws);
  };
  if (!g.ta && !g.tb) launch(k_gemm<false, false>);
  else if (g.ta && !g.tb) launch(k_gemm<true, false>);
  else if (!g.ta && g.tb) launch(k_gemm<false, true>);
  else launch(k_gemm<true, true>);
  if (split > 1) {
    int64_t mn = g.m * g.n;
    hipLaunchKernelGGL(k_splitk_reduce, dim3(std::min<unsigned>(blocks_for(mn, 256), 8192)), dim3(256), 0, s, ws,
                       g.c, g.bias, g.m, g.n, g.ldc, split);
  }
}

// ---------------------------------------------------------------------------------------------
__global__ void k_transpose(const float* __restrict__ a, float* __restrict__ o, int64_t rows, int64_t cols) {
  __shared__ float t[32][33];
  int64_t c0 = int64_t(blockIdx.x) * 32, r0 = int64_t(blockIdx.y) * 32;
  for (int y = threadIdx.y; y < 32; y += 8) {
    int64_t r = r0 + y, c = c0 + threadIdx.x;
    if (r < rows && c < cols) t[y][threadIdx.x] = a[r * cols + c];
  }
  __syncthreads();
  for (int y = threadIdx.y; y < 32; y += 8) {
    int64_t c = c0 + y, r = r0 + threadIdx.x;
    if (r < rows && c < cols) o[c * rows + r] = t[threadIdx.x][y];
  }
}
void transpose(hipStream_t s, const float* a, float* o, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return;
  dim3 grid(unsigned((cols + 31) / 32), unsigned((rows + 31) / 32));
  if (grid.y > 65535) bad("transpose too tall");
  hipLaunchKernelGGL(k_transpose, grid, dim3(32, 8), 0, s, a, o, rows, cols);
}

// ---------------------------------------------------------------------------------------------
__global__ void k_add_rows(const float* __restrict__ x, const float* __restrict__ b, float* __restrict__ o,
                           int64_t n, int64_t h) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i < n; i += int64_t(gridDim.x) * blockDim.x) o[i] = x[i] + b[i % h];
}
void add_rows(hipStream_t s, const float* x, const float* b, float* o, int64_t rows, int64_t h) {
  int64_t n = rows * h;
  if (n <= 0) return;
  hipLaunchKernelGGL(k_add_rows, dim3(std::min<unsigned>(blocks_for(n, 256), 8192)), dim3(256), 0, s, x, b, o, n, h);
}

int64_t column_chunks(int64_t rows, int64_t h) {
  int64_t colblocks = (h + 255) / 256;
  int64_t chunks = (rows + 63) / 64;
  int64_t cap = std::max<int64_t>(1, 2048 / colblocks);
  return std::max<int64_t>(1, std::min(chunks, cap));
}

// Partial column sums over row chunks; with stats, of g * xhat (LayerNormGradGamma).
__global__ void k_column_partial(const float* __restrict__ x, const float* __restrict__ g,
                                 const float* __restrict__ stats, float* __restrict__ partial, int64_t rows, int64_t h,
                                 int64_t rows_per) {
  int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= h) return;
  int64_t r0 = int64_t(blockIdx.y) * rows_per, r1 = std::min(rows, r0 + rows_per);
  float acc = 0.0f;
  bool first = true;
  for (int64_t r = r0; r < r1; ++r) {
    float t;
    if (stats) {
      float xhat = (x[r * h + c] - stats[2 * r]) * stats[2 * r + 1];
      t = g[r * h + c] * xhat;
    } else {
      t = x[r * h + c];
    }
    acc = first ? t : acc + t;
    first = false;
  }
  partial[int64_t(blockIdx.y) * h + c] = acc;
}
__global__ void k_column_final(const float* __restrict__ partial, float* __restrict__ out, int64_t h, int64_t chunks) {
  int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= h) return;
  float acc = partial[c];
  for (int64_t z = 1; z < chunks; ++z) acc = acc + partial[z * h + c];
  out[c] = acc;
}
static void column_reduce(hipStream_t s, const float* x, const float* g, const float* stats, float* out, int64_t rows,
                          int64_t h, float* partial, int64_t partial_floats) {
  if (h <= 0) return;
  if (rows <= 0) { fill_zero(s, out, h * 4); return; }
  int64_t chunks = column_chunks(rows, h);
  if (partial_floats < chunks * h) bad("column reduction partial buffer too small");
  int64_t per = (rows + chunks - 1) / chunks;
  chunks = (rows + per - 1) / per;
  hipLaunchKernelGGL(k_column_partial, dim3(unsigned((h + 255) / 256), unsigned(chunks)), dim3(256), 0, s, x, g,
                     stats, partial, rows, h, per);
  hipLaunchKernelGGL(k_column_final, dim3(unsigned((h + 255) / 256)), dim3(256), 0, s, partial, out, h, chunks);
}
void column_sum(hipStream_t s, const float* x, float* out, int64_t rows, int64_t h, float* partial, int64_t pf) {
  column_reduce(s, x, nullptr, nullptr, out, rows, h, partial, pf);
}
void ln_grad_gamma(hipStream_t s, const float* x, const float* g, const float* stats, float* out, int64_t rows,
                   int64_t h, float* partial, int64_t pf) {
  column_reduce(s, x, g, stats, out, rows, h, partial, pf);
}

// ---------------------------------------------------------------------------------------------
// LayerNorm family: one wave per row, four rows per block.
__global__ void k_ln_stats(const float* __restrict__ x, float* __restrict__ stats, int64_t rows, int64_t h) {
  int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * h;
  float s = 0.0f;
  for (int64_t c = lane; c < h; c += 64) s += xr[c];
  float mean = wave_sum(s) / float(h);
  float q = 0.0f;
  for (int64_t c = lane; c < h; c += 64) { float d = xr[c] - mean; q = __builtin_fmaf(d, d, q); }
  float var = wave_sum(q) / float(h);
  if (lane == 0) { stats[2 * row] = mean; stats[2 * row + 1] = 1.0f / sqrtf(var + 1e-12f); }
}
void ln_stats(hipStream_t s, const float* x, float* stats, int64_t rows, int64_t h) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_ln_stats, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, stats, rows, h);
}

__global__ void k_layer_norm(const float* __restrict__ x, const float* __restrict__ gamma,
                             const float* __restrict__ beta, float* __restrict__ y, float* __restrict__ stats,
                             int64_t rows, int64_t h) {
  int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * h;
  float s = 0.0f;
  for (int64_t c = lane; c < h; c += 64) s += xr[c];
  float mean = wave_sum(s) / float(h);
  float q = 0.0f;
  for (int64_t c = lane; c < h; c += 64) { float d = xr[c] - mean; q = __builtin_fmaf(d, d, q); }
  float var = wave_sum(q) / float(h);
  float rstd = 1.0f / sqrtf(var + 1e-12f);
  for (int64_t c = lane; c < h; c += 64) y[row * h + c] = (xr[c] - mean) * rstd * gamma[c] + beta[c];
  if (stats && lane == 0) { stats[2 * row] = mean; stats[2 * row + 1] = rstd; }
}
void layer_norm(hipStream_t s, const float* x, const float* gamma, const float* beta, float* y, float* stats,
                int64_t rows, int64_t h) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_layer_norm, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, gamma, beta, y, stats, rows, h);
}

__global__ void k_ln_grad_x(const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ g,
                            const float* __restrict__ stats, float* __restrict__ dx, int64_t rows, int64_t h) {
  int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float mean = stats[2 * row], rstd = stats[2 * row + 1];
  const float* xr = x + row * h;
  const float* gr = g + row * h;
  float s1 = 0.0f, s2 = 0.0f;
  for (int64_t c = lane; c < h; c += 64) {
    float gx = gr[c] * gamma[c];
    float xhat = (xr[c] - mean) * rstd;
    s1 += gx;
    s2 = __builtin_fmaf(gx, xhat, s2);
  }
  const float width = float(h);
  const float mean_gx = wave_sum(s1) / width, mean_gx_xhat = wave_sum(s2) / width;
  for (int64_t c = lane; c < h; c += 64) {
    float gx = gr[c] * gamma[c];
    float xhat = (xr[c] - mean) * rstd;
    dx[row * h + c] = rstd * ((gx - mean_gx) - xhat * mean_gx_xhat);
  }
}
void ln_grad_x(hipStream_t s, const float* x, const float* gamma, const float* g, const float* stats, float* dx,
               int64_t rows, int64_t h) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_ln_grad_x, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, gamma, g, stats, dx, rows, h);
}

// ---------------------------------------------------------------------------------------------
__global__ void k_embedding(const float* __restrict__ table, const int32_t* __restrict__ ids, float* __restrict__ o,
                            int64_t n, int64_t rows, int64_t h) {
  int64_t r = blockIdx.x;
  int32_t id = ids[r];
  bool ok = id >= 0 && id < rows;
  for (int64_t c = threadIdx.x; c < h; c += blockDim.x) o[r * h + c] = ok ? table[int64_t(id) * h + c] : 0.0f;
}
void embedding(hipStream_t s, const float* table, const int32_t* ids, float* o, int64_t n, int64_t rows, int64_t h) {
  if (n <= 0) return;
  if (n > 2147483647) bad("embedding rows");
  hipLaunchKernelGGL(k_embedding, dim3(unsigned(n)), dim3(h >= 256 ? 256 : (h >= 128 ? 128 : 64)), 0, s, table, ids,
                     o, n, rows, h);
}

// Stable order of (id, k): one block bitonic-sorts the unique keys id << 32 | k in LDS.
__global__ __launch_bounds__(1024) void k_sort_ids(const int32_t* __restrict__ ids, uint64_t* __restrict__ keys,
                                                   int64_t n, int64_t pow2) {
  extern __shared__ uint64_t sk[];
  for (int64_t i = threadIdx.x; i < pow2; i += blockDim.x)
    sk[i] = i < n ? (uint64_t(uint32_t(ids[i])) << 32) | uint64_t(i) : ~uint64_t(0);
  __syncthreads();
  for (int64_t size = 2; size <= pow2; size <<= 1) {
    for (int64_t stride = size >> 1; stride > 0; stride >>= 1) {
      for (int64_t i = threadIdx.x; i < pow2; i += blockDim.x) {
        int64_t j = i ^ stride;
        if (j > i) {
          bool up = (i & size) == 0;
          uint64_t a = sk[i], b = sk[j];
          if ((a > b) == up) { sk[i] = b; sk[j] = a; }
        }
      }
      __syncthreads();
    }
  }
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) keys[i] = sk[i];
}

// One block per sorted position; the first position of each id sums its rows in ascending k.
__global__ void k_segment_sum(const uint64_t* __restrict__ keys, const float* __restrict__ g, float* __restrict__ out,
                              int64_t n, int64_t rows, int64_t h) {
  int64_t p = blockIdx.x;
  uint32_t id = uint32_t(keys[p] >> 32);
  if (p > 0 && uint32_t(keys[p - 1] >> 32) == id) return;
  if (int64_t(id) >= rows) return;
  for (int64_t c = threadIdx.x; c < h; c += blockDim.x) {
    float acc = 0.0f;
    for (int64_t q = p; q < n && uint32_t(keys[q] >> 32) == id; ++q) acc = acc + g[int64_t(uint32_t(keys[q])) * h + c];
    out[int64_t(id) * h + c] = acc;
  }
}

void embedding_grad(hipStream_t s, const int32_t* ids, const float* g, float* out, int64_t n, int64_t rows, int64_t h,
                    uint64_t* keys) {
  fill_zero(s, out, rows * h * 4);
  if (n <= 0) return;
  int64_t pow2 = 1;
  while (pow2 < n) pow2 <<= 1;
  if (pow2 * 8 > 160 * 1024) bad("embedding gradient over more than 16384 ids");
  hipLaunchKernelGGL(k_sort_ids, dim3(1), dim3(1024), size_t(pow2 * 8), s, ids, keys, n, pow2);
  hipLaunchKernelGGL(k_segment_sum, dim3(unsigned(n)), dim3(h >= 256 ? 256 : (h >= 128 ? 128 : 64)), 0, s, keys, g,
                     out, n, rows, h);
}

// ---------------------------------------------------------------------------------------------
__global__ void k_dropout(const float* __restrict__ x, float* __restrict__ o, int64_t n,
                          const int32_t* __restrict__ token, uint32_t seed_lo, uint32_t seed_hi, uint64_t threshold,
                          float scale) {
  const uint32_t id_lo = uint32_t(token[0]), id_hi = uint32_t(token[1]);
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    uint32_t w = philox_w0(uint32_t(i), 4u, id_lo, id_hi, seed_lo, seed_hi);
    o[i] = uint64_t(w) >= threshold ? x[i] * scale : 0.0f;
  }
}
void dropout(hipStream_t s, const float* x, float* o, int64_t n, const int32_t* token, uint64_t seed,
             uint64_t threshold, float scale) {
  if (n <= 0) return;
  if (n > (int64_t(1) << 32)) bad("dropout over more than 2^32 elements");
  hipLaunchKernelGGL(k_dropout, dim3(std::min<unsigned>(blocks_for(n, 256), 8192)), dim3(256), 0, s, x, o, n, token,
                     uint32_t(seed), uint32_t(seed >> 32), threshold, scale);
}

// ---------------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------------
// Cross-entropy. Row statistics once per logits tensor; the loss sums in f64 in one block.
__global__ void k_ce_stats(const float* __restrict__ x, float* __restrict__ stats, int64_t v) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const float* row = x + r * v;
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < v; c += blockDim.x) m = fmaxf(m, row[c]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float t = 0.0f;
  for (int64_t c = threadIdx.x; c < v; c += blockDim.x) t += expf(row[c] - m);
  t = wave_sum(t);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  if (threadIdx.x == 0) { stats[2 * r] = m; stats[2 * r + 1] = (red[0] + red[1]) + (red[2] + red[3]); }
}
void ce_stats(hipStream_t s, const float* logits, float* stats, int64_t rows, int64_t v) {
  if (rows <= 0) return;
  if (rows > 2147483647) bad("cross_entropy rows");
  hipLaunchKernelGGL(k_ce_stats, dim3(unsigned(rows)), dim3(256), 0, s, logits, stats, v);
}

__global__ __launch_bounds__(256) void k_ce_loss(const float* __restrict__ x, const int32_t* __restrict__ labels,
                                                 const float* __restrict__ w, const float* __restrict__ stats,
                                                 float* __restrict__ loss, float* __restrict__ den_out, int64_t rows,
                                                 int64_t v) {
  __shared__ double num_s[256], den_s[256];
  double num = 0.0, den = 0.0;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) {
    int32_t lab = labels[r];
    float xl = (lab >= 0 && lab < v) ? x[r * v + lab] : 0.0f;
    float l = stats[2 * r] + logf(stats[2 * r + 1]) - xl;
    num = __builtin_fma(double(w[r]), double(l), num);
    den += double(w[r]);
  }
  num_s[threadIdx.x] = num;
  den_s[threadIdx.x] = den;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (int(threadIdx.x) < o) {
      num_s[threadIdx.x] += num_s[threadIdx.x + o];
      den_s[threadIdx.x] += den_s[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    double n = num_s[0], d = den_s[0];
    loss[0] = d == 0.0 ? 0.0f : float(n / d);
    if (den_out) den_out[0] = float(d);
  }
}
void ce_loss(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* stats, float* loss,
             float* den, int64_t rows, int64_t v) {
  hipLaunchKernelGGL(k_ce_loss, dim3(1), dim3(256), 0, s, logits, labels, w, stats, loss, den, rows, v);
}

__global__ void k_ce_grad(const float* __restrict__ x, const int32_t* __restrict__ labels, const float* __restrict__ w,
                          const float* __restrict__ stats, const float* __restrict__ den, const float* __restrict__ g,
                          float* __restrict__ o, int64_t v) {
  const int64_t r = blockIdx.y;
  const float d = den[0];
  const float scale = d == 0.0f ? 0.0f : g[0] * w[r] / d;
  const float mx = stats[2 * r], total = stats[2 * r + 1];
  const int32_t lab = labels[r];
  for (int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; c < v; c += int64_t(gridDim.x) * blockDim.x) {
    float target = c == lab ? 1.0f : 0.0f;
    o[r * v + c] = d == 0.0f ? 0.0f : scale * (expf(x[r * v + c] - mx) / total - target);
  }
}
void ce_grad(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* stats,
             const float* den, const float* g, float* o, int64_t rows, int64_t v) {
  if (rows <= 0) return;
  if (rows > 65535) bad("cross_entropy gradient rows");
  dim3 grid(unsigned(std::min<int64_t>((v + 255) / 256, 64)), unsigned(rows));
  hipLaunchKernelGGL(k_ce_grad, grid, dim3(256), 0, s, logits, labels, w, stats, den, g, o, v);
}

// ---------------------------------------------------------------------------------------------
__global__ void k_softmax(const float* __restrict__ x, float* __restrict__ o, int64_t k) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const float* row = x + r * k;
  float m = -INFINITY;
  for (int64_t c = threadIdx.x; c < k; c += blockDim.x) m = fmaxf(m, row[c]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float t = 0.0f;
  for (int64_t c = threadIdx.x; c < k; c += blockDim.x) t += expf(row[c] - m);
  t = wave_sum(t);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  t = (red[0] + red[1]) + (red[2] + red[3]);
  for (int64_t c = threadIdx.x; c < k; c += blockDim.x) o[r * k + c] = expf(row[c] - m) / t;
}
void softmax(hipStream_t s, const float* x, float* o, int64_t rows, int64_t k) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_softmax, dim3(unsigned(rows)), dim3(256), 0, s, x, o, k);
}
__global__ void k_softmax_grad(const float* __restrict__ y, const float* __restrict__ g, float* __restrict__ o,
                               int64_t k) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  float t = 0.0f;
  for (int64_t c = threadIdx.x; c < k; c += blockDim.x) t = __builtin_fmaf(g[r * k + c], y[r * k + c], t);
  t = wave_sum(t);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  t = (red[0] + red[1]) + (red[2] + red[3]);
  for (int64_t c = threadIdx.x; c < k; c += blockDim.x) o[r * k + c] = y[r * k + c] * (g[r * k + c] - t);
}
void softmax_grad(hipStream_t s, const float* y, const float* g, float* o, int64_t rows, int64_t k) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_softmax_grad, dim3(unsigned(rows)), dim3(256), 0, s, y, g, o, k);
}

// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_reduce(const float* __restrict__ a, const float* __restrict__ b,
                                                 float* __restrict__ o, int64_t n, int mode) {
  __shared__ double red[1024];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    if (mode == 2) {
      double d = double(a[i]) - double(b[i]);
      acc = __builtin_fma(d, d, acc);
    } else {
      acc += double(a[i]);
    }
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 512; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) o[0] = float(mode == 0 ? red[0] : red[0] / double(n));
}
void reduce_sum(hipStream_t s, const float* a, float* o, int64_t n, bool mean) {
  hipLaunchKernelGGL(k_reduce, dim3(1), dim3(1024), 0, s, a, nullptr, o, n, mean ? 1 : 0);
}
void mse(hipStream_t s, const float* a, const float* b, float* o, int64_t n) {
  hipLaunchKernelGGL(k_reduce, dim3(1), dim3(1024), 0, s, a, b, o, n, 2);
}

// ---------------------------------------------------------------------------------------------
__global__ void k_adamw(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                        float* __restrict__ v, int64_t n, AdamWConsts k, const float* __restrict__ lr_t,
                        const float* __restrict__ c1, const float* __restrict__ c2) {
  const float lr = lr_t[0], b1 = c1[0], b2 = c2[0];
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float gi = g[i], pi = p[i];
    const float m2 = k.beta1 * m[i] + k.rest1 * gi;
    const float v2 = k.beta2 * v[i] + (k.rest2 * gi) * gi;
    const float dir = (m2 * b1) / (sqrtf(v2 * b2) + k.eps);
    const float step = dir + k.decay * pi;
    p[i] = pi - lr * step;
    m[i] = m2;
    v[i] = v2;
  }
}
void adamw(hipStream_t s, float* p, const float* g, float* m, float* v, int64_t n, AdamWConsts k, const float* lr_t,
           const float* c1, const float* c2) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_adamw, dim3(std::min<unsigned>(blocks_for(n, 256), 16384)), dim3(256), 0, s, p, g, m, v, n, k,
                     lr_t, c1, c2);
}

__global__ void k_sgd(float* __restrict__ p, const float* __restrict__ g, int64_t n, const float* __restrict__ lr) {
  const float r = lr[0];
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i < n; i += int64_t(gridDim.x) * blockDim.x) p[i] = p[i] - r * g[i];
}
void sgd(hipStream_t s, float* p, const float* g, int64_t n, const float* lr) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_sgd, dim3(std::min<unsigned>(blocks_for(n, 256), 16384)), dim3(256), 0, s, p, g, n, lr);
}

__global__ void k_record_loss(const float* __restrict__ loss, float* __restrict__ losses, uint32_t* __restrict__ counter,
                              uint32_t capacity) {
  uint32_t c = counter[0];
  if (c < capacity) losses[c] = loss[0];
  counter[0] = c + 1;
}
void prepare() {
  // Kernels whose dynamic LDS may exceed the 64 KiB default; set once, outside any capture.
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_sort_ids),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (e != hipSuccess) throw std::runtime_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
  prepare_attention();
}

void record_loss(hipStream_t s, const float* loss, float* losses, uint32_t* counter, uint32_t capacity) {
  hipLaunchKernelGGL(k_record_loss, dim3(1), dim3(1), 0, s, loss, losses, counter, capacity);
}

}  // namespace msx::hk
