// CDNA4 (gfx950) kernels of the training step other than the GEMMs (gemm.hip) and attention
// (attention.hip). Wave64 throughout; reductions use cross-lane shuffles within a wave and LDS
// across waves. Built with -ffp-contract=off: every f32 expression rounds as written, and fused
// multiply-adds appear only where a kernel calls __builtin_fmaf.
#include "kernels.h"
#include "device.h"

#include <algorithm>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

namespace msx::hk {


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
  MSX_LAUNCH(k_elementwise, dim3(grid), dim3(256), 0, s, op, a, b, o, n, int(as), int(bs));
}

__device__ __forceinline__ float ew_apply(int op, float x, float y) {
  switch (op) {
    case EW_ADD: return x + y;
    case EW_SUB: return x - y;
    case EW_MUL: return x * y;
    default: return x / y;
  }
}
__global__ void k_elementwise2(int op1, const float* __restrict__ a, const float* __restrict__ b, int op2,
                               const float* __restrict__ sc, int inner_left, float* __restrict__ o, int64_t n) {
  const float sv = sc[0];
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float t = ew_apply(op1, a[i], b[i]);
    o[i] = inner_left ? ew_apply(op2, t, sv) : ew_apply(op2, sv, t);
  }
}
void elementwise2(hipStream_t s, int op1, const float* a, const float* b, int op2, const float* sc, bool inner_left,
                  float* o, int64_t n) {
  if (n <= 0) return;
  if (op1 < EW_ADD || op1 > EW_DIV || op2 < EW_ADD || op2 > EW_DIV) bad("elementwise2 takes binary arithmetic");
  unsigned grid = std::min<unsigned>(blocks_for(n, 256), 8192);
  MSX_LAUNCH(k_elementwise2, dim3(grid), dim3(256), 0, s, op1, a, b, op2, sc, int(inner_left), o, n);
}

void copy(hipStream_t s, const float* a, float* o, int64_t n) { elementwise(s, EW_COPY, a, nullptr, o, n, false, false); }

__global__ void k_fill_from(const float* __restrict__ v, float* __restrict__ o, int64_t n) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  float x = v[0];
  for (; i < n; i += int64_t(gridDim.x) * blockDim.x) o[i] = x;
}
void fill_from(hipStream_t s, const float* v, float* o, int64_t n) {
  if (n <= 0) return;
  MSX_LAUNCH(k_fill_from, dim3(std::min<unsigned>(blocks_for(n, 256), 8192)), dim3(256), 0, s, v, o, n);
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
  MSX_LAUNCH(k_fill_zero, dim3(std::min<unsigned>(blocks_for(words / 4 + 1, 256), 8192)), dim3(256), 0, s,
                     static_cast<uint32_t*>(o), words);
}

__global__ __launch_bounds__(256) void k_to_f16_rows(const float* __restrict__ x, int64_t ldx, _Float16* __restrict__ y,
                                                     int64_t ldy, int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < n; e += int64_t(gridDim.x) * 256) {
    const int64_t r = e / cols, c = e - r * cols;
    y[r * ldy + c] = _Float16(x[r * ldx + c]);
  }
}
// Rows in 16-byte groups: block (x, y) converts groups 256 x + t of rows y, y + gridDim.y, ...
// When cols is not a multiple of 4 the last group of a row reaches into the row padding (both
// strides hold it): its columns past cols are written as zero, so a GEMM that reads the padded
// f16 row multiplies zeros there.
__global__ __launch_bounds__(256) void k_to_f16_rows4(const float* __restrict__ x, int64_t ldx, _Float16* __restrict__ y,
                                                      int64_t ldy, int64_t rows, int64_t cols) {
  const int64_t gq = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (4 * gq >= cols) return;
  const int live = int(cols - 4 * gq < 4 ? cols - 4 * gq : 4);
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const v4f v = *reinterpret_cast<const v4f*>(x + r * ldx + 4 * gq);
    v4h h;
#pragma unroll
    for (int u = 0; u < 4; ++u) h[u] = u < live ? _Float16(v[u]) : _Float16(0.0f);
    *reinterpret_cast<v4h*>(y + r * ldy + 4 * gq) = h;
  }
}
void to_f16_rows(hipStream_t s, const float* x, int64_t ldx, _Float16* y, int64_t ldy, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return;
  const int64_t groups = (cols + 3) / 4;
  if (4 * groups <= std::min(ldx, ldy) && ldx % 4 == 0 && ldy % 4 == 0 &&
      reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 8 == 0 &&
      groups <= int64_t(256) * 2147483647) {
    MSX_LAUNCH(k_to_f16_rows4, dim3(blocks_for(groups, 256), unsigned(std::min<int64_t>(rows, 65535))), dim3(256), 0, s, x,
               ldx, y, ldy, rows, cols);
    return;
  }
  MSX_LAUNCH(k_to_f16_rows, dim3(std::min<unsigned>(blocks_for(rows * cols, 256), 16384)), dim3(256), 0, s, x, ldx, y, ldy,
             rows, cols);
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
  MSX_LAUNCH(k_transpose, grid, dim3(32, 8), 0, s, a, o, rows, cols);
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
  MSX_LAUNCH(k_add_rows, dim3(std::min<unsigned>(blocks_for(n, 256), 8192)), dim3(256), 0, s, x, b, o, n, h);
}

// Partial column sums: block (x, y) adds columns 256 x + t over the rows of chunk y (rows ld
// floats apart), eight rows in flight a thread, into partial[y, c]; column_finalize adds the chunks.
__global__ __launch_bounds__(256) void k_column_partial(const float* __restrict__ x, float* __restrict__ partial,
                                                        int64_t rows, int64_t h, int64_t ld, int64_t rows_per) {
  const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t r0 = int64_t(blockIdx.y) * rows_per, r1 = std::min<int64_t>(rows, r0 + rows_per);
  if (c >= h) return;
  float s = 0.0f;
  for (int64_t r = r0; r < r1; r += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = x[(r + u < r1 ? r + u : r1 - 1) * ld + c];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (r + u < r1) s += t[u];
  }
  partial[int64_t(blockIdx.y) * h + c] = s;
}
// The same sums four columns a thread: block (x, y) takes column groups 64 x + (t mod 64) (four
// columns each, 16-byte loads) over the rows of chunk y, its four waves the rows r = r0 + w mod 4,
// four such rows in flight a wave; the waves' sums are added in wave order through LDS.
__global__ __launch_bounds__(256) void k_column_partial4(const float* __restrict__ x, float* __restrict__ partial,
                                                         int64_t rows, int64_t h, int64_t ld, int64_t rows_per) {
  __shared__ v4f part[3][64];
  const int g = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = (int64_t(blockIdx.x) * 64 + g) * 4;
  const int64_t r0 = int64_t(blockIdx.y) * rows_per, r1 = std::min<int64_t>(rows, r0 + rows_per);
  v4f s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (c < h) {
    for (int64_t r = r0 + w; r < r1; r += 16) {
      v4f t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t rr = r + 4 * u < r1 ? r + 4 * u : r;
        t[u] = *reinterpret_cast<const v4f*>(x + rr * ld + c);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (r + 4 * u < r1) s += t[u];
    }
  }
  if (w > 0) part[w - 1][g] = s;
  __syncthreads();
  if (w == 0 && c < h) {
    s += part[0][g];
    s += part[1][g];
    s += part[2][g];
    *reinterpret_cast<v4f*>(partial + int64_t(blockIdx.y) * h + c) = s;
  }
}
int64_t column_partial_chunks(int64_t rows, int64_t h) {
  const int64_t tiles = (h + 255) / 256;
  const int64_t want = std::max<int64_t>(1, 512 / tiles);  // about 512 blocks
  const int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(want, (rows + 15) / 16));
  // The chunks that rows of ceil(rows / chunks) each make: no empty last chunk.
  const int64_t per = (rows + chunks - 1) / chunks;
  return std::max<int64_t>(1, (rows + per - 1) / per);
}
void column_partial(hipStream_t s, const float* x, float* partial, int64_t rows, int64_t h, int64_t ld) {
  if (rows <= 0 || h <= 0) return;
  if (ld < 0) ld = h;
  if (ld < h) bad("column partial pitch below its width");
  const int64_t chunks = column_partial_chunks(rows, h);
  const int64_t per = (rows + chunks - 1) / chunks;
  if ((rows + per - 1) / per != chunks) bad("column partial chunking");
  if (h % 4 == 0 && ld % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(partial) % 16 == 0) {
    MSX_LAUNCH(k_column_partial4, dim3(unsigned((h + 255) / 256), unsigned(chunks)), dim3(256), 0, s, x, partial,
               rows, h, ld, per);
    return;
  }
  MSX_LAUNCH(k_column_partial, dim3(unsigned((h + 255) / 256), unsigned(chunks)), dim3(256), 0, s, x, partial,
                     rows, h, ld, per);
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
  MSX_LAUNCH(k_ln_stats, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, stats, rows, h);
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
  MSX_LAUNCH(k_layer_norm, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, gamma, beta, y, stats, rows, h);
}

// f16 copies a kernel writes beside two of its f32 outputs (mixed precision: GEMM operands).
struct Out16 { _Float16* a; _Float16* b; };

// LayerNorm with its neighbours in one pass, a wave a row: s = [a +] [dropout](b), y = LN(s) (the
// arithmetic of k_layer_norm), optionally yd = dropout(y); s, y, yd and the statistics each
// written when asked. The dropout keep rule is k_dropout's (Philox word 0 of the element index).
// With `gather`, output row r takes its a, b and input dropout from row gather[r] of those
// (an Embedding of the sum: element indices are the source rows'; an id out of range gives 0).
// With `ga` (`gb`), a (b) is itself an Embedding: row r of a is row ga.ids[r] of the table `a`, 0
// for an id outside [0, ga.rows) (k_embedding's rule), and the gathered rows are not written.
// o16 (mixed precision): f16 copies of y (a) and yd (b), written when non-null.
struct DropoutSpec { const int32_t* token; uint64_t threshold; float scale; };
struct RowGather { const int32_t* ids; int64_t rows; };
template <int CPL>
__global__ __launch_bounds__(256) void k_ln_fused(const float* __restrict__ a, const float* __restrict__ b,
                                                  DropoutSpec din, const float* __restrict__ gamma,
                                                  const float* __restrict__ beta, float* __restrict__ s_out,
                                                  float* __restrict__ y_out, float* __restrict__ stats,
                                                  DropoutSpec dout, float* __restrict__ yd_out, int64_t rows, int64_t h,
                                                  uint32_t seed_lo, uint32_t seed_hi, const int32_t* __restrict__ gather,
                                                  int64_t src_rows, RowGather ga, RowGather gb, Out16 o16) {
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t src = gather ? int64_t(gather[row]) : row;
  const bool src_ok = src >= 0 && src < src_rows;
  const uint32_t il = din.token ? uint32_t(din.token[0]) : 0u, ih = din.token ? uint32_t(din.token[1]) : 0u;
  const int64_t ra = ga.ids ? int64_t(ga.ids[row]) : src, rb = gb.ids ? int64_t(gb.ids[row]) : src;
  const bool a_ok = ga.ids ? ra >= 0 && ra < ga.rows : src_ok, b_ok = gb.ids ? rb >= 0 && rb < gb.rows : src_ok;
  float sv[CPL];
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t c = lane + 64 * j;
    sv[j] = 0.0f;
    if (c < h) {
      if (ga.ids || gb.ids) {
        const float v = b_ok ? b[rb * h + c] : 0.0f;
        sv[j] = a ? (a_ok ? a[ra * h + c] : 0.0f) + v : v;
      } else if (src_ok) {
        const int64_t i = src * h + c;
        float v = b[i];
        if (din.token) v = uint64_t(philox_w0(uint32_t(i), 4u, il, ih, seed_lo, seed_hi)) >= din.threshold ? v * din.scale : 0.0f;
        sv[j] = a ? a[i] + v : v;
      }
      sum += sv[j];
    }
  }
  const float mean = wave_sum(sum) / float(h);
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if (lane + 64 * j < h) { const float d = sv[j] - mean; q = __builtin_fmaf(d, d, q); }
  const float var = wave_sum(q) / float(h);
  const float rstd = 1.0f / sqrtf(var + 1e-12f);
  const uint32_t ol = dout.token ? uint32_t(dout.token[0]) : 0u, oh = dout.token ? uint32_t(dout.token[1]) : 0u;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t c = lane + 64 * j;
    if (c >= h) continue;
    const int64_t i = row * h + c;
    const float y = (sv[j] - mean) * rstd * gamma[c] + beta[c];
    if (s_out) s_out[i] = sv[j];
    if (y_out) y_out[i] = y;
    if (o16.a) o16.a[i] = _Float16(y);
    if (yd_out || o16.b) {
      const float yd =
          uint64_t(philox_w0(uint32_t(i), 4u, ol, oh, seed_lo, seed_hi)) >= dout.threshold ? y * dout.scale : 0.0f;
      if (yd_out) yd_out[i] = yd;
      if (o16.b) o16.b[i] = _Float16(yd);
    }
  }
  if (stats && lane == 0) { stats[2 * row] = mean; stats[2 * row + 1] = rstd; }
}
// The same without row gathers or gathered operands, for rows of 256 VPL floats: lane l of a row's
// wave takes the float4 groups l + 64 v (v < VPL), so every access is 16 bytes.
template <int VPL>
__global__ __launch_bounds__(256) void k_ln_fused4(const float* __restrict__ a, const float* __restrict__ b,
                                                   DropoutSpec din, const float* __restrict__ gamma,
                                                   const float* __restrict__ beta, float* __restrict__ s_out,
                                                   float* __restrict__ y_out, float* __restrict__ stats,
                                                   DropoutSpec dout, float* __restrict__ yd_out, int64_t rows,
                                                   uint32_t seed_lo, uint32_t seed_hi, Out16 o16,
                                                   const _Float16* __restrict__ b16) {
  constexpr int64_t h = 256 * VPL;
  typedef _Float16 h4_ __attribute__((ext_vector_type(4)));
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint32_t il = din.token ? uint32_t(din.token[0]) : 0u, ih = din.token ? uint32_t(din.token[1]) : 0u;
  float4 sv[VPL];
  float sum = 0.0f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int64_t i = row * h + 4 * (lane + 64 * v);
    float4 x;
    if (b16) {
      const h4_ hb = *reinterpret_cast<const h4_*>(b16 + i);
      x = make_float4(float(hb[0]), float(hb[1]), float(hb[2]), float(hb[3]));
    } else {
      x = *reinterpret_cast<const float4*>(b + i);
    }
    if (din.token) {
      float* xs = reinterpret_cast<float*>(&x);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        xs[u] = uint64_t(philox_w0(uint32_t(i + u), 4u, il, ih, seed_lo, seed_hi)) >= din.threshold ? xs[u] * din.scale : 0.0f;
    }
    if (a) {
      const float4 y = *reinterpret_cast<const float4*>(a + i);
      x = make_float4(y.x + x.x, y.y + x.y, y.z + x.z, y.w + x.w);
    }
    sv[v] = x;
    sum += ((x.x + x.y) + x.z) + x.w;
  }
  const float mean = wave_sum(sum) / float(h);
  float q = 0.0f;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const float* xs = reinterpret_cast<const float*>(&sv[v]);
#pragma unroll
    for (int u = 0; u < 4; ++u) { const float d = xs[u] - mean; q = __builtin_fmaf(d, d, q); }
  }
  const float var = wave_sum(q) / float(h);
  const float rstd = 1.0f / sqrtf(var + 1e-12f);
  const uint32_t ol = dout.token ? uint32_t(dout.token[0]) : 0u, oh = dout.token ? uint32_t(dout.token[1]) : 0u;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int64_t c = 4 * (lane + 64 * v), i = row * h + c;
    const float4 g = *reinterpret_cast<const float4*>(gamma + c), be = *reinterpret_cast<const float4*>(beta + c);
    const float* xs = reinterpret_cast<const float*>(&sv[v]);
    const float* gs = reinterpret_cast<const float*>(&g);
    const float* bs = reinterpret_cast<const float*>(&be);
    float y[4], yd[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      y[u] = (xs[u] - mean) * rstd * gs[u] + bs[u];
      yd[u] = (yd_out || o16.b) && uint64_t(philox_w0(uint32_t(i + u), 4u, ol, oh, seed_lo, seed_hi)) >= dout.threshold
                  ? y[u] * dout.scale
                  : 0.0f;
    }
    if (s_out) *reinterpret_cast<float4*>(s_out + i) = sv[v];
    if (y_out) *reinterpret_cast<float4*>(y_out + i) = make_float4(y[0], y[1], y[2], y[3]);
    if (o16.a) *reinterpret_cast<h4_*>(o16.a + i) = h4_{_Float16(y[0]), _Float16(y[1]), _Float16(y[2]), _Float16(y[3])};
    if (yd_out) *reinterpret_cast<float4*>(yd_out + i) = make_float4(yd[0], yd[1], yd[2], yd[3]);
    if (o16.b) *reinterpret_cast<h4_*>(o16.b + i) = h4_{_Float16(yd[0]), _Float16(yd[1]), _Float16(yd[2]), _Float16(yd[3])};
  }
  if (stats && lane == 0) { stats[2 * row] = mean; stats[2 * row + 1] = rstd; }
}

void ln_fused(hipStream_t s, const float* a, const float* b, const int32_t* din_token, uint64_t din_threshold,
              float din_scale, const float* gamma, const float* beta, float* s_out, float* y_out, float* stats,
              const int32_t* dout_token, uint64_t dout_threshold, float dout_scale, float* yd_out, int64_t rows,
              int64_t h, uint64_t seed, const int32_t* gather, int64_t src_rows, const int32_t* a_ids, int64_t a_rows,
              const int32_t* b_ids, int64_t b_rows, _Float16* y16, _Float16* yd16, const _Float16* b16) {
  if (rows <= 0 || h <= 0) return;
  if (!b && !b16) bad("fused LayerNorm without its second operand");
  if (!gather) src_rows = rows;
  if ((a_ids || b_ids) && (gather || din_token)) bad("fused LayerNorm: gathered operands with a row gather or an input dropout");
  if (h > 1024) bad("fused LayerNorm rows wider than 1024");
  if (rows * h > (int64_t(1) << 32)) bad("fused LayerNorm over more than 2^32 elements");
  const DropoutSpec din{din_token, din_threshold, din_scale}, dout{dout_token, dout_threshold, dout_scale};
  auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!gather && !a_ids && !b_ids && h % 256 == 0 && h <= 1024 && al16(a) && al16(b) && al16(gamma) && al16(beta) &&
      al16(s_out) && al16(y_out) && al16(yd_out) && reinterpret_cast<uintptr_t>(y16) % 8 == 0 &&
      reinterpret_cast<uintptr_t>(yd16) % 8 == 0 && reinterpret_cast<uintptr_t>(b16) % 8 == 0) {
#define MSX_LNF4(V) MSX_LAUNCH(k_ln_fused4<V>, dim3(blocks_for(rows, 4)), dim3(256), 0, s, a, b, din, gamma, beta, s_out, \
                               y_out, stats, dout, yd_out, rows, uint32_t(seed), uint32_t(seed >> 32), Out16{y16, yd16}, b16)
    if (h == 256) MSX_LNF4(1);
    else if (h == 512) MSX_LNF4(2);
    else if (h == 768) MSX_LNF4(3);
    else MSX_LNF4(4);
#undef MSX_LNF4
    return;
  }
  if (b16) bad("fused LayerNorm: an f16 second operand needs rows of 256..1024 floats without gathers");
  const int cpl = int((h + 63) / 64);
#define MSX_LNF(C) MSX_LAUNCH(k_ln_fused<C>, dim3(blocks_for(rows, 4)), dim3(256), 0, s, a, b, din, gamma, beta, s_out, y_out, \
                              stats, dout, yd_out, rows, h, uint32_t(seed), uint32_t(seed >> 32), gather, src_rows, \
                              RowGather{a_ids, a_rows}, RowGather{b_ids, b_rows}, Out16{y16, yd16})
  if (cpl <= 1) MSX_LNF(1);
  else if (cpl <= 2) MSX_LNF(2);
  else if (cpl <= 4) MSX_LNF(4);
  else if (cpl <= 8) MSX_LNF(8);
  else MSX_LNF(16);
#undef MSX_LNF
}

// The LayerNorm backward of one input in one pass: dx (LayerNormGradX) and, per block of rows, the
// partial column sums of g * xhat (LayerNormGradGamma) and of g (the beta gradient, SumRows), to
// partial[block] = [gamma sums (h), beta sums (h)]; column_finalize adds the blocks' partials. A
// wave takes a row at a time, lane l holding columns l + 64 j.
template <int CPL>
__global__ __launch_bounds__(256) void k_ln_backward(const float* __restrict__ x, const float* __restrict__ gamma,
                                                     const float* __restrict__ g, const float* __restrict__ stats,
                                                     float* __restrict__ dx, float* __restrict__ partial, int64_t rows,
                                                     int64_t h, int64_t rows_per, float* __restrict__ dx2, int post,
                                                     const float* __restrict__ pre, DropoutSpec dsp, uint32_t seed_lo,
                                                     uint32_t seed_hi, Out16 o16) {
  extern __shared__ float red[];  // [4 waves][2 h]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r0 = int64_t(blockIdx.x) * rows_per, r1 = std::min<int64_t>(rows, r0 + rows_per);
  float gm[CPL], pg[CPL], pb[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t c = lane + 64 * j;
    gm[j] = c < h && gamma ? gamma[c] : 0.0f;
    pg[j] = 0.0f;
    pb[j] = 0.0f;
  }
  const float width = float(h);
  for (int64_t row = r0 + wave; row < r1; row += 4) {
    const float mean = stats[2 * row], rstd = stats[2 * row + 1];
    float xv[CPL], gv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int64_t c = lane + 64 * j;
      xv[j] = c < h ? x[row * h + c] : 0.0f;
      gv[j] = c < h ? g[row * h + c] : 0.0f;
    }
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const float xhat = (xv[j] - mean) * rstd;
      const float gx = gv[j] * gm[j];
      s1 += gx;
      s2 = __builtin_fmaf(gx, xhat, s2);
      pg[j] += gv[j] * xhat;
      pb[j] += gv[j];
    }
    if (dx || dx2 || o16.a || o16.b) {
      const float mean_gx = wave_sum(s1) / width, mean_gx_xhat = wave_sum(s2) / width;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int64_t c = lane + 64 * j;
        const float xhat = (xv[j] - mean) * rstd;
        const float gx = gv[j] * gm[j];
        if (c < h) {
          const int64_t i = row * h + c;
          const float v = rstd * ((gx - mean_gx) - xhat * mean_gx_xhat);
          if (dx) dx[i] = v;
          if (o16.a) o16.a[i] = _Float16(v);
          if (dx2 || o16.b) {
            float w;
            if (post == LNB_DROPOUT)
              w = uint64_t(philox_w0(uint32_t(i), 4u, uint32_t(dsp.token[0]), uint32_t(dsp.token[1]), seed_lo, seed_hi)) >=
                          dsp.threshold
                      ? v * dsp.scale
                      : 0.0f;
            else if (post == LNB_GELU_GRAD)
              w = d_gelu_grad(pre[i], v);
            else
              w = pre[i] > 0.0f ? v : 0.0f;
            if (dx2) dx2[i] = w;
            if (o16.b) o16.b[i] = _Float16(w);
          }
        }
      }
    }
  }
  if (!partial) return;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int64_t c = lane + 64 * j;
    if (c < h) {
      red[wave * 2 * h + c] = pg[j];
      red[wave * 2 * h + h + c] = pb[j];
    }
  }
  __syncthreads();
  for (int64_t c = threadIdx.x; c < 2 * h; c += 256)
    partial[int64_t(blockIdx.x) * 2 * h + c] = ((red[c] + red[2 * h + c]) + red[4 * h + c]) + red[6 * h + c];
}

int64_t ln_backward_blocks(int64_t rows, int64_t h) {
  (void)h;
  // One row a wave (4 rows a block) up to 1024 blocks (4 a CU), then more rows a block: each wave
  // walks its rows one after another, so short walks keep the pass off the load latency (BERT-tiny's
  // 4096 rows: 1024 blocks take 18 us a step less than 256 blocks of 16 rows); at BERT-base's 16384
  // rows, 1024 blocks take 1.2 ms a step against 2.0 ms for 256, and more blocks cost more in the
  // finalize of their partials than they gain.
  return std::max<int64_t>(1, std::min<int64_t>((rows + 3) / 4, 1024));
}
void ln_backward(hipStream_t s, const float* x, const float* gamma, const float* g, const float* stats, float* dx,
                 float* partial, int64_t rows, int64_t h, float* dx2, int post, const float* pre,
                 const int32_t* token, uint64_t threshold, float scale, uint64_t seed, _Float16* dx16,
                 _Float16* dx2_16) {
  if ((dx2 || dx2_16) && post == LNB_DROPOUT && !token) bad("LayerNorm backward dropout without its token");
  if ((dx2 || dx2_16) && post != LNB_DROPOUT && !pre) bad("LayerNorm backward activation gradient without its input");
  const DropoutSpec dsp{token, threshold, scale};
  if (rows <= 0 || h <= 0) return;
  if (h > 1024) bad("LayerNorm backward rows wider than 1024");
  const int64_t blocks = ln_backward_blocks(rows, h);
  const int64_t per = (rows + blocks - 1) / blocks;
  const size_t lds = size_t(8 * h) * 4;
  const int cpl = int((h + 63) / 64);
#define MSX_LNB(C) MSX_LAUNCH(k_ln_backward<C>, dim3(unsigned(blocks)), dim3(256), lds, s, x, gamma, g, stats, dx, \
                              partial, rows, h, per, dx2, post, pre, dsp, uint32_t(seed), uint32_t(seed >> 32), \
                              Out16{dx16, dx2_16})
  // 12 columns a lane for H = 768 (BERT-base): 16 would hold a third of the registers idle and
  // cost a wave of occupancy on a bandwidth-bound pass.
  if (cpl <= 1) MSX_LNB(1);
  else if (cpl <= 2) MSX_LNB(2);
  else if (cpl <= 4) MSX_LNB(4);
  else if (cpl <= 8) MSX_LNB(8);
  else if (cpl <= 12) MSX_LNB(12);
  else MSX_LNB(16);
#undef MSX_LNB
}

// Column sums of block partials for several reductions in one launch. Job j owns blocks [first,
// first + ceil(width / cols)), cols = 256 / parts: a block takes cols columns, and its `parts`
// thread groups each add a contiguous share of a column's chunks in ascending order (8 loads in
// flight); the shares' sums are then added in share order. The order is fixed, so the result does
// not depend on timing. A job of many chunks (a LayerNorm's gamma and beta partials: few columns)
// takes up to 32 parts (a share of at least 32 chunks each) so that no thread walks all of them;
// one of few chunks takes 1. The sum goes to out_lo[c] (c < split) or out_hi[c - split] (a null
// output is skipped).
// A job of few chunks whose columns, split point and pointers allow it (parts 0) takes four
// columns a thread as 16-byte vectors, 1024 a block, each column still summed in ascending chunk
// order: BERT-base's split-K weight gradients otherwise take hundreds of thousands of small
// blocks a step.
int finalize_parts(int chunks) { return std::min(32, std::max(1, chunks / 32)); }
int finalize_parts(const ColumnJob& J) {
  const int parts = finalize_parts(J.chunks);
  auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  const bool vec = parts == 1 && J.width % 4 == 0 && J.split % 4 == 0 && a16(J.partial) && a16(J.out_lo) &&
                   a16(J.out_hi);
  return vec ? 0 : parts;
}
int finalize_blocks(const ColumnJob& J) {
  const int cols = J.parts == 0 ? 1024 : 256 / J.parts;
  return int((J.width + cols - 1) / cols);
}
// The vector form: thread t of block lb sums columns 4 (256 lb + t) .. + 3; returns false when
// past the job's width. *out is where the four sums went (null for a skipped output).
__device__ __forceinline__ bool finalize_vec(const ColumnJob& J, int lb, v4f& sum, float*& out) {
  const int64_t c = (int64_t(lb) * 256 + threadIdx.x) * 4;
  if (c >= J.width) return false;
  const v4f* src = reinterpret_cast<const v4f*>(J.partial + c);
  const int64_t stride = J.width / 4;
  for (int z0 = 0; z0 < J.chunks; z0 += 8) {
    v4f t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = src[int64_t(z0 + u < J.chunks ? z0 + u : J.chunks - 1) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (z0 + u < J.chunks) sum = (z0 + u == 0) ? t[u] : sum + t[u];
  }
  out = c < J.split ? (J.out_lo ? J.out_lo + c : nullptr) : (J.out_hi ? J.out_hi + (c - J.split) : nullptr);
  if (out) *reinterpret_cast<v4f*>(out) = sum;
  return true;
}
__global__ __launch_bounds__(256) void k_column_finalize(ColumnJobs jobs) {
  __shared__ float red[256];
  int j = 0;
  while (j + 1 < jobs.count && int(blockIdx.x) >= jobs.job[j + 1].first) ++j;
  const ColumnJob& J = jobs.job[j];
  if (J.parts == 0) {
    v4f sum{0.0f, 0.0f, 0.0f, 0.0f};
    float* out = nullptr;
    finalize_vec(J, int(blockIdx.x) - J.first, sum, out);
    return;
  }
  const int parts = J.parts, cols = 256 / parts;
  const int lc = threadIdx.x % cols, part = threadIdx.x / cols;
  const int64_t c = int64_t(int(blockIdx.x) - J.first) * cols + lc;
  const int per = (J.chunks + parts - 1) / parts;
  const int z_beg = part * per, z_end = min(J.chunks, z_beg + per);
  float s = 0.0f;
  if (c < J.width) {
    for (int z0 = z_beg; z0 < z_end; z0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int z = z0 + u < z_end ? z0 + u : z_end - 1;
        t[u] = J.partial[int64_t(z) * J.width + c];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (z0 + u < z_end) s = (z0 + u == z_beg) ? t[u] : s + t[u];
    }
  }
  if (parts > 1) {
    red[threadIdx.x] = s;
    __syncthreads();
    if (part != 0) return;
    // Shares past the last chunk hold nothing and are not added.
    for (int q = 1; q < parts && q * per < J.chunks; ++q) s += red[q * cols + lc];
  }
  if (c >= J.width) return;
  if (c < J.split) {
    if (J.out_lo) J.out_lo[c] = s;
  } else if (J.out_hi) {
    J.out_hi[c - J.split] = s;
  }
}
void column_finalize(hipStream_t s, const ColumnJob* jobs, int count) {
  for (int base = 0; base < count; base += kColumnJobs) {
    ColumnJobs b{};
    int blocks = 0;
    b.count = std::min(kColumnJobs, count - base);
    for (int j = 0; j < b.count; ++j) {
      b.job[j] = jobs[base + j];
      if (b.job[j].chunks <= 0 || b.job[j].width <= 0) bad("column finalize job without partials");
      b.job[j].first = blocks;
      b.job[j].parts = finalize_parts(b.job[j]);
      blocks += finalize_blocks(b.job[j]);
    }
    MSX_LAUNCH(k_column_finalize, dim3(unsigned(blocks)), dim3(256), 0, s, b);
  }
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
  MSX_LAUNCH(k_embedding, dim3(unsigned(n)), dim3(h >= 256 ? 256 : (h >= 128 ? 128 : 64)), 0, s, table, ids,
                     o, n, rows, h);
}

// EmbeddingGrad in one launch, deterministic, with no float atomics, optionally added to `addend`
// (out = addend + EmbeddingGrad, elementwise). Blocks [0, n) take a position each: the block of an
// id's first position collects the id's positions in ascending k (wave ballots over the ids) and
// adds the rows g[k] in that order from +0, one f32 rounding per add: the reference's order
// (interpreter.rs:931-941), bit for bit. The rows come through LDS a chunk of `ch` at a time, with
// kDepth chunks' loads in flight in registers ahead of the adds. Blocks from n on write the rows
// of their stripe of the table that no id names.
constexpr int kEgThreads = 256, kDepth = 4, kEgVec = 4;  // float4 loads a thread per chunk
constexpr int kEgIds = 16;                                // ids a thread a round

// One chunk of rows in registers: kEgVec float4 a thread.
struct EgChunk { float4 v[kEgVec]; };
// Chunk q's loads: float4 e = tid + u * 256 of its cnt * h4; the tail (and a chunk past the end)
// reads an in-range element that is never stored.
__device__ __forceinline__ EgChunk eg_issue(const float* __restrict__ g, const int32_t* list, int64_t h, int h4, int q,
                                            int ch, int total, int tid) {
  const int q0 = q * ch;
  const int cnt = q0 < total ? min(ch, total - q0) : 1;
  const int tot = cnt * h4;
  const int base = q0 < total ? q0 : 0;
  EgChunk r;
#pragma unroll
  for (int u = 0; u < kEgVec; ++u) {
    int e = tid + u * kEgThreads;
    e = e < tot ? e : tot - 1;
    const int rr = e / h4;
    r.v[u] = reinterpret_cast<const float4*>(g + int64_t(list[base + rr]) * h)[e - rr * h4];
  }
  return r;
}
// Stores chunk q from r into LDS, refills r with chunk q + kDepth, and adds the chunk's rows in order.
__device__ __forceinline__ void eg_step(const float* __restrict__ g, const int32_t* list, float* stage, int64_t h,
                                        int h4, int q, int ch, int total, int chunks, int tid, EgChunk& r,
                                        float& a0, float& a1, float& a2, float& a3) {
  if (q >= chunks) return;  // uniform across the block
  const int cnt = min(ch, total - q * ch), tot = cnt * h4;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kEgVec; ++u) {
    const int e = tid + u * kEgThreads;
    if (e < tot) reinterpret_cast<float4*>(stage)[e] = r.v[u];
  }
  __syncthreads();
  if (q + kDepth < chunks) r = eg_issue(g, list, h, h4, q + kDepth, ch, total, tid);
  const int64_t c0 = tid, c1 = tid + kEgThreads, c2 = tid + 2 * kEgThreads, c3 = tid + 3 * kEgThreads;
  if (c0 < h) for (int rr = 0; rr < cnt; ++rr) a0 = a0 + stage[int64_t(rr) * h + c0];
  if (c1 < h) for (int rr = 0; rr < cnt; ++rr) a1 = a1 + stage[int64_t(rr) * h + c1];
  if (c2 < h) for (int rr = 0; rr < cnt; ++rr) a2 = a2 + stage[int64_t(rr) * h + c2];
  if (c3 < h) for (int rr = 0; rr < cnt; ++rr) a3 = a3 + stage[int64_t(rr) * h + c3];
}

__global__ __launch_bounds__(kEgThreads) void k_embedding_grad(const int32_t* __restrict__ ids, const float* __restrict__ g,
                                                               const float* __restrict__ addend, float* __restrict__ out,
                                                               int n, int64_t rows, int64_t h, int64_t stripe, int ch,
                                                               bool vec) {
  extern __shared__ int32_t eg_lds[];
  int32_t* list = eg_lds;                                     // [n] the positions of this block's id
  float* stage = reinterpret_cast<float*>(list + n);          // [ch * h]
  __shared__ uint32_t mask;
  __shared__ int cnt[kEgIds][kEgThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (int64_t(blockIdx.x) >= n) {
    // A stripe block: the rows of its stripe (at most 32) that no id names are zero, or the
    // addend's row + 0.
    const int64_t z0 = (int64_t(blockIdx.x) - n) * stripe, z1 = std::min<int64_t>(rows, z0 + stripe);
    if (tid == 0) mask = 0;
    __syncthreads();
    for (int base = 0; base < n; base += kEgThreads * kEgIds) {
      int32_t t[kEgIds];
#pragma unroll
      for (int u = 0; u < kEgIds; ++u) {
        const int j = base + tid + u * kEgThreads;
        t[u] = ids[j < n ? j : n - 1];
      }
      uint32_t bits = 0;
#pragma unroll
      for (int u = 0; u < kEgIds; ++u) bits |= (t[u] >= z0 && t[u] < z1) ? 1u << uint32_t(t[u] - z0) : 0u;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) bits |= __shfl_xor(bits, d, 64);
      if (lane == 0 && bits) atomicOr(&mask, bits);
    }
    __syncthreads();
    const uint32_t m = mask;
    if (vec) {
      // float4 cells of the stripe, four a thread in flight.
      const int h4 = int(h >> 2), cells = int(z1 - z0) * h4;
      float4* o4 = reinterpret_cast<float4*>(out + z0 * h);
      const float4* a4 = addend ? reinterpret_cast<const float4*>(addend + z0 * h) : nullptr;
      for (int e0 = tid; e0 < cells; e0 += kEgThreads * 4) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = e0 + u * kEgThreads;
          v[u] = a4 ? a4[e < cells ? e : cells - 1] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int e = e0 + u * kEgThreads;
          if (e < cells && !((m >> uint32_t(e / h4)) & 1u))
            o4[e] = make_float4(v[u].x + 0.0f, v[u].y + 0.0f, v[u].z + 0.0f, v[u].w + 0.0f);
        }
      }
    } else {
      const int64_t cells = (z1 - z0) * h;
      for (int64_t e = tid; e < cells; e += kEgThreads) {
        const int64_t r = z0 + e / h;
        if (!((m >> uint32_t(r - z0)) & 1u)) out[z0 * h + e] = addend ? addend[z0 * h + e] + 0.0f : 0.0f;
      }
    }
    return;
  }
  const int b = int(blockIdx.x);
  const int32_t id = ids[b];
  if (id < 0 || int64_t(id) >= rows) return;
  // One pass over the ids, kEgIds a thread a round with all loads in flight: an earlier position
  // holding the id ends the block (only the first position goes on), and ballots in position order
  // collect the positions k >= b holding it.
  int total = 0;
  const uint64_t below = (uint64_t(1) << lane) - 1;
  for (int base = 0; base < n; base += kEgThreads * kEgIds) {
    int32_t t[kEgIds];
#pragma unroll
    for (int u = 0; u < kEgIds; ++u) {
      const int j = base + tid + u * kEgThreads;
      t[u] = ids[j < n ? j : n - 1];
    }
    int dup = 0;
#pragma unroll
    for (int u = 0; u < kEgIds; ++u) {
      const int j = base + tid + u * kEgThreads;
      dup |= (j < b && t[u] == id) ? 1 : 0;
    }
    if (__syncthreads_or(dup)) return;
    if (base + kEgThreads * kEgIds <= b) continue;
#pragma unroll
    for (int u = 0; u < kEgIds; ++u) {
      const int j = base + tid + u * kEgThreads;
      const uint64_t bal = __ballot(j < n && j >= b && t[u] == id);
      if (lane == 0) cnt[u][wave] = __popcll(bal);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kEgIds; ++u) {
      const int j = base + tid + u * kEgThreads;
      const bool hit = j < n && j >= b && t[u] == id;
      const uint64_t bal = __ballot(hit);
      int off = total;
      for (int w = 0; w < wave; ++w) off += cnt[u][w];
      if (hit) list[off + __popcll(bal & below)] = j;
#pragma unroll
      for (int w = 0; w < kEgThreads / 64; ++w) total += cnt[u][w];
    }
    __syncthreads();
  }
  // Thread tid adds columns tid, tid + 256, tid + 512, tid + 768 (h <= 1024).
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  if (vec) {
    const int h4 = int(h >> 2);
    const int chunks = (total + ch - 1) / ch;
    EgChunk r0 = eg_issue(g, list, h, h4, 0, ch, total, tid);
    EgChunk r1 = eg_issue(g, list, h, h4, 1, ch, total, tid);
    EgChunk r2 = eg_issue(g, list, h, h4, 2, ch, total, tid);
    EgChunk r3 = eg_issue(g, list, h, h4, 3, ch, total, tid);
    for (int q = 0; q < chunks; q += kDepth) {
      eg_step(g, list, stage, h, h4, q, ch, total, chunks, tid, r0, a0, a1, a2, a3);
      eg_step(g, list, stage, h, h4, q + 1, ch, total, chunks, tid, r1, a0, a1, a2, a3);
      eg_step(g, list, stage, h, h4, q + 2, ch, total, chunks, tid, r2, a0, a1, a2, a3);
      eg_step(g, list, stage, h, h4, q + 3, ch, total, chunks, tid, r3, a0, a1, a2, a3);
    }
  } else {
    for (int q0 = 0; q0 < total; q0 += ch) {
      const int cnt = min(ch, total - q0);
      __syncthreads();
      for (int64_t e = tid; e < int64_t(cnt) * h; e += kEgThreads) {
        const int r = int(e / h);
        stage[e] = g[int64_t(list[q0 + r]) * h + (e - int64_t(r) * h)];
      }
      __syncthreads();
      const int64_t c0 = tid, c1 = tid + kEgThreads, c2 = tid + 2 * kEgThreads, c3 = tid + 3 * kEgThreads;
      if (c0 < h) for (int rr = 0; rr < cnt; ++rr) a0 = a0 + stage[int64_t(rr) * h + c0];
      if (c1 < h) for (int rr = 0; rr < cnt; ++rr) a1 = a1 + stage[int64_t(rr) * h + c1];
      if (c2 < h) for (int rr = 0; rr < cnt; ++rr) a2 = a2 + stage[int64_t(rr) * h + c2];
      if (c3 < h) for (int rr = 0; rr < cnt; ++rr) a3 = a3 + stage[int64_t(rr) * h + c3];
    }
  }
  float* o = out + int64_t(id) * h;
  const float* ad = addend ? addend + int64_t(id) * h : nullptr;
  if (tid < h) o[tid] = ad ? ad[tid] + a0 : a0;
  if (tid + kEgThreads < h) o[tid + kEgThreads] = ad ? ad[tid + kEgThreads] + a1 : a1;
  if (tid + 2 * kEgThreads < h) o[tid + 2 * kEgThreads] = ad ? ad[tid + 2 * kEgThreads] + a2 : a2;
  if (tid + 3 * kEgThreads < h) o[tid + 3 * kEgThreads] = ad ? ad[tid + 3 * kEgThreads] + a3 : a3;
}

void embedding_grad(hipStream_t s, const int32_t* ids, const float* g, float* out, int64_t n, int64_t rows, int64_t h,
                    const float* addend) {
  if (n > 16384) bad("embedding gradient over more than 16384 ids");
  if (h > 1024) bad("embedding gradient rows wider than 1024");
  if (rows <= 0 || h <= 0) return;
  if (n <= 0 && !addend) { fill_zero(s, out, rows * h * 4); return; }
  const int64_t stripes = (rows + 31) / 32, stripe = (rows + stripes - 1) / stripes;  // stripe <= 32 rows
  const int64_t blocks = std::max<int64_t>(n, 0) + stripes;
  if (blocks > 2147483647) bad("embedding gradient table too large");
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool vec = h % 4 == 0 && a16(g) && a16(out) && a16(addend);
  // A chunk fills the float4 registers of every thread (vec) or 4096 floats.
  const int ch = int(vec ? std::max<int64_t>(1, int64_t(kEgThreads) * kEgVec / (h / 4)) : std::max<int64_t>(1, 4096 / h));
  const size_t lds = size_t(n) * 4 + size_t(ch) * size_t(h) * 4;
  MSX_LAUNCH(k_embedding_grad, dim3(unsigned(blocks)), dim3(kEgThreads), lds, s, ids, g, addend, out, int(n),
                     rows, h, stripe, ch, vec);
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
  MSX_LAUNCH(k_dropout, dim3(std::min<unsigned>(blocks_for(n, 256), 8192)), dim3(256), 0, s, x, o, n, token,
                     uint32_t(seed), uint32_t(seed >> 32), threshold, scale);
}

// ---------------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------------
// Cross-entropy. Row statistics once per logits tensor; the loss sums in f64 in one block.
// Row maximum, then the sum of exp(x - max), each pass with eight loads in flight per thread.
__global__ __launch_bounds__(256) void k_ce_stats(const float* __restrict__ x, float* __restrict__ stats, int64_t v,
                                                  int64_t ld) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const float* row = x + r * ld;
  const int tid = threadIdx.x;
  float m = -INFINITY;
  for (int64_t c0 = 0; c0 < v; c0 += 256 * 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t c = c0 + tid + 256 * u;
      t[u] = c < v ? row[c] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) m = fmaxf(m, t[u]);
  }
  m = wave_max(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float total = 0.0f;
  for (int64_t c0 = 0; c0 < v; c0 += 256 * 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t c = c0 + tid + 256 * u;
      t[u] = c < v ? row[c] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) total += expf(t[u] - m);
  }
  total = wave_sum(total);
  if ((tid & 63) == 0) red[tid >> 6] = total;
  __syncthreads();
  if (tid == 0) { stats[2 * r] = m; stats[2 * r + 1] = (red[0] + red[1]) + (red[2] + red[3]); }
}
void ce_stats(hipStream_t s, const float* logits, float* stats, int64_t rows, int64_t v, int64_t ld) {
  if (rows <= 0) return;
  if (rows > 2147483647) bad("cross_entropy rows");
  if (ld < v) bad("cross_entropy row pitch");
  MSX_LAUNCH(k_ce_stats, dim3(unsigned(rows)), dim3(256), 0, s, logits, stats, v, ld);
}

// The loss of one block of 256 threads (k_ce_loss, and the tail block of k_finalize_adamw).
__device__ __forceinline__ void ce_loss_block(const float* __restrict__ x, const int32_t* __restrict__ labels,
                                              const float* __restrict__ w, const float* __restrict__ stats,
                                              float* __restrict__ loss, float* __restrict__ den_out, int64_t rows,
                                              int64_t v, int64_t ld, const float* __restrict__ rowloss, LossLog log) {
  __shared__ double num_s[256], den_s[256];
  double num = 0.0, den = 0.0;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) {
    float l;
    if (rowloss) {
      l = rowloss[r];
    } else {
      int32_t lab = labels[r];
      float xl = (lab >= 0 && lab < v) ? x[r * ld + lab] : 0.0f;
      l = stats[2 * r] + logf(stats[2 * r + 1]) - xl;
    }
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
    const float l = d == 0.0 ? 0.0f : float(n / d);
    loss[0] = l;
    if (den_out) den_out[0] = float(d);
    if (log.losses) {  // k_record_loss's append
      const uint32_t c = log.counter[0];
      if (c < log.capacity) log.losses[c] = l;
      log.counter[0] = c + 1;
    }
  }
}
__global__ __launch_bounds__(256) void k_ce_loss(const float* __restrict__ x, const int32_t* __restrict__ labels,
                                                 const float* __restrict__ w, const float* __restrict__ stats,
                                                 float* __restrict__ loss, float* __restrict__ den_out, int64_t rows,
                                                 int64_t v, int64_t ld, const float* __restrict__ rowloss, LossLog log) {
  ce_loss_block(x, labels, w, stats, loss, den_out, rows, v, ld, rowloss, log);
}
void ce_loss(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* stats, float* loss,
             float* den, int64_t rows, int64_t v, int64_t ld, const float* rowloss, LossLog log) {
  MSX_LAUNCH(k_ce_loss, dim3(1), dim3(256), 0, s, logits, labels, w, stats, loss, den, rows, v, ld, rowloss, log);
}

__global__ void k_ce_grad(const float* __restrict__ x, const int32_t* __restrict__ labels, const float* __restrict__ w,
                          const float* __restrict__ stats, const float* __restrict__ den, const float* __restrict__ g,
                          float* __restrict__ o, int64_t v, int64_t ld) {
  const int64_t r = blockIdx.y;
  const float d = den[0];
  const float scale = d == 0.0f ? 0.0f : g[0] * w[r] / d;
  const float mx = stats[2 * r], total = stats[2 * r + 1];
  const int32_t lab = labels[r];
  for (int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; c < v; c += int64_t(gridDim.x) * blockDim.x) {
    float target = c == lab ? 1.0f : 0.0f;
    o[r * ld + c] = d == 0.0f ? 0.0f : scale * (expf(x[r * ld + c] - mx) / total - target);
  }
}
void ce_grad(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* stats,
             const float* den, const float* g, float* o, int64_t rows, int64_t v, int64_t ld) {
  if (rows <= 0) return;
  if (rows > 65535) bad("cross_entropy gradient rows");
  dim3 grid(unsigned(std::min<int64_t>((v + 255) / 256, 64)), unsigned(rows));
  MSX_LAUNCH(k_ce_grad, grid, dim3(256), 0, s, logits, labels, w, stats, den, g, o, v, ld);
}

// Cross-entropy of whole rows in one pass over the logits: a block of kCeThreads holds its row in
// registers (NV float4 a thread), takes the max and the sum of exp, writes them to stats, the
// row's loss term max + log(sum) - x[label] to rowloss (when non-null) and, when grad is
// non-null, the gradient g w / den (exp(x - max) / sum - onehot), the quotient taken as a product
// with the reciprocal of the sum, zero in the padding columns. den is formed in each block exactly
// as k_ce_loss forms it.
constexpr int kCeThreads = 1024;
template <int NV>
__global__ __launch_bounds__(kCeThreads) void k_ce_rows(const float* __restrict__ x, const int32_t* __restrict__ labels,
                                                        const float* __restrict__ w, const float* __restrict__ g,
                                                        float* __restrict__ stats, float* __restrict__ rowloss,
                                                        float* __restrict__ grad, int64_t rows, int64_t v, int64_t ld) {
  constexpr int W = kCeThreads / 64;
  __shared__ float red[W];
  __shared__ double dred[256];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float4* row = reinterpret_cast<const float4*>(x + r * ld);
  const int64_t nq = (v + 3) / 4;
  float e[NV][4];
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int64_t q = tid + int64_t(kCeThreads) * u;
    const float4 f = row[q < nq ? q : nq - 1];
    e[u][0] = f.x; e[u][1] = f.y; e[u][2] = f.z; e[u][3] = f.w;
  }
  auto col = [&](int u, int c) { return 4 * (tid + int64_t(kCeThreads) * u) + c; };
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < NV; ++u)
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (col(u, c) < v) m = fmaxf(m, e[u][c]);
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int i = 1; i < W; ++i) m = fmaxf(m, red[i]);
  __syncthreads();
  float sum = 0.0f;
#pragma unroll
  for (int u = 0; u < NV; ++u)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      e[u][c] = col(u, c) < v ? expf(e[u][c] - m) : 0.0f;
      sum += e[u][c];
    }
  sum = wave_sum(sum);
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < W; i += 2) total += red[i] + red[i + 1];
  const int32_t lab = labels[r];
  if (tid == 0) {
    stats[2 * r] = m;
    stats[2 * r + 1] = total;
    if (rowloss) rowloss[r] = m + logf(total) - ((lab >= 0 && lab < v) ? x[r * ld + lab] : 0.0f);
  }
  if (!grad) return;
  double dd = 0.0;
  if (tid < 256)
    for (int64_t i = tid; i < rows; i += 256) dd += double(w[i]);
  if (tid < 256) dred[tid] = dd;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) dred[tid] += dred[tid + o];
    __syncthreads();
  }
  const float d = float(dred[0]);
  const float scale = d == 0.0f ? 0.0f : g[0] * w[r] / d, inv = 1.0f / total;
  float4* out = reinterpret_cast<float4*>(grad + r * ld);
  auto gv = [&](int u, int c) {
    const int64_t cc = col(u, c);
    if (cc >= v || d == 0.0f) return 0.0f;
    return scale * (e[u][c] * inv - (cc == lab ? 1.0f : 0.0f));
  };
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int64_t q = tid + int64_t(kCeThreads) * u;
    if (q < nq) out[q] = make_float4(gv(u, 0), gv(u, 1), gv(u, 2), gv(u, 3));
  }
}

// The same, persistent: a block (the grid holds two for each CU) walks rows blockIdx.x,
// + gridDim.x, ..., the next row's loads in flight while the current row is reduced and its
// gradient written (rows of 30522 classes: a block alone on its CU otherwise waits out each row's
// load latency between its reductions). The weight sum is taken once a block.
template <int NV>
__global__ __launch_bounds__(kCeThreads) void k_ce_rows_p(const float* __restrict__ x, const int32_t* __restrict__ labels,
                                                          const float* __restrict__ w, const float* __restrict__ g,
                                                          float* __restrict__ stats, float* __restrict__ rowloss,
                                                          float* __restrict__ grad, int64_t rows, int64_t v, int64_t ld) {
  constexpr int W = kCeThreads / 64;
  __shared__ float redm[W], reds[W];
  __shared__ double dred[256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // Columns in 32 bits (v < 2^31 is checked by the launcher).
  const int nq = int((v + 3) / 4), vi = int(v);
  auto col = [&](int u, int c) { return 4 * (tid + kCeThreads * u) + c; };
  float d = 0.0f;
  if (grad) {
    double dd = 0.0;
    if (tid < 256)
      for (int64_t i = tid; i < rows; i += 256) dd += double(w[i]);
    if (tid < 256) dred[tid] = dd;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (tid < o) dred[tid] += dred[tid + o];
      __syncthreads();
    }
    d = float(dred[0]);
  }
  const float gs = grad ? g[0] : 0.0f;
  v4f cur[NV], nxt[NV];
  // Columns past the row hold -inf from the load on: the maximum, exp and sum below then need no
  // per-column masks (each one a live lane mask), exp(-inf - m) is +0, and so is their gradient.
  auto fetch = [&](v4f (&e)[NV], int64_t r) {
    const v4f* row = reinterpret_cast<const v4f*>(x + r * ld);
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int q = tid + kCeThreads * u;
      const v4f f = row[q < nq ? q : nq - 1];
#pragma unroll
      for (int c = 0; c < 4; ++c) e[u][c] = 4 * q + c < vi ? f[c] : -INFINITY;
    }
  };
  int64_t r = blockIdx.x;
  if (r < rows) fetch(cur, r);
  for (; r < rows; r += gridDim.x) {
    // The row's label, weight and labelled logit are loaded first, so that their latency passes
    // under the row's reductions rather than after them.
    const int32_t lab = labels[r];
    const float wr = grad ? w[r] : 0.0f;
    const float xlab = (tid == 0 && rowloss && lab >= 0 && lab < v) ? x[r * ld + lab] : 0.0f;
    const int64_t rn = r + gridDim.x;
    if (rn < rows) fetch(nxt, rn);
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < NV; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) m = fmaxf(m, cur[u][c]);
    m = wave_max(m);
    if (lane == 0) redm[wave] = m;
    __syncthreads();
    m = redm[0];
#pragma unroll
    for (int i = 1; i < W; ++i) m = fmaxf(m, redm[i]);
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < NV; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        cur[u][c] = expf(cur[u][c] - m);
        sum += cur[u][c];
      }
    sum = wave_sum(sum);
    if (lane == 0) reds[wave] = sum;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < W; i += 2) total += reds[i] + reds[i + 1];
    if (tid == 0) {
      stats[2 * r] = m;
      stats[2 * r + 1] = total;
      if (rowloss) rowloss[r] = m + logf(total) - xlab;
    }
    if (grad) {
      const float scale = d == 0.0f ? 0.0f : gs * wr / d, inv = 1.0f / total;
      v4f* out = reinterpret_cast<v4f*>(grad + r * ld);
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const int q = tid + kCeThreads * u;
        v4f o;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          o[c] = d == 0.0f ? 0.0f : scale * (cur[u][c] * inv - (col(u, c) == lab ? 1.0f : 0.0f));
        }
        if (q < nq) out[q] = o;
      }
    }
#pragma unroll
    for (int u = 0; u < NV; ++u) cur[u] = nxt[u];
  }
}

// The rows of a cross-entropy whose logits came from a GEMM that left each row's column-tile
// partials (max, sum of exp(v - max)): one wave a row combines them in tile order (the maximum,
// then the partial sums rescaled to it), then writes the row's statistics and loss term as
// k_ce_rows_p does, and its gradient entry for the GEMMs that form the gradient from the logits.
// Every block sums the weights (f64, as k_ce_rows_p and k_ce_loss do) for the entries' scale.
__global__ __launch_bounds__(256) void k_ce_head_rows(const float2* __restrict__ part, int64_t tiles,
                                                      const float* __restrict__ x, int64_t ld,
                                                      const int32_t* __restrict__ labels, const float* __restrict__ w,
                                                      const float* __restrict__ g, float* __restrict__ stats,
                                                      float* __restrict__ rowloss, float4* __restrict__ tab, int64_t rows,
                                                      int64_t v) {
  __shared__ double dred[256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  double dd = 0.0;
  for (int64_t i = tid; i < rows; i += 256) dd += double(w[i]);
  dred[tid] = dd;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) dred[tid] += dred[tid + o];
    __syncthreads();
  }
  const float d = float(dred[0]);
  const int64_t r = int64_t(blockIdx.x) * 4 + wave;
  if (r >= rows) return;
  const int32_t lab = labels[r];
  const float wr = w[r];
  const float xl = (lab >= 0 && lab < v) ? x[r * ld + lab] : 0.0f;
  const float2* pr = part + r * tiles;
  float m = -INFINITY;
  for (int64_t t = lane; t < tiles; t += 64) m = fmaxf(m, pr[t].x);
  m = wave_max(m);
  float s = 0.0f;
  for (int64_t t = lane; t < tiles; t += 64) s += pr[t].y * expf(pr[t].x - m);
  s = wave_sum(s);
  if (lane == 0) {
    stats[2 * r] = m;
    stats[2 * r + 1] = s;
    if (rowloss) rowloss[r] = m + logf(s) - xl;
    const float scale = d == 0.0f ? 0.0f : g[0] * wr / d;
    tab[r] = make_float4(m, 1.0f / s, scale, __int_as_float(d == 0.0f ? -2 : lab));
  }
}
void ce_head_rows(hipStream_t s, const float* part, int64_t tiles, const float* logits, int64_t ld, const int32_t* labels,
                  const float* w, const float* g, float* stats, float* rowloss, float4* tab, int64_t rows, int64_t v) {
  if (rows <= 0) return;
  MSX_LAUNCH(k_ce_head_rows, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, s, reinterpret_cast<const float2*>(part), tiles,
             logits, ld, labels, w, g, stats, rowloss, tab, rows, v);
}

int cu_count() {
  static int counts[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!counts[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

bool ce_rows_fits(int64_t v, int64_t ld) { return ld % 4 == 0 && (v + 3) / 4 <= int64_t(kCeThreads) * 8; }

void ce_rows(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* g, float* stats,
             float* rowloss, float* grad, int64_t rows, int64_t v, int64_t ld) {
  if (rows <= 0) return;
  if (rows > 2147483647) bad("cross_entropy rows");
  if (!ce_rows_fits(v, ld) || reinterpret_cast<uintptr_t>(logits) % 16 || (grad && reinterpret_cast<uintptr_t>(grad) % 16))
    bad("cross_entropy row kernel needs float4-aligned rows of at most 32768 classes");
  if (grad && !g) bad("cross_entropy gradient without the upstream gradient");
  const int64_t per = ((v + 3) / 4 + kCeThreads - 1) / kCeThreads;
  // Two blocks a CU's worth of blocks: on BERT-tiny's 832 rows the graph-launched step takes 3 us
  // less than with one (0.798 against 0.801 ms, A/B alternated on one box), four 3 us more.
  const unsigned blocks = unsigned(std::min<int64_t>(rows, 2 * int64_t(cu_count())));
#define MSX_CER(NV) MSX_LAUNCH(k_ce_rows_p<NV>, dim3(blocks), dim3(kCeThreads), 0, s, logits, labels, w, g, \
                                       stats, rowloss, grad, rows, v, ld)
  if (per <= 2) MSX_CER(2);
  else if (per <= 4) MSX_CER(4);
  else MSX_CER(8);
#undef MSX_CER
}

// ---------------------------------------------------------------------------------------------
// Held-out evaluation: one block of 256 per row. The first pass finds the largest logit and its
// first index (each thread scans its columns ascending, and equal maxima of different threads
// resolve to the lower index, which is the first largest of the row) and whether a NaN occurs;
// the second sums exp(x - max). A NaN or an infinity among the logits makes the nll NaN through
// the arithmetic itself, as the sequential restatement does.
__device__ __forceinline__ void better_of(float& m, int64_t& at, float m2, int64_t at2) {
  if (m2 > m || (m2 == m && at2 < at)) {
    m = m2;
    at = at2;
  }
}
__global__ __launch_bounds__(256) void k_held_out_rows(const float* __restrict__ x, const int32_t* __restrict__ labels,
                                                       float* __restrict__ out, int64_t v, int64_t ld) {
  __shared__ float red_m[4];
  __shared__ int64_t red_at[4];
  __shared__ int red_nan[4];
  const int64_t r = blockIdx.x;
  const float* row = x + r * ld;
  const int tid = threadIdx.x;
  float m = -INFINITY;
  int64_t at = v;  // no column yet: loses every tie
  bool nan = false;
  for (int64_t c0 = 0; c0 < v; c0 += 256 * 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t c = c0 + tid + 256 * u;
      t[u] = c < v ? row[c] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      nan = nan || (t[u] != t[u]);
      if (t[u] > m) {
        m = t[u];
        at = c0 + tid + 256 * u;
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64);
    const int64_t at2 = __shfl_xor(at, o, 64);
    better_of(m, at, m2, at2);
  }
  const bool wave_nan = __any(nan);
  if ((tid & 63) == 0) {
    red_m[tid >> 6] = m;
    red_at[tid >> 6] = at;
    red_nan[tid >> 6] = wave_nan;
  }
  __syncthreads();
  m = red_m[0];
  at = red_at[0];
  for (int k = 1; k < 4; ++k) better_of(m, at, red_m[k], red_at[k]);
  const bool row_nan = red_nan[0] | red_nan[1] | red_nan[2] | red_nan[3];
  if (at >= v) at = 0;  // every logit -inf: the first column is the first largest
  float total = 0.0f;
  for (int64_t c0 = 0; c0 < v; c0 += 256 * 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t c = c0 + tid + 256 * u;
      t[u] = c < v ? row[c] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) total += expf(t[u] - m);
  }
  total = wave_sum(total);
  __syncthreads();
  if ((tid & 63) == 0) red_m[tid >> 6] = total;
  __syncthreads();
  if (tid == 0) {
    const int32_t label = labels[r];
    total = (red_m[0] + red_m[1]) + (red_m[2] + red_m[3]);
    out[2 * r] = m + logf(total) - row[label];
    out[2 * r + 1] = (!row_nan && at == int64_t(label)) ? 1.0f : 0.0f;
  }
}
void held_out_rows(hipStream_t s, const float* logits, const int32_t* labels, float* out, int64_t rows, int64_t v,
                   int64_t ld) {
  if (rows <= 0) return;
  if (rows > 2147483647) bad("held-out rows");
  if (v <= 0 || ld < v) bad("held-out logits pitch");
  MSX_LAUNCH(k_held_out_rows, dim3(unsigned(rows)), dim3(256), 0, s, logits, labels, out, v, ld);
}

__global__ __launch_bounds__(1024) void k_held_out_sum(const float* __restrict__ rows_in, const float* __restrict__ w,
                                                       int64_t rows, HeldOutState* __restrict__ state) {
  __shared__ double num_s[16], den_s[16];
  __shared__ unsigned long long hit_s[16], sel_s[16];
  double num = 0.0, den = 0.0;
  unsigned long long hits = 0, sel = 0;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) {
    const float wr = w[r];
    num = __builtin_fma(double(wr), double(rows_in[2 * r]), num);
    den += double(wr);
    hits += (wr > 0.0f && rows_in[2 * r + 1] == 1.0f) ? 1 : 0;
    sel += wr > 0.0f ? 1 : 0;
  }
  for (int o = 32; o > 0; o >>= 1) {
    num += __shfl_xor(num, o, 64);
    den += __shfl_xor(den, o, 64);
    hits += __shfl_xor(hits, o, 64);
    sel += __shfl_xor(sel, o, 64);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    num_s[wave] = num;
    den_s[wave] = den;
    hit_s[wave] = hits;
    sel_s[wave] = sel;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < int(blockDim.x >> 6); ++k) {
      num += num_s[k];
      den += den_s[k];
      hits += hit_s[k];
      sel += sel_s[k];
    }
    state->numerator += num;
    state->correct += hits;
    state->denominator += den;
    state->selected += sel;
  }
}
void held_out_sum(hipStream_t s, const float* rows_in, const float* w, int64_t rows, HeldOutState* state) {
  if (rows <= 0) return;
  MSX_LAUNCH(k_held_out_sum, dim3(1), dim3(1024), 0, s, rows_in, w, rows, state);
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
  MSX_LAUNCH(k_softmax, dim3(unsigned(rows)), dim3(256), 0, s, x, o, k);
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
  MSX_LAUNCH(k_softmax_grad, dim3(unsigned(rows)), dim3(256), 0, s, y, g, o, k);
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
  MSX_LAUNCH(k_reduce, dim3(1), dim3(1024), 0, s, a, nullptr, o, n, mean ? 1 : 0);
}
void mse(hipStream_t s, const float* a, const float* b, float* o, int64_t n) {
  MSX_LAUNCH(k_reduce, dim3(1), dim3(1024), 0, s, a, b, o, n, 2);
}

// ---------------------------------------------------------------------------------------------
// One element of the update, every operation rounded on its own (compiled without contraction).
__device__ __forceinline__ void adamw_one(float& p, float g, float& m, float& v, const AdamWConsts& k, float lr, float b1,
                                          float b2) {
  const float m2 = k.beta1 * m + k.rest1 * g;
  const float v2 = k.beta2 * v + (k.rest2 * g) * g;
  const float dir = (m2 * b1) / (sqrtf(v2 * b2) + k.eps);
  const float step = dir + k.decay * p;
  p = p - lr * step;
  m = m2;
  v = v2;
}
// Four elements a thread as native 16-byte vectors (the arenas are 256-byte aligned), the tail of
// n mod 4 elements by the first threads.
__global__ __launch_bounds__(256) void k_adamw(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                                               float* __restrict__ v, int64_t n, AdamWConsts k,
                                               const float* __restrict__ lr_t, const float* __restrict__ c1,
                                               const float* __restrict__ c2, const LossScaleState* __restrict__ ls,
                                               _Float16* __restrict__ p16) {
  // A step whose scaled gradients overflowed makes no update (the loss scale halves instead).
  if (ls && ls->overflow) return;
  typedef _Float16 h4_ __attribute__((ext_vector_type(4)));
  const float lr = lr_t[0], b1 = c1[0], b2 = c2[0], inv = ls ? ls->inv : 1.0f;
  const bool scaled = ls != nullptr;
  const int64_t quads = n / 4, stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  v4f* p4 = reinterpret_cast<v4f*>(p);
  const v4f* g4 = reinterpret_cast<const v4f*>(g);
  v4f* m4 = reinterpret_cast<v4f*>(m);
  v4f* v4 = reinterpret_cast<v4f*>(v);
  for (int64_t q = t; q < quads; q += stride) {
    v4f pq = p4[q], gq = g4[q], mq = m4[q], vq = v4[q];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float pc = pq[c], mc = mq[c], vc = vq[c];
      adamw_one(pc, scaled ? gq[c] * inv : gq[c], mc, vc, k, lr, b1, b2);
      pq[c] = pc;
      mq[c] = mc;
      vq[c] = vc;
    }
    p4[q] = pq;
    m4[q] = mq;
    v4[q] = vq;
    if (p16) reinterpret_cast<h4_*>(p16)[q] = h4_{_Float16(pq[0]), _Float16(pq[1]), _Float16(pq[2]), _Float16(pq[3])};
  }
  for (int64_t i = quads * 4 + t; i < n; i += stride) {
    adamw_one(p[i], scaled ? g[i] * inv : g[i], m[i], v[i], k, lr, b1, b2);
    if (p16) p16[i] = _Float16(p[i]);
  }
}
void adamw(hipStream_t s, float* p, const float* g, float* m, float* v, int64_t n, AdamWConsts k, const float* lr_t,
           const float* c1, const float* c2, const LossScaleState* ls, _Float16* p16) {
  if (n <= 0) return;
  for (const void* a : {static_cast<const void*>(p), static_cast<const void*>(g), static_cast<const void*>(m),
                        static_cast<const void*>(v)})
    if (reinterpret_cast<uintptr_t>(a) % 16) bad("AdamW arenas must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(p16) % 8) bad("AdamW f16 parameter copy must be 8-byte aligned");
  // Up to 65536 blocks (BERT-base's 110 M parameters: 643 -> 608 us against 16384, A/B in one run).
  MSX_LAUNCH(k_adamw, dim3(std::min<unsigned>(blocks_for((n + 3) / 4, 256), 65536)), dim3(256), 0, s, p, g, m, v, n,
             k, lr_t, c1, c2, ls, p16);
}

// The arena outside the finalize jobs' outputs: `segs` runs of whole 16-byte quads (first quad,
// quads before it in the list), then up to kFaLoose single elements.
constexpr int kFaSegs = 2 * kColumnJobs + 1;
constexpr int kFaLoose = 64;
struct FaRest {  // (32-bit indices: the launch's arguments stay under 4 KiB)
  uint32_t quad0[kFaSegs], before[kFaSegs];
  int64_t quads;
  int32_t segs, loose;
  uint32_t loose_at[kFaLoose];
};
__global__ __launch_bounds__(256) void k_finalize_adamw(ColumnJobs jobs, int fin_blocks, FaRest rest, float* __restrict__ p,
                                                        float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
                                                        AdamWConsts k, const float* __restrict__ lr_t,
                                                        const float* __restrict__ c1, const float* __restrict__ c2,
                                                        CeLossJob tail, int has_tail) {
  if (has_tail && blockIdx.x == 0) {
    ce_loss_block(tail.logits, tail.labels, tail.w, tail.stats, tail.loss, tail.den, tail.rows, tail.v, tail.ld,
                  tail.rowloss, tail.log);
    return;
  }
  const int bid = int(blockIdx.x) - has_tail;
  const float lr = lr_t[0], b1 = c1[0], b2 = c2[0];
  if (bid < fin_blocks) {
    // A finalize block (k_column_finalize's arithmetic), then the update of each finished element.
    __shared__ float red[256];
    int j = 0;
    while (j + 1 < jobs.count && bid >= jobs.job[j + 1].first) ++j;
    const ColumnJob& J = jobs.job[j];
    if (J.parts == 0) {
      v4f sum{0.0f, 0.0f, 0.0f, 0.0f};
      float* out = nullptr;
      if (!finalize_vec(J, bid - J.first, sum, out) || !out) return;
      const int64_t i = out - g;
#pragma unroll
      for (int e = 0; e < 4; ++e) adamw_one(p[i + e], sum[e], m[i + e], v[i + e], k, lr, b1, b2);
      return;
    }
    const int parts = J.parts, cols = 256 / parts;
    const int lc = threadIdx.x % cols, part = threadIdx.x / cols;
    const int64_t c = int64_t(bid - J.first) * cols + lc;
    const int per = (J.chunks + parts - 1) / parts;
    const int z_beg = part * per, z_end = min(J.chunks, z_beg + per);
    float sum = 0.0f;
    if (c < J.width) {
      for (int z0 = z_beg; z0 < z_end; z0 += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int z = z0 + u < z_end ? z0 + u : z_end - 1;
          t[u] = J.partial[int64_t(z) * J.width + c];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (z0 + u < z_end) sum = (z0 + u == z_beg) ? t[u] : sum + t[u];
      }
    }
    if (parts > 1) {
      red[threadIdx.x] = sum;
      __syncthreads();
      if (part != 0) return;
      for (int q = 1; q < parts && q * per < J.chunks; ++q) sum += red[q * cols + lc];
    }
    if (c >= J.width) return;
    float* const out = c < J.split ? (J.out_lo ? J.out_lo + c : nullptr) : (J.out_hi ? J.out_hi + (c - J.split) : nullptr);
    if (!out) return;
    *out = sum;
    const int64_t i = out - g;
    adamw_one(p[i], sum, m[i], v[i], k, lr, b1, b2);
    return;
  }
  // The rest of the arena: quad t of the runs, then the loose elements.
  const int64_t t = int64_t(bid - fin_blocks) * 256 + threadIdx.x;
  if (t < rest.quads) {
    int lo = 0, hi = rest.segs - 1;  // the last run starting at or before t
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (int64_t(rest.before[mid]) <= t) lo = mid; else hi = mid - 1;
    }
    const int64_t q = int64_t(rest.quad0[lo]) + (t - int64_t(rest.before[lo]));
    v4f* p4 = reinterpret_cast<v4f*>(p);
    const v4f* g4 = reinterpret_cast<const v4f*>(g);
    v4f* m4 = reinterpret_cast<v4f*>(m);
    v4f* v4 = reinterpret_cast<v4f*>(v);
    v4f pq = p4[q], gq = g4[q], mq = m4[q], vq = v4[q];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float pc = pq[c], mc = mq[c], vc = vq[c];
      adamw_one(pc, gq[c], mc, vc, k, lr, b1, b2);
      pq[c] = pc;
      mq[c] = mc;
      vq[c] = vc;
    }
    p4[q] = pq;
    m4[q] = mq;
    v4[q] = vq;
  } else if (t - rest.quads < rest.loose) {
    const int64_t i = int64_t(rest.loose_at[t - rest.quads]);
    adamw_one(p[i], g[i], m[i], v[i], k, lr, b1, b2);
  }
}
void finalize_adamw(hipStream_t s, const ColumnJob* jobs, int count, float* p, float* g, float* m, float* v, int64_t n,
                    AdamWConsts k, const float* lr_t, const float* c1, const float* c2, const CeLossJob* loss) {
  if (n <= 0) return;
  if (count <= 0 || count > kColumnJobs) bad("finalize_adamw takes 1 to 48 jobs");
  if (n >= (int64_t(1) << 32)) bad("finalize_adamw: an arena of 2^32 elements or more");
  for (const void* a : {static_cast<const void*>(p), static_cast<const void*>(g), static_cast<const void*>(m),
                        static_cast<const void*>(v)})
    if (reinterpret_cast<uintptr_t>(a) % 16) bad("AdamW arenas must be 16-byte aligned");
  ColumnJobs b{};
  int blocks = 0;
  b.count = count;
  // The jobs' outputs as element ranges of the arena.
  std::vector<std::pair<int64_t, int64_t>> taken;
  for (int j = 0; j < count; ++j) {
    b.job[j] = jobs[j];
    const ColumnJob& J = b.job[j];
    if (J.chunks <= 0 || J.width <= 0) bad("column finalize job without partials");
    b.job[j].first = blocks;
    b.job[j].parts = finalize_parts(J);
    blocks += finalize_blocks(b.job[j]);
    const std::pair<const float*, int64_t> outs[2] = {{J.out_lo, int64_t(std::min(J.split, J.width))},
                                                      {J.out_hi, int64_t(J.width) - std::min(J.split, J.width)}};
    for (auto [o, len] : outs) {
      if (!o || len <= 0) continue;
      const int64_t at = o - g;
      if (o < g || at + len > n) bad("finalize_adamw: a job's output lies outside the gradient arena");
      taken.push_back({at, at + len});
    }
  }
  std::sort(taken.begin(), taken.end());
  FaRest rest{};
  auto add_free = [&](int64_t a, int64_t e) {  // [a, e) is updated by the AdamW blocks
    if (a >= e) return;
    const int64_t qa = (a + 3) / 4, qe = e / 4;
    if (qa >= qe) {
      for (int64_t i = a; i < e; ++i) {
        if (rest.loose >= kFaLoose) bad("finalize_adamw: too many unaligned elements");
        rest.loose_at[rest.loose++] = uint32_t(i);
      }
      return;
    }
    for (int64_t i = a; i < 4 * qa; ++i) {
      if (rest.loose >= kFaLoose) bad("finalize_adamw: too many unaligned elements");
      rest.loose_at[rest.loose++] = uint32_t(i);
    }
    for (int64_t i = 4 * qe; i < e; ++i) {
      if (rest.loose >= kFaLoose) bad("finalize_adamw: too many unaligned elements");
      rest.loose_at[rest.loose++] = uint32_t(i);
    }
    if (rest.segs >= kFaSegs) bad("finalize_adamw: too many runs");
    rest.quad0[rest.segs] = uint32_t(qa);
    rest.before[rest.segs] = uint32_t(rest.quads);
    rest.quads += qe - qa;
    ++rest.segs;
  };
  int64_t at = 0;
  for (auto [a, e] : taken) {
    if (a < at) bad("finalize_adamw: overlapping job outputs");
    add_free(at, a);
    at = e;
  }
  add_free(at, n);
  if (rest.segs == 0) {  // (one empty run keeps the search well defined)
    rest.segs = 1;
    rest.quad0[0] = 0;
    rest.before[0] = 0;
  }
  const int64_t rest_blocks = (rest.quads + rest.loose + 255) / 256;
  const int tail = loss ? 1 : 0;
  MSX_LAUNCH(k_finalize_adamw, dim3(unsigned(tail + blocks + rest_blocks)), dim3(256), 0, s, b, blocks, rest, p, g, m, v,
             k, lr_t, c1, c2, loss ? *loss : CeLossJob{}, tail);
}

__global__ void k_sgd(float* __restrict__ p, const float* __restrict__ g, int64_t n, const float* __restrict__ lr,
                      const LossScaleState* __restrict__ ls) {
  if (ls && ls->overflow) return;
  const float r = lr[0], inv = ls ? ls->inv : 1.0f;
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i < n; i += int64_t(gridDim.x) * blockDim.x) p[i] = p[i] - r * (ls ? g[i] * inv : g[i]);
}
void sgd(hipStream_t s, float* p, const float* g, int64_t n, const float* lr, const LossScaleState* ls) {
  if (n <= 0) return;
  MSX_LAUNCH(k_sgd, dim3(std::min<unsigned>(blocks_for(n, 256), 16384)), dim3(256), 0, s, p, g, n, lr, ls);
}

// Dynamic loss scaling: any non-finite scaled gradient marks the step as overflowed.
__global__ __launch_bounds__(256) void k_grad_check(const float* __restrict__ g, int64_t n,
                                                    LossScaleState* __restrict__ ls) {
  bool bad = false;
  const int64_t quads = n / 4;
  const float4* g4 = reinterpret_cast<const float4*>(g);
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t q = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; q < quads; q += stride) {
    const float4 x = g4[q];
    bad = bad || !isfinite(x.x) || !isfinite(x.y) || !isfinite(x.z) || !isfinite(x.w);
  }
  for (int64_t i = quads * 4 + int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    bad = bad || !isfinite(g[i]);
  if (__any(bad) && (threadIdx.x & 63) == 0) ls->overflow = 1u;
}
// After the update: halve the scale on an overflow (and count the skipped step), double it after
// `window` clean steps in a row; keep it in [1, 2^24].
__global__ void k_loss_scale_update(LossScaleState* __restrict__ ls) {
  if (threadIdx.x != 0) return;
  if (ls->overflow) {
    ls->scale = fmaxf(ls->scale * 0.5f, 1.0f);
    ls->good = 0;
    ls->skipped += 1;
  } else if (++ls->good >= ls->window) {
    ls->scale = fminf(ls->scale * 2.0f, 16777216.0f);
    ls->good = 0;
  }
  ls->inv = 1.0f / ls->scale;
  ls->overflow = 0;
}
void grad_check(hipStream_t s, const float* g, int64_t n, LossScaleState* ls) {
  if (n <= 0) return;
  if (reinterpret_cast<uintptr_t>(g) % 16) bad("grad_check needs 16-byte aligned gradients");
  MSX_LAUNCH(k_grad_check, dim3(std::min<unsigned>(blocks_for(n / 4 + 1, 256), 4096)), dim3(256), 0, s, g, n, ls);
}
void loss_scale_update(hipStream_t s, LossScaleState* ls) { MSX_LAUNCH(k_loss_scale_update, dim3(1), dim3(64), 0, s, ls); }

__global__ void k_record_loss(const float* __restrict__ loss, float* __restrict__ losses, uint32_t* __restrict__ counter,
                              uint32_t capacity) {
  uint32_t c = counter[0];
  if (c < capacity) losses[c] = loss[0];
  counter[0] = c + 1;
}
namespace {
thread_local std::vector<std::string>* g_kernel_log = nullptr;
}  // namespace
void kernel_log(std::vector<std::string>* log) { g_kernel_log = log; }
void note_kernel(const char* expr) {
  if (!g_kernel_log) return;
  // "(k_name<...>)" or "k_name<...>": the name.
  std::string s(expr);
  size_t b = s.find_first_not_of("( ");
  size_t e = s.find_first_of("<( )", b);
  g_kernel_log->push_back(s.substr(b, e == std::string::npos ? std::string::npos : e - b));
}

void prepare() {
  // Kernels whose dynamic LDS may exceed the 64 KiB default; set once, outside any capture.
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_embedding_grad),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
  if (e != hipSuccess) throw std::runtime_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
  prepare_attention();
}

void record_loss(hipStream_t s, const float* loss, float* losses, uint32_t* counter, uint32_t capacity) {
  MSX_LAUNCH(k_record_loss, dim3(1), dim3(1), 0, s, loss, losses, counter, capacity);
}

}  // namespace msx::hk
