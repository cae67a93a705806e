// Attention of a training step on gfx950: the forward, and its gradients with respect to q, k and
// v, per (sequence, head). The main path runs on the f32 MFMA (v_mfma_f32_16x16x4f32) in a flash
// layout: a wave owns 16 query rows (forward, dQ) or 16 key rows (dK, dV); the scores are
// computed transposed (K Q^T) so that the probabilities of a query sit in the lanes that feed
// them to the P V and dS K MFMAs without an LDS round trip. The forward saves each query's
// softmax maximum and sum; the backward recomputes P from them and takes
// d_i = sum_j P_ij dP_ij as rowsum(dO_i * O_i) from the forward's output. Shapes outside the MFMA
// tiling run a scalar fallback (one thread per row). Semantics: interpreter.rs:1035-1119,
// 1298-1510 (masked keys excluded; a masked key's dK and dV rows are +0).
#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>

#include "kernels.h"
#include "device.h"

namespace msx::hk {

namespace {
typedef float v4f __attribute__((ext_vector_type(4)));
[[noreturn]] void refuse(const std::string& what) { throw std::runtime_error("kernel launch refused: " + what); }
const size_t kLdsMax = 160 * 1024;

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
}  // namespace

// ---------------------------------------------------------------------------------------------
// Scalar fallback.
template <int D>
__global__ __launch_bounds__(64) void k_attn_fwd_scalar(const float* __restrict__ q, const float* __restrict__ k,
                                                 const float* __restrict__ v, const float* __restrict__ mask,
                                                 float* __restrict__ o, int L, int S, int H, int heads, float scale) {
  extern __shared__ float sm[];
  float* Ks = sm;
  float* Vs = sm + S * D;
  float* Ms = sm + 2 * S * D;
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  for (int e = threadIdx.x; e < S * D; e += blockDim.x) {
    int j = e / D, c = e % D;
    Ks[e] = k[(int64_t(b) * S + j) * H + head * D + c];
    Vs[e] = v[(int64_t(b) * S + j) * H + head * D + c];
  }
  for (int j = threadIdx.x; j < S; j += blockDim.x) Ms[j] = mask[int64_t(b) * S + j];
  __syncthreads();
  const int i = blockIdx.y * blockDim.x + threadIdx.x;
  if (i >= L) return;
  const int64_t row = int64_t(b) * L + i;
  float qr[D], acc[D];
#pragma unroll
  for (int c = 0; c < D; ++c) { qr[c] = q[row * H + head * D + c]; acc[c] = 0.0f; }
  float mx = 0.0f;
  bool first = true;
  for (int j = 0; j < S; ++j) {
    if (Ms[j] == 0.0f) continue;
    const float* kj = Ks + j * D;
    float sc = qr[0] * kj[0];
#pragma unroll
    for (int c = 1; c < D; ++c) sc = __builtin_fmaf(qr[c], kj[c], sc);
    sc = sc * scale;
    if (first || sc > mx) mx = sc;
    first = false;
  }
  float total = 0.0f;
  for (int j = 0; j < S; ++j) {
    if (Ms[j] == 0.0f) continue;
    const float* kj = Ks + j * D;
    float sc = qr[0] * kj[0];
#pragma unroll
    for (int c = 1; c < D; ++c) sc = __builtin_fmaf(qr[c], kj[c], sc);
    float e = expf(sc * scale - mx);
    total += e;
    const float* vj = Vs + j * D;
#pragma unroll
    for (int c = 0; c < D; ++c) acc[c] = __builtin_fmaf(e, vj[c], acc[c]);
  }
#pragma unroll
  for (int c = 0; c < D; ++c) o[row * H + head * D + c] = acc[c] / total;
}

template <int D>
__global__ __launch_bounds__(256) void k_attn_bwd_scalar(const float* __restrict__ q, const float* __restrict__ k,
                                                  const float* __restrict__ v, const float* __restrict__ mask,
                                                  const float* __restrict__ g, float* __restrict__ dq,
                                                  float* __restrict__ dk, float* __restrict__ dv, int L, int S, int H,
                                                  int heads, float scale) {
  extern __shared__ float sm[];
  float* Qs = sm;
  float* Gs = Qs + L * D;
  float* Ks = Gs + L * D;
  float* Vs = Ks + S * D;
  float* Ms = Vs + S * D;
  float* st_m = Ms + S;
  float* st_l = st_m + L;
  float* st_d = st_l + L;
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  for (int e = threadIdx.x; e < L * D; e += blockDim.x) {
    int i = e / D, c = e % D;
    Qs[e] = q[(int64_t(b) * L + i) * H + head * D + c];
    Gs[e] = g[(int64_t(b) * L + i) * H + head * D + c];
  }
  for (int e = threadIdx.x; e < S * D; e += blockDim.x) {
    int j = e / D, c = e % D;
    Ks[e] = k[(int64_t(b) * S + j) * H + head * D + c];
    Vs[e] = v[(int64_t(b) * S + j) * H + head * D + c];
  }
  for (int j = threadIdx.x; j < S; j += blockDim.x) Ms[j] = mask[int64_t(b) * S + j];
  __syncthreads();
  auto dot = [](const float* x, const float* y) {
    float s = x[0] * y[0];
#pragma unroll
    for (int c = 1; c < D; ++c) s = __builtin_fmaf(x[c], y[c], s);
    return s;
  };
  // Phase 1, per query row: softmax statistics, d = sum_j P dP, and dQ.
  for (int i = threadIdx.x; i < L; i += blockDim.x) {
    const float* qi = Qs + i * D;
    const float* gi = Gs + i * D;
    float mx = 0.0f;
    bool first = true;
    for (int j = 0; j < S; ++j) {
      if (Ms[j] == 0.0f) continue;
      float sc = dot(qi, Ks + j * D) * scale;
      if (first || sc > mx) mx = sc;
      first = false;
    }
    float total = 0.0f;
    for (int j = 0; j < S; ++j) {
      if (Ms[j] == 0.0f) continue;
      total += expf(dot(qi, Ks + j * D) * scale - mx);
    }
    float dd = 0.0f;
    for (int j = 0; j < S; ++j) {
      if (Ms[j] == 0.0f) continue;
      float p = expf(dot(qi, Ks + j * D) * scale - mx) / total;
      dd = __builtin_fmaf(p, dot(gi, Vs + j * D), dd);
    }
    st_m[i] = mx;
    st_l[i] = total;
    st_d[i] = dd;
    if (dq) {
      float acc[D];
#pragma unroll
      for (int c = 0; c < D; ++c) acc[c] = 0.0f;
      for (int j = 0; j < S; ++j) {
        if (Ms[j] == 0.0f) continue;
        float p = expf(dot(qi, Ks + j * D) * scale - mx) / total;
        float ds = p * (dot(gi, Vs + j * D) - dd);
        const float* kj = Ks + j * D;
#pragma unroll
        for (int c = 0; c < D; ++c) acc[c] = __builtin_fmaf(ds, kj[c], acc[c]);
      }
#pragma unroll
      for (int c = 0; c < D; ++c) dq[(int64_t(b) * L + i) * H + head * D + c] = acc[c] * scale;
    }
  }
  __syncthreads();
  // Phase 2, per key row: dV = sum_i P g_i, dK = scale * sum_i dS q_i; a masked key stays +0.
  for (int j = threadIdx.x; j < S; j += blockDim.x) {
    const int64_t out = (int64_t(b) * S + j) * H + head * D;
    const bool live = Ms[j] != 0.0f;
    if (dv) {
      float acc[D];
#pragma unroll
      for (int c = 0; c < D; ++c) acc[c] = 0.0f;
      if (live)
        for (int i = 0; i < L; ++i) {
          float p = expf(dot(Qs + i * D, Ks + j * D) * scale - st_m[i]) / st_l[i];
          const float* gi = Gs + i * D;
#pragma unroll
          for (int c = 0; c < D; ++c) acc[c] = __builtin_fmaf(p, gi[c], acc[c]);
        }
#pragma unroll
      for (int c = 0; c < D; ++c) dv[out + c] = acc[c];
    }
    if (dk) {
      float acc[D];
#pragma unroll
      for (int c = 0; c < D; ++c) acc[c] = 0.0f;
      if (live)
        for (int i = 0; i < L; ++i) {
          const float* qi = Qs + i * D;
          float p = expf(dot(qi, Ks + j * D) * scale - st_m[i]) / st_l[i];
          float ds = p * (dot(Gs + i * D, Vs + j * D) - st_d[i]);
#pragma unroll
          for (int c = 0; c < D; ++c) acc[c] = __builtin_fmaf(ds, qi[c], acc[c]);
        }
#pragma unroll
      for (int c = 0; c < D; ++c) dk[out + c] = live ? acc[c] * scale : 0.0f;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// MFMA path. Row stride of every LDS tile is D + 4 floats: the 16 rows x 4 columns an MFMA
// operand read touches fall in distinct banks.
constexpr int kU = 4;      // row tiles whose MFMA chains interleave
constexpr int kWaves = 2;  // waves (16 rows each) a block: a block's K/V (or Q/dO) LDS copy limits
                           // a CU to two blocks, so smaller blocks spread a sequence over more CUs

// Stages rows [0, rows) of two [., H] head slices (x at xs + row H, y likewise, D floats each)
// into LDS tiles of row stride D + 4, eight float4 of each a thread in flight before any store.
template <int D>
__device__ __forceinline__ void stage_pair(float* X, float* Y, const float* __restrict__ xs,
                                           const float* __restrict__ ys, int rows, int H) {
  constexpr int DP = D + 4, Q = D / 4;
  const int total = rows * Q;
  for (int e0 = threadIdx.x; e0 < total; e0 += 8 * int(blockDim.x)) {
    float4 xv[8], yv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int e = e0 + u * int(blockDim.x);
      e = e < total ? e : total - 1;
      const int64_t off = int64_t(e / Q) * H + (e % Q) * 4;
      xv[u] = *reinterpret_cast<const float4*>(xs + off);
      yv[u] = *reinterpret_cast<const float4*>(ys + off);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + u * int(blockDim.x);
      if (e < total) {
        float* xd = X + (e / Q) * DP + (e % Q) * 4;
        float* yd = Y + (e / Q) * DP + (e % Q) * 4;
        xd[0] = xv[u].x; xd[1] = xv[u].y; xd[2] = xv[u].z; xd[3] = xv[u].w;
        yd[0] = yv[u].x; yd[1] = yv[u].y; yd[2] = yv[u].z; yd[3] = yv[u].w;
      }
    }
  }
}


// Scores of kU tiles of 16 LDS rows R (tiles t0 .. t0 + kU, the ones past nt repeat the last
// tile and are ignored by the caller) against the 16 columns whose operand fragments xb a lane
// holds: acc[u][r] = sum over d of R[(t0 + u) 16 + c][d] x[4 g + r][d], each in d order.
template <int D>
__device__ __forceinline__ void score_tiles(const float* R, const float (&xb)[D / 4], int t0, int nt, int c, int g,
                                            v4f (&acc)[kU]) {
  constexpr int DP = D + 4;
  const float* rr[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    acc[u] = v4f{0, 0, 0, 0};
    rr[u] = R + ((t0 + u < nt ? t0 + u : nt - 1) * 16 + c) * DP + g;
  }
#pragma unroll
  for (int t = 0; t < D / 4; ++t)
#pragma unroll
    for (int u = 0; u < kU; ++u) acc[u] = mfma4(rr[u][4 * t], xb[t], acc[u]);
}
// Stages rows [0, rows) of one [., H] head slice into an LDS tile of row stride D + 4.
template <int D>
__device__ __forceinline__ void stage_one(float* X, const float* __restrict__ xs, int rows, int H) {
  constexpr int DP = D + 4, Q = D / 4;
  const int total = rows * Q;
  for (int e0 = threadIdx.x; e0 < total; e0 += 8 * int(blockDim.x)) {
    float4 xv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int e = e0 + u * int(blockDim.x);
      e = e < total ? e : total - 1;
      xv[u] = *reinterpret_cast<const float4*>(xs + int64_t(e / Q) * H + (e % Q) * 4);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + u * int(blockDim.x);
      if (e < total) {
        float* xd = X + (e / Q) * DP + (e % Q) * 4;
        xd[0] = xv[u].x; xd[1] = xv[u].y; xd[2] = xv[u].z; xd[3] = xv[u].w;
      }
    }
  }
}

// The kernels below stream the other side of the attention (keys for the forward and dQ, queries
// for dK/dV) through LDS `chunk` rows at a time, in ascending order, so a sequence of any length
// fits; a sequence that fits one chunk is staged once. Every wave of a block takes part in the
// staging; waves past the last row tile compute nothing.
template <int D>
__global__ __launch_bounds__(256) void k_attn_fwd_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, const float* __restrict__ mask,
                                                       float* __restrict__ o, float* __restrict__ stats, int L, int S,
                                                       int H, int heads, float scale, int chunk) {
  constexpr int DP = D + 4;
  extern __shared__ float sm[];
  float* Ks = sm;
  float* Vs = sm + chunk * DP;
  float* Ms = sm + 2 * chunk * DP;
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t kbase = int64_t(b) * S * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int i0 = blockIdx.y * int(blockDim.x / 4) + wave * 16;
  const bool active = i0 < L;
  const bool single = S <= chunk;
  const int64_t qrow = (int64_t(b) * L + (active ? i0 : 0) + c) * H + head * D;
  float qb[D / 4];
#pragma unroll
  for (int t = 0; t < D / 4; ++t) qb[t] = q[qrow + 4 * t + g];
  // Pass 1: the maximum score of query i0 + c over the unmasked keys. kU key tiles at a time, so
  // that kU independent MFMA chains interleave.
  float mx = -INFINITY;
  for (int s0 = 0; s0 < S; s0 += chunk) {
    const int n = S - s0 < chunk ? S - s0 : chunk;
    __syncthreads();
    if (single) stage_pair<D>(Ks, Vs, k + kbase, v + kbase, n, H);
    else stage_one<D>(Ks, k + kbase + int64_t(s0) * H, n, H);
    for (int j = threadIdx.x; j < n; j += blockDim.x) Ms[j] = mask[int64_t(b) * S + s0 + j];
    __syncthreads();
    if (!active) continue;
    const int nt = n / 16;
    for (int jt0 = 0; jt0 < nt; jt0 += kU) {
      v4f acc[kU];
      score_tiles<D>(Ks, qb, jt0, nt, c, g, acc);
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (jt0 + u < nt && Ms[(jt0 + u) * 16 + 4 * g + r] != 0.0f) mx = fmaxf(mx, acc[u][r] * scale);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  // Pass 2: P = exp(s - max) into the P V MFMA, the sum of P alongside.
  float total = 0.0f;
  v4f oacc[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) oacc[ct] = v4f{0, 0, 0, 0};
  for (int s0 = 0; s0 < S; s0 += chunk) {
    const int n = S - s0 < chunk ? S - s0 : chunk;
    if (!single) {
      __syncthreads();
      stage_pair<D>(Ks, Vs, k + kbase + int64_t(s0) * H, v + kbase + int64_t(s0) * H, n, H);
      for (int j = threadIdx.x; j < n; j += blockDim.x) Ms[j] = mask[int64_t(b) * S + s0 + j];
      __syncthreads();
    }
    if (!active) continue;
    const int nt = n / 16;
    for (int jt0 = 0; jt0 < nt; jt0 += kU) {
      v4f acc[kU];
      score_tiles<D>(Ks, qb, jt0, nt, c, g, acc);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (jt0 + u >= nt) break;
        const int jt = jt0 + u;
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = Ms[jt * 16 + 4 * g + r] != 0.0f ? expf(acc[u][r] * scale - mx) : 0.0f;
          total += p[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* vr = Vs + (jt * 16 + 4 * g + r) * DP + c;
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) oacc[ct] = mfma4(p[r], vr[ct * 16], oacc[ct]);
        }
      }
    }
  }
  if (!active) return;
  total += __shfl_xor(total, 16, 64);
  total += __shfl_xor(total, 32, 64);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float row_total = __shfl(total, 4 * g + r, 64);
    const int64_t orow = (int64_t(b) * L + i0 + 4 * g + r) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) o[orow + ct * 16 + c] = oacc[ct][r] / row_total;
  }
  if (stats && g == 0) {
    const int64_t at = (int64_t(blockIdx.x) * L + i0 + c) * 2;
    stats[at] = mx;
    stats[at + 1] = total;
  }
}

// dQ and d_i = rowsum(dO * O), per 16 query rows.
template <int D>
__global__ __launch_bounds__(256) void k_attn_bwd_q_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, const float* __restrict__ mask,
                                                         const float* __restrict__ o, const float* __restrict__ stats,
                                                         const float* __restrict__ go, float* __restrict__ dq,
                                                         float* __restrict__ dsum, int L, int S, int H, int heads,
                                                         float scale, int chunk) {
  constexpr int DP = D + 4;
  extern __shared__ float sm[];
  float* Ks = sm;
  float* Vs = sm + chunk * DP;
  float* Ms = sm + 2 * chunk * DP;
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t kbase = int64_t(b) * S * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int i0 = blockIdx.y * int(blockDim.x / 4) + wave * 16;
  const bool active = i0 < L;
  const int64_t row = (int64_t(b) * L + (active ? i0 : 0) + c) * H + head * D;
  // d_i for query i0 + c: lane group g sums columns [g D/4, (g + 1) D/4).
  float dd = 0.0f;
#pragma unroll
  for (int t = 0; t < D / 4; ++t) dd = __builtin_fmaf(go[row + g * (D / 4) + t], o[row + g * (D / 4) + t], dd);
  dd += __shfl_xor(dd, 16, 64);
  dd += __shfl_xor(dd, 32, 64);
  const int64_t srow = int64_t(blockIdx.x) * L + (active ? i0 : 0) + c;
  if (active && g == 0) dsum[srow] = dd;
  const float mx = stats[2 * srow], total = stats[2 * srow + 1];
  float qb[D / 4], gb[D / 4];
#pragma unroll
  for (int t = 0; t < D / 4; ++t) { qb[t] = q[row + 4 * t + g]; gb[t] = go[row + 4 * t + g]; }
  v4f acc[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) acc[ct] = v4f{0, 0, 0, 0};
  for (int s0 = 0; s0 < S; s0 += chunk) {
    const int n = S - s0 < chunk ? S - s0 : chunk;
    __syncthreads();
    stage_pair<D>(Ks, Vs, k + kbase + int64_t(s0) * H, v + kbase + int64_t(s0) * H, n, H);
    for (int j = threadIdx.x; j < n; j += blockDim.x) Ms[j] = mask[int64_t(b) * S + s0 + j];
    __syncthreads();
    if (!active) continue;
    const int nt = n / 16;
    for (int jt0 = 0; jt0 < nt; jt0 += kU) {
      v4f st[kU], dpt[kU];
      score_tiles<D>(Ks, qb, jt0, nt, c, g, st);
      score_tiles<D>(Vs, gb, jt0, nt, c, g, dpt);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (jt0 + u >= nt) break;
        const int jt = jt0 + u;
        float ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float p = Ms[jt * 16 + 4 * g + r] != 0.0f ? expf(st[u][r] * scale - mx) / total : 0.0f;
          ds[r] = p * (dpt[u][r] - dd);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* kk = Ks + (jt * 16 + 4 * g + r) * DP + c;
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) acc[ct] = mfma4(ds[r], kk[ct * 16], acc[ct]);
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t orow = (int64_t(b) * L + i0 + 4 * g + r) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) dq[orow + ct * 16 + c] = acc[ct][r] * scale;
  }
}

// dK and dV, per 16 key rows, over every query of the sequence.
template <int D>
__global__ __launch_bounds__(256) void k_attn_bwd_kv_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, const float* __restrict__ mask,
                                                          const float* __restrict__ stats, const float* __restrict__ go,
                                                          const float* __restrict__ dsum, float* __restrict__ dk,
                                                          float* __restrict__ dv, int L, int S, int H, int heads,
                                                          float scale, int chunk) {
  constexpr int DP = D + 4;
  extern __shared__ float sm[];
  float* Qs = sm;
  float* Gs = sm + chunk * DP;
  float* Sm = sm + 2 * chunk * DP;  // max, sum, d per query of the chunk
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t qbase = int64_t(b) * L * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int j0 = blockIdx.y * int(blockDim.x / 4) + wave * 16;
  const bool active = j0 < S;
  const int64_t krow = (int64_t(b) * S + (active ? j0 : 0) + c) * H + head * D;
  const bool live = mask[int64_t(b) * S + (active ? j0 : 0) + c] != 0.0f;
  float kb[D / 4], vb[D / 4];
#pragma unroll
  for (int t = 0; t < D / 4; ++t) { kb[t] = k[krow + 4 * t + g]; vb[t] = v[krow + 4 * t + g]; }
  v4f dka[D / 16], dva[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) { dka[ct] = v4f{0, 0, 0, 0}; dva[ct] = v4f{0, 0, 0, 0}; }
  for (int l0 = 0; l0 < L; l0 += chunk) {
    const int n = L - l0 < chunk ? L - l0 : chunk;
    __syncthreads();
    stage_pair<D>(Qs, Gs, q + qbase + int64_t(l0) * H, go + qbase + int64_t(l0) * H, n, H);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int64_t srow = int64_t(blockIdx.x) * L + l0 + i;
      Sm[3 * i] = stats[2 * srow];
      Sm[3 * i + 1] = stats[2 * srow + 1];
      Sm[3 * i + 2] = dsum[srow];
    }
    __syncthreads();
    if (!active) continue;
    const int nt = n / 16;
    for (int it0 = 0; it0 < nt; it0 += kU) {
      v4f s[kU], dp[kU];
      score_tiles<D>(Qs, kb, it0, nt, c, g, s);
      score_tiles<D>(Gs, vb, it0, nt, c, g, dp);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        if (it0 + u >= nt) break;
        const int it = it0 + u;
        float p[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* st = Sm + 3 * (it * 16 + 4 * g + r);
          p[r] = live ? expf(s[u][r] * scale - st[0]) / st[1] : 0.0f;
          ds[r] = p[r] * (dp[u][r] - st[2]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* gq = Gs + (it * 16 + 4 * g + r) * DP + c;
          const float* qq = Qs + (it * 16 + 4 * g + r) * DP + c;
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) {
            dva[ct] = mfma4(p[r], gq[ct * 16], dva[ct]);
            dka[ct] = mfma4(ds[r], qq[ct * 16], dka[ct]);
          }
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int j = j0 + 4 * g + r;
    const bool keep = mask[int64_t(b) * S + j] != 0.0f;
    const int64_t orow = (int64_t(b) * S + j) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) {
      if (dv) dv[orow + ct * 16 + c] = keep ? dva[ct][r] : 0.0f;
      if (dk) dk[orow + ct * 16 + c] = keep ? dka[ct][r] * scale : 0.0f;
    }
  }
}

// ---------------------------------------------------------------------------------------------
namespace {
size_t scalar_fwd_lds(int64_t S, int64_t d) { return size_t((2 * S * d + S) * 4); }
size_t scalar_bwd_lds(int64_t L, int64_t S, int64_t d) { return size_t((2 * L * d + 2 * S * d + S + 3 * L) * 4); }
// The rows an MFMA kernel streams through LDS at a time: the fewest chunks of at most what fits
// (two tiles of row stride d + 4 and three floats a row), of equal size in whole 16-row tiles.
int64_t mfma_chunk(int64_t n, int64_t d) {
  const int64_t most = int64_t(kLdsMax) / ((2 * (d + 4) + 3) * 4) / 16 * 16;
  const int64_t chunks = (n + most - 1) / most;
  return ((n + chunks - 1) / chunks + 15) / 16 * 16;
}
size_t mfma_fwd_lds(int64_t chunk, int64_t d) { return size_t((2 * chunk * (d + 4) + chunk) * 4); }
size_t mfma_kv_lds(int64_t chunk, int64_t d) { return size_t((2 * chunk * (d + 4) + 3 * chunk) * 4); }
bool head_ok(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128; }

template <template <int> class K>
struct ByD;
}  // namespace

bool attention_mfma(int64_t L, int64_t S, int64_t d) {
  return head_ok(d) && L % 16 == 0 && S % 16 == 0;
}

bool attention_fits(int64_t s, int64_t d) {
  return head_ok(d) && s <= 65535 && (attention_mfma(s, s, d) || scalar_bwd_lds(s, s, d) <= kLdsMax);
}

#define MSX_BY_D(d, call)                          \
  switch (d) {                                     \
    case 16: call(16); break;                      \
    case 32: call(32); break;                      \
    case 64: call(64); break;                      \
    default: call(128); break;                     \
  }

void attention_fwd(hipStream_t s, const float* q, const float* k, const float* v, const float* mask, float* o,
                   float* stats, int64_t B, int64_t L, int64_t S, int64_t H, int64_t heads) {
  int64_t d = H / heads;
  if (!head_ok(d) || L > S) refuse("attention head width or query rows");
  float scale = 1.0f / sqrtf(float(d));
  if (attention_mfma(L, S, d)) {
    dim3 grid(unsigned(B * heads), unsigned((L + 16 * kWaves - 1) / (16 * kWaves)));
    const int chunk = int(mfma_chunk(S, d));
    size_t lds = mfma_fwd_lds(chunk, d);
#define GO(D) MSX_LAUNCH(k_attn_fwd_mfma<D>, grid, dim3(64 * kWaves), lds, s, q, k, v, mask, o, stats, int(L), int(S), int(H), int(heads), scale, chunk)
    MSX_BY_D(d, GO)
#undef GO
    return;
  }
  if (scalar_fwd_lds(S, d) > kLdsMax || stats) refuse("attention shape outside the kernels' LDS budget");
  dim3 grid(unsigned(B * heads), unsigned((L + 63) / 64));
  size_t lds = scalar_fwd_lds(S, d);
#define GO(D) MSX_LAUNCH(k_attn_fwd_scalar<D>, grid, dim3(64), lds, s, q, k, v, mask, o, int(L), int(S), int(H), int(heads), scale)
  MSX_BY_D(d, GO)
#undef GO
}

void attention_bwd(hipStream_t s, const float* q, const float* k, const float* v, const float* mask, const float* o,
                   const float* stats, const float* g, float* dq, float* dk, float* dv, float* dsum, int64_t B,
                   int64_t L, int64_t S, int64_t H, int64_t heads) {
  int64_t d = H / heads;
  if (!head_ok(d) || L > S) refuse("attention head width or query rows");
  float scale = 1.0f / sqrtf(float(d));
  if (attention_mfma(L, S, d)) {
    if (!o || !stats || !dsum) refuse("the MFMA attention backward needs the forward output and statistics");
    dim3 gq(unsigned(B * heads), unsigned((L + 16 * kWaves - 1) / (16 * kWaves)));
    if (dq || dk || dv) {
      // dQ (written only when asked) and the d_i the key pass reads.
      float* dq_out = dq;
      const int chunk = int(mfma_chunk(S, d));
      size_t lq = mfma_fwd_lds(chunk, d);
#define GO(D) MSX_LAUNCH(k_attn_bwd_q_mfma<D>, gq, dim3(64 * kWaves), lq, s, q, k, v, mask, o, stats, g, dq_out, dsum, int(L), int(S), int(H), int(heads), scale, chunk)
      if (dq_out) { MSX_BY_D(d, GO) }
#undef GO
      if (!dq_out) refuse("the MFMA attention backward computes d_i in its dQ pass: dQ is required");
    }
    if (dk || dv) {
      dim3 gk(unsigned(B * heads), unsigned((S + 16 * kWaves - 1) / (16 * kWaves)));
      const int chunk = int(mfma_chunk(L, d));
      size_t lk = mfma_kv_lds(chunk, d);
#define GO(D) MSX_LAUNCH(k_attn_bwd_kv_mfma<D>, gk, dim3(64 * kWaves), lk, s, q, k, v, mask, stats, g, dsum, dk, dv, int(L), int(S), int(H), int(heads), scale, chunk)
      MSX_BY_D(d, GO)
#undef GO
    }
    return;
  }
  if (scalar_bwd_lds(L, S, d) > kLdsMax) refuse("attention shape outside the kernels' LDS budget");
  size_t lds = scalar_bwd_lds(L, S, d);
  int threads = int(std::min<int64_t>(256, std::max<int64_t>(64, (S + 63) / 64 * 64)));
#define GO(D) MSX_LAUNCH(k_attn_bwd_scalar<D>, dim3(unsigned(B * heads)), dim3(threads), lds, s, q, k, v, mask, g, dq, dk, dv, int(L), int(S), int(H), int(heads), scale)
  MSX_BY_D(d, GO)
#undef GO
}

void prepare_attention() {
  const void* kernels[] = {
      reinterpret_cast<const void*>(k_attn_fwd_scalar<16>), reinterpret_cast<const void*>(k_attn_fwd_scalar<32>),
      reinterpret_cast<const void*>(k_attn_fwd_scalar<64>), reinterpret_cast<const void*>(k_attn_fwd_scalar<128>),
      reinterpret_cast<const void*>(k_attn_bwd_scalar<16>), reinterpret_cast<const void*>(k_attn_bwd_scalar<32>),
      reinterpret_cast<const void*>(k_attn_bwd_scalar<64>), reinterpret_cast<const void*>(k_attn_bwd_scalar<128>),
      reinterpret_cast<const void*>(k_attn_fwd_mfma<16>),   reinterpret_cast<const void*>(k_attn_fwd_mfma<32>),
      reinterpret_cast<const void*>(k_attn_fwd_mfma<64>),   reinterpret_cast<const void*>(k_attn_fwd_mfma<128>),
      reinterpret_cast<const void*>(k_attn_bwd_q_mfma<16>), reinterpret_cast<const void*>(k_attn_bwd_q_mfma<32>),
      reinterpret_cast<const void*>(k_attn_bwd_q_mfma<64>), reinterpret_cast<const void*>(k_attn_bwd_q_mfma<128>),
      reinterpret_cast<const void*>(k_attn_bwd_kv_mfma<16>), reinterpret_cast<const void*>(k_attn_bwd_kv_mfma<32>),
      reinterpret_cast<const void*>(k_attn_bwd_kv_mfma<64>), reinterpret_cast<const void*>(k_attn_bwd_kv_mfma<128>)};
  for (const void* kern : kernels) {
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, int(kLdsMax));
    if (e != hipSuccess) throw std::runtime_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
  }
}

}  // namespace msx::hk
