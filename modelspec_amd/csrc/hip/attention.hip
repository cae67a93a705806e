// Attention of a training step on gfx950: the forward, and its gradients with respect to q, k and
// v, per (sequence, head). The main path runs on the f32 MFMA (v_mfma_f32_16x16x4f32) in a flash
// layout: a wave owns 16 query rows (forward, dQ) or 16 key rows (dK, dV); the scores are
// computed transposed (K Q^T) so that the probabilities of a query sit in the lanes that feed
// them to the P V and dS K MFMAs without an LDS round trip. The forward is one pass over the keys
// (online softmax) and saves each query's softmax maximum and sum; the backward recomputes P from
// them and takes
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
// MFMA path. A block is four waves; each wave owns 16 rows of its side (queries for the forward
// and dQ, keys for dK/dV) and the block streams the other side through LDS in tiles of T rows,
// double-buffered: the next tile's global loads are in flight while the current one is in the
// MFMAs, and one barrier a tile hands the buffers over. Row stride of every LDS tile is D + 4
// floats: the 16 rows x 4 columns an MFMA operand read touches fall in distinct banks.

// Scores of U tiles of 16 LDS rows R against the 16 columns whose operand fragments xb a lane
// holds: acc[u][r] = sum over d of R[16 u + c][d] x[4 g + r][d], each in d order. Tiles at or past
// nt (a partial last tile) repeat tile nt - 1, branch-free; the caller ignores them.
template <int D, int U>
__device__ __forceinline__ void score_tiles(const float* R, const float (&xb)[D / 4], int nt, int c, int g,
                                            v4f (&acc)[U]) {
  constexpr int DP = D + 4;
  const float* rr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    acc[u] = v4f{0, 0, 0, 0};
    rr[u] = R + (16 * (u < nt ? u : nt - 1) + c) * DP + g;
  }
#pragma unroll
  for (int t = 0; t < D / 4; ++t)
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = mfma4(rr[u][4 * t], xb[t], acc[u]);
}

// One tile of two [., H] head slices (rows 0 .. n of x and y, D floats each) on its way to LDS
// through registers: fetch_pair issues the global loads (rows past n repeat row n - 1), put_pair
// stores them as tiles of row stride D + 4. NT threads take part, PT = tile_groups 4-float groups
// of each slice a thread, held as native vectors (a float4 struct array is copied through private
// memory).
template <int D, int T, int NT>
constexpr int tile_groups() { return (T * (D / 4) + NT - 1) / NT; }
template <int D, int T, int NT, int PT>
__device__ __forceinline__ void fetch_pair(v4f (&xv)[PT], v4f (&yv)[PT], const float* __restrict__ xs,
                                           const float* __restrict__ ys, int64_t H, int n) {
  constexpr int Q = D / 4, G = T * Q;
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int e = int(threadIdx.x) + NT * p;
    int row = e / Q;
    row = row < n ? row : n - 1;
    const int64_t off = int64_t(row) * H + (e % Q) * 4;
    if (G % NT == 0 || e < G) {
      xv[p] = *reinterpret_cast<const v4f*>(xs + off);
      yv[p] = *reinterpret_cast<const v4f*>(ys + off);
    }
  }
}
template <int D, int T, int NT, int PT>
__device__ __forceinline__ void put_pair(float* X, float* Y, const v4f (&xv)[PT], const v4f (&yv)[PT]) {
  constexpr int DP = D + 4, Q = D / 4, G = T * Q;
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int e = int(threadIdx.x) + NT * p;
    if (G % NT == 0 || e < G) {
      *reinterpret_cast<v4f*>(X + (e / Q) * DP + (e % Q) * 4) = xv[p];
      *reinterpret_cast<v4f*>(Y + (e / Q) * DP + (e % Q) * 4) = yv[p];
    }
  }
}
// Floats of LDS a streaming kernel takes: two buffers of two T x (D + 4) tiles and E floats a row.
// Floats of LDS a streaming kernel takes: E floats a row for two buffers (first), then `buffers`
// buffers of two T x (D + 4) tiles.
constexpr int64_t stream_lds_floats(int64_t T, int64_t D, int64_t E, int64_t buffers = 2) {
  return 2 * E * T + buffers * 2 * T * (D + 4);
}

// The forward, in one pass over the keys (online softmax): per tile, the scores of the wave's 16
// queries against the tile's unmasked keys raise the running maximum m; the running sum l and
// output O are rescaled by exp(m_old - m_new); P = exp(s - m) feeds the P V MFMA and l. Saves m
// and l (the sum relative to the final maximum) per query for the backward.
template <int D, int T, int W, int KS = 1>
__global__ __launch_bounds__(64 * W) void k_attn_fwd_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, const float* __restrict__ mask,
                                                       float* __restrict__ o, float* __restrict__ stats, int L, int S,
                                                       int H, int heads, float scale) {
  constexpr int DP = D + 4, U = T / 16 / KS;
  static_assert(T % (16 * KS) == 0, "a wave's share of a tile is whole 16-row tiles");
  extern __shared__ float sm[];
  float* const Mb = sm;                    // Mb + j T (first: a one-tile launch has one tile buffer)
  float* const Kb = sm + 2 * T;            // buffer j: Kb + j 2 T DP
  float* const Vb = Kb + T * DP;           // Vb + j 2 T DP
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t kbase = int64_t(b) * S * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  // KS waves share a query tile, each taking rows [half U 16, (half + 1) U 16) of every key tile.
  const int half = wave % KS;
  const int i0 = blockIdx.y * (16 * W / KS) + (wave / KS) * 16;
  const bool active = i0 < L;
  const int64_t qrow = (int64_t(b) * L + (active ? i0 : 0) + c) * H + head * D;
  float qb[D / 4];
#pragma unroll
  for (int t = 0; t < D / 4; ++t) qb[t] = q[qrow + 4 * t + g];
  const float* mrow = mask + int64_t(b) * S;
  constexpr int NT = 64 * W, PT = tile_groups<D, T, NT>();
  static_assert(NT >= T, "a thread a row of the mask");
  const int ntiles = (S + T - 1) / T;
  const int tid = int(threadIdx.x);
  {
    v4f kv[PT], vv[PT];
    fetch_pair<D, T, NT>(kv, vv, k + kbase, v + kbase, H, S < T ? S : T);
    const float mv = tid < T ? mrow[tid < S ? tid : S - 1] : 0.0f;
    put_pair<D, T, NT>(Kb, Vb, kv, vv);
    if (tid < T) Mb[tid] = mv;
  }
  __syncthreads();
  float m = -INFINITY, l = 0.0f;
  v4f oacc[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) oacc[ct] = v4f{0, 0, 0, 0};
  for (int t = 0; t < ntiles; ++t) {
    const int j = t & 1, s0 = t * T, n = S - s0 < T ? S - s0 : T;
    const bool more = t + 1 < ntiles;
    v4f kv[PT], vv[PT];
    float mv = 0.0f;
    if (more) {
      const int s1 = s0 + T, n1 = S - s1 < T ? S - s1 : T;
      fetch_pair<D, T, NT>(kv, vv, k + kbase + int64_t(s1) * H, v + kbase + int64_t(s1) * H, H, n1);
      if (tid < T) mv = mrow[s1 + (tid < n1 ? tid : n1 - 1)];
    }
    const int nt = KS == 1 ? n / 16 : std::min(U, n / 16 - half * U);
    if (active && nt > 0) {
      const float* Ks = Kb + j * 2 * T * DP + half * U * 16 * DP;
      const float* Vs = Vb + j * 2 * T * DP + half * U * 16 * DP;
      const float* Ms = Mb + j * T + half * U * 16;
      v4f acc[U];
      score_tiles<D, U>(Ks, qb, nt, c, g, acc);
      float tmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (u < nt && Ms[16 * u + 4 * g + r] != 0.0f) tmax = fmaxf(tmax, acc[u][r] * scale);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mn = fmaxf(m, tmax);
      // No unmasked key yet (mn = -inf): nothing has accumulated, nothing to rescale.
      const float alpha = mn == -INFINITY ? 1.0f : expf(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) oacc[ct][r] *= ar;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u >= nt) break;
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = Ms[16 * u + 4 * g + r] != 0.0f ? expf(acc[u][r] * scale - m) : 0.0f;
          l += p[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* vr = Vs + (16 * u + 4 * g + r) * DP + c;
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) oacc[ct] = mfma4(p[r], vr[ct * 16], oacc[ct]);
        }
      }
    }
    if (more) {
      put_pair<D, T, NT>(Kb + (j ^ 1) * 2 * T * DP, Vb + (j ^ 1) * 2 * T * DP, kv, vv);
      if (tid < T) Mb[(j ^ 1) * T + tid] = mv;
    }
    __syncthreads();
  }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if constexpr (KS > 1) {
    // The group's other waves hand their maximum, sum and output rows over through LDS (the tiles
    // are done with: the loop ended on a barrier); the first rescales them all to the largest
    // maximum and adds them in wave order.
    constexpr int CB = 32 + 16 * D;
    float* cb = sm + (wave / KS) * (KS - 1) * CB;
    if (half > 0 && active) {
      float* mine = cb + (half - 1) * CB;
      if (g == 0) {
        mine[c] = m;
        mine[16 + c] = l;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) mine[32 + (4 * g + r) * D + 16 * ct + c] = oacc[ct][r];
    }
    __syncthreads();
    if (half > 0 || !active) return;
    float mn = m;
#pragma unroll
    for (int h = 0; h < KS - 1; ++h) mn = fmaxf(mn, cb[h * CB + c]);
    const float a0 = m == -INFINITY ? 0.0f : expf(m - mn);
    l *= a0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float b0 = __shfl(a0, 4 * g + r, 64);
#pragma unroll
      for (int ct = 0; ct < D / 16; ++ct) oacc[ct][r] *= b0;
    }
#pragma unroll
    for (int h = 0; h < KS - 1; ++h) {
      const float* th = cb + h * CB;
      const float m1 = th[c], a1 = m1 == -INFINITY ? 0.0f : expf(m1 - mn);
      l += th[16 + c] * a1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float b1 = __shfl(a1, 4 * g + r, 64);
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) oacc[ct][r] += th[32 + (4 * g + r) * D + 16 * ct + c] * b1;
      }
    }
    m = mn;
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float row_total = __shfl(l, 4 * g + r, 64);
    const int64_t orow = (int64_t(b) * L + i0 + 4 * g + r) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) o[orow + ct * 16 + c] = oacc[ct][r] / row_total;
  }
  if (stats && g == 0) {
    const int64_t at = (int64_t(blockIdx.x) * L + i0 + c) * 2;
    stats[at] = m;
    stats[at + 1] = l;
  }
}

// The forward for rows of 128 keys and 64-wide heads (BERT-tiny's attention), with its operands in
// registers: a block is KS waves on one 16-query tile, each taking 128 / KS of the keys. Every
// operand goes from global memory straight into MFMA operand registers by 16-byte loads, all
// issued at the start, so no LDS staging or barrier precedes the MFMA chains. The contraction
// over d runs in the order d = 16 g + t (lane group g holds columns 16 g .. 16 g + 15 of its key
// and query rows), and output column 4 c + ct is lane c's ct-th accumulator, so a lane's values
// and its stores are four consecutive columns. The waves' maxima, sums and outputs combine
// through LDS in wave order, rescaled to the largest maximum, as k_attn_fwd_mfma's do.
template <int KS>
__global__ __launch_bounds__(64 * KS) void k_attn_fwd_reg(const float* __restrict__ q, const float* __restrict__ k,
                                                        const float* __restrict__ v, const float* __restrict__ mask,
                                                        float* __restrict__ o, float* __restrict__ stats, int L, int H,
                                                        int heads, float scale) {
  constexpr int D = 64, S = 128, U = S / 16 / KS, CB = 32 + 16 * D;
  __shared__ float cb[(KS - 1) * CB];
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int i0 = blockIdx.y * 16, key0 = wave * (S / KS);
  const int64_t kbase = int64_t(b) * S * H + head * D;
  v4f qv[4], kv[U][4], vv[U][4], mv[U];
  const float* qr = q + (int64_t(b) * L + i0 + c) * H + head * D + 16 * g;
#pragma unroll
  for (int t4 = 0; t4 < 4; ++t4) qv[t4] = *reinterpret_cast<const v4f*>(qr + 4 * t4);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float* kr = k + kbase + int64_t(key0 + 16 * u + c) * H + 16 * g;
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) kv[u][t4] = *reinterpret_cast<const v4f*>(kr + 4 * t4);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    mv[u] = *reinterpret_cast<const v4f*>(mask + int64_t(b) * S + key0 + 16 * u + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      vv[u][r] = *reinterpret_cast<const v4f*>(v + kbase + int64_t(key0 + 16 * u + 4 * g + r) * H + 4 * c);
  }
  // Every load is issued before any is waited for (otherwise the scheduler spreads them between
  // the MFMAs, one round trip each): the empty asm takes each register as its operand.
#pragma unroll
  for (int t4 = 0; t4 < 4; ++t4) asm volatile("" : "+v"(qv[t4]));
#pragma unroll
  for (int u = 0; u < U; ++u) {
    asm volatile("" : "+v"(mv[u]));
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) asm volatile("" : "+v"(kv[u][t4]), "+v"(vv[u][t4]));
  }
  // Scores: acc[u][r] = S[key key0 + 16 u + 4 g + r][query i0 + c].
  v4f acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = v4f{0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = mfma4(kv[u][t >> 2][t & 3], qv[t >> 2][t & 3], acc[u]);
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (mv[u][r] != 0.0f) m = fmaxf(m, acc[u][r] * scale);
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float l = 0.0f;
  v4f oacc[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) oacc[ct] = v4f{0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = mv[u][r] != 0.0f ? expf(acc[u][r] * scale - m) : 0.0f;
      l += p[r];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) oacc[ct] = mfma4(p[r], vv[u][r][ct], oacc[ct]);
  }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (wave > 0) {
    float* mine = cb + (wave - 1) * CB;
    if (g == 0) {
      mine[c] = m;
      mine[16 + c] = l;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) mine[32 + (4 * g + r) * D + 4 * c + ct] = oacc[ct][r];
  }
  __syncthreads();
  if (wave > 0) return;
  float mn = m;
#pragma unroll
  for (int h = 0; h < KS - 1; ++h) mn = fmaxf(mn, cb[h * CB + c]);
  const float a0 = m == -INFINITY ? 0.0f : expf(m - mn);
  l *= a0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float b0 = __shfl(a0, 4 * g + r, 64);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) oacc[ct][r] *= b0;
  }
#pragma unroll
  for (int h = 0; h < KS - 1; ++h) {
    const float* th = cb + h * CB;
    const float m1 = th[c], a1 = m1 == -INFINITY ? 0.0f : expf(m1 - mn);
    l += th[16 + c] * a1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float b1 = __shfl(a1, 4 * g + r, 64);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) oacc[ct][r] += th[32 + (4 * g + r) * D + 4 * c + ct] * b1;
    }
  }
  m = mn;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float row_total = __shfl(l, 4 * g + r, 64);
    const int64_t orow = (int64_t(b) * L + i0 + 4 * g + r) * H + head * D + 4 * c;
    *reinterpret_cast<v4f*>(o + orow) =
        v4f{oacc[0][r] / row_total, oacc[1][r] / row_total, oacc[2][r] / row_total, oacc[3][r] / row_total};
  }
  if (stats && g == 0) {
    const int64_t at = (int64_t(blockIdx.x) * L + i0 + c) * 2;
    stats[at] = m;
    stats[at + 1] = l;
  }
}

// dQ and d_i = rowsum(dO * O), per 16 query rows, streaming key and value tiles; `by` is the
// block's query-tile index (blockIdx.y of its own launch).
template <int D, int T, int W, int KS>
__device__ __forceinline__ void attn_bwd_q_body(const float* __restrict__ q, const float* __restrict__ k,
                                                const float* __restrict__ v, const float* __restrict__ mask,
                                                const float* __restrict__ o, const float* __restrict__ stats,
                                                const float* __restrict__ go, float* __restrict__ dq,
                                                float* __restrict__ dsum, int L, int S, int H, int heads, float scale,
                                                int by, float* sm) {
  constexpr int DP = D + 4, U = T / 16 / KS;
  static_assert(T % (16 * KS) == 0, "a wave's share of a tile is whole 16-row tiles");
  float* const Mb = sm;
  float* const Kb = sm + 2 * T;
  float* const Vb = Kb + T * DP;
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t kbase = int64_t(b) * S * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int half = wave % KS;  // KS waves share a query tile, each a share of every key tile
  const int i0 = by * (16 * W / KS) + (wave / KS) * 16;
  const bool active = i0 < L;
  const int64_t row = (int64_t(b) * L + (active ? i0 : 0) + c) * H + head * D;
  // d_i for query i0 + c: lane group g sums columns [g D/4, (g + 1) D/4).
  float dd = 0.0f;
#pragma unroll
  for (int t = 0; t < D / 16; ++t) {
    const v4f a = *reinterpret_cast<const v4f*>(go + row + g * (D / 4) + 4 * t);
    const v4f e = *reinterpret_cast<const v4f*>(o + row + g * (D / 4) + 4 * t);
#pragma unroll
    for (int u = 0; u < 4; ++u) dd = __builtin_fmaf(a[u], e[u], dd);
  }
  dd += __shfl_xor(dd, 16, 64);
  dd += __shfl_xor(dd, 32, 64);
  const int64_t srow = int64_t(blockIdx.x) * L + (active ? i0 : 0) + c;
  if (dsum && active && g == 0 && half == 0) dsum[srow] = dd;
  const float mx = stats[2 * srow], total = stats[2 * srow + 1];
  float qb[D / 4], gb[D / 4];
#pragma unroll
  for (int t = 0; t < D / 4; ++t) { qb[t] = q[row + 4 * t + g]; gb[t] = go[row + 4 * t + g]; }
  const float* mrow = mask + int64_t(b) * S;
  constexpr int NT = 64 * W, PT = tile_groups<D, T, NT>();
  static_assert(NT >= T, "a thread a row of the mask");
  const int ntiles = (S + T - 1) / T;
  const int tid = int(threadIdx.x);
  {
    v4f kv[PT], vv[PT];
    fetch_pair<D, T, NT>(kv, vv, k + kbase, v + kbase, H, S < T ? S : T);
    const float mv = tid < T ? mrow[tid < S ? tid : S - 1] : 0.0f;
    put_pair<D, T, NT>(Kb, Vb, kv, vv);
    if (tid < T) Mb[tid] = mv;
  }
  __syncthreads();
  v4f acc[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) acc[ct] = v4f{0, 0, 0, 0};
  for (int t = 0; t < ntiles; ++t) {
    const int j = t & 1, s0 = t * T, n = S - s0 < T ? S - s0 : T;
    const bool more = t + 1 < ntiles;
    v4f kv[PT], vv[PT];
    float mv = 0.0f;
    if (more) {
      const int s1 = s0 + T, n1 = S - s1 < T ? S - s1 : T;
      fetch_pair<D, T, NT>(kv, vv, k + kbase + int64_t(s1) * H, v + kbase + int64_t(s1) * H, H, n1);
      if (tid < T) mv = mrow[s1 + (tid < n1 ? tid : n1 - 1)];
    }
    const int nt = KS == 1 ? n / 16 : std::min(U, n / 16 - half * U);
    if (active && nt > 0) {
      const float* Ks = Kb + j * 2 * T * DP + half * U * 16 * DP;
      const float* Vs = Vb + j * 2 * T * DP + half * U * 16 * DP;
      const float* Ms = Mb + j * T + half * U * 16;
      v4f st[U], dpt[U];
      score_tiles<D, U>(Ks, qb, nt, c, g, st);
      score_tiles<D, U>(Vs, gb, nt, c, g, dpt);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u >= nt) break;
        float ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = Ms[16 * u + 4 * g + r] != 0.0f ? expf(st[u][r] * scale - mx) / total : 0.0f;
          ds[r] = p * (dpt[u][r] - dd);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* kk = Ks + (16 * u + 4 * g + r) * DP + c;
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) acc[ct] = mfma4(ds[r], kk[ct * 16], acc[ct]);
        }
      }
    }
    if (more) {
      put_pair<D, T, NT>(Kb + (j ^ 1) * 2 * T * DP, Vb + (j ^ 1) * 2 * T * DP, kv, vv);
      if (tid < T) Mb[(j ^ 1) * T + tid] = mv;
    }
    __syncthreads();
  }
  if constexpr (KS > 1) {
    // The group's partial dQ, added in wave order.
    float* cb = sm + (wave / KS) * (KS - 1) * (16 * D);
    if (half > 0 && active)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) cb[(half - 1) * 16 * D + (4 * g + r) * D + 16 * ct + c] = acc[ct][r];
    __syncthreads();
    if (half > 0) return;
    if (active)
#pragma unroll
      for (int h = 0; h < KS - 1; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) acc[ct][r] += cb[h * 16 * D + (4 * g + r) * D + 16 * ct + c];
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t orow = (int64_t(b) * L + i0 + 4 * g + r) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) dq[orow + ct * 16 + c] = acc[ct][r] * scale;
  }
}
template <int D, int T, int W, int KS = 1>
__global__ __launch_bounds__(64 * W) void k_attn_bwd_q_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, const float* __restrict__ mask,
                                                         const float* __restrict__ o, const float* __restrict__ stats,
                                                         const float* __restrict__ go, float* __restrict__ dq,
                                                         float* __restrict__ dsum, int L, int S, int H, int heads,
                                                         float scale) {
  extern __shared__ float sm[];
  attn_bwd_q_body<D, T, W, KS>(q, k, v, mask, o, stats, go, dq, dsum, L, S, H, heads, scale, int(blockIdx.y), sm);
}

// dK and dV, per 16 key rows, streaming query and output-gradient tiles (with each query's
// maximum, sum and d). d is read from dsum, or, when dsum is null, formed here from dO and O in
// the dQ pass's order (so the two passes can run in one launch); `by` is the block's key-tile
// index.
template <int D, int T, int W, int KS>
__device__ __forceinline__ void attn_bwd_kv_body(const float* __restrict__ q, const float* __restrict__ k,
                                                 const float* __restrict__ v, const float* __restrict__ mask,
                                                 const float* __restrict__ o, const float* __restrict__ stats,
                                                 const float* __restrict__ go, const float* __restrict__ dsum,
                                                 float* __restrict__ dk, float* __restrict__ dv, int L, int S, int H,
                                                 int heads, float scale, int by, float* sm) {
  constexpr int DP = D + 4, U = T / 16 / KS;
  static_assert(T % (16 * KS) == 0, "a wave's share of a tile is whole 16-row tiles");
  float* const Sb = sm;  // max, sum, d per query of the tile; buffer j at Sb + j 3 T
  float* const Qb = sm + 6 * T;
  float* const Gb = Qb + T * DP;
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t qbase = int64_t(b) * L * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int half = wave % KS;  // KS waves share a key tile, each a share of every query tile
  const int j0 = by * (16 * W / KS) + (wave / KS) * 16;
  const bool active = j0 < S;
  const int64_t krow = (int64_t(b) * S + (active ? j0 : 0) + c) * H + head * D;
  const bool live = mask[int64_t(b) * S + (active ? j0 : 0) + c] != 0.0f;
  float kb[D / 4], vb[D / 4];
#pragma unroll
  for (int t = 0; t < D / 4; ++t) { kb[t] = k[krow + 4 * t + g]; vb[t] = v[krow + 4 * t + g]; }
  const int64_t sbase = int64_t(blockIdx.x) * L;
  constexpr int NT = 64 * W, PT = tile_groups<D, T, NT>();
  static_assert(NT >= T, "a thread a row of the statistics");
  const int ntiles = (L + T - 1) / T;
  const int tid = int(threadIdx.x);
  // The maximum and sum of query l0 + row (row clamped to the n rows of the tile), and its d: read
  // from dsum, or formed as the dQ pass forms it (four sequential fma chains over a quarter of the
  // columns each, then (p0 + p1) + (p2 + p3)), here by four neighbouring lanes a query, one chain
  // each on 16-byte loads, combined by two lane swaps (the sums are symmetric, so every lane of
  // the four holds the same value).
  constexpr int PD = (4 * T + NT - 1) / NT;
  auto fetch_stats = [&](float (&e)[2 + PD], int l0, int n) {
    if (tid < T) {
      const int64_t at = sbase + l0 + (tid < n ? tid : n - 1);
      e[0] = stats[2 * at];
      e[1] = stats[2 * at + 1];
    }
#pragma unroll
    for (int pd = 0; pd < PD; ++pd) {
      const int it = tid + NT * pd, rr = it >> 2, gg = it & 3;
      float a = 0.0f;
      if (dsum) {
        if (gg == 0 && rr < T) a = dsum[sbase + l0 + (rr < n ? rr : n - 1)];
      } else if (4 * T % NT == 0 || rr < T) {
        const int64_t qrow = qbase + int64_t(l0 + (rr < n ? rr : n - 1)) * H + gg * (D / 4);
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
          const v4f x = *reinterpret_cast<const v4f*>(go + qrow + 4 * t);
          const v4f y = *reinterpret_cast<const v4f*>(o + qrow + 4 * t);
#pragma unroll
          for (int u = 0; u < 4; ++u) a = __builtin_fmaf(x[u], y[u], a);
        }
        a += __shfl_xor(a, 1, 64);
        a += __shfl_xor(a, 2, 64);
      }
      e[2 + pd] = a;
    }
  };
  auto put_stats = [&](float* X, const float (&e)[2 + PD]) {
    if (tid < T) {
      X[3 * tid] = e[0];
      X[3 * tid + 1] = e[1];
    }
#pragma unroll
    for (int pd = 0; pd < PD; ++pd) {
      const int it = tid + NT * pd;
      if ((it & 3) == 0 && (it >> 2) < T) X[3 * (it >> 2) + 2] = e[2 + pd];
    }
  };
  {
    v4f qv[PT], gv[PT];
    float e[2 + PD] = {};
    fetch_pair<D, T, NT>(qv, gv, q + qbase, go + qbase, H, L < T ? L : T);
    fetch_stats(e, 0, L < T ? L : T);
    put_pair<D, T, NT>(Qb, Gb, qv, gv);
    put_stats(Sb, e);
  }
  __syncthreads();
  v4f dka[D / 16], dva[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) { dka[ct] = v4f{0, 0, 0, 0}; dva[ct] = v4f{0, 0, 0, 0}; }
  for (int t = 0; t < ntiles; ++t) {
    const int j = t & 1, l0 = t * T, n = L - l0 < T ? L - l0 : T;
    const bool more = t + 1 < ntiles;
    v4f qv[PT], gv[PT];
    float e[2 + PD] = {};
    if (more) {
      const int l1 = l0 + T, n1 = L - l1 < T ? L - l1 : T;
      fetch_pair<D, T, NT>(qv, gv, q + qbase + int64_t(l1) * H, go + qbase + int64_t(l1) * H, H, n1);
      fetch_stats(e, l1, n1);
    }
    const int nt = KS == 1 ? n / 16 : std::min(U, n / 16 - half * U);
    if (active && nt > 0) {
      const float* Qs = Qb + j * 2 * T * DP + half * U * 16 * DP;
      const float* Gs = Gb + j * 2 * T * DP + half * U * 16 * DP;
      const float* Ss = Sb + j * 3 * T + half * U * 16 * 3;
      v4f s[U], dp[U];
      score_tiles<D, U>(Qs, kb, nt, c, g, s);
      score_tiles<D, U>(Gs, vb, nt, c, g, dp);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u >= nt) break;
        float p[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* st = Ss + 3 * (16 * u + 4 * g + r);
          p[r] = live ? expf(s[u][r] * scale - st[0]) / st[1] : 0.0f;
          ds[r] = p[r] * (dp[u][r] - st[2]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* gq = Gs + (16 * u + 4 * g + r) * DP + c;
          const float* qq = Qs + (16 * u + 4 * g + r) * DP + c;
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) {
            dva[ct] = mfma4(p[r], gq[ct * 16], dva[ct]);
            dka[ct] = mfma4(ds[r], qq[ct * 16], dka[ct]);
          }
        }
      }
    }
    if (more) {
      put_pair<D, T, NT>(Qb + (j ^ 1) * 2 * T * DP, Gb + (j ^ 1) * 2 * T * DP, qv, gv);
      put_stats(Sb + (j ^ 1) * 3 * T, e);
    }
    __syncthreads();
  }
  if constexpr (KS > 1) {
    // The group's partial dK and dV, added in wave order.
    float* cb = sm + (wave / KS) * (KS - 1) * (32 * D);
    if (half > 0 && active)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) {
          cb[(half - 1) * 32 * D + (4 * g + r) * D + 16 * ct + c] = dka[ct][r];
          cb[(half - 1) * 32 * D + 16 * D + (4 * g + r) * D + 16 * ct + c] = dva[ct][r];
        }
    __syncthreads();
    if (half > 0) return;
    if (active)
#pragma unroll
      for (int h = 0; h < KS - 1; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int ct = 0; ct < D / 16; ++ct) {
            dka[ct][r] += cb[h * 32 * D + (4 * g + r) * D + 16 * ct + c];
            dva[ct][r] += cb[h * 32 * D + 16 * D + (4 * g + r) * D + 16 * ct + c];
          }
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int jj = j0 + 4 * g + r;
    const bool keep = mask[int64_t(b) * S + jj] != 0.0f;
    const int64_t orow = (int64_t(b) * S + jj) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) {
      if (dv) dv[orow + ct * 16 + c] = keep ? dva[ct][r] : 0.0f;
      if (dk) dk[orow + ct * 16 + c] = keep ? dka[ct][r] * scale : 0.0f;
    }
  }
}
template <int D, int T, int W, int KS = 1>
__global__ __launch_bounds__(64 * W) void k_attn_bwd_kv_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, const float* __restrict__ mask,
                                                          const float* __restrict__ stats, const float* __restrict__ go,
                                                          const float* __restrict__ dsum, float* __restrict__ dk,
                                                          float* __restrict__ dv, int L, int S, int H, int heads,
                                                          float scale) {
  extern __shared__ float sm[];
  attn_bwd_kv_body<D, T, W, KS>(q, k, v, mask, nullptr, stats, go, dsum, dk, dv, L, S, H, heads, scale,
                                int(blockIdx.y), sm);
}
// Both backward passes in one launch (self-attention, one plan for both): blocks with
// blockIdx.y < qy take query tiles (dQ), the rest key tiles (dK, dV, forming each query's d
// themselves), so that the two passes' blocks share the chip instead of each leaving most of it
// idle in turn.
template <int D, int T, int W, int KS = 1>
__global__ __launch_bounds__(64 * W, 2) void k_attn_bwd_mfma(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, const float* __restrict__ mask,
                                                       const float* __restrict__ o, const float* __restrict__ stats,
                                                       const float* __restrict__ go, float* __restrict__ dq,
                                                       float* __restrict__ dk, float* __restrict__ dv, int L, int S,
                                                       int H, int heads, float scale, int qy) {
  extern __shared__ float sm[];
  if (int(blockIdx.y) < qy)
    attn_bwd_q_body<D, T, W, KS>(q, k, v, mask, o, stats, go, dq, nullptr, L, S, H, heads, scale, int(blockIdx.y), sm);
  else
    attn_bwd_kv_body<D, T, W, KS>(q, k, v, mask, o, stats, go, nullptr, dk, dv, L, S, H, heads, scale,
                                  int(blockIdx.y) - qy, sm);
}

// ---------------------------------------------------------------------------------------------
// Mixed precision: the same kernels with their QK^T, P V, dS K, P^T dO and dS^T Q contractions on
// the f16 MFMA (v_mfma_f32_16x16x16f16, f32 accumulation). Its lane layout is the f32 one's with four
// consecutive K values a lane group (K 4g .. 4g + 3 where the f32 instruction has K = g): the four
// probabilities (or dS values) a lane holds after a score MFMA, keys 4g + r of a 16-key tile, are
// the A operand of the next contraction as they stand, and that contraction's B operand is read
// from a transposed f16 copy of its tile (8 bytes a lane). Tiles are staged from f32 into f16 LDS
// tiles: row-major (row stride D + 8 halves) for score operands, transposed (row stride T + 8)
// for the others. Softmax statistics, exp and the running sums stay f32.
namespace {
__device__ __forceinline__ v4f mfma16h(v4h a, v4h b, v4f c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ v4h to_h4(float a, float b, float c, float d) {
  return v4h{_Float16(a), _Float16(b), _Float16(c), _Float16(d)};
}
}  // namespace

// Rows 0 .. T of a fetched tile (fetch_pair's registers) into a row-major f16 tile (row stride KP)
// and, when Xt is non-null, a transposed one (row stride VP: column d of the tile is row d).
template <int D, int T, int NT, int PT>
__device__ __forceinline__ void put_h(_Float16* Xr, _Float16* Xt, const v4f (&xv)[PT]) {
  constexpr int KP = D + 8, VP = T + 8, Q = D / 4, G = T * Q;
#pragma unroll
  for (int p = 0; p < PT; ++p) {
    const int e = int(threadIdx.x) + NT * p;
    if (G % NT == 0 || e < G) {
      const int row = e / Q, col = (e % Q) * 4;
      const v4f x = xv[p];
      if (Xr) *reinterpret_cast<v4h*>(Xr + row * KP + col) = to_h4(x[0], x[1], x[2], x[3]);
      if (Xt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) Xt[(col + j) * VP + row] = _Float16(x[j]);
      }
    }
  }
}

// f16 scores of U tiles of 16 rows of the row-major tile R against the 16 rows whose fragments xh
// a lane holds: acc[u][r] = sum over d of R[16 u + 4 g + r][d] x[c][d] (the f32 score_tiles' layout).
template <int D, int U>
__device__ __forceinline__ void score_tiles_h(const _Float16* R, const v4h (&xh)[D / 16], int nt, int c, int g,
                                              v4f (&acc)[U]) {
  constexpr int KP = D + 8;
  const _Float16* rr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    acc[u] = v4f{0, 0, 0, 0};
    rr[u] = R + (16 * (u < nt ? u : nt - 1) + c) * KP + 4 * g;
  }
#pragma unroll
  for (int t = 0; t < D / 16; ++t)
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = mfma16h(*reinterpret_cast<const v4h*>(rr[u] + 16 * t), xh[t], acc[u]);
}

// A row's D values at x as the f16 B fragments of a score MFMA: xh[t] = x[16 t + 4 g .. + 3].
template <int D>
__device__ __forceinline__ void row_fragments_h(const float* __restrict__ x, int g, v4h (&xh)[D / 16]) {
#pragma unroll
  for (int t = 0; t < D / 16; ++t) {
    const v4f f = *reinterpret_cast<const v4f*>(x + 16 * t + 4 * g);
    xh[t] = to_h4(f[0], f[1], f[2], f[3]);
  }
}

template <int D, int T>
constexpr int h16_lds_bytes(int row_tiles, int col_tiles, int extras) {
  return 2 * (row_tiles * T * (D + 8) + col_tiles * D * (T + 8)) * 2 + 2 * extras * T * 4;
}

template <int D, int T, int W>
__global__ __launch_bounds__(64 * W) void k_attn_fwd_h16(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, const float* __restrict__ mask,
                                                         float* __restrict__ o, float* __restrict__ stats, int L, int S,
                                                         int H, int heads, float scale) {
  constexpr int KP = D + 8, VP = T + 8, U = T / 16, NT = 64 * W, PT = tile_groups<D, T, NT>();
  static_assert(NT >= T, "a thread a row of the mask");
  extern __shared__ float sm[];
  _Float16* const Kh = reinterpret_cast<_Float16*>(sm);  // buffer j: + j T KP
  _Float16* const Vt = Kh + 2 * T * KP;                     // buffer j: + j D VP
  float* const Mb = reinterpret_cast<float*>(Vt + 2 * D * VP);
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t kbase = int64_t(b) * S * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int i0 = blockIdx.y * (16 * W) + wave * 16;
  const bool active = i0 < L;
  v4h qh[D / 16];
  row_fragments_h<D>(q + (int64_t(b) * L + (active ? i0 : 0) + c) * H + head * D, g, qh);
  const float* mrow = mask + int64_t(b) * S;
  const int ntiles = (S + T - 1) / T, tid = int(threadIdx.x);
  {
    v4f kv[PT], vv[PT];
    fetch_pair<D, T, NT>(kv, vv, k + kbase, v + kbase, H, S < T ? S : T);
    const float mv = tid < T ? mrow[tid < S ? tid : S - 1] : 0.0f;
    put_h<D, T, NT>(Kh, nullptr, kv);
    put_h<D, T, NT>(nullptr, Vt, vv);
    if (tid < T) Mb[tid] = mv;
  }
  __syncthreads();
  float m = -INFINITY, l = 0.0f;
  v4f oacc[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) oacc[ct] = v4f{0, 0, 0, 0};
  for (int t = 0; t < ntiles; ++t) {
    const int j = t & 1, s0 = t * T, n = S - s0 < T ? S - s0 : T;
    const bool more = t + 1 < ntiles;
    v4f kv[PT], vv[PT];
    float mv = 0.0f;
    if (more) {
      const int s1 = s0 + T, n1 = S - s1 < T ? S - s1 : T;
      fetch_pair<D, T, NT>(kv, vv, k + kbase + int64_t(s1) * H, v + kbase + int64_t(s1) * H, H, n1);
      if (tid < T) mv = mrow[s1 + (tid < n1 ? tid : n1 - 1)];
    }
    if (active) {
      const _Float16* Ks = Kh + j * T * KP;
      const _Float16* Vs = Vt + j * D * VP;
      const float* Ms = Mb + j * T;
      const int nt = n / 16;
      v4f acc[U];
      score_tiles_h<D, U>(Ks, qh, nt, c, g, acc);
      float tmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (u < nt && Ms[16 * u + 4 * g + r] != 0.0f) tmax = fmaxf(tmax, acc[u][r] * scale);
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mn = fmaxf(m, tmax);
      const float alpha = mn == -INFINITY ? 1.0f : expf(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) oacc[ct][r] *= ar;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u >= nt) break;
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = Ms[16 * u + 4 * g + r] != 0.0f ? expf(acc[u][r] * scale - m) : 0.0f;
          l += p[r];
        }
        const v4h ph = to_h4(p[0], p[1], p[2], p[3]);
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct)
          oacc[ct] = mfma16h(ph, *reinterpret_cast<const v4h*>(Vs + (16 * ct + c) * VP + 16 * u + 4 * g), oacc[ct]);
      }
    }
    if (more) {
      put_h<D, T, NT>(Kh + (j ^ 1) * T * KP, nullptr, kv);
      put_h<D, T, NT>(nullptr, Vt + (j ^ 1) * D * VP, vv);
      if (tid < T) Mb[(j ^ 1) * T + tid] = mv;
    }
    __syncthreads();
  }
  if (!active) return;
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float row_total = __shfl(l, 4 * g + r, 64);
    const int64_t orow = (int64_t(b) * L + i0 + 4 * g + r) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) o[orow + ct * 16 + c] = oacc[ct][r] / row_total;
  }
  if (stats && g == 0) {
    const int64_t at = (int64_t(blockIdx.x) * L + i0 + c) * 2;
    stats[at] = m;
    stats[at + 1] = l;
  }
}

template <int D, int T, int W>
__global__ __launch_bounds__(64 * W) void k_attn_bwd_q_h16(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, const float* __restrict__ mask,
                                                           const float* __restrict__ o, const float* __restrict__ stats,
                                                           const float* __restrict__ go, float* __restrict__ dq,
                                                           float* __restrict__ dsum, int L, int S, int H, int heads,
                                                           float scale) {
  constexpr int KP = D + 8, VP = T + 8, U = T / 16, NT = 64 * W, PT = tile_groups<D, T, NT>();
  static_assert(NT >= T, "a thread a row of the mask");
  extern __shared__ float sm[];
  _Float16* const Kh = reinterpret_cast<_Float16*>(sm);  // keys, row-major; buffer j: + j T KP
  _Float16* const Vh = Kh + 2 * T * KP;                    // values, row-major
  _Float16* const Kt = Vh + 2 * T * KP;                    // keys, transposed; buffer j: + j D VP
  float* const Mb = reinterpret_cast<float*>(Kt + 2 * D * VP);
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t kbase = int64_t(b) * S * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int i0 = blockIdx.y * (16 * W) + wave * 16;
  const bool active = i0 < L;
  const int64_t row = (int64_t(b) * L + (active ? i0 : 0) + c) * H + head * D;
  float dd = 0.0f;
#pragma unroll
  for (int t = 0; t < D / 16; ++t) {
    const v4f a = *reinterpret_cast<const v4f*>(go + row + g * (D / 4) + 4 * t);
    const v4f e = *reinterpret_cast<const v4f*>(o + row + g * (D / 4) + 4 * t);
#pragma unroll
    for (int u = 0; u < 4; ++u) dd = __builtin_fmaf(a[u], e[u], dd);
  }
  dd += __shfl_xor(dd, 16, 64);
  dd += __shfl_xor(dd, 32, 64);
  const int64_t srow = int64_t(blockIdx.x) * L + (active ? i0 : 0) + c;
  if (active && g == 0) dsum[srow] = dd;
  const float mx = stats[2 * srow], total = stats[2 * srow + 1];
  v4h qh[D / 16], gh[D / 16];
  row_fragments_h<D>(q + row, g, qh);
  row_fragments_h<D>(go + row, g, gh);
  const float* mrow = mask + int64_t(b) * S;
  const int ntiles = (S + T - 1) / T, tid = int(threadIdx.x);
  {
    v4f kv[PT], vv[PT];
    fetch_pair<D, T, NT>(kv, vv, k + kbase, v + kbase, H, S < T ? S : T);
    const float mv = tid < T ? mrow[tid < S ? tid : S - 1] : 0.0f;
    put_h<D, T, NT>(Kh, Kt, kv);
    put_h<D, T, NT>(Vh, nullptr, vv);
    if (tid < T) Mb[tid] = mv;
  }
  __syncthreads();
  v4f acc[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) acc[ct] = v4f{0, 0, 0, 0};
  for (int t = 0; t < ntiles; ++t) {
    const int j = t & 1, s0 = t * T, n = S - s0 < T ? S - s0 : T;
    const bool more = t + 1 < ntiles;
    v4f kv[PT], vv[PT];
    float mv = 0.0f;
    if (more) {
      const int s1 = s0 + T, n1 = S - s1 < T ? S - s1 : T;
      fetch_pair<D, T, NT>(kv, vv, k + kbase + int64_t(s1) * H, v + kbase + int64_t(s1) * H, H, n1);
      if (tid < T) mv = mrow[s1 + (tid < n1 ? tid : n1 - 1)];
    }
    if (active) {
      const _Float16* Ks = Kh + j * T * KP;
      const _Float16* Vs = Vh + j * T * KP;
      const _Float16* Kts = Kt + j * D * VP;
      const float* Ms = Mb + j * T;
      const int nt = n / 16;
      v4f st[U], dpt[U];
      score_tiles_h<D, U>(Ks, qh, nt, c, g, st);
      score_tiles_h<D, U>(Vs, gh, nt, c, g, dpt);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u >= nt) break;
        float ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = Ms[16 * u + 4 * g + r] != 0.0f ? expf(st[u][r] * scale - mx) / total : 0.0f;
          ds[r] = p * (dpt[u][r] - dd);
        }
        const v4h dh = to_h4(ds[0], ds[1], ds[2], ds[3]);
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct)
          acc[ct] = mfma16h(dh, *reinterpret_cast<const v4h*>(Kts + (16 * ct + c) * VP + 16 * u + 4 * g), acc[ct]);
      }
    }
    if (more) {
      put_h<D, T, NT>(Kh + (j ^ 1) * T * KP, Kt + (j ^ 1) * D * VP, kv);
      put_h<D, T, NT>(Vh + (j ^ 1) * T * KP, nullptr, vv);
      if (tid < T) Mb[(j ^ 1) * T + tid] = mv;
    }
    __syncthreads();
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t orow = (int64_t(b) * L + i0 + 4 * g + r) * H + head * D;
#pragma unroll
    for (int ct = 0; ct < D / 16; ++ct) dq[orow + ct * 16 + c] = acc[ct][r] * scale;
  }
}

template <int D, int T, int W>
__global__ __launch_bounds__(64 * W) void k_attn_bwd_kv_h16(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v, const float* __restrict__ mask,
                                                            const float* __restrict__ stats, const float* __restrict__ go,
                                                            const float* __restrict__ dsum, float* __restrict__ dk,
                                                            float* __restrict__ dv, int L, int S, int H, int heads,
                                                            float scale) {
  constexpr int KP = D + 8, VP = T + 8, U = T / 16, NT = 64 * W, PT = tile_groups<D, T, NT>();
  static_assert(NT >= T, "a thread a row of the statistics");
  extern __shared__ float sm[];
  _Float16* const Qh = reinterpret_cast<_Float16*>(sm);  // queries, row-major; buffer j: + j T KP
  _Float16* const Gh = Qh + 2 * T * KP;                    // output gradients, row-major
  _Float16* const Qt = Gh + 2 * T * KP;                    // queries, transposed; buffer j: + j D VP
  _Float16* const Gt = Qt + 2 * D * VP;                    // output gradients, transposed
  float* const Sb = reinterpret_cast<float*>(Gt + 2 * D * VP);  // max, sum, d a query; buffer j: + j 3 T
  const int b = blockIdx.x / heads, head = blockIdx.x % heads;
  const int64_t qbase = int64_t(b) * L * H + head * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int j0 = blockIdx.y * (16 * W) + wave * 16;
  const bool active = j0 < S;
  const int64_t krow = (int64_t(b) * S + (active ? j0 : 0) + c) * H + head * D;
  const bool live = mask[int64_t(b) * S + (active ? j0 : 0) + c] != 0.0f;
  v4h kh[D / 16], vh[D / 16];
  row_fragments_h<D>(k + krow, g, kh);
  row_fragments_h<D>(v + krow, g, vh);
  const int64_t sbase = int64_t(blockIdx.x) * L;
  const int ntiles = (L + T - 1) / T, tid = int(threadIdx.x);
  auto fetch_stats = [&](float (&e)[3], int l0, int n) {
    if (tid < T) {
      const int64_t at = sbase + l0 + (tid < n ? tid : n - 1);
      e[0] = stats[2 * at];
      e[1] = stats[2 * at + 1];
      e[2] = dsum[at];
    }
  };
  auto put_stats = [&](float* X, const float (&e)[3]) {
    if (tid < T) {
      X[3 * tid] = e[0];
      X[3 * tid + 1] = e[1];
      X[3 * tid + 2] = e[2];
    }
  };
  {
    v4f qv[PT], gv[PT];
    float e[3] = {0.0f, 0.0f, 0.0f};
    fetch_pair<D, T, NT>(qv, gv, q + qbase, go + qbase, H, L < T ? L : T);
    fetch_stats(e, 0, L < T ? L : T);
    put_h<D, T, NT>(Qh, Qt, qv);
    put_h<D, T, NT>(Gh, Gt, gv);
    put_stats(Sb, e);
  }
  __syncthreads();
  v4f dka[D / 16], dva[D / 16];
#pragma unroll
  for (int ct = 0; ct < D / 16; ++ct) { dka[ct] = v4f{0, 0, 0, 0}; dva[ct] = v4f{0, 0, 0, 0}; }
  for (int t = 0; t < ntiles; ++t) {
    const int j = t & 1, l0 = t * T, n = L - l0 < T ? L - l0 : T;
    const bool more = t + 1 < ntiles;
    v4f qv[PT], gv[PT];
    float e[3] = {0.0f, 0.0f, 0.0f};
    if (more) {
      const int l1 = l0 + T, n1 = L - l1 < T ? L - l1 : T;
      fetch_pair<D, T, NT>(qv, gv, q + qbase + int64_t(l1) * H, go + qbase + int64_t(l1) * H, H, n1);
      fetch_stats(e, l1, n1);
    }
    if (active) {
      const _Float16* Qs = Qh + j * T * KP;
      const _Float16* Gs = Gh + j * T * KP;
      const _Float16* Qts = Qt + j * D * VP;
      const _Float16* Gts = Gt + j * D * VP;
      const float* Ss = Sb + j * 3 * T;
      const int nt = n / 16;
      v4f s[U], dp[U];
      score_tiles_h<D, U>(Qs, kh, nt, c, g, s);
      score_tiles_h<D, U>(Gs, vh, nt, c, g, dp);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u >= nt) break;
        float p[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float* st = Ss + 3 * (16 * u + 4 * g + r);
          p[r] = live ? expf(s[u][r] * scale - st[0]) / st[1] : 0.0f;
          ds[r] = p[r] * (dp[u][r] - st[2]);
        }
        const v4h ph = to_h4(p[0], p[1], p[2], p[3]), dh = to_h4(ds[0], ds[1], ds[2], ds[3]);
#pragma unroll
        for (int ct = 0; ct < D / 16; ++ct) {
          const int at = (16 * ct + c) * VP + 16 * u + 4 * g;
          dva[ct] = mfma16h(ph, *reinterpret_cast<const v4h*>(Gts + at), dva[ct]);
          dka[ct] = mfma16h(dh, *reinterpret_cast<const v4h*>(Qts + at), dka[ct]);
        }
      }
    }
    if (more) {
      put_h<D, T, NT>(Qh + (j ^ 1) * T * KP, Qt + (j ^ 1) * D * VP, qv);
      put_h<D, T, NT>(Gh + (j ^ 1) * T * KP, Gt + (j ^ 1) * D * VP, gv);
      put_stats(Sb + (j ^ 1) * 3 * T, e);
    }
    __syncthreads();
  }
  if (!active) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int jj = j0 + 4 * g + r;
    const bool keep = mask[int64_t(b) * S + jj] != 0.0f;
    const int64_t orow = (int64_t(b) * S + jj) * H + head * D;
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
bool head_ok(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128; }
// The streaming shape, from measured MI355X timings: problems of 4096 or more 16-row wave tiles
// (BERT-base: 12288) take blocks of four waves and tiles of 32 rows (35 KB of LDS a block at
// D = 64, four blocks a CU); smaller ones (BERT-tiny: 512) blocks of two waves and tiles of 64
// rows (32 for D = 128), so that the few waves spread over more CUs with longer MFMA chains.
// ks: waves sharing a row tile (each a share of every streamed tile); one: the streamed side fits
// one tile, so one LDS buffer and no prefetch. Small problems whose streamed side is at most 128
// rows (BERT-tiny: 512 wave tiles on 1024 SIMDs) take one 128-row tile shared by two waves a row
// tile, twice the waves (f32 only; on BERT-tiny the backward pair went from 34 to 27 us a layer
// and the step from 0.955 to 0.935 ms; four waves a row tile in blocks of eight took the forward
// from 10.0 to 11.3 us and the backward from 21.3 to 32.4 us).
struct AttnPlan { int T, W, KS; bool one; };
AttnPlan attn_plan(int64_t bh, int64_t rows, int64_t streamed, int64_t d, bool h16) {
  const int64_t tiles = bh * ((rows + 15) / 16);
  AttnPlan p;
  if (tiles >= 4096) p = {32, 4, 1, false};
  else if (!h16 && streamed <= 128 && d <= 64) p = {128, 4, 2, false};
  else p = {d >= 128 ? 32 : 64, 2, 1, false};
  p.one = streamed <= p.T;
  return p;
}
unsigned row_blocks(int64_t rows, const AttnPlan& p) { return unsigned((rows + 16 * p.W / p.KS - 1) / (16 * p.W / p.KS)); }
template <int D, int T, int W, int KS>
void launch_fwd(hipStream_t s, dim3 grid, bool one, const float* q, const float* k, const float* v, const float* mask,
                float* o, float* stats, int L, int S, int H, int heads, float scale) {
  const size_t lds = size_t(stream_lds_floats(T, D, 1, one ? 1 : 2)) * 4;
  MSX_LAUNCH((k_attn_fwd_mfma<D, T, W, KS>), grid, dim3(64 * W), lds, s, q, k, v, mask, o, stats, L, S, H, heads, scale);
}
template <int D, int T, int W, int KS>
void launch_bwd_q(hipStream_t s, dim3 grid, bool one, const float* q, const float* k, const float* v, const float* mask,
                  const float* o, const float* stats, const float* g, float* dq, float* dsum, int L, int S, int H,
                  int heads, float scale) {
  const size_t lds = size_t(stream_lds_floats(T, D, 1, one ? 1 : 2)) * 4;
  MSX_LAUNCH((k_attn_bwd_q_mfma<D, T, W, KS>), grid, dim3(64 * W), lds, s, q, k, v, mask, o, stats, g, dq, dsum, L, S,
             H, heads, scale);
}
template <int D, int T, int W>
void launch_fwd_h(hipStream_t s, dim3 grid, const float* q, const float* k, const float* v, const float* mask,
                  float* o, float* stats, int L, int S, int H, int heads, float scale) {
  const size_t lds = size_t(h16_lds_bytes<D, T>(1, 1, 1));
  MSX_LAUNCH((k_attn_fwd_h16<D, T, W>), grid, dim3(64 * W), lds, s, q, k, v, mask, o, stats, L, S, H, heads, scale);
}
template <int D, int T, int W>
void launch_bwd_q_h(hipStream_t s, dim3 grid, const float* q, const float* k, const float* v, const float* mask,
                    const float* o, const float* stats, const float* g, float* dq, float* dsum, int L, int S, int H,
                    int heads, float scale) {
  const size_t lds = size_t(h16_lds_bytes<D, T>(2, 1, 1));
  MSX_LAUNCH((k_attn_bwd_q_h16<D, T, W>), grid, dim3(64 * W), lds, s, q, k, v, mask, o, stats, g, dq, dsum, L, S, H,
             heads, scale);
}
template <int D, int T, int W>
void launch_bwd_kv_h(hipStream_t s, dim3 grid, const float* q, const float* k, const float* v, const float* mask,
                     const float* stats, const float* g, const float* dsum, float* dk, float* dv, int L, int S, int H,
                     int heads, float scale) {
  const size_t lds = size_t(h16_lds_bytes<D, T>(2, 2, 3));
  MSX_LAUNCH((k_attn_bwd_kv_h16<D, T, W>), grid, dim3(64 * W), lds, s, q, k, v, mask, stats, g, dsum, dk, dv, L, S, H,
             heads, scale);
}
template <int D, int T, int W, int KS>
void launch_bwd_kv(hipStream_t s, dim3 grid, bool one, const float* q, const float* k, const float* v, const float* mask,
                   const float* stats, const float* g, const float* dsum, float* dk, float* dv, int L, int S, int H,
                   int heads, float scale) {
  const size_t lds = size_t(stream_lds_floats(T, D, 3, one ? 1 : 2)) * 4;
  MSX_LAUNCH((k_attn_bwd_kv_mfma<D, T, W, KS>), grid, dim3(64 * W), lds, s, q, k, v, mask, stats, g, dsum, dk, dv, L,
             S, H, heads, scale);
}
template <int D, int T, int W, int KS>
void launch_bwd(hipStream_t s, dim3 grid, unsigned qy, bool one, const float* q, const float* k, const float* v,
                const float* mask, const float* o, const float* stats, const float* g, float* dq, float* dk, float* dv,
                int L, int S, int H, int heads, float scale) {
  const size_t lds =
      size_t(std::max(stream_lds_floats(T, D, 1, one ? 1 : 2), stream_lds_floats(T, D, 3, one ? 1 : 2))) * 4;
  MSX_LAUNCH((k_attn_bwd_mfma<D, T, W, KS>), grid, dim3(64 * W), lds, s, q, k, v, mask, o, stats, g, dq, dk, dv, L, S,
             H, heads, scale, int(qy));
}
// Dispatch on a plan: the f16 kernels (never split) or the f32 ones.
#define MSX_BY_PLAN(plan, h16, GO_H, GO_F)                 \
  if (h16) {                                               \
    if ((plan).W == 4) GO_H(32, 4);                        \
    else if ((plan).T == 64) GO_H(64, 2);                  \
    else GO_H(32, 2);                                      \
  } else {                                                 \
    if ((plan).KS == 2) GO_F(128, 4, 2);                   \
    else if ((plan).W == 4) GO_F(32, 4, 1);                \
    else if ((plan).T == 64) GO_F(64, 2, 1);               \
    else GO_F(32, 2, 1);                                   \
  }
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
                   float* stats, int64_t B, int64_t L, int64_t S, int64_t H, int64_t heads, bool h16) {
  int64_t d = H / heads;
  if (!head_ok(d) || L > S) refuse("attention head width or query rows");
  float scale = 1.0f / sqrtf(float(d));
  if (attention_mfma(L, S, d)) {
    // 128 keys of 64-wide heads in f32 (BERT-tiny): the register-operand forward, four waves a
    // 16-query tile (8.5 us a layer against 10.0 for the LDS-staged kernel; two waves 9.9, eight
    // 9.5; the step 0.755 -> 0.751 ms). Its 16-byte loads need 16-byte aligned rows.
    const auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (!h16 && d == 64 && S == 128 && H % 4 == 0 && al16(q) && al16(k) && al16(v) && al16(mask) && al16(o)) {
      dim3 grid(unsigned(B * heads), unsigned(L / 16));
      MSX_LAUNCH(k_attn_fwd_reg<4>, grid, dim3(256), 0, s, q, k, v, mask, o, stats, int(L), int(H), int(heads), scale);
      return;
    }
    const AttnPlan plan = attn_plan(B * heads, L, S, d, h16);
    dim3 grid(unsigned(B * heads), row_blocks(L, plan));
#define GO_H(T, W) launch_fwd_h<D, T, W>(s, grid, q, k, v, mask, o, stats, int(L), int(S), int(H), int(heads), scale)
#define GO_F(T, W, KS) \
  launch_fwd<D, T, W, KS>(s, grid, plan.one, q, k, v, mask, o, stats, int(L), int(S), int(H), int(heads), scale)
#define GO(D_) { constexpr int D = D_; MSX_BY_PLAN(plan, h16, GO_H, GO_F) }
    MSX_BY_D(d, GO)
#undef GO
#undef GO_F
#undef GO_H
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
                   int64_t L, int64_t S, int64_t H, int64_t heads, bool h16) {
  int64_t d = H / heads;
  if (!head_ok(d) || L > S) refuse("attention head width or query rows");
  float scale = 1.0f / sqrtf(float(d));
  if (attention_mfma(L, S, d)) {
    if (!o || !stats || !dsum) refuse("the MFMA attention backward needs the forward output and statistics");
    if (!dq) refuse("the MFMA attention backward computes d_i in its dQ pass: dQ is required");
    const AttnPlan pq = attn_plan(B * heads, L, S, d, h16);
    dim3 gq(unsigned(B * heads), row_blocks(L, pq));
    if (!h16 && dk && dv && L == S) {
      // Self-attention in f32: one launch for both passes (the key pass plans as the query pass).
      dim3 gb(unsigned(B * heads), 2 * row_blocks(L, pq));
#define GO_H(T, W)
#define GO_F(T, W, KS)                                                                                              \
  launch_bwd<D, T, W, KS>(s, gb, row_blocks(L, pq), pq.one, q, k, v, mask, o, stats, g, dq, dk, dv, int(L), int(S), \
                          int(H), int(heads), scale)
#define GO(D_) { constexpr int D = D_; MSX_BY_PLAN(pq, false, GO_H, GO_F) }
      MSX_BY_D(d, GO)
#undef GO
#undef GO_F
#undef GO_H
      return;
    }
#define GO_H(T, W) \
  launch_bwd_q_h<D, T, W>(s, gq, q, k, v, mask, o, stats, g, dq, dsum, int(L), int(S), int(H), int(heads), scale)
#define GO_F(T, W, KS)                                                                                            \
  launch_bwd_q<D, T, W, KS>(s, gq, pq.one, q, k, v, mask, o, stats, g, dq, dsum, int(L), int(S), int(H), int(heads), \
                            scale)
#define GO(D_) { constexpr int D = D_; MSX_BY_PLAN(pq, h16, GO_H, GO_F) }
    MSX_BY_D(d, GO)
#undef GO
#undef GO_F
#undef GO_H
    if (dk || dv) {
      const AttnPlan pk = attn_plan(B * heads, S, L, d, h16);
      dim3 gk(unsigned(B * heads), row_blocks(S, pk));
#define GO_H(T, W) \
  launch_bwd_kv_h<D, T, W>(s, gk, q, k, v, mask, stats, g, dsum, dk, dv, int(L), int(S), int(H), int(heads), scale)
#define GO_F(T, W, KS)                                                                                             \
  launch_bwd_kv<D, T, W, KS>(s, gk, pk.one, q, k, v, mask, stats, g, dsum, dk, dv, int(L), int(S), int(H), int(heads), \
                             scale)
#define GO(D_) { constexpr int D = D_; MSX_BY_PLAN(pk, h16, GO_H, GO_F) }
      MSX_BY_D(d, GO)
#undef GO
#undef GO_F
#undef GO_H
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
#define MSX_ATTN_W(D, T, W)                                         \
  reinterpret_cast<const void*>(k_attn_fwd_mfma<D, T, W>),          \
      reinterpret_cast<const void*>(k_attn_bwd_q_mfma<D, T, W>),    \
      reinterpret_cast<const void*>(k_attn_bwd_kv_mfma<D, T, W>),   \
      reinterpret_cast<const void*>(k_attn_fwd_mfma<D, 128, 4, 2>), \
      reinterpret_cast<const void*>(k_attn_bwd_q_mfma<D, 128, 4, 2>), \
      reinterpret_cast<const void*>(k_attn_bwd_kv_mfma<D, 128, 4, 2>), \
      reinterpret_cast<const void*>(k_attn_bwd_mfma<D, T, W>),      \
      reinterpret_cast<const void*>(k_attn_bwd_mfma<D, 128, 4, 2>)
#define MSX_ATTN_H(D, T, W)                                         \
  reinterpret_cast<const void*>(k_attn_fwd_h16<D, T, W>),           \
      reinterpret_cast<const void*>(k_attn_bwd_q_h16<D, T, W>),     \
      reinterpret_cast<const void*>(k_attn_bwd_kv_h16<D, T, W>)
#define MSX_ATTN_K(D)                                                                            \
  MSX_ATTN_W(D, 32, 4), MSX_ATTN_W(D, 64, 2), MSX_ATTN_W(D, 32, 2), MSX_ATTN_H(D, 32, 4), \
      MSX_ATTN_H(D, 64, 2), MSX_ATTN_H(D, 32, 2)
      MSX_ATTN_K(16), MSX_ATTN_K(32), MSX_ATTN_K(64), MSX_ATTN_K(128)};
#undef MSX_ATTN_K
#undef MSX_ATTN_H
#undef MSX_ATTN_W
  for (const void* kern : kernels) {
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, int(kLdsMax));
    if (e != hipSuccess) throw std::runtime_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
  }
  prepare_flash16();
}

}  // namespace msx::hk
