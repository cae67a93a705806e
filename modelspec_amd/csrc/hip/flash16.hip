// Mixed-precision attention for 64-wide heads on the f16 MFMA of gfx950 (v_mfma_f32_16x16x32_f16,
// f32 accumulation), reading the f16 copies of its operands that their producers write. The
// attention of attention.hip's kernels (reference: ir/kernel.rs Attention, AttentionGrad*):
//   forward   o_i = sum_j p_ij v_j / l_i,  p_ij = mask_j ? exp(s_ij scale - m_i) : 0,
//             s_ij = q_i . k_j,  m_i = max over unmasked j of s_ij scale,  l_i = sum_j p_ij;
//   backward  P = p / l,  dP = dO V^T,  dS = P (dP - d_i),  d_i = dO_i . O_i,
//             dQ = scale dS K,  dK = scale dS^T Q,  dV = P^T dO  (rows of masked keys zero).
// Softmax statistics, exponentials and sums stay f32 (exponentials as 2^x of log2(e)-scaled
// scores); the contractions take f16 operands: q, k, v, dO, and p, dS rounded to f16.
//
// Tiles of 64 rows of 64 halves (a [row][d] slice of a head) move from global memory straight into
// a 3-stage LDS ring (global_load_lds, as the direct-to-LDS GEMMs), the 16-byte chunk ch of row r
// at slot ch ^ (r mod 8). Two read patterns serve every contraction:
//   - row fragments: lane (c, q) reads row 16 u + c, d 32 h + 8 q .. + 7 (16 bytes), the operand
//     of a contraction over d;
//   - transposed fragments (ds_read_b64_tr_b16): lane c of group q gets column d = base + c at rows
//     k0 .. k0 + 3, the operand of a contraction over the tile's rows.
// Score tiles come out of the MFMA as 16x16 blocks in which lane (c, q) holds rows 4 q + r of one
// side and column c of the other. A contraction over those rows takes, in K slot 8 q + e of a
// 32-row chunk w, the row 32 w + 4 q + e (e < 4) or 32 w + 16 + 4 q + e - 4 (e >= 4): the two
// score blocks' values a lane holds, as they stand, against two transposed reads at rows
// 32 w + 4 q and 32 w + 16 + 4 q. Accumulating the transposed output (O^T, dQ^T, dK^T, dV^T) puts
// one query (key) a lane in every accumulator: per-row scaling needs no shuffles and each lane
// stores four consecutive d.
#include "device.h"
#include "kernels.h"
#include "lds_util.h"

#include <algorithm>
#include <cmath>

namespace msx::hk {

namespace {
constexpr int FD = 64;             // head width
constexpr int FT = 64;             // rows a streamed tile
constexpr int FNS = 3;             // LDS ring stages
constexpr int FTILE = FT * FD;     // halves a tile
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

// The 16-byte chunk ch of row r of a staged tile.
__device__ __forceinline__ int chunk_at(int r, int ch) { return r * FD + 8 * (ch ^ (r & 7)); }

// Issue this wave's share of one tile: W waves, 8 load instructions a tile (1 KB = 8 rows each).
// src: row 0 of the tile at column 0 of the head; ld: halves between rows.
template <int W>
__device__ __forceinline__ void issue_tile(const _Float16* src, int64_t ld, _Float16* dst, int wave, int lane) {
#pragma unroll
  for (int h = 0; h < 8 / W; ++h) {
    const int t = wave * (8 / W) + h;
    const int r = 8 * t + lane / 8, slot = lane % 8, ch = slot ^ (r & 7);
    load_lds16(src + int64_t(r) * ld + 8 * ch, dst + 512 * t);
  }
}

// Row fragment: row r, d chunk 4 h + q (8 halves).
__device__ __forceinline__ v8h row_frag(const _Float16* X, int r, int h, int q) {
  return *reinterpret_cast<const v8h*>(X + chunk_at(r, 4 * h + q));
}

// LDS address of the transposed read of source lane c in group q: tile row k0 + c / 4, columns
// d0 + 4 (c mod 4) .. + 3 (d0 a multiple of 16).
__device__ __forceinline__ uint32_t tr_addr(const _Float16* X, int k0, int d0, int c) {
  const int r = k0 + c / 4, d = d0 + 4 * (c % 4);
  return lds_at(X + chunk_at(r, d / 8) + (d % 8));
}

__device__ __forceinline__ v8h join(v4s16 lo, v4s16 hi) {
  const v4h16 a = __builtin_bit_cast(v4h16, lo), b = __builtin_bit_cast(v4h16, hi);
  return v8h{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Transposed fragments of a tile for the four 16-column d blocks of 32-row chunk w: f[dblk] holds,
// lane (c, q), column 16 dblk + c at rows 32 w + 4 q .. + 3 and 32 w + 16 + 4 q .. + 3.
__device__ __forceinline__ void tr_frags(const _Float16* X, int w, int c, int q, v8h (&f)[4]) {
  uint32_t at[8];
#pragma unroll
  for (int dblk = 0; dblk < 4; ++dblk) {
    at[2 * dblk] = tr_addr(X, 32 * w + 4 * q, 16 * dblk, c);
    at[2 * dblk + 1] = tr_addr(X, 32 * w + 16 + 4 * q, 16 * dblk, c);
  }
  v4s16 r[8];
  tr_read16x8(at, r);
#pragma unroll
  for (int dblk = 0; dblk < 4; ++dblk) f[dblk] = join(r[2 * dblk], r[2 * dblk + 1]);
}

__device__ __forceinline__ v4f mfma(v8h a, v8h b, v4f c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

__device__ __forceinline__ v8h pack8(const v4f& x, const v4f& y) {
  return v8h{_Float16(x[0]), _Float16(x[1]), _Float16(x[2]), _Float16(x[3]),
             _Float16(y[0]), _Float16(y[1]), _Float16(y[2]), _Float16(y[3])};
}

// A global row's 16-byte fragment (d 32 h + 8 q .. + 7).
__device__ __forceinline__ v8h glob_frag(const _Float16* row, int h, int q) {
  return *reinterpret_cast<const v8h*>(row + 32 * h + 8 * q);
}

__device__ __forceinline__ float at4(const float4& v, int r) { return r == 0 ? v.x : r == 1 ? v.y : r == 2 ? v.z : v.w; }

// The mask bias of tile t's keys 16 u + 4 q .. + 3, u = 0 .. 3.
__device__ __forceinline__ void bias_of(const float* mb, int t, int q, float4 (&bias)[4]) {
  uint32_t at[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) at[u] = lds_at(mb + t * FT + 16 * u + 4 * q);
  lds_read4x16(at, bias);
}

// Stores four consecutive d (f32, and f16 when o16) of one row.
__device__ __forceinline__ void store4(float* o, _Float16* o16, int64_t at, v4f v) {
  if (o) *reinterpret_cast<v4f*>(o + at) = v;
  if (o16) *reinterpret_cast<v4h16*>(o16 + at) = v4h16{_Float16(v[0]), _Float16(v[1]), _Float16(v[2]), _Float16(v[3])};
}
}  // namespace

// Forward. Block (bh, y): W waves of 32 queries (two 16-row blocks) each, rows y 32 W ..; keys
// streamed in tiles of 64. mb: the key mask as an additive bias (0 or -inf), S floats.
template <int W>
__global__ __launch_bounds__(64 * W) void k_flash_fwd16(const _Float16* __restrict__ q, const _Float16* __restrict__ k,
                                                        const _Float16* __restrict__ v, const float* __restrict__ mask,
                                                        float* __restrict__ o, _Float16* __restrict__ o16,
                                                        float* __restrict__ stats, int L, int S, int H, int heads,
                                                        float scale) {
  __shared__ __align__(16) _Float16 ring[FNS][2][FTILE];
  extern __shared__ float mb[];
  constexpr int LPT = 2 * 8 / W;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, qq = lane >> 4;
  const int bh = blockIdx.x, b = bh / heads, head = bh % heads;
  const int i0 = blockIdx.y * (32 * W) + 32 * wave;
  const float sl2 = scale * kLog2e;
  for (int j = tid; j < S; j += 64 * W) mb[j] = mask[int64_t(b) * S + j] != 0.0f ? 0.0f : -INFINITY;
  const _Float16* kb = k + int64_t(b) * S * H + head * FD;
  const _Float16* vb = v + int64_t(b) * S * H + head * FD;
  v8h qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int h = 0; h < 2; ++h) qf[qb][h] = glob_frag(q + (int64_t(b) * L + i0 + 16 * qb + c) * H + head * FD, h, qq);
  __syncthreads();
  const int tiles = S / FT;
  auto issue = [&](int t) {
    t = t < tiles ? t : tiles - 1;
    issue_tile<W>(kb + int64_t(t) * FT * H, H, ring[t % FNS][0], wave, lane);
    issue_tile<W>(vb + int64_t(t) * FT * H, H, ring[t % FNS][1], wave, lane);
  };
#pragma unroll
  for (int t = 0; t < FNS - 1; ++t) issue(t);
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
  v4f oacc[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int d = 0; d < 4; ++d) oacc[qb][d] = v4f{0, 0, 0, 0};
#pragma unroll 1
  for (int t = 0; t < tiles; ++t) {
    wait_vm((FNS - 2) * LPT);
    __builtin_amdgcn_s_barrier();
    issue(t + FNS - 1);
    const _Float16* Ks = ring[t % FNS][0];
    const _Float16* Vs = ring[t % FNS][1];
    // S^T blocks: keys 16 u + 4 qq + r (rows), query c of block qb (column).
    v4f sc[2][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const v8h k0 = row_frag(Ks, 16 * u + c, 0, qq), k1 = row_frag(Ks, 16 * u + c, 1, qq);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) sc[qb][u] = mfma(k1, qf[qb][1], mfma(k0, qf[qb][0], v4f{0, 0, 0, 0}));
    }
    float4 bias[4];
    bias_of(mb, t, qq, bias);
    v8h pf[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float tmax = -INFINITY;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[qb][u][r] = sc[qb][u][r] * sl2 + at4(bias[u], r);
          tmax = fmaxf(tmax, sc[qb][u][r]);
        }
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mn = fmaxf(m[qb], tmax), mu = mn == -INFINITY ? 0.0f : mn;
      const float alpha = exp2_(m[qb] - mu);
      m[qb] = mn;
      float ls = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[qb][u][r] = exp2_(sc[qb][u][r] - mu);
          ls += sc[qb][u][r];
        }
      l[qb] = l[qb] * alpha + ls;
#pragma unroll
      for (int d = 0; d < 4; ++d) oacc[qb][d] *= alpha;
      pf[qb][0] = pack8(sc[qb][0], sc[qb][1]);
      pf[qb][1] = pack8(sc[qb][2], sc[qb][3]);
    }
    // O^T += V^T P^T over the tile's two 32-key chunks.
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      v8h vf[4];
      tr_frags(Vs, w, c, qq, vf);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int d = 0; d < 4; ++d) oacc[qb][d] = mfma(vf[d], pf[qb][w], oacc[qb][d]);
    }
  }
  wait_vm(0);  // no load may still write LDS when the block ends
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float lt = l[qb];
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    const int i = i0 + 16 * qb + c;
    const int64_t row = (int64_t(b) * L + i) * H + head * FD;
#pragma unroll
    for (int d = 0; d < 4; ++d) store4(o, o16, row + 16 * d + 4 * qq, oacc[qb][d] / lt);
    if (stats && qq == 0) {
      const int64_t at = (int64_t(bh) * L + i) * 2;
      stats[at] = m[qb] * 0.6931471805599453f;  // back to natural-log units
      stats[at + 1] = lt;
    }
  }
}

// Backward, query side: d_i (from the f16 copies of the output and its gradient) and dQ. Block (bh, y) as the
// forward's; keys and values streamed. Writes the per-query terms the key side reads, three planes
// of B heads L floats: m_i log2(e), 1 / l_i, d_i.
template <int W>
__global__ __launch_bounds__(64 * W) void k_flash_bwd_q16(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    const float* __restrict__ mask, const _Float16* __restrict__ o16, const _Float16* __restrict__ go16, const float* __restrict__ stats, float* __restrict__ qterms,
    float* __restrict__ dq, _Float16* __restrict__ dq16, int L, int S, int H, int heads, float scale, int64_t plane) {
  __shared__ __align__(16) _Float16 ring[FNS][2][FTILE];
  extern __shared__ float mb[];
  constexpr int LPT = 2 * 8 / W;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, qq = lane >> 4;
  const int bh = blockIdx.x, b = bh / heads, head = bh % heads;
  const int i0 = blockIdx.y * (32 * W) + 32 * wave;
  const float sl2 = scale * kLog2e;
  for (int j = tid; j < S; j += 64 * W) mb[j] = mask[int64_t(b) * S + j] != 0.0f ? 0.0f : -INFINITY;
  v8h qf[2][2], gf[2][2];
  float m2[2], il[2], dd[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int i = i0 + 16 * qb + c;
    const int64_t row = (int64_t(b) * L + i) * H + head * FD;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      qf[qb][h] = glob_frag(q + row, h, qq);
      gf[qb][h] = glob_frag(go16 + row, h, qq);
    }
    // d_i from the f16 copies of the output and its gradient (the lane's 16 d, the fragments'),
    // f32 products and sums.
    float s = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v8h a = glob_frag(o16 + row, h, qq);
#pragma unroll
      for (int e = 0; e < 8; ++e) s = __builtin_fmaf(float(gf[qb][h][e]), float(a[e]), s);
    }
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    dd[qb] = s;
    const int64_t at = int64_t(bh) * L + i;
    m2[qb] = stats[2 * at] * kLog2e;
    il[qb] = 1.0f / stats[2 * at + 1];
    if (qq == 0) {
      qterms[at] = m2[qb];
      qterms[plane + at] = il[qb];
      qterms[2 * plane + at] = dd[qb];
    }
  }
  __syncthreads();
  if (!dq && !dq16) return;
  const _Float16* kb = k + int64_t(b) * S * H + head * FD;
  const _Float16* vb = v + int64_t(b) * S * H + head * FD;
  const int tiles = S / FT;
  auto issue = [&](int t) {
    t = t < tiles ? t : tiles - 1;
    issue_tile<W>(kb + int64_t(t) * FT * H, H, ring[t % FNS][0], wave, lane);
    issue_tile<W>(vb + int64_t(t) * FT * H, H, ring[t % FNS][1], wave, lane);
  };
#pragma unroll
  for (int t = 0; t < FNS - 1; ++t) issue(t);
  v4f acc[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int d = 0; d < 4; ++d) acc[qb][d] = v4f{0, 0, 0, 0};
#pragma unroll 1
  for (int t = 0; t < tiles; ++t) {
    wait_vm((FNS - 2) * LPT);
    __builtin_amdgcn_s_barrier();
    issue(t + FNS - 1);
    const _Float16* Ks = ring[t % FNS][0];
    const _Float16* Vs = ring[t % FNS][1];
    // S^T and dP^T blocks: keys 16 u + 4 qq + r, query c of block qb.
    v8h dsf[2][2];
    v4f sc[2][4], dp[2][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const v8h k0 = row_frag(Ks, 16 * u + c, 0, qq), k1 = row_frag(Ks, 16 * u + c, 1, qq);
      const v8h v0 = row_frag(Vs, 16 * u + c, 0, qq), v1 = row_frag(Vs, 16 * u + c, 1, qq);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        sc[qb][u] = mfma(k1, qf[qb][1], mfma(k0, qf[qb][0], v4f{0, 0, 0, 0}));
        dp[qb][u] = mfma(v1, gf[qb][1], mfma(v0, gf[qb][0], v4f{0, 0, 0, 0}));
      }
    }
    float4 bias[4];
    bias_of(mb, t, qq, bias);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = exp2_(sc[qb][u][r] * sl2 + at4(bias[u], r) - m2[qb]) * il[qb];
          sc[qb][u][r] = p * (dp[qb][u][r] - dd[qb]);
        }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      dsf[qb][0] = pack8(sc[qb][0], sc[qb][1]);
      dsf[qb][1] = pack8(sc[qb][2], sc[qb][3]);
    }
    // dQ^T += K^T dS^T.
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      v8h kf[4];
      tr_frags(Ks, w, c, qq, kf);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[qb][d] = mfma(kf[d], dsf[qb][w], acc[qb][d]);
    }
  }
  wait_vm(0);
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int64_t row = (int64_t(b) * L + i0 + 16 * qb + c) * H + head * FD;
#pragma unroll
    for (int d = 0; d < 4; ++d) store4(dq, dq16, row + 16 * d + 4 * qq, acc[qb][d] * scale);
  }
}

// Backward, key side: dK and dV. Block (bh, y): W waves of 32 keys each, keys y 32 W ..; queries
// and their output gradients streamed in tiles of 64 with the query terms (m_i log2(e), 1 / l_i,
// d_i) of each tile.
template <int W>
__global__ __launch_bounds__(64 * W) void k_flash_bwd_kv16(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    const float* __restrict__ mask, const _Float16* __restrict__ go16, const float* __restrict__ qterms,
    float* __restrict__ dk, _Float16* __restrict__ dk16, float* __restrict__ dv, _Float16* __restrict__ dv16, int L,
    int S, int H, int heads, float scale, int64_t plane) {
  // A stage: the query tile, the output-gradient tile, then the query terms (3 planes of FT floats
  // and the spare lanes' landing), in one array (a separate one made the compiler wait for every
  // load in flight before reading the tiles).
  constexpr int SST = 2 * FTILE + 8 * FT;
  __shared__ __align__(16) _Float16 ring[FNS][SST];
  constexpr int LPT = 2 * 8 / W + 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, qq = lane >> 4;
  const int bh = blockIdx.x, b = bh / heads, head = bh % heads;
  const int j0 = blockIdx.y * (32 * W) + 32 * wave;
  const float sl2 = scale * kLog2e;
  v8h kf[2][2], vf[2][2];
  bool live[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int j = j0 + 16 * kb + c;
    const int64_t row = (int64_t(b) * S + j) * H + head * FD;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      kf[kb][h] = glob_frag(k + row, h, qq);
      vf[kb][h] = glob_frag(v + row, h, qq);
    }
    live[kb] = mask[int64_t(b) * S + j] != 0.0f;
  }
  const _Float16* qb_ = q + int64_t(b) * L * H + head * FD;
  const _Float16* gb_ = go16 + int64_t(b) * L * H + head * FD;
  const float* tb_ = qterms + int64_t(bh) * L;
  const int tiles = L / FT;
  auto issue = [&](int t) {
    t = t < tiles ? t : tiles - 1;
    issue_tile<W>(qb_ + int64_t(t) * FT * H, H, ring[t % FNS], wave, lane);
    issue_tile<W>(gb_ + int64_t(t) * FT * H, H, ring[t % FNS] + FTILE, wave, lane);
    // The tile's query terms, 3 x 64 floats: lane l < 48 loads 4 of plane l / 16, the others
    // land past them (every wave the same bytes, so that every wave counts the same loads).
    const int pl = lane < 48 ? lane / 16 : 2, e = lane < 48 ? 4 * (lane % 16) : 60;
    load_lds16(tb_ + pl * plane + int64_t(t) * FT + e, ring[t % FNS] + 2 * FTILE);
  };
#pragma unroll
  for (int t = 0; t < FNS - 1; ++t) issue(t);
  v4f dka[2][4], dva[2][4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int d = 0; d < 4; ++d) { dka[kb][d] = v4f{0, 0, 0, 0}; dva[kb][d] = v4f{0, 0, 0, 0}; }
#pragma unroll 1
  for (int t = 0; t < tiles; ++t) {
    wait_vm((FNS - 2) * LPT);
    __builtin_amdgcn_s_barrier();
    issue(t + FNS - 1);
    const _Float16* Qs = ring[t % FNS];
    const _Float16* Gs = Qs + FTILE;
    const float* Ts = reinterpret_cast<const float*>(Qs + 2 * FTILE);
    // S and dP blocks: queries 16 u + 4 qq + r (rows), key c of block kb (column).
    v4f sc[2][4], dp[2][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const v8h q0 = row_frag(Qs, 16 * u + c, 0, qq), q1 = row_frag(Qs, 16 * u + c, 1, qq);
      const v8h g0 = row_frag(Gs, 16 * u + c, 0, qq), g1 = row_frag(Gs, 16 * u + c, 1, qq);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sc[kb][u] = mfma(q1, kf[kb][1], mfma(q0, kf[kb][0], v4f{0, 0, 0, 0}));
        dp[kb][u] = mfma(g1, vf[kb][1], mfma(g0, vf[kb][0], v4f{0, 0, 0, 0}));
      }
    }
    v8h pf[2][2], dsf[2][2];
    float4 tm[4], ti[4], td[4];
    {
      uint32_t a0[4], a1[4], a2[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a0[u] = lds_at(Ts + 16 * u + 4 * qq);
        a1[u] = lds_at(Ts + FT + 16 * u + 4 * qq);
        a2[u] = lds_at(Ts + 2 * FT + 16 * u + 4 * qq);
      }
      lds_read4x16(a0, tm);
      lds_read4x16(a1, ti);
      lds_read4x16(a2, td);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = live[kb] ? exp2_(sc[kb][u][r] * sl2 - at4(tm[u], r)) * at4(ti[u], r) : 0.0f;
          sc[kb][u][r] = p;
          dp[kb][u][r] = p * (dp[kb][u][r] - at4(td[u], r));
        }
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      pf[kb][0] = pack8(sc[kb][0], sc[kb][1]);
      pf[kb][1] = pack8(sc[kb][2], sc[kb][3]);
      dsf[kb][0] = pack8(dp[kb][0], dp[kb][1]);
      dsf[kb][1] = pack8(dp[kb][2], dp[kb][3]);
    }
    // dV^T += dO^T P, dK^T += Q^T dS over the tile's two 32-query chunks.
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      v8h gt[4], qt[4];
      tr_frags(Gs, w, c, qq, gt);
      tr_frags(Qs, w, c, qq, qt);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          dva[kb][d] = mfma(gt[d], pf[kb][w], dva[kb][d]);
          dka[kb][d] = mfma(qt[d], dsf[kb][w], dka[kb][d]);
        }
    }
  }
  wait_vm(0);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int64_t row = (int64_t(b) * S + j0 + 16 * kb + c) * H + head * FD;
    const v4f zero{0, 0, 0, 0};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      if (dv || dv16) store4(dv, dv16, row + 16 * d + 4 * qq, live[kb] ? dva[kb][d] : zero);
      if (dk || dk16) store4(dk, dk16, row + 16 * d + 4 * qq, live[kb] ? dka[kb][d] * scale : zero);
    }
  }
}

namespace {
constexpr int kFlashW = 4;
bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
}  // namespace

void prepare_flash16() {
  // The mask bias (S <= 4096 floats) beside 48 KB of static LDS.
  for (const void* kern : {reinterpret_cast<const void*>(k_flash_fwd16<kFlashW>),
                           reinterpret_cast<const void*>(k_flash_bwd_q16<kFlashW>)}) {
    const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 16 * 1024);
    if (e != hipSuccess) throw std::runtime_error(std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
  }
}

bool flash16_fits(int64_t L, int64_t S, int64_t d) {
  return d == FD && L > 0 && S > 0 && L % (32 * kFlashW) == 0 && S % (32 * kFlashW) == 0 && S <= 4096 && L <= 65535 * 128;
}

void flash16_fwd(hipStream_t s, const _Float16* q, const _Float16* k, const _Float16* v, const float* mask, float* o,
                 _Float16* o16, float* stats, int64_t B, int64_t L, int64_t S, int64_t H, int64_t heads) {
  if (H / heads != FD || H % heads || !flash16_fits(L, S, FD)) bad("f16 attention: 64-wide heads, rows a multiple of 128");
  if (!q || !k || !v || !stats || H % 8 || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) ||
      !aligned16(o16))
    bad("f16 attention: f16 operands, statistics and 16-byte aligned rows");
  const float scale = 1.0f / sqrtf(float(FD));
  const dim3 grid(unsigned(B * heads), unsigned(L / (32 * kFlashW)));
  MSX_LAUNCH(k_flash_fwd16<kFlashW>, grid, dim3(64 * kFlashW), size_t(S) * 4, s, q, k, v, mask, o, o16, stats, int(L),
             int(S), int(H), int(heads), scale);
}

void flash16_bwd(hipStream_t s, const _Float16* q, const _Float16* k, const _Float16* v, const float* mask,
                 const _Float16* o16, const _Float16* go16, const float* stats, float* qterms, float* dq, _Float16* dq16,
                 float* dk, _Float16* dk16, float* dv, _Float16* dv16, int64_t B, int64_t L, int64_t S, int64_t H,
                 int64_t heads) {
  if (H / heads != FD || H % heads || !flash16_fits(L, S, FD)) bad("f16 attention: 64-wide heads, rows a multiple of 128");
  if (!q || !k || !v || !o16 || !go16 || !stats || !qterms || H % 8 || !aligned16(q) || !aligned16(k) ||
      !aligned16(v) || !aligned16(o16) || !aligned16(go16) || !aligned16(qterms) || !aligned16(dq) ||
      !aligned16(dq16) || !aligned16(dk) || !aligned16(dk16) || !aligned16(dv) || !aligned16(dv16))
    bad("f16 attention backward: f16 operands, output, statistics, query terms and 16-byte aligned rows");
  const float scale = 1.0f / sqrtf(float(FD));
  const int64_t plane = B * heads * L;
  if (plane % 4) bad("f16 attention backward: query-term planes of whole 16-byte groups");
  MSX_LAUNCH(k_flash_bwd_q16<kFlashW>, dim3(unsigned(B * heads), unsigned(L / (32 * kFlashW))), dim3(64 * kFlashW),
             size_t(S) * 4, s, q, k, v, mask, o16, go16, stats, qterms, dq, dq16, int(L), int(S), int(H), int(heads),
             scale, plane);
  if (!dk && !dk16 && !dv && !dv16) return;
  MSX_LAUNCH(k_flash_bwd_kv16<kFlashW>, dim3(unsigned(B * heads), unsigned(S / (32 * kFlashW))), dim3(64 * kFlashW), 0,
             s, q, k, v, mask, go16, qterms, dk, dk16, dv, dv16, int(L), int(S), int(H), int(heads), scale, plane);
}

}  // namespace msx::hk
