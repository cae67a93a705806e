// GEMM kernels of the training step on the gfx950 f32 MFMA (v_mfma_f32_16x16x4f32), with bias,
// column-sum and split-K epilogues, and the shape-based choice of tile and split.
#include "kernels.h"
#include "device.h"
#include "gemm_common.h"

#include <algorithm>

namespace msx::hk {

// ---------------------------------------------------------------------------------------------
namespace {
constexpr int kSliceAlign = 32;  // split-K slices are multiples of this many K steps
}  // namespace

// Sums the split-K partial products in ascending slice order, one output element a thread, every
// slice's load issued before the adds; the threads past M * N do the same for the slices' column
// (row) sums.
template <int SPLIT>
__global__ __launch_bounds__(256) void k_splitk_sum(const float* __restrict__ ws, float* __restrict__ C, GemmEpi epi,
                                                    int64_t M, int64_t N, int64_t ldc, int splits,
                                                    float* __restrict__ colsum, int64_t width,
                                                    _Float16* __restrict__ C16) {
  const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t mn = M * N;
  const bool cs = e >= mn;
  if (cs && (!colsum || e - mn >= width)) return;
  const float* src = cs ? ws + int64_t(splits) * mn + (e - mn) : ws + e;
  const int64_t stride = cs ? width : mn;
  // SPLIT slices' loads in flight at a time, added in slice order.
  float s = 0.0f;
  for (int z0 = 0; z0 < splits; z0 += SPLIT) {
    float t[SPLIT];
#pragma unroll
    for (int u = 0; u < SPLIT; ++u) t[u] = src[int64_t(z0 + u < splits ? z0 + u : splits - 1) * stride];
#pragma unroll
    for (int u = 0; u < SPLIT; ++u)
      if (z0 + u < splits) s = (z0 + u == 0) ? t[u] : s + t[u];
  }
  if (cs) {
    colsum[e - mn] = s;
  } else {
    const int64_t row = e / N, col = e - row * N;
    const float v = gemm_epilogue(epi, s, row, col, ldc);
    if (C) C[row * ldc + col] = v;
    if (C16) C16[row * ldc + col] = _Float16(v);
  }
}

// ---------------------------------------------------------------------------------------------
// The GEMM: a block of 2 x 2 waves, each wave a
// (16 WM) x (16 WN) tile as WM x WN MFMA 16x16x4 accumulators, K advancing WK at a time through
// double-buffered LDS whose row strides (tile width + 16 floats) keep the fragment reads of a
// wave's two half-groups in disjoint banks. Operands may be read transposed in place. Epilogues:
// bias, split-K partials (summed in slice order by k_splitk_sum or a deferred column finalize:
// deterministic), column (row) sums from the LDS tiles.
namespace {
// One float4 group e of a K tile: the (row, k) element of a KC operand is P[row * ld + k] (four
// consecutive k), else P[k * ld + row] (four consecutive rows). Out-of-range groups read a
// clamped address and are zeroed, branch-free.
// V: the group is 16-byte aligned and wholly in or out of range, or its out-of-range part lies in
// zero padding of the rows: one float4 load; otherwise four clamped scalar loads.
// The cross-entropy gradient of logit x at column c of a row with entry t = (max, 1 / sum,
// g w / sum(w), label): (g w / sum(w)) (exp(x - max) / sum - [c = label]), in k_ce_rows' operation
// order; 0 past the row's `cols` columns and in a row of a batch whose weights sum to 0.
__device__ __forceinline__ float ce_grad_of(float x, const float4 t, int64_t c, int64_t cols) {
  const int lab = __float_as_int(t.w);
  if (c >= cols || lab == -2) return 0.0f;
  return t.z * (__expf(x - t.x) * t.y - (c == lab ? 1.0f : 0.0f));
}
// XF: the operand is a cross-entropy gradient formed from the logits P holds (tab, cols); its
// stored element (row, column) is P[row * ld + column].
template <bool KC, int R, int WK, bool V, bool XF = false>
__device__ __forceinline__ float4 wide_load(const float* __restrict__ P, int64_t ld, int64_t rows, int64_t kend,
                                            int64_t r0, int64_t k0, int e, const float4* __restrict__ tab = nullptr,
                                            int64_t cols = 0) {
  int r, k;
  if (KC) { r = e / (WK / 4); k = (e % (WK / 4)) * 4; } else { k = e / (R / 4); r = (e % (R / 4)) * 4; }
  const int64_t gr = r0 + r, gk = k0 + k;
  if (V) {
    const bool ok = gr < rows && gk < kend;
    // A group past the end reads the aligned group holding the last element instead.
    const int64_t cr = KC ? (gr < rows ? gr : rows - 1) : (gr < rows ? gr : (rows - 1) & ~int64_t(3));
    const int64_t ck = KC ? (gk < kend ? gk : (kend - 1) & ~int64_t(3)) : (gk < kend ? gk : kend - 1);
    float4 f = *reinterpret_cast<const float4*>(KC ? P + cr * ld + ck : P + ck * ld + cr);
    if (XF) {
      const int64_t srow = KC ? cr : ck, scol = KC ? ck : cr;
      const float4 t = tab[srow];
      f = make_float4(ce_grad_of(f.x, t, scol, cols), ce_grad_of(f.y, t, scol + 1, cols),
                      ce_grad_of(f.z, t, scol + 2, cols), ce_grad_of(f.w, t, scol + 3, cols));
    }
    return ok ? f : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t rr = KC ? gr : gr + j, kk = KC ? gk + j : gk;
    const int64_t cr = rr < rows ? rr : rows - 1, ck = kk < kend ? kk : kend - 1;
    float x = KC ? P[cr * ld + ck] : P[ck * ld + cr];
    if (XF) x = ce_grad_of(x, tab[KC ? cr : ck], KC ? ck : cr, cols);
    v[j] = rr < rows && kk < kend ? x : 0.0f;
  }
  return make_float4(v[0], v[1], v[2], v[3]);
}
// The column a KC operand's element (row r, k) takes in its [k][row] LDS tile: r XOR a multiple of
// 128 / WK chosen by k / 4. A float4 group's four stores (k .. k + 3 of one row) go to four rows of
// the tile, and the 32 lanes of a half-wave hold 32 / (WK / 4) rows at WK / 4 k offsets each:
// without the XOR the lanes of one row all land in one bank; with it the half-wave's stores fill
// 32 distinct banks. The fragment reads keep 16 consecutive columns a row (the XOR permutes a
// 16-aligned segment or swaps it with its neighbour), so they stay conflict-free.
template <int WK>
__device__ __forceinline__ int kc_swizzle(int k) { return (k >> 2) * (128 / WK); }
template <bool KC, int R, int L, int WK>
__device__ __forceinline__ void wide_store(float* S, int e, float4 v) {
  if (KC) {
    const int k = (e % (WK / 4)) * 4, r = (e / (WK / 4)) ^ kc_swizzle<WK>(k);
    S[(k + 0) * L + r] = v.x;
    S[(k + 1) * L + r] = v.y;
    S[(k + 2) * L + r] = v.z;
    S[(k + 3) * L + r] = v.w;
  } else {
    const int k = e / (R / 4), r = (e % (R / 4)) * 4;
    *reinterpret_cast<float4*>(S + k * L + r) = v;
  }
}
// The f16 K tiles of the mixed-precision GEMM: row r of the operand at S + r P, its K slice
// contiguous (P halves a row), each f32 rounded to the nearest f16.
template <bool KC, int R, int P, int WK>
__device__ __forceinline__ void wide_store_h(_Float16* S, int e, float4 v) {
  if (KC) {
    const int r = e / (WK / 4), k = (e % (WK / 4)) * 4;
    *reinterpret_cast<v4h*>(S + r * P + k) = v4h{_Float16(v.x), _Float16(v.y), _Float16(v.z), _Float16(v.w)};
  } else {
    const int k = e / (R / 4), r = (e % (R / 4)) * 4;
    S[(r + 0) * P + k] = _Float16(v.x);
    S[(r + 1) * P + k] = _Float16(v.y);
    S[(r + 2) * P + k] = _Float16(v.z);
    S[(r + 3) * P + k] = _Float16(v.w);
  }
}
// The f16 tiles of an operand whose rows are not contiguous along K: a thread holds N float4
// groups of 4 rows at N consecutive K (the groups hk_group numbers), and stores each of the 4 rows
// as one vector of N halves.
template <int R, int N>
__device__ __forceinline__ int hk_group(int t, int h) {
  return ((t / (R / 4)) * N + h) * (R / 4) + t % (R / 4);
}
template <int R, int P, int N>
__device__ __forceinline__ void rows_store_h(_Float16* S, int t, const float4 (&v)[N]) {
  const int r = (t % (R / 4)) * 4, k = (t / (R / 4)) * N;
  typedef _Float16 vh __attribute__((ext_vector_type(N)));
  vh x0, x1, x2, x3;
#pragma unroll
  for (int h = 0; h < N; ++h) {
    x0[h] = _Float16(v[h].x);
    x1[h] = _Float16(v[h].y);
    x2[h] = _Float16(v[h].z);
    x3[h] = _Float16(v[h].w);
  }
  *reinterpret_cast<vh*>(S + (r + 0) * P + k) = x0;
  *reinterpret_cast<vh*>(S + (r + 1) * P + k) = x1;
  *reinterpret_cast<vh*>(S + (r + 2) * P + k) = x2;
  *reinterpret_cast<vh*>(S + (r + 3) * P + k) = x3;
}
}  // namespace

// H: the mixed-precision variant. The operands are rounded to f16 as they are staged into LDS
// (rows of their K slice contiguous) and multiplied by v_mfma_f32_16x16x32_f16 with f32
// accumulation; K tiles of 32; everything else (split-K, epilogues, output) as in f32.
// CE: 1 or 2, operand A or B is a cross-entropy gradient formed from its logits (ce_grad_of);
// 3, the row partials of a cross-entropy over the output (ce_part).
// KS: the product is a sum of K segments (GemmPtrs::ksegs), read in place segment by segment.
template <bool TA, bool TB, int WM, int WN, int WK, bool VA, bool VB, bool H = false, int CE = 0, bool KS = false>
__global__ __launch_bounds__(256) void k_gemm_w(GemmPtrs ptrs, int64_t M, int64_t N, int64_t K, int64_t lda,
                                                int64_t ldb, int64_t ldc, int64_t kchunk, bool sum_a, bool vo,
                                                GemmOrder order) {
  constexpr int TM = 32 * WM, TN = 32 * WN, LA = TM + 16, LB = TN + 16, LC = TN + 4;
  constexpr int GA = TM * WK / 4, GB = TN * WK / 4;              // float4 groups a K tile
  constexpr int HA = (GA + 255) / 256, HB = (GB + 255) / 256;     // a thread's groups
  // The K tiles (double-buffered), and afterwards the output tile on its way to memory.
  // Deep K tiles (WK >= 128, meant for K <= WK: one tile) are single-buffered.
  constexpr int NB = WK >= 128 ? 1 : 2;
  constexpr int PH = WK + 8;  // f16 tile row: the K slice and 16 bytes of pad
  constexpr int TILES = H ? (NB * (TM + TN) * PH + 1) / 2 : NB * WK * LA + NB * WK * LB;
  static_assert(!H || WK % 32 == 0, "the f16 MFMA takes K 32 at a time");
  constexpr int PASSES = TM > 64 ? TM / 64 : 1, PR = TM / PASSES;  // output rows staged at a time
  __shared__ __align__(16) float smem[TILES > PR * LC ? TILES : PR * LC];
  float* const As0 = smem;                  // As(buf) = As0 + buf WK LA
  float* const Bs0 = smem + NB * WK * LA;   // Bs(buf) = Bs0 + buf WK LB
  _Float16* const Ah0 = reinterpret_cast<_Float16*>(smem);  // Ah(buf) = Ah0 + buf TM PH
  _Float16* const Bh0 = Ah0 + NB * TM * PH;                  // Bh(buf) = Bh0 + buf TN PH
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The tile of this block: consecutive blocks go to the 8 XCDs in turn, so block b takes tile
  // (b mod 8) * per + b / 8 of the grouped order, and each XCD runs one contiguous run of it.
  const uint32_t per = gridDim.x / 8, tg = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (tg >= order.tiles * ptrs.count) return;
  // The problem of the group this block works on, and its tile in that problem's order.
  const int q = int(tg / order.tiles);
  const uint32_t t = tg - uint32_t(q) * order.tiles;
  const float* __restrict__ A = ptrs.a[q];
  const float* __restrict__ B = ptrs.b[q];
  float* __restrict__ C = ptrs.c[q];
  const GemmEpi epi = ptrs.epi[q];
  float* __restrict__ ws = ptrs.ws[q];
  float* __restrict__ colsum = ptrs.colsum[q];
  uint32_t tm, tn;
  const uint32_t tz = t / (order.mt * order.nt), tr = t % (order.mt * order.nt);
  if (order.m_fastest) {
    tm = tr % order.mt;
    tn = tr / order.mt;
  } else {
    tn = tr % order.nt;
    tm = tr / order.nt;
  }
  const int64_t m0 = int64_t(tm) * TM, n0 = int64_t(tn) * TN;
  const int64_t kbeg = int64_t(tz) * kchunk;
  const int64_t kend = K < kbeg + kchunk ? K : kbeg + kchunk;
  const int wm = (wave >> 1) * 16 * WM, wn = (wave & 1) * 16 * WN;
  v4f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // op(A) is KC (contiguous along k) unless TA; op(B)^T is KC when TB. Under H an operand that is
  // not KC is loaded as consecutive K groups a thread (hk_group; GA and GB are multiples of 256).
  constexpr bool RA = H && TA, RB = H && !TB;
  static_assert((!RA || GA % 256 == 0) && (!RB || GB % 256 == 0), "row-vector staging takes whole groups a thread");
  auto ga = [&](int h) { return RA ? hk_group<TM, HA>(tid, h) : tid + 256 * h; };
  auto gb = [&](int h) { return RB ? hk_group<TN, HB>(tid, h) : tid + 256 * h; };
  const float4* __restrict__ ce_tab = CE == 1 || CE == 2 ? ptrs.ce_tab[q] : nullptr;
  // K segments: the tiles are loaded in ascending k0, so the segment (its operands and K offset)
  // advances when k0 reaches its end (kseg a multiple of WK; one segment: never).
  const float* sa = A;
  const float* sb = B;
  int64_t s_lo = 0, s_hi = KS ? ptrs.kseg : INT64_MAX;
  int sn = 0;
  auto advance = [&](int64_t k0) {
    if (KS && k0 >= s_hi) {
      ++sn;
      s_lo = s_hi;
      s_hi += ptrs.kseg;
      sa = ptrs.a[sn];
      sb = ptrs.b[sn];
    }
  };
  auto load_a = [&](int64_t k0, int h) {
    if constexpr (KS)
      return wide_load<!TA, TM, WK, VA, CE == 1>(sa, lda, M, kend - s_lo, m0, k0 - s_lo, ga(h), ce_tab, ptrs.ce_cols);
    else
      return wide_load<!TA, TM, WK, VA, CE == 1>(A, lda, M, kend, m0, k0, ga(h), ce_tab, ptrs.ce_cols);
  };
  auto load_b = [&](int64_t k0, int h) {
    if constexpr (KS)
      return wide_load<TB, TN, WK, VB, CE == 2>(sb, ldb, N, kend - s_lo, n0, k0 - s_lo, gb(h), ce_tab, ptrs.ce_cols);
    else
      return wide_load<TB, TN, WK, VB, CE == 2>(B, ldb, N, kend, n0, k0, gb(h), ce_tab, ptrs.ce_cols);
  };
  float4 ra[HA], rb[HB];
#pragma unroll
  for (int h = 0; h < HA; ++h)
    if (GA % 256 == 0 || tid + 256 * h < GA) ra[h] = load_a(kbeg, h);
#pragma unroll
  for (int h = 0; h < HB; ++h)
    if (GB % 256 == 0 || tid + 256 * h < GB) rb[h] = load_b(kbeg, h);
  // Column sums: thread t adds tile column t mod T over the K rows (t / T) per .. + per of each
  // K tile, per = WK / (256 / T).
  const int T = sum_a ? TM : TN;
  const bool sums = colsum != nullptr && (sum_a ? tn == 0 : tm == 0);
  const int sum_per = WK / (256 / T), sum_ld = sum_a ? LA : LB;
  // (A KC operand's columns are swizzled by k: its reads take the row's swizzle.)
  const bool sum_kc = sum_a ? !TA : TB;
  const int sum_k0 = (tid / T) * sum_per, sum_col = tid % T;
  float csum = 0.0f;
  int buf = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += WK) {
    if (NB == 1 && k0 != kbeg) __syncthreads();  // the single buffer is free again
    if constexpr (H) {
      if constexpr (RA) {
        rows_store_h<TM, PH, HA>(Ah0 + buf * (TM * PH), tid, ra);
      } else {
#pragma unroll
        for (int h = 0; h < HA; ++h)
          if (GA % 256 == 0 || tid + 256 * h < GA) wide_store_h<!TA, TM, PH, WK>(Ah0 + buf * (TM * PH), tid + 256 * h, ra[h]);
      }
      if constexpr (RB) {
        rows_store_h<TN, PH, HB>(Bh0 + buf * (TN * PH), tid, rb);
      } else {
#pragma unroll
        for (int h = 0; h < HB; ++h)
          if (GB % 256 == 0 || tid + 256 * h < GB) wide_store_h<TB, TN, PH, WK>(Bh0 + buf * (TN * PH), tid + 256 * h, rb[h]);
      }
    } else {
#pragma unroll
      for (int h = 0; h < HA; ++h)
        if (GA % 256 == 0 || tid + 256 * h < GA) wide_store<!TA, TM, LA, WK>(As0 + buf * (WK * LA), tid + 256 * h, ra[h]);
#pragma unroll
      for (int h = 0; h < HB; ++h)
        if (GB % 256 == 0 || tid + 256 * h < GB) wide_store<TB, TN, LB, WK>(Bs0 + buf * (WK * LB), tid + 256 * h, rb[h]);
    }
    __syncthreads();
    if (k0 + WK < kend) {
      if constexpr (KS) advance(k0 + WK);
#pragma unroll
      for (int h = 0; h < HA; ++h)
        if (GA % 256 == 0 || tid + 256 * h < GA) ra[h] = load_a(k0 + WK, h);
#pragma unroll
      for (int h = 0; h < HB; ++h)
        if (GB % 256 == 0 || tid + 256 * h < GB) rb[h] = load_b(k0 + WK, h);
    }
    if constexpr (H) {
      const _Float16* ah = Ah0 + buf * (TM * PH) + (wm + (lane & 15)) * PH + 8 * (lane >> 4);
      const _Float16* bh = Bh0 + buf * (TN * PH) + (wn + (lane & 15)) * PH + 8 * (lane >> 4);
#pragma unroll
      for (int kk = 0; kk < WK; kk += 32) {
        v8h a[WM], b[WN];
#pragma unroll
        for (int i = 0; i < WM; ++i) a[i] = *reinterpret_cast<const v8h*>(ah + 16 * i * PH + kk);
#pragma unroll
        for (int j = 0; j < WN; ++j) b[j] = *reinterpret_cast<const v8h*>(bh + 16 * j * PH + kk);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
      }
      buf = NB == 2 ? buf ^ 1 : 0;
      continue;
    }
    const float* as = As0 + buf * (WK * LA);
    const float* bs = Bs0 + buf * (WK * LB);
#pragma unroll
    for (int kk = 0; kk < WK; kk += 4) {
      // A is KC unless TA, B when TB: their columns carry the swizzle of k = kk .. kk + 3.
      const int swa = !TA ? kc_swizzle<WK>(kk) : 0, swb = TB ? kc_swizzle<WK>(kk) : 0;
      const int ka = (kk + (lane >> 4)) * LA, kb = (kk + (lane >> 4)) * LB;
      float a[WM], b[WN];
#pragma unroll
      for (int i = 0; i < WM; ++i) a[i] = as[ka + ((wm + 16 * i + (lane & 15)) ^ swa)];
#pragma unroll
      for (int j = 0; j < WN; ++j) b[j] = bs[kb + ((wn + 16 * j + (lane & 15)) ^ swb)];
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (sums) {
      const float* ss = sum_a ? as : bs;
      for (int j = 0; j < sum_per; ++j) {
        const int kr = sum_k0 + j;
        csum += ss[kr * sum_ld + (sum_kc ? sum_col ^ kc_swizzle<WK>(kr) : sum_col)];
      }
    }
    buf = NB == 2 ? buf ^ 1 : 0;
  }
  if (sums) {
    __syncthreads();
    float* red = smem;
    red[tid] = csum;
    __syncthreads();
    const int64_t base = sum_a ? m0 : n0, width = sum_a ? M : N;
    if (tid < T && base + tid < width) {
      float v = red[tid];
      for (int g = 1; g < 256 / T; ++g) v += red[g * T + tid];
      colsum[(ws ? int64_t(tz) * width : 0) + base + tid] = v;
    }
  }
  // The output tile goes through LDS so that each row leaves as whole float4 groups (when `vo`:
  // 16-byte aligned rows whose width is a multiple of 4, or padded to one), the epilogue applied
  // on the way; a tile of more than 64 rows goes in passes of 64 rows (the waves of one half).
  float* out = ws ? ws + int64_t(tz) * M * N : C;
  const int64_t ldo = ws ? N : ldc;
  constexpr int Q = TN / 4;
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    __syncthreads();
    if (PASSES == 1 || wm / PR == pass) {
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            smem[(wm - pass * PR + 16 * i + 4 * (lane >> 4) + r) * LC + wn + 16 * j + (lane & 15)] = acc[i][j][r];
    }
    __syncthreads();
#pragma unroll
    for (int e0 = 0; e0 < PR * Q; e0 += 256) {
      const int e = e0 + tid;
      if (PR * Q % 256 != 0 && e >= PR * Q) break;
      const int rl = e / Q, c4 = (e % Q) * 4;
      const int64_t row = m0 + pass * PR + rl, col = n0 + c4;
      if constexpr (CE == 3) {
        // The row's (max, sum of exp(v - max)) over this tile's columns, after the epilogue: the Q
        // lanes of a row are consecutive, reduced by shuffles in a fixed order.
        static_assert(Q <= 64 && 256 % Q == 0, "a row's output groups lie in one wave");
        const float4 raw = *reinterpret_cast<const float4*>(smem + rl * LC + c4);
        float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (row < M && col < N) {
          const float4 f = col + 3 < N ? gemm_epilogue4(epi, raw, row, col, ldo)
                                       : make_float4(gemm_epilogue(epi, raw.x, row, col, ldo),
                                                     col + 1 < N ? gemm_epilogue(epi, raw.y, row, col + 1, ldo) : 0.0f,
                                                     col + 2 < N ? gemm_epilogue(epi, raw.z, row, col + 2, ldo) : 0.0f, 0.0f);
          v = make_float4(f.x, col + 1 < N ? f.y : -INFINITY, col + 2 < N ? f.z : -INFINITY,
                          col + 3 < N ? f.w : -INFINITY);
        }
        float mx = fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w));
#pragma unroll
        for (int o = Q / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        float sm = (__expf(v.x - mx) + __expf(v.y - mx)) + (__expf(v.z - mx) + __expf(v.w - mx));
#pragma unroll
        for (int o = Q / 2; o > 0; o >>= 1) sm += __shfl_xor(sm, o, 64);
        if (c4 == 0 && row < M) {
          const int64_t tiles = (N + TN - 1) / TN;
          reinterpret_cast<float2*>(ptrs.ce_part[q])[row * tiles + tn] = make_float2(mx, sm);
        }
      }
      if (row >= M) continue;
      const float4 v = *reinterpret_cast<const float4*>(smem + rl * LC + c4);
      if (vo && col + 3 < N) {
        *reinterpret_cast<float4*>(out + row * ldo + col) = ws ? v : gemm_epilogue4(epi, v, row, col, ldo);
      } else if (vo && col < N) {
        // The last group of a row padded to a multiple of 4: zeros in the padding.
        const float vs[4] = {v.x, v.y, v.z, v.w};
        float r4[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) r4[c] = col + c < N ? (ws ? vs[c] : gemm_epilogue(epi, vs[c], row, col + c, ldo)) : 0.0f;
        *reinterpret_cast<float4*>(out + row * ldo + col) = make_float4(r4[0], r4[1], r4[2], r4[3]);
      } else {
        const float vs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (col + c < N) out[row * ldo + col + c] = ws ? vs[c] : gemm_epilogue(epi, vs[c], row, col + c, ldo);
      }
    }
  }
}

namespace {
// The tile shape and split-K of a GEMM, from measured MI355X timings of the step's shapes: large
// outputs (and very deep K) take 64 x 64 tiles, outputs up to 2^19 elements 32 x 32, the rest
// 32 x 64. Split-K, whose slice sum costs a launch unless deferred to a batched finalize, is used
// when deferred or when K is deep, to fill the chip. The f16 MFMA does eight times the work of
// the f32 one an instruction, so mixed-precision GEMMs of 2^21 outputs or more (or K of 8192 or
// more) take 128 x 128 tiles: four times the MFMAs per operand byte staged.
struct SplitPlan { int wm, wn, wk, split; int64_t chunk; };
SplitPlan split_plan(int64_t m, int64_t n, int64_t k, bool defer, bool h16, bool ce = false) {
  const int64_t mn = m * n;
  SplitPlan p{};
  // A cross-entropy head (ce) always takes the largest tile, the one its kernels are built for.
  // Mixed precision: the 128 x 128 tiles of k_gemm_lds16 (and k_gemm_w's largest f16 tile).
  if (h16) { p.wm = 4; p.wn = 4; p.wk = 32; }
  else if (ce || mn >= (int64_t(1) << 21) || k >= 8192) { p.wm = 2; p.wn = 2; p.wk = 16; }
  else if (mn <= (int64_t(1) << 19)) { p.wm = 1; p.wn = 1; p.wk = 32; }
  else { p.wm = 1; p.wn = 2; p.wk = 16; }
  const int64_t tiles = ((m + 32 * p.wm - 1) / (32 * p.wm)) * ((n + 32 * p.wn - 1) / (32 * p.wn));
  int64_t want = 1;
  if (defer || k >= 1024) {
    const int64_t blocks = p.wm == 2 ? 2048 : 1024;  // 128 x 128 tiles: 1024 (4 a CU)
    want = tiles < blocks / 4 ? (blocks + tiles - 1) / tiles : 1;
    // An f32 product of K 8192 or more summed by its own launch (BERT-tiny's decoder input
    // gradient, K 30522): half as many slices, 74 -> 37 (A/B in one run: 74 -> 68 us, half the
    // partials written and read back; a quarter as many 74 us, 1.5 times as many 81 us).
    if (!h16 && !defer && k >= 8192) want = std::max<int64_t>(1, want / 2);
  }
  // Deferred slices keep 128 K steps or more (4096 for 128 x 128 tiles, whose f16 blocks get
  // through K fastest): their partials all go through the finalize, m n floats a slice
  // (BERT-base's K = 16384 weight gradients: 4 slices 37.7 ms a step, 16 slices 38.0, 2 slices
  // 38.1).
  // (A deferred f16 product of K under 8192 takes slices of at least 512: BERT-base's head dense
  // weight gradient, 768x768 at K = 2880, otherwise runs 36 blocks.)
  const int64_t min_slice = defer ? (p.wm == 4 ? (k >= 8192 ? 4096 : 512) : 128) : 64;
  const int64_t split = std::max<int64_t>(1, std::min(want, k / min_slice));
  p.chunk = ((k + split - 1) / split + kSliceAlign - 1) / kSliceAlign * kSliceAlign;
  p.split = int((k + p.chunk - 1) / p.chunk);
  return p;
}
}  // namespace

int gemm_split_for(int64_t m, int64_t n, int64_t k, bool defer, bool h16, bool ce) {
  return split_plan(m, n, k, defer, h16, ce).split;
}

int64_t gemm_tile_n(int64_t m, int64_t n, int64_t k, bool defer, bool h16) {
  return 32 * split_plan(m, n, k, defer, h16, true).wn;
}

int64_t gemm_workspace(int64_t m, int64_t n, int64_t k, bool colsum, bool sum_a, bool defer, bool h16, bool ce) {
  const int split = gemm_split_for(m, n, k, defer, h16, ce);
  if (split <= 1) return 0;
  return int64_t(split) * m * n + (colsum ? int64_t(split) * (sum_a ? m : n) : 0);  // partials, then sums
}

int gemm_deferred_jobs(const GemmArgs& g, ColumnJob* jobs) {
  const int split = gemm_split_for(g.m, g.n, g.k, g.defer, g.h16, g.ce_operand != 0 || g.ce_part);
  if (split <= 1) return 0;
  if (g.bias || g.addend || g.act || g.drop_token || g.ldc != g.n) bad("deferred split-K needs a dense output without epilogue");
  if (g.m * g.n > INT32_MAX) bad("deferred split-K output too large");
  jobs[0] = ColumnJob{g.workspace, g.c, nullptr, split, int32_t(g.m * g.n), int32_t(g.m * g.n), 0};
  if (!g.colsum) return 1;
  const int64_t width = g.sum_a ? g.m : g.n;
  jobs[1] = ColumnJob{g.workspace + int64_t(split) * g.m * g.n, g.colsum, nullptr, split, int32_t(width), int32_t(width), 0};
  return 2;
}

bool gemm_lds16_fits(const GemmArgs& g) {
  if (!g.h16 || g.ksegs > 1 || g.ce_operand || g.ce_part || g.m <= 0 || g.n <= 0 || g.k <= 0) return false;
  return lds16_layout(g, split_plan(g.m, g.n, g.k, g.defer, true, false).chunk);
}

void gemm(hipStream_t s, const GemmArgs& g) { gemm_group(s, &g, 1); }


// A group of problems of one shape and configuration (the first one's), one launch: every
void gemm_group(hipStream_t s, const GemmArgs* list, int count) {
  if (count < 1 || count > kGemmGroupMax) bad("gemm group size");
  const GemmArgs& g = list[0];
  if (g.m <= 0 || g.n <= 0) return;
  if (g.k <= 0) bad("gemm with k = 0");
  for (int q = 1; q < count; ++q) {
    const GemmArgs& o = list[q];
    if (o.m != g.m || o.n != g.n || o.k != g.k || o.lda != g.lda || o.ldb != g.ldb || o.ldc != g.ldc || o.ta != g.ta ||
        o.tb != g.tb || o.sum_a != g.sum_a || o.defer != g.defer || o.pad_a != g.pad_a || o.pad_b != g.pad_b ||
        o.pad_c != g.pad_c || o.h16 != g.h16 || o.act != g.act || (o.colsum == nullptr) != (g.colsum == nullptr) ||
        (o.bias == nullptr) != (g.bias == nullptr) || (o.addend == nullptr) != (g.addend == nullptr) ||
        (o.workspace == nullptr) != (g.workspace == nullptr) || (o.drop_token == nullptr) != (g.drop_token == nullptr))
      bad("gemm group of unlike problems");
  }
  const int ce = g.ce_part ? 3 : g.ce_operand;
  if (ce && (count != 1 || (ce == 3 && g.k > 0 && split_plan(g.m, g.n, g.k, g.defer, g.h16, true).split > 1)))
    bad("a cross-entropy head GEMM runs alone, and its forward without split-K");
  const SplitPlan plan = split_plan(g.m, g.n, g.k, g.defer, g.h16, ce != 0);
  const int split = plan.split;
  const int ksegs = g.ksegs > 1 ? g.ksegs : 1;
  if (ksegs > 1 && (count != 1 || ksegs > kGemmGroupMax || g.k % ksegs != 0 || (g.k / ksegs) % 32 != 0 || split != 1 ||
                    g.colsum || ce))
    bad("K segments need one problem, at most 4 segments of a multiple of 32 K, no split-K, column sums or "
        "cross-entropy");
  const int64_t chunk = plan.chunk;
  if (split > 1 && count > 1 && !g.defer) bad("a gemm group sums split-K slices by deferral only");
  GemmPtrs ptrs{};
  ptrs.count = count;
  const int problems = count;
  for (int q = 0; q < problems; ++q) {
    const GemmArgs& o = list[q];
    float* ws = nullptr;
    if (split > 1) {
      if (!o.workspace ||
          o.workspace_floats < gemm_workspace(o.m, o.n, o.k, o.colsum != nullptr, o.sum_a, o.defer, o.h16, ce != 0))
        bad("gemm split-K workspace too small");
      ws = o.workspace;
    }
    ptrs.a[q] = o.a;
    ptrs.b[q] = o.b;
    ptrs.c[q] = o.c;
    ptrs.epi[q] = GemmEpi{o.bias, o.addend, o.pre_in, o.pre_out, o.act, o.drop_token, o.drop_threshold, o.drop_scale, o.drop_seed,
                          o.pre16};
    ptrs.ws[q] = ws;
    ptrs.colsum[q] = o.colsum ? (ws ? ws + int64_t(split) * o.m * o.n : o.colsum) : nullptr;
    ptrs.ce_part[q] = o.ce_part;
    ptrs.ce_tab[q] = o.ce_tab;
    ptrs.a16[q] = o.a16;
    ptrs.b16[q] = o.b16;
    ptrs.c16[q] = o.c16;
    if ((o.a16 || o.b16 || o.c16) && !o.h16) bad("f16 operand copies outside mixed precision");
    if (o.c16 && o.defer) bad("a deferred split-K output has no f16 copy");
  }
  ptrs.ce_cols = g.ce_cols;
  ptrs.ksegs = ksegs;
  ptrs.kseg = g.k / ksegs;
  if (ksegs > 1)
    for (int q = 0; q < ksegs; ++q) {
      ptrs.a[q] = g.seg_a[q];
      ptrs.b[q] = g.seg_b[q];
    }
  float* ws = ptrs.ws[0];
  // Tiles in the grouped order: split slices outermost; within a slice the tiles that share the
  // larger operand's panel are adjacent (M tiles of one column when B is the larger, N tiles of
  // one row otherwise), so that each XCD's L2 serves the panel to all of them.
  const int64_t nt = (g.n + 32 * plan.wn - 1) / (32 * plan.wn), mt = (g.m + 32 * plan.wm - 1) / (32 * plan.wm);
  const int64_t tiles = nt * mt * split;
  if (tiles * problems > (int64_t(1) << 30)) bad("gemm has too many tiles");
  const GemmOrder order{uint32_t(mt), uint32_t(nt), uint32_t(tiles), g.n * g.k >= g.m * g.k};
  const dim3 wgrid(unsigned((tiles * problems + 7) / 8 * 8));
  const int64_t width = g.sum_a ? g.m : g.n;
  for (int q = 0; q < count; ++q) {
    const GemmArgs& o = list[q];
    if ((o.act == EPI_GELU_GRAD || o.act == EPI_RELU_GRAD) && !o.pre_in && !o.pre16)
      bad("gemm activation gradient without its input");
    if (o.pre16 && (!o.h16 || o.act == EPI_NONE || reinterpret_cast<uintptr_t>(o.pre16) % 8 || o.ldc % 4))
      bad("an f16 pre-activation needs mixed precision, an activation and 8-byte aligned rows");
  }
  const GemmEpi epi{g.bias, g.addend, g.pre_in, g.pre_out, g.act, g.drop_token, g.drop_threshold, g.drop_scale, g.drop_seed,
                    g.pre16};
  if (g.drop_token && (g.ldc != g.n || g.m * g.n > (int64_t(1) << 32)))
    bad("a GEMM's dropout epilogue needs a dense output of at most 2^32 elements");
  // float4 output groups: every row the epilogue touches 16-byte aligned (in every problem).
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  bool vo = true, va = true, vb = true;
  // float4 loads need 16-byte aligned groups and a contiguous extent that is a multiple of 4.
  // (A zero-padded operand may be read up to its leading dimension.)
  auto aligned = [](const float* p, int64_t ld, int64_t extent) {
    return (reinterpret_cast<uintptr_t>(p) % 16 == 0) && ld % 4 == 0 && extent % 4 == 0;
  };
  for (int q = 0; q < problems; ++q) {
    const GemmArgs& o = list[q];
    vo = vo && (ptrs.ws[q] ? (o.n % 4 == 0 && a16(ptrs.ws[q]))
                           : ((o.n % 4 == 0 || (o.pad_c && !o.act && !o.addend)) && o.ldc % 4 == 0 && a16(o.c) &&
                              a16(o.bias) && a16(o.addend) && a16(o.pre_in) && a16(o.pre_out) && a16(o.pre16)));
    va = va && aligned(o.a, o.lda, o.pad_a ? o.lda : (o.ta ? o.m : o.k / ksegs));
    vb = vb && aligned(o.b, o.ldb, o.pad_b ? o.ldb : (o.tb ? o.k / ksegs : o.n));
  }
  for (int q = 0; q < ksegs && ksegs > 1; ++q) {
    va = va && aligned(ptrs.a[q], g.lda, g.pad_a ? g.lda : (g.ta ? g.m : g.k / ksegs));
    vb = vb && aligned(ptrs.b[q], g.ldb, g.pad_b ? g.ldb : (g.tb ? g.k / ksegs : g.n));
  }
#define MSX_WIDE_V(TA, TB, WM, WN, WK, VA, VB)                                                              \
  MSX_LAUNCH((k_gemm_w<TA, TB, WM, WN, WK, VA, VB>), wgrid, dim3(256), 0, s, ptrs, g.m, g.n, g.k, g.lda,     \
             g.ldb, g.ldc, chunk, g.sum_a, vo, order)
  // float4 variants for both operands aligned, or the right one only; scalar loads otherwise.
#define MSX_WIDE(TA, TB, WM, WN, WK)                                \
  if (va && vb) MSX_WIDE_V(TA, TB, WM, WN, WK, true, true);         \
  else if (vb) MSX_WIDE_V(TA, TB, WM, WN, WK, false, true);         \
  else MSX_WIDE_V(TA, TB, WM, WN, WK, false, false)
#define MSX_WIDE_T(TA, TB)                                  \
  if (plan.wm == 2) MSX_WIDE(TA, TB, 2, 2, 16);             \
  else if (plan.wn == 2) MSX_WIDE(TA, TB, 1, 2, 16);        \
  else MSX_WIDE(TA, TB, 1, 1, 32);
  // The mixed-precision variants: the same tiles with f16 K tiles of 32.
#define MSX_WIDE_HV(TA, TB, WM, WN, VA, VB)                                                                 \
  MSX_LAUNCH((k_gemm_w<TA, TB, WM, WN, 32, VA, VB, true>), wgrid, dim3(256), 0, s, ptrs, g.m, g.n, g.k,     \
             g.lda, g.ldb, g.ldc, chunk, g.sum_a, vo, order)
#define MSX_WIDE_H(TA, TB, WM, WN)                                  \
  if (va && vb) MSX_WIDE_HV(TA, TB, WM, WN, true, true);            \
  else if (vb) MSX_WIDE_HV(TA, TB, WM, WN, false, true);            \
  else MSX_WIDE_HV(TA, TB, WM, WN, false, false)
#define MSX_WIDE_HT(TA, TB)                                 \
  if (plan.wm == 4) MSX_WIDE_H(TA, TB, 4, 4);               \
  else if (plan.wm == 2) MSX_WIDE_H(TA, TB, 2, 2);          \
  else if (plan.wn == 2) MSX_WIDE_H(TA, TB, 1, 2);          \
  else MSX_WIDE_H(TA, TB, 1, 1);
  // The cross-entropy head kernels: the largest tile of each precision, both operands float4.
#define MSX_CE_V(TA, TB, WM, WN, WK, H, CE)                                                                    \
  MSX_LAUNCH((k_gemm_w<TA, TB, WM, WN, WK, true, true, H, CE>), wgrid, dim3(256), 0, s, ptrs, g.m, g.n, g.k,  \
             g.lda, g.ldb, g.ldc, chunk, g.sum_a, vo, order)
#define MSX_CE_T(TA, TB, WM, WN, WK, H)                       \
  if (ce == 1) MSX_CE_V(TA, TB, WM, WN, WK, H, 1);            \
  else if (ce == 2) MSX_CE_V(TA, TB, WM, WN, WK, H, 2);       \
  else MSX_CE_V(TA, TB, WM, WN, WK, H, 3);
#define MSX_CE(WM, WN, WK, H)                                 \
  if (!g.ta && !g.tb) { MSX_CE_T(false, false, WM, WN, WK, H) } \
  else if (g.ta && !g.tb) { MSX_CE_T(true, false, WM, WN, WK, H) } \
  else if (!g.ta && g.tb) { MSX_CE_T(false, true, WM, WN, WK, H) } \
  else { MSX_CE_T(true, true, WM, WN, WK, H) }
  // K segments: the f32 kernels with both operands float4.
#define MSX_KS_V(TA, TB, WM, WN, WK)                                                                           \
  MSX_LAUNCH((k_gemm_w<TA, TB, WM, WN, WK, true, true, false, 0, true>), wgrid, dim3(256), 0, s, ptrs, g.m, g.n, \
             g.k, g.lda, g.ldb, g.ldc, chunk, g.sum_a, vo, order)
#define MSX_KS_T(TA, TB)                                    \
  if (plan.wm == 2) MSX_KS_V(TA, TB, 2, 2, 16);             \
  else if (plan.wn == 2) MSX_KS_V(TA, TB, 1, 2, 16);        \
  else MSX_KS_V(TA, TB, 1, 1, 32);
  // The large f32 shapes take k_gemm_lds when their layout allows it, mixed-precision GEMMs whose
  // operands both have f16 copies k_gemm_lds16 (gemm_lds.hip).
  bool f16_out = false;  // the launched kernel writes the f16 output copies itself
  const bool lds = !g.h16 && ksegs == 1 && count == 1 && !ce && gemm_lds(s, g, ptrs, split, chunk);
  const bool lds16 = !lds && g.h16 && ksegs == 1 && !ce && gemm_lds16(s, list, count, ptrs, split, chunk);
  if (lds16) f16_out = true;
  for (int q = 0; q < count && !lds16; ++q)
    if (!list[q].a || !list[q].b || !list[q].c)
      bad("a GEMM on an f16-only operand or output needs k_gemm_lds16 (f16 copies, its layout)");
  if (lds || lds16) {
    // launched
  } else if (ksegs > 1) {
    if (!va || !vb || g.h16) bad("K segments need aligned f32 operands");
    if (!g.ta && !g.tb) { MSX_KS_T(false, false) }
    else if (g.ta && !g.tb) { MSX_KS_T(true, false) }
    else if (!g.ta && g.tb) { MSX_KS_T(false, true) }
    else { MSX_KS_T(true, true) }
  } else if (ce) {
    if (!va || !vb || (ce == 3 && !vo)) bad("a cross-entropy head GEMM needs aligned, padded operands");
    if (g.h16 && g.colsum) bad("the mixed-precision GEMM takes no column sums");
    if (g.h16) { MSX_CE(4, 4, 32, true) }
    else { MSX_CE(2, 2, 16, false) }
  } else if (g.h16) {
    if (g.colsum) bad("mixed-precision column sums need k_gemm_lds16's layout (f16 copies, K a multiple of 32)");
    if (!g.ta && !g.tb) { MSX_WIDE_HT(false, false) }
    else if (g.ta && !g.tb) { MSX_WIDE_HT(true, false) }
    else if (!g.ta && g.tb) { MSX_WIDE_HT(false, true) }
    else { MSX_WIDE_HT(true, true) }
  } else if (!g.ta && !g.tb) { MSX_WIDE_T(false, false) }
  else if (g.ta && !g.tb) { MSX_WIDE_T(true, false) }
  else if (!g.ta && g.tb) { MSX_WIDE_T(false, true) }
  else { MSX_WIDE_T(true, true) }
#undef MSX_KS_T
#undef MSX_KS_V
#undef MSX_CE
#undef MSX_CE_T
#undef MSX_CE_V
#undef MSX_WIDE_HT
#undef MSX_WIDE_H
#undef MSX_WIDE_HV
#undef MSX_WIDE_T
#undef MSX_WIDE
#undef MSX_WIDE_V
  if (split > 1 && !g.defer) {
    const int64_t total = g.m * g.n + (g.colsum ? width : 0);
    const unsigned blocks = unsigned((total + 255) / 256);
#define MSX_SPLITK(S) MSX_LAUNCH(k_splitk_sum<S>, dim3(blocks), dim3(256), 0, s, ws, g.c, epi, g.m, g.n, g.ldc, \
                                         split, g.colsum, width, g.c16)
    if (split <= 8) MSX_SPLITK(8);
    else if (split <= 16) MSX_SPLITK(16);
    else MSX_SPLITK(32);
#undef MSX_SPLITK
    f16_out = true;
  }
  // f16 output copies a kernel did not write: rounded from the f32 output.
  for (int q = 0; q < count && !f16_out; ++q)
    if (list[q].c16) to_f16_rows(s, list[q].c, list[q].ldc, list[q].c16, list[q].ldc, list[q].m, list[q].n);
}

}  // namespace msx::hk
