// The large-shape f32 GEMM on gfx950: operand K tiles loaded straight into LDS.
#include "gemm_common.h"
#include "lds_util.h"

#include <algorithm>

namespace msx::hk {

// ---------------------------------------------------------------------------------------------
// The large-shape f32 GEMM (k_gemm_lds): operand K tiles move from global memory straight into an
// NS-stage LDS ring (global_load_lds_dwordx4: no staging registers, no LDS store instructions), one
// barrier a K tile, the loads of tile t + NS - 1 in flight while tile t is multiplied.
//
// Index mapping. The 16x16x4 f32 MFMA takes lane (c = l % 16, q = l / 16) to supply row c of its
// 16-row operands at K index q of a K step. Step s (0..3) of a 16-K block maps q to the K index
// 4 q + s, so a lane's four steps read four consecutive K of one row: one 16-byte LDS read. Which
// output row or column an MFMA lane stands for is free as long as both operands and the output
// agree, and is chosen so that every LDS read is 16 bytes:
//   - an operand contiguous along K (KC) is staged as [row][K] (BK floats a row, the K group of
//     row r at slot kq ^ f(r), so the 16 rows a quarter-wave reads at one K group hit distinct
//     banks; the loading lane fetches the group its slot holds); MFMA block i of a wave takes rows
//     16 i + c;
//   - an operand contiguous along its rows (not KC) is staged as [K][row], as it lies in memory;
//     lane c takes rows I c .. I c + I - 1 of the wave tile, one per MFMA block, one 16-byte read a
//     K step.
// The MFMA computes C^T tiles (B's fragment in the first operand), so a lane holds four
// consecutive output columns: float4 stores of the output.
// K must be a multiple of BK, or a KC operand's rows zero-padded up to the next multiple (its
// leading dimension); a non-KC operand's K rows past K are clamped to the last one (their products
// with the zero padding vanish). SUMS: 1, the row sums of op(A) over K; 2, the column sums of
// op(B) (a bias gradient), taken from the fragments of the waves of the first wave column (row).

template <int BM, int BN, int WGM, int WGN, int BK, bool AKC, bool BKC, int NS, bool FP, int SUMS>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm_lds(GemmPtrs ptrs, int64_t M, int64_t N, int64_t K,
                                                             int64_t lda, int64_t ldb, int64_t ldc, int64_t kchunk,
                                                             int64_t zero_to, bool vo, GemmOrder order) {
  constexpr int W = WGM * WGN;
  constexpr int WTM = BM / WGM, WTN = BN / WGN, I = WTM / 16, J = WTN / 16;
  static_assert((I == 4 || I == 2) && (J == 4 || J == 2), "wave tiles of 2 or 4 MFMA blocks a side");
  static_assert(BK == 16 || BK == 32, "K tiles of 16 or 32");
  constexpr int SA = BM * BK, SB = BN * BK, SS = SA + SB;  // floats a stage
  constexpr int LA = SA / 256, LB = SB / 256;              // 1 KB wave load instructions a tile
  static_assert(LA % W == 0 && LB % W == 0, "whole load instructions a wave");
  constexpr int PA = LA / W, PB = LB / W, LPT = PA + PB;   // a wave's load instructions a tile
  constexpr int RPI = 256 / BK, LPR = BK / 4;              // KC: rows an instruction, lanes a row
  constexpr int KB = BK / 16;                              // 16-K blocks a tile
  __shared__ __align__(16) float smem[NS * SS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, q = lane >> 4;
  // Consecutive blocks go to the 8 XCDs in turn; each XCD takes a contiguous run of the tile order.
  const uint32_t per = gridDim.x / 8, tg = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (tg >= order.tiles) return;
  const uint32_t tz = tg / (order.mt * order.nt), tr = tg % (order.mt * order.nt);
  const uint32_t tm = order.m_fastest ? tr % order.mt : tr / order.nt;
  const uint32_t tn = order.m_fastest ? tr / order.mt : tr % order.nt;
  const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
  // The slices cover K rounded up to BK.
  const int64_t kpad = (K + BK - 1) / BK * BK;
  const int64_t kbeg = int64_t(tz) * kchunk, kend = kpad < kbeg + kchunk ? kpad : kbeg + kchunk;
  const int tiles = int((kend - kbeg) / BK);
  const int wm = (wave / WGN) * WTM, wn = (wave % WGN) * WTN;
  const float* __restrict__ A = ptrs.a[0];
  const float* __restrict__ B = ptrs.b[0];
  const GemmEpi epi = ptrs.epi[0];
  const float* __restrict__ bias = epi.bias;
  float* __restrict__ ws = ptrs.ws[0];
  float* __restrict__ colsum = ptrs.colsum[0];
  auto fsw = [](int r) { return BK == 16 ? (r >> 2) & 3 : (r >> 1) & 7; };
  // Each load instruction's per-lane source at the slice's first K tile. KC: instruction t holds
  // rows t RPI .. (lane L: row L / LPR, K group (L % LPR) ^ f(row)). Not KC: K rows t (256 / R) ..
  // of R = BM (BN) floats (lane L: rows 4 (L % (R / 4)) .. + 3 at K row L / (R / 4)); the last
  // K row a lane may read is kmax (clamped).
  const float* srcA[PA];
  const float* srcB[PB];
  int kofA[PA], kofB[PB];
  const int64_t kmax = K - 1;
#pragma unroll
  for (int h = 0; h < PA; ++h) {
    const int t = wave * PA + h;
    if (AKC) {
      const int r = t * RPI + lane / LPR, kq = (lane % LPR) ^ fsw(t * RPI + lane / LPR);
      const int64_t row = m0 + r < M ? m0 + r : M - 1;
      srcA[h] = A + row * lda + kbeg + 4 * kq;
      kofA[h] = 0;
    } else {
      constexpr int RQ = BM / 4, KR = 256 / BM;
      const int kr = t * KR + lane / RQ;
      int64_t col = m0 + 4 * (lane % RQ);
      col = col + 3 < M ? col : ((M - 1) & ~int64_t(3));
      srcA[h] = A + col;
      kofA[h] = kr;
    }
  }
#pragma unroll
  for (int h = 0; h < PB; ++h) {
    const int t = wave * PB + h;
    if (BKC) {
      const int r = t * RPI + lane / LPR, kq = (lane % LPR) ^ fsw(t * RPI + lane / LPR);
      const int64_t row = n0 + r < N ? n0 + r : N - 1;
      srcB[h] = B + row * ldb + kbeg + 4 * kq;
      kofB[h] = 0;
    } else {
      constexpr int RQ = BN / 4, KR = 256 / BN;
      const int kr = t * KR + lane / RQ;
      int64_t col = n0 + 4 * (lane % RQ);
      col = col + 3 < N ? col : ((N - 1) & ~int64_t(3));
      srcB[h] = B + col;
      kofB[h] = kr;
    }
  }
  // Tile `tile` of the slice into its stage; past the last tile, the last tile again (into a stage
  // nobody reads), so every iteration issues the same number of loads.
  auto issue = [&](int tile) {
    tile = tile < tiles ? tile : tiles - 1;
    float* st = smem + (tile % NS) * SS;
    const int64_t k0 = int64_t(tile) * BK;
#pragma unroll
    for (int h = 0; h < PA; ++h) {
      const int t = wave * PA + h;
      if (AKC) {
        load_lds16(srcA[h] + k0, st + t * 256);
      } else {
        const int64_t kr = kbeg + k0 + kofA[h];
        load_lds16(srcA[h] + (kr < kmax ? kr : kmax) * lda, st + t * 256);
      }
    }
#pragma unroll
    for (int h = 0; h < PB; ++h) {
      const int t = wave * PB + h;
      if (BKC) {
        load_lds16(srcB[h] + k0, st + SA + t * 256);
      } else {
        const int64_t kr = kbeg + k0 + kofB[h];
        load_lds16(srcB[h] + (kr < kmax ? kr : kmax) * ldb, st + SA + t * 256);
      }
    }
  };
  // This lane's output columns: group j is n0 + wn + 16 j + 4 q .. + 3 (KC B), or n0 + wn + 4 J q +
  // 4 j .. + 3 (B not KC); the bias of each is loaded before the K loop.
  v4f bias4[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    bias4[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (bias && !ws) {
      const int64_t col0 = n0 + wn + (BKC ? 16 * j + 4 * q : 4 * J * q + 4 * j);
#pragma unroll
      for (int u = 0; u < 4; ++u) bias4[j][u] = col0 + u < N ? bias[col0 + u] : 0.0f;
    }
  }
  v4f acc[I][J];
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // Sums over K of this lane's operand rows (SUMS): per MFMA block, the lane's K indices only.
  constexpr int SN = SUMS == 1 ? I : SUMS == 2 ? J : 1;
  float ksum[SN];
#pragma unroll
  for (int u = 0; u < SN; ++u) ksum[u] = 0.0f;
  const bool sum_wave = SUMS == 1 ? wn == 0 : SUMS == 2 ? wm == 0 : false;
  struct Frag { v4f a[KB][4], b[KB][4]; };
  auto kc_at = [&](int r, int kq) { return (r / RPI) * 256 + (r % RPI) * BK + 4 * (kq ^ fsw(r)); };
  auto read = [&](int tile, Frag& f) {
    const float* As = smem + (tile % NS) * SS;
    const float* Bs = As + SA;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (AKC) {
#pragma unroll
        for (int i = 0; i < I; ++i) f.a[kb][i] = *reinterpret_cast<const v4f*>(As + kc_at(wm + 16 * i + c, 4 * kb + q));
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float* p = As + (16 * kb + 4 * q + s) * BM + wm + I * c;
          if constexpr (I == 4) {
            f.a[kb][s] = *reinterpret_cast<const v4f*>(p);
          } else {
            const float2 t2 = *reinterpret_cast<const float2*>(p);
            f.a[kb][s] = v4f{t2.x, t2.y, 0.0f, 0.0f};
          }
        }
      }
      if (BKC) {
#pragma unroll
        for (int j = 0; j < J; ++j) f.b[kb][j] = *reinterpret_cast<const v4f*>(Bs + kc_at(wn + 16 * j + c, 4 * kb + q));
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float* p = Bs + (16 * kb + 4 * q + s) * BN + wn + J * c;
          if constexpr (J == 4) {
            f.b[kb][s] = *reinterpret_cast<const v4f*>(p);
          } else {
            const float2 t2 = *reinterpret_cast<const float2*>(p);
            f.b[kb][s] = v4f{t2.x, t2.y, 0.0f, 0.0f};
          }
        }
      }
    }
  };
  auto mfma = [&](const Frag& f) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < I; ++i)
#pragma unroll
          for (int j = 0; j < J; ++j) {
            const float a = AKC ? f.a[kb][i][s] : f.a[kb][s][i];
            const float b = BKC ? f.b[kb][j][s] : f.b[kb][s][j];
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b, a, acc[i][j], 0, 0, 0);
          }
      if (SUMS != 0 && sum_wave) {
#pragma unroll
        for (int u = 0; u < SN; ++u)
#pragma unroll
          for (int s = 0; s < 4; ++s)
            ksum[u] += SUMS == 1 ? (AKC ? f.a[kb][u][s] : f.a[kb][s][u]) : (BKC ? f.b[kb][u][s] : f.b[kb][s][u]);
      }
    }
  };
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) issue(p);
  if constexpr (!FP) {
    // Tile t landed (the later tiles may still fly), then a bare barrier (a workgroup fence would
    // wait for the prefetches too): every wave is past tile t - 1, whose stage takes tile t + NS - 1.
    for (int t = 0; t < tiles; ++t) {
      wait_vm((NS - 2) * LPT);
      __builtin_amdgcn_s_barrier();
      issue(t + NS - 1);
      Frag f;
      read(t, f);
      mfma(f);
    }
  } else {
    // Fragments one tile ahead: iteration t waits for tile t + 1 and reads its fragments, then
    // multiplies tile t's, read in the iteration before.
    static_assert(NS >= 3, "fragment prefetch needs three stages");
    Frag f0, f1;
    wait_vm((NS - 2) * LPT);
    __builtin_amdgcn_s_barrier();
    read(0, f0);
    auto body = [&](int t, const Frag& cur, Frag& nxt) {
      wait_vm((NS - 3) * LPT);
      __builtin_amdgcn_s_barrier();
      issue(t + NS - 1);
      read(t + 1, nxt);
      mfma(cur);
    };
    int t = 0;
    for (; t + 2 <= tiles; t += 2) {
      body(t, f0, f1);
      body(t + 1, f1, f0);
    }
    if (t < tiles) mfma(f0);
  }
  wait_vm(0);  // no load may still write LDS when the block ends
  float* out = ws ? ws + int64_t(tz) * M * N : ptrs.c[0];
  const int64_t ldo = ws ? N : ldc, zto = ws ? N : zero_to;
#pragma unroll
  for (int i = 0; i < I; ++i) {
    const int64_t row = m0 + wm + (AKC ? 16 * i + c : I * c + i);
    if (row >= M) continue;
    float* orow = out + row * ldo;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      int64_t col;
      v4f v;
      if (BKC) {
        col = n0 + wn + 16 * j + 4 * q;
        v = acc[i][j] + bias4[j];
      } else {
        // Columns wn + J (4 q + r) + jj: group j holds r = (4 j + u) / J, jj = (4 j + u) % J.
        col = n0 + wn + 4 * J * q + 4 * j;
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = acc[i][(4 * j + u) % J][(4 * j + u) / J];
        v += bias4[j];
      }
      // The rest of the epilogue (activation or its gradient, addend, dropout gradient) after the
      // bias, as the other kernel applies it.
      const bool more = !ws && (epi.act != EPI_NONE || epi.addend || epi.drop_token);
      if (vo && col + 3 < N) {
        if (more) {
          const float4 f = gemm_epilogue4(GemmEpi{nullptr, epi.addend, epi.pre_in, epi.pre_out, epi.act, epi.drop_token,
                                                  epi.drop_threshold, epi.drop_scale, epi.drop_seed, epi.pre16},
                                          make_float4(v[0], v[1], v[2], v[3]), row, col, ldo);
          v = v4f{f.x, f.y, f.z, f.w};
        }
        *reinterpret_cast<v4f*>(orow + col) = v;
      } else {
        const GemmEpi rest{nullptr, epi.addend, epi.pre_in, epi.pre_out, epi.act, epi.drop_token, epi.drop_threshold,
                           epi.drop_scale, epi.drop_seed, epi.pre16};
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (col + u < zto) orow[col + u] = col + u < N ? (more ? gemm_epilogue(rest, v[u], row, col + u, ldo) : v[u]) : 0.0f;
      }
    }
  }
  if constexpr (SUMS != 0) {
    // The four lane groups q hold disjoint K indices: added across q (fixed order), then written by
    // q = 0. Rows (SUMS 1): wm + 16 u + c (KC A) or wm + I c + u; columns (SUMS 2): wn + 16 u + c
    // (KC B) or wn + J c + u.
#pragma unroll
    for (int u = 0; u < SN; ++u) {
      ksum[u] += __shfl_xor(ksum[u], 16, 64);
      ksum[u] += __shfl_xor(ksum[u], 32, 64);
    }
    if (sum_wave && q == 0 && colsum) {
      const int64_t base = SUMS == 1 ? m0 + wm : n0 + wn, width = SUMS == 1 ? M : N;
      constexpr bool kc = SUMS == 1 ? AKC : BKC;
      constexpr int SPAN = SUMS == 1 ? I : J;
      float* dst = colsum + (ws ? int64_t(tz) * width : 0);
#pragma unroll
      for (int u = 0; u < SN; ++u) {
        const int64_t at = base + (kc ? 16 * u + c : SPAN * c + u);
        if (at < width) dst[at] = ksum[u];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// The mixed-precision GEMM on f16 operands in HBM (k_gemm_lds16): K tiles of 32 halves move straight
// into a 3-stage LDS ring as in k_gemm_lds, and v_mfma_f32_16x16x32_f16 takes 8 consecutive K of a
// row a lane, f32 accumulation.
//   - An operand contiguous along K (KC) is staged [row][32 K]: 64 bytes a row, its 16-byte chunk
//     kq at slot kq ^ ((row >> 2) & 3), so the 16 rows a quarter-wave reads at one chunk hit
//     distinct banks; lane (c, q) reads row c's chunk q with one 16-byte read.
//   - An operand contiguous along its rows is staged [K][rows] as in memory, the 16-byte chunk ch of
//     K row k at ch ^ 2 (k mod 4) within its group of 8 (128 bytes). A lane's 8 K of one row come
//     from two ds_read_b64_tr_b16: in each 16-lane group, source lane l reads 4 rows x 1 K (8 bytes)
//     at K row k0 + l / 4, rows base + 4 (l mod 4) .. + 3, and after the transpose lane c holds row
//     base + c at K k0 .. k0 + 3.
// Lane (c, q) thus supplies row c of its 16-row block at K 8q .. 8q + 7 in both layouts, and holds
// output rows 16 i + c, columns 16 j + 4 q .. + 3 (the MFMA takes B's fragment first: C^T tiles).
// K must be a multiple of 32, or the K-contiguous operands zero-padded to it; the K rows of an
// operand along its rows are clamped to the last (their products with the padding vanish).

template <int BM, int BN, int WGM, int WGN, bool AKC, bool BKC, int NS, int SUMS, int MF = 16, int BK = 32>
__global__ __launch_bounds__(64 * WGM * WGN) void k_gemm_lds16(GemmPtrs ptrs, int64_t M, int64_t N, int64_t K,
                                                               int64_t lda, int64_t ldb, int64_t ldc, int64_t kchunk,
                                                               int64_t zero_to, bool vo, GemmOrder order) {
  constexpr int W = WGM * WGN;
  static_assert(BK == 32 || BK == 64, "K tiles of 32 or 64 halves");
  constexpr int WTM = BM / WGM, WTN = BN / WGN, I = WTM / MF, J = WTN / MF;
  static_assert(MF == 16 || MF == 32, "16x16x32 or 32x32x16 MFMA blocks");
  static_assert(I >= 1 && J >= 1 && WTM % MF == 0 && WTN % MF == 0, "whole MFMA blocks a wave");
  // MFMA blocks of MF rows: 16x16x32 (KS = 1 K step of 32 a tile) or 32x32x16 (KS = 2 of 16).
  constexpr int KS = BK / (MF == 16 ? 32 : 16), NV = MF == 16 ? 4 : 16;
  // A K-contiguous tile's rows: CPR 16-byte chunks (BK 32: 64 bytes, BK 64: a whole 128-byte line),
  // RPI rows a 1 KB load instruction; chunk c of row r at slot c ^ swz(r).
  constexpr int CPR = BK / 8, RPI = 64 / CPR;
  typedef float vacc __attribute__((ext_vector_type(NV)));
  constexpr int SA = BM * BK, SB = BN * BK, SS = SA + SB;  // halves a stage
  constexpr int LA = SA / 512, LB = SB / 512;               // 1 KB wave load instructions a tile
  static_assert(LA % W == 0 && LB % W == 0, "whole load instructions a wave");
  constexpr int PA = LA / W, PB = LB / W, LPT = PA + PB;
  __shared__ __align__(16) _Float16 smem[NS * SS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, q = lane >> 4;
  const uint32_t per = gridDim.x / 8, tg = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (tg >= order.tiles * uint32_t(ptrs.count)) return;
  // The problem of the group, then its tile.
  const int qp = int(tg / order.tiles);
  const uint32_t t0 = tg - uint32_t(qp) * order.tiles;
  const uint32_t tz = t0 / (order.mt * order.nt), tr = t0 % (order.mt * order.nt);
  const uint32_t tm = order.m_fastest ? tr % order.mt : tr / order.nt;
  const uint32_t tn = order.m_fastest ? tr / order.mt : tr % order.nt;
  const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
  const int64_t kpad = (K + BK - 1) / BK * BK;
  const int64_t kbeg = int64_t(tz) * kchunk, kend = kpad < kbeg + kchunk ? kpad : kbeg + kchunk;
  const int tiles = int((kend - kbeg) / BK);
  const int wm = (wave / WGN) * WTM, wn = (wave % WGN) * WTN;
  const _Float16* __restrict__ A = ptrs.a16[qp];
  const _Float16* __restrict__ B = ptrs.b16[qp];
  const GemmEpi epi = ptrs.epi[qp];
  float* __restrict__ ws = ptrs.ws[qp];
  float* __restrict__ colsum = ptrs.colsum[qp];
  auto swz = [](int r) { return BK == 32 ? ((r >> 2) & 3) : (r & 7); };
  const int64_t kmax = K - 1;
  const _Float16* srcA[PA];
  const _Float16* srcB[PB];
  int kofA[PA], kofB[PB];
#pragma unroll
  for (int h = 0; h < PA; ++h) {
    const int t = wave * PA + h;
    if (AKC) {
      const int r = t * RPI + lane / CPR, ch = (lane % CPR) ^ swz(r);
      const int64_t row = m0 + r < M ? m0 + r : M - 1;
      srcA[h] = A + row * lda + kbeg + 8 * ch;
      kofA[h] = 0;
    } else {
      constexpr int RQ = BM / 8, KR = 512 / BM;
      const int kr = t * KR + lane / RQ, slot = lane % RQ;
      const int ch = (slot & ~7) | ((slot & 7) ^ (2 * (kr & 3)));
      int64_t col = m0 + 8 * ch;
      col = col < M ? col : ((M - 1) & ~int64_t(7));
      srcA[h] = A + col;
      kofA[h] = kr;
    }
  }
#pragma unroll
  for (int h = 0; h < PB; ++h) {
    const int t = wave * PB + h;
    if (BKC) {
      const int r = t * RPI + lane / CPR, ch = (lane % CPR) ^ swz(r);
      const int64_t row = n0 + r < N ? n0 + r : N - 1;
      srcB[h] = B + row * ldb + kbeg + 8 * ch;
      kofB[h] = 0;
    } else {
      constexpr int RQ = BN / 8, KR = 512 / BN;
      const int kr = t * KR + lane / RQ, slot = lane % RQ;
      const int ch = (slot & ~7) | ((slot & 7) ^ (2 * (kr & 3)));
      int64_t col = n0 + 8 * ch;
      col = col < N ? col : ((N - 1) & ~int64_t(7));
      srcB[h] = B + col;
      kofB[h] = kr;
    }
  }
  auto issue = [&](int tile) {
    tile = tile < tiles ? tile : tiles - 1;
    _Float16* st = smem + (tile % NS) * SS;
    const int64_t k0 = int64_t(tile) * BK;
#pragma unroll
    for (int h = 0; h < PA; ++h) {
      const int t = wave * PA + h;
      const int64_t kr = kbeg + k0 + kofA[h];
      const _Float16* src = AKC ? srcA[h] + k0 : srcA[h] + (kr < kmax ? kr : kmax) * lda;
      load_lds16(reinterpret_cast<const float*>(src), reinterpret_cast<float*>(st + t * 512));
    }
#pragma unroll
    for (int h = 0; h < PB; ++h) {
      const int t = wave * PB + h;
      const int64_t kr = kbeg + k0 + kofB[h];
      const _Float16* src = BKC ? srcB[h] + k0 : srcB[h] + (kr < kmax ? kr : kmax) * ldb;
      load_lds16(reinterpret_cast<const float*>(src), reinterpret_cast<float*>(st + SA + t * 512));
    }
  };
  vacc acc[I][J];
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < NV; ++e) acc[i][j][e] = 0.0f;
  // Lane roles. MF 16: lane (c = l mod 16, q = l / 16) supplies row c of a 16-row block at K
  // 8 q .. 8 q + 7. MF 32: lane (c = l mod 32, h = l / 32) supplies row c of a 32-row block at K
  // 16 ks + 8 h .. + 7 of K step ks. Either way the lane's 8 K are one 16-byte chunk kq (kq = q,
  // or 2 ks + h) of the row.
  const int fc = MF == 16 ? c : lane & 31, fh = MF == 16 ? q : lane >> 5;
  auto kc_frag = [&](const _Float16* S, int r, int kq) {
    return *reinterpret_cast<const v8h*>(S + r * BK + 8 * (kq ^ swz(r)));
  };
  // The LDS address of the transposed read of K rows k0 .. k0 + 3 of the 16 rows from base: in each
  // 16-lane group, source lane li reads K row k0 + li / 4, rows base + 4 (li mod 4) .. + 3.
  auto tr_at = [&](const _Float16* S, int R, int base, int k0) {
    const int k = k0 + c / 4;
    const int row = base + 4 * (c % 4);
    const int ch = row / 8, slot = (ch & ~7) | ((ch & 7) ^ (2 * (k & 3)));
    return lds_at(S + k * R + slot * 8 + (row % 8));
  };
  // The transposed reads (base row, first K row) of one 8-half fragment of this lane: MF 16, rows
  // base .. + 15 at K 8 q + {0, 4}; MF 32, rows base + 16 (g mod 2) .. (g = l / 16) at K
  // 16 ks + 8 (g / 2) + {0, 4}.
  auto tr_pair = [&](int base, int ks, int hh, int& rb, int& k0) {
    if constexpr (MF == 16) {
      rb = base;
      k0 = 32 * ks + 8 * q + 4 * hh;
    } else {
      rb = base + 16 * (q & 1);
      k0 = 16 * ks + 8 * (q >> 1) + 4 * hh;
    }
  };
  static_assert((AKC || (I * KS) % 4 == 0) && (BKC || (J * KS) % 4 == 0),
                "an operand along its rows takes its fragments in fours");
  // Fragments (ks, u) of an operand along its rows, rows base0 + MF u, eight transposed reads a group
  // of four.
  auto tr_frags = [&](const _Float16* S, int R, int base0, auto& out) {
    constexpr int U = sizeof(out[0]) / sizeof(out[0][0]);
    constexpr int G = KS * U / 4;
#pragma unroll
    for (int g4 = 0; g4 < G; ++g4) {
      uint32_t at[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int fi = 4 * g4 + e, ks = fi / U, u = fi % U;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          int rb, k0;
          tr_pair(base0 + MF * u, ks, hh, rb, k0);
          at[2 * e + hh] = tr_at(S, R, rb, k0);
        }
      }
      v4s16 r[8];
      tr_read16x8(at, r);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int fi = 4 * g4 + e, ks = fi / U, u = fi % U;
        const v4h16 lo = __builtin_bit_cast(v4h16, r[2 * e]), hi = __builtin_bit_cast(v4h16, r[2 * e + 1]);
        out[ks][u] = v8h{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  };
  struct Frag { v8h a[KS][I], b[KS][J]; };
  auto read = [&](int tile, Frag& f) {
    const _Float16* As = smem + (tile % NS) * SS;
    const _Float16* Bs = As + SA;
    if constexpr (AKC) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int i = 0; i < I; ++i) f.a[ks][i] = kc_frag(As, wm + MF * i + fc, MF == 16 ? 4 * ks + q : 2 * ks + fh);
    } else {
      tr_frags(As, BM, wm, f.a);
    }
    if constexpr (BKC) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < J; ++j) f.b[ks][j] = kc_frag(Bs, wn + MF * j + fc, MF == 16 ? 4 * ks + q : 2 * ks + fh);
    } else {
      tr_frags(Bs, BN, wn, f.b);
    }
  };
  // Sums over K of this lane's operand rows (SUMS 1: op(A)'s rows, 2: op(B)'s columns, i.e. the
  // fragments' rows), by the waves of the first wave column (row), which read every row of the
  // operand: the lane adds its 8 K of rows MF u + fc of the wave tile, in K order.
  constexpr int SN = SUMS == 1 ? I : SUMS == 2 ? J : 1;
  float ksum[SN];
#pragma unroll
  for (int u = 0; u < SN; ++u) ksum[u] = 0.0f;
  const bool sum_wave = SUMS == 1 ? wn == 0 : SUMS == 2 ? wm == 0 : false;
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) issue(p);
#pragma unroll 1
  for (int t = 0; t < tiles; ++t) {
    wait_vm((NS - 2) * LPT);
    __builtin_amdgcn_s_barrier();
    issue(t + NS - 1);
    Frag f;
    read(t, f);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int i = 0; i < I; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j) {
          if constexpr (MF == 16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.b[ks][j], f.a[ks][i], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.b[ks][j], f.a[ks][i], acc[i][j], 0, 0, 0);
        }
    if (SUMS != 0 && sum_wave) {
#pragma unroll
      for (int u = 0; u < SN; ++u) {
        // v_dot2_f32_f16 against (1, 1): two halves added into the f32 sum a VALU op.
        typedef _Float16 v2h_ __attribute__((ext_vector_type(2)));
        const v2h_ one{_Float16(1.0f), _Float16(1.0f)};
        float x = ksum[u];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const v8h h = SUMS == 1 ? f.a[ks][u] : f.b[ks][u];
#pragma unroll
          for (int e = 0; e < 4; ++e) x = __builtin_amdgcn_fdot2(v2h_{h[2 * e], h[2 * e + 1]}, one, x, false);
        }
        ksum[u] = x;
      }
    }
  }
  wait_vm(0);  // no load may still write LDS when the block ends
  float* out = ws ? ws + int64_t(tz) * M * N : ptrs.c[qp];
  _Float16* out16 = ws ? nullptr : ptrs.c16[qp];
  const int64_t ldo = ws ? N : ldc, zto = ws ? N : zero_to;
  const bool more = !ws && (epi.bias || epi.act != EPI_NONE || epi.addend || epi.drop_token);
  // Output element (row, col) of block (i, j): the MFMA took B's fragment first, so the lane holds
  // output row MF i + fc and, for each group g of 4 accumulators, the columns MF j + 8 g + 4 fh
  // (MF 32) or 16 j + 4 q (MF 16) .. + 3.
#pragma unroll
  for (int i = 0; i < I; ++i) {
    const int64_t row = m0 + wm + MF * i + fc;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int g = 0; g < NV / 4; ++g) {
        const int64_t col = n0 + wn + MF * j + (MF == 16 ? 4 * q : 8 * g + 4 * fh);
        float4 v = make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
        if (vo && col + 3 < N) {
          if (more) v = gemm_epilogue4(epi, v, row, col, ldo);
          if (out) *reinterpret_cast<float4*>(out + row * ldo + col) = v;
          if (out16)
            *reinterpret_cast<v4h16*>(out16 + row * ldo + col) =
                v4h16{_Float16(v.x), _Float16(v.y), _Float16(v.z), _Float16(v.w)};
        } else {
          const float vs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (col + u >= zto) continue;
            const float x = col + u < N ? (more ? gemm_epilogue(epi, vs[u], row, col + u, ldo) : vs[u]) : 0.0f;
            if (out) out[row * ldo + col + u] = x;
            if (out16) out16[row * ldo + col + u] = _Float16(x);
          }
        }
      }
  }
  if constexpr (SUMS != 0) {
    // The lane groups (q for MF 16, h for MF 32) hold disjoint K: added across them (fixed order),
    // written by group 0 at row (column) base + MF u + fc; split-K slices into the workspace's
    // sums, slice tz.
#pragma unroll
    for (int u = 0; u < SN; ++u) {
      if constexpr (MF == 16) ksum[u] += __shfl_xor(ksum[u], 16, 64);
      ksum[u] += __shfl_xor(ksum[u], 32, 64);
    }
    if (sum_wave && fh == 0 && colsum) {
      const int64_t base = SUMS == 1 ? m0 + wm : n0 + wn, width = SUMS == 1 ? M : N;
      float* dst = colsum + (ws ? int64_t(tz) * width : 0);
#pragma unroll
      for (int u = 0; u < SN; ++u) {
        const int64_t at = base + MF * u + fc;
        if (at < width) dst[at] = ksum[u];
      }
    }
  }
}

namespace {
// Whether k_gemm_lds can read this problem with K tiles of bk: 16-byte aligned operands and rows;
// a K tail only where every operand contiguous along K (KC) is zero-padded to the next multiple of
// bk (an operand not contiguous along K has its K rows clamped, which only a zero partner
// cancels), so both operands KC, or one KC and one clamped; the summed operand of a column sum
// over a K tail KC (padding, not clamped rows); an operand contiguous along its rows whole groups
// of 4 rows, or a pitch that holds the last group.
bool lds_fits(const GemmArgs& g, int bk) {
  const bool akc = !g.ta, bkc = g.tb;
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!a16(g.a) || !a16(g.b) || g.lda % 4 != 0 || g.ldb % 4 != 0) return false;
  const int64_t kpad = (g.k + bk - 1) / bk * bk;
  if (g.k % bk != 0) {
    if (!akc && !bkc) return false;
    if (akc && !(g.pad_a && g.lda >= kpad)) return false;
    if (bkc && !(g.pad_b && g.ldb >= kpad)) return false;
    if (g.colsum && !(g.sum_a ? akc : bkc)) return false;
  }
  auto rows_ok = [](bool kc, int64_t ld, int64_t extent) { return kc || extent % 4 == 0 || ld >= (extent + 3) / 4 * 4; };
  return rows_ok(akc, g.lda, g.m) && rows_ok(bkc, g.ldb, g.n);
}
}  // namespace

bool gemm_lds(hipStream_t s, const GemmArgs& g, const GemmPtrs& ptrs, int split, int64_t chunk) {
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  float* ws = ptrs.ws[0];
  const bool akc = !g.ta, bkc = g.tb;
  const int lds_bk = !bkc ? 32 : 16;  // the K tile of the configuration chosen below
  // Measured: faster for outputs of 2^21 or more (the decoder head, the FFN's 4096 x 512 products and
  // their input gradients) and K of 8192 or more; slower for the K = 4096 weight gradients of
  // 512 x 128 or smaller and the 4096 x 128 products. A cross-entropy head's fused variants (the
  // gradient formed from the logits in the K loop) stay on k_gemm_w.
  const bool lds = (g.m * g.n >= (int64_t(1) << 21) || g.k >= 8192) && chunk % lds_bk == 0 && lds_fits(g, lds_bk);
  if (lds) {
    // Tiles (measured on the decoder head shapes of BERT-tiny, 832 x 30522 x 128 and its two
    // gradients): both operands KC 64 x 64, A KC 64 x 128 with eight waves and K tiles of 32,
    // neither 128 x 128 (each wave 64 x 64: 16 accumulators) with K tiles of 32. A/B in one run on
    // one box (step ms): the weight gradient's K tiles of 32 against 16, 0.7604 against 0.7644; for
    // the forward K tiles of 32, 128 x 64 or 64 x 128 tiles, and for A KC 64 x 128 with four waves
    // (K tiles of 16 or 32) or 128 x 128, each 3-80 us a step slower.
    const int bm = akc && bkc ? 64 : akc ? 64 : !bkc ? 128 : 64;
    const int bn = akc && bkc ? 64 : akc ? 128 : !bkc ? 128 : 64;
    const int64_t lmt = (g.m + bm - 1) / bm, lnt = (g.n + bn - 1) / bn;
    const int64_t ltiles = lmt * lnt * split;
    if (ltiles > (int64_t(1) << 30)) bad("gemm has too many tiles");
    const GemmOrder lorder{uint32_t(lmt), uint32_t(lnt), uint32_t(ltiles), g.n * g.k >= g.m * g.k};
    const dim3 lgrid(unsigned((ltiles + 7) / 8 * 8));
    const bool lvo = ws ? (g.n % 4 == 0 && a16(ws))
                        : (g.ldc % 4 == 0 && a16(g.c) && a16(g.addend) && a16(g.pre_in) && a16(g.pre_out));
    const int64_t zero_to = g.pad_c ? g.ldc : g.n;
    const int sums = g.colsum ? (g.sum_a ? 1 : 2) : 0;
#define MSX_LDS(BM, BN, WGM, WGN, BK, AK, BKC_, NS, FP, S)                                                         \
  MSX_LAUNCH((k_gemm_lds<BM, BN, WGM, WGN, BK, AK, BKC_, NS, FP, S>), lgrid, dim3(64 * WGM * WGN), 0, s, ptrs, g.m, \
             g.n, g.k, g.lda, g.ldb, g.ldc, chunk, zero_to, lvo, lorder)
#define MSX_LDS_S(BM, BN, WGM, WGN, BK, AK, BKC_, NS, FP)          \
  if (sums == 1) MSX_LDS(BM, BN, WGM, WGN, BK, AK, BKC_, NS, FP, 1); \
  else if (sums == 2) MSX_LDS(BM, BN, WGM, WGN, BK, AK, BKC_, NS, FP, 2); \
  else MSX_LDS(BM, BN, WGM, WGN, BK, AK, BKC_, NS, FP, 0)
    if (akc && bkc) { MSX_LDS_S(64, 64, 2, 2, 16, true, true, 3, true); }
    else if (akc) { MSX_LDS_S(64, 128, 2, 4, 32, true, false, 3, true); }
    else if (!bkc) { MSX_LDS_S(128, 128, 2, 2, 32, false, false, 3, false); }
    else { MSX_LDS_S(64, 64, 2, 2, 16, false, true, 3, true); }
#undef MSX_LDS_S
#undef MSX_LDS
    return true;
  }
  return false;
}

bool lds16_layout(const GemmArgs& o, int64_t chunk) {
  constexpr int BK = 32;
  const bool akc = !o.ta, bkc = o.tb;
  const int64_t kpad = (o.k + BK - 1) / BK * BK;
  if (chunk % BK != 0 || o.lda % 8 != 0 || o.ldb % 8 != 0) return false;
  // A K tail only over zero padding of the K-contiguous operands (the other kind is clamped, and
  // a summed operand's clamped rows would enter its sums).
  if (o.k % BK != 0 && ((!akc && !bkc) || (akc && !(o.pad_a && o.lda >= kpad)) || (bkc && !(o.pad_b && o.ldb >= kpad)) ||
                        (o.colsum && !(o.sum_a ? akc : bkc))))
    return false;
  // An operand along its rows: whole 8-row chunks, or a pitch that holds the last one.
  if (!akc && o.m % 8 != 0 && o.lda < (o.m + 7) / 8 * 8) return false;
  if (!bkc && o.n % 8 != 0 && o.ldb < (o.n + 7) / 8 * 8) return false;
  return true;
}

bool gemm_lds16(hipStream_t s, const GemmArgs* list, int count, const GemmPtrs& ptrs, int split, int64_t chunk) {
  const GemmArgs& g = list[0];
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool akc = !g.ta, bkc = g.tb;
  for (int q = 0; q < count; ++q) {
    const GemmArgs& o = list[q];
    if (!o.a16 || !o.b16 || !a16(o.a16) || !a16(o.b16) || !lds16_layout(o, chunk)) return false;
  }
  constexpr int BM = 128, BN = 128;
  const int64_t lmt = (g.m + BM - 1) / BM, lnt = (g.n + BN - 1) / BN;
  const int64_t ltiles = lmt * lnt * split;
  if (ltiles * count > (int64_t(1) << 30)) bad("gemm has too many tiles");
  const GemmOrder lorder{uint32_t(lmt), uint32_t(lnt), uint32_t(ltiles), g.n * g.k >= g.m * g.k};
  const dim3 lgrid(unsigned((ltiles * count + 7) / 8 * 8));
  bool vo = true;
  for (int q = 0; q < count; ++q) {
    const GemmArgs& o = list[q];
    vo = vo && (ptrs.ws[q] ? (o.n % 4 == 0 && a16(ptrs.ws[q]))
                           : (o.ldc % 4 == 0 && a16(o.c) && a16(o.c16) && a16(o.bias) && a16(o.addend) && a16(o.pre_in) &&
                              a16(o.pre_out) && a16(o.pre16)));
  }
  const int64_t zero_to = g.pad_c ? g.ldc : g.n;
  const int sums = g.colsum ? (g.sum_a ? 1 : 2) : 0;
  // 128x128 tiles, 2x2 waves, K tiles of 32 in a 2-stage ring, 16x16x32 blocks. Measured on the
  // BERT-base step, A/B in one run on one box: a 3-stage ring 23.43 ms (2 stages 23.18); 32x32x16
  // blocks 25.45; 4 stages 26.30; 256x128, 128x256 and 256x256 tiles 26.0, 25.8 and 26.6; K tiles
  // of 64 (whole 128-byte rows of a K-contiguous operand a load) 24.6.
#define MSX_L16S(AK, BKC_, S)                                                                                         \
  MSX_LAUNCH((k_gemm_lds16<BM, BN, 2, 2, AK, BKC_, 2, S, 16, 32>), lgrid, dim3(256), 0, s, ptrs, g.m, g.n, g.k, g.lda, \
             g.ldb, g.ldc, chunk, zero_to, vo, lorder);
#define MSX_L16(AK, BKC_)                  \
  if (sums == 1) { MSX_L16S(AK, BKC_, 1) }      \
  else if (sums == 2) { MSX_L16S(AK, BKC_, 2) } \
  else { MSX_L16S(AK, BKC_, 0) }
  if (akc && bkc) { MSX_L16(true, true); }
  else if (akc) { MSX_L16(true, false); }
  else if (bkc) { MSX_L16(false, true); }
  else { MSX_L16(false, false); }
#undef MSX_L16
#undef MSX_L16S
  return true;
}

}  // namespace msx::hk
