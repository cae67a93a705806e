// EmbeddingGrad as a sorted-segment scatter-add (gfx950, wave64): deterministic, no float atomics,
// bit-exact with the reference's sequential accumulation (interpreter.rs:931-941: out starts at
// +0 and out[ids[k]] += g[k] for ascending k, one f32 rounding per add).
//
// Two launches a step. eg_plan (one 1024-thread block per table, run once the ids exist) groups
// the positions by id: a counting sort through an LDS histogram of the table's rows (integer
// atomics: exact counts, positions within a segment in no particular order), or, for a table
// too large for the histogram, a block radix sort. It lists each distinct id's segment of
// positions, short (at most kShortMax positions) or long, and marks the rows some id names in a
// bitmap. eg_apply (every table of the same gradient in one launch) then writes each table row
// exactly once, restoring ascending position order inside each segment before adding:
//   - a short segment: one wave sorts its positions across lanes, then with lanes over columns
//     loads the segment's rows together and adds them in position order;
//   - a long segment (a frequent id, or the padding slots that all name row 0): one block per
//     32-column group takes the positions in ascending order (as listed by a sorted plan, or
//     ordered through an LDS bitmap of all n positions), then stages 256 rows a round through LDS
//     with every thread, leaving out rows that are all zeros in the group, while one lane a column
//     adds the staged rows in position order and the next round's loads are in flight;
//   - the rows no id names: 32-row stripes of zeros (or of the addend).
// The work per row is the reference's; only who adds which column differs.
#include "kernels.h"
#include "device.h"

#include <rocprim/block/block_radix_sort.hpp>
#include <rocprim/block/block_scan.hpp>

#include <algorithm>
#include <vector>

namespace msx::hk {

namespace {
constexpr int kPlanThreads = 1024;
constexpr int kShortMax = 16;    // positions a short segment holds at most
constexpr int kLongCols = 32;    // columns of one long-segment block
constexpr int kLongRows = 256;   // positions a long-segment block stages a round (one a thread)
constexpr int kTilePitch = 36;   // floats a staged row takes in LDS (32 + 4: float4 stores spread over banks)
#ifndef MSX_EG_ADD_BATCH
#define MSX_EG_ADD_BATCH 32
#endif
constexpr int kAddBatch = MSX_EG_ADD_BATCH;  // staged values a column reads ahead of its adds
constexpr int kApplyThreads = 256;
constexpr int kCountRows = 36864;
constexpr int kMaxPositions = 16384;  // ids a table's EmbeddingGrad takes on this path (apply)
constexpr int kPlanPositions = 8192;  // ids the device radix plan takes (the counting plan: kMaxPositions)

int bit_length(uint64_t v) {
  int b = 0;
  while (v) { ++b; v >>= 1; }
  return b;
}

// Word offsets of one table's plan in its buffer.
struct PlanLayout {
  int64_t counts, order, seg_start, seg_id, longs, covered, words;
  __host__ __device__ PlanLayout(int64_t n, int64_t rows) {
    counts = 0;  // [0] segments, [1] segments the short region walks, [2] long segments,
                 // [3] positions, [4] 1 when each segment's positions are listed ascending
    order = 8;
    seg_start = order + n;
    seg_id = seg_start + n + 1;
    longs = seg_id + n;
    covered = longs + n;
    words = covered + (rows + 31) / 32;
  }
};
}  // namespace

bool eg_sorted_fits(int64_t n, int64_t rows) {
  if (n <= 0 || n > kMaxPositions || rows <= 0) return false;
  const int pb = bit_length(uint64_t(n - 1)) > 0 ? bit_length(uint64_t(n - 1)) : 1;
  return pb + bit_length(uint64_t(rows)) <= 32;
}
bool eg_device_plan_fits(int64_t n, int64_t rows) {
  return (rows <= kCountRows ? n <= kMaxPositions : n <= kPlanPositions) && eg_sorted_fits(n, rows);
}

size_t eg_plan_bytes(int64_t n, int64_t rows) { return size_t(PlanLayout(n, rows).words) * 4; }

// ---------------------------------------------------------------------------------------------
// The wave-aggregated append of `flag` lanes to an LDS-counted list: one atomic a wave; returns
// the lane's slot (valid where flag holds).
__device__ __forceinline__ int wave_append(bool flag, int* counter, int lane) {
  const uint64_t bal = __ballot(flag);
  int base = 0;
  if (bal) {
    const int leader = __ffsll((unsigned long long)bal) - 1;
    if (lane == leader) base = atomicAdd(counter, __popcll(bal));
    base = __shfl(base, leader, 64);
  }
  return base + __popcll(bal & ((uint64_t(1) << lane) - 1));
}

// The inclusive prefix sum of v over the lanes of a wave.
__device__ __forceinline__ int wave_inclusive_sum(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(v, d, 64);
    v += lane >= d ? t : 0;
  }
  return v;
}

// Counting plan: counts[rows] in LDS by integer atomics, then each of the 16 waves walks its
// contiguous range of rows 64 at a time (one lane a row): prefix sums give every row's base and
// segment index, ballots the covered bitmap's words.
__global__ __launch_bounds__(kPlanThreads) void k_eg_plan_count(EgPlanSet set) {
  const EgPlanJob j = set.job[blockIdx.x];
  using Scan = rocprim::block_scan<uint64_t, kPlanThreads>;
  __shared__ typename Scan::storage_type scan_lds;
  extern __shared__ uint32_t counts[];  // [rows]: counts, then each row's segment base; then the
                                        // covered bitmap [words]
  const int n = j.n, rows = j.rows, words = (rows + 31) / 32;
  uint32_t* named_rows = counts + rows;
  const PlanLayout L(n, rows);
  int32_t* out = j.plan;
  const int tid = threadIdx.x, lane = tid & 63;
  for (int r = tid; r < rows; r += kPlanThreads) counts[r] = 0;
  for (int w = tid; w < words; w += kPlanThreads) named_rows[w] = 0;
  // Every id load in flight before the first atomic.
  constexpr int kMaxPer = kMaxPositions / kPlanThreads;
  int32_t id_of[kMaxPer], slot[kMaxPer];
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int i = tid + k * kPlanThreads;
    id_of[k] = i < n ? j.ids[i] : -1;
  }
  __syncthreads();
  // Each position's slot within its id's segment, in arrival order.
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    if (id_of[k] < 0 || id_of[k] >= rows) id_of[k] = -1;
    else slot[k] = int(atomicAdd(&counts[id_of[k]], 1u));
  }
  __syncthreads();
  // Thread t owns the rows [t*per, t*per + per): their counts in registers; positions, named
  // rows and long segments counted in 16-bit fields of one 64-bit value, scanned over the block
  // once (each count is at most 16384).
  constexpr int kMaxRowsPer = kCountRows / kPlanThreads;
  const int per = (rows + kPlanThreads - 1) / kPlanThreads;
  const int r0 = tid * per;
  int cnt[kMaxRowsPer];
  uint64_t packed = 0;
#pragma unroll
  for (int k = 0; k < kMaxRowsPer; ++k) {
    cnt[k] = (k < per && r0 + k < rows) ? int(counts[r0 + k]) : 0;
    packed += uint64_t(cnt[k]) + (cnt[k] ? (uint64_t(1) << 16) : 0) + (cnt[k] > kShortMax ? (uint64_t(1) << 32) : 0);
  }
  uint64_t base = 0, all = 0;
  Scan().exclusive_scan(packed, base, uint64_t(0), all, scan_lds);
  const int all_pos = int(all & 0xFFFF), all_seg = int((all >> 16) & 0xFFFF), all_long = int(all >> 32);
  int pos_base = int(base & 0xFFFF), seg = int((base >> 16) & 0xFFFF), lng = int(base >> 32);
#pragma unroll
  for (int k = 0; k < kMaxRowsPer; ++k) {
    const int r = r0 + k;
    if (k >= per || r >= rows) continue;
    const int c = cnt[k];
    counts[r] = uint32_t(pos_base);
    if (c) {
      out[L.seg_start + seg] = pos_base;
      out[L.seg_id + seg] = r;
      atomicOr(&named_rows[r >> 5], 1u << (r & 31));
      if (c > kShortMax) out[L.longs + lng++] = seg;
      ++seg;
    }
    pos_base += c;
  }
  if (tid == 0) out[L.seg_start + all_seg] = all_pos;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k)
    if (id_of[k] >= 0) out[L.order + int(counts[id_of[k]]) + slot[k]] = tid + k * kPlanThreads;
  for (int w = tid; w < words; w += kPlanThreads) out[L.covered + w] = int32_t(named_rows[w]);
  if (tid == 0) {
    out[L.counts + 0] = all_seg;
    out[L.counts + 1] = all_seg;  // the short region walks every segment and skips the long ones
    out[L.counts + 2] = all_long;
    out[L.counts + 3] = all_pos;
    out[L.counts + 4] = 0;  // positions within a segment in arrival order
  }
}

template <int IT>
__global__ __launch_bounds__(kPlanThreads) void k_eg_plan(EgPlanSet set) {
  const EgPlanJob j = set.job[blockIdx.x];
  using Sort = rocprim::block_radix_sort<uint32_t, kPlanThreads, IT, uint32_t>;
  using Scan = rocprim::block_scan<int, kPlanThreads>;
  __shared__ typename Sort::storage_type sort_lds;
  __shared__ typename Scan::storage_type scan_lds;
  __shared__ uint32_t keys_lds[kPlanThreads * IT];
  __shared__ int n_valid, n_long;
  extern __shared__ uint32_t dyn[];
  const int n = j.n, rows = j.rows, words = (rows + 31) / 32;
  int32_t* starts = reinterpret_cast<int32_t*>(dyn);  // [n + 1] segment starts in sorted order
  uint32_t* covered = dyn + (n + 1);                    // [words] rows some id names
  const PlanLayout L(n, rows);
  int32_t* out = j.plan;
  const int tid = threadIdx.x;
  const int pb = j.pos_bits, ebits = j.key_bits;
  for (int w = tid; w < words; w += kPlanThreads) covered[w] = 0;
  if (tid == 0) { n_valid = 0; n_long = 0; }
  // Sorted by id alone with the position as the value: the radix sort is stable and the positions
  // enter in ascending order, so each id's positions leave ascending. An out-of-range id or a slot
  // past n takes the key 2^idbits - 1, above every row, and sorts last. The key then becomes the
  // id above the position bits.
  const uint32_t none = (1u << (ebits - pb)) - 1u;
  uint32_t key[IT], val[IT];
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int i = tid * IT + k;
    key[k] = none;
    val[k] = uint32_t(i);
    if (i < n) {
      const int32_t id = j.ids[i];
      if (id >= 0 && id < rows) key[k] = uint32_t(id);
    }
  }
  __syncthreads();
  Sort().sort(key, val, sort_lds, 0, unsigned(ebits - pb));
#pragma unroll
  for (int k = 0; k < IT; ++k) key[k] = key[k] == none ? 0xFFFFFFFFu : (key[k] << pb) | val[k];
#pragma unroll
  for (int k = 0; k < IT; ++k) keys_lds[tid * IT + k] = key[k];
  __syncthreads();
  int flags = 0, valid = 0;
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int i = tid * IT + k;
    const bool ok = key[k] != 0xFFFFFFFFu;
    valid += ok ? 1 : 0;
    flags += (ok && (i == 0 || (keys_lds[i - 1] >> pb) != (key[k] >> pb))) ? 1 : 0;
  }
  int base = 0, segments = 0;
  Scan().exclusive_scan(flags, base, 0, segments, scan_lds);
  // The valid keys sort first: the last one's slot + 1 is their count.
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int i = tid * IT + k;
    if (key[k] != 0xFFFFFFFFu && (i + 1 == kPlanThreads * IT || keys_lds[i + 1] == 0xFFFFFFFFu)) n_valid = i + 1;
  }
#pragma unroll
  for (int k = 0; k < IT; ++k) {
    const int i = tid * IT + k;
    if (key[k] == 0xFFFFFFFFu) continue;
    const uint32_t id = key[k] >> pb;
    out[L.order + i] = int32_t(key[k] & ((1u << pb) - 1u));
    if (i == 0 || (keys_lds[i - 1] >> pb) != id) {
      starts[base] = i;
      out[L.seg_id + base] = int32_t(id);
      atomicOr(&covered[id >> 5], 1u << (id & 31u));
      ++base;
    }
  }
  __syncthreads();
  if (tid == 0) starts[segments] = n_valid;
  __syncthreads();
  // The long list: one LDS atomic a wave.
  for (int s0 = 0; s0 <= segments; s0 += kPlanThreads) {
    const int s = s0 + tid;
    if (s <= segments) out[L.seg_start + s] = starts[s];
    const bool is_long = s < segments && starts[s + 1] - starts[s] > kShortMax;
    const int ql = wave_append(is_long, &n_long, tid & 63);
    if (is_long) out[L.longs + ql] = s;
  }
  __syncthreads();
  for (int w = tid; w < words; w += kPlanThreads) out[L.covered + w] = int32_t(covered[w]);
  __syncthreads();
  if (tid == 0) {
    out[L.counts + 0] = segments;
    out[L.counts + 1] = segments;
    out[L.counts + 2] = n_long;
    out[L.counts + 3] = n_valid;
    out[L.counts + 4] = 1;  // the stable sort keeps positions ascending
  }
}

void eg_plan_host(const int32_t* ids, int32_t n, int32_t rows, int32_t* out) {
  if (!eg_sorted_fits(n, rows)) bad("eg_plan_host: ids or table too large for the plan");
  const PlanLayout L(n, rows);
  // Counting sort by id: counts, then each named row's first slot; positions enter ascending.
  std::vector<int32_t> base(size_t(rows) + 1, 0);
  for (int32_t i = 0; i < n; ++i)
    if (ids[i] >= 0 && ids[i] < rows) ++base[size_t(ids[i]) + 1];
  int32_t seg = 0, lng = 0;
  const int32_t words = (rows + 31) / 32;
  for (int32_t w = 0; w < words; ++w) out[L.covered + w] = 0;
  for (int32_t r = 0; r < rows; ++r) {
    const int32_t c = base[size_t(r) + 1];
    base[size_t(r) + 1] = base[size_t(r)] + c;
    if (c) {
      out[L.seg_start + seg] = base[size_t(r)];
      out[L.seg_id + seg] = r;
      out[L.covered + (r >> 5)] |= int32_t(1u << (r & 31));
      if (c > kShortMax) out[L.longs + lng++] = seg;
      ++seg;
    }
  }
  const int32_t all_pos = base[size_t(rows)];
  out[L.seg_start + seg] = all_pos;
  for (int32_t i = 0; i < n; ++i)
    if (ids[i] >= 0 && ids[i] < rows) out[L.order + base[size_t(ids[i])]++] = i;
  out[L.counts + 0] = seg;
  out[L.counts + 1] = seg;  // the short region walks every segment and skips the long ones
  out[L.counts + 2] = lng;
  out[L.counts + 3] = all_pos;
  out[L.counts + 4] = 1;
}

void eg_plan(hipStream_t s, const EgPlanJob* jobs, int njobs) {
  if (njobs <= 0) return;
  if (njobs > kEgJobs) bad("eg_plan: too many tables");
  EgPlanSet set{};
  int64_t max_n = 0, dyn = 0;
  for (int q = 0; q < njobs; ++q) {
    EgPlanJob j = jobs[q];
    if (!eg_device_plan_fits(j.n, j.rows)) bad("eg_plan: ids or table too large for the block sort");
    j.pos_bits = std::max(1, bit_length(uint64_t(j.n - 1)));
    j.key_bits = j.pos_bits + bit_length(uint64_t(j.rows));
    set.job[q] = j;
    max_n = std::max<int64_t>(max_n, j.n);
    dyn = std::max<int64_t>(dyn, (j.n + 1 + (j.rows + 31) / 32) * 4);
  }
  set.count = njobs;
  int64_t max_rows = 0;
  for (int q = 0; q < njobs; ++q) max_rows = std::max<int64_t>(max_rows, set.job[q].rows);
  if (max_rows <= kCountRows) {
    static bool raised = false;
    if (!raised) {
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_eg_plan_count),
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              (kCountRows + kCountRows / 32) * 4) != hipSuccess)
        bad("eg_plan: the LDS histogram's size was refused");
      raised = true;
    }
    MSX_LAUNCH(k_eg_plan_count, dim3(unsigned(njobs)), dim3(kPlanThreads), size_t(max_rows + (max_rows + 31) / 32) * 4,
               s, set);
  } else if (max_n <= 4096) {
    MSX_LAUNCH(k_eg_plan<4>, dim3(unsigned(njobs)), dim3(kPlanThreads), size_t(dyn), s, set);
  } else {
    MSX_LAUNCH(k_eg_plan<8>, dim3(unsigned(njobs)), dim3(kPlanThreads), size_t(dyn), s, set);
  }
}

// ---------------------------------------------------------------------------------------------
namespace {
template <int V> struct Vec;
template <> struct Vec<1> {
  using T = float;
  static __device__ __forceinline__ T zero() { return 0.0f; }
  static __device__ __forceinline__ T add(T a, T b) { return a + b; }
};
template <> struct Vec<2> {
  using T = float2;
  static __device__ __forceinline__ T zero() { return make_float2(0.0f, 0.0f); }
  static __device__ __forceinline__ T add(T a, T b) { return make_float2(a.x + b.x, a.y + b.y); }
};
template <> struct Vec<4> {
  using T = float4;
  static __device__ __forceinline__ T zero() { return make_float4(0.0f, 0.0f, 0.0f, 0.0f); }
  static __device__ __forceinline__ T add(T a, T b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
};

// out2 = DropoutGrad(out) for the V consecutive elements from `at` (their values v), when asked.
template <int V>
__device__ __forceinline__ void put_dropped(const EgApplyJob& j, int64_t at, const float* v) {
  if (!j.out2) return;
  const uint32_t tl = uint32_t(j.drop_token[0]), th = uint32_t(j.drop_token[1]);
  float o[V];
#pragma unroll
  for (int u = 0; u < V; ++u) {
    const uint32_t w = philox_w0(uint32_t(at + u), 4u, tl, th, uint32_t(j.seed), uint32_t(j.seed >> 32));
    o[u] = uint64_t(w) >= j.drop_threshold ? v[u] * j.drop_scale : 0.0f;
  }
  if constexpr (V == 4) *reinterpret_cast<float4*>(j.out2 + at) = make_float4(o[0], o[1], o[2], o[3]);
  else if constexpr (V == 2) *reinterpret_cast<float2*>(j.out2 + at) = make_float2(o[0], o[1]);
  else j.out2[at] = o[0];
}

// A short segment: one wave; lane l takes columns c0 + l*V .. + V - 1 of each 64*V-column pass.
template <int V>
__device__ __forceinline__ void short_segment(const EgApplyJob& j, const int32_t* plan, const PlanLayout& L, int q,
                                              int lane) {
  using W = Vec<V>;
  using T = typename W::T;
  const int seg = q;
  const int st = plan[L.seg_start + seg];
  const int len = plan[L.seg_start + seg + 1] - st;
  if (len > kShortMax) return;  // a long segment: the long region's
  const int64_t id = plan[L.seg_id + seg];
  const int64_t h = j.h;
  // The segment's positions in ascending order: lane l < len holds one, finds its rank among
  // them and pushes it to the lane of that rank; then every lane takes them all.
  const int mine = plan[L.order + st + (lane < len ? lane : 0)];
  int rank = 0;
#pragma unroll
  for (int k = 0; k < kShortMax; ++k) {
    const int other = __shfl(mine, k, 64);
    rank += (k < len && other < mine) ? 1 : 0;
  }
  const int sorted = __builtin_amdgcn_ds_permute((lane < len ? rank : lane) * 4, mine);
  int32_t pos[kShortMax];
#pragma unroll
  for (int k = 0; k < kShortMax; ++k) pos[k] = __shfl(sorted, k < len ? k : 0, 64);
  for (int64_t c0 = 0; c0 < h; c0 += 64 * V) {
    const int64_t c = c0 + int64_t(lane) * V;
    if (c >= h) break;
    T v[kShortMax];
#pragma unroll
    for (int k = 0; k < kShortMax; ++k)
      if (k < len) v[k] = *reinterpret_cast<const T*>(j.g + int64_t(pos[k]) * h + c);
    T acc = W::zero();
#pragma unroll
    for (int k = 0; k < kShortMax; ++k)
      if (k < len) acc = W::add(acc, v[k]);
    if (j.addend) acc = W::add(*reinterpret_cast<const T*>(j.addend + id * h + c), acc);
    *reinterpret_cast<T*>(j.out + id * h + c) = acc;
    put_dropped<V>(j, id * h + c, reinterpret_cast<const float*>(&acc));
  }
}

// The position of rank k among a long segment's: the bitmap `bm` of its positions (nw words) and
// the exclusive prefix `pre` of the words' bit counts; the word is the last whose prefix is at most
// k, the position its (k - prefix)-th set bit.
__device__ __forceinline__ int position_of_rank(int k, const int* pre, const uint32_t* bm, int nw) {
  int lo = 0, hi = nw - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= k) lo = mid;
    else hi = mid - 1;
  }
  uint32_t word = bm[lo];
  for (int need = k - pre[lo]; need > 0; --need) word &= word - 1;
  return lo * 32 + __ffs(int(word)) - 1;
}

// The positions of ranks r0 .. r0 + 255 of a long segment, columns [c_lo, c_lo + cw): thread t's
// row in registers (8 float4 when the group is whole and aligned). With `ordered` the segment's
// positions are listed ascending at `ord`; otherwise ranks come from the bitmap.
struct LongRow { float4 v[kLongCols / 4]; };
__device__ __forceinline__ LongRow long_load(const EgApplyJob& j, bool ordered, const int32_t* ord, const int* pre,
                                             const uint32_t* bm, int nw, int len, int r0, int64_t c_lo, int cw,
                                             bool vec, int t) {
  LongRow r;
  const int k = r0 + t;
  if (k < len) {
    const int p = ordered ? ord[k] : position_of_rank(k, pre, bm, nw);
    const float* src = j.g + int64_t(p) * j.h + c_lo;
    if (vec) {
#pragma unroll
      for (int u = 0; u < kLongCols / 4; ++u) r.v[u] = reinterpret_cast<const float4*>(src)[u];
    } else {
      float* f = reinterpret_cast<float*>(r.v);
#pragma unroll
      for (int u = 0; u < kLongCols; ++u) f[u] = u < cw ? src[u] : 0.0f;
    }
  }
  return r;
}
}  // namespace

__global__ __launch_bounds__(kApplyThreads) void k_eg_apply(EgApplySet set) {
  __shared__ float tile[kLongRows * kTilePitch];
  __shared__ uint32_t bm[kMaxPositions / 32];
  __shared__ int pre[kMaxPositions / 32];
  using WordScan = rocprim::block_scan<int, kApplyThreads>;
  __shared__ typename WordScan::storage_type word_scan;
  int b = int(blockIdx.x), q = 0;
  while (q + 1 < set.count && b >= set.job[q].blocks) b -= set.job[q++].blocks;
  const EgApplyJob& j = set.job[q];
  const PlanLayout L(j.n, j.rows);
  const int32_t* plan = j.plan;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t h = j.h;
  // The long segments' blocks come first in the job's range: their order-keeping add chains are
  // the longest work of the launch, so they start before the short segments and stripes.
  if (b >= j.blocks_long && b < j.blocks_long + j.blocks_short) {
    const int s = (b - j.blocks_long) * (kApplyThreads / 64) + wave;
    if (s >= plan[L.counts + 1]) return;
    if (j.vec == 4) short_segment<4>(j, plan, L, s, lane);
    else if (j.vec == 2) short_segment<2>(j, plan, L, s, lane);
    else short_segment<1>(j, plan, L, s, lane);
    return;
  }
  if (b < j.blocks_long) {
    const int groups = int((h + kLongCols - 1) / kLongCols);
    if (b >= plan[L.counts + 2] * groups) return;
    const int seg = plan[L.longs + b / groups];
    const int64_t c_lo = int64_t(b % groups) * kLongCols;
    const int cw = int(std::min<int64_t>(kLongCols, h - c_lo));
    const bool vec = cw == kLongCols && (h & 3) == 0;
    const int st = plan[L.seg_start + seg];
    const int len = plan[L.seg_start + seg + 1] - st;
    const int64_t id = plan[L.seg_id + seg];
    const int nw = (j.n + 31) / 32;
    const bool ordered = plan[L.counts + 4] != 0;
    const int32_t* ord = plan + L.order + st;
    if (!ordered) {
      // The segment's positions into a bitmap of all n, then each word's rank base.
      for (int w = tid; w < nw; w += kApplyThreads) bm[w] = 0;
      __syncthreads();
      for (int k = tid; k < len; k += kApplyThreads) {
        const int p = ord[k];
        atomicOr(&bm[p >> 5], 1u << (p & 31));
      }
      __syncthreads();
      for (int w0 = 0; w0 < nw; w0 += kApplyThreads) {
        const int w = w0 + tid;
        int base = 0, all = 0;
        WordScan().exclusive_scan(w < nw ? __popc(bm[w]) : 0, base, 0, all, word_scan);
        if (w < nw) pre[w] = base + (w0 ? pre[w0 - 1] + __popc(bm[w0 - 1]) : 0);
        __syncthreads();
      }
    }
    // Rows whose values in this column group are all +0 or -0 are left out of the add chain. From
    // the +0 start the running sum is never -0 (an exact zero from nonzero operands rounds to +0,
    // and +0 + -0 is +0), so adding a zero of either sign leaves it unchanged: the sum over the
    // remaining rows, in position order, is the reference's bit for bit. The padding slots of a
    // masked-row gather (weight 0, all naming row 0) make such a segment with no adds at all.
    float acc = 0.0f;
    LongRow r = long_load(j, ordered, ord, pre, bm, nw, len, 0, c_lo, cw, vec, tid);
    for (int r0 = 0; r0 < len; r0 += kLongRows) {
      bool nz = false;
      if (r0 + tid < len) {
#pragma unroll
        for (int u = 0; u < kLongCols / 4; ++u)
          nz |= r.v[u].x != 0.0f || r.v[u].y != 0.0f || r.v[u].z != 0.0f || r.v[u].w != 0.0f;
      }
      __syncthreads();  // the previous round's adds are done with the tile
      int slot = 0, cnt = 0;
      WordScan().exclusive_scan(nz ? 1 : 0, slot, 0, cnt, word_scan);
      if (nz) {
#pragma unroll
        for (int u = 0; u < kLongCols / 4; ++u) *reinterpret_cast<float4*>(&tile[slot * kTilePitch + 4 * u]) = r.v[u];
      }
      __syncthreads();
      if (r0 + kLongRows < len)
        r = long_load(j, ordered, ord, pre, bm, nw, len, r0 + kLongRows, c_lo, cw, vec, tid);
      if (tid < cw) {
        int rr = 0;
        // kAddBatch staged values read ahead of their adds: the adds are one dependent chain, and
        // the reads' latency is paid once a batch.
        for (; rr + kAddBatch <= cnt; rr += kAddBatch) {
          float t[kAddBatch];
#pragma unroll
          for (int u = 0; u < kAddBatch; ++u) t[u] = tile[(rr + u) * kTilePitch + tid];
#pragma unroll
          for (int u = 0; u < kAddBatch; ++u) acc = acc + t[u];
        }
        for (; rr < cnt; ++rr) acc = acc + tile[rr * kTilePitch + tid];
      }
    }
    if (tid < cw) {
      const int64_t at = id * h + c_lo + tid;
      const float v = j.addend ? j.addend[at] + acc : acc;
      j.out[at] = v;
      put_dropped<1>(j, at, &v);
    }
    return;
  }
  b -= j.blocks_long + j.blocks_short;
  // A stripe of 32 rows: the rows no id names are +0, or the addend's row + 0 (-0 becomes +0 as
  // the reference's zero-initialised sum added to it would make it).
  const int64_t z0 = int64_t(b) * 32, z1 = std::min<int64_t>(j.rows, z0 + 32);
  if (z0 >= z1) return;
  const uint32_t m = uint32_t(plan[L.covered + b]);
  if (m == 0xFFFFFFFFu) return;
  if ((h & 3) == 0) {
    const int64_t h4 = h >> 2, cells = (z1 - z0) * h4;
    float4* o4 = reinterpret_cast<float4*>(j.out + z0 * h);
    const float4* a4 = j.addend ? reinterpret_cast<const float4*>(j.addend + z0 * h) : nullptr;
    for (int64_t e = tid; e < cells; e += kApplyThreads) {
      if ((m >> uint32_t(e / h4)) & 1u) continue;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (a4) {
        const float4 a = a4[e];
        v = make_float4(a.x + 0.0f, a.y + 0.0f, a.z + 0.0f, a.w + 0.0f);
      }
      o4[e] = v;
      put_dropped<4>(j, z0 * h + 4 * e, reinterpret_cast<const float*>(&v));
    }
  } else {
    const int64_t cells = (z1 - z0) * h;
    for (int64_t e = tid; e < cells; e += kApplyThreads) {
      if ((m >> uint32_t(e / h)) & 1u) continue;
      const float v = j.addend ? j.addend[z0 * h + e] + 0.0f : 0.0f;
      j.out[z0 * h + e] = v;
      put_dropped<1>(j, z0 * h + e, &v);
    }
  }
}

void eg_apply(hipStream_t s, const EgApplyJob* jobs, int njobs) {
  if (njobs <= 0) return;
  if (njobs > kEgJobs) bad("eg_apply: too many tables");
  EgApplySet set{};
  int64_t total = 0;
  for (int q = 0; q < njobs; ++q) {
    EgApplyJob j = jobs[q];
    if (!eg_sorted_fits(j.n, j.rows) || j.h <= 0) bad("eg_apply: shape outside the sorted-segment path");
    if (j.out2 && (!j.drop_token || int64_t(j.rows) * j.h > (int64_t(1) << 32)))
      bad("eg_apply: a dropout output needs its token and at most 2^32 elements");
    const int64_t groups = (j.h + kLongCols - 1) / kLongCols;
    j.vec = (j.h % 256 == 0) ? 4 : (j.h % 128 == 0) ? 2 : 1;
    j.blocks_short = int(blocks_for(std::min<int64_t>(j.n, j.rows), kApplyThreads / 64));
    j.blocks_long = int(int64_t(j.n / (kShortMax + 1)) * groups);
    j.blocks = j.blocks_short + j.blocks_long + int(blocks_for(j.rows, 32));
    total += j.blocks;
    set.job[q] = j;
  }
  set.count = njobs;
  if (total > 2147483647) bad("eg_apply: grid");
  MSX_LAUNCH(k_eg_apply, dim3(unsigned(total)), dim3(kApplyThreads), 0, s, set);
}

}  // namespace msx::hk
