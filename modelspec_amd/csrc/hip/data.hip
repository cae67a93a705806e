// The masked-language-model batch of a step drawn on the device from a packed corpus resident in
// HBM, and the masked-row gather of its selected rows.
//
// k_mlm_rows restates crates/modelspec-runtime/src/dataset/mlm.rs:761-788 for every row at once:
// row r = b * S + p of the batch reads id p of the step's b-th sequence as its label and takes
// the Philox block of index r and the step's draw id on the Masking stream (tag 3). A row whose
// label is not special is selected when word 0 is below the selection threshold; a selected row
// becomes [MASK] (4) when word 1 is below the mask threshold, a random token
// 5 + ((w2 * (V - 5)) >> 32) when below the mask-or-random threshold, else keeps its id. The
// thresholds are the integer forms of the reference's f64 comparisons, so the masks are the
// reference's bits. Positions are p, the key mask is all ones, the weight 1 exactly at selected
// rows.
//
// k_masked_gather restates crates/modelspec-runtime/src/train/masked.rs:58-118: the rows of
// non-zero weight in ascending order, then padding rows 0 / label 0 / weight +0 up to the
// capacity. One block: each thread counts a contiguous run of rows, a block-wide exclusive scan
// gives each run its first output slot, so the output order is the row order. More selected rows
// than the capacity is the reference's refusal E-DATA-012: the kernel records the first such
// batch (its count and draw id) in an error word the host reads at its next wait, and writes
// only the first `capacity` rows.
#include "device.h"
#include "kernels.h"

namespace msx::hk {
namespace {

__global__ __launch_bounds__(256) void k_mlm_rows(MlmCorpus c, const int32_t* __restrict__ draw, int64_t rows,
                                                  int32_t* __restrict__ ids, int32_t* __restrict__ positions,
                                                  float* __restrict__ key_mask, int32_t* __restrict__ labels,
                                                  float* __restrict__ weights) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int32_t* split = draw[0] == 0 ? c.train : c.heldout;
  const uint32_t id_lo = uint32_t(draw[1]), id_hi = uint32_t(draw[2]);
  const int64_t b = r / c.seq_len, p = r - b * c.seq_len;
  const uint64_t sequence = uint32_t(draw[3 + b]);
  const int32_t label = split[sequence * uint64_t(c.seq_len) + uint64_t(p)];
  const uint4 w = philox_block4(uint32_t(r), 3u, id_lo, id_hi, uint32_t(c.seed), uint32_t(c.seed >> 32));
  const bool selected = label >= int32_t(kMlmSpecials) && uint64_t(w.x) < c.select;
  int32_t id = label;
  if (selected) {
    if (uint64_t(w.y) < c.mask) id = kMlmMask;
    else if (uint64_t(w.y) < c.mask_or_random) id = int32_t(uint64_t(kMlmSpecials) + ((uint64_t(w.z) * c.random_tokens) >> 32));
  }
  if (ids) ids[r] = id;
  if (positions) positions[r] = int32_t(p);
  if (key_mask) key_mask[r] = 1.0f;
  if (labels) labels[r] = label;
  if (weights) weights[r] = selected ? 1.0f : 0.0f;
}

constexpr int kGatherThreads = 1024;

__global__ __launch_bounds__(kGatherThreads) void k_masked_gather(const int32_t* __restrict__ labels,
                                                                  const float* __restrict__ weights, int64_t rows,
                                                                  int64_t capacity, const int32_t* __restrict__ draw,
                                                                  int32_t* __restrict__ out_rows,
                                                                  int32_t* __restrict__ out_labels,
                                                                  float* __restrict__ out_weights,
                                                                  uint32_t* __restrict__ error) {
  __shared__ int64_t wave_total[kGatherThreads / 64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t per = (rows + kGatherThreads - 1) / kGatherThreads;
  const int64_t lo = rows < int64_t(t) * per ? rows : int64_t(t) * per, hi = rows < lo + per ? rows : lo + per;
  int64_t mine = 0;
  for (int64_t r = lo; r < hi; ++r) mine += weights[r] != 0.0f;
  // Inclusive scan across the wave, then across the waves.
  int64_t incl = mine;
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t up = __shfl_up(incl, o, 64);
    if (lane >= o) incl += up;
  }
  if (lane == 63) wave_total[wave] = incl;
  __syncthreads();
  int64_t before = 0, total = 0;
  for (int k = 0; k < kGatherThreads / 64; ++k) {
    if (k < wave) before += wave_total[k];
    total += wave_total[k];
  }
  int64_t slot = before + incl - mine;
  for (int64_t r = lo; r < hi && slot < capacity; ++r) {
    const float w = weights[r];
    if (w != 0.0f) {
      out_rows[slot] = int32_t(r);
      out_labels[slot] = labels ? labels[r] : 0;
      out_weights[slot] = w;
      ++slot;
    }
  }
  for (int64_t s = total + t; s < capacity; s += kGatherThreads) {
    out_rows[s] = 0;
    out_labels[s] = 0;
    out_weights[s] = 0.0f;
  }
  if (t == 0 && total > capacity && error[0] == 0) {
    error[1] = uint32_t(total < int64_t(UINT32_MAX) ? total : int64_t(UINT32_MAX));
    error[2] = uint32_t(draw ? draw[1] : 0);
    error[3] = uint32_t(draw ? draw[2] : 0);
    error[0] = 1;
  }
}

}  // namespace

void mlm_rows(hipStream_t s, const MlmCorpus& c, const int32_t* draw, int64_t batch, int32_t* ids, int32_t* positions,
              float* key_mask, int32_t* labels, float* weights) {
  const int64_t rows = batch * c.seq_len;
  if (rows <= 0) return;
  if (rows > (int64_t(1) << 32) || c.seq_len <= 0) bad("mlm batch rows");
  MSX_LAUNCH(k_mlm_rows, dim3(blocks_for(rows, 256)), dim3(256), 0, s, c, draw, rows, ids, positions, key_mask, labels,
             weights);
}

void masked_gather(hipStream_t s, const int32_t* labels, const float* weights, int64_t rows, int64_t capacity,
                   const int32_t* draw, int32_t* out_rows, int32_t* out_labels, float* out_weights, uint32_t* error) {
  if (capacity <= 0) return;
  if (rows > 2147483647 || capacity > 2147483647) bad("masked gather size");
  MSX_LAUNCH(k_masked_gather, dim3(1), dim3(kGatherThreads), 0, s, labels, weights, rows, capacity, draw, out_rows,
             out_labels, out_weights, error);
}

}  // namespace msx::hk
