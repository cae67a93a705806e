// The packed masked-language-model data path: a packed directory read into memory, the epoch
// order of its Train sequences and the sequences each step draws.
//
// Restates crates/modelspec-runtime/src/dataset/mlm.rs:30-190 (the records, binding_id),
// :588-705 (load, epoch_order), :717-760 (which sequences a step draws and its draw id) and
// dataset/mod.rs:212-227 (uuid_of); train/data.rs:1448-1640 (the binding's checks). The 80/10/10
// masking of the drawn rows (mlm.rs:761-788) and the masked-row gather run on the device
// (hip/data.hip); the CPU restatement the device is checked against is the oracle's.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "ir.h"

namespace msx {

// modelspec.data.MaskingPolicy (mlm.rs:52-74).
struct MaskingPolicy {
  double selection_rate = 0.15, mask_fraction = 0.8, random_fraction = 0.1, keep_fraction = 0.1;
};

enum class SplitRole : uint8_t { Train = 0, HeldOut = 1 };

// The number of special tokens at the head of every vocabulary ([MASK] = 4).
constexpr uint32_t kSpecialTokens = 5;
constexpr int32_t kMaskToken = 4;

// A refused packed directory (DataError::Packed / PackError): the message names the file.
struct PackedError : IrError {
  using IrError::IrError;
};

struct PackedCorpus {
  std::string dir;
  // binding.json (TrainingDataBinding)
  std::string binding_id, dataset_id, tokenizer_id;
  uint64_t seq_len = 0;
  MaskingPolicy policy;
  // packed.json (PackedDataset)
  std::string packed_id;
  uint64_t vocabulary_size = 0;
  double heldout_unigram_baseline_nats = 0;
  // The ids of each split, sequence after sequence.
  std::vector<int32_t> train, heldout;

  const std::vector<int32_t>& ids(SplitRole r) const { return r == SplitRole::Train ? train : heldout; }
  uint64_t sequences(SplitRole r) const { return seq_len ? ids(r).size() / seq_len : 0; }
};

// Reads the packed directory `dir` (binding.json, packed.json, train.tokens, heldout.tokens),
// refusing, with a PackedError naming the file: an unreadable or malformed record, a binding_id
// that is not the id of its fields, a packed.json of another binding or seq_len, a vocabulary of
// 5 ids or fewer or beyond 2^31, a packed file whose length, BLAKE3 or ids disagree with its
// record.
PackedCorpus load_packed(const std::string& dir);

// Writes a packed directory of the given ids (whole sequences of `seq_len` each) under `policy`
// (BERT's by default): the files load_packed reads, with the records pack() writes (mlm.rs:395-535) for a
// dataset and tokenizer given by their ids. The held-out unigram baseline is computed from the
// ids as pack() computes it.
void write_packed(const std::string& dir, const std::vector<int32_t>& train, const std::vector<int32_t>& heldout,
                  uint64_t seq_len, uint64_t vocabulary_size, const std::string& dataset_id,
                  const std::string& tokenizer_id, const MaskingPolicy& policy = MaskingPolicy());

// The first 16 bytes of `hash` as a version-8 UUID (dataset/mod.rs:212-227).
std::string uuid_of(const uint8_t hash[32]);
// mlm.rs:161-185; empty when an id is not a UUID.
std::string binding_id(const std::string& dataset_id, const std::string& tokenizer_id, uint64_t seq_len,
                       const MaskingPolicy& policy);

// The order epoch `epoch` visits `n` sequences: ascending by w1 * 2^32 + w0 of the DataOrder block
// of sequence i with id `epoch`, ties by i (mlm.rs:665-680).
std::vector<uint32_t> epoch_order(uint64_t seed, uint64_t epoch, uint32_t n);

// What step `step` of `role` draws with `batch` sequences per step (mlm.rs:717-760): the
// sequences in row order and the Masking draw id (the step; HeldOut: step + 2^63). Refuses a batch
// of 0, more sequences than the split holds, or more than 2^32 rows.
struct SequenceDraw {
  std::vector<int32_t> sequences;
  uint64_t draw_id = 0;
};
// The input a step on a device-resident corpus stages in place of its batch: i32 [split (0 Train,
// 1 HeldOut), draw id low, draw id high, the B sequences in row order].
extern const char* const kDrawInput;  // "#draw"
std::vector<int32_t> draw_words(SplitRole role, const SequenceDraw& d);

class EpochOrders {
 public:
  SequenceDraw draw(const PackedCorpus& c, SplitRole role, uint64_t seed, uint64_t step, uint64_t batch);

 private:
  uint64_t seed_ = 0, epoch_ = 0;
  bool have_ = false;
  std::vector<uint32_t> order_;
};

// The batch tensors of a masked-language-model batch, by the names a program declares them under
// (train/data.rs BatchTensor): ids, positions, key_mask, labels, weights.
extern const char* const kBatchTensors[5];

// Binds `corpus` to the data inputs of `forward` (train/data.rs:1640-1760) and returns the batch
// B: every data input names a batch tensor (else E-DATA-005); the first of ids, positions,
// key_mask, labels, weights gives B from [B, S] or [B*S]; every one has its tensor's dtype and
// one of those shapes, and the embedding tables the ids index and the logits the labels classify
// are as wide as the vocabulary (else E-DATA-006); B is at most the Train sequences.
uint64_t bind_corpus(const Program& forward, const PackedCorpus& corpus);

// The integer thresholds the device compares Philox words with: uniform(w) < rate exactly when
// w < threshold, uniform(w) = (w + 0.5) / 2^32 in f64 (mlm.rs:706-709).
struct MaskingThresholds {
  uint64_t select = 0;         // word 0: selected
  uint64_t mask = 0;           // word 1: [MASK]
  uint64_t mask_or_random = 0; // word 1: [MASK] or a random token (mask + random fraction, in f64)
};
MaskingThresholds masking_thresholds(const MaskingPolicy& p);

}  // namespace msx
