// The programs this backend trains, built the way the reference's lowering builds them from
// their `.mspec` sources, and the compile pipeline that turns each into a training step.
//
// The pipeline restates crates/modelspec-core/src/compile.rs:85-118: lower, dead-code
// elimination, the masked-row gather at a capacity, autodiff, optimizer attachment; the forward
// program of the final loss is the lowered program with every dropout the identity.
#pragma once
#include <string>
#include <vector>

#include "ir.h"

namespace msx {

// How a config's batches are made (the data each step feeds).
enum class FeedKind : uint8_t {
  Teacher,     // one standard-normal input, target = teacher prediction (train/data.rs:189-211)
  Classifier,  // f32 U(0,1) input, uniform labels, unit weights
  NextToken,   // Zipf token ids, labels = ids shifted by one, per-sequence positions
  MaskedLm,    // Zipf token ids with BERT 80/10/10 masking (dataset/mlm.rs:717-788)
};

struct TrainConfig {
  std::string name;
  uint64_t steps = 0;
  uint64_t seed = 0;
  FeedKind feed = FeedKind::Teacher;
  // data shapes
  int64_t batch = 0, seq = 0, vocab = 0, features = 0, classes = 0;
  double zipf_s = 1.1;
  uint32_t first_token = 0;  // smallest id a Zipf draw yields (5 under MLM: the special tokens)
  uint64_t masked_rows = 0;  // masked-row gather capacity (0 = none)
  // names of the data inputs
  std::string x, y, ids, positions, key_mask, labels, weights;
  // Mixed precision: GEMMs on the f16 MFMA with f32 accumulation and dynamic loss scaling (the
  // BERT-base config); the step program itself is the f32 program.
  bool mixed = false;
};

struct Compiled {
  TrainConfig config;
  TrainingStep step;       // gathered, differentiated, optimizer attached
  Program forward;         // dropout-free forward program; outputs = [loss, prediction]
  uint32_t prediction = 0;
};

// The configs of this build by name: "linear_regression", "mlp_classifier",
// "transformer_block", "bert_tiny", and small variants used by tests ("bert_micro"). A name
// ending in ".mspec" is the path of a source file, compiled by the front-end (mspec.h).
std::vector<std::string> config_names();
Compiled compile_config(const std::string& name, int64_t masked_rows_override = -1,
                        int64_t steps_override = -1);

// The compile pipeline after lowering: dead-code elimination, the masked-row gather when
// cfg.masked_rows, autodiff of `loss`, the optimizer, and the dropout-free forward program whose
// outputs are [loss, prediction].
Compiled compile_lowered(TrainConfig cfg, Program lowered, uint32_t loss, uint32_t prediction, Rule rule, float lr,
                         const AdamWConfig& adamw);
// A run of `steps` (>= 0) instead of the config's: an AdamW warm-up that would not end before it
// becomes a tenth of it.
void apply_steps_override(Compiled& c, int64_t steps);

// default_masked_rows of crates/modelspec-cli/src/train.rs:380-389.
uint64_t default_masked_rows(uint64_t rows, double rate);

}  // namespace msx
