// The `.msckpt` checkpoint, format version 1: writer, validating reader, and the match against a
// compiled step.
//
// Restates crates/modelspec-runtime/src/train/checkpoint.rs (the format of the reference's
// DESIGN.md 6.2): a 56-byte little-endian header (magic MSCK, version 1, endian marker
// 0x01020304, a reserved zero word, the manifest size, a BLAKE3 checksum over header and manifest
// with the checksum bytes counted as zero), a compact JSON manifest, and the payload of
// little-endian f32 tensors at multiples of 64 bytes, zero bytes between, the file ending with
// the last tensor. `payload_hash` is BLAKE3 over the payload; `checkpoint_id` a version-8 UUID
// from BLAKE3 over the manifest with the nil UUID in its place.
//
// Beyond the reference: AdamW moments are written as optimizer slots (records with "slot": "m"
// or "v", after the parameters), so an AdamW run resumes with its moments. The reference's reader
// accepts such a file (its invariants allow named slots) and reads its parameters.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "ir.h"

namespace msx {

// A refused checkpoint: `code` is E-CKPT-001 (unreadable: header, checksum, manifest), 002 (an
// offset, length or size outside the file or misaligned), 003 (does not match the compiled
// file), 004 (payload hash).
struct CheckpointError : IrError {
  CheckpointError(const std::string& code, const std::string& what) : IrError(code + ": " + what), code(code) {}
  std::string code;
};

// modelspec.training.OptimizerConfig (checkpoint.rs:93-150): the AdamW fields and the warmup
// schedule present exactly for AdamW.
struct CheckpointOptimizer {
  bool adamw = false;
  double learning_rate = 0, weight_decay = 0, beta1 = 0, beta2 = 0, epsilon = 0;
  uint64_t warmup_steps = 0;
  bool operator==(const CheckpointOptimizer& o) const;
  bool operator!=(const CheckpointOptimizer& o) const { return !(*this == o); }
};

struct CheckpointTensor {
  std::string path;
  std::string slot;  // "" for a parameter; "m" or "v" for an AdamW moment
  std::vector<uint64_t> shape;
  std::vector<float> data;
};

struct Checkpoint {
  uint64_t step = 0;         // updates the parameters have had
  std::string schema_hash;   // lowercase hex
  CheckpointOptimizer optimizer;
  uint64_t seed = 0, counter = 0;  // rng: Philox4x32x10 at the run's seed, counter 0
  std::vector<CheckpointTensor> parameters;  // path order
  std::vector<CheckpointTensor> slots;       // (path, slot) order
};

// BLAKE3 over "modelspec-schema/1\n" and each parameter's path length, path, dtype, rank and
// dimensions in ParamId order (core/src/artifact.rs:169-193), lowercase hex.
std::string schema_hash(const Program& p);

CheckpointOptimizer optimizer_of(const TrainingStep& step);

// The checkpoint of `step` after `updates` updates: `values` by ParamId; `m` and `v` by ParamId
// (empty vectors, or empty entries, for parameters without moments) become AdamW slots.
Checkpoint checkpoint_of(const TrainingStep& step, uint64_t seed, uint64_t updates,
                         const std::vector<std::vector<float>>& values, const std::vector<std::vector<float>>& m,
                         const std::vector<std::vector<float>>& v);

// The file's bytes (checkpoint.rs:440-520); the same state gives the same bytes.
std::vector<uint8_t> encode(const Checkpoint& c);
// Writes through `<path>.tmp` and a rename, so a failed write leaves the earlier file.
void write_checkpoint(const std::string& path, const Checkpoint& c);
// Reads and validates `path` in the reference's order (checkpoint.rs:650-870).
Checkpoint read_checkpoint(const std::string& path);
Checkpoint decode_checkpoint(const std::vector<uint8_t>& bytes, const std::string& shown);

// The parameter values of `c` by ParamId of `step`'s program; E-CKPT-003 at the first path,
// dtype or shape that differs in path order, then at a differing schema hash.
std::vector<std::vector<float>> parameters_for(const Checkpoint& c, const TrainingStep& step);

// What a resumed run starts from: parameters_for, the optimizer checked (E-CKPT-003), and for
// AdamW the moments from the slots (every trained parameter's m and v; a checkpoint of step 0
// may have none, its moments are 0).
struct ResumeState {
  uint64_t step = 0;
  std::vector<std::vector<float>> values, m, v;
};
ResumeState resume_into(const Checkpoint& c, const TrainingStep& step);

// serde_json's text of an f64 (the shortest digits that read back, Ryu's layout).
std::string json_f64(double v);

}  // namespace msx
