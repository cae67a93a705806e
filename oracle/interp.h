// TEST INFRASTRUCTURE — the CPU oracle. Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load it, and only as the checker; the HIP backend never calls it.
//
// A single-threaded f32 interpreter of Tensor IR restating the arithmetic of the reference's CPU
// interpreter, crates/modelspec-runtime/src/cpu/interpreter.rs:860-1944, cpu/matmul.rs:263-290
// and cpu/tensor.rs:95-140: every f32 operation rounded once in the order the reference writes
// it, `mul_add` as fmaf, whole-tensor sums in f64, glibc expf/logf/sqrtf. Built with
// -ffp-contract=off so that no expression is fused that the reference does not fuse.
#pragma once
#include <map>
#include <string>
#include <vector>

#include "../modelspec_amd/csrc/host/ir.h"

namespace oracle {

struct Tensor {
  msx::Type ty;
  std::vector<float> f;
  std::vector<int32_t> i;
};

class Interpreter {
 public:
  Interpreter(const msx::Program& p, bool has_seed, uint64_t seed);
  // Evaluates every node the outputs depend on, in definition order. Throws msx::IrError for
  // what the reference's RuntimeError refuses (ids, labels, weights, key masks).
  void run(const std::map<std::string, std::vector<float>>& f32, const std::map<std::string, std::vector<int32_t>>& i32,
           const std::vector<std::vector<float>>& params);
  const std::vector<float>& value(uint32_t id) const;

 private:
  const msx::Program& p_;
  bool has_seed_;
  uint64_t seed_;
  std::vector<Tensor> vals_;  // by node position
  std::vector<bool> needed_;
  void eval(size_t at, const std::map<std::string, std::vector<float>>& f32,
            const std::map<std::string, std::vector<int32_t>>& i32, const std::vector<std::vector<float>>& params);
  const Tensor& arg(size_t at, size_t k) const;
};

// The held-out tally of crates/modelspec-runtime/src/train/eval.rs:520-575 (Tally::add and
// Tally::metrics), every row's nll computed (the reference skips rows of weight +0 whose nll is
// finite, which adds +0 to each sum and leaves its bits unchanged, eval.rs:531-537).
struct HeldOutTally {
  bool started = false;           // a first term was added (the sums are Options in eval.rs)
  double numerator = 0, denominator = 0;
  uint64_t correct = 0, selected = 0;
  // Adds `rows` rows of `v` logits; false (and nothing added) when a label is outside [0, v).
  bool add(const float* logits, const int32_t* labels, const float* weights, size_t rows, size_t v);
  float loss() const;
  float accuracy() const;
};

// max + ln(sum exp(x - max)) - row[label], the sum from its first term in ascending order
// (eval.rs:593-601).
float row_nll(const float* row, size_t v, size_t label);
// The first largest logit, lowest id among ties; -1 when the row holds a NaN (runner.rs:633-638).
int64_t first_argmax(const float* row, size_t v);

}  // namespace oracle
