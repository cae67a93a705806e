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

}  // namespace oracle
