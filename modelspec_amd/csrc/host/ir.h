// Tensor IR, Training IR and the compiler passes the HIP backend consumes.
//
// The graph is the reference's tensor SSA (crates/modelspec-core/src/ir/tensor.rs:129-272):
// one node per value, nodes in definition order. The passes restate
//   - the operator registry's typing and gradient rules (ops.rs:334, ops.rs:752-963),
//   - reverse-mode autodiff with adjoints summed in contribution order (autodiff.rs:57-175,
//     autodiff.rs:460-534),
//   - SGD and AdamW attachment (ir/training.rs:737-980),
//   - dead-code elimination (passes/dce.rs:16-22), the masked-row gather of a weighted
//     cross_entropy (passes/masked_rows.rs:117-320) and the dropout-free forward program
//     (lower.rs:163-195),
// and the printer of ir/print.rs:28-300, whose text is the interchange format of the C ABI.
#pragma once
#include <cstdint>
#include <map>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace msx {

struct IrError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

enum class DType : uint8_t { F32, I32 };

enum class Op : uint8_t {
  Input, ParamRead, Scalar, Add, Sub, Mul, MatMul, Relu, Transpose, ReduceSum, ReduceMean, Mse,
  ReluGrad, BroadcastScalar, Embedding, EmbeddingGrad, AddRows, SumRows, Gelu, GeluGrad, LayerNorm,
  LayerNormGradX, LayerNormGradGamma, Softmax, SoftmaxGrad, Attention, AttentionGradQ,
  AttentionGradK, AttentionGradV, CrossEntropy, CrossEntropyGrad, Dropout, DropoutGrad,
  StopGradient, Sqrt, Div,
  Count_
};

const char* op_name(Op op);
std::optional<Op> op_from_name(const std::string& name);

struct Type {
  DType dtype = DType::F32;
  std::vector<int64_t> shape;
  int rank() const { return int(shape.size()); }
  int64_t count() const {
    int64_t n = 1;
    for (auto d : shape) n *= d;
    return n;
  }
  bool operator==(const Type& o) const { return dtype == o.dtype && shape == o.shape; }
  bool operator!=(const Type& o) const { return !(*this == o); }
  static Type f32(std::vector<int64_t> s) { return Type{DType::F32, std::move(s)}; }
  static Type i32(std::vector<int64_t> s) { return Type{DType::I32, std::move(s)}; }
};
std::string type_string(const Type& t);

enum class Init : uint8_t { XavierUniform, Zeros, Ones };
const char* init_name(Init i);

struct ParamDecl {
  std::string path;
  Type ty;
  Init init = Init::Zeros;
};

struct Node {
  uint32_t id = 0;
  Op op = Op::Input;
  std::vector<uint32_t> operands;
  Type ty;
  std::string name;          // Input
  uint32_t param = 0;        // ParamRead
  float scalar = 0.0f;       // Scalar value; Dropout / DropoutGrad p
  int64_t heads = 0;         // Attention family
  int64_t rows = 0;          // EmbeddingGrad
  std::vector<int64_t> bshape;  // BroadcastScalar
};

struct Program {
  std::vector<ParamDecl> params;  // index = ParamId
  std::vector<Node> nodes;
  std::vector<uint32_t> inputs;
  std::vector<uint32_t> outputs;

  // id -> position in `nodes`; rebuilt by reindex().
  std::unordered_map<uint32_t, size_t> pos;
  void reindex();
  const Node& node(uint32_t id) const;
  Node& node(uint32_t id);
  bool has(uint32_t id) const { return pos.count(id) != 0; }
  uint32_t next_id() const;
  // The Input node named `name`, if any.
  const Node* input(const std::string& name) const;
};

// Result type of `op` over operand types (ops.rs:334), checked; throws IrError.
Type infer(const Node& proto, const std::vector<const Type*>& operands);

// Index of the RNG-token operand of Dropout (1) and DropoutGrad (0), -1 otherwise (ops.rs).
int token_operand(Op op);

enum class Subgraph : uint8_t { Forward, Loss, Gradient, Optimizer };
enum class Rule : uint8_t { Sgd, AdamW };

struct AdamWConfig {
  float weight_decay = 0.01f, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-6f;
  uint64_t warmup_steps = 0;
  // ir/training.rs:190-200: beta1, 1-beta1, beta2, 1-beta2 (complements in f64), eps, decay.
  void constants(float out[6]) const;
};

struct StepScalars { float lr_t, c1, c2; };
// ir/training.rs:209-230: warmup/decay schedule and bias corrections at step t (from 1).
StepScalars adamw_scalars(const AdamWConfig& a, float lr, uint64_t t, uint64_t steps);

struct Moments { uint32_t m, v, m_next, v_next; };

struct Effect {
  uint32_t token;
  uint32_t param;
  bool write;
  uint64_t version;
  char moment = 0;  // 0 for parameter state, 'm' / 'v' for a moment
};

struct TrainingStep {
  Program program;
  std::map<uint32_t, Subgraph> subgraphs;
  uint32_t loss = 0;
  std::map<uint32_t, uint32_t> gradients;  // ParamId -> value
  bool has_optimizer = false;
  Rule rule = Rule::Sgd;
  float lr = 0.0f;
  AdamWConfig adamw;
  std::map<uint32_t, uint32_t> updates;   // ParamId -> value
  std::map<uint32_t, Moments> moments;    // ParamId -> moments (AdamW)
  std::optional<uint32_t> lr_t, c1, c2;   // AdamW host inputs
  std::map<uint32_t, Effect> effects;     // value -> effect (printing only)
};

// --- builder ---------------------------------------------------------------------------------
// Appends typed nodes in definition order, the way lowering does (lower.rs:95-160).
class Builder {
 public:
  Program prog;
  uint32_t declare_param(const std::string& path, Type ty, Init init);
  uint32_t input(const std::string& name, Type ty);
  uint32_t param_read(uint32_t param);
  uint32_t scalar(float v);
  uint32_t op(Op op, std::vector<uint32_t> operands, float attr = 0.0f, int64_t heads = 0);
  void output(uint32_t v) { prog.outputs.push_back(v); }
  Program finish();
};

// --- passes ----------------------------------------------------------------------------------
Program dce(Program p);                                 // passes/dce.rs:16-22
Program masked_rows_gather(Program p, uint64_t capacity);  // passes/masked_rows.rs:117-320
Program without_dropout(Program p);                     // lower.rs:163-195
TrainingStep differentiate(const Program& forward, uint32_t loss);  // autodiff.rs:57-175
void attach_sgd(TrainingStep& t, float lr);             // ir/training.rs:737-808
void attach_adamw(TrainingStep& t, float lr, const AdamWConfig& a);  // ir/training.rs:822-980

// Names the reference gives the optimizer's host inputs (ir/training.rs:310-347).
extern const char* const kLrTInput;
extern const char* const kC1Input;
extern const char* const kC2Input;
std::string moment_input(char moment, const std::string& path);
extern const char* const kMaskedRowsInput;      // "masked.rows"
extern const char* const kMaskedLabelsPrefix;   // "masked.labels."
extern const char* const kMaskedWeightsPrefix;  // "masked.weights."

// Token inputs of every dropout site, in input order (ir/training.rs:550-566).
std::vector<std::string> dropout_sites(const Program& p);

// --- text form -------------------------------------------------------------------------------
std::string print_program(const Program& p);       // print.rs TensorProgram Display
std::string print_step(const TrainingStep& t);     // print.rs write_training
TrainingStep parse_step(const std::string& text);  // inverse of print_step
Program parse_program(const std::string& text);    // inverse of print_program

// Rust `{:?}` and `{}` of an f32: shortest round-trip digits.
std::string f32_debug(float v);
std::string f32_display(float v);

}  // namespace msx
