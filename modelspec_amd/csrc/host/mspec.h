// The `.mspec` front-end: a subset of the reference's source language, parsed and lowered to the
// Tensor IR the rest of this build compiles.
//
// Grammar (crates/modelspec-core/src/syntax/parser.rs, ast.rs): one `model Name { ... }` of
// `param name: Tensor<dtype, [dims]> = init();` declarations and `fn name(args) -> Type { let
// ...; return ...; }` functions, and one `train Name { ... }` block of `model = Name;`,
// `input`/`target` declarations, `loss = expr;`, `optimizer = sgd(lr = ..)` or
// `adamw(lr, weight_decay, beta1, beta2, eps, warmup_steps)`, `steps`, `seed` and `device`.
// Expressions are names, number literals, operator calls (resolve.rs:64-84: matmul, add, sub,
// mul, relu, transpose, sum, mean, mse, embedding, add_rows, gelu, layer_norm, softmax,
// attention(heads = A), cross_entropy, dropout(p = P), stop_gradient), calls of the model's
// functions, and `model.<fn>(...)` in the loss. Not in the subset: generic models and modules
// (`model M<B: dim>`, `layer`), which the reference marks as target syntax, and `sigreg`.
//
// Lowering follows crates/modelspec-core/src/lower.rs:95-470: parameters in source order, one
// Input per `input`/`target` in source order, one ParamRead per parameter, then the loss with
// operands before the operation and each function call inlined afresh; a dropout site is the
// Input `<Model>.<fn>.dropout#<k>`, k the call's rank among the function's dropout calls by
// source position, `<fn>@<c>` for a function's inlining c >= 1, `train` for the loss.
//
// The data a run feeds is read off the train block (the reference feeds packed `--data` or
// synthetic teacher data): `mse` over an f32 input and target is teacher data; `cross_entropy`
// over i32 `ids` (with `positions` and `key_mask` [B, S]) is masked-LM data on the vocabulary of
// the logits; `cross_entropy` over an f32 input is classifier data.
#pragma once
#include <string>

#include "models.h"

namespace msx {

// A source the front-end refuses: `code` is E-SYNTAX-001 (not in the grammar), E-NAME-001 (an
// unknown name), E-TYPE-001 (operand types an operator refuses) or E-TRAIN-002 (a train block
// the subset cannot run); the message carries `line:column`.
struct MspecError : IrError {
  MspecError(const std::string& code, int line, int col, const std::string& what)
      : IrError(code + ": " + std::to_string(line) + ":" + std::to_string(col) + ": " + what), code(code) {}
  std::string code;
};

// Compiles `source` (the text of an .mspec file) as compile_config compiles a built-in config;
// `name` names the config.
Compiled compile_mspec(const std::string& source, const std::string& name, int64_t masked_rows_override = -1,
                       int64_t steps_override = -1);

// The text of the file at `path` (E-SYNTAX-001 when it cannot be read).
std::string read_mspec(const std::string& path);

}  // namespace msx
