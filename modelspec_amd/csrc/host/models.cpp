// Programmatic builders of the configs, in the node order the reference's lowering produces.
#include "models.h"

#include <cmath>

#include "mspec.h"
#include <functional>

namespace msx {

uint64_t default_masked_rows(uint64_t rows, double rate) {
  double n = double(rows);
  rate = std::min(1.0, std::max(0.0, rate));
  double bound = n * rate + 8.0 * std::sqrt(n * rate * (1.0 - rate));
  uint64_t capacity = (uint64_t(std::ceil(bound)) + 63) / 64 * 64;
  return std::min(capacity, rows);
}

namespace {

// Lowering state (lower.rs:95-160): parameters declared in source order, one Input per data
// declaration in source order, one shared ParamRead per parameter in source order, then the loss
// with operands before the operation. Dropout sites `<Model>.<fn>.dropout#<k>` get their token
// Input at first use (lower.rs:404-446).
struct Lowering {
  Builder b;
  std::string model;
  std::vector<std::pair<std::string, Type>> param_decls;
  std::vector<Init> inits;
  std::map<std::string, uint32_t> reads;
  std::map<std::string, uint32_t> data;
  std::string function = "forward";
  int dropout_k = 0;

  void param(const std::string& name, Type ty, Init init) {
    param_decls.push_back({name, ty});
    inits.push_back(init);
  }
  void declare(const std::vector<std::pair<std::string, Type>>& data_decls) {
    for (size_t i = 0; i < param_decls.size(); ++i)
      b.declare_param(model + "." + param_decls[i].first, param_decls[i].second, inits[i]);
    for (auto& [name, ty] : data_decls) data[name] = b.input(name, ty);
    for (size_t i = 0; i < param_decls.size(); ++i) reads[param_decls[i].first] = b.param_read(uint32_t(i));
  }
  uint32_t p(const std::string& name) { return reads.at(name); }
  uint32_t d(const std::string& name) { return data.at(name); }
  uint32_t op(Op o, std::vector<uint32_t> operands, float attr = 0, int64_t heads = 0) {
    return b.op(o, std::move(operands), attr, heads);
  }
  uint32_t matmul(uint32_t a, uint32_t w) { return op(Op::MatMul, {a, w}); }
  uint32_t add_rows(uint32_t x, uint32_t bias) { return op(Op::AddRows, {x, bias}); }
  uint32_t linear(uint32_t x, const std::string& w, const std::string& bias) { return add_rows(matmul(x, p(w)), p(bias)); }
  uint32_t layer_norm(uint32_t x, const std::string& g, const std::string& beta) { return op(Op::LayerNorm, {x, p(g), p(beta)}); }
  uint32_t dropout(uint32_t x, float prob) {
    if (prob == 0.0f) return x;
    std::string site = model + "." + function + ".dropout#" + std::to_string(dropout_k++);
    uint32_t token = b.input(site, Type::i32({2}));
    return op(Op::Dropout, {x, token}, prob);
  }
};

Compiled finish(TrainConfig cfg, Program lowered, uint32_t loss, uint32_t prediction, Rule rule, float lr,
                const AdamWConfig& adamw) {
  lowered.outputs = {loss};
  Program program = dce(std::move(lowered));
  Program gathered = cfg.masked_rows ? masked_rows_gather(program, cfg.masked_rows) : program;
  Compiled c;
  c.step = differentiate(gathered, loss);
  if (rule == Rule::Sgd) attach_sgd(c.step, lr);
  else attach_adamw(c.step, lr, adamw);
  Program fwd = program;
  fwd.outputs = {loss, prediction};
  c.forward = without_dropout(std::move(fwd));
  c.prediction = c.forward.outputs.at(1);
  c.config = std::move(cfg);
  return c;
}

// examples/linear_regression.mspec.
Compiled linear_regression() {
  Lowering L;
  L.model = "LinearReg";
  L.param("w", Type::f32({4, 1}), Init::XavierUniform);
  L.declare({{"x", Type::f32({8, 4})}, {"y", Type::f32({8, 1})}});
  uint32_t pred = L.matmul(L.d("x"), L.p("w"));
  uint32_t loss = L.op(Op::Mse, {pred, L.d("y")});
  TrainConfig c;
  c.name = "linear_regression";
  c.steps = 500;
  c.seed = 42;
  c.feed = FeedKind::Teacher;
  c.x = "x";
  c.y = "y";
  return finish(c, L.b.finish(), loss, pred, Rule::Sgd, 0.1f, {});
}

// examples/mnist_mlp.mspec: 784 -> 64 relu -> 10, no bias, mse, SGD 0.1, teacher data.
Compiled mnist_mlp() {
  Lowering L;
  L.model = "MnistMlp";
  L.param("w1", Type::f32({784, 64}), Init::XavierUniform);
  L.param("w2", Type::f32({64, 10}), Init::XavierUniform);
  L.declare({{"x", Type::f32({100, 784})}, {"y", Type::f32({100, 10})}});
  uint32_t pred = L.matmul(L.op(Op::Relu, {L.matmul(L.d("x"), L.p("w1"))}), L.p("w2"));
  uint32_t loss = L.op(Op::Mse, {pred, L.d("y")});
  TrainConfig c;
  c.name = "mnist_mlp";
  c.steps = 1800;
  c.seed = 42;
  c.feed = FeedKind::Teacher;
  c.x = "x";
  c.y = "y";
  return finish(c, L.b.finish(), loss, pred, Rule::Sgd, 0.1f, {});
}

// The MLP classifier of the configs: 784-256-10 with biases, ReLU, softmax cross_entropy.
Compiled mlp_classifier(int64_t batch, uint64_t steps) {
  Lowering L;
  L.model = "MlpClassifier";
  L.param("w1", Type::f32({784, 256}), Init::XavierUniform);
  L.param("b1", Type::f32({256}), Init::Zeros);
  L.param("w2", Type::f32({256, 10}), Init::XavierUniform);
  L.param("b2", Type::f32({10}), Init::Zeros);
  L.declare({{"x", Type::f32({batch, 784})}, {"labels", Type::i32({batch})}, {"weights", Type::f32({batch})}});
  uint32_t h = L.op(Op::Relu, {L.linear(L.d("x"), "w1", "b1")});
  uint32_t logits = L.linear(h, "w2", "b2");
  uint32_t loss = L.op(Op::CrossEntropy, {logits, L.d("labels"), L.d("weights")});
  TrainConfig c;
  c.name = "mlp_classifier";
  c.steps = steps;
  c.seed = 7;
  c.feed = FeedKind::Classifier;
  c.batch = batch;
  c.features = 784;
  c.classes = 10;
  c.x = "x";
  c.labels = "labels";
  c.weights = "weights";
  return finish(c, L.b.finish(), loss, logits, Rule::Sgd, 0.01f, {});
}

// The single pre-layer-norm encoder block of the configs over a token and position table, with
// an untied output head and next-token cross_entropy.
Compiled transformer_block(int64_t V, int64_t H, int64_t heads, int64_t F, int64_t B, int64_t S, uint64_t steps,
                           const std::string& name) {
  Lowering L;
  L.model = "PreLnBlock";
  L.param("tok_table", Type::f32({V, H}), Init::XavierUniform);
  L.param("pos_table", Type::f32({S, H}), Init::XavierUniform);
  L.param("ln1_gamma", Type::f32({H}), Init::Ones);
  L.param("ln1_beta", Type::f32({H}), Init::Zeros);
  for (const char* w : {"wq", "wk", "wv", "wo"}) {
    L.param(w, Type::f32({H, H}), Init::XavierUniform);
    L.param(std::string("b") + (w + 1), Type::f32({H}), Init::Zeros);
  }
  L.param("ln2_gamma", Type::f32({H}), Init::Ones);
  L.param("ln2_beta", Type::f32({H}), Init::Zeros);
  L.param("w1", Type::f32({H, F}), Init::XavierUniform);
  L.param("b1", Type::f32({F}), Init::Zeros);
  L.param("w2", Type::f32({F, H}), Init::XavierUniform);
  L.param("b2", Type::f32({H}), Init::Zeros);
  L.param("lnf_gamma", Type::f32({H}), Init::Ones);
  L.param("lnf_beta", Type::f32({H}), Init::Zeros);
  L.param("head_w", Type::f32({H, V}), Init::XavierUniform);
  L.param("head_b", Type::f32({V}), Init::Zeros);
  int64_t N = B * S;
  L.declare({{"ids", Type::i32({N})}, {"positions", Type::i32({N})}, {"key_mask", Type::f32({B, S})},
             {"labels", Type::i32({N})}, {"weights", Type::f32({N})}});
  uint32_t x = L.op(Op::Add, {L.op(Op::Embedding, {L.p("tok_table"), L.d("ids")}),
                              L.op(Op::Embedding, {L.p("pos_table"), L.d("positions")})});
  uint32_t h = L.layer_norm(x, "ln1_gamma", "ln1_beta");
  uint32_t q = L.linear(h, "wq", "bq");
  uint32_t k = L.linear(h, "wk", "bk");
  uint32_t v = L.linear(h, "wv", "bv");
  uint32_t att = L.op(Op::Attention, {q, k, v, L.d("key_mask")}, 0, heads);
  uint32_t x1 = L.op(Op::Add, {x, L.linear(att, "wo", "bo")});
  uint32_t h2 = L.layer_norm(x1, "ln2_gamma", "ln2_beta");
  uint32_t f = L.linear(L.op(Op::Gelu, {L.linear(h2, "w1", "b1")}), "w2", "b2");
  uint32_t x2 = L.op(Op::Add, {x1, f});
  uint32_t logits = L.linear(L.layer_norm(x2, "lnf_gamma", "lnf_beta"), "head_w", "head_b");
  uint32_t loss = L.op(Op::CrossEntropy, {logits, L.d("labels"), L.d("weights")});
  TrainConfig c;
  c.name = name;
  c.steps = steps;
  c.seed = 42;
  c.feed = FeedKind::NextToken;
  c.batch = B;
  c.seq = S;
  c.vocab = V;
  c.first_token = 0;
  c.ids = "ids";
  c.positions = "positions";
  c.key_mask = "key_mask";
  c.labels = "labels";
  c.weights = "weights";
  AdamWConfig a;
  a.weight_decay = 0.01f;
  a.beta1 = 0.9f;
  a.beta2 = 0.999f;
  a.eps = 1e-6f;  // the reference examples' eps (examples/bert_tiny.mspec); the config names none
  a.warmup_steps = 0;
  return finish(c, L.b.finish(), loss, logits, Rule::AdamW, 1e-3f, a);
}

// examples/bert_tiny.mspec (and its hidden-32 twin crates/modelspec-cli/tests/fixtures/bert_cpu.mspec)
// at vocabulary V, hidden H, F, S and B.
Compiled bert(const std::string& name, int64_t V, int64_t H, int64_t heads, int64_t F, int64_t B, int64_t S,
              int layers, float lr, uint64_t warmup, uint64_t steps, int64_t masked_rows) {
  Lowering L;
  L.model = "BertTiny";
  L.param("tok_table", Type::f32({V, H}), Init::XavierUniform);
  L.param("pos_table", Type::f32({S, H}), Init::XavierUniform);
  L.param("emb_ln_gamma", Type::f32({H}), Init::Ones);
  L.param("emb_ln_beta", Type::f32({H}), Init::Zeros);
  for (int l = 0; l < layers; ++l) {
    std::string p = "l" + std::to_string(l) + "_";
    for (const char* w : {"wq", "wk", "wv", "wo"}) {
      L.param(p + w, Type::f32({H, H}), Init::XavierUniform);
      L.param(p + "b" + (w + 1), Type::f32({H}), Init::Zeros);
    }
    L.param(p + "ln1_gamma", Type::f32({H}), Init::Ones);
    L.param(p + "ln1_beta", Type::f32({H}), Init::Zeros);
    L.param(p + "w1", Type::f32({H, F}), Init::XavierUniform);
    L.param(p + "b1", Type::f32({F}), Init::Zeros);
    L.param(p + "w2", Type::f32({F, H}), Init::XavierUniform);
    L.param(p + "b2", Type::f32({H}), Init::Zeros);
    L.param(p + "ln2_gamma", Type::f32({H}), Init::Ones);
    L.param(p + "ln2_beta", Type::f32({H}), Init::Zeros);
  }
  L.param("mlm_w", Type::f32({H, H}), Init::XavierUniform);
  L.param("mlm_b", Type::f32({H}), Init::Zeros);
  L.param("mlm_ln_gamma", Type::f32({H}), Init::Ones);
  L.param("mlm_ln_beta", Type::f32({H}), Init::Zeros);
  L.param("mlm_bias", Type::f32({V}), Init::Zeros);
  int64_t N = B * S;
  L.declare({{"ids", Type::i32({N})}, {"positions", Type::i32({N})}, {"key_mask", Type::f32({B, S})},
             {"labels", Type::i32({N})}, {"weights", Type::f32({N})}});
  const float p_drop = 0.1f;
  uint32_t e = L.dropout(L.layer_norm(L.op(Op::Add, {L.op(Op::Embedding, {L.p("tok_table"), L.d("ids")}),
                                                      L.op(Op::Embedding, {L.p("pos_table"), L.d("positions")})}),
                                      "emb_ln_gamma", "emb_ln_beta"),
                         p_drop);
  uint32_t x = e;
  for (int l = 0; l < layers; ++l) {
    std::string p = "l" + std::to_string(l) + "_";
    uint32_t q = L.linear(x, p + "wq", p + "bq");
    uint32_t k = L.linear(x, p + "wk", p + "bk");
    uint32_t v = L.linear(x, p + "wv", p + "bv");
    uint32_t a = L.linear(L.op(Op::Attention, {q, k, v, L.d("key_mask")}, 0, heads), p + "wo", p + "bo");
    uint32_t h = L.layer_norm(L.op(Op::Add, {x, L.dropout(a, p_drop)}), p + "ln1_gamma", p + "ln1_beta");
    uint32_t f = L.linear(L.op(Op::Gelu, {L.linear(h, p + "w1", p + "b1")}), p + "w2", p + "b2");
    x = L.layer_norm(L.op(Op::Add, {h, L.dropout(f, p_drop)}), p + "ln2_gamma", p + "ln2_beta");
  }
  uint32_t m = L.layer_norm(L.op(Op::Gelu, {L.linear(x, "mlm_w", "mlm_b")}), "mlm_ln_gamma", "mlm_ln_beta");
  uint32_t tied = L.op(Op::Transpose, {L.p("tok_table")});
  uint32_t logits = L.add_rows(L.matmul(m, tied), L.p("mlm_bias"));
  uint32_t loss = L.op(Op::CrossEntropy, {logits, L.d("labels"), L.d("weights")});
  TrainConfig c;
  c.name = name;
  c.steps = steps;
  c.seed = 42;
  c.feed = FeedKind::MaskedLm;
  c.batch = B;
  c.seq = S;
  c.vocab = V;
  c.first_token = 5;
  c.masked_rows = masked_rows >= 0 ? uint64_t(masked_rows) : default_masked_rows(uint64_t(N), 0.15);
  c.ids = "ids";
  c.positions = "positions";
  c.key_mask = "key_mask";
  c.labels = "labels";
  c.weights = "weights";
  AdamWConfig a;
  a.weight_decay = 0.01f;
  a.beta1 = 0.9f;
  a.beta2 = 0.999f;
  a.eps = 1e-6f;
  a.warmup_steps = warmup;
  return finish(c, L.b.finish(), loss, logits, Rule::AdamW, lr, a);
}

}  // namespace

Compiled compile_lowered(TrainConfig cfg, Program lowered, uint32_t loss, uint32_t prediction, Rule rule, float lr,
                         const AdamWConfig& adamw) {
  return finish(std::move(cfg), std::move(lowered), loss, prediction, rule, lr, adamw);
}

void apply_steps_override(Compiled& c, int64_t steps) {
  if (steps < 0) return;
  c.config.steps = uint64_t(steps);
  if (c.step.rule == Rule::AdamW && c.step.adamw.warmup_steps >= c.config.steps && c.config.steps > 0)
    c.step.adamw.warmup_steps = c.config.steps / 10;
}

std::vector<std::string> config_names() {
  return {"linear_regression", "mnist_mlp", "mlp_classifier", "transformer_block", "bert_tiny", "bert_cpu", "bert_micro",
          "block_micro", "mlp_micro", "bert_base", "bert_micro_mixed", "bert_mini_mixed"};
}

Compiled compile_config(const std::string& name, int64_t masked_rows, int64_t steps_override) {
  const std::string ext = ".mspec";
  if (name.size() > ext.size() && name.compare(name.size() - ext.size(), ext.size(), ext) == 0)
    return compile_mspec(read_mspec(name), name, masked_rows, steps_override);
  Compiled c;
  if (name == "linear_regression") c = linear_regression();
  else if (name == "mnist_mlp") c = mnist_mlp();
  else if (name == "mlp_classifier") c = mlp_classifier(64, 1000);
  else if (name == "mlp_micro") c = mlp_classifier(8, 20);
  else if (name == "transformer_block") c = transformer_block(4096, 128, 2, 512, 32, 128, 500, name);
  else if (name == "block_micro") c = transformer_block(96, 32, 2, 64, 2, 16, 20, name);
  else if (name == "bert_tiny") c = bert(name, 30522, 128, 2, 512, 32, 128, 2, 1e-4f, 100, 1000, masked_rows);
  else if (name == "bert_cpu") c = bert(name, 300, 32, 2, 64, 2, 16, 2, 3e-3f, 80, 800, masked_rows);
  else if (name == "bert_micro") c = bert(name, 300, 32, 2, 64, 8, 16, 2, 3e-3f, 4, 20, masked_rows);
  else if (name == "bert_base") {
    // BERT-base shape at seq 512, batch 32 (12 layers, hidden 768, 12 heads, FFN 3072), mixed
    // precision, 200 steps with a 20-step warmup.
    c = bert(name, 30522, 768, 12, 3072, 32, 512, 12, 1e-4f, 20, 200, masked_rows);
    c.config.mixed = true;
  } else if (name == "bert_micro_mixed") {
    c = bert(name, 300, 32, 2, 64, 8, 16, 2, 3e-3f, 4, 20, masked_rows);
    c.config.mixed = true;
  } else if (name == "bert_mini_mixed") {
    // A seq-512 BERT of two layers at hidden 256 (4 heads of 64), for tests of the mixed path at
    // the sequence length of the BERT-base config.
    c = bert(name, 1000, 256, 4, 1024, 4, 512, 2, 1e-3f, 4, 20, masked_rows);
    c.config.mixed = true;
  }
  else throw IrError("unknown config `" + name + "`");
  apply_steps_override(c, steps_override);
  return c;
}

}  // namespace msx
