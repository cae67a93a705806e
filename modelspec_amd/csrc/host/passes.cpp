// Compiler passes over Tensor IR: dead-code elimination, the masked-row gather, the dropout-free
// forward program, reverse-mode autodiff and optimizer attachment. See ir.h for the reference
// functions each restates.
#include <algorithm>
#include <cmath>
#include <optional>
#include <set>

#include "ir.h"

namespace msx {

namespace {
[[noreturn]] void fail(const std::string& what) { throw IrError(what); }

Node make(uint32_t id, Op op, std::vector<uint32_t> operands) {
  Node n;
  n.id = id;
  n.op = op;
  n.operands = std::move(operands);
  return n;
}
}  // namespace

Program dce(Program p) {
  p.reindex();
  std::set<uint32_t> live(p.outputs.begin(), p.outputs.end());
  for (auto it = p.nodes.rbegin(); it != p.nodes.rend(); ++it)
    if (live.count(it->id)) live.insert(it->operands.begin(), it->operands.end());
  std::vector<Node> kept;
  for (auto& n : p.nodes)
    if (live.count(n.id)) kept.push_back(std::move(n));
  p.nodes = std::move(kept);
  std::vector<uint32_t> inputs;
  for (auto v : p.inputs)
    if (live.count(v)) inputs.push_back(v);
  p.inputs = std::move(inputs);
  p.reindex();
  return p;
}

Program without_dropout(Program p) {
  p.reindex();
  std::map<uint32_t, uint32_t> identity;
  std::vector<Node> nodes;
  for (auto& n : p.nodes) {
    for (auto& o : n.operands) {
      auto it = identity.find(o);
      if (it != identity.end()) o = it->second;
    }
    if (n.op == Op::Dropout) identity[n.id] = n.operands[0];
    else nodes.push_back(std::move(n));
  }
  p.nodes = std::move(nodes);
  for (auto& o : p.outputs) {
    auto it = identity.find(o);
    if (it != identity.end()) o = it->second;
  }
  return dce(std::move(p));
}

// --- masked-row gather (passes/masked_rows.rs:117-320) ---------------------------------------
Program masked_rows_gather(Program p, uint64_t capacity) {
  p.reindex();
  if (p.outputs.size() != 1) return p;
  uint32_t loss = p.outputs[0];
  size_t loss_at = p.pos.at(loss);
  const Node& ce = p.nodes[loss_at];
  if (ce.op != Op::CrossEntropy) return p;
  const Node& labels_node = p.node(ce.operands[1]);
  const Node& weights_node = p.node(ce.operands[2]);
  if (labels_node.op != Op::Input || weights_node.op != Op::Input) return p;
  const Type& logits_ty = p.node(ce.operands[0]).ty;
  if (logits_ty.rank() != 2) return p;
  int64_t rows = logits_ty.shape[0];
  if (capacity == 0 || int64_t(capacity) >= rows) return p;

  // Values that depend on no Input: parameters, constants and what they alone compute.
  std::set<uint32_t> row_free;
  for (auto& n : p.nodes) {
    bool leaf = n.op == Op::ParamRead || n.op == Op::Scalar;
    bool derived = !n.operands.empty() && n.op != Op::Input &&
                   std::all_of(n.operands.begin(), n.operands.end(), [&](uint32_t v) { return row_free.count(v) != 0; });
    if (leaf || derived) row_free.insert(n.id);
  }
  std::map<uint32_t, int> consumers;
  for (auto& n : p.nodes)
    for (auto o : n.operands) consumers[o] += 1;
  for (auto o : p.outputs) consumers[o] += 1;

  std::vector<std::pair<Op, Node>> chain;  // op and its node (operands after the first kept)
  const Node* current = &p.node(ce.operands[0]);
  while (true) {
    bool row_local = current->op == Op::AddRows || current->op == Op::MatMul || current->op == Op::Gelu ||
                     current->op == Op::LayerNorm;
    bool rest_free = true;
    for (size_t k = 1; k < current->operands.size(); ++k)
      if (!row_free.count(current->operands[k])) rest_free = false;
    if (!row_local || consumers[current->id] != 1 || !rest_free) break;
    chain.push_back({current->op, *current});
    current = &p.node(current->operands[0]);
  }
  if (chain.empty() || current->ty.dtype != DType::F32 || current->ty.rank() != 2) return p;
  std::reverse(chain.begin(), chain.end());

  uint32_t next = p.next_id();
  std::vector<Node> added;
  std::map<uint32_t, const Type*> types;
  for (auto& n : p.nodes) types[n.id] = &n.ty;
  auto add_input = [&](const std::string& name, Type ty) {
    Node n = make(next++, Op::Input, {});
    n.name = name;
    n.ty = std::move(ty);
    added.push_back(n);
    return added.back().id;
  };
  int64_t cap = int64_t(capacity);
  uint32_t rows_in = add_input(kMaskedRowsInput, Type::i32({cap}));
  uint32_t labels_in = add_input(std::string(kMaskedLabelsPrefix) + labels_node.name, Type::i32({cap}));
  uint32_t weights_in = add_input(std::string(kMaskedWeightsPrefix) + weights_node.name, Type::f32({cap}));
  auto type_of = [&](uint32_t v) -> const Type* {
    for (auto& a : added)
      if (a.id == v) return &a.ty;
    return types.at(v);
  };
  auto add_op = [&](const Node& proto, std::vector<uint32_t> operands) {
    Node n = proto;
    n.id = next++;
    n.operands = std::move(operands);
    std::vector<const Type*> ts;
    for (auto v : n.operands) ts.push_back(type_of(v));
    n.ty = infer(n, ts);
    added.push_back(n);
    return added.back().id;
  };
  Node emb = make(0, Op::Embedding, {});
  uint32_t cur = add_op(emb, {current->id, rows_in});
  for (auto& [op, proto] : chain) {
    std::vector<uint32_t> operands{cur};
    operands.insert(operands.end(), proto.operands.begin() + 1, proto.operands.end());
    Node bare = proto;
    cur = add_op(bare, operands);
  }
  std::vector<Node> result;
  for (size_t at = 0; at < p.nodes.size(); ++at) {
    if (at == loss_at) {
      for (auto& a : added) result.push_back(a);
      Node l = p.nodes[at];
      l.operands = {cur, labels_in, weights_in};
      result.push_back(l);
    } else {
      result.push_back(p.nodes[at]);
    }
  }
  p.nodes = std::move(result);
  p.inputs.clear();
  for (auto& n : p.nodes)
    if (n.op == Op::Input) p.inputs.push_back(n.id);
  p.reindex();
  return p;
}

// --- autodiff (autodiff.rs:57-175, 460-534; ops.rs:752-963) -----------------------------------
namespace {
struct Sink {
  Program program;
  std::map<uint32_t, Subgraph> subgraphs;
  uint32_t next;
  std::optional<uint32_t> seed;
  Subgraph tag = Subgraph::Gradient;

  const Type& type_of(uint32_t v) const { return program.node(v).ty; }

  uint32_t push(Node n) {
    std::vector<const Type*> ts;
    for (auto v : n.operands) ts.push_back(&program.node(v).ty);
    n.ty = infer(n, ts);
    n.id = next++;
    bool on_seed = false;
    for (auto o : n.operands)
      if ((seed && o == *seed) || subgraphs.at(o) == Subgraph::Gradient) on_seed = true;
    Subgraph t = (on_seed || tag == Subgraph::Loss) ? tag : Subgraph::Forward;
    subgraphs[n.id] = t;
    program.nodes.push_back(n);
    program.pos[n.id] = program.nodes.size() - 1;
    return n.id;
  }
  uint32_t emit(Op op, std::vector<uint32_t> operands) { return push(make(0, op, std::move(operands))); }
  uint32_t emit_scalar(float v) {
    Node n = make(0, Op::Scalar, {});
    n.scalar = v;
    return push(n);
  }
  uint32_t sum(const std::vector<uint32_t>& values) {
    uint32_t acc = values.at(0);
    for (size_t i = 1; i < values.size(); ++i) acc = emit(Op::Add, {acc, values[i]});
    return acc;
  }
  uint32_t unbroadcast(uint32_t c, uint32_t operand) {
    if (type_of(operand).rank() == 0 && type_of(c).rank() > 0) return emit(Op::ReduceSum, {c});
    return c;
  }
  uint32_t broadcast(uint32_t s, uint32_t operand) {
    auto shape = type_of(operand).shape;
    if (shape.empty()) return s;
    Node n = make(0, Op::BroadcastScalar, {s});
    n.bshape = shape;
    return push(n);
  }
  uint32_t negate(uint32_t c) {
    uint32_t minus_one = emit_scalar(-1.0f);
    return emit(Op::Mul, {c, minus_one});
  }
  static float per_element(const Type& t, double factor) { return float(factor / double(t.count())); }

  // The gradient rule of `n` (ops.rs:752-930): one optional contribution per operand.
  std::vector<std::optional<uint32_t>> gradient(const Node& n, uint32_t g, const std::vector<bool>& want) {
    std::vector<std::optional<uint32_t>> out(n.operands.size());
    auto w = [&](size_t i) { return i < want.size() && want[i]; };
    const auto& o = n.operands;
    switch (n.op) {
      case Op::Input: case Op::ParamRead: case Op::Scalar: break;
      case Op::Add:
        for (size_t i = 0; i < o.size(); ++i)
          if (w(i)) out[i] = unbroadcast(g, o[i]);
        break;
      case Op::Sub:
        if (w(0)) out[0] = unbroadcast(g, o[0]);
        if (w(1)) out[1] = negate(unbroadcast(g, o[1]));
        break;
      case Op::Mul:
        if (w(0)) out[0] = unbroadcast(emit(Op::Mul, {g, o[1]}), o[0]);
        if (w(1)) out[1] = unbroadcast(emit(Op::Mul, {g, o[0]}), o[1]);
        break;
      case Op::MatMul:
        if (w(0)) { uint32_t bt = emit(Op::Transpose, {o[1]}); out[0] = emit(Op::MatMul, {g, bt}); }
        if (w(1)) { uint32_t at = emit(Op::Transpose, {o[0]}); out[1] = emit(Op::MatMul, {at, g}); }
        break;
      case Op::Relu: if (w(0)) out[0] = emit(Op::ReluGrad, {o[0], g}); break;
      case Op::Transpose: if (w(0)) out[0] = emit(Op::Transpose, {g}); break;
      case Op::ReduceSum: if (w(0)) out[0] = broadcast(g, o[0]); break;
      case Op::ReduceMean:
        if (w(0)) {
          uint32_t c = emit_scalar(per_element(type_of(o[0]), 1.0));
          uint32_t scaled = emit(Op::Mul, {g, c});
          out[0] = broadcast(scaled, o[0]);
        }
        break;
      case Op::Mse:
        if (w(0) || w(1)) {
          float scale = per_element(type_of(o[0]), 2.0);
          uint32_t d = emit(Op::Sub, {o[0], o[1]});
          uint32_t c = emit_scalar(scale);
          uint32_t scaled = emit(Op::Mul, {g, c});
          uint32_t dy = emit(Op::Mul, {d, scaled});
          if (w(0)) out[0] = dy;
          if (w(1)) out[1] = negate(dy);
        }
        break;
      case Op::Embedding:
        if (w(0)) {
          Node e = make(0, Op::EmbeddingGrad, {o[1], g});
          e.rows = type_of(o[0]).shape[0];
          out[0] = push(e);
        }
        break;
      case Op::AddRows:
        if (w(0)) out[0] = g;
        if (w(1)) out[1] = emit(Op::SumRows, {g});
        break;
      case Op::Gelu: if (w(0)) out[0] = emit(Op::GeluGrad, {o[0], g}); break;
      case Op::LayerNorm:
        if (w(0)) out[0] = emit(Op::LayerNormGradX, {o[0], o[1], g});
        if (w(1)) out[1] = emit(Op::LayerNormGradGamma, {o[0], g});
        if (w(2)) out[2] = emit(Op::SumRows, {g});
        break;
      case Op::Softmax: if (w(0)) out[0] = emit(Op::SoftmaxGrad, {n.id, g}); break;
      case Op::Attention: {
        const Op rules[3] = {Op::AttentionGradQ, Op::AttentionGradK, Op::AttentionGradV};
        for (size_t i = 0; i < 3; ++i)
          if (w(i)) {
            Node a = make(0, rules[i], {o[0], o[1], o[2], o[3], g});
            a.heads = n.heads;
            out[i] = push(a);
          }
        break;
      }
      case Op::CrossEntropy:
        if (w(0)) out[0] = emit(Op::CrossEntropyGrad, {o[0], o[1], o[2], g});
        break;
      case Op::Dropout:
        if (w(0)) {
          Node d = make(0, Op::DropoutGrad, {o[1], g});
          d.scalar = n.scalar;
          out[0] = push(d);
        }
        break;
      case Op::StopGradient: break;
      default:
        fail(std::string("%") + std::to_string(n.id) + ": " + op_name(n.op) + " has no gradient rule");
    }
    return out;
  }
};
}  // namespace

TrainingStep differentiate(const Program& forward_in, uint32_t loss) {
  Program forward = forward_in;
  forward.reindex();
  const auto& nodes = forward.nodes;
  auto loss_it = forward.pos.find(loss);
  if (loss_it == forward.pos.end()) fail("loss is not defined");
  size_t loss_at = loss_it->second;
  if (nodes[loss_at].ty.rank() != 0) fail("loss is not rank 0");

  std::vector<bool> reaches(nodes.size());
  for (size_t i = 0; i < nodes.size(); ++i) {
    bool any = false;
    for (auto o : nodes[i].operands) any = any || reaches[forward.pos.at(o)];
    reaches[i] = nodes[i].op != Op::StopGradient && (nodes[i].op == Op::ParamRead || any);
  }

  Sink sink;
  sink.program = forward;
  for (auto& n : nodes) sink.subgraphs[n.id] = n.id == loss ? Subgraph::Loss : Subgraph::Forward;
  sink.next = forward.next_id();

  std::map<uint32_t, std::vector<uint32_t>> adjoints;
  std::vector<std::pair<uint32_t, uint32_t>> leaves;
  if (reaches[loss_at]) {
    sink.tag = Subgraph::Loss;
    uint32_t seed = sink.emit_scalar(1.0f);
    sink.tag = Subgraph::Gradient;
    sink.seed = seed;
    adjoints[loss].push_back(seed);
  }
  for (size_t k = loss_at + 1; k-- > 0;) {
    const Node node = nodes[k];  // copy: the sink appends to its own program, not `nodes`
    auto it = adjoints.find(node.id);
    if (it == adjoints.end()) continue;
    std::vector<uint32_t> contributions = std::move(it->second);
    adjoints.erase(it);
    uint32_t g = sink.sum(contributions);
    if (node.op == Op::ParamRead || node.op == Op::Input) {
      leaves.push_back({node.id, g});
      continue;
    }
    std::vector<bool> wanted;
    for (auto o : node.operands) wanted.push_back(reaches[forward.pos.at(o)]);
    auto per_operand = sink.gradient(node, g, wanted);
    for (size_t i = 0; i < node.operands.size(); ++i)
      if (per_operand[i]) adjoints[node.operands[i]].push_back(*per_operand[i]);
  }
  std::map<uint32_t, std::vector<uint32_t>> reads;
  for (auto& [leaf, g] : leaves) {
    const Node& n = forward.node(leaf);
    if (n.op == Op::ParamRead) reads[n.param].push_back(g);
  }
  TrainingStep t;
  for (auto& [param, list] : reads) t.gradients[param] = sink.sum(list);
  t.program = std::move(sink.program);
  t.program.outputs.clear();
  t.program.outputs.push_back(loss);
  for (auto& [param, g] : t.gradients) t.program.outputs.push_back(g);
  t.subgraphs = std::move(sink.subgraphs);
  t.loss = loss;
  t.program.reindex();
  return t;
}

// --- optimizer attachment (ir/training.rs:737-980) --------------------------------------------
namespace {
struct Appender {
  TrainingStep& t;
  uint32_t next;
  explicit Appender(TrainingStep& step) : t(step), next(step.program.next_id()) {}
  uint32_t push(Node n) {
    n.id = next++;
    if (n.op != Op::Input) {
      std::vector<const Type*> ts;
      for (auto v : n.operands) ts.push_back(&t.program.node(v).ty);
      n.ty = infer(n, ts);
    } else {
      t.program.inputs.push_back(n.id);
    }
    t.program.nodes.push_back(n);
    t.program.pos[n.id] = t.program.nodes.size() - 1;
    t.subgraphs[n.id] = Subgraph::Optimizer;
    return n.id;
  }
  uint32_t op(Op o, std::vector<uint32_t> operands) { return push(make(0, o, std::move(operands))); }
  uint32_t scalar(float v) {
    Node n = make(0, Op::Scalar, {});
    n.scalar = v;
    return push(n);
  }
  uint32_t input(const std::string& name, const Type& ty) {
    Node n = make(0, Op::Input, {});
    n.name = name;
    n.ty = ty;
    return push(n);
  }
};

uint32_t first_read(const Program& p, uint32_t param) {
  for (auto& n : p.nodes)
    if (n.op == Op::ParamRead && n.param == param) return n.id;
  fail("a parameter with a gradient is not read");
}

void check_attach(const TrainingStep& t, float lr) {
  if (t.has_optimizer) fail("the step already has an optimizer");
  if (!(lr > 0.0f) || !std::isfinite(lr)) fail("the learning rate is not positive and finite");
}
}  // namespace

void attach_sgd(TrainingStep& t, float lr) {
  check_attach(t, lr);
  Appender app(t);
  if (!t.gradients.empty()) {
    uint32_t rate = app.scalar(lr);
    for (auto& [param, grad] : t.gradients) {
      uint32_t read = first_read(t.program, param);
      uint32_t scaled = app.op(Op::Mul, {rate, grad});
      t.updates[param] = app.op(Op::Sub, {read, scaled});
    }
  }
  for (auto& [param, u] : t.updates) t.program.outputs.push_back(u);
  uint32_t token = 0;
  for (auto& n : t.program.nodes)
    if (n.op == Op::ParamRead) t.effects[n.id] = Effect{token++, n.param, false, 0, 0};
  for (auto& [param, u] : t.updates) t.effects[u] = Effect{token++, param, true, 1, 0};
  t.has_optimizer = true;
  t.rule = Rule::Sgd;
  t.lr = lr;
}

void attach_adamw(TrainingStep& t, float lr, const AdamWConfig& a) {
  check_attach(t, lr);
  auto beta_ok = [](float b) { return b >= 0.0f && b < 1.0f; };
  if (!(std::isfinite(a.weight_decay) && a.weight_decay >= 0.0f && beta_ok(a.beta1) && beta_ok(a.beta2) &&
        std::isfinite(a.eps) && a.eps > 0.0f))
    fail("AdamW hyperparameters are out of range");
  Appender app(t);
  if (!t.gradients.empty()) {
    float k[6];
    a.constants(k);
    uint32_t c[6];
    for (int i = 0; i < 6; ++i) c[i] = app.scalar(k[i]);
    const uint32_t beta1 = c[0], rest1 = c[1], beta2 = c[2], rest2 = c[3], eps = c[4], decay = c[5];
    Type rank0 = Type::f32({});
    t.lr_t = app.input(kLrTInput, rank0);
    t.c1 = app.input(kC1Input, rank0);
    t.c2 = app.input(kC2Input, rank0);
    for (auto& [param, g] : t.gradients) {
      const ParamDecl decl = t.program.params.at(param);
      uint32_t p = first_read(t.program, param);
      uint32_t m = app.input(moment_input('m', decl.path), decl.ty);
      uint32_t v = app.input(moment_input('v', decl.path), decl.ty);
      uint32_t decayed_m = app.op(Op::Mul, {beta1, m});
      uint32_t new_m = app.op(Op::Mul, {rest1, g});
      uint32_t m_next = app.op(Op::Add, {decayed_m, new_m});
      uint32_t decayed_v = app.op(Op::Mul, {beta2, v});
      uint32_t scaled_g = app.op(Op::Mul, {rest2, g});
      uint32_t new_v = app.op(Op::Mul, {scaled_g, g});
      uint32_t v_next = app.op(Op::Add, {decayed_v, new_v});
      uint32_t m_hat = app.op(Op::Mul, {m_next, *t.c1});
      uint32_t v_hat = app.op(Op::Mul, {v_next, *t.c2});
      uint32_t root = app.op(Op::Sqrt, {v_hat});
      uint32_t denominator = app.op(Op::Add, {root, eps});
      uint32_t direction = app.op(Op::Div, {m_hat, denominator});
      uint32_t shrink = app.op(Op::Mul, {decay, p});
      uint32_t step = app.op(Op::Add, {direction, shrink});
      uint32_t scaled = app.op(Op::Mul, {*t.lr_t, step});
      t.updates[param] = app.op(Op::Sub, {p, scaled});
      t.moments[param] = Moments{m, v, m_next, v_next};
    }
  }
  for (auto& [param, u] : t.updates) t.program.outputs.push_back(u);
  for (auto& [param, m] : t.moments) {
    t.program.outputs.push_back(m.m_next);
    t.program.outputs.push_back(m.v_next);
  }
  uint32_t token = 0;
  for (auto& n : t.program.nodes)
    if (n.op == Op::ParamRead) t.effects[n.id] = Effect{token++, n.param, false, 0, 0};
  for (auto& [param, m] : t.moments) {
    t.effects[m.m] = Effect{token++, param, false, 0, 'm'};
    t.effects[m.v] = Effect{token++, param, false, 0, 'v'};
  }
  for (auto& [param, u] : t.updates) t.effects[u] = Effect{token++, param, true, 1, 0};
  for (auto& [param, m] : t.moments) {
    t.effects[m.m_next] = Effect{token++, param, true, 1, 'm'};
    t.effects[m.v_next] = Effect{token++, param, true, 1, 'v'};
  }
  t.has_optimizer = true;
  t.rule = Rule::AdamW;
  t.lr = lr;
  t.adamw = a;
}

}  // namespace msx
