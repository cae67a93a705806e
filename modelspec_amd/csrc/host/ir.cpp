// Tensor IR types, typing rules, the builder and the text form. See ir.h.
#include "ir.h"
#include "rng.h"

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <set>
#include <sstream>

namespace msx {

namespace {
const char* const kOpNames[] = {
    "Input", "ParamRead", "Scalar", "Add", "Sub", "Mul", "MatMul", "Relu", "Transpose", "ReduceSum",
    "ReduceMean", "Mse", "ReluGrad", "BroadcastScalar", "Embedding", "EmbeddingGrad", "AddRows",
    "SumRows", "Gelu", "GeluGrad", "LayerNorm", "LayerNormGradX", "LayerNormGradGamma", "Softmax",
    "SoftmaxGrad", "Attention", "AttentionGradQ", "AttentionGradK", "AttentionGradV", "CrossEntropy",
    "CrossEntropyGrad", "Dropout", "DropoutGrad", "StopGradient", "Sqrt", "Div"};
static_assert(sizeof(kOpNames) / sizeof(kOpNames[0]) == size_t(Op::Count_), "op names");

[[noreturn]] void fail(const std::string& what) { throw IrError(what); }
}  // namespace

const char* const kLrTInput = "optimizer.lr_t";
const char* const kC1Input = "optimizer.c1";
const char* const kC2Input = "optimizer.c2";
const char* const kMaskedRowsInput = "masked.rows";
const char* const kMaskedLabelsPrefix = "masked.labels.";
const char* const kMaskedWeightsPrefix = "masked.weights.";

std::string moment_input(char moment, const std::string& path) {
  return std::string("optimizer.") + moment + "@" + path;
}

const char* op_name(Op op) { return kOpNames[size_t(op)]; }

std::optional<Op> op_from_name(const std::string& name) {
  for (size_t i = 0; i < size_t(Op::Count_); ++i)
    if (name == kOpNames[i]) return Op(i);
  return std::nullopt;
}

const char* init_name(Init i) {
  switch (i) {
    case Init::XavierUniform: return "xavier_uniform";
    case Init::Zeros: return "zeros";
    case Init::Ones: return "ones";
  }
  return "?";
}

std::string type_string(const Type& t) {
  std::string s = "Tensor<";
  s += t.dtype == DType::F32 ? "f32" : "i32";
  s += ", [";
  for (size_t i = 0; i < t.shape.size(); ++i) {
    if (i) s += ", ";
    s += std::to_string(t.shape[i]);
  }
  return s + "]>";
}

void Program::reindex() {
  pos.clear();
  for (size_t i = 0; i < nodes.size(); ++i) pos[nodes[i].id] = i;
}

const Node& Program::node(uint32_t id) const {
  auto it = pos.find(id);
  if (it == pos.end()) fail("value %" + std::to_string(id) + " is not defined");
  return nodes[it->second];
}

Node& Program::node(uint32_t id) {
  auto it = pos.find(id);
  if (it == pos.end()) fail("value %" + std::to_string(id) + " is not defined");
  return nodes[it->second];
}

uint32_t Program::next_id() const {
  uint32_t n = 0;
  for (auto& x : nodes) n = std::max(n, x.id + 1);
  return n;
}

const Node* Program::input(const std::string& name) const {
  for (auto& n : nodes)
    if (n.op == Op::Input && n.name == name) return &n;
  return nullptr;
}

int token_operand(Op op) {
  if (op == Op::Dropout) return 1;
  if (op == Op::DropoutGrad) return 0;
  return -1;
}

// ---------------------------------------------------------------------------------------------
// Typing (ops.rs:334 `infer`): the result type of each op, with the operand checks that keep the
// kernels' shape assumptions true.
Type infer(const Node& n, const std::vector<const Type*>& a) {
  auto need = [&](size_t k) {
    if (a.size() != k)
      fail(std::string(op_name(n.op)) + " takes " + std::to_string(k) + " operands; got " + std::to_string(a.size()));
  };
  auto f32 = [&](const Type* t) {
    if (t->dtype != DType::F32) fail(std::string(op_name(n.op)) + ": operand is not f32");
  };
  auto rank = [&](const Type* t, int r) {
    if (t->rank() != r) fail(std::string(op_name(n.op)) + ": operand " + type_string(*t) + " is not rank " + std::to_string(r));
  };
  switch (n.op) {
    case Op::Input: case Op::ParamRead: fail("Input and ParamRead are typed by their declaration");
    case Op::Scalar: need(0); return Type::f32({});
    case Op::Add: case Op::Sub: case Op::Mul: case Op::Div: {
      need(2); f32(a[0]); f32(a[1]);
      if (*a[0] == *a[1]) return *a[0];
      if (a[1]->rank() == 0) return *a[0];
      if (a[0]->rank() == 0) return *a[1];
      fail(std::string(op_name(n.op)) + ": shapes " + type_string(*a[0]) + " and " + type_string(*a[1]));
    }
    case Op::MatMul: {
      need(2); f32(a[0]); f32(a[1]); rank(a[0], 2); rank(a[1], 2);
      if (a[0]->shape[1] != a[1]->shape[0]) fail("MatMul: inner dimensions differ");
      return Type::f32({a[0]->shape[0], a[1]->shape[1]});
    }
    case Op::Relu: case Op::Gelu: case Op::Sqrt: case Op::StopGradient: need(1); f32(a[0]); return *a[0];
    case Op::Softmax: need(1); f32(a[0]); rank(a[0], 2); return *a[0];
    case Op::Transpose: need(1); f32(a[0]); rank(a[0], 2); return Type::f32({a[0]->shape[1], a[0]->shape[0]});
    case Op::ReduceSum: case Op::ReduceMean: need(1); f32(a[0]); return Type::f32({});
    case Op::Mse: need(2); f32(a[0]); if (*a[0] != *a[1]) fail("Mse: shapes differ"); return Type::f32({});
    case Op::ReluGrad: case Op::GeluGrad: case Op::SoftmaxGrad:
      need(2); f32(a[0]); if (*a[0] != *a[1]) fail(std::string(op_name(n.op)) + ": shapes differ"); return *a[0];
    case Op::BroadcastScalar: need(1); f32(a[0]); rank(a[0], 0); return Type::f32(n.bshape);
    case Op::Embedding: {
      need(2); f32(a[0]); rank(a[0], 2); rank(a[1], 1);
      if (a[1]->dtype != DType::I32) fail("Embedding: ids are not i32");
      return Type::f32({a[1]->shape[0], a[0]->shape[1]});
    }
    case Op::EmbeddingGrad: {
      need(2); rank(a[0], 1); rank(a[1], 2); f32(a[1]);
      if (a[0]->dtype != DType::I32) fail("EmbeddingGrad: ids are not i32");
      if (a[0]->shape[0] != a[1]->shape[0]) fail("EmbeddingGrad: ids and rows differ");
      return Type::f32({n.rows, a[1]->shape[1]});
    }
    case Op::AddRows: {
      need(2); f32(a[0]); f32(a[1]); rank(a[0], 2); rank(a[1], 1);
      if (a[0]->shape[1] != a[1]->shape[0]) fail("AddRows: widths differ");
      return *a[0];
    }
    case Op::SumRows: need(1); f32(a[0]); rank(a[0], 2); return Type::f32({a[0]->shape[1]});
    case Op::LayerNorm: case Op::LayerNormGradX: {
      need(3); f32(a[0]); rank(a[0], 2); rank(a[1], 1);
      if (a[1]->shape[0] != a[0]->shape[1]) fail("LayerNorm: gamma width differs");
      if (n.op == Op::LayerNorm) { rank(a[2], 1); if (a[2]->shape[0] != a[0]->shape[1]) fail("LayerNorm: beta width differs"); }
      else if (*a[2] != *a[0]) fail("LayerNormGradX: gradient shape differs");
      return *a[0];
    }
    case Op::LayerNormGradGamma: need(2); rank(a[0], 2); if (*a[0] != *a[1]) fail("LayerNormGradGamma: shapes differ"); return Type::f32({a[0]->shape[1]});
    case Op::Attention: case Op::AttentionGradQ: case Op::AttentionGradK: case Op::AttentionGradV: {
      need(n.op == Op::Attention ? 4 : 5);
      rank(a[0], 2); rank(a[1], 2); rank(a[2], 2); rank(a[3], 2);
      if (n.heads <= 0 || a[0]->shape[1] % n.heads) fail("Attention: heads do not divide the width");
      if (a[1]->shape != a[2]->shape || a[0]->shape[1] != a[1]->shape[1]) fail("Attention: q, k, v widths differ");
      if (a[3]->dtype == DType::F32) {
        int64_t b = a[3]->shape[0], s = a[3]->shape[1];
        if (a[1]->shape[0] != b * s) fail("Attention: key rows are not B*S");
        if (a[0]->shape[0] % b || a[0]->shape[0] / b > s || a[0]->shape[0] / b < 1) fail("Attention: query rows");
      } else if (a[3]->shape[1] != 2) {
        fail("Attention: spans are not [U, 2]");
      }
      if (n.op == Op::Attention) return *a[0];
      if (*a[4] != *a[0]) fail("Attention gradient: G is not q's shape");
      if (n.op == Op::AttentionGradQ) return *a[0];
      return n.op == Op::AttentionGradK ? *a[1] : *a[2];
    }
    case Op::CrossEntropy: case Op::CrossEntropyGrad: {
      need(n.op == Op::CrossEntropy ? 3 : 4);
      rank(a[0], 2); f32(a[0]); rank(a[1], 1); rank(a[2], 1);
      if (a[1]->dtype != DType::I32) fail("CrossEntropy: labels are not i32");
      if (a[1]->shape[0] != a[0]->shape[0] || a[2]->shape[0] != a[0]->shape[0]) fail("CrossEntropy: rows differ");
      if (n.op == Op::CrossEntropy) return Type::f32({});
      rank(a[3], 0);
      return *a[0];
    }
    case Op::Dropout: {
      need(2); f32(a[0]);
      if (*a[1] != Type::i32({2})) fail("Dropout: the token is not i32[2]");
      return *a[0];
    }
    case Op::DropoutGrad: {
      need(2); f32(a[1]);
      if (*a[0] != Type::i32({2})) fail("DropoutGrad: the token is not i32[2]");
      return *a[1];
    }
    case Op::Count_: break;
  }
  fail("unknown op");
}

// ---------------------------------------------------------------------------------------------
uint32_t Builder::declare_param(const std::string& path, Type ty, Init init) {
  prog.params.push_back(ParamDecl{path, std::move(ty), init});
  return uint32_t(prog.params.size() - 1);
}

uint32_t Builder::input(const std::string& name, Type ty) {
  Node n;
  n.id = uint32_t(prog.nodes.size() ? prog.nodes.back().id + 1 : 0);
  n.op = Op::Input;
  n.name = name;
  n.ty = std::move(ty);
  prog.nodes.push_back(n);
  prog.inputs.push_back(n.id);
  prog.pos[n.id] = prog.nodes.size() - 1;
  return n.id;
}

uint32_t Builder::param_read(uint32_t param) {
  Node n;
  n.id = uint32_t(prog.nodes.size() ? prog.nodes.back().id + 1 : 0);
  n.op = Op::ParamRead;
  n.param = param;
  n.ty = prog.params.at(param).ty;
  prog.nodes.push_back(n);
  prog.pos[n.id] = prog.nodes.size() - 1;
  return n.id;
}

uint32_t Builder::scalar(float v) { return op(Op::Scalar, {}, v); }

uint32_t Builder::op(Op o, std::vector<uint32_t> operands, float attr, int64_t heads) {
  Node n;
  n.id = uint32_t(prog.nodes.size() ? prog.nodes.back().id + 1 : 0);
  n.op = o;
  n.operands = std::move(operands);
  n.scalar = attr;
  n.heads = heads;
  std::vector<const Type*> types;
  for (auto v : n.operands) types.push_back(&prog.node(v).ty);
  n.ty = infer(n, types);
  prog.nodes.push_back(n);
  prog.pos[n.id] = prog.nodes.size() - 1;
  return n.id;
}

Program Builder::finish() {
  prog.reindex();
  return std::move(prog);
}

// ---------------------------------------------------------------------------------------------
// Rust float formatting: the shortest digits that round-trip, from std::to_chars.
namespace {
struct Digits {
  bool neg;
  std::string digits;  // no leading zeros (or "0")
  int exp10;           // value = 0.digits * 10^exp10 ... we use: d1.d2d3 * 10^exp10
};

Digits shortest(float v) {
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
  std::string s(buf, r.ptr);
  Digits d;
  d.neg = s[0] == '-';
  if (d.neg) s = s.substr(1);
  auto e = s.find('e');
  std::string mant = s.substr(0, e);
  d.exp10 = std::atoi(s.c_str() + e + 1);
  for (char c : mant)
    if (c != '.') d.digits.push_back(c);
  while (d.digits.size() > 1 && d.digits.back() == '0') d.digits.pop_back();
  return d;
}

std::string fixed(const Digits& d, bool force_fraction) {
  std::string out = d.neg ? "-" : "";
  int n = int(d.digits.size());
  int point = d.exp10 + 1;  // digits before the decimal point
  if (d.digits == "0") {
    out += force_fraction ? "0.0" : "0";
    return out;
  }
  if (point <= 0) {
    out += "0.";
    out += std::string(size_t(-point), '0');
    out += d.digits;
  } else if (point >= n) {
    out += d.digits;
    out += std::string(size_t(point - n), '0');
    if (force_fraction) out += ".0";
  } else {
    out += d.digits.substr(0, size_t(point));
    out += ".";
    out += d.digits.substr(size_t(point));
  }
  return out;
}
}  // namespace

std::string f32_display(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
  return fixed(shortest(v), false);
}

std::string f32_debug(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
  float a = std::fabs(v);
  Digits d = shortest(v);
  if ((a != 0.0f && a < 1e-4f) || a >= 1e16f) {
    std::string out = d.neg ? "-" : "";
    out += d.digits.substr(0, 1);
    if (d.digits.size() > 1) out += "." + d.digits.substr(1);
    out += "e" + std::to_string(d.exp10);
    return out;
  }
  return fixed(d, true);
}

// ---------------------------------------------------------------------------------------------
namespace {
std::string shape_list(const std::vector<int64_t>& s) {
  std::string out = "[";
  for (size_t i = 0; i < s.size(); ++i) {
    if (i) out += ", ";
    out += std::to_string(s[i]);
  }
  return out + "]";
}

std::string quoted(const std::string& s) {
  std::string out = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') out += '\\';
    out += c;
  }
  return out + "\"";
}

void write_node(std::string& out, const Program& p, const Node& n) {
  out += "%" + std::to_string(n.id) + ": " + type_string(n.ty) + " = " + op_name(n.op);
  switch (n.op) {
    case Op::Input: out += " " + quoted(n.name); break;
    case Op::ParamRead: out += " @" + p.params.at(n.param).path; break;
    case Op::Scalar: out += " " + f32_debug(n.scalar); break;
    case Op::BroadcastScalar: out += " " + shape_list(n.bshape); break;
    case Op::EmbeddingGrad: out += " [" + std::to_string(n.rows) + "]"; break;
    case Op::Attention: case Op::AttentionGradQ: case Op::AttentionGradK: case Op::AttentionGradV:
      out += " [heads = " + std::to_string(n.heads) + "]";
      break;
    case Op::Dropout: case Op::DropoutGrad: {
      out += " [p = " + f32_debug(n.scalar) + ", site = ";
      uint32_t t = n.operands.at(size_t(token_operand(n.op)));
      const Node* tok = p.has(t) ? &p.node(t) : nullptr;
      out += (tok && tok->op == Op::Input) ? tok->name : "?";
      out += "]";
      break;
    }
    default: break;
  }
  for (size_t i = 0; i < n.operands.size(); ++i) out += std::string(i ? ", " : " ") + "%" + std::to_string(n.operands[i]);
}

const char* tag_name(Subgraph s) {
  switch (s) {
    case Subgraph::Forward: return "forward";
    case Subgraph::Loss: return "loss";
    case Subgraph::Gradient: return "gradient";
    case Subgraph::Optimizer: return "optimizer";
  }
  return "?";
}
}  // namespace

std::string print_program(const Program& p) {
  std::string out;
  for (auto& d : p.params) out += "param @" + d.path + ": " + type_string(d.ty) + " = " + init_name(d.init) + "\n";
  for (auto& n : p.nodes) {
    write_node(out, p, n);
    out += "\n";
  }
  for (auto o : p.outputs) out += "output %" + std::to_string(o) + "\n";
  return out;
}

std::string print_step(const TrainingStep& t) {
  const Program& p = t.program;
  std::string out;
  for (size_t i = 0; i < p.params.size(); ++i) {
    auto& d = p.params[i];
    out += "param @" + d.path + ": " + type_string(d.ty) + " = " + init_name(d.init);
    if (t.has_optimizer) out += " {v0}";
    out += "\n";
  }
  if (t.has_optimizer) {
    if (t.rule == Rule::Sgd) {
      out += "optimizer sgd lr = " + f32_debug(t.lr) + "\n";
    } else {
      auto& a = t.adamw;
      out += "optimizer adamw lr = " + f32_debug(t.lr) + " weight_decay = " + f32_debug(a.weight_decay) +
             " beta1 = " + f32_debug(a.beta1) + " beta2 = " + f32_debug(a.beta2) + " eps = " + f32_debug(a.eps) +
             " warmup_steps = " + std::to_string(a.warmup_steps) + "\n";
    }
  }
  for (auto& n : p.nodes) {
    auto tag = t.subgraphs.find(n.id);
    if (tag != t.subgraphs.end()) out += std::string(tag_name(tag->second)) + " ";
    write_node(out, p, n);
    auto e = t.effects.find(n.id);
    if (e != t.effects.end()) {
      const Effect& f = e->second;
      out += " {!" + std::to_string(f.token) + (f.write ? " write " : " read ");
      if (f.moment) out += std::string(1, f.moment);
      out += "@" + p.params.at(f.param).path + " v" + std::to_string(f.version) + "}";
    }
    out += "\n";
  }
  for (auto o : p.outputs) {
    out += "output %" + std::to_string(o);
    bool done = false;
    if (o == t.loss) { out += " loss"; done = true; }
    if (!done)
      for (auto& [param, v] : t.gradients)
        if (v == o) { out += " gradient @" + p.params[param].path; done = true; break; }
    if (!done)
      for (auto& [param, v] : t.updates)
        if (v == o) { out += " update @" + p.params[param].path; done = true; break; }
    if (!done)
      for (auto& [param, m] : t.moments) {
        if (m.m_next == o) { out += " moment m @" + p.params[param].path; done = true; break; }
        if (m.v_next == o) { out += " moment v @" + p.params[param].path; done = true; break; }
      }
    out += "\n";
  }
  return out;
}

// ---------------------------------------------------------------------------------------------
// The parser: the inverse of print_step / print_program over the ops this backend runs.
namespace {
struct Cursor {
  const std::string& s;
  size_t i = 0;
  explicit Cursor(const std::string& line) : s(line) {}
  void ws() { while (i < s.size() && s[i] == ' ') ++i; }
  bool eat(const std::string& t) {
    ws();
    if (s.compare(i, t.size(), t) == 0) { i += t.size(); return true; }
    return false;
  }
  void expect(const std::string& t) {
    if (!eat(t)) fail("IR text: expected `" + t + "` at column " + std::to_string(i) + " of: " + s);
  }
  std::string word() {  // up to a space, comma, bracket or colon
    ws();
    size_t j = i;
    while (j < s.size() && s[j] != ' ' && s[j] != ',' && s[j] != ']' && s[j] != ':' && s[j] != '}') ++j;
    std::string w = s.substr(i, j - i);
    i = j;
    return w;
  }
  int64_t integer() {
    std::string w = word();
    char* end = nullptr;
    long long v = std::strtoll(w.c_str(), &end, 10);
    if (w.empty() || *end) fail("IR text: expected an integer, got `" + w + "` in: " + s);
    return v;
  }
  float number() {
    std::string w = word();
    char* end = nullptr;
    float v = std::strtof(w.c_str(), &end);
    if (w.empty() || *end) fail("IR text: expected a number, got `" + w + "` in: " + s);
    return v;
  }
  uint32_t value() {
    expect("%");
    return uint32_t(integer());
  }
  std::string str() {
    expect("\"");
    std::string out;
    while (i < s.size() && s[i] != '"') {
      if (s[i] == '\\' && i + 1 < s.size()) ++i;
      out += s[i++];
    }
    expect("\"");
    return out;
  }
  std::vector<int64_t> shape() {
    expect("[");
    std::vector<int64_t> out;
    if (eat("]")) return out;
    do { out.push_back(integer()); } while (eat(","));
    expect("]");
    return out;
  }
  Type type() {
    expect("Tensor<");
    Type t;
    std::string d = word();
    if (d == "f32") t.dtype = DType::F32;
    else if (d == "i32") t.dtype = DType::I32;
    else fail("IR text: unknown dtype " + d);
    expect(",");
    t.shape = shape();
    expect(">");
    return t;
  }
  bool done() { ws(); return i >= s.size(); }
};

std::map<std::string, uint32_t> param_index(const Program& p) {
  std::map<std::string, uint32_t> m;
  for (size_t k = 0; k < p.params.size(); ++k) m[p.params[k].path] = uint32_t(k);
  return m;
}

uint32_t param_at(const std::map<std::string, uint32_t>& m, const std::string& path) {
  auto it = m.find(path);
  if (it == m.end()) fail("IR text: unknown parameter @" + path);
  return it->second;
}

// One node line after its optional tag. Returns the node; `effect` is filled when present.
Node parse_node(Cursor& c, const Program& p, const std::map<std::string, uint32_t>& params,
                std::optional<Effect>* effect) {
  Node n;
  n.id = c.value();
  c.expect(":");
  n.ty = c.type();
  c.expect("=");
  std::string name = c.word();
  auto op = op_from_name(name);
  if (!op) fail("IR text: unknown op " + name);
  n.op = *op;
  std::string site;
  switch (n.op) {
    case Op::Input: n.name = c.str(); break;
    case Op::ParamRead: c.expect("@"); n.param = param_at(params, c.word()); break;
    case Op::Scalar: n.scalar = c.number(); break;
    case Op::BroadcastScalar: n.bshape = c.shape(); break;
    case Op::EmbeddingGrad: c.expect("["); n.rows = c.integer(); c.expect("]"); break;
    case Op::Attention: case Op::AttentionGradQ: case Op::AttentionGradK: case Op::AttentionGradV:
      c.expect("["); c.expect("heads"); c.expect("="); n.heads = c.integer(); c.expect("]");
      break;
    case Op::Dropout: case Op::DropoutGrad:
      c.expect("["); c.expect("p"); c.expect("="); n.scalar = c.number(); c.expect(",");
      c.expect("site"); c.expect("="); site = c.word(); c.expect("]");
      break;
    default: break;
  }
  if (c.eat("%")) {
    c.i -= 1;
    do { n.operands.push_back(c.value()); } while (c.eat(","));
  }
  if (c.eat("{")) {
    Effect e{};
    c.expect("!");
    e.token = uint32_t(c.integer());
    std::string access = c.word();
    e.write = access == "write";
    c.ws();
    if (c.s[c.i] != '@') { e.moment = c.s[c.i]; ++c.i; }
    c.expect("@");
    e.param = param_at(params, c.word());
    c.expect("v");
    e.version = uint64_t(c.integer());
    c.expect("}");
    if (effect) *effect = e;
  }
  if (!c.done()) fail("IR text: trailing text in: " + c.s);
  (void)p;
  return n;
}

Init init_from(const std::string& w) {
  if (w == "xavier_uniform") return Init::XavierUniform;
  if (w == "zeros") return Init::Zeros;
  if (w == "ones") return Init::Ones;
  fail("IR text: unknown initializer " + w);
}

// Re-types every node by the registry and checks it against the printed type.
void retype(Program& p) {
  p.reindex();
  for (auto& n : p.nodes) {
    if (n.op == Op::Input) continue;
    if (n.op == Op::ParamRead) {
      if (p.params.at(n.param).ty != n.ty) fail("IR text: ParamRead type differs from its declaration");
      continue;
    }
    std::vector<const Type*> types;
    for (auto v : n.operands) {
      auto it = p.pos.find(v);
      if (it == p.pos.end() || it->second >= size_t(&n - p.nodes.data()))
        fail("IR text: %" + std::to_string(n.id) + " reads %" + std::to_string(v) + " before its definition");
      types.push_back(&p.nodes[it->second].ty);
    }
    Type t = infer(n, types);
    if (t != n.ty) fail("IR text: %" + std::to_string(n.id) + " is printed " + type_string(n.ty) + " but types as " + type_string(t));
  }
}
}  // namespace

TrainingStep parse_step(const std::string& text) {
  TrainingStep t;
  Program& p = t.program;
  std::istringstream in(text);
  std::string line;
  std::map<std::string, uint32_t> params;
  struct Role { uint32_t value; std::string kind, arg; };
  std::vector<Role> roles;
  while (std::getline(in, line)) {
    if (line.empty()) continue;
    Cursor c(line);
    if (c.eat("param ")) {
      c.expect("@");
      ParamDecl d;
      d.path = c.word();
      c.expect(":");
      d.ty = c.type();
      c.expect("=");
      d.init = init_from(c.word());
      if (c.eat("{")) { c.word(); c.expect("}"); t.has_optimizer = true; }
      p.params.push_back(d);
      params = param_index(p);
      continue;
    }
    if (c.eat("optimizer sgd")) {
      t.has_optimizer = true;
      t.rule = Rule::Sgd;
      c.expect("lr"); c.expect("="); t.lr = c.number();
      continue;
    }
    if (c.eat("optimizer adamw")) {
      t.has_optimizer = true;
      t.rule = Rule::AdamW;
      c.expect("lr"); c.expect("="); t.lr = c.number();
      c.expect("weight_decay"); c.expect("="); t.adamw.weight_decay = c.number();
      c.expect("beta1"); c.expect("="); t.adamw.beta1 = c.number();
      c.expect("beta2"); c.expect("="); t.adamw.beta2 = c.number();
      c.expect("eps"); c.expect("="); t.adamw.eps = c.number();
      c.expect("warmup_steps"); c.expect("="); t.adamw.warmup_steps = uint64_t(c.integer());
      continue;
    }
    if (c.eat("output ")) {
      Role r;
      r.value = c.value();
      r.kind = c.done() ? "" : c.word();
      if (r.kind == "moment") { r.arg = c.word(); c.expect("@"); r.arg += "@" + c.word(); }
      else if (!r.kind.empty() && r.kind != "loss") { c.expect("@"); r.arg = c.word(); }
      roles.push_back(r);
      p.outputs.push_back(r.value);
      continue;
    }
    Subgraph tag = Subgraph::Forward;
    bool tagged = true;
    if (c.eat("forward ")) tag = Subgraph::Forward;
    else if (c.eat("loss ")) tag = Subgraph::Loss;
    else if (c.eat("gradient ")) tag = Subgraph::Gradient;
    else if (c.eat("optimizer ")) tag = Subgraph::Optimizer;
    else tagged = false;
    std::optional<Effect> effect;
    Node n = parse_node(c, p, params, &effect);
    if (tagged) t.subgraphs[n.id] = tag;
    if (effect) t.effects[n.id] = *effect;
    if (n.op == Op::Input) p.inputs.push_back(n.id);
    p.nodes.push_back(n);
  }
  retype(p);
  bool have_loss = false;
  for (auto& r : roles) {
    if (r.kind == "loss") { t.loss = r.value; have_loss = true; }
    else if (r.kind == "gradient") t.gradients[param_at(params, r.arg)] = r.value;
    else if (r.kind == "update") t.updates[param_at(params, r.arg)] = r.value;
    else if (r.kind == "moment") {
      char m = r.arg[0];
      uint32_t param = param_at(params, r.arg.substr(2));
      auto& mo = t.moments[param];
      const Node* in = p.input(moment_input(m, p.params[param].path));
      if (!in) fail("IR text: no moment input for " + r.arg);
      if (m == 'm') { mo.m_next = r.value; mo.m = in->id; }
      else { mo.v_next = r.value; mo.v = in->id; }
    }
  }
  if (!have_loss) {
    if (p.outputs.empty()) fail("IR text: the step has no loss output");
    t.loss = p.outputs[0];
  }
  if (const Node* n = p.input(kLrTInput)) t.lr_t = n->id;
  if (const Node* n = p.input(kC1Input)) t.c1 = n->id;
  if (const Node* n = p.input(kC2Input)) t.c2 = n->id;
  if (t.rule == Rule::AdamW && (!t.lr_t || !t.c1 || !t.c2)) fail("IR text: an AdamW step lacks its host inputs");
  return t;
}

Program parse_program(const std::string& text) {
  TrainingStep t = parse_step(text);
  t.program.outputs.clear();
  std::istringstream in(text);
  std::string line;
  while (std::getline(in, line)) {
    Cursor c(line);
    if (c.eat("output ")) t.program.outputs.push_back(c.value());
  }
  return std::move(t.program);
}

std::vector<std::string> dropout_sites(const Program& p) {
  std::set<uint32_t> tokens;
  for (auto& n : p.nodes) {
    int k = token_operand(n.op);
    if (k >= 0 && size_t(k) < n.operands.size()) tokens.insert(n.operands[size_t(k)]);
  }
  std::vector<std::string> out;
  for (auto v : p.inputs)
    if (tokens.count(v)) out.push_back(p.node(v).name);
  return out;
}

void AdamWConfig::constants(float out[6]) const {
  out[0] = beta1;
  out[1] = float(1.0 - double(beta1));
  out[2] = beta2;
  out[3] = float(1.0 - double(beta2));
  out[4] = eps;
  out[5] = weight_decay;
}

StepScalars adamw_scalars(const AdamWConfig& a, float lr, uint64_t t, uint64_t steps) {
  double peak = double(lr);
  uint64_t warmup = a.warmup_steps;
  double rate;
  if (t <= warmup) {
    rate = peak * double(t) / double(warmup);
  } else {
    uint64_t span = steps > warmup ? steps - warmup : 0;
    rate = span == 0 ? 0.0 : peak * double(steps > t ? steps - t : 0) / double(span);
  }
  int power = t > uint64_t(INT32_MAX) ? INT32_MAX : int(t);
  auto correction = [&](float beta) { return float(1.0 / (1.0 - powi(double(beta), power))); };
  return StepScalars{float(rate), correction(a.beta1), correction(a.beta2)};
}

}  // namespace msx
