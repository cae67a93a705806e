// The `.mspec` front-end: lexer, recursive-descent parser and lowering of the subset mspec.h
// describes.
#include "mspec.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <fstream>
#include <map>
#include <memory>
#include <set>
#include <sstream>

namespace msx {

namespace {

// --- lexer -------------------------------------------------------------------------------------

enum class Tok : uint8_t { Ident, Int, Float, Punct, End };

struct Token {
  Tok kind = Tok::End;
  std::string text;
  int line = 0, col = 0;
};

std::vector<Token> lex(const std::string& src) {
  std::vector<Token> out;
  int line = 1, col = 1;
  size_t i = 0;
  auto advance = [&](size_t n) {
    for (size_t k = 0; k < n; ++k, ++i) {
      if (src[i] == '\n') {
        ++line;
        col = 1;
      } else {
        ++col;
      }
    }
  };
  while (i < src.size()) {
    const char ch = src[i];
    if (ch == ' ' || ch == '\t' || ch == '\r' || ch == '\n') {
      advance(1);
      continue;
    }
    if (ch == '/' && i + 1 < src.size() && src[i + 1] == '/') {
      while (i < src.size() && src[i] != '\n') advance(1);
      continue;
    }
    Token t;
    t.line = line;
    t.col = col;
    if (std::isalpha(static_cast<unsigned char>(ch)) || ch == '_') {
      size_t j = i;
      while (j < src.size() && (std::isalnum(static_cast<unsigned char>(src[j])) || src[j] == '_')) ++j;
      t.kind = Tok::Ident;
      t.text = src.substr(i, j - i);
      advance(j - i);
    } else if (std::isdigit(static_cast<unsigned char>(ch))) {
      size_t j = i;
      bool real = false;
      while (j < src.size() && std::isdigit(static_cast<unsigned char>(src[j]))) ++j;
      if (j + 1 < src.size() && src[j] == '.' && std::isdigit(static_cast<unsigned char>(src[j + 1]))) {
        real = true;
        ++j;
        while (j < src.size() && std::isdigit(static_cast<unsigned char>(src[j]))) ++j;
      }
      if (j < src.size() && (src[j] == 'e' || src[j] == 'E')) {
        size_t k = j + 1;
        if (k < src.size() && (src[k] == '+' || src[k] == '-')) ++k;
        if (k < src.size() && std::isdigit(static_cast<unsigned char>(src[k]))) {
          real = true;
          j = k;
          while (j < src.size() && std::isdigit(static_cast<unsigned char>(src[j]))) ++j;
        }
      }
      t.kind = real ? Tok::Float : Tok::Int;
      t.text = src.substr(i, j - i);
      advance(j - i);
    } else if (ch == '-' && i + 1 < src.size() && src[i + 1] == '>') {
      t.kind = Tok::Punct;
      t.text = "->";
      advance(2);
    } else if (std::string("{}()[]<>,;:=.-").find(ch) != std::string::npos) {
      t.kind = Tok::Punct;
      t.text = std::string(1, ch);
      advance(1);
    } else {
      throw MspecError("E-SYNTAX-001", line, col, std::string("unexpected character `") + ch + "`");
    }
    out.push_back(t);
  }
  Token end;
  end.line = line;
  end.col = col;
  out.push_back(end);
  return out;
}

// --- syntax tree -------------------------------------------------------------------------------

struct Expr;
using ExprPtr = std::shared_ptr<Expr>;

struct Arg {
  std::string name;  // empty: positional
  ExprPtr value;
};

// A name, a number, `callee(args)` or `receiver.callee(args)`; line and column of its start (for
// a call, of the callee's name, the position the dropout sites are ranked by).
struct Expr {
  enum Kind { Name, Number, Call, MemberCall } kind = Name;
  std::string text;      // name, literal or callee
  std::string receiver;  // MemberCall
  bool integer = false;
  double number = 0;
  std::vector<Arg> args;
  int line = 0, col = 0;
};

struct Decl {
  std::string name;
  Type ty;
  int line = 0, col = 0;
};

struct ParamItem {
  Decl decl;
  std::string init;
  int init_line = 0, init_col = 0;
};

struct Function {
  std::string name;
  std::vector<Decl> args;
  Type result;
  std::vector<std::pair<std::string, ExprPtr>> lets;
  ExprPtr ret;
  int line = 0, col = 0;
};

struct ModelAst {
  std::string name;
  std::vector<ParamItem> params;
  std::vector<Function> functions;
  int line = 0, col = 0;
};

struct TrainAst {
  std::string name, model, device;
  std::vector<std::pair<Decl, bool>> data;  // (declaration, is target)
  ExprPtr loss;
  ExprPtr optimizer;
  int64_t steps = -1, seed = -1;
  int line = 0, col = 0;
};

// --- parser ------------------------------------------------------------------------------------

class Parser {
 public:
  explicit Parser(std::vector<Token> toks) : t_(std::move(toks)) {}

  void file(std::vector<ModelAst>& models, std::vector<TrainAst>& trains) {
    while (peek().kind != Tok::End) {
      const Token& k = peek();
      if (is("model")) models.push_back(model());
      else if (is("train")) trains.push_back(train());
      else fail(k, "expected `model` or `train`, found `" + k.text + "`");
    }
  }

 private:
  std::vector<Token> t_;
  size_t i_ = 0;

  const Token& peek(size_t ahead = 0) const { return t_[std::min(i_ + ahead, t_.size() - 1)]; }
  bool is(const std::string& text, size_t ahead = 0) const {
    const Token& k = peek(ahead);
    return (k.kind == Tok::Ident || k.kind == Tok::Punct) && k.text == text;
  }
  [[noreturn]] void fail(const Token& k, const std::string& what) const { throw MspecError("E-SYNTAX-001", k.line, k.col, what); }
  Token take() { return t_[std::min(i_++, t_.size() - 1)]; }
  void expect(const std::string& text) {
    if (!is(text)) fail(peek(), "expected `" + text + "`, found `" + (peek().kind == Tok::End ? "end of file" : peek().text) + "`");
    take();
  }
  Token ident(const std::string& what) {
    if (peek().kind != Tok::Ident) fail(peek(), "expected " + what);
    return take();
  }
  int64_t integer() {
    if (peek().kind != Tok::Int) fail(peek(), "expected an integer");
    return std::stoll(take().text);
  }

  Type type() {
    const Token at = peek();
    if (ident("a tensor type").text != "Tensor") fail(at, "expected `Tensor<dtype, [dims]>`");
    expect("<");
    const Token dt = ident("`f32` or `i32`");
    Type ty;
    if (dt.text == "f32") ty.dtype = DType::F32;
    else if (dt.text == "i32") ty.dtype = DType::I32;
    else fail(dt, "unknown element type `" + dt.text + "` (the subset has f32 and i32)");
    expect(",");
    expect("[");
    while (!is("]")) {
      ty.shape.push_back(integer());
      if (!is("]")) expect(",");
    }
    expect("]");
    expect(">");
    return ty;
  }

  Decl decl() {
    Decl d;
    const Token n = ident("a name");
    d.name = n.text;
    d.line = n.line;
    d.col = n.col;
    expect(":");
    d.ty = type();
    return d;
  }

  ExprPtr expr() {
    auto e = std::make_shared<Expr>();
    const Token& k = peek();
    e->line = k.line;
    e->col = k.col;
    if (is("-") && (peek(1).kind == Tok::Int || peek(1).kind == Tok::Float)) {
      take();
      const Token n = take();
      e->kind = Expr::Number;
      e->integer = n.kind == Tok::Int;
      e->number = -std::stod(n.text);
      e->text = "-" + n.text;
      return e;
    }
    if (k.kind == Tok::Int || k.kind == Tok::Float) {
      const Token n = take();
      e->kind = Expr::Number;
      e->integer = n.kind == Tok::Int;
      e->number = std::stod(n.text);
      e->text = n.text;
      return e;
    }
    const Token n = ident("an expression");
    if (is(".")) {
      take();
      const Token m = ident("a function name");
      e->kind = Expr::MemberCall;
      e->receiver = n.text;
      e->text = m.text;
      e->line = m.line;
      e->col = m.col;
      call_args(*e);
      return e;
    }
    e->text = n.text;
    if (is("(")) {
      e->kind = Expr::Call;
      call_args(*e);
    }
    return e;
  }

  void call_args(Expr& e) {
    expect("(");
    while (!is(")")) {
      Arg a;
      if (peek().kind == Tok::Ident && is("=", 1)) {
        a.name = take().text;
        take();
      }
      a.value = expr();
      e.args.push_back(a);
      if (!is(")")) expect(",");
    }
    expect(")");
  }

  ModelAst model() {
    ModelAst m;
    const Token kw = take();
    m.line = kw.line;
    m.col = kw.col;
    m.name = ident("a model name").text;
    if (is("<")) fail(peek(), "generic models are not in the subset");
    expect("{");
    while (!is("}")) {
      if (is("param")) {
        take();
        ParamItem p;
        p.decl = decl();
        expect("=");
        const Token init = ident("an initializer");
        p.init = init.text;
        p.init_line = init.line;
        p.init_col = init.col;
        expect("(");
        expect(")");
        expect(";");
        m.params.push_back(p);
      } else if (is("fn")) {
        const Token f = take();
        Function fn;
        fn.line = f.line;
        fn.col = f.col;
        fn.name = ident("a function name").text;
        if (is("<")) fail(peek(), "generic functions are not in the subset");
        expect("(");
        while (!is(")")) {
          fn.args.push_back(decl());
          if (!is(")")) expect(",");
        }
        expect(")");
        expect("->");
        fn.result = type();
        expect("{");
        while (!is("}")) {
          if (is("let")) {
            take();
            const std::string name = ident("a name").text;
            expect("=");
            fn.lets.push_back({name, expr()});
            expect(";");
          } else if (is("return")) {
            if (fn.ret) fail(peek(), "a function returns once");
            take();
            fn.ret = expr();
            expect(";");
          } else {
            fail(peek(), "expected `let` or `return`");
          }
        }
        expect("}");
        if (!fn.ret) fail(f, "function `" + fn.name + "` has no `return`");
        m.functions.push_back(fn);
      } else if (is("layer")) {
        fail(peek(), "`layer` items are not in the subset");
      } else {
        fail(peek(), "expected `param` or `fn`");
      }
    }
    expect("}");
    return m;
  }

  TrainAst train() {
    TrainAst tr;
    const Token kw = take();
    tr.line = kw.line;
    tr.col = kw.col;
    tr.name = ident("a train block name").text;
    expect("{");
    std::set<std::string> seen;
    while (!is("}")) {
      const Token key = ident("a train setting");
      const bool once = key.text != "input" && key.text != "target";
      if (once && !seen.insert(key.text).second) fail(key, "`" + key.text + "` is set twice");
      if (key.text == "model") {
        expect("=");
        tr.model = ident("a model name").text;
        if (is("<")) fail(peek(), "generic models are not in the subset");
      } else if (key.text == "input" || key.text == "target") {
        tr.data.push_back({decl(), key.text == "target"});
      } else if (key.text == "loss") {
        expect("=");
        tr.loss = expr();
      } else if (key.text == "optimizer") {
        expect("=");
        tr.optimizer = expr();
      } else if (key.text == "steps") {
        expect("=");
        tr.steps = integer();
      } else if (key.text == "seed") {
        expect("=");
        tr.seed = integer();
      } else if (key.text == "device") {
        expect("=");
        tr.device = ident("a device").text;
        if (is("(")) {
          take();
          tr.device += "(" + std::to_string(integer()) + ")";
          expect(")");
        }
      } else {
        fail(key, "unknown train setting `" + key.text + "`");
      }
      expect(";");
    }
    expect("}");
    for (const char* need : {"model", "loss", "optimizer", "steps", "seed"})
      if (!seen.count(need)) fail(kw, std::string("train block `") + tr.name + "` sets no `" + need + "`");
    return tr;
  }
};

// --- lowering ----------------------------------------------------------------------------------

// The source operators (resolve.rs:64-84) this IR has.
const std::map<std::string, Op>& operators() {
  static const std::map<std::string, Op> ops = {
      {"matmul", Op::MatMul},       {"add", Op::Add},         {"sub", Op::Sub},
      {"mul", Op::Mul},             {"relu", Op::Relu},       {"transpose", Op::Transpose},
      {"sum", Op::ReduceSum},       {"mean", Op::ReduceMean}, {"mse", Op::Mse},
      {"embedding", Op::Embedding}, {"add_rows", Op::AddRows}, {"gelu", Op::Gelu},
      {"layer_norm", Op::LayerNorm}, {"softmax", Op::Softmax}, {"attention", Op::Attention},
      {"cross_entropy", Op::CrossEntropy}, {"dropout", Op::Dropout}, {"stop_gradient", Op::StopGradient},
  };
  return ops;
}

// The dropout calls of `e` by source position, not entering the functions it calls
// (lower.rs:229-246).
void dropout_calls(const ExprPtr& e, std::vector<std::pair<int, int>>& out) {
  if (!e) return;
  if (e->kind == Expr::Call && e->text == "dropout") out.push_back({e->line, e->col});
  for (auto& a : e->args) dropout_calls(a.value, out);
}

struct Frame {
  const Function* fn = nullptr;  // null: the train block
  int instance = 0;
  std::map<std::string, uint32_t> values;  // arguments and lets (function) or data (train)
};

struct Lowerer {
  const ModelAst& model;
  const TrainAst& train;
  Builder b;
  std::map<std::string, uint32_t> reads;
  std::map<std::string, uint32_t> tokens;
  std::map<std::string, int> inlined;  // inlinings so far, by function
  std::vector<std::string> stack;      // functions being inlined
  std::vector<uint32_t> predictions;
  // The operator call that produced a value, for the feed inference.
  std::map<uint32_t, const Expr*> producer;

  Lowerer(const ModelAst& m, const TrainAst& t) : model(m), train(t) {}

  const Function* function(const std::string& name) const {
    for (auto& f : model.functions)
      if (f.name == name) return &f;
    return nullptr;
  }

  uint32_t token(const Expr& call, const Frame& frame) {
    std::vector<std::pair<int, int>> calls;
    std::string fname = "train";
    if (frame.fn) {
      for (auto& [_, e] : frame.fn->lets) dropout_calls(e, calls);
      dropout_calls(frame.fn->ret, calls);
      fname = frame.instance == 0 ? frame.fn->name : frame.fn->name + "@" + std::to_string(frame.instance);
    } else {
      dropout_calls(train.loss, calls);
    }
    std::sort(calls.begin(), calls.end());
    const auto at = std::lower_bound(calls.begin(), calls.end(), std::make_pair(call.line, call.col));
    const size_t k = size_t(at - calls.begin());
    const std::string site = model.name + "." + fname + ".dropout#" + std::to_string(k);
    auto it = tokens.find(site);
    if (it != tokens.end()) return it->second;
    const uint32_t t = b.input(site, Type::i32({2}));
    tokens[site] = t;
    return t;
  }

  double keyword(const Expr& call, const Arg& a, bool integer) {
    if (!a.value || a.value->kind != Expr::Number)
      throw MspecError("E-TYPE-001", call.line, call.col, "`" + a.name + "` of `" + call.text + "` takes a number");
    if (integer && !a.value->integer)
      throw MspecError("E-TYPE-001", call.line, call.col, "`" + a.name + "` of `" + call.text + "` takes an integer");
    return a.value->number;
  }

  uint32_t inline_call(const Function& f, std::vector<uint32_t> args, const Expr& at) {
    if (std::find(stack.begin(), stack.end(), f.name) != stack.end())
      throw MspecError("E-NAME-001", at.line, at.col, "function `" + f.name + "` calls itself");
    if (args.size() != f.args.size())
      throw MspecError("E-TYPE-001", at.line, at.col,
                       "`" + f.name + "` takes " + std::to_string(f.args.size()) + " argument(s); got " + std::to_string(args.size()));
    Frame frame;
    frame.fn = &f;
    frame.instance = inlined[f.name]++;
    for (size_t i = 0; i < args.size(); ++i) {
      const Type& have = b.prog.node(args[i]).ty;
      if (have != f.args[i].ty)
        throw MspecError("E-TYPE-001", at.line, at.col,
                         "argument `" + f.args[i].name + "` of `" + f.name + "` is " + type_string(f.args[i].ty) + "; got " + type_string(have));
      frame.values[f.args[i].name] = args[i];
    }
    stack.push_back(f.name);
    for (auto& [name, e] : f.lets) frame.values[name] = expr(*e, frame);
    const uint32_t v = expr(*f.ret, frame);
    stack.pop_back();
    if (b.prog.node(v).ty != f.result)
      throw MspecError("E-TYPE-001", f.line, f.col,
                       "`" + f.name + "` returns " + type_string(b.prog.node(v).ty) + ", not its declared " + type_string(f.result));
    return v;
  }

  uint32_t expr(const Expr& e, const Frame& frame) {
    switch (e.kind) {
      case Expr::Name: {
        auto it = frame.values.find(e.text);
        if (it != frame.values.end()) return it->second;
        if (frame.fn) {
          auto r = reads.find(e.text);
          if (r != reads.end()) return r->second;
        }
        throw MspecError("E-NAME-001", e.line, e.col, "unknown name `" + e.text + "`");
      }
      case Expr::Number:
        return b.scalar(float(e.number));
      case Expr::MemberCall: {
        if (e.receiver != "model")
          throw MspecError("E-NAME-001", e.line, e.col, "unknown receiver `" + e.receiver + "` (calls go to `model`)");
        const Function* f = function(e.text);
        if (!f) throw MspecError("E-NAME-001", e.line, e.col, "model `" + model.name + "` has no function `" + e.text + "`");
        std::vector<uint32_t> args;
        for (auto& a : e.args) {
          if (!a.name.empty()) throw MspecError("E-TYPE-001", e.line, e.col, "model functions take positional arguments");
          args.push_back(expr(*a.value, frame));
        }
        const uint32_t v = inline_call(*f, args, e);
        if (f->name == "forward") predictions.push_back(v);
        return v;
      }
      case Expr::Call: {
        if (const Function* f = frame.fn ? function(e.text) : nullptr) {
          std::vector<uint32_t> args;
          for (auto& a : e.args) args.push_back(expr(*a.value, frame));
          return inline_call(*f, args, e);
        }
        auto op = operators().find(e.text);
        if (op == operators().end())
          throw MspecError("E-NAME-001", e.line, e.col, "unknown operator `" + e.text + "`");
        std::vector<uint32_t> operands;
        float p = 0.0f;
        int64_t heads = 0;
        bool has_p = false, has_heads = false;
        for (auto& a : e.args) {
          if (a.name.empty()) {
            operands.push_back(expr(*a.value, frame));
          } else if (a.name == "p" && op->second == Op::Dropout) {
            p = float(keyword(e, a, false));
            has_p = true;
          } else if (a.name == "heads" && op->second == Op::Attention) {
            heads = int64_t(keyword(e, a, true));
            has_heads = true;
          } else {
            throw MspecError("E-TYPE-001", e.line, e.col, "`" + e.text + "` takes no argument `" + a.name + "`");
          }
        }
        if (op->second == Op::Dropout) {
          if (!has_p) throw MspecError("E-TYPE-001", e.line, e.col, "`dropout` needs `p = P`");
          if (operands.size() != 1) throw MspecError("E-TYPE-001", e.line, e.col, "`dropout` takes 1 operand");
          if (!(p >= 0.0f && p < 1.0f)) throw MspecError("E-TYPE-001", e.line, e.col, "`dropout` needs 0 <= p < 1");
          if (p == 0.0f) return operands[0];
          operands.push_back(token(e, frame));
        }
        if (op->second == Op::Attention && !has_heads) throw MspecError("E-TYPE-001", e.line, e.col, "`attention` needs `heads = A`");
        try {
          const uint32_t v = b.op(op->second, operands, p, heads);
          producer[v] = &e;
          return v;
        } catch (const MspecError&) {
          throw;
        } catch (const IrError& err) {
          throw MspecError("E-TYPE-001", e.line, e.col, "`" + e.text + "`: " + err.what());
        }
      }
    }
    throw MspecError("E-SYNTAX-001", e.line, e.col, "malformed expression");
  }
};

Init init_of(const ParamItem& p) {
  if (p.init == "xavier_uniform") return Init::XavierUniform;
  if (p.init == "zeros") return Init::Zeros;
  if (p.init == "ones") return Init::Ones;
  throw MspecError("E-NAME-001", p.init_line, p.init_col, "unknown initializer `" + p.init + "`");
}

}  // namespace

std::string read_mspec(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw MspecError("E-SYNTAX-001", 0, 0, "cannot read `" + path + "`");
  std::ostringstream s;
  s << f.rdbuf();
  return s.str();
}

Compiled compile_mspec(const std::string& source, const std::string& name, int64_t masked_rows_override,
                       int64_t steps_override) {
  std::vector<ModelAst> models;
  std::vector<TrainAst> trains;
  Parser(lex(source)).file(models, trains);
  if (trains.size() != 1) throw MspecError("E-TRAIN-002", 1, 1, "a file holds one `train` block, not " + std::to_string(trains.size()));
  const TrainAst& tr = trains[0];
  const ModelAst* model = nullptr;
  for (auto& m : models)
    if (m.name == tr.model) model = &m;
  if (!model) throw MspecError("E-NAME-001", tr.line, tr.col, "unknown model `" + tr.model + "`");

  Lowerer L(*model, tr);
  std::set<std::string> names;
  for (auto& p : model->params) {
    if (!names.insert(p.decl.name).second)
      throw MspecError("E-NAME-001", p.decl.line, p.decl.col, "`" + p.decl.name + "` is declared twice");
    L.b.declare_param(model->name + "." + p.decl.name, p.decl.ty, init_of(p));
  }
  Frame top;
  for (auto& [d, target] : tr.data) {
    if (top.values.count(d.name)) throw MspecError("E-NAME-001", d.line, d.col, "`" + d.name + "` is declared twice");
    top.values[d.name] = L.b.input(d.name, d.ty);
  }
  for (size_t i = 0; i < model->params.size(); ++i) L.reads[model->params[i].decl.name] = L.b.param_read(uint32_t(i));
  const uint32_t loss = L.expr(*tr.loss, top);
  if (L.predictions.size() != 1)
    throw MspecError("E-TRAIN-002", tr.loss->line, tr.loss->col,
                     "the loss calls `model.forward` " + std::to_string(L.predictions.size()) + " time(s), not once");
  if (L.b.prog.node(loss).ty.rank() != 0)
    throw MspecError("E-TYPE-001", tr.loss->line, tr.loss->col, "the loss is " + type_string(L.b.prog.node(loss).ty) + ", not a scalar");
  const uint32_t prediction = L.predictions[0];

  // The data of a run, read off the loss and the declarations.
  TrainConfig c;
  c.name = name;
  c.steps = uint64_t(tr.steps);
  c.seed = uint64_t(tr.seed);
  const Node& ln = L.b.prog.node(loss);
  auto data_named = [&](uint32_t v) -> std::string {
    for (auto& [d, _] : tr.data)
      if (top.values.at(d.name) == v) return d.name;
    return "";
  };
  auto decl = [&](const std::string& n) -> const Decl* {
    for (auto& [d, _] : tr.data)
      if (d.name == n) return &d;
    return nullptr;
  };
  auto refuse = [&](const std::string& what) { throw MspecError("E-TRAIN-002", tr.loss->line, tr.loss->col, what); };
  if (ln.op == Op::Mse) {
    const std::string x = [&] {
      for (auto& [d, target] : tr.data)
        if (!target && d.ty.dtype == DType::F32) return d.name;
      return std::string();
    }();
    std::string y = data_named(ln.operands[1]);
    if (y.empty()) y = data_named(ln.operands[0]);
    if (x.empty() || y.empty())
      refuse("`mse` trains on teacher data: an f32 input, and a target as an operand of `mse`");
    c.feed = FeedKind::Teacher;
    c.x = x;
    c.y = y;
  } else if (ln.op == Op::CrossEntropy) {
    const std::string labels = data_named(ln.operands[1]), weights = data_named(ln.operands[2]);
    if (labels.empty() || weights.empty() || ln.operands[0] != prediction)
      refuse("`cross_entropy(model.forward(...), labels, weights)` takes its labels and weights from targets");
    const Type& logits = L.b.prog.node(prediction).ty;
    c.labels = labels;
    c.weights = weights;
    c.vocab = logits.shape[1];
    const Decl* ids = decl("ids");
    if (ids && ids->ty.dtype == DType::I32) {
      const Decl* km = decl("key_mask");
      const Decl* pos = decl("positions");
      if (!km || km->ty.rank() != 2 || !pos)
        refuse("a token program declares `ids`, `positions` and a `key_mask` of [B, S]");
      c.feed = FeedKind::MaskedLm;
      c.batch = km->ty.shape[0];
      c.seq = km->ty.shape[1];
      c.first_token = 5;
      c.ids = "ids";
      c.positions = "positions";
      c.key_mask = "key_mask";
      const uint64_t rows = uint64_t(c.batch * c.seq);
      c.masked_rows = masked_rows_override >= 0 ? uint64_t(masked_rows_override) : default_masked_rows(rows, 0.15);
    } else {
      std::string x;
      for (auto& [d, target] : tr.data)
        if (!target && d.ty.dtype == DType::F32 && d.ty.rank() == 2) x = d.name;
      if (x.empty()) refuse("a classifier declares an f32 input of [B, features]");
      c.feed = FeedKind::Classifier;
      c.x = x;
      c.batch = decl(x)->ty.shape[0];
      c.features = decl(x)->ty.shape[1];
      c.classes = c.vocab;
    }
  } else {
    refuse("the subset trains `mse` and `cross_entropy` losses");
  }

  // optimizer = sgd(lr = ..) | adamw(lr = .., weight_decay, beta1, beta2, eps, warmup_steps)
  const Expr& opt = *tr.optimizer;
  if (opt.kind != Expr::Call) throw MspecError("E-SYNTAX-001", opt.line, opt.col, "expected `sgd(...)` or `adamw(...)`");
  std::map<std::string, double> kw;
  for (auto& a : opt.args) {
    if (a.name.empty() || !a.value || a.value->kind != Expr::Number)
      throw MspecError("E-TYPE-001", opt.line, opt.col, "optimizer settings are named numbers");
    kw[a.name] = a.value->number;
  }
  auto take = [&](const std::string& k, double dflt, bool required) {
    auto it = kw.find(k);
    if (it == kw.end()) {
      if (required) throw MspecError("E-TYPE-001", opt.line, opt.col, "`" + opt.text + "` needs `" + k + "`");
      return dflt;
    }
    const double v = it->second;
    kw.erase(it);
    return v;
  };
  Rule rule;
  float lr;
  AdamWConfig a;
  if (opt.text == "sgd") {
    rule = Rule::Sgd;
    lr = float(take("lr", 0, true));
    if (!(lr > 0.0f) || !std::isfinite(lr)) throw MspecError("E-TYPE-001", opt.line, opt.col, "`lr` is a positive number");
  } else if (opt.text == "adamw") {
    // Every argument named once (types.rs:53-62).
    rule = Rule::AdamW;
    lr = float(take("lr", 0, true));
    a.weight_decay = float(take("weight_decay", 0, true));
    a.beta1 = float(take("beta1", 0, true));
    a.beta2 = float(take("beta2", 0, true));
    a.eps = float(take("eps", 0, true));
    const double warmup = take("warmup_steps", 0, true);
    if (!(a.weight_decay >= 0.0f) || !(a.beta1 >= 0.0f && a.beta1 < 1.0f) || !(a.beta2 >= 0.0f && a.beta2 < 1.0f) ||
        !(a.eps > 0.0f) || !std::isfinite(a.eps))
      throw MspecError("E-TYPE-001", opt.line, opt.col, "`adamw` settings out of range");
    if (warmup < 0 || warmup != std::floor(warmup) || warmup >= double(tr.steps))
      throw MspecError("E-TYPE-001", opt.line, opt.col, "`warmup_steps` is a whole number below `steps`");
    a.warmup_steps = uint64_t(warmup);
  } else {
    throw MspecError("E-NAME-001", opt.line, opt.col, "unknown optimizer `" + opt.text + "`");
  }
  if (!kw.empty()) throw MspecError("E-TYPE-001", opt.line, opt.col, "`" + opt.text + "` takes no `" + kw.begin()->first + "`");

  Compiled out = compile_lowered(c, L.b.finish(), loss, prediction, rule, lr, a);
  apply_steps_override(out, steps_override);
  return out;
}

}  // namespace msx
