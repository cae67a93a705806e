// TEST INFRASTRUCTURE — the CPU oracle interpreter. See interp.h.
#include "interp.h"

#include <cmath>
#include <cstring>

#include "../modelspec_amd/csrc/host/rng.h"

namespace oracle {
using msx::DType;
using msx::IrError;
using msx::Node;
using msx::Op;

namespace {
[[noreturn]] void fail(const std::string& what) { throw IrError(what); }

// sum of iteration order from the first term, +0 for none (interpreter.rs:1894-1900).
template <class F>
float seq_sum(size_t n, F term) {
  if (n == 0) return 0.0f;
  float acc = term(0);
  for (size_t k = 1; k < n; ++k) acc = acc + term(k);
  return acc;
}

// sum_of_products: the first product rounded, every later fused (interpreter.rs:1528-1537).
template <class F>
float sum_of_products(size_t n, F pair) {
  if (n == 0) return 0.0f;
  auto [a, b] = pair(0);
  float acc = a * b;
  for (size_t k = 1; k < n; ++k) {
    auto [x, y] = pair(k);
    acc = std::fmaf(x, y, acc);
  }
  return acc;
}

template <class F>
double sum_of_products_f64(size_t n, F pair) {
  if (n == 0) return 0.0;
  auto [a, b] = pair(0);
  double acc = a * b;
  for (size_t k = 1; k < n; ++k) {
    auto [x, y] = pair(k);
    acc = std::fma(x, y, acc);
  }
  return acc;
}

double wide_sum(const float* v, size_t n) {
  if (n == 0) return 0.0;
  double acc = double(v[0]);
  for (size_t k = 1; k < n; ++k) acc = acc + double(v[k]);
  return acc;
}

inline float relu_where(float a, float g) { return a > 0.0f ? g : 0.0f; }

// GELU constants: the nearest f32 to sqrt(2/pi) and 0.044715 (interpreter.rs:1539-1556).
const float kGeluScale = float(0.7978845608028654);
const float kGeluCubic = float(0.044715);

inline float gelu_twice_inner(float x) {
  float two = 2.0f;
  return two * kGeluScale * (x + kGeluCubic * x * x * x);
}
inline float logistic(float v) { return 1.0f / (1.0f + std::exp(0.0f - v)); }
inline float gelu(float x) { return x * logistic(gelu_twice_inner(x)); }
inline float gelu_grad(float x, float g) {
  float v = gelu_twice_inner(x);
  float s = logistic(v), r = logistic(0.0f - v);
  float slope = kGeluScale * (1.0f + 3.0f * kGeluCubic * x * x);
  return (s + 2.0f * (s * x) * r * slope) * g;
}

// row_moments (interpreter.rs:1513-1526).
inline void row_moments(const float* row, size_t h, float& mean, float& rstd) {
  float width = float(h);
  mean = seq_sum(h, [&](size_t j) { return row[j]; }) / width;
  float m = mean;
  float var = sum_of_products(h, [&](size_t j) { return std::pair<float, float>(row[j] - m, row[j] - m); }) / width;
  rstd = 1.0f / std::sqrt(var + 1e-12f);
}

// matmul: i, k, j loop, the k = 0 products first, every later k fused (matmul.rs:263-290).
// `at` reads the left operand transposed in place, exact either way. The AVX2 build of the loop
// rounds each lane as the scalar fmaf does (cpu/matmul.rs:1-17), so both give the same bits.
template <int>
inline void matmul_loop(float* out, const float* a, bool at, const float* b, size_t m, size_t k, size_t n) {
  for (size_t i = 0; i < m; ++i) {
    float* row = out + i * n;
    float x = at ? a[i] : a[i * k];
    for (size_t j = 0; j < n; ++j) row[j] = x * b[j];
    for (size_t p = 1; p < k; ++p) {
      float xp = at ? a[p * m + i] : a[i * k + p];
      const float* br = b + p * n;
      for (size_t j = 0; j < n; ++j) row[j] = __builtin_fmaf(xp, br[j], row[j]);
    }
  }
}
__attribute__((target("avx2,fma"))) void matmul_avx2(float* out, const float* a, bool at, const float* b, size_t m,
                                                     size_t k, size_t n) {
  matmul_loop<1>(out, a, at, b, m, k, n);
}
void matmul_portable(float* out, const float* a, bool at, const float* b, size_t m, size_t k, size_t n) {
  matmul_loop<0>(out, a, at, b, m, k, n);
}
void matmul(float* out, const float* a, bool at, const float* b, size_t m, size_t k, size_t n) {
  static const bool avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  if (avx2) matmul_avx2(out, a, at, b, m, k, n);
  else matmul_portable(out, a, at, b, m, k, n);
}

// The attention operands of one node (interpreter.rs:1300-1510), key mask form.
struct Attend {
  const float *q, *k, *v, *mask;
  size_t rows, key_rows, h, heads, d, s, l;
  float scale;
  size_t key_start(size_t i) const { return i / l * s; }
  bool unmasked(size_t j) const { return mask[j] != 0.0f; }
  float score(size_t i, size_t j, size_t head) const {
    const float* qi = q + i * h + head * d;
    const float* kj = k + j * h + head * d;
    return sum_of_products(d, [&](size_t c) { return std::pair<float, float>(qi[c], kj[c]); }) * scale;
  }
  void softmax(size_t i, size_t head, float& max, float& total) const {
    size_t st = key_start(i);
    bool first = true;
    for (size_t j = st; j < st + s; ++j) {
      if (!unmasked(j)) continue;
      float x = score(i, j, head);
      if (first) { max = x; first = false; }
      else if (x > max) max = x;
    }
    first = true;
    for (size_t j = st; j < st + s; ++j) {
      if (!unmasked(j)) continue;
      float e = std::exp(score(i, j, head) - max);
      total = first ? e : total + e;
      first = false;
    }
  }
  float probability(size_t i, size_t j, size_t head, float max, float total) const {
    return std::exp(score(i, j, head) - max) / total;
  }
  float probability_grad(size_t i, size_t j, size_t head, const float* g) const {
    const float* gi = g + i * h + head * d;
    const float* vj = v + j * h + head * d;
    return sum_of_products(d, [&](size_t c) { return std::pair<float, float>(gi[c], vj[c]); });
  }
  float row_dot(size_t i, size_t head, float max, float total, const float* g) const {
    size_t st = key_start(i);
    bool first = true;
    float acc = 0.0f;
    for (size_t j = st; j < st + s; ++j) {
      if (!unmasked(j)) continue;
      float p = probability(i, j, head, max, total);
      float dp = probability_grad(i, j, head, g);
      acc = first ? p * dp : std::fmaf(p, dp, acc);
      first = false;
    }
    return acc;
  }
};

inline float fused(bool first, float a, float b, float acc) { return first ? a * b : std::fmaf(a, b, acc); }

void row_softmax(const float* row, size_t v, float& max, float& total) {
  max = row[0];
  for (size_t c = 1; c < v; ++c)
    if (row[c] > max) max = row[c];
  float m = max;
  total = seq_sum(v, [&](size_t c) { return std::exp(row[c] - m); });
}
}  // namespace

Interpreter::Interpreter(const msx::Program& p, bool has_seed, uint64_t seed) : p_(p), has_seed_(has_seed), seed_(seed) {
  vals_.resize(p.nodes.size());
  // Only the values an output depends on are evaluated; the others cannot change an output.
  needed_.assign(p.nodes.size(), false);
  for (auto o : p.outputs) needed_[p.pos.at(o)] = true;
  for (size_t k = p.nodes.size(); k-- > 0;)
    if (needed_[k])
      for (auto o : p.nodes[k].operands) needed_[p.pos.at(o)] = true;
}

const std::vector<float>& Interpreter::value(uint32_t id) const { return vals_.at(p_.pos.at(id)).f; }

const Tensor& Interpreter::arg(size_t at, size_t k) const { return vals_[p_.pos.at(p_.nodes[at].operands[k])]; }

void Interpreter::run(const std::map<std::string, std::vector<float>>& f32,
                      const std::map<std::string, std::vector<int32_t>>& i32,
                      const std::vector<std::vector<float>>& params) {
  for (size_t at = 0; at < p_.nodes.size(); ++at)
    if (needed_[at]) eval(at, f32, i32, params);
}

void Interpreter::eval(size_t at, const std::map<std::string, std::vector<float>>& f32,
                       const std::map<std::string, std::vector<int32_t>>& i32,
                       const std::vector<std::vector<float>>& params) {
  const Node& n = p_.nodes[at];
  Tensor& out = vals_[at];
  out.ty = n.ty;
  const size_t count = size_t(n.ty.count());
  auto& o = out.f;
  auto A = [&](size_t k) -> const std::vector<float>& { return arg(at, k).f; };
  auto T = [&](size_t k) -> const msx::Type& { return arg(at, k).ty; };
  auto ids = [&](size_t k) -> const std::vector<int32_t>& { return arg(at, k).i; };

  switch (n.op) {
    case Op::Input: {
      if (n.ty.dtype == DType::I32) {
        auto it = i32.find(n.name);
        if (it == i32.end()) fail("missing i32 input `" + n.name + "`");
        if (it->second.size() != count) fail("input `" + n.name + "` has the wrong element count");
        out.i = it->second;
      } else {
        auto it = f32.find(n.name);
        if (it == f32.end()) fail("missing input `" + n.name + "`");
        if (it->second.size() != count) fail("input `" + n.name + "` has the wrong element count");
        o = it->second;
      }
      return;
    }
    case Op::ParamRead:
      o = params.at(n.param);
      if (o.size() != count) fail("parameter has the wrong element count");
      return;
    case Op::Scalar: o = {n.scalar}; return;
    case Op::Add: case Op::Sub: case Op::Mul: case Op::Div: {
      const auto &a = A(0), &b = A(1);
      o.resize(count);
      auto f = [&](float x, float y) {
        switch (n.op) {
          case Op::Add: return x + y;
          case Op::Sub: return x - y;
          case Op::Mul: return x * y;
          default: return x / y;
        }
      };
      if (T(0).shape == T(1).shape) for (size_t i = 0; i < count; ++i) o[i] = f(a[i], b[i]);
      else if (T(1).rank() == 0) for (size_t i = 0; i < count; ++i) o[i] = f(a[i], b[0]);
      else for (size_t i = 0; i < count; ++i) o[i] = f(a[0], b[i]);
      return;
    }
    case Op::MatMul: {
      // A `Transpose` operand is read in place (interpreter.rs:1877-1900): same bits as a copy.
      const Node& lhs = p_.node(n.operands[0]);
      bool at_t = lhs.op == Op::Transpose;
      const Tensor& a = at_t ? vals_[p_.pos.at(lhs.operands[0])] : arg(at, 0);
      if (at_t && a.f.empty()) fail("in-place transpose source is not evaluated");
      size_t m = size_t(n.ty.shape[0]), nn = size_t(n.ty.shape[1]), k = size_t(T(1).shape[0]);
      o.resize(count);
      if (k == 0) { std::fill(o.begin(), o.end(), 0.0f); return; }
      matmul(o.data(), a.f.data(), at_t, A(1).data(), m, k, nn);
      return;
    }
    case Op::Relu: { const auto& a = A(0); o.resize(count); for (size_t i = 0; i < count; ++i) o[i] = relu_where(a[i], a[i]); return; }
    case Op::Transpose: {
      const auto& a = A(0);
      size_t m = size_t(T(0).shape[0]), nn = size_t(T(0).shape[1]);
      o.resize(count);
      for (size_t j = 0; j < nn; ++j)
        for (size_t i = 0; i < m; ++i) o[j * m + i] = a[i * nn + j];
      return;
    }
    case Op::ReduceSum: o = {float(wide_sum(A(0).data(), A(0).size()))}; return;
    case Op::ReduceMean: o = {float(wide_sum(A(0).data(), A(0).size()) / double(A(0).size()))}; return;
    case Op::Mse: {
      const auto &a = A(0), &b = A(1);
      double s = sum_of_products_f64(a.size(), [&](size_t i) {
        double d = double(a[i]) - double(b[i]);
        return std::pair<double, double>(d, d);
      });
      o = {float(s / double(a.size()))};
      return;
    }
    case Op::ReluGrad: { const auto &a = A(0), &g = A(1); o.resize(count); for (size_t i = 0; i < count; ++i) o[i] = relu_where(a[i], g[i]); return; }
    case Op::BroadcastScalar: o.assign(count, A(0)[0]); return;
    case Op::Embedding: {
      const auto& table = A(0);
      const auto& id = ids(1);
      size_t h = size_t(T(0).shape[1]), rows = size_t(T(0).shape[0]);
      o.resize(count);
      for (size_t r = 0; r < id.size(); ++r) {
        if (id[r] < 0 || size_t(id[r]) >= rows) fail("E-DATA-011: id " + std::to_string(id[r]) + " at " + std::to_string(r) + " is outside the table");
        std::memcpy(&o[r * h], &table[size_t(id[r]) * h], h * sizeof(float));
      }
      return;
    }
    case Op::EmbeddingGrad: {
      const auto& id = ids(0);
      const auto& g = A(1);
      size_t h = size_t(T(1).shape[1]);
      o.assign(count, 0.0f);
      for (size_t k = 0; k < id.size(); ++k) {
        if (id[k] < 0 || id[k] >= n.rows) fail("E-DATA-011: id out of range");
        float* row = &o[size_t(id[k]) * h];
        for (size_t c = 0; c < h; ++c) row[c] = row[c] + g[k * h + c];
      }
      return;
    }
    case Op::AddRows: {
      const auto &x = A(0), &b = A(1);
      size_t h = b.size();
      o.resize(count);
      for (size_t i = 0; i < count; ++i) o[i] = x[i] + b[i % h];
      return;
    }
    case Op::SumRows: {
      const auto& g = A(0);
      size_t h = count, rows = size_t(T(0).shape[0]);
      if (rows == 0) { o.assign(h, 0.0f); return; }
      o.assign(g.begin(), g.begin() + long(h));
      for (size_t r = 1; r < rows; ++r)
        for (size_t c = 0; c < h; ++c) o[c] = o[c] + g[r * h + c];
      return;
    }
    case Op::Gelu: { const auto& a = A(0); o.resize(count); for (size_t i = 0; i < count; ++i) o[i] = gelu(a[i]); return; }
    case Op::GeluGrad: { const auto &a = A(0), &g = A(1); o.resize(count); for (size_t i = 0; i < count; ++i) o[i] = gelu_grad(a[i], g[i]); return; }
    case Op::LayerNorm: {
      const auto &x = A(0), &gamma = A(1), &beta = A(2);
      size_t h = gamma.size(), rows = count / h;
      o.resize(count);
      for (size_t r = 0; r < rows; ++r) {
        const float* row = &x[r * h];
        float mean, rstd;
        row_moments(row, h, mean, rstd);
        for (size_t j = 0; j < h; ++j) o[r * h + j] = (row[j] - mean) * rstd * gamma[j] + beta[j];
      }
      return;
    }
    case Op::LayerNormGradX: {
      const auto &x = A(0), &gamma = A(1), &g = A(2);
      size_t h = gamma.size(), rows = count / h;
      float width = float(h);
      o.resize(count);
      for (size_t r = 0; r < rows; ++r) {
        const float* row = &x[r * h];
        const float* gr = &g[r * h];
        float mean, rstd;
        row_moments(row, h, mean, rstd);
        auto xhat = [&](size_t j) { return (row[j] - mean) * rstd; };
        auto gx = [&](size_t j) { return gr[j] * gamma[j]; };
        float mean_gx = seq_sum(h, gx) / width;
        float mean_gx_xhat = sum_of_products(h, [&](size_t j) { return std::pair<float, float>(gx(j), xhat(j)); }) / width;
        for (size_t j = 0; j < h; ++j) o[r * h + j] = rstd * ((gx(j) - mean_gx) - xhat(j) * mean_gx_xhat);
      }
      return;
    }
    case Op::LayerNormGradGamma: {
      const auto &x = A(0), &g = A(1);
      size_t h = count, rows = size_t(T(0).shape[0]);
      o.assign(h, 0.0f);
      for (size_t r = 0; r < rows; ++r) {
        const float* row = &x[r * h];
        float mean, rstd;
        row_moments(row, h, mean, rstd);
        for (size_t j = 0; j < h; ++j) {
          float xhat = (row[j] - mean) * rstd;
          o[j] = r == 0 ? g[r * h + j] * xhat : std::fmaf(g[r * h + j], xhat, o[j]);
        }
      }
      return;
    }
    case Op::Softmax: {
      const auto& x = A(0);
      size_t k = size_t(T(0).shape[1]), rows = count / k;
      o.resize(count);
      for (size_t r = 0; r < rows; ++r) {
        const float* row = &x[r * k];
        float max = row[0];
        for (size_t c = 1; c < k; ++c) if (row[c] > max) max = row[c];
        for (size_t c = 0; c < k; ++c) o[r * k + c] = std::exp(row[c] - max);
        float total = seq_sum(k, [&](size_t c) { return o[r * k + c]; });
        for (size_t c = 0; c < k; ++c) o[r * k + c] = o[r * k + c] / total;
      }
      return;
    }
    case Op::SoftmaxGrad: {
      const auto &y = A(0), &g = A(1);
      size_t k = size_t(T(0).shape[1]), rows = count / k;
      o.resize(count);
      for (size_t r = 0; r < rows; ++r) {
        float d = sum_of_products(k, [&](size_t c) { return std::pair<float, float>(g[r * k + c], y[r * k + c]); });
        for (size_t c = 0; c < k; ++c) o[r * k + c] = y[r * k + c] * (g[r * k + c] - d);
      }
      return;
    }
    case Op::Attention: case Op::AttentionGradQ: case Op::AttentionGradK: case Op::AttentionGradV: {
      if (T(3).dtype != DType::F32) fail("attention spans are not supported by this oracle");
      Attend at_{};
      at_.q = A(0).data(); at_.k = A(1).data(); at_.v = A(2).data(); at_.mask = A(3).data();
      at_.rows = size_t(T(0).shape[0]); at_.key_rows = size_t(T(1).shape[0]); at_.h = size_t(T(0).shape[1]);
      at_.heads = size_t(n.heads); at_.d = at_.h / at_.heads;
      at_.s = size_t(T(3).shape[1]); at_.l = at_.rows / size_t(T(3).shape[0]);
      at_.scale = 1.0f / std::sqrt(float(at_.d));
      // check_key_mask (interpreter.rs:1240-1262)
      for (size_t b = 0; b < size_t(T(3).shape[0]); ++b) {
        bool any = false;
        for (size_t j = 0; j < at_.s; ++j) {
          float m = at_.mask[b * at_.s + j];
          if (m != 0.0f && m != 1.0f) fail("key mask value is neither 0 nor 1");
          any = any || m == 1.0f;
        }
        if (!any) fail("a sequence has no unmasked key");
      }
      const float* g = n.op == Op::Attention ? nullptr : A(4).data();
      o.assign(count, 0.0f);
      const size_t h = at_.h, d = at_.d, s = at_.s;
      for (size_t i = 0; i < at_.rows; ++i) {
        size_t st = at_.key_start(i);
        bool first_query = i % at_.l == 0;
        for (size_t head = 0; head < at_.heads; ++head) {
          float max = 0, total = 0;
          at_.softmax(i, head, max, total);
          size_t c0 = head * d;
          if (n.op == Op::Attention) {
            bool first = true;
            for (size_t j = st; j < st + s; ++j) {
              if (!at_.unmasked(j)) continue;
              float p = at_.probability(i, j, head, max, total);
              for (size_t c = c0; c < c0 + d; ++c) o[i * h + c] = fused(first, p, at_.v[j * h + c], o[i * h + c]);
              first = false;
            }
          } else if (n.op == Op::AttentionGradQ) {
            float dd = at_.row_dot(i, head, max, total, g);
            bool first = true;
            for (size_t j = st; j < st + s; ++j) {
              if (!at_.unmasked(j)) continue;
              float p = at_.probability(i, j, head, max, total);
              float ds = p * (at_.probability_grad(i, j, head, g) - dd);
              for (size_t c = c0; c < c0 + d; ++c) o[i * h + c] = fused(first, ds, at_.k[j * h + c], o[i * h + c]);
              first = false;
            }
            for (size_t c = c0; c < c0 + d; ++c) o[i * h + c] = o[i * h + c] * at_.scale;
          } else if (n.op == Op::AttentionGradK) {
            float dd = at_.row_dot(i, head, max, total, g);
            for (size_t j = st; j < st + s; ++j) {
              if (!at_.unmasked(j)) continue;
              float p = at_.probability(i, j, head, max, total);
              float ds = p * (at_.probability_grad(i, j, head, g) - dd);
              for (size_t c = c0; c < c0 + d; ++c) o[j * h + c] = fused(first_query, ds, at_.q[i * h + c], o[j * h + c]);
            }
          } else {
            for (size_t j = st; j < st + s; ++j) {
              if (!at_.unmasked(j)) continue;
              float p = at_.probability(i, j, head, max, total);
              for (size_t c = c0; c < c0 + d; ++c) o[j * h + c] = fused(first_query, p, g[i * h + c], o[j * h + c]);
            }
          }
        }
      }
      if (n.op == Op::AttentionGradK)
        for (size_t j = 0; j < at_.key_rows; ++j)
          if (at_.unmasked(j))
            for (size_t c = 0; c < h; ++c) o[j * h + c] = o[j * h + c] * at_.scale;
      return;
    }
    case Op::CrossEntropy: case Op::CrossEntropyGrad: {
      const auto& logits = A(0);
      const auto& labels = ids(1);
      const auto& w = A(2);
      size_t v = size_t(T(0).shape[1]), rows = size_t(T(0).shape[0]);
      // check_loss_rows (interpreter.rs:1146-1175)
      for (size_t r = 0; r < rows; ++r) {
        if (labels[r] < 0 || size_t(labels[r]) >= v) fail("E-DATA-011: label out of range");
        if (!(w[r] * 0.0f == 0.0f) || w[r] < 0.0f) fail("a loss weight is negative or not finite");
      }
      if (n.op == Op::CrossEntropy) {
        std::vector<double> losses(rows);
        for (size_t r = 0; r < rows; ++r) {
          float max, total;
          row_softmax(&logits[r * v], v, max, total);
          losses[r] = double(max + std::log(total) - logits[r * v + size_t(labels[r])]);
        }
        double num = sum_of_products_f64(rows, [&](size_t r) { return std::pair<double, double>(double(w[r]), losses[r]); });
        double den = wide_sum(w.data(), rows);
        o = {den == 0.0 ? 0.0f : float(num / den)};
      } else {
        float g = A(3)[0];
        float den = float(wide_sum(w.data(), rows));
        o.assign(count, 0.0f);
        if (den == 0.0f) return;
        for (size_t r = 0; r < rows; ++r) {
          float max, total;
          const float* row = &logits[r * v];
          row_softmax(row, v, max, total);
          float scale = g * w[r] / den;
          for (size_t c = 0; c < v; ++c) {
            float target = c == size_t(labels[r]) ? 1.0f : 0.0f;
            o[r * v + c] = scale * (std::exp(row[c] - max) / total - target);
          }
        }
      }
      return;
    }
    case Op::Dropout: case Op::DropoutGrad: {
      if (!has_seed_) fail("dropout without a seed");
      const auto& tok = ids(size_t(msx::token_operand(n.op)));
      const auto& x = A(n.op == Op::Dropout ? 0 : 1);
      if (count > (size_t(1) << 32)) fail("dropout over more than 2^32 elements");
      int32_t t[2] = {tok[0], tok[1]};
      uint64_t id = msx::token_id(t);
      float scale = 1.0f / (1.0f - n.scalar);
      o.resize(count);
      for (size_t i = 0; i < count; ++i) o[i] = msx::dropout_keeps(seed_, id, uint32_t(i), n.scalar) ? x[i] * scale : 0.0f;
      return;
    }
    case Op::StopGradient: o = A(0); return;
    case Op::Sqrt: { const auto& a = A(0); o.resize(count); for (size_t i = 0; i < count; ++i) o[i] = std::sqrt(a[i]); return; }
    case Op::Count_: break;
  }
  fail(std::string("the oracle has no rule for ") + msx::op_name(n.op));
}

float row_nll(const float* row, size_t v, size_t label) {
  float max, total;
  row_softmax(row, v, max, total);
  return max + std::log(total) - row[label];
}

int64_t first_argmax(const float* row, size_t v) {
  for (size_t c = 0; c < v; ++c)
    if (std::isnan(row[c])) return -1;
  size_t best = 0;
  for (size_t c = 1; c < v; ++c)
    if (row[c] > row[best]) best = c;
  return int64_t(best);
}

bool HeldOutTally::add(const float* logits, const int32_t* labels, const float* weights, size_t rows, size_t v) {
  for (size_t n = 0; n < rows; ++n)
    if (labels[n] < 0 || size_t(labels[n]) >= v) return false;
  for (size_t n = 0; n < rows; ++n) {
    const float* row = logits + n * v;
    const double wide = double(weights[n]), nll = double(row_nll(row, v, size_t(labels[n])));
    numerator = started ? std::fma(wide, nll, numerator) : wide * nll;
    denominator = started ? denominator + wide : wide;
    started = true;
    if (weights[n] > 0.0f) {
      ++selected;
      if (first_argmax(row, v) == int64_t(labels[n])) ++correct;
    }
  }
  return true;
}

float HeldOutTally::loss() const { return denominator == 0.0 ? 0.0f : float(numerator / denominator); }
float HeldOutTally::accuracy() const { return selected == 0 ? 0.0f : float(correct) / float(selected); }

}  // namespace oracle
