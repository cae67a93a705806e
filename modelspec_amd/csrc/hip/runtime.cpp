// The HIP device runtime. See runtime.h.
#include "runtime.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <array>
#include <map>
#include <memory>
#include <mutex>
#include <set>

// The device memory of Session::held_out_static: the row results [rows, 2] of at most
// kStaticEvalRows rows, then the HeldOutState at the next 256-byte boundary (512 KiB + 256 bytes).
// Each device holds its own copy until the process ends. In host code `scratch` names a host-side
// stand-in, so its device address is looked up once per device (static_scratch) and only that
// address is used.
static constexpr size_t kStaticStateAt = size_t(msx::Session::kStaticEvalRows) * 8;
static constexpr size_t kStaticScratchBytes = kStaticStateAt + 256;
static __device__ __align__(256) char scratch[kStaticScratchBytes];

namespace msx {

namespace {
// One entry per device: the address of its copy of `scratch`, and the mutex that a call holds for
// as long as it uses that copy, so calls on one device from several threads run one at a time.
struct StaticScratch {
  void* ptr = nullptr;
  std::mutex use;
};
std::mutex g_scratch_mu;
std::map<int, std::unique_ptr<StaticScratch>> g_scratch_at;

// The scratch entry of `device`. Its address is looked up on first use with that device current;
// the caller's current device is restored afterwards.
StaticScratch& static_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch_at.find(device);
  if (it != g_scratch_at.end()) return *it->second;
  int current = -1;
  hip_check(hipGetDevice(&current), "hipGetDevice (static scratch)");
  if (current != device) hip_check(hipSetDevice(device), "hipSetDevice (static scratch)");
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (current != device) hip_check(hipSetDevice(current), "hipSetDevice (restore)");
  hip_check(e, "hipGetSymbolAddress (static scratch)");
  if (!ptr) throw HipError("hipGetSymbolAddress (static scratch): no address");
  auto entry = std::make_unique<StaticScratch>();
  entry->ptr = ptr;
  return *(g_scratch_at[device] = std::move(entry));
}
}  // namespace

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw HipError(std::string(what) + ": " + hipGetErrorString(e));
}

DeviceArena::~DeviceArena() {
  if (base_) (void)hipFree(base_);
}

void* DeviceArena::reserve(size_t bytes) {
  size_t at = size_;
  size_ += (std::max<size_t>(bytes, 4) + 255) / 256 * 256;
  return reinterpret_cast<void*>(at + 1);  // a token: offset + 1, never null
}

void DeviceArena::commit() {
  if (base_) throw HipError("arena committed twice");
  if (size_ == 0) size_ = 256;
  hip_check(hipMalloc(&base_, size_), "hipMalloc (plan arena)");
  hip_check(hipMemset(base_, 0, size_), "hipMemset (plan arena)");
}

void* DeviceArena::at(void* token) const {
  if (!base_) throw HipError("arena used before commit");
  return base_ + (reinterpret_cast<size_t>(token) - 1);
}

namespace {
bool is_moment_input(const std::string& name) { return name.rfind("optimizer.m@", 0) == 0 || name.rfind("optimizer.v@", 0) == 0; }

// A MatMul operand with its Transpose chain folded: the source value and whether it is read
// transposed.
struct Resolved { uint32_t src; bool flip; };
Resolved resolve(const Program& p, uint32_t v) {
  bool flip = false;
  while (p.node(v).op == Op::Transpose) {
    flip = !flip;
    v = p.node(v).operands[0];
  }
  return {v, flip};
}
}  // namespace

// ---------------------------------------------------------------------------------------------
Executor::Executor(Session& s, const Program& p, bool is_step) : s_(s), p_(p), is_step_(is_step) {
  build();
  if (s_.opt_.plan_only) return;
  for (int i = 0; i < kRing; ++i) {
    hip_check(hipHostMalloc(&pinned_[i], std::max<size_t>(input_bytes_, 256), hipHostMallocDefault), "hipHostMalloc");
    hip_check(hipEventCreateWithFlags(&slot_done_[i], hipEventDisableTiming), "hipEventCreate");
  }
}

Executor::~Executor() {
  for (int i = 0; i < kRing; ++i) {
    if (slot_done_[i]) (void)hipEventDestroy(slot_done_[i]);
    if (pinned_[i]) (void)hipHostFree(pinned_[i]);
  }
}

void* Executor::ptr(uint32_t id) const {
  auto f = fixed_.find(id);
  if (f != fixed_.end()) return f->second;
  auto t = token_.find(id);
  if (t != token_.end()) return arena_.at(t->second);
  throw IrError("value %" + std::to_string(id) + " has no device storage");
}

const void* Executor::value(uint32_t id) const { return ptr(id); }

_Float16* Executor::ptr16(uint32_t id) const {
  auto f = fixed16_.find(id);
  if (f != fixed16_.end()) return f->second;
  auto t = token16_.find(id);
  if (t != token16_.end()) return static_cast<_Float16*>(arena_.at(t->second));
  return nullptr;
}

void Executor::build() {
  const Program& p = p_;
  const size_t n = p.nodes.size();
  const TrainingStep& st = s_.step_;

  // --- which nodes run ----------------------------------------------------------------------
  std::set<uint32_t> optimizer;  // nodes the fused optimizer launch computes
  std::vector<uint32_t> roots(p.outputs.begin(), p.outputs.end());
  if (is_step_) {
    std::set<uint32_t> state_outputs;
    for (auto& [param, u] : st.updates) state_outputs.insert(u);
    for (auto& [param, m] : st.moments) { state_outputs.insert(m.m_next); state_outputs.insert(m.v_next); }
    // Match the optimizer's per-parameter template (ir/training.rs:737-980) node by node.
    auto nd = [&](uint32_t v) -> const Node& { return p.node(v); };
    auto expect = [&](uint32_t v, Op op, size_t arity) -> const Node& {
      const Node& x = nd(v);
      if (x.op != op || x.operands.size() != arity)
        throw IrError(std::string("the optimizer subgraph is not the AdamW/SGD template at %") + std::to_string(v));
      optimizer.insert(v);
      return x;
    };
    auto scalar_is = [&](uint32_t v, float want) {
      const Node& x = nd(v);
      if (x.op != Op::Scalar || std::memcmp(&x.scalar, &want, 4) != 0)
        throw IrError("an optimizer constant differs from the step's hyperparameters");
      optimizer.insert(v);
    };
    if (st.rule == Rule::AdamW) {
      float k[6];
      st.adamw.constants(k);
      for (auto& [param, u] : st.updates) {
        uint32_t g = st.gradients.at(param);
        const Moments& mo = st.moments.at(param);
        uint32_t pr = 0;
        for (auto& x : p.nodes)
          if (x.op == Op::ParamRead && x.param == param) { pr = x.id; break; }
        const Node& sub = expect(u, Op::Sub, 2);
        if (sub.operands[0] != pr) throw IrError("AdamW update does not read the parameter");
        const Node& scaled = expect(sub.operands[1], Op::Mul, 2);
        if (scaled.operands[0] != *st.lr_t) throw IrError("AdamW step is not scaled by lr_t");
        const Node& stp = expect(scaled.operands[1], Op::Add, 2);
        const Node& dir = expect(stp.operands[0], Op::Div, 2);
        const Node& shrink = expect(stp.operands[1], Op::Mul, 2);
        scalar_is(shrink.operands[0], k[5]);
        if (shrink.operands[1] != pr) throw IrError("AdamW decay does not read the parameter");
        const Node& mhat = expect(dir.operands[0], Op::Mul, 2);
        const Node& den = expect(dir.operands[1], Op::Add, 2);
        scalar_is(den.operands[1], k[4]);
        const Node& root = expect(den.operands[0], Op::Sqrt, 1);
        const Node& vhat = expect(root.operands[0], Op::Mul, 2);
        if (mhat.operands[0] != mo.m_next || mhat.operands[1] != *st.c1) throw IrError("AdamW m_hat");
        if (vhat.operands[0] != mo.v_next || vhat.operands[1] != *st.c2) throw IrError("AdamW v_hat");
        const Node& mn = expect(mo.m_next, Op::Add, 2);
        const Node& dm = expect(mn.operands[0], Op::Mul, 2);
        const Node& nm = expect(mn.operands[1], Op::Mul, 2);
        scalar_is(dm.operands[0], k[0]);
        scalar_is(nm.operands[0], k[1]);
        if (dm.operands[1] != mo.m || nm.operands[1] != g) throw IrError("AdamW first moment");
        const Node& vn = expect(mo.v_next, Op::Add, 2);
        const Node& dv = expect(vn.operands[0], Op::Mul, 2);
        const Node& nv = expect(vn.operands[1], Op::Mul, 2);
        scalar_is(dv.operands[0], k[2]);
        if (dv.operands[1] != mo.v || nv.operands[1] != g) throw IrError("AdamW second moment");
        const Node& sg = expect(nv.operands[0], Op::Mul, 2);
        scalar_is(sg.operands[0], k[3]);
        if (sg.operands[1] != g) throw IrError("AdamW scaled gradient");
      }
    } else {
      for (auto& [param, u] : st.updates) {
        const Node& sub = expect(u, Op::Sub, 2);
        const Node& scaled = expect(sub.operands[1], Op::Mul, 2);
        scalar_is(scaled.operands[0], st.lr);
        if (scaled.operands[1] != st.gradients.at(param)) throw IrError("SGD update does not read the gradient");
      }
    }
  }
  std::vector<bool> need(n, false);
  for (auto o : roots) need[p.pos.at(o)] = true;
  for (size_t k = n; k-- > 0;)
    if (need[k])
      for (auto o : p.nodes[k].operands) need[p.pos.at(o)] = true;

  std::vector<std::vector<size_t>> consumers(n);
  for (size_t k = 0; k < n; ++k)
    if (need[k])
      for (auto o : p.nodes[k].operands) consumers[p.pos.at(o)].push_back(k);
  std::set<uint32_t> outputs(p.outputs.begin(), p.outputs.end());

  // --- fusions ------------------------------------------------------------------------------
  // Transposes read in place by every consumer: MatMuls read through them, and a Transpose of one
  // is computed from the source.
  std::set<uint32_t> folded;
  std::set<uint32_t> mm_fused;   // MatMuls whose one consumer AddRows takes them as a biased GEMM
  for (size_t k = 0; k < n; ++k) {
    if (!need[k]) continue;
    const Node& x = p.nodes[k];
    if (x.op == Op::Transpose && !outputs.count(x.id) && !consumers[k].empty()) {
      bool all_mm = true;
      for (auto c : consumers[k]) all_mm = all_mm && (p.nodes[c].op == Op::MatMul || p.nodes[c].op == Op::Transpose);
      if (all_mm) folded.insert(x.id);
    }
    if (x.op == Op::MatMul && !outputs.count(x.id) && consumers[k].size() == 1) {
      const Node& c = p.nodes[consumers[k][0]];
      if (c.op == Op::AddRows && c.operands[0] == x.id && c.operands[1] != x.id) mm_fused.insert(x.id);
    }
  }
  // A MatMul read only by a Transpose that nothing reads through (no MatMul or Transpose reader)
  // is computed transposed, as B^T A^T, straight into the Transpose's value.
  std::map<uint32_t, uint32_t> mm_transposed;  // MatMul -> Transpose
  for (size_t k = 0; k < n; ++k) {
    const Node& x = p.nodes[k];
    if (!need[k] || x.op != Op::MatMul || outputs.count(x.id) || mm_fused.count(x.id) || consumers[k].size() != 1) continue;
    const Node& t = p.nodes[consumers[k][0]];
    if (t.op != Op::Transpose || folded.count(t.id)) continue;
    bool through = false;
    for (auto c : consumers[p.pos.at(t.id)]) through = through || p.nodes[c].op == Op::MatMul || p.nodes[c].op == Op::Transpose;
    if (!through) mm_transposed[x.id] = t.id;
  }
  std::set<uint32_t> transposed_out;
  for (auto [m, t] : mm_transposed) transposed_out.insert(t);
  // A SumRows of a MatMul's un-transposed B operand (the bias gradient beside its weight gradient)
  // is taken by that GEMM from its LDS tiles, when no reader of the sum comes before the GEMM.
  // Under mixed precision only the f16 GEMM on the operands' f16 copies (k_gemm_lds16) takes the
  // sums (of the f16 values): both operands' rows whole 16-byte groups of f16, K a multiple of 32.
  std::map<uint32_t, uint32_t> colsum_of;  // MatMul -> SumRows
  std::set<uint32_t> colsum_fused;
  const bool mixed_twins = s_.opt_.mixed && !s_.opt_.fuse_ce_head;
  auto sums_fit = [&](const Node& m) {
    if (!s_.opt_.mixed) return true;
    if (!mixed_twins || optimizer.count(m.id)) return false;
    const Resolved ra = resolve(p, m.operands[0]), rb = resolve(p, m.operands[1]);
    const auto &sa = p.node(ra.src).ty.shape, &sb = p.node(rb.src).ty.shape;
    const int64_t k = p.node(m.operands[0]).ty.shape[1];
    return sa.size() == 2 && sb.size() == 2 && sa[1] % 8 == 0 && sb[1] % 8 == 0 && k % 32 == 0;
  };
  for (size_t k = 0; k < n; ++k) {
    if (!need[k] || p.nodes[k].op != Op::SumRows) continue;
    const uint32_t a = p.nodes[k].operands[0];
    for (auto c : consumers[p.pos.at(a)]) {
      const Node& m = p.nodes[c];
      if (m.op != Op::MatMul || mm_fused.count(m.id) || colsum_of.count(m.id) || !sums_fit(m)) continue;
      Resolved rb = resolve(p, m.operands[1]);
      if (rb.src != a || rb.flip) continue;
      bool late = true;
      for (auto r2 : consumers[k]) late = late && r2 > c;
      if (!late) continue;
      colsum_of[m.id] = p.nodes[k].id;
      colsum_fused.insert(p.nodes[k].id);
      break;
    }
  }
  // Add(X, EmbeddingGrad) with the EmbeddingGrad read only there and X computed before it: the
  // scatter writes X + its result straight into the Add's value.
  std::map<uint32_t, std::pair<uint32_t, uint32_t>> eg_add;  // EmbeddingGrad -> (Add, X)
  std::set<uint32_t> eg_add_nodes;
  for (size_t k = 0; k < n; ++k) {
    const Node& x = p.nodes[k];
    if (!need[k] || x.op != Op::EmbeddingGrad || outputs.count(x.id) || consumers[k].size() != 1) continue;
    const Node& a = p.nodes[consumers[k][0]];
    if (a.op != Op::Add || a.operands[0] == a.operands[1]) continue;
    const uint32_t other = a.operands[0] == x.id ? a.operands[1] : a.operands[0];
    if (p.node(other).ty.shape != x.ty.shape || p.pos.at(other) > k) continue;
    eg_add[x.id] = {a.id, other};
    eg_add_nodes.insert(a.id);
  }
  std::set<uint32_t> grad_values_pre;  // values the optimizer reads as gradients
  if (is_step_)
    for (auto& pg : st.gradients) grad_values_pre.insert(pg.second);
  // GEMM epilogues. A GEMM's value (an unswapped MatMul, or the AddRows taking one as a biased
  // GEMM) that is read only by Add(X, value) with X computed earlier, or only as the incoming
  // gradient of GeluGrad/ReluGrad, is not materialized: the GEMM writes the consumer's value. A
  // Gelu/Relu of a GEMM's value is written by the GEMM beside the value itself.
  // consumer, hk::GemmAct, addend or pre-activation; `drop`: a DropoutGrad of the Add consumer (its
  // only reader) whose value the GEMM writes instead, the Add then not materialized.
  struct Epi { uint32_t node; int act; int64_t aux; int64_t drop = -1; };
  std::map<uint32_t, Epi> gemm_epi;                     // GEMM value -> consumer it writes
  std::set<uint32_t> epi_nodes;                         // consumers written by their GEMM
  std::set<uint32_t> epi_unstored;                      // epilogue values never materialized
  // Where a value is written: a fused writer's position when it runs before the value's own node.
  std::map<uint32_t, size_t> written_at;
  for (auto& [eg, add] : eg_add) written_at[add.first] = p.pos.at(eg);
  auto ready = [&](uint32_t v) { return written_at.count(v) ? written_at.at(v) : p.pos.at(v); };
  for (size_t k = 0; k < n; ++k) {
    const Node& x = p.nodes[k];
    if (!need[k] || outputs.count(x.id)) continue;
    const bool gemm_value = (x.op == Op::MatMul && !mm_fused.count(x.id) && !mm_transposed.count(x.id) &&
                             !colsum_of.count(x.id)) ||
                            (x.op == Op::AddRows && mm_fused.count(x.operands[0]));
    if (!gemm_value) continue;
    std::vector<size_t> cs = consumers[k];
    if (cs.size() == 1) {
      const Node& c = p.nodes[cs[0]];
      if (c.op == Op::Add && !eg_add_nodes.count(c.id) && c.operands[0] != c.operands[1] && !epi_nodes.count(c.id)) {
        const uint32_t other = c.operands[0] == x.id ? c.operands[1] : c.operands[0];
        if (ready(other) < k && p.node(other).ty.shape == x.ty.shape) {
          gemm_epi[x.id] = {c.id, hk::EPI_NONE, int64_t(other)};
          epi_nodes.insert(c.id);
          written_at[c.id] = k;
          const std::vector<size_t>& dc = consumers[cs[0]];
          if (dc.size() == 1 && !outputs.count(c.id) && !grad_values_pre.count(c.id)) {
            const Node& d = p.nodes[dc[0]];
            if (d.op == Op::DropoutGrad && d.operands[1] == c.id && d.ty.count() == c.ty.count() && c.ty.rank() == 2) {
              gemm_epi[x.id].drop = d.id;
              epi_nodes.insert(d.id);
              written_at[d.id] = k;
              epi_unstored.insert(c.id);
            }
          }
          continue;
        }
      }
      if ((c.op == Op::GeluGrad || c.op == Op::ReluGrad) && c.operands[1] == x.id && c.operands[0] != x.id &&
          ready(c.operands[0]) < k) {
        gemm_epi[x.id] = {c.id, c.op == Op::GeluGrad ? hk::EPI_GELU_GRAD : hk::EPI_RELU_GRAD, int64_t(c.operands[0])};
        epi_nodes.insert(c.id);
        written_at[c.id] = k;
        continue;
      }
    }
    for (auto c : cs) {
      const Node& cn = p.nodes[c];
      if ((cn.op == Op::Gelu || cn.op == Op::Relu) && !epi_nodes.count(cn.id)) {
        gemm_epi[x.id] = {cn.id, cn.op == Op::Gelu ? hk::EPI_GELU : hk::EPI_RELU, -1};
        epi_nodes.insert(cn.id);
        written_at[cn.id] = k;
        break;
      }
    }
  }
  // A LayerNorm with its neighbours in one pass: its input X = Add(A, B) (B possibly a Dropout read
  // only there, not materialized) written beside the normalized value, and a Dropout that is the
  // LayerNorm output's only reader applied on the way out (the output then not materialized).
  struct LnFused { int64_t add = -1, a = -1, b = -1, din = -1, dout = -1, gather = -1, ea = -1, eb = -1; };
  std::map<uint32_t, LnFused> ln_fused;  // LayerNorm -> parts
  std::set<uint32_t> ln_fused_nodes;     // the Add and Dropouts a fused LayerNorm writes or applies
  std::set<uint32_t> ln_skip_storage;    // values of those never materialized
  for (size_t k = 0; k < n; ++k) {
    const Node& y = p.nodes[k];
    if (!need[k] || y.op != Op::LayerNorm) continue;
    LnFused f;
    uint32_t xv = y.operands[0];
    // X is written at the LayerNorm: no reader may run earlier (a GEMM epilogue reading it runs at
    // its GEMM).
    auto later_readers = [&](uint32_t v) {
      bool ok = true;
      for (auto c : consumers[p.pos.at(v)]) ok = ok && (c == k || c > k) && !epi_nodes.count(p.nodes[c].id);
      return ok;
    };
    bool later = later_readers(xv);
    // LayerNorm(Embedding(Add(..), ids)) with the Add read only by that gather: the pass sums the
    // gathered rows only.
    if (p.node(xv).op == Op::Embedding && later && !outputs.count(p.node(xv).operands[0])) {
      const uint32_t tv = p.node(xv).operands[0];
      const Node& tn = p.node(tv);
      if (tn.op == Op::Add && consumers[p.pos.at(tv)].size() == 1 && !epi_nodes.count(tv) && !eg_add_nodes.count(tv) &&
          tn.ty.rank() == 2 && tn.ty.shape[1] == y.ty.shape[1]) {
        f.gather = xv;
        xv = tv;
        later = true;
      }
    }
    const Node& xn = p.node(xv);
    if (xn.op == Op::Add && xn.operands[0] != xn.operands[1] && later && !epi_nodes.count(xv) && !eg_add_nodes.count(xv) &&
        xn.ty.shape[1] == y.ty.shape[1]) {
      f.add = xv;
      f.a = xn.operands[0];
      f.b = xn.operands[1];
      for (int side = 1; side >= 0; --side) {
        const uint32_t d = xn.operands[size_t(side)];
        const Node& dn = p.node(d);
        if (dn.op == Op::Dropout && consumers[p.pos.at(d)].size() == 1 && !outputs.count(d)) {
          f.din = d;
          f.b = dn.operands[0];
          f.a = xn.operands[size_t(1 - side)];
          break;
        }
      }
    }
    // Add(Embedding(T, ids), Embedding(U, ids2)) summed by this pass: the pass gathers the table
    // rows itself and the Embedding outputs, read only by the Add, are never formed.
    if (f.add >= 0 && f.din < 0 && f.gather < 0) {
      for (int side = 0; side < 2; ++side) {
        const uint32_t e = uint32_t(side == 0 ? f.a : f.b);
        const Node& en = p.node(e);
        if (en.op != Op::Embedding || consumers[p.pos.at(e)].size() != 1 || outputs.count(e) || f.a == f.b) continue;
        const Node& tn = p.node(en.operands[0]);
        if (tn.ty.rank() != 2 || tn.ty.shape[1] != y.ty.shape[1] || p.node(en.operands[1]).ty.count() != y.ty.shape[0])
          continue;
        (side == 0 ? f.ea : f.eb) = e;
      }
    }
    if (consumers[k].size() == 1 && !outputs.count(y.id)) {
      const Node& d = p.nodes[consumers[k][0]];
      if (d.op == Op::Dropout && d.operands[0] == y.id) f.dout = d.id;
    }
    if (f.gather >= 0 && f.add < 0) f.gather = -1;
    if (f.add < 0 && f.dout < 0) continue;
    ln_fused[y.id] = f;
    for (auto v : {f.add, f.din, f.dout, f.gather, f.ea, f.eb})
      if (v >= 0) ln_fused_nodes.insert(uint32_t(v));
    for (auto v : {f.ea, f.eb})
      if (v >= 0) ln_skip_storage.insert(uint32_t(v));
    if (f.din >= 0) ln_skip_storage.insert(uint32_t(f.din));
    if (f.gather >= 0) ln_skip_storage.insert(uint32_t(f.add));  // only the gathered rows are formed
    if (f.dout >= 0) ln_skip_storage.insert(y.id);
  }
  // The LayerNorm gradients of one (input, output gradient) pair run as one pass: dx, and block
  // partials of the gamma and beta sums, finished by a batched column reduction, deferred to the
  // end of the step when only the optimizer reads them. The pass runs at its first member.
  struct LnGroup {
    int64_t dx = -1, gamma = -1, beta = -1, gm = -1;
    size_t first = SIZE_MAX;
    int64_t post = -1, aux = -1;  // a DropoutGrad / GeluGrad / ReluGrad of dx the pass writes; token or input
    int kind = 0;                 // hk::LnbPost
    bool keep_dx = true;          // dx has readers besides the post
  };
  std::map<std::pair<uint32_t, uint32_t>, LnGroup> ln_groups;
  for (size_t k = 0; k < n; ++k) {
    if (!need[k]) continue;
    const Node& x = p.nodes[k];
    if (x.op == Op::LayerNormGradX) {
      auto& gr = ln_groups[{x.operands[0], x.operands[2]}];
      gr.dx = x.id;
      gr.gm = x.operands[1];
      gr.first = std::min(gr.first, k);
    } else if (x.op == Op::LayerNormGradGamma) {
      auto& gr = ln_groups[{x.operands[0], x.operands[1]}];
      gr.gamma = x.id;
      gr.first = std::min(gr.first, k);
    }
  }
  // The dropout or activation gradient of dx written by the same pass.
  std::set<uint32_t> ln_post_nodes;
  for (auto& [key, gr] : ln_groups) {
    if (gr.dx < 0) continue;
    const size_t dk = p.pos.at(uint32_t(gr.dx));
    for (auto c : consumers[dk]) {
      const Node& cn = p.nodes[c];
      if (epi_nodes.count(cn.id) || ln_fused_nodes.count(cn.id) || cn.operands[1] != uint32_t(gr.dx)) continue;
      if (cn.op == Op::DropoutGrad && cn.operands[0] != uint32_t(gr.dx)) {
        gr.post = cn.id; gr.kind = hk::LNB_DROPOUT; gr.aux = cn.operands[0];
      } else if ((cn.op == Op::GeluGrad || cn.op == Op::ReluGrad) && cn.operands[0] != uint32_t(gr.dx) &&
                 p.pos.at(cn.operands[0]) < gr.first) {
        gr.post = cn.id; gr.kind = cn.op == Op::GeluGrad ? hk::LNB_GELU_GRAD : hk::LNB_RELU_GRAD; gr.aux = cn.operands[0];
      } else {
        continue;
      }
      ln_post_nodes.insert(cn.id);
      gr.keep_dx = consumers[dk].size() > 1 || outputs.count(uint32_t(gr.dx)) || grad_values_pre.count(uint32_t(gr.dx));
      if (!gr.keep_dx) ln_skip_storage.insert(uint32_t(gr.dx));
      break;
    }
  }
  std::map<uint32_t, std::pair<uint32_t, uint32_t>> ln_member;  // member -> group key
  for (auto& [key, gr] : ln_groups) {
    for (auto v : {gr.dx, gr.gamma})
      if (v >= 0) ln_member[uint32_t(v)] = key;
  }
  for (size_t k = 0; k < n; ++k) {
    if (!need[k] || p.nodes[k].op != Op::SumRows || colsum_fused.count(p.nodes[k].id)) continue;
    for (auto& [key, gr] : ln_groups) {
      if (key.second != p.nodes[k].operands[0] || gr.beta >= 0) continue;
      gr.beta = p.nodes[k].id;
      gr.first = std::min(gr.first, k);
      ln_member[p.nodes[k].id] = key;
      break;
    }
  }
  // (Program outputs are read after the last launch, so they do not hold a reduction back.)
  auto only_optimizer_reads = [&](int64_t v) {
    if (v < 0) return true;
    for (auto c : consumers[p.pos.at(uint32_t(v))])
      if (!optimizer.count(p.nodes[c].id)) return false;
    return true;
  };
  // Attention gradients over the same operands run as one launch.
  std::map<std::vector<uint32_t>, std::array<int64_t, 3>> attn_groups;
  for (size_t k = 0; k < n; ++k) {
    if (!need[k]) continue;
    const Node& x = p.nodes[k];
    int slot = x.op == Op::AttentionGradQ ? 0 : x.op == Op::AttentionGradK ? 1 : x.op == Op::AttentionGradV ? 2 : -1;
    if (slot < 0) continue;
    auto key = x.operands;
    key.push_back(uint32_t(x.heads));
    auto it = attn_groups.find(key);
    if (it == attn_groups.end()) it = attn_groups.emplace(key, std::array<int64_t, 3>{-1, -1, -1}).first;
    it->second[size_t(slot)] = int64_t(x.id);
  }

  // Cross-entropy nodes over the same (logits, labels, weights): the loss and the gradient.
  struct CeGroup { int64_t loss = -1, grad = -1; bool done = false, grad_done = false; };
  std::map<std::array<uint32_t, 3>, CeGroup> ce_groups;
  for (size_t k = 0; k < n; ++k) {
    const Node& x = p.nodes[k];
    if (!need[k] || (x.op != Op::CrossEntropy && x.op != Op::CrossEntropyGrad)) continue;
    auto& grp = ce_groups[{x.operands[0], x.operands[1], x.operands[2]}];
    if (x.op == Op::CrossEntropy && grp.loss < 0) grp.loss = x.id;
    if (x.op == Op::CrossEntropyGrad && grp.grad < 0) grp.grad = x.id;
  }
  // Row pitch: a wide 2-D value whose rows are not a whole number of float4 groups gets its rows
  // padded to 64 floats when its producer and every reader take a leading dimension (GEMMs, the
  // cross-entropy kernels), so that GEMMs load it with aligned float4s.
  std::set<uint32_t> grad_values;
  if (is_step_)
    for (auto& pg : st.gradients) grad_values.insert(pg.second);
  std::map<uint32_t, int64_t> pitch;
  for (size_t k = 0; k < n; ++k) {
    const Node& x = p.nodes[k];
    if (!need[k] || x.ty.rank() != 2 || x.ty.dtype != DType::F32 || outputs.count(x.id) || grad_values.count(x.id)) continue;
    const int64_t rows = x.ty.shape[0], cols = x.ty.shape[1];
    if (cols % 4 == 0 || rows * cols < (int64_t(1) << 16)) continue;
    const bool producer = (x.op == Op::AddRows && mm_fused.count(x.operands[0])) ||
                          (x.op == Op::MatMul && !mm_fused.count(x.id) && !mm_transposed.count(x.id)) ||
                          x.op == Op::CrossEntropyGrad;
    if (!producer) continue;
    bool readers = true;
    for (auto c : consumers[k]) {
      const Node& cn = p.nodes[c];
      if (cn.op == Op::CrossEntropy || cn.op == Op::CrossEntropyGrad) {
        readers = readers && cn.operands[0] == x.id && cn.operands[1] != x.id && cn.operands[2] != x.id;
      } else if (cn.op == Op::MatMul) {
      } else if (cn.op == Op::Transpose && folded.count(cn.id)) {
        for (auto c2 : consumers[c]) readers = readers && p.nodes[c2].op == Op::MatMul;
      } else if (cn.op == Op::SumRows && (colsum_fused.count(cn.id) || !ln_member.count(cn.id))) {
        // taken by its GEMM, or its own column-sum launch, which reads rows at a pitch
      } else {
        readers = false;
      }
    }
    if (readers) pitch[x.id] = (cols + 63) / 64 * 64;
  }
  // The cross-entropy kernels walk the logits and their gradient with one pitch: both padded or
  // neither (the gradient stays unpadded when a reader of it takes no leading dimension).
  for (size_t k = 0; k < n; ++k) {
    const Node& x = p.nodes[k];
    if (!need[k] || x.op != Op::CrossEntropyGrad) continue;
    if (pitch.count(x.id) != pitch.count(x.operands[0])) {
      pitch.erase(x.id);
      pitch.erase(x.operands[0]);
    }
  }
  auto ld_of = [&](uint32_t v) {
    auto it = pitch.find(v);
    return it != pitch.end() ? it->second : p.node(v).ty.shape.back();
  };

  // Cross-entropy fused into its decoder head: when the logits come from one GEMM (with or
  // without its bias) that nothing else follows, and the loss gradient is read only by GEMMs (and
  // their fused column sums), the forward GEMM leaves each row's column-tile partials of max and
  // sum of exp, one launch finishes the rows (statistics, loss terms, gradient entries), and the
  // GEMMs that read the gradient form it from the logits as they load them: the gradient is never
  // stored, and no separate pass reads the logits.
  struct CeHead {
    uint32_t logits, labels, weights, grad, seed;
    int64_t loss, rows, cols, tiles;
    size_t emit_at;  // the node position its rows launch takes
    void* part = nullptr;
    void* tab = nullptr;
    bool done = false;
  };
  std::map<uint32_t, CeHead> ce_head;         // logits value -> its head
  std::map<uint32_t, uint32_t> ce_head_grad;  // gradient value -> its logits
  // Off by default: on BERT-tiny (one MI355X) the gradient formed at load costs the two backward
  // GEMMs 20-24 us each (each element of it is loaded, and its exp taken, by two tiles) and the
  // forward's partials 12 us, more than the 54 us row pass it replaces (0.917 against 0.900 ms a
  // step). SessionOptions::fuse_ce_head turns it on.
  if (s_.opt_.fuse_ce_head) {
    for (auto& [key, grp] : ce_groups) {
      if (grp.grad < 0) continue;
      const uint32_t lg = key[0];
      const Node& lx = p.node(lg);
      const uint32_t gv = uint32_t(grp.grad);
      if (lx.ty.rank() != 2 || outputs.count(lg) || grad_values.count(lg) || outputs.count(gv) || grad_values.count(gv))
        continue;
      // The producer: a MatMul, alone or with its bias (AddRows), written as itself.
      const bool with_bias = lx.op == Op::AddRows && mm_fused.count(lx.operands[0]);
      const uint32_t mm = with_bias ? lx.operands[0] : lg;
      if (!with_bias && (lx.op != Op::MatMul || mm_fused.count(lg))) continue;
      if (mm_transposed.count(mm) || (gemm_epi.count(lg) && gemm_epi.at(lg).node != lg)) continue;
      const int64_t rows = lx.ty.shape[0], cols = lx.ty.shape[1];
      if (ld_of(lg) % 4 != 0 || pitch.count(lg) != pitch.count(gv)) continue;
      const uint32_t seed = p.node(gv).operands[3];
      bool ok = true;
      for (auto c : consumers[p.pos.at(lg)]) {
        const Node& cn = p.nodes[c];
        ok = ok && (cn.op == Op::CrossEntropy || cn.op == Op::CrossEntropyGrad) && cn.operands[0] == lg &&
             cn.operands[1] == key[1] && cn.operands[2] == key[2];
      }
      auto gemm_reader = [&](uint32_t c) {
        const Node& cn = p.nodes[c];
        return cn.op == Op::MatMul && cn.operands[0] != cn.operands[1];
      };
      for (auto c : consumers[p.pos.at(gv)]) {
        const Node& cn = p.nodes[c];
        if (gemm_reader(c)) continue;
        if (cn.op == Op::Transpose && folded.count(cn.id)) {
          for (auto c2 : consumers[c]) ok = ok && gemm_reader(c2);
          continue;
        }
        ok = ok && cn.op == Op::SumRows && colsum_fused.count(cn.id);
      }
      // The rows' launch goes where the group's first node is, or, when the upstream gradient is
      // computed inside the step, at the gradient node (its operand exists there), provided
      // nothing reads the loss before that.
      const size_t at_grad = p.pos.at(gv);
      size_t emit_at = grp.loss >= 0 ? std::min(at_grad, p.pos.at(uint32_t(grp.loss))) : at_grad;
      const Op seed_op = p.node(seed).op;
      if (seed_op != Op::Scalar && seed_op != Op::Input && p.pos.at(seed) > emit_at) {
        emit_at = at_grad;
        for (auto c : consumers[p.pos.at(uint32_t(grp.loss))]) ok = ok && c > at_grad;
      }
      if (!ok) continue;
      const int64_t K = p.node(p.node(mm).operands[0]).ty.shape[1];
      const int64_t tn = hk::gemm_tile_n(rows, cols, K, false, s_.opt_.mixed);
      ce_head[lg] = CeHead{lg, key[1], key[2], gv, seed, grp.loss, rows, cols, (cols + tn - 1) / tn, emit_at};
      ce_head_grad[gv] = lg;
    }
  }

  // Elementwise chains (the reference's elementwise fusion groups, spirv kernel "Sub>Mul@0"): a
  // binary elementwise value read only by a binary elementwise op with a rank-0 other operand is
  // computed inside that op's launch, y = (a op1 b) op2 s, and never stored.
  struct EwChain { uint32_t inner; int op1, op2; bool inner_left; };
  std::map<uint32_t, EwChain> ew_chain;  // outer value -> its inner op
  std::set<uint32_t> ew_inner;           // inner values so computed
  auto ew_code = [](Op op) {
    return op == Op::Add ? hk::EW_ADD : op == Op::Sub ? hk::EW_SUB : op == Op::Mul ? hk::EW_MUL : hk::EW_DIV;
  };
  auto binary_ew = [](Op op) { return op == Op::Add || op == Op::Sub || op == Op::Mul || op == Op::Div; };
  for (size_t k = 0; k < n; ++k) {
    const Node& x = p.nodes[k];
    if (!need[k] || !binary_ew(x.op) || optimizer.count(x.id) || x.ty.rank() == 0 || outputs.count(x.id) ||
        grad_values.count(x.id) || consumers[k].size() != 1)
      continue;
    if (eg_add_nodes.count(x.id) || epi_nodes.count(x.id) || ln_fused_nodes.count(x.id) || ln_post_nodes.count(x.id))
      continue;
    const Node& a = p.node(x.operands[0]);
    const Node& b = p.node(x.operands[1]);
    if (a.ty.count() != x.ty.count() || b.ty.count() != x.ty.count()) continue;  // no broadcast inside
    const Node& y = p.nodes[consumers[k][0]];
    if (!binary_ew(y.op) || optimizer.count(y.id) || y.ty.count() != x.ty.count() || ew_inner.count(y.id)) continue;
    if (eg_add_nodes.count(y.id) || epi_nodes.count(y.id) || ln_fused_nodes.count(y.id) || ln_post_nodes.count(y.id))
      continue;
    const bool left = y.operands[0] == x.id;
    const uint32_t other = left ? y.operands[1] : y.operands[0];
    if (other == x.id || p.node(other).ty.rank() != 0) continue;
    ew_chain[y.id] = EwChain{x.id, ew_code(x.op), ew_code(y.op), left};
    ew_inner.insert(x.id);
  }
  // Rank-0 arithmetic on constants is folded once, in f32 as the kernel would round it (the
  // reference folds the mse gradient's 1.0 * 0.25 the same way); the loss-scaled seed is not a
  // constant and is never folded.
  std::set<uint32_t> folded_scalar;

  // Mixed precision: every value a GEMM reads as an operand gets an f16 copy in HBM, which the
  // f16 GEMM (k_gemm_lds16) reads straight into LDS: a GEMM output's copy is written by the GEMM's
  // epilogue, a LayerNorm's (forward or backward) by the LayerNorm pass, a parameter's by the
  // optimizer launch (and every upload); other producers (attention, cross-entropy) are followed by
  // a rounding pass. The f32 values stay for the kernels that read them in f32.
  // The f16 attention (flash16) reads its operands' copies the same way: q, k, v and the output
  // gradient.
  std::set<uint32_t> gemm_operands;
  auto flash = [&](const Node& x) {
    if (!s_.opt_.mixed || s_.opt_.fuse_ce_head) return false;
    if (x.op != Op::Attention && x.op != Op::AttentionGradQ && x.op != Op::AttentionGradK && x.op != Op::AttentionGradV)
      return false;
    const auto& ms = p.node(x.operands[3]).ty;
    if (ms.dtype != DType::F32 || ms.rank() != 2 || x.heads <= 0) return false;
    const int64_t B = ms.shape[0], S = ms.shape[1], L = p.node(x.operands[0]).ty.shape[0] / B;
    const int64_t H = p.node(x.operands[0]).ty.shape[1];
    return H % x.heads == 0 && hk::flash16_fits(L, S, H / x.heads);
  };
  if (s_.opt_.mixed && !s_.opt_.fuse_ce_head)
    for (size_t k = 0; k < n; ++k) {
      const Node& x = p.nodes[k];
      if (!need[k] || optimizer.count(x.id)) continue;
      if (x.op == Op::MatMul)
        for (int side = 0; side < 2; ++side) gemm_operands.insert(resolve(p, x.operands[size_t(side)]).src);
      if (flash(x)) {
        for (int side = 0; side < 3; ++side) gemm_operands.insert(x.operands[size_t(side)]);
        if (x.op != Op::Attention) gemm_operands.insert(x.operands[4]);
        else gemm_operands.insert(x.id);  // the output's f16 copy: the backward's d_i reads it
      }
    }
  // A fused LayerNorm's second addend produced by a GEMM (the sublayer output, before its input
  // dropout) is read from its f16 copy, as an f16 forward would hold it (rows of 256 .. 1024).
  std::map<uint32_t, uint32_t> ln_b16;  // LayerNorm -> the addend it reads as f16
  if (s_.opt_.mixed && !s_.opt_.fuse_ce_head)
    for (auto& [lid, f] : ln_fused) {
      if (f.add < 0 || f.b < 0 || f.gather >= 0 || f.ea >= 0 || f.eb >= 0) continue;
      const Node& bn = p.node(uint32_t(f.b));
      const int64_t h = p.node(lid).ty.shape[1];
      if ((bn.op != Op::MatMul && bn.op != Op::AddRows) || bn.ty.rank() != 2 || bn.ty.dtype != DType::F32 ||
          h % 256 != 0 || h > 1024)
        continue;
      gemm_operands.insert(uint32_t(f.b));
      ln_b16[lid] = uint32_t(f.b);
    }

  // --- storage ------------------------------------------------------------------------------
  std::map<uint32_t, float> constants;
  for (size_t k = 0; k < n; ++k) {
    if (!need[k]) continue;
    const Node& x = p.nodes[k];
    if (optimizer.count(x.id) && x.op != Op::Scalar) continue;
    switch (x.op) {
      case Op::Input:
        if (is_moment_input(x.name)) {
          // optimizer.<m|v>@<path>: the moment arena slice of that parameter.
          std::string path = x.name.substr(12);
          uint32_t param = UINT32_MAX;
          for (size_t q = 0; q < p.params.size(); ++q)
            if (p.params[q].path == path) param = uint32_t(q);
          if (param == UINT32_MAX) throw IrError("moment input of an unknown parameter: " + x.name);
          fixed_[x.id] = (x.name[10] == 'm' ? s_.m_ : s_.v_) + s_.offset_[param];
        } else {
          inputs_.push_back(InputSlot{x.name, x.ty.dtype, x.ty.count(), 0, x.id, s_.corpus_fed(p, x.name)});
        }
        break;
      case Op::ParamRead:
        fixed_[x.id] = s_.param_ + s_.offset_[x.param];
        if (gemm_operands.count(x.id) && s_.param16_) fixed16_[x.id] = s_.param16_ + s_.offset_[x.param];
        break;
      case Op::Scalar:
        // Under loss scaling the loss gradient's seed (the Scalar 1.0 of the loss subgraph) is
        // the device's current loss scale.
        if (is_step_ && s_.scaler_ && x.scalar == 1.0f && st.subgraphs.count(x.id) &&
            st.subgraphs.at(x.id) == Subgraph::Loss) {
          fixed_[x.id] = &s_.scaler_->scale;
          break;
        }
        token_[x.id] = arena_.reserve(4);
        constants[x.id] = x.scalar;
        break;
      case Op::Add: case Op::Sub: case Op::Mul: case Op::Div:
        if (x.ty.rank() == 0 && constants.count(x.operands[0]) && constants.count(x.operands[1]) &&
            !optimizer.count(x.id)) {
          const float a = constants.at(x.operands[0]), b = constants.at(x.operands[1]);
          const volatile float r = x.op == Op::Add ? a + b : x.op == Op::Sub ? a - b : x.op == Op::Mul ? a * b : a / b;
          token_[x.id] = arena_.reserve(4);
          constants[x.id] = r;
          folded_scalar.insert(x.id);
          break;
        }
        if (ew_inner.count(x.id)) break;  // computed inside its consumer's launch
        [[fallthrough]];
      default:
        if (folded.count(x.id) || mm_fused.count(x.id) || mm_transposed.count(x.id) || eg_add.count(x.id)) break;
        if (gemm_epi.count(x.id) && gemm_epi.at(x.id).act != hk::EPI_GELU && gemm_epi.at(x.id).act != hk::EPI_RELU) break;
        if (ln_skip_storage.count(x.id) || ce_head_grad.count(x.id) || epi_unstored.count(x.id)) break;
        token_[x.id] = arena_.reserve(size_t(pitch.count(x.id) ? x.ty.shape[0] * pitch.at(x.id) : x.ty.count()) * 4);
        break;
    }
  }
  // Gradients the optimizer reads live in the gradient arena at their parameter's offset.
  std::vector<std::pair<uint32_t, uint32_t>> grad_copies;  // (value, param)
  if (is_step_) {
    std::set<uint32_t> claimed;
    for (auto& [param, g] : st.gradients) {
      const Node& x = p.node(g);
      bool own = token_.count(g) && !claimed.count(g) && x.op != Op::Scalar;
      if (own) {
        token_.erase(g);
        fixed_[g] = s_.grad_ + s_.offset_[param];
        claimed.insert(g);
      } else {
        grad_copies.push_back({g, param});
      }
    }
  }
  // The input block: the corpus draw of the step first (when a packed corpus feeds the batch),
  // then every input the host stages, then the inputs the device writes, so that one copy of the
  // block's head carries a step's host inputs.
  auto slot_bytes = [](int64_t count) { return (size_t(std::max<int64_t>(count, 1)) * 4 + 255) / 256 * 256; };
  input_bytes_ = 0;
  if (s_.corpus_) {
    draw_offset_ = 0;
    input_bytes_ += slot_bytes(3 + int64_t(s_.corpus_batch_));
  }
  for (int device_pass = 0; device_pass < 2; ++device_pass) {
    for (auto& slot : inputs_)
      if (slot.device == (device_pass == 1)) {
        slot.offset = input_bytes_;
        input_bytes_ += slot_bytes(slot.count);
      }
    if (device_pass == 0) {
      // The plans of EmbeddingGrads whose ids the host stages: made on the host beside the inputs
      // (the ids are in host memory before the step), so the step holds no plan launch.
      plan_slots_.clear();
      for (size_t k = 0; k < n && is_step_; ++k) {
        const Node& x = p.nodes[k];
        if (!need[k] || x.op != Op::EmbeddingGrad || optimizer.count(x.id)) continue;
        const Node& ids = p.node(x.operands[0]);
        const int64_t nn = ids.ty.shape[0], rows = x.rows;
        if (ids.op != Op::Input || ids.ty.dtype != DType::I32 || !hk::eg_sorted_fits(nn, rows)) continue;
        bool host = false;
        for (auto& slot : inputs_) host = host || (slot.id == ids.id && !slot.device);
        bool have = false;
        for (auto& ps : plan_slots_) have = have || (ps.ids == ids.id && ps.rows == rows);
        if (!host || have) continue;
        plan_slots_.push_back({ids.name, ids.id, int32_t(nn), int32_t(rows), input_bytes_});
        input_bytes_ += slot_bytes(int64_t(hk::eg_plan_bytes(nn, rows) / 4));
      }
      host_bytes_ = input_bytes_;
    }
  }
  input_token_ = arena_.reserve(std::max<size_t>(input_bytes_, 256));

  // Workspaces, reserved per launch now; resolved after commit.
  // A GEMM of the plan as the grouping pass sees it: its arguments (pointers resolved at launch)
  // and the values it reads and writes.
  struct GemmJob {
    hk::GemmArgs g;
    uint32_t asrc = 0, bsrc = 0, out_id = 0, id = 0;
    int64_t bias_id = -1, cs_id = -1;
    Epi epi;
    void* ws = nullptr;
    void* ce_part = nullptr;  // a cross-entropy head: the forward's row partials
    void* ce_tab = nullptr;   // or the gradient entries of the operand formed from logits
    uint32_t drop_tok = 0;    // the DropoutGrad epilogue's token, threshold and scale
    uint64_t drop_thr = 0;
    float drop_scale = 1.0f;
    // Further K segments (A, B sources) of a chain of like GEMMs added into one value.
    std::vector<std::pair<uint32_t, uint32_t>> segs;
    std::string what;
    bool c16 = false;  // mixed precision: the output's f16 copy is written too
    // Mixed precision: false for an operand or output held only as its f16 copy.
    bool a32 = true, b32 = true, c32 = true;
    // Mixed precision: the epilogue's pre-activation (written by an activation, read by an
    // activation gradient) held only as its f16 copy.
    bool pre16 = false;
  };
  struct Pending {
    std::function<Launch()> make;
    double flop = 0, bytes = 0;
    bool side = false;
    std::vector<std::shared_ptr<GemmJob>> gemm;  // the GEMM(s) this launch runs, for grouping
    bool pure = false;
    // A loss launch that may instead run as a block of the optimizer launch (finalize_adamw): its
    // arguments at run time.
    std::function<hk::CeLossJob()> loss_tail;
  };
  std::vector<Pending> pending;
  // Outputs of non-GEMM launches that write an f16 copy and may drop the f32 value (LayerNorm
  // backward's second output, the f16 attention's outputs and gradients).
  std::vector<uint32_t> ln_posts;
  std::map<uint32_t, void*> ln_stats_tok;             // LN input value -> stats [rows, 2]
  std::map<uint32_t, void*> ce_stats_tok;             // logits value -> stats [rows, 2]
  std::map<std::pair<uint32_t, uint32_t>, void*> ce_den_tok;  // (logits, weights) -> den
  std::map<std::vector<uint32_t>, std::pair<uint32_t, void*>> attn_fwd;  // operands -> (output, stats)
  // Reductions left to the batched column finalize: partial sums at `offset` floats into the
  // workspace `tok`, finished into the values lo (columns below split) and hi.
  struct DeferredJob { void* tok; int64_t offset, lo, hi; int32_t chunks, width, split; };
  std::vector<DeferredJob> deferred;
  auto R = [&](size_t bytes) { return arena_.reserve(bytes); };
  auto A = [this](void* tok) { return arena_.at(tok); };
  auto P = [this](uint32_t id) { return ptr(id); };
  auto F = [this](uint32_t id) { return static_cast<float*>(ptr(id)); };
  auto I = [this](uint32_t id) { return static_cast<int32_t*>(ptr(id)); };
  auto shape = [&](uint32_t v) -> const std::vector<int64_t>& { return p.node(v).ty.shape; };
  const uint64_t seed = s_.seed_;
  // Reserves the f16 copy of v when a GEMM reads v (see gemm_operands); true when it has one.
  auto want16 = [&](int64_t v) -> bool {
    if (v < 0 || !gemm_operands.count(uint32_t(v))) return false;
    const uint32_t vid = uint32_t(v);
    if (token16_.count(vid) || fixed16_.count(vid)) return true;
    const Node& x = p.node(vid);
    if (x.ty.rank() != 2 || x.ty.dtype != DType::F32) return false;
    token16_[vid] = arena_.reserve(size_t(x.ty.shape[0] * ld_of(vid)) * 2);
    return true;
  };
  auto H16 = [this](int64_t v) -> _Float16* { return v >= 0 ? ptr16(uint32_t(v)) : nullptr; };
  // The launch of one GEMM or a group of like GEMMs (one hk::gemm_group call).
  auto gemm_launch = [this, F, A, I](std::vector<std::shared_ptr<GemmJob>> jobs) {
    return [this, F, A, I, jobs]() {
      std::string what = jobs[0]->what;
      for (size_t q = 1; q < jobs.size(); ++q) what += " & %" + std::to_string(jobs[q]->id);
      return Launch{what, [this, F, A, I, jobs](hipStream_t s) {
                      hk::GemmArgs list[hk::kGemmGroupMax];
                      for (size_t q = 0; q < jobs.size(); ++q) {
                        const GemmJob& j = *jobs[q];
                        hk::GemmArgs a = j.g;
                        a.a = j.a32 ? F(j.asrc) : nullptr;
                        a.b = j.b32 ? F(j.bsrc) : nullptr;
                        a.c = j.c32 ? F(j.out_id) : nullptr;
                        a.bias = j.bias_id >= 0 ? F(uint32_t(j.bias_id)) : nullptr;
                        a.workspace = j.ws ? static_cast<float*>(A(j.ws)) : nullptr;
                        a.ce_part = j.ce_part ? static_cast<float*>(A(j.ce_part)) : nullptr;
                        a.ce_tab = j.ce_tab ? static_cast<const float4*>(A(j.ce_tab)) : nullptr;
                        a.colsum = j.cs_id >= 0 ? F(uint32_t(j.cs_id)) : nullptr;
                        a.act = j.epi.act;
                        if (!j.segs.empty()) {
                          a.ksegs = int(1 + j.segs.size());
                          a.seg_a[0] = a.a;
                          a.seg_b[0] = a.b;
                          for (size_t t = 0; t < j.segs.size(); ++t) {
                            a.seg_a[t + 1] = F(j.segs[t].first);
                            a.seg_b[t + 1] = F(j.segs[t].second);
                          }
                        }
                        if (j.epi.node != j.id && j.epi.act == hk::EPI_NONE) a.addend = F(uint32_t(j.epi.aux));
                        if (j.epi.act == hk::EPI_GELU_GRAD || j.epi.act == hk::EPI_RELU_GRAD) {
                          if (j.pre16) a.pre16 = ptr16(uint32_t(j.epi.aux));
                          else a.pre_in = F(uint32_t(j.epi.aux));
                        }
                        if (j.epi.act == hk::EPI_GELU || j.epi.act == hk::EPI_RELU) {
                          if (j.pre16) a.pre16 = ptr16(j.id);
                          else a.pre_out = F(j.id);
                        }
                        if (j.epi.drop >= 0) {
                          a.drop_token = I(j.drop_tok);
                          a.drop_threshold = j.drop_thr;
                          a.drop_scale = j.drop_scale;
                          a.drop_seed = s_.seed_;
                        }
                        if (a.h16 && a.ce_operand == 0 && a.ksegs <= 1) {
                          a.a16 = ptr16(j.asrc);
                          a.b16 = ptr16(j.bsrc);
                        }
                        if (j.c16) a.c16 = ptr16(j.out_id);
                        list[q] = a;
                      }
                      hk::gemm_group(s, list, int(jobs.size()));
                    }};
    };
  };

  // A packed corpus feeds the batch: the step's rows drawn and masked on the device, then the
  // masked-row gather of the selected rows, ahead of everything that reads them.
  if (s_.corpus_) {
    // An input the plan keeps (one no launch reads has no slot, and is not written).
    auto slot_of = [&](const std::string& name) -> int64_t {
      for (auto& slot : inputs_)
        if (slot.name == name) return int64_t(slot.id);
      return -1;
    };
    const int64_t ids = slot_of("ids"), positions = slot_of("positions"), key_mask = slot_of("key_mask");
    int64_t labels = slot_of("labels"), weights = slot_of("weights");
    const Node* rows_in = p.input(kMaskedRowsInput);
    void* lab_tok = nullptr;
    void* w_tok = nullptr;
    const int64_t rows = int64_t(s_.corpus_batch_ * uint64_t(s_.corpus_->c.seq_len));
    if (rows_in && labels < 0) lab_tok = R(size_t(rows) * 4);
    if (rows_in && weights < 0) w_tok = R(size_t(rows) * 4);
    const uint64_t batch = s_.corpus_batch_;
    const hk::MlmCorpus mc = s_.corpus_->c;
    auto draw = [this] { return static_cast<const int32_t*>(static_cast<void*>(static_cast<char*>(arena_.at(input_token_)) + draw_offset_)); };
    auto opt_i = [this](int64_t v) { return v >= 0 ? static_cast<int32_t*>(ptr(uint32_t(v))) : nullptr; };
    auto opt_f = [this](int64_t v) { return v >= 0 ? static_cast<float*>(ptr(uint32_t(v))) : nullptr; };
    pending.push_back({[=] {
      return Launch{"MlmBatch", [=](hipStream_t st) {
                      hk::mlm_rows(st, mc, draw(), int64_t(batch), opt_i(ids), opt_i(positions), opt_f(key_mask),
                                   lab_tok ? static_cast<int32_t*>(A(lab_tok)) : opt_i(labels),
                                   w_tok ? static_cast<float*>(A(w_tok)) : opt_f(weights));
                    }};
    }});
    pending.back().bytes = 4.0 * double(rows) * 6;
    if (rows_in) {
      const Node* ml = nullptr;
      const Node* mw = nullptr;
      for (auto& x : p.nodes)
        if (x.op == Op::Input) {
          if (x.name.rfind(kMaskedLabelsPrefix, 0) == 0) ml = &x;
          if (x.name.rfind(kMaskedWeightsPrefix, 0) == 0) mw = &x;
        }
      if (!ml || !mw) throw IrError("the masked-row gather inputs are incomplete");
      const uint32_t rid = rows_in->id, lid = ml->id, wid = mw->id;
      const int64_t cap = rows_in->ty.count();
      uint32_t* err = s_.corpus_->error;
      pending.push_back({[=] {
        return Launch{"MaskedGather", [=](hipStream_t st) {
                        hk::masked_gather(st, lab_tok ? static_cast<int32_t*>(A(lab_tok)) : opt_i(labels),
                                          w_tok ? static_cast<float*>(A(w_tok)) : opt_f(weights), rows, cap, draw(),
                                          I(rid), I(lid), F(wid), err);
                      }};
      }});
      pending.back().bytes = 4.0 * double(2 * rows + 3 * cap);
    }
  }

  // EmbeddingGrads whose ids are step inputs take the sorted-segment path: each distinct ids
  // input is sorted once, by one launch at the head of the step (the ids exist before any
  // kernel runs), and each EmbeddingGrad then reads its plan.
  std::map<uint32_t, void*> eg_plan_tok;  // EmbeddingGrad node -> plan buffer of its ids
  std::set<uint32_t> eg_deferred;                      // launched with a later EmbeddingGrad
  std::map<uint32_t, std::vector<uint32_t>> eg_group;  // last EmbeddingGrad -> every one it launches
  std::map<uint32_t, uint32_t> eg_drop;                // EmbeddingGrad -> the DropoutGrad of it written beside
  std::set<uint32_t> eg_drop_nodes;
  {
    std::map<std::pair<uint32_t, int64_t>, void*> by_ids;
    struct PlanJob { uint32_t ids; int64_t n, rows; void* tok; };
    std::vector<PlanJob> jobs;
    for (size_t k = 0; k < n; ++k) {
      const Node& x = p.nodes[k];
      if (!need[k] || x.op != Op::EmbeddingGrad || optimizer.count(x.id)) continue;
      const uint32_t ids = x.operands[0];
      const int64_t nn = shape(ids)[0], rows = x.rows;
      if (p.node(ids).op != Op::Input || !hk::eg_sorted_fits(nn, rows)) continue;
      auto key = std::make_pair(ids, rows);
      if (!by_ids.count(key)) {
        for (auto& ps : plan_slots_)
          if (ps.ids == ids && ps.rows == rows)  // made by the host in the input block (a token there)
            by_ids[key] = static_cast<char*>(input_token_) + ps.offset;
        if (!by_ids.count(key)) {
          if (!hk::eg_device_plan_fits(nn, rows)) continue;  // the scatter kernel takes it instead
          by_ids[key] = R(hk::eg_plan_bytes(nn, rows));
          jobs.push_back({ids, nn, rows, by_ids[key]});
        }
      }
      eg_plan_tok[x.id] = by_ids[key];
    }
    // EmbeddingGrads of one gradient (the token and position tables of the same embedding sum)
    // share one launch, at the last of them, when nothing in between reads an earlier one's output.
    std::map<uint32_t, std::vector<uint32_t>> by_g;
    for (size_t k = 0; k < n; ++k) {
      const Node& x = p.nodes[k];
      if (need[k] && x.op == Op::EmbeddingGrad && eg_plan_tok.count(x.id)) by_g[x.operands[1]].push_back(x.id);
    }
    for (auto& [g, members] : by_g) {
      std::vector<uint32_t> group;
      for (uint32_t m : members) {
        if (group.size() == size_t(hk::kEgJobs)) break;
        group.push_back(m);
      }
      if (group.size() < 2) continue;
      const size_t last = p.pos.at(group.back());
      bool ok = true;
      for (size_t q = 0; q + 1 < group.size() && ok; ++q) {
        const uint32_t out = eg_add.count(group[q]) ? eg_add.at(group[q]).first : group[q];
        for (size_t k = p.pos.at(group[q]) + 1; k < last && ok; ++k)
          if (need[k] && !optimizer.count(p.nodes[k].id) && p.nodes[k].id != out)
            for (uint32_t o : p.nodes[k].operands) ok = ok && o != out && o != group[q];
      }
      if (!ok) continue;
      for (size_t q = 0; q + 1 < group.size(); ++q) eg_deferred.insert(group[q]);
      eg_group[group.back()] = group;
    }
    // A DropoutGrad of such an EmbeddingGrad's own output is written by the same apply pass, beside
    // it (the pass holds each element; the mask is the dropout's, by element index).
    for (size_t k = 0; k < n; ++k) {
      const Node& x = p.nodes[k];
      if (!need[k] || x.op != Op::DropoutGrad || optimizer.count(x.id)) continue;
      const uint32_t e = x.operands[1];
      if (!eg_plan_tok.count(e) || eg_add.count(e) || eg_drop.count(e) || p.node(e).ty.count() != x.ty.count()) continue;
      eg_drop[e] = x.id;
      eg_drop_nodes.insert(x.id);
    }
    for (size_t q0 = 0; q0 < jobs.size(); q0 += hk::kEgJobs) {
      std::vector<PlanJob> part(jobs.begin() + q0, jobs.begin() + std::min(jobs.size(), q0 + hk::kEgJobs));
      std::string what = "EmbeddingPlan";
      double bytes = 0;
      for (auto& j : part) {
        what += " %" + std::to_string(j.ids);
        bytes += double(j.n) * 4 + double(hk::eg_plan_bytes(j.n, j.rows));
      }
      pending.push_back({[=] {
        return Launch{what, [=](hipStream_t st) {
                        hk::EgPlanJob js[hk::kEgJobs];
                        for (size_t q = 0; q < part.size(); ++q)
                          js[q] = hk::EgPlanJob{I(part[q].ids), static_cast<int32_t*>(A(part[q].tok)), int32_t(part[q].n),
                                                int32_t(part[q].rows), 0, 0};
                        hk::eg_plan(st, js, int(part.size()));
                      }};
      }});
      pending.back().bytes = bytes;
    }
  }

  // A step's loss formed by a cross-entropy loss launch is appended to the loss log by that launch,
  // in place of a RecordLoss launch after the optimizer (the value is the same: nothing between
  // writes it).
  bool loss_logged = false;
  auto logs_loss = [&](uint32_t v, std::string& what) {
    if (!is_step_ || v != st.loss || loss_logged) return false;
    loss_logged = true;
    what += " +RecordLoss";
    return true;
  };
  auto loss_log = [this](bool rec) {
    return rec ? hk::LossLog{s_.losses_dev_, s_.counter_, s_.loss_capacity_} : hk::LossLog{};
  };

  for (size_t k = 0; k < n; ++k) {
    if (!need[k]) continue;
    const Node& x = p.nodes[k];
    if (optimizer.count(x.id)) continue;
    const uint32_t id = x.id;
    const auto& o = x.operands;
    const int64_t count = x.ty.count();
    std::string what = std::string(op_name(x.op)) + " %" + std::to_string(id) + " " + type_string(x.ty);
    if (x.op == Op::MatMul || (x.op == Op::AddRows && mm_fused.count(o[0]))) {
      const Node& m = p.node(x.op == Op::MatMul ? id : o[0]);
      what += " k=" + std::to_string(shape(m.operands[0])[1]);
      if (x.op == Op::AddRows) what = "MatMul+AddRows" + what.substr(7);
      if (x.op == Op::MatMul && colsum_of.count(id)) what += " +SumRows %" + std::to_string(colsum_of.at(id));
    }
    auto push = [&](std::function<void(hipStream_t)> f) { pending.push_back({[what, f] { return Launch{what, f}; }}); };
    const size_t first_pending = pending.size();
    // Algorithmic cost of the node (kernel.rs:1221, 1565): flops of contractions, bytes of the
    // values every other op reads and writes.
    double flop = 0, bytes = 0;
    auto elems = [&](uint32_t v) { return double(p.node(v).ty.count()); };
    switch (x.op) {
      case Op::MatMul: case Op::AddRows: {
        if (x.op == Op::AddRows && !mm_fused.count(o[0])) { bytes = 4 * (2 * elems(id) + elems(o[1])); break; }
        const Node& m = p.node(x.op == Op::MatMul ? id : o[0]);
        double M = double(m.ty.shape[0]), N = double(m.ty.shape[1]), K = double(shape(m.operands[0])[1]);
        flop = 2 * M * N * K;
        bytes = 4 * (M * K + K * N + M * N + (x.op == Op::AddRows ? N : 0));
        break;
      }
      case Op::Attention: case Op::AttentionGradQ: case Op::AttentionGradK: case Op::AttentionGradV: {
        int64_t B = shape(o[3])[0], S = shape(o[3])[1], L = shape(o[0])[0] / B, H = shape(o[0])[1];
        flop = (x.op == Op::Attention ? 4.0 : 8.0) * double(B) * double(L) * double(S) * double(H);
        break;
      }
      case Op::Input: case Op::ParamRead: case Op::Scalar: break;
      default:
        for (auto v : o) bytes += 4 * elems(v);
        bytes += 4 * double(count);
        break;
    }
    switch (x.op) {
      case Op::Input: case Op::ParamRead: case Op::Scalar: break;
      case Op::Add: case Op::Sub: case Op::Mul: case Op::Div: {
        if (eg_add_nodes.count(id) || epi_nodes.count(id) || ln_fused_nodes.count(id)) break;  // written by a fused launch
        if (folded_scalar.count(id) || ew_inner.count(id)) break;  // a constant, or inside its consumer's launch
        if (ew_chain.count(id)) {
          const EwChain c = ew_chain.at(id);
          const Node& in = p.node(c.inner);
          const uint32_t a = in.operands[0], b = in.operands[1];
          const uint32_t sc = c.inner_left ? o[1] : o[0];
          const int op1 = c.op1, op2 = c.op2;
          const bool left = c.inner_left;
          what = std::string(op_name(in.op)) + ">" + op_name(x.op) + " %" + std::to_string(c.inner) + " %" +
                 std::to_string(id) + " " + type_string(x.ty);
          push([=](hipStream_t s) { hk::elementwise2(s, op1, F(a), F(b), op2, F(sc), left, F(id), count); });
          bytes = 4.0 * (3.0 * double(count) + 1.0);
          break;
        }
        int op = x.op == Op::Add ? hk::EW_ADD : x.op == Op::Sub ? hk::EW_SUB : x.op == Op::Mul ? hk::EW_MUL : hk::EW_DIV;
        bool as = p.node(o[0]).ty.rank() == 0 && count > 1, bs = p.node(o[1]).ty.rank() == 0 && count > 1;
        uint32_t a = o[0], b = o[1];
        push([=](hipStream_t s) { hk::elementwise(s, op, F(a), F(b), F(id), count, as, bs); });
        break;
      }
      case Op::Relu: case Op::Gelu: case Op::Sqrt: case Op::StopGradient: {
        if (epi_nodes.count(id)) break;  // written by its GEMM
        int op = x.op == Op::Relu ? hk::EW_RELU : x.op == Op::Gelu ? hk::EW_GELU : x.op == Op::Sqrt ? hk::EW_SQRT : hk::EW_COPY;
        uint32_t a = o[0];
        push([=](hipStream_t s) { hk::elementwise(s, op, F(a), nullptr, F(id), count, false, false); });
        break;
      }
      case Op::ReluGrad: case Op::GeluGrad: {
        if (epi_nodes.count(id) || ln_post_nodes.count(id)) break;  // written by its GEMM or LayerNorm backward
        int op = x.op == Op::ReluGrad ? hk::EW_RELU_GRAD : hk::EW_GELU_GRAD;
        uint32_t a = o[0], g = o[1];
        push([=](hipStream_t s) { hk::elementwise(s, op, F(a), F(g), F(id), count, false, false); });
        break;
      }
      case Op::MatMul: case Op::AddRows: {
        uint32_t mm = x.op == Op::MatMul ? id : o[0];
        if (x.op == Op::MatMul && mm_fused.count(id)) break;
        bool fused = x.op == Op::AddRows && mm_fused.count(o[0]);
        const bool swap = x.op == Op::MatMul && mm_transposed.count(id);
        // The value the GEMM writes: its own, the Transpose's (swapped), or an epilogue consumer's.
        const Epi epi = gemm_epi.count(id) ? gemm_epi.at(id) : Epi{id, hk::EPI_NONE, -1};
        const uint32_t out_id = swap ? mm_transposed.at(id) : epi.drop >= 0 ? uint32_t(epi.drop) : epi.node;
        if (epi.node != id) what += " +" + std::string(op_name(p.node(epi.node).op)) + " %" + std::to_string(epi.node);
        if (epi.drop >= 0) what += " +DropoutGrad %" + std::to_string(epi.drop);
        if (x.op == Op::AddRows && !fused) {
          uint32_t a = o[0], b = o[1];
          int64_t rows = x.ty.shape[0], h = x.ty.shape[1];
          push([=](hipStream_t s) { hk::add_rows(s, F(a), F(b), F(id), rows, h); });
          break;
        }
        const Node& m = p.node(mm);
        Resolved ra = resolve(p, m.operands[0]), rb = resolve(p, m.operands[1]);
        int64_t M = m.ty.shape[0], N = m.ty.shape[1], K = shape(m.operands[0])[1];
        hk::GemmArgs g{};
        uint32_t asrc = ra.src, bsrc = rb.src;
        // Leading dimensions are the sources' row pitches (their widths unless padded).
        if (!swap) {
          g.m = M; g.n = N; g.k = K;
          g.ta = ra.flip;
          g.tb = rb.flip;
        } else {
          // C^T [N, M] = op(B)^T op(A)^T: B's source becomes the left operand, A's the right.
          g.m = N; g.n = M; g.k = K;
          g.ta = !rb.flip;
          g.tb = !ra.flip;
          std::swap(asrc, bsrc);
        }
        // A cross-entropy head: an operand that is the loss gradient is formed from the logits.
        void* ce_tab = nullptr;
        for (int side = 0; side < 2; ++side) {
          uint32_t& src = side == 0 ? asrc : bsrc;
          if (!ce_head_grad.count(src)) continue;
          CeHead& hd = ce_head.at(ce_head_grad.at(src));
          if (!hd.tab) hd.tab = R(size_t(hd.rows) * 16);
          ce_tab = hd.tab;
          g.ce_operand = side + 1;
          g.ce_cols = hd.cols;
          src = hd.logits;
          what += " (cross-entropy gradient of %" + std::to_string(hd.logits) + ")";
        }
        void* ce_part = nullptr;
        if (ce_head.count(out_id)) {
          CeHead& hd = ce_head.at(out_id);
          hd.part = R(size_t(hd.rows * hd.tiles) * 8);
          ce_part = hd.part;
        }
        g.lda = ld_of(asrc);
        g.ldb = ld_of(bsrc);
        g.ldc = ld_of(out_id);
        g.pad_a = pitch.count(asrc) != 0;
        g.pad_b = pitch.count(bsrc) != 0;
        g.pad_c = pitch.count(out_id) != 0;
        g.h16 = s_.opt_.mixed;
        const int64_t cs_id = x.op == Op::MatMul && colsum_of.count(id) ? int64_t(colsum_of.at(id)) : -1;
        g.sum_a = swap;  // the column sums of B are the row sums of the swapped left operand
        int64_t bias_id = fused ? int64_t(o[1]) : -1;
        // Split-K partials only the optimizer reads are summed by the batched column finalize.
        g.defer = bias_id < 0 && epi.node == id && only_optimizer_reads(int64_t(out_id)) && only_optimizer_reads(cs_id);
        int64_t wsf = hk::gemm_workspace(g.m, g.n, g.k, cs_id >= 0, g.sum_a, g.defer, g.h16, g.ce_operand || ce_part);
        void* ws = wsf > 0 ? R(size_t(wsf) * 4) : nullptr;
        g.workspace_floats = wsf;
        auto job = std::make_shared<GemmJob>();
        job->g = g;
        job->asrc = asrc;
        job->bsrc = bsrc;
        job->out_id = out_id;
        job->id = id;
        job->bias_id = bias_id;
        job->cs_id = cs_id;
        job->epi = epi;
        if (epi.drop >= 0) {
          const Node& d = p.node(uint32_t(epi.drop));
          job->drop_tok = d.operands[size_t(token_operand(Op::DropoutGrad))];
          job->drop_thr = dropout_threshold(d.scalar);
          job->drop_scale = 1.0f / (1.0f - d.scalar);
        }
        job->ws = ws;
        job->ce_part = ce_part;
        job->ce_tab = ce_tab;
        job->what = what;
        job->c16 = g.h16 && !ce_part && g.ce_operand == 0 && !g.defer && want16(int64_t(out_id));
        pending.push_back({gemm_launch({job}), 0, 0, is_step_ && g.defer, {job}});
        pending.back().pure = true;
        if (g.defer && wsf > 0) {
          const int split = hk::gemm_split_for(g.m, g.n, g.k, true, g.h16, g.ce_operand != 0);
          const int32_t mn = int32_t(g.m * g.n);
          deferred.push_back({ws, 0, int64_t(out_id), -1, split, mn, mn});
          if (cs_id >= 0) {
            const int32_t w = int32_t(g.sum_a ? g.m : g.n);
            deferred.push_back({ws, int64_t(split) * g.m * g.n, cs_id, -1, split, w, w});
          }
        }
        break;
      }
      case Op::Transpose: {
        if (folded.count(id) || transposed_out.count(id)) break;
        Resolved r = resolve(p, o[0]);
        uint32_t src = r.src;
        if (r.flip) {  // the transpose of a transpose: a copy of the source
          push([=](hipStream_t s) { hk::copy(s, F(src), F(id), count); });
        } else {
          int64_t rows = shape(src)[0], cols = shape(src)[1];
          push([=](hipStream_t s) { hk::transpose(s, F(src), F(id), rows, cols); });
        }
        break;
      }
      case Op::ReduceSum: case Op::ReduceMean: {
        uint32_t a = o[0];
        int64_t na = p.node(a).ty.count();
        bool mean = x.op == Op::ReduceMean;
        push([=](hipStream_t s) { hk::reduce_sum(s, F(a), F(id), na, mean); });
        break;
      }
      case Op::Mse: {
        uint32_t a = o[0], b = o[1];
        int64_t na = p.node(a).ty.count();
        push([=](hipStream_t s) { hk::mse(s, F(a), F(b), F(id), na); });
        break;
      }
      case Op::BroadcastScalar: {
        uint32_t a = o[0];
        push([=](hipStream_t s) { hk::fill_from(s, F(a), F(id), count); });
        break;
      }
      case Op::Embedding: {
        if (ln_fused_nodes.count(id)) break;  // gathered by its fused LayerNorm
        uint32_t t = o[0], ids = o[1];
        int64_t rows = shape(t)[0], h = shape(t)[1], nn = shape(ids)[0];
        if (p.node(ids).op == Op::Input) id_bounds_[p.node(ids).name] = rows;
        push([=](hipStream_t s) { hk::embedding(s, F(t), I(ids), F(id), nn, rows, h); });
        break;
      }
      case Op::EmbeddingGrad: {
        uint32_t ids = o[0], g = o[1];
        int64_t nn = shape(ids)[0], h = shape(g)[1], rows = x.rows;
        if (p.node(ids).op == Op::Input) {
          auto it = id_bounds_.find(p.node(ids).name);
          id_bounds_[p.node(ids).name] = it == id_bounds_.end() ? rows : std::min(it->second, rows);
        }
        if (eg_deferred.count(id)) break;  // launched with a later EmbeddingGrad of the same gradient
        if (eg_plan_tok.count(id)) {
          struct Job { void* plan; uint32_t g, out; int64_t addend, n, rows, h, drop = -1, drop_tok = -1; uint64_t thr = 0; float scale = 1; };
          std::vector<Job> jobs;
          const std::vector<uint32_t> members = eg_group.count(id) ? eg_group.at(id) : std::vector<uint32_t>{id};
          what.clear();
          bytes = 0;
          for (uint32_t m : members) {
            const Node& e = p.node(m);
            const bool add = eg_add.count(m) != 0;
            const uint32_t out = add ? eg_add.at(m).first : m;
            jobs.push_back({eg_plan_tok.at(m), e.operands[1], out, add ? int64_t(eg_add.at(m).second) : -1,
                            shape(e.operands[0])[0], e.rows, shape(e.operands[1])[1]});
            what += (what.empty() ? "" : " & ") + std::string(add ? "EmbeddingGrad+Add %" : "EmbeddingGrad %") +
                    std::to_string(m) + (add ? " %" + std::to_string(out) : "") + " " + type_string(e.ty);
            if (eg_drop.count(m)) {
              const Node& d = p.node(eg_drop.at(m));
              Job& jb = jobs.back();
              jb.drop = d.id;
              jb.drop_tok = d.operands[size_t(token_operand(Op::DropoutGrad))];
              jb.thr = dropout_threshold(d.scalar);
              jb.scale = 1.0f / (1.0f - d.scalar);
              what += " +DropoutGrad %" + std::to_string(d.id);
              bytes += 4.0 * double(e.ty.count());
            }
            const double cnt = double(e.ty.count());
            bytes += 4.0 * (double(shape(e.operands[0])[0]) * (1 + double(shape(e.operands[1])[1])) + cnt) +
                     (add ? 8.0 * cnt : 0.0);
          }
          push([=](hipStream_t s) {
            hk::EgApplyJob js[hk::kEgJobs];
            for (size_t q = 0; q < jobs.size(); ++q) {
              hk::EgApplyJob j{};
              j.plan = static_cast<const int32_t*>(A(jobs[q].plan));
              j.g = F(jobs[q].g);
              j.addend = jobs[q].addend >= 0 ? F(uint32_t(jobs[q].addend)) : nullptr;
              j.out = F(jobs[q].out);
              j.n = int32_t(jobs[q].n);
              j.rows = int32_t(jobs[q].rows);
              j.h = jobs[q].h;
              if (jobs[q].drop >= 0) {
                j.out2 = F(uint32_t(jobs[q].drop));
                j.drop_token = I(uint32_t(jobs[q].drop_tok));
                j.drop_threshold = jobs[q].thr;
                j.drop_scale = jobs[q].scale;
                j.seed = seed;
              }
              js[q] = j;
            }
            hk::eg_apply(s, js, int(jobs.size()));
          });
        } else if (eg_add.count(id)) {
          const uint32_t sum_id = eg_add.at(id).first, addend = eg_add.at(id).second;
          what = "EmbeddingGrad+Add %" + std::to_string(id) + " %" + std::to_string(sum_id) + " " + type_string(x.ty);
          push([=](hipStream_t s) { hk::embedding_grad(s, I(ids), F(g), F(sum_id), nn, rows, h, F(addend)); });
          bytes += 8.0 * double(count);
        } else {
          push([=](hipStream_t s) { hk::embedding_grad(s, I(ids), F(g), F(id), nn, rows, h); });
        }
        break;
      }
      case Op::SumRows: {
        if (colsum_fused.count(id)) break;  // taken by its GEMM
        if (ln_member.count(id)) goto layer_norm_backward;
        uint32_t a = o[0];
        int64_t rows = shape(a)[0], h = shape(a)[1];
        if (rows == 0) {
          push([=](hipStream_t s) { hk::fill_zero(s, F(id), h * 4); });
          break;
        }
        const int64_t chunks = hk::column_partial_chunks(rows, h);
        void* part = R(size_t(chunks * h) * 4);
        const int64_t lda = ld_of(a);
        push([=](hipStream_t s) { hk::column_partial(s, F(a), static_cast<float*>(A(part)), rows, h, lda); });
        DeferredJob d{part, 0, int64_t(id), -1, int32_t(chunks), int32_t(h), int32_t(h)};
        if (only_optimizer_reads(int64_t(id))) {
          deferred.push_back(d);
        } else {
          push([=](hipStream_t s) {
            hk::ColumnJob j{static_cast<float*>(A(d.tok)), F(uint32_t(d.lo)), nullptr, d.chunks, d.width, d.split, 0};
            hk::column_finalize(s, &j, 1);
          });
        }
        break;
      }
      case Op::LayerNorm: case Op::LayerNormGradX: case Op::LayerNormGradGamma: {
        if (x.op != Op::LayerNorm) goto layer_norm_backward;
        uint32_t xv = o[0];
        int64_t rows = shape(xv)[0], h = shape(xv)[1];
        bool have = ln_stats_tok.count(xv) != 0;
        if (!have) ln_stats_tok[xv] = R(size_t(rows) * 8);
        void* stats = ln_stats_tok[xv];
        if (x.op == Op::LayerNorm && ln_fused.count(id)) {
          const LnFused f = ln_fused.at(id);
          const uint32_t gm = o[1], bt = o[2];
          const bool write_stats = !have;
          // (threshold, scale) of a Dropout node, as its own launch would use them.
          auto spec = [&](int64_t d) {
            if (d < 0) return std::make_pair(uint64_t(0), 1.0f);
            const float pr = p.node(uint32_t(d)).scalar;
            return std::make_pair(dropout_threshold(pr), 1.0f / (1.0f - pr));
          };
          const auto si = spec(f.din), so = spec(f.dout);
          const int64_t tin = f.din >= 0 ? int64_t(p.node(uint32_t(f.din)).operands[size_t(token_operand(Op::Dropout))]) : -1;
          const int64_t tout = f.dout >= 0 ? int64_t(p.node(uint32_t(f.dout)).operands[size_t(token_operand(Op::Dropout))]) : -1;
          const int64_t s_val = f.gather >= 0 ? f.gather : f.add;  // the LayerNorm input as stored
          const int64_t gids = f.gather >= 0 ? int64_t(p.node(uint32_t(f.gather)).operands[1]) : -1;
          const int64_t src_rows = f.gather >= 0 ? shape(uint32_t(f.add))[0] : rows;
          if (gids >= 0 && p.node(uint32_t(gids)).op == Op::Input) {
            auto it = id_bounds_.find(p.node(uint32_t(gids)).name);
            id_bounds_[p.node(uint32_t(gids)).name] = it == id_bounds_.end() ? src_rows : std::min(it->second, src_rows);
          }
          // An Embedding operand: its table, its ids and the table's rows.
          struct Emb { int64_t table = -1, ids = -1, rows = 0; };
          auto emb = [&](int64_t e) {
            Emb r;
            if (e < 0) return r;
            r.table = p.node(uint32_t(e)).operands[0];
            r.ids = p.node(uint32_t(e)).operands[1];
            r.rows = shape(uint32_t(r.table))[0];
            if (p.node(uint32_t(r.ids)).op == Op::Input) {
              auto it = id_bounds_.find(p.node(uint32_t(r.ids)).name);
              id_bounds_[p.node(uint32_t(r.ids)).name] = it == id_bounds_.end() ? r.rows : std::min(it->second, r.rows);
            }
            return r;
          };
          const Emb ea = emb(f.ea), eb = emb(f.eb);
          const int64_t av = f.add >= 0 ? (ea.table >= 0 ? ea.table : f.a) : -1;
          const int64_t bv = f.add >= 0 ? (eb.table >= 0 ? eb.table : f.b) : int64_t(xv);
          const int64_t yv = f.dout >= 0 ? -1 : int64_t(id);
          what = "LayerNorm+fused %" + std::to_string(id);
          for (auto [tag, v] : {std::pair<const char*, int64_t>{" add %", f.add}, {" dropout-in %", f.din},
                                {" dropout-out %", f.dout}, {" gather %", f.gather}, {" embedding %", f.ea},
                                {" embedding %", f.eb}})
            if (v >= 0) what += tag + std::to_string(v);
          what += " " + type_string(x.ty);
          const bool y16 = want16(yv), yd16 = want16(f.dout);
          const bool b16 = ln_b16.count(id) && ln_b16.at(id) == uint32_t(bv) && want16(bv);
          push([=](hipStream_t s) {
            auto fp = [&](int64_t v2) { return v2 >= 0 ? F(uint32_t(v2)) : nullptr; };
            hk::ln_fused(s, fp(av), b16 && only16_.count(uint32_t(bv)) ? nullptr : F(uint32_t(bv)),
                         tin >= 0 ? I(uint32_t(tin)) : nullptr, si.first, si.second, F(gm), F(bt),
                         fp(s_val), fp(yv), write_stats ? static_cast<float*>(A(stats)) : nullptr,
                         tout >= 0 ? I(uint32_t(tout)) : nullptr, so.first, so.second, fp(f.dout), rows, h, seed,
                         gids >= 0 ? I(uint32_t(gids)) : nullptr, src_rows, ea.ids >= 0 ? I(uint32_t(ea.ids)) : nullptr,
                         ea.rows, eb.ids >= 0 ? I(uint32_t(eb.ids)) : nullptr, eb.rows, y16 ? H16(yv) : nullptr,
                         yd16 ? H16(f.dout) : nullptr, b16 ? H16(bv) : nullptr);
          });
          bytes = 4.0 * double(count) * (2 + (av >= 0) + (f.add >= 0) + (yv >= 0) + (f.dout >= 0));
          break;
        }
        if (x.op == Op::LayerNorm) {
          uint32_t gm = o[1], bt = o[2];
          bool write_stats = !have;
          push([=](hipStream_t s) {
            hk::layer_norm(s, F(xv), F(gm), F(bt), F(id), write_stats ? static_cast<float*>(A(stats)) : nullptr, rows, h);
          });
          break;
        }
        goto layer_norm_backward;
      }
      layer_norm_backward: {
        const auto key = ln_member.at(id);
        const LnGroup gr = ln_groups.at(key);
        if (gr.first != k) break;  // launched with the group's first member
        const uint32_t xv = key.first, g = key.second;
        const int64_t rows = shape(xv)[0], h = shape(xv)[1];
        if (!ln_stats_tok.count(xv)) {
          void* st2 = ln_stats_tok[xv] = R(size_t(rows) * 8);
          push([=](hipStream_t s) { hk::ln_stats(s, F(xv), static_cast<float*>(A(st2)), rows, h); });
        }
        void* stats = ln_stats_tok.at(xv);
        const bool sums = gr.gamma >= 0 || gr.beta >= 0;
        const int64_t chunks = hk::ln_backward_blocks(rows, h);
        void* part = sums ? R(size_t(chunks * 2 * h) * 4) : nullptr;
        const int64_t dxv = gr.keep_dx ? gr.dx : -1, gmv = gr.gm, post = gr.post, aux = gr.aux;
        const int kind = gr.kind;
        what = "LayerNormBackward";
        for (auto [tag, v] : {std::pair<const char*, int64_t>{" dx %", gr.dx}, {" gamma %", gr.gamma}, {" beta %", gr.beta},
                              {" post %", gr.post}})
          if (v >= 0) what += tag + std::to_string(v);
        what += " " + type_string(p.node(xv).ty);
        uint64_t thr = 0;
        float scl = 1.0f;
        if (post >= 0 && kind == hk::LNB_DROPOUT) {
          const float pr = p.node(uint32_t(post)).scalar;
          thr = dropout_threshold(pr);
          scl = 1.0f / (1.0f - pr);
        }
        const bool dx16 = want16(dxv), post16 = want16(post);
        if (post16) ln_posts.push_back(uint32_t(post));
        push([=](hipStream_t s) {
          hk::ln_backward(s, F(xv), gmv >= 0 ? F(uint32_t(gmv)) : nullptr, F(g), static_cast<float*>(A(stats)),
                          dxv >= 0 ? F(uint32_t(dxv)) : nullptr, part ? static_cast<float*>(A(part)) : nullptr, rows, h,
                          post >= 0 && !only16_.count(uint32_t(post)) ? F(uint32_t(post)) : nullptr, kind,
                          post >= 0 && kind != hk::LNB_DROPOUT ? F(uint32_t(aux)) : nullptr,
                          post >= 0 && kind == hk::LNB_DROPOUT ? I(uint32_t(aux)) : nullptr, thr, scl, seed,
                          dx16 ? H16(dxv) : nullptr, post16 ? H16(post) : nullptr);
        });
        bytes = 4.0 * double(rows * h * (dxv >= 0 ? 3 : 2) + (gmv >= 0 ? h : 0) + (sums ? 2 * h : 0));
        if (sums) {
          DeferredJob d{part, 0, gr.gamma, gr.beta, int32_t(chunks), int32_t(2 * h), int32_t(h)};
          if (only_optimizer_reads(gr.gamma) && only_optimizer_reads(gr.beta)) {
            deferred.push_back(d);
          } else {
            pending.back().bytes = bytes;
            push([=](hipStream_t s) {
              hk::ColumnJob j{static_cast<float*>(A(d.tok)), d.lo >= 0 ? F(uint32_t(d.lo)) : nullptr,
                              d.hi >= 0 ? F(uint32_t(d.hi)) : nullptr, d.chunks, d.width, d.split, 0};
              hk::column_finalize(s, &j, 1);
            });
            bytes = 4.0 * double(chunks * 2 * h + 2 * h);
          }
        }
        break;
      }
      case Op::Softmax: {
        uint32_t a = o[0];
        int64_t rows = x.ty.shape[0], kk = x.ty.shape[1];
        push([=](hipStream_t s) { hk::softmax(s, F(a), F(id), rows, kk); });
        break;
      }
      case Op::SoftmaxGrad: {
        uint32_t y = o[0], g = o[1];
        int64_t rows = x.ty.shape[0], kk = x.ty.shape[1];
        push([=](hipStream_t s) { hk::softmax_grad(s, F(y), F(g), F(id), rows, kk); });
        break;
      }
      case Op::Attention: case Op::AttentionGradQ: case Op::AttentionGradK: case Op::AttentionGradV: {
        if (p.node(o[3]).ty.dtype != DType::F32) throw IrError("attention over key spans has no HIP kernel yet");
        uint32_t q = o[0], kv = o[1], v = o[2], mask = o[3];
        int64_t B = shape(mask)[0], S = shape(mask)[1], L = shape(q)[0] / B, H = shape(q)[1], heads = x.heads;
        if (!hk::attention_fits(S, H / heads)) throw IrError("attention shape has no HIP kernel (head width or sequence too large)");
        if (p.node(mask).op == Op::Input) key_masks_.push_back(p.node(mask).name);
        auto fkey = std::vector<uint32_t>{q, kv, v, mask, uint32_t(heads)};
        bool mfma = hk::attention_mfma(L, S, H / heads);
        const bool h16 = s_.opt_.mixed;  // mixed precision: the f16 MFMA
        if (flash(x)) {
          // The f16 attention on the operands' f16 copies, writing its outputs' copies itself.
          if (!want16(q) || !want16(kv) || !want16(v) || (x.op != Op::Attention && !want16(o[4])))
            throw IrError("f16 attention: an operand without its f16 copy");
          if (x.op == Op::Attention) {
            void* st2 = R(size_t(B * heads * L) * 8);
            attn_fwd[fkey] = {id, st2};
            const bool o16 = want16(id);
            if (o16) ln_posts.push_back(id);  // kept as its f16 copy alone when only f16 kernels read it
            push([=](hipStream_t s) {
              hk::flash16_fwd(s, H16(q), H16(kv), H16(v), F(mask), only16_.count(id) ? nullptr : F(id), o16 ? H16(id) : nullptr,
                              static_cast<float*>(A(st2)), B, L, S, H, heads);
            });
            pending.back().pure = true;
            break;
          }
          auto key = o;
          key.push_back(uint32_t(x.heads));
          auto& grp = attn_groups.at(key);
          int64_t first = -1;
          for (auto g2 : grp)
            if (g2 >= 0 && (first < 0 || p.pos.at(uint32_t(g2)) < p.pos.at(uint32_t(first)))) first = g2;
          if (first != int64_t(id)) break;  // the group's first member launches for all three
          const uint32_t g = o[4];
          const std::array<int64_t, 3> members = grp;
          what = "AttentionGrad16";
          for (int e = 0; e < 3; ++e)
            if (members[e] >= 0) what += std::string(" ") + "QKV"[e] + " %" + std::to_string(members[e]);
          int64_t fwd_out = -1;
          void *stats_tok = nullptr, *scratch_o = nullptr;
          auto f = attn_fwd.find(fkey);
          if (f != attn_fwd.end()) {
            fwd_out = int64_t(f->second.first);
            stats_tok = f->second.second;
          } else {
            scratch_o = R(size_t(shape(q)[0] * H) * 4);
            stats_tok = R(size_t(B * heads * L) * 8);
            push([=](hipStream_t s) {
              hk::flash16_fwd(s, H16(q), H16(kv), H16(v), F(mask), nullptr, static_cast<_Float16*>(A(scratch_o)),
                              static_cast<float*>(A(stats_tok)), B, L, S, H, heads);
            });
          }
          void* qterms = R(size_t(3 * B * heads * L) * 4);
          bool m16[3];
          for (int e = 0; e < 3; ++e) {
            m16[e] = members[e] >= 0 && want16(members[e]);
            if (m16[e]) ln_posts.push_back(uint32_t(members[e]));
          }
          push([=](hipStream_t s) {
            auto out = [&](int64_t v2) { return v2 >= 0 && !only16_.count(uint32_t(v2)) ? F(uint32_t(v2)) : nullptr; };
            auto out16 = [&](int e) { return m16[e] ? H16(members[e]) : nullptr; };
            const _Float16* fo = fwd_out >= 0 ? H16(fwd_out) : static_cast<_Float16*>(A(scratch_o));
            hk::flash16_bwd(s, H16(q), H16(kv), H16(v), F(mask), fo, H16(g), static_cast<float*>(A(stats_tok)),
                            static_cast<float*>(A(qterms)), out(members[0]), out16(0), out(members[1]), out16(1),
                            out(members[2]), out16(2), B, L, S, H, heads);
          });
          pending.back().pure = true;
          break;
        }
        if (x.op == Op::Attention) {
          void* st2 = mfma ? R(size_t(B * heads * L) * 8) : nullptr;
          attn_fwd[fkey] = {id, st2};
          push([=](hipStream_t s) {
            hk::attention_fwd(s, F(q), F(kv), F(v), F(mask), F(id), st2 ? static_cast<float*>(A(st2)) : nullptr, B, L, S, H, heads,
                              h16);
          });
          pending.back().pure = true;
          break;
        }
        auto key = o;
        key.push_back(uint32_t(x.heads));
        auto& grp = attn_groups.at(key);
        int64_t first = -1;
        for (auto g : grp)
          if (g >= 0 && (first < 0 || p.pos.at(uint32_t(g)) < p.pos.at(uint32_t(first)))) first = g;
        if (first != int64_t(id)) break;  // the group's first member launches for all three
        uint32_t g = o[4];
        std::array<int64_t, 3> members = grp;
        // The backward reads the forward's output and softmax statistics: those of the step's own
        // Attention over the same operands, else a forward run into scratch first.
        int64_t fwd_out = -1;
        void *stats_tok = nullptr, *scratch_o = nullptr, *dsum = nullptr, *dq_scratch = nullptr;
        if (mfma) {
          auto f = attn_fwd.find(fkey);
          if (f != attn_fwd.end()) {
            fwd_out = int64_t(f->second.first);
            stats_tok = f->second.second;
          } else {
            scratch_o = R(size_t(shape(q)[0] * H) * 4);
            stats_tok = R(size_t(B * heads * L) * 8);
            push([=](hipStream_t s) {
              hk::attention_fwd(s, F(q), F(kv), F(v), F(mask), static_cast<float*>(A(scratch_o)),
                                static_cast<float*>(A(stats_tok)), B, L, S, H, heads, h16);
            });
          }
          dsum = R(size_t(B * heads * L) * 4);
          if (members[0] < 0) dq_scratch = R(size_t(shape(q)[0] * H) * 4);
        }
        push([=](hipStream_t s) {
          auto out = [&](int64_t v2) { return v2 >= 0 ? F(uint32_t(v2)) : nullptr; };
          float* dq = members[0] >= 0 ? F(uint32_t(members[0])) : (dq_scratch ? static_cast<float*>(A(dq_scratch)) : nullptr);
          const float* fo = fwd_out >= 0 ? F(uint32_t(fwd_out)) : (scratch_o ? static_cast<float*>(A(scratch_o)) : nullptr);
          hk::attention_bwd(s, F(q), F(kv), F(v), F(mask), fo, stats_tok ? static_cast<float*>(A(stats_tok)) : nullptr, F(g), dq,
                            out(members[1]), out(members[2]), dsum ? static_cast<float*>(A(dsum)) : nullptr, B, L, S, H, heads,
                            h16);
        });
        pending.back().pure = true;
        break;
      }
      case Op::CrossEntropy: case Op::CrossEntropyGrad: {
        uint32_t lg = o[0], lab = o[1], w = o[2];
        int64_t rows = shape(lg)[0], v = shape(lg)[1];
        const int64_t ld = ld_of(lg);
        if (ce_head.count(lg)) {
          if (p.node(lab).op == Op::Input) id_bounds_["#labels:" + p.node(lab).name] = v;
          if (p.node(w).op == Op::Input) id_bounds_["#weights:" + p.node(w).name] = 0;
          CeHead& hd = ce_head.at(lg);
          if (hd.done || k != hd.emit_at) break;
          hd.done = true;
          if (!hd.part) throw IrError("cross-entropy head: its forward GEMM was not planned first");
          if (!hd.tab) hd.tab = R(size_t(rows) * 16);
          if (!ce_stats_tok.count(lg)) ce_stats_tok[lg] = R(size_t(rows) * 8);
          void* st2 = ce_stats_tok.at(lg);
          void* rl = R(size_t(rows) * 4);
          void* part = hd.part;
          void* tab = hd.tab;
          const int64_t tiles = hd.tiles;
          const uint32_t seed = hd.seed;
          what = "CrossEntropyHeadRows" + std::string(hd.loss >= 0 ? " loss %" + std::to_string(hd.loss) : "") + " grad %" +
                 std::to_string(hd.grad) + " " + type_string(p.node(lg).ty);
          push([=](hipStream_t s) {
            hk::ce_head_rows(s, static_cast<const float*>(A(part)), tiles, F(lg), ld, I(lab), F(w), F(seed),
                             static_cast<float*>(A(st2)), static_cast<float*>(A(rl)), static_cast<float4*>(A(tab)), rows,
                             v);
          });
          pending.back().bytes = 4.0 * double(rows * tiles * 2 + rows * (3 + 2 + 1 + 4));
          if (hd.loss >= 0) {
            auto dkey = std::make_pair(lg, w);
            if (!ce_den_tok.count(dkey)) ce_den_tok[dkey] = R(4);
            void* den = ce_den_tok.at(dkey);
            const uint32_t lid = uint32_t(hd.loss);
            what = "CrossEntropyLoss %" + std::to_string(hd.loss);
            const bool rec = logs_loss(lid, what);
            push([=](hipStream_t s) {
              const hk::LossLog log = loss_log(rec);
              hk::ce_loss(s, F(lg), I(lab), F(w), static_cast<float*>(A(st2)), F(lid), static_cast<float*>(A(den)), rows, v,
                          ld, static_cast<float*>(A(rl)), log);
            });
            bytes = 4.0 * double(2 * rows + 2);
          } else {
            bytes = pending.back().bytes;
          }
          break;
        }
        if (x.op == Op::CrossEntropyGrad && ld_of(id) != ld) throw IrError("cross-entropy gradient pitch differs from its logits'");
        if (p.node(lab).op == Op::Input) id_bounds_["#labels:" + p.node(lab).name] = v;
        if (p.node(w).op == Op::Input) id_bounds_["#weights:" + p.node(w).name] = 0;
        // One pass over the rows where the kernel fits: at the group's first node, the statistics,
        // the loss terms when the group has a loss, and the gradient when it has one whose upstream
        // gradient is available (a constant, or this node's own operand).
        auto& grp = ce_groups.at({lg, lab, w});
        if (hk::ce_rows_fits(v, ld) && (grp.loss == int64_t(id) || grp.grad == int64_t(id))) {
          if (x.op == Op::CrossEntropyGrad && grp.grad_done) break;
          if (!grp.done || (x.op == Op::CrossEntropyGrad && !grp.grad_done)) {
            const int64_t gnode = grp.grad;
            const bool with_grad = gnode >= 0 && !grp.grad_done &&
                                   (x.op == Op::CrossEntropyGrad || p.node(p.node(uint32_t(gnode)).operands[3]).op == Op::Scalar);
            const bool with_loss = grp.loss >= 0 && !grp.done;
            if (!ce_stats_tok.count(lg)) ce_stats_tok[lg] = R(size_t(rows) * 8);
            void* st2 = ce_stats_tok.at(lg);
            void* rl = with_loss ? R(size_t(rows) * 4) : nullptr;
            const uint32_t gsc = with_grad ? p.node(uint32_t(gnode)).operands[3] : 0;
            const int64_t gout = with_grad ? gnode : -1;
            what = std::string("CrossEntropyRows") + (with_loss ? " loss %" + std::to_string(grp.loss) : "") +
                   (with_grad ? " grad %" + std::to_string(gnode) : "") + " " + type_string(p.node(lg).ty);
            push([=](hipStream_t s) {
              hk::ce_rows(s, F(lg), I(lab), F(w), with_grad ? F(gsc) : nullptr, static_cast<float*>(A(st2)),
                          rl ? static_cast<float*>(A(rl)) : nullptr, gout >= 0 ? F(uint32_t(gout)) : nullptr, rows, v, ld);
            });
            // The row pass reads the logits, labels and weights and writes the gradient and the
            // row statistics; the loss launch behind it reads the row terms and weights.
            pending.back().bytes = 4.0 * double(rows * v * (with_grad ? 2 : 1) + rows * (2 + 2 + (with_loss ? 1 : 0)));
            const size_t rows_launch = pending.size() - 1;
            if (with_loss) {
              auto dkey = std::make_pair(lg, w);
              if (!ce_den_tok.count(dkey)) ce_den_tok[dkey] = R(4);
              void* den = ce_den_tok.at(dkey);
              const uint32_t lid = uint32_t(grp.loss);
              const bool rec = logs_loss(lid, what);
              push([=](hipStream_t s) {
                const hk::LossLog log = loss_log(rec);
                hk::ce_loss(s, F(lg), I(lab), F(w), static_cast<float*>(A(st2)), F(lid), static_cast<float*>(A(den)), rows,
                            v, ld, static_cast<float*>(A(rl)), log);
              });
              // Nothing but the optimizer reads the loss, and the row pass forms its own weight sum:
              // the loss may be summed by a block of the optimizer launch instead.
              if (is_step_ && only_optimizer_reads(int64_t(lid)))
                pending.back().loss_tail = [=] {
                  return hk::CeLossJob{F(lg), I(lab), F(w), static_cast<float*>(A(st2)), F(lid),
                                       static_cast<float*>(A(den)), rows, v, ld, static_cast<float*>(A(rl)),
                                       loss_log(rec)};
                };
              bytes = 4.0 * double(2 * rows + 2);
            } else {
              bytes = pending[rows_launch].bytes;
            }
            grp.done = true;
            grp.grad_done = grp.grad_done || with_grad;
          }
          break;
        }
        bool have = ce_stats_tok.count(lg) != 0;
        if (!have) {
          ce_stats_tok[lg] = R(size_t(rows) * 8);
          void* st2 = ce_stats_tok[lg];
          push([=](hipStream_t s) { hk::ce_stats(s, F(lg), static_cast<float*>(A(st2)), rows, v, ld); });
        }
        void* stats = ce_stats_tok[lg];
        auto dkey = std::make_pair(lg, w);
        bool have_den = ce_den_tok.count(dkey) != 0;
        if (!have_den) ce_den_tok[dkey] = R(4);
        void* den = ce_den_tok[dkey];
        if (x.op == Op::CrossEntropy) {
          const bool rec = logs_loss(id, what);
          push([=](hipStream_t s) {
            const hk::LossLog log = loss_log(rec);
            hk::ce_loss(s, F(lg), I(lab), F(w), static_cast<float*>(A(stats)), F(id), static_cast<float*>(A(den)), rows, v, ld,
                        nullptr, log);
          });
        } else {
          if (!have_den) {
            void* scratch = R(4);
            push([=](hipStream_t s) {
              hk::ce_loss(s, F(lg), I(lab), F(w), static_cast<float*>(A(stats)), static_cast<float*>(A(scratch)),
                          static_cast<float*>(A(den)), rows, v, ld);
            });
          }
          uint32_t g = o[3];
          push([=](hipStream_t s) {
            hk::ce_grad(s, F(lg), I(lab), F(w), static_cast<float*>(A(stats)), static_cast<float*>(A(den)), F(g), F(id), rows, v, ld);
          });
        }
        break;
      }
      case Op::Dropout: case Op::DropoutGrad: {
        if (ln_fused_nodes.count(id) || ln_post_nodes.count(id)) break;  // applied by a fused LayerNorm pass
        if (eg_drop_nodes.count(id)) break;  // written by its EmbeddingGrad's apply pass
        if (epi_nodes.count(id)) break;      // written by its GEMM's epilogue
        uint32_t tok = o[size_t(token_operand(x.op))], a = o[x.op == Op::Dropout ? 0 : 1];
        uint64_t threshold = dropout_threshold(x.scalar);
        float scale = 1.0f / (1.0f - x.scalar);
        push([=](hipStream_t s) { hk::dropout(s, F(a), F(id), count, I(tok), seed, threshold, scale); });
        break;
      }
      case Op::Count_: break;
    }
    if (pending.size() > first_pending) {
      pending.back().flop = flop;
      pending.back().bytes = bytes;
    }
    // A GEMM operand from a producer that writes no f16 copy (attention, its gradients, the
    // cross-entropy gradient, the masked-row scatter, an input written before the plan runs): a
    // rounding pass right after the launch that wrote it.
    // (Ops whose value is written by a launch at or before their own place in the plan.)
    const bool round_after = x.op == Op::Attention || x.op == Op::AttentionGradQ || x.op == Op::AttentionGradK ||
                             x.op == Op::AttentionGradV || x.op == Op::CrossEntropyGrad || x.op == Op::LayerNorm ||
                             x.op == Op::DropoutGrad || x.op == Op::EmbeddingGrad || x.op == Op::Add ||
                             x.op == Op::Sub || x.op == Op::Mul || x.op == Op::Gelu || x.op == Op::GeluGrad ||
                             x.op == Op::Dropout || x.op == Op::Embedding || (x.op == Op::Input && !is_moment_input(x.name));
    if (round_after && (token_.count(id) || x.op == Op::Input) && gemm_operands.count(id) && !token16_.count(id) &&
        want16(int64_t(id))) {
      const int64_t rows = x.ty.shape[0], cols = x.ty.shape[1], ld = ld_of(id);
      pending.push_back({[=] {
        return Launch{"RoundF16 %" + std::to_string(id), [=](hipStream_t s) { hk::to_f16_rows(s, F(id), ld, H16(id), ld, rows, cols); }};
      }});
      pending.back().bytes = 6.0 * double(rows * cols);
    }
  }
  // GEMM chains: Add(..Add(Add(X, A1 B1), A2 B2).., An Bn), each product a GEMM of one shape and
  // configuration whose sum only the next Add reads, is one GEMM over the concatenated K (the
  // K tiles of segment s read As and Bs in place) with X added in its epilogue, at the last
  // GEMM's place. The sum is one contraction instead of n rounded partial products: within the
  // per-kernel tolerance of the reference's order, not bit-identical to it. (The backward of the
  // Q, K and V projections: the three input gradients added into the residual gradient.)
  {
    auto chainable = [&](const GemmJob& j) {
      return j.epi.node != j.id && j.epi.act == hk::EPI_NONE && j.bias_id < 0 && j.cs_id < 0 && !j.ws &&
             !j.ce_part && !j.ce_tab && j.segs.empty() && !j.g.defer && !j.g.h16 && j.g.k % 32 == 0 &&
             hk::gemm_split_for(j.g.m, j.g.n, j.g.k, false, j.g.h16) == 1;
    };
    auto same = [](const hk::GemmArgs& a, const hk::GemmArgs& b) {
      return a.m == b.m && a.n == b.n && a.k == b.k && a.lda == b.lda && a.ldb == b.ldb && a.ldc == b.ldc &&
             a.ta == b.ta && a.tb == b.tb && a.pad_a == b.pad_a && a.pad_b == b.pad_b && a.pad_c == b.pad_c &&
             a.h16 == b.h16;
    };
    std::vector<bool> gone(pending.size(), false);
    for (size_t i = 0; i < pending.size(); ++i) {
      if (gone[i] || pending[i].gemm.size() != 1 || pending[i].side) continue;
      const GemmJob& head = *pending[i].gemm[0];
      if (!chainable(head) || head.epi.drop >= 0) continue;
      std::vector<size_t> chain{i};
      while (chain.size() < size_t(hk::kGemmGroupMax)) {
        const GemmJob& cur = *pending[chain.back()].gemm[0];
        if (cur.epi.drop >= 0 || consumers[p.pos.at(cur.out_id)].size() != 1) break;
        size_t nxt = SIZE_MAX;
        for (size_t j = chain.back() + 1; j < pending.size() && nxt == SIZE_MAX; ++j)
          if (!gone[j] && pending[j].gemm.size() == 1 && !pending[j].side && chainable(*pending[j].gemm[0]) &&
              pending[j].gemm[0]->epi.aux == int64_t(cur.out_id) && same(pending[j].gemm[0]->g, head.g))
            nxt = j;
        if (nxt == SIZE_MAX) break;
        chain.push_back(nxt);
      }
      if (chain.size() < 2) continue;
      auto job = std::make_shared<GemmJob>(*pending[chain.back()].gemm[0]);
      job->asrc = head.asrc;
      job->bsrc = head.bsrc;
      job->epi.aux = head.epi.aux;
      job->g.k = head.g.k * int64_t(chain.size());
      job->what = head.what;
      Pending merged = pending[chain.back()];
      merged.flop = 0;
      merged.bytes = 0;
      for (size_t c = 0; c < chain.size(); ++c) {
        const GemmJob& m = *pending[chain[c]].gemm[0];
        if (c > 0) {
          job->segs.push_back({m.asrc, m.bsrc});
          job->what += " (+) " + m.what.substr(m.what.find('%'));
        }
        merged.flop += pending[chain[c]].flop;
        merged.bytes += pending[chain[c]].bytes;
        if (c + 1 < chain.size()) gone[chain[c]] = true;
      }
      merged.gemm = {job};
      merged.make = gemm_launch({job});
      pending[chain.back()] = merged;
    }
    std::vector<Pending> kept;
    for (size_t i = 0; i < pending.size(); ++i)
      if (!gone[i]) kept.push_back(pending[i]);
    pending = std::move(kept);
  }
  // GEMM groups: like GEMMs (one shape and configuration, split-K slices only by deferral) that
  // read nothing the others write run as one launch. Main-stream GEMMs group when adjacent in the
  // launch order (the group takes the first one's place: nothing runs between them). Side-stream
  // GEMMs, whose outputs only the optimizer reads, group with later ones up to the join and take
  // the last one's place (every member's operands exist there; the arena reuses no buffer within
  // a step). The Q, K and V projections of a layer and their weight gradients are such groups.
  {
    auto like = [](const GemmJob& x, const GemmJob& y) {
      const hk::GemmArgs &a = x.g, &b = y.g;
      const int split = hk::gemm_split_for(a.m, a.n, a.k, a.defer, a.h16);
      return a.m == b.m && a.n == b.n && a.k == b.k && a.lda == b.lda && a.ldb == b.ldb && a.ldc == b.ldc &&
             a.ta == b.ta && a.tb == b.tb && a.sum_a == b.sum_a && a.defer == b.defer && a.pad_a == b.pad_a &&
             a.pad_b == b.pad_b && a.pad_c == b.pad_c && a.h16 == b.h16 && x.epi.act == y.epi.act &&
             (x.bias_id >= 0) == (y.bias_id >= 0) && (x.cs_id >= 0) == (y.cs_id >= 0) &&
             (x.epi.node != x.id) == (y.epi.node != y.id) && (x.ws != nullptr) == (y.ws != nullptr) &&
             (split == 1 || a.defer) && !x.ce_part && !x.ce_tab && !y.ce_part && !y.ce_tab && x.epi.drop < 0 &&
             y.epi.drop < 0 && x.segs.empty() && y.segs.empty();
    };
    auto reads = [](const GemmJob& j) {
      std::vector<int64_t> r{int64_t(j.asrc), int64_t(j.bsrc), j.bias_id};
      if (j.epi.node != j.id) r.push_back(j.epi.aux);
      return r;
    };
    auto writes = [](const GemmJob& j) {
      std::vector<int64_t> w{int64_t(j.out_id), j.cs_id};
      if (j.epi.node != j.id) w.push_back(int64_t(j.id));
      return w;
    };
    auto independent = [&](const std::vector<std::shared_ptr<GemmJob>>& group, const GemmJob& y) {
      for (auto& x : group) {
        for (int64_t w : writes(*x))
          for (int64_t r : reads(y))
            if (w >= 0 && w == r) return false;
        for (int64_t w : writes(y))
          for (int64_t r : reads(*x))
            if (w >= 0 && w == r) return false;
      }
      return true;
    };
    std::vector<Pending> merged;
    std::vector<bool> taken(pending.size(), false);
    for (size_t i = 0; i < pending.size(); ++i) {
      if (taken[i]) continue;
      Pending pd = pending[i];
      if (pd.gemm.size() == 1 && !pd.side) {
        size_t j = i + 1;
        while (j < pending.size() && pd.gemm.size() < size_t(hk::kGemmGroupMax) && pending[j].gemm.size() == 1 &&
               !pending[j].side && like(*pd.gemm[0], *pending[j].gemm[0]) && independent(pd.gemm, *pending[j].gemm[0])) {
          pd.gemm.push_back(pending[j].gemm[0]);
          pd.flop += pending[j].flop;
          pd.bytes += pending[j].bytes;
          taken[j++] = true;
        }
      } else if (pd.gemm.size() == 1 && pd.side) {
        // Later like side GEMMs join this one; the group runs at the last member's place.
        size_t last = i;
        for (size_t j = i + 1; j < pending.size() && pd.gemm.size() < size_t(hk::kGemmGroupMax); ++j)
          if (!taken[j] && pending[j].gemm.size() == 1 && pending[j].side && like(*pd.gemm[0], *pending[j].gemm[0]) &&
              independent(pd.gemm, *pending[j].gemm[0])) {
            pd.gemm.push_back(pending[j].gemm[0]);
            pd.flop += pending[j].flop;
            pd.bytes += pending[j].bytes;
            taken[j] = true;
            last = j;
          }
        if (last != i) {
          pd.make = gemm_launch(pd.gemm);
          // Re-insert at the last member's place: mark it and emit when the scan reaches it.
          pending[last] = pd;
          taken[last] = false;
          continue;
        }
      }
      if (pd.gemm.size() > 1) pd.make = gemm_launch(pd.gemm);
      merged.push_back(pd);
    }
    pending = std::move(merged);
  }
  // Mixed precision: a GEMM output that only k_gemm_lds16 launches read (as operands, or the
  // column sums they take) is kept as its f16 copy alone: its producer (itself on k_gemm_lds16)
  // writes no f32 value, and its readers get no f32 pointer for it, so that any other kernel
  // refuses the problem loudly.
  if (mixed_twins && !s_.opt_.plan_only) {
    auto has16 = [&](uint32_t v) { return token16_.count(v) || fixed16_.count(v); };
    std::map<uint32_t, GemmJob*> job_of;   // MatMul node -> its GEMM job
    std::map<int64_t, GemmJob*> sums_of;  // fused SumRows node -> its GEMM job
    std::map<uint32_t, GemmJob*> producer;
    std::set<const GemmJob*> certain;     // jobs whose launch runs k_gemm_lds16
    for (auto& pd : pending) {
      bool all = !pd.gemm.empty();
      for (auto& j : pd.gemm)
        all = all && j->segs.empty() && has16(j->asrc) && has16(j->bsrc) && hk::gemm_lds16_fits(j->g);
      for (auto& j : pd.gemm) {
        const Node& jn = p.node(j->id);
        job_of[jn.op == Op::AddRows ? jn.operands[0] : j->id] = j.get();
        if (j->cs_id >= 0) sums_of[j->cs_id] = j.get();
        producer[j->out_id] = j.get();
        if (all) certain.insert(j.get());
      }
    }
    auto gemm_only = [&](uint32_t v) {
      if (outputs.count(v) || grad_values_pre.count(v) || !has16(v)) return false;
      std::vector<size_t> readers = consumers[p.pos.at(v)];
      for (size_t r = 0; r < readers.size(); ++r) {
        const Node& c = p.nodes[readers[r]];
        if (c.op == Op::Transpose && folded.count(c.id)) {
          for (auto c2 : consumers[readers[r]]) readers.push_back(c2);
          continue;
        }
        // A fused LayerNorm reads its GEMM-produced addend as its f16 copy only (the Add, or the
        // Dropout of it, that the pass applies).
        {
          bool ln_reads = false;
          for (auto& [lid, bvv] : ln_b16) {
            const LnFused& f = ln_fused.at(lid);
            ln_reads = ln_reads || (bvv == v && (int64_t(c.id) == f.add || int64_t(c.id) == f.din));
          }
          if (ln_reads) continue;
        }
        // The f16 attention reads q, k, v and the output gradient as their f16 copies only.
        if (flash(c) && (c.operands[0] == v || c.operands[1] == v || c.operands[2] == v ||
                         (c.op != Op::Attention && c.operands[4] == v)) && c.operands[3] != v)
          continue;
        GemmJob* j = nullptr;
        if (c.op == Op::MatMul && job_of.count(c.id)) j = job_of.at(c.id);
        if (c.op == Op::SumRows && sums_of.count(c.id)) j = sums_of.at(c.id);
        if (!j || !certain.count(j) || j->bias_id == int64_t(v) || (j->epi.node != j->id && j->epi.aux == int64_t(v)))
          return false;
        if (j->asrc != v && j->bsrc != v) return false;
      }
      return !readers.empty();
    };
    // A pre-activation written by an activation epilogue and read only by activation-gradient
    // epilogues (the GELU of the FFN and its gradient) is kept as f16 alone, as an f16 forward
    // would have kept its input.
    std::map<uint32_t, GemmJob*> epi_writer;  // epilogue consumer node -> its GEMM job
    for (auto& pd : pending)
      for (auto& j : pd.gemm)
        if (j->epi.node != j->id) epi_writer[j->epi.node] = j.get();
    for (auto& pd : pending)
      for (auto& jp : pd.gemm) {
        GemmJob* j = jp.get();
        if ((j->epi.act != hk::EPI_GELU && j->epi.act != hk::EPI_RELU) || j->pre16 || j->g.ldc % 4) continue;
        const uint32_t pv = j->id;
        if (outputs.count(pv) || grad_values_pre.count(pv)) continue;
        std::vector<GemmJob*> grads;
        bool ok = true;
        for (auto r : consumers[p.pos.at(pv)]) {
          const Node& cn = p.nodes[r];
          if (cn.id == j->epi.node) continue;
          auto w = epi_writer.find(cn.id);
          const bool fused_grad = (cn.op == Op::GeluGrad || cn.op == Op::ReluGrad) && w != epi_writer.end() &&
                                  (w->second->epi.act == hk::EPI_GELU_GRAD || w->second->epi.act == hk::EPI_RELU_GRAD) &&
                                  w->second->epi.aux == int64_t(pv) && w->second->g.ldc == j->g.ldc;
          if (!fused_grad) { ok = false; break; }
          grads.push_back(w->second);
        }
        if (!ok || grads.empty()) continue;
        if (!token16_.count(pv)) token16_[pv] = arena_.reserve(size_t(j->g.m * j->g.ldc) * 2);
        j->pre16 = true;
        for (GemmJob* gj : grads) gj->pre16 = true;
      }
    std::set<uint32_t> only16;
    for (auto& [v, j] : producer)
      if (j->c16 && certain.count(j) && !j->ws && gemm_only(v)) only16.insert(v);
    // The same for a LayerNorm backward's second output (the dropout gradient of its dx) and the
    // f16 attention's outputs and gradients that only f16 kernels read: their launches write the
    // f16 copy alone.
    for (uint32_t v : ln_posts)
      if (gemm_only(v)) {
        only16.insert(v);
        only16_.insert(v);
      }
    for (auto& pd : pending)
      for (auto& j : pd.gemm) {
        if (only16.count(j->out_id)) {
          j->c32 = false;
          j->what += " (f16 only)";
        }
        if (only16.count(j->asrc)) j->a32 = false;
        if (only16.count(j->bsrc)) j->b32 = false;
      }
  }
  // The reductions only the optimizer reads (LayerNorm gamma and beta sums, split-K weight
  // gradients and their bias sums), in one launch; in the AdamW launch itself when every one is a
  // gradient held in the arena and no loss scaling sits between them (finalize_adamw).
  bool fuse_finalize = s_.opt_.fuse_optimizer && is_step_ && !deferred.empty() && deferred.size() <= size_t(hk::kColumnJobs) &&
                       st.rule == Rule::AdamW && !st.updates.empty() && !s_.scaler_;
  if (fuse_finalize) {
    std::set<uint32_t> in_arena;
    for (auto& [param, g] : st.gradients)
      if (fixed_.count(g) && fixed_.at(g) == static_cast<void*>(s_.grad_ + s_.offset_[param])) in_arena.insert(g);
    for (auto& d : deferred)
      for (int64_t o : {d.lo, d.hi})
        if (o >= 0 && !in_arena.count(uint32_t(o))) fuse_finalize = false;
  }
  // The loss launch joins the optimizer launch as one more block.
  std::function<hk::CeLossJob()> loss_tail;
  std::string loss_what;
  if (fuse_finalize) {
    size_t tails = 0;
    for (auto& pd : pending) tails += pd.loss_tail ? 1 : 0;
    if (tails == 1)
      for (size_t q = 0; q < pending.size(); ++q)
        if (pending[q].loss_tail) {
          loss_tail = pending[q].loss_tail;
          loss_what = pending[q].make().what;
          pending.erase(pending.begin() + std::ptrdiff_t(q));
          break;
        }
  }
  const size_t join_at = pending.size();
  double finalize_bytes = 0;
  for (auto& d : deferred) finalize_bytes += 4.0 * double(int64_t(d.chunks) * d.width + d.width);
  auto finalize_jobs = [deferred, F, A] {
    std::vector<hk::ColumnJob> jobs;
    for (auto& d : deferred)
      jobs.push_back({static_cast<float*>(A(d.tok)) + d.offset, d.lo >= 0 ? F(uint32_t(d.lo)) : nullptr,
                      d.hi >= 0 ? F(uint32_t(d.hi)) : nullptr, d.chunks, d.width, d.split, 0});
    return jobs;
  };
  if (!deferred.empty() && !fuse_finalize) {
    std::string what = "ColumnFinalize x" + std::to_string(deferred.size());
    const double bytes = finalize_bytes;
    pending.push_back({[what, finalize_jobs] {
                         return Launch{what, [finalize_jobs](hipStream_t s) {
                                         const std::vector<hk::ColumnJob> jobs = finalize_jobs();
                                         hk::column_finalize(s, jobs.data(), int(jobs.size()));
                                       }};
                       },
                       0, bytes});
  }
  // The optimizer: gradients not computed in place are copied into the arena, then one launch
  // updates every trained parameter and its moments.
  if (is_step_) {
    for (auto [g, param] : grad_copies) {
      int64_t cnt = p.node(g).ty.count();
      float* dst = s_.grad_ + s_.offset_[param];
      pending.push_back({[=] { return Launch{"GradientCopy", [=](hipStream_t s) { hk::copy(s, F(g), dst, cnt); }}; }});
    }
    int64_t nt = s_.trained_;
    if (st.rule == Rule::AdamW && !st.updates.empty()) {
      float k[6];
      st.adamw.constants(k);
      hk::AdamWConsts c{k[0], k[1], k[2], k[3], k[4], k[5]};
      uint32_t lr = *st.lr_t, c1 = *st.c1, c2 = *st.c2;
      hk::LossScaleState* ls = s_.scaler_;
      if (ls) {
        pending.push_back({[=] { return Launch{"GradCheck", [=](hipStream_t s) { hk::grad_check(s, s_.grad_, nt, ls); }}; }});
        pending.back().bytes = 4.0 * double(nt);
      }
      if (fuse_finalize) {
        const std::string what =
            "ColumnFinalize x" + std::to_string(deferred.size()) + " + AdamW" + (loss_tail ? " + " + loss_what : "");
        pending.push_back({[=] {
          return Launch{what, [=](hipStream_t s) {
                          const std::vector<hk::ColumnJob> jobs = finalize_jobs();
                          hk::CeLossJob tail{};
                          if (loss_tail) tail = loss_tail();
                          hk::finalize_adamw(s, jobs.data(), int(jobs.size()), s_.param_, s_.grad_, s_.m_, s_.v_, nt, c,
                                             F(lr), F(c1), F(c2), loss_tail ? &tail : nullptr);
                        }};
        }});
        pending.back().bytes = finalize_bytes + 7.0 * 4.0 * double(nt);
      } else {
        // Mixed precision: the launch writes the parameters' f16 copies as it updates them.
        pending.push_back({[=] {
          return Launch{"AdamW", [=](hipStream_t s) {
                          hk::adamw(s, s_.param_, s_.grad_, s_.m_, s_.v_, nt, c, F(lr), F(c1), F(c2), ls, s_.param16_);
                        }};
        }});
        pending.back().bytes = (7.0 * 4.0 + (s_.opt_.mixed ? 2.0 : 0.0)) * double(nt);
      }
      if (ls) pending.push_back({[=] { return Launch{"LossScale", [=](hipStream_t s) { hk::loss_scale_update(s, ls); }}; }});
      if (fuse_finalize && (s_.param16_ || (s_.opt_.plan_only && s_.opt_.mixed))) {
        pending.push_back({[=] {
          return Launch{"ParamF16", [=](hipStream_t s) { hk::to_f16_rows(s, s_.param_, nt, s_.param16_, nt, 1, nt); }};
        }});
        pending.back().bytes = 6.0 * double(nt);
      }
    } else if (st.rule == Rule::Sgd && !st.updates.empty()) {
      uint32_t rate = p.node(st.updates.begin()->second).operands[1];
      uint32_t lr_scalar = p.node(rate).operands[0];
      hk::LossScaleState* ls = s_.scaler_;
      if (ls) pending.push_back({[=] { return Launch{"GradCheck", [=](hipStream_t s) { hk::grad_check(s, s_.grad_, nt, ls); }}; }});
      pending.push_back({[=] { return Launch{"SGD", [=](hipStream_t s) { hk::sgd(s, s_.param_, s_.grad_, nt, F(lr_scalar), ls); }}; }});
      if (ls) pending.push_back({[=] { return Launch{"LossScale", [=](hipStream_t s) { hk::loss_scale_update(s, ls); }}; }});
    }
    loss_value = st.loss;
    uint32_t loss = st.loss;
    if (!loss_logged)
      pending.push_back({[=] {
        return Launch{"RecordLoss", [=](hipStream_t s) { hk::record_loss(s, F(loss), s_.losses_dev_, s_.counter_, s_.loss_capacity_); }};
      }});
  } else {
    loss_value = p.outputs.at(0);
  }

  if (!s_.opt_.plan_only) {
    arena_.commit();
    for (auto& [vid, val] : constants) hip_check(hipMemcpy(ptr(vid), &val, 4, hipMemcpyHostToDevice), "hipMemcpy (constants)");
    for (auto& slot : inputs_) fixed_[slot.id] = static_cast<char*>(arena_.at(input_token_)) + slot.offset;
  }
  for (auto& pd : pending) {
    launches_.push_back(pd.make());
    launches_.back().flop = pd.flop;
    launches_.back().bytes = pd.bytes;
    launches_.back().side = pd.side;
    launches_.back().pure = pd.pure;
  }
  join_at_ = join_at;
}

std::string Executor::plan_text() const {
  std::string out;
  size_t k = 0;
  for (auto& l : launches_) {
    char work[96];
    std::snprintf(work, sizeof work, " flop %.0f bytes %.0f", l.flop, l.bytes);
    out += "  " + std::to_string(k++) + ": " + l.what + (l.side ? " [side]" : "") + work + "\n";
  }
  std::vector<std::pair<size_t, uint32_t>> slices;
  for (auto& [vid, tok] : token_) slices.push_back({DeviceArena::offset(tok), vid});
  std::sort(slices.begin(), slices.end());
  out += "  arena " + std::to_string(arena_.bytes()) + " bytes, " + std::to_string(slices.size()) + " values";
  for (auto& [off, vid] : slices) out += " %" + std::to_string(vid) + "@" + std::to_string(off);
  out += "\n";
  return out;
}

void Executor::stage(const Batch& batch) {
  auto fed = [&](const std::string& name) {
    for (auto& in : inputs_)
      if (in.device && in.name == name) return true;
    return false;
  };
  // The checks the reference makes before a step reads an id (interpreter.rs:700-715,
  // 1146-1262): ids inside their table, labels inside the classes, weights finite and not
  // negative, key masks of 0 and 1 with a 1 in every sequence.
  for (auto& [key, rows] : id_bounds_) {
    if (key.rfind("#weights:", 0) == 0) {
      auto it = batch.f32.find(key.substr(9));
      if (it == batch.f32.end() || fed(key.substr(9))) continue;
      for (size_t r = 0; r < it->second.size(); ++r) {
        float w = it->second[r];
        if (!(w * 0.0f == 0.0f) || w < 0.0f) throw IrError("loss weight " + std::to_string(r) + " is negative or not finite");
      }
      continue;
    }
    bool label = key.rfind("#labels:", 0) == 0;
    std::string name = label ? key.substr(8) : key;
    if (fed(name)) continue;
    auto it = batch.i32.find(name);
    if (it == batch.i32.end()) continue;
    for (size_t r = 0; r < it->second.size(); ++r) {
      int32_t v = it->second[r];
      if (v < 0 || v >= rows)
        throw IrError("E-DATA-011: `" + name + "` holds " + std::to_string(v) + " at " + std::to_string(r) + ", outside [0, " +
                      std::to_string(rows) + ")");
    }
  }
  for (auto& name : key_masks_) {
    auto it = batch.f32.find(name);
    if (it == batch.f32.end() || fed(name)) continue;
    const Node* in = p_.input(name);
    int64_t S = in->ty.shape[1];
    for (size_t b = 0; b * size_t(S) < it->second.size(); ++b) {
      bool any = false;
      for (int64_t j = 0; j < S; ++j) {
        float m = it->second[b * size_t(S) + size_t(j)];
        if (m != 0.0f && m != 1.0f) throw IrError("key mask `" + name + "` holds a value other than 0 and 1");
        any = any || m == 1.0f;
      }
      if (!any) throw IrError("key mask `" + name + "`: sequence " + std::to_string(b) + " has no unmasked key");
    }
  }
  int slot = next_slot_;
  next_slot_ = (next_slot_ + 1) % kRing;
  hip_check(hipEventSynchronize(slot_done_[slot]), "hipEventSynchronize (staging slot)");
  char* host = static_cast<char*>(pinned_[slot]);
  if (s_.corpus_) {
    auto it = batch.i32.find(kDrawInput);
    if (it == batch.i32.end() || it->second.size() != 3 + s_.corpus_batch_)
      throw IrError(std::string("a step on a packed corpus takes `") + kDrawInput + "` of " +
                    std::to_string(3 + s_.corpus_batch_) + " words");
    std::memcpy(host + draw_offset_, it->second.data(), it->second.size() * 4);
  }
  for (auto& in : inputs_) {
    if (in.device) continue;
    const void* src = nullptr;
    size_t have = 0;
    if (in.dtype == DType::F32) {
      auto it = batch.f32.find(in.name);
      if (it != batch.f32.end()) { src = it->second.data(); have = it->second.size(); }
    } else {
      auto it = batch.i32.find(in.name);
      if (it != batch.i32.end()) { src = it->second.data(); have = it->second.size(); }
    }
    if (!src && in.count > 0) throw IrError("missing input `" + in.name + "`");
    if (int64_t(have) != in.count) throw IrError("input `" + in.name + "` has " + std::to_string(have) + " elements, not " + std::to_string(in.count));
    std::memcpy(host + in.offset, src, size_t(in.count) * 4);
  }
  for (auto& ps : plan_slots_) {
    auto it = batch.i32.find(ps.ids_name);
    if (it == batch.i32.end() || int64_t(it->second.size()) != ps.n) throw IrError("missing input `" + ps.ids_name + "`");
    hk::eg_plan_host(it->second.data(), ps.n, ps.rows, reinterpret_cast<int32_t*>(host + ps.offset));
  }
  if (host_bytes_) {
    hip_check(hipMemcpyAsync(arena_.at(input_token_), host, host_bytes_, hipMemcpyHostToDevice, s_.stream_), "hipMemcpyAsync (inputs)");
    s_.stats_.bytes_uploaded += host_bytes_;
  }
  hip_check(hipEventRecord(slot_done_[slot], s_.stream_), "hipEventRecord");
}

void Executor::run(hipStream_t s) {
  // Side launches are held and issued on the side stream eight at a time, forked from the main
  // stream's work so far; the main stream joins them at the first launch after the backward and
  // at the end (under capture these are graph edges, not nodes). Each fork and join is a wait
  // across hardware queues, which costs about what a small launch does: forking every weight
  // gradient on its own was measured slower than the single stream on BERT-tiny, eight at a time
  // faster on BERT-tiny and BERT-base.
  constexpr size_t kSideBatch = 8;
  bool open = false;
  std::vector<const Launch*> held;
  auto flush = [&] {
    if (held.empty()) return;
    hip_check(hipEventRecord(s_.fork_, s), "hipEventRecord (fork)");
    hip_check(hipStreamWaitEvent(s_.side_, s_.fork_, 0), "hipStreamWaitEvent (fork)");
    for (auto* l : held) l->run(s_.side_);
    held.clear();
    open = true;
  };
  auto join = [&] {
    flush();
    hip_check(hipEventRecord(s_.join_, s_.side_), "hipEventRecord (join)");
    hip_check(hipStreamWaitEvent(s, s_.join_, 0), "hipStreamWaitEvent (join)");
    open = false;
  };
  for (size_t i = 0; i < launches_.size(); ++i) {
    const Launch& l = launches_[i];
    if ((open || !held.empty()) && i >= join_at_) join();
    if (l.side && s_.side_) {
      held.push_back(&l);
      if (held.size() >= kSideBatch) flush();
    } else {
      l.run(s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw HipError(l.what + ": " + hipGetErrorString(e));
  }
  if (open || !held.empty()) join();
}

// ---------------------------------------------------------------------------------------------
Session::DeviceCorpus::~DeviceCorpus() {
  if (mem) (void)hipFree(mem);
}

bool Session::corpus_fed(const Program& p, const std::string& name) const {
  if (!corpus_) return false;
  for (const char* t : kBatchTensors)
    if (name == t) return true;
  return name == kMaskedRowsInput || name.rfind(kMaskedLabelsPrefix, 0) == 0 || name.rfind(kMaskedWeightsPrefix, 0) == 0;
}

hk::LossScaleState Session::loss_scale() {
  hk::LossScaleState out{};
  if (!scaler_) return out;
  sync();
  hip_check(hipMemcpy(&out, scaler_, sizeof out, hipMemcpyDeviceToHost), "hipMemcpy (loss scale)");
  return out;
}

void Session::check_data_error() {
  if (!corpus_) return;
  uint32_t e[4] = {};
  hip_check(hipMemcpy(e, corpus_->error, sizeof e, hipMemcpyDeviceToHost), "hipMemcpy (gather error)");
  if (!e[0]) return;
  const uint64_t draw = uint64_t(e[2]) | (uint64_t(e[3]) << 32);
  const bool held = draw >> 63;
  throw IrError(std::string("E-DATA-012: the batch of ") + (held ? "held-out batch " : "step ") +
                std::to_string(held ? draw - (uint64_t(1) << 63) : draw) + " has " + std::to_string(e[1]) +
                " rows of non-zero weight, more than the rows the masked-row gather holds");
}

Session::Session(int device, const TrainingStep& step, const Program& forward, uint64_t seed, uint32_t prediction,
                 const PackedCorpus* corpus, SessionOptions options)
    : device_(device), step_(step), forward_(forward), seed_(seed), prediction_(prediction), opt_(options) {
  step_.program.reindex();
  forward_.reindex();
  if (opt_.plan_only) {
    // No device: the plans only. Parameter, gradient and moment slices are offsets from a null
    // base, never dereferenced.
    if (corpus) throw IrError("a plan-only session takes no packed corpus");
    const auto& params = step_.program.params;
    offset_.assign(params.size(), 0);
    int64_t at = 0;
    for (int pass = 0; pass < 2; ++pass) {
      for (size_t q = 0; q < params.size(); ++q) {
        if ((step_.updates.count(uint32_t(q)) != 0) != (pass == 0)) continue;
        offset_[q] = at;
        at += (params[q].ty.count() + 63) / 64 * 64;
      }
      if (pass == 0) trained_ = at;
    }
    total_ = std::max<int64_t>(at, 64);
    if (step_.has_optimizer) step_exec_ = std::make_unique<Executor>(*this, step_.program, true);
    fwd_exec_ = std::make_unique<Executor>(*this, forward_, false);
    return;
  }
  hip_check(hipSetDevice(device), "hipSetDevice");
  hk::prepare();
  if (corpus) {
    // Both splits resident in HBM for the whole run, and the four error words behind them.
    corpus_batch_ = bind_corpus(forward_, *corpus);
    corpus_ = std::make_unique<DeviceCorpus>();
    const size_t tb = corpus->train.size() * 4, hb = corpus->heldout.size() * 4;
    const size_t hoff = (tb + 255) / 256 * 256, eoff = hoff + (hb + 255) / 256 * 256;
    hip_check(hipMalloc(&corpus_->mem, eoff + 256), "hipMalloc (packed corpus)");
    char* base = static_cast<char*>(corpus_->mem);
    hip_check(hipMemcpy(base, corpus->train.data(), tb, hipMemcpyHostToDevice), "hipMemcpy (train split)");
    hip_check(hipMemcpy(base + hoff, corpus->heldout.data(), hb, hipMemcpyHostToDevice), "hipMemcpy (held-out split)");
    hip_check(hipMemset(base + eoff, 0, 256), "hipMemset (gather error)");
    const MaskingThresholds t = masking_thresholds(corpus->policy);
    corpus_->c = hk::MlmCorpus{reinterpret_cast<const int32_t*>(base), reinterpret_cast<const int32_t*>(base + hoff),
                               int64_t(corpus->seq_len), seed, t.select, t.mask, t.mask_or_random,
                               corpus->vocabulary_size - kSpecialTokens};
    corpus_->error = reinterpret_cast<uint32_t*>(base + eoff);
    stats_.device_bytes += eoff + 256;
  }
  hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  if (!std::getenv("MSX_NO_SIDE_STREAM"))
    hip_check(hipStreamCreateWithFlags(&side_, hipStreamNonBlocking), "hipStreamCreate (side)");
  if (std::getenv("MSX_NO_GRAPH")) use_graph_ = false;
  hip_check(hipEventCreateWithFlags(&fork_, hipEventDisableTiming), "hipEventCreate (fork)");
  hip_check(hipEventCreateWithFlags(&join_, hipEventDisableTiming), "hipEventCreate (join)");
  const auto& params = step_.program.params;
  offset_.assign(params.size(), 0);
  int64_t at = 0;
  for (int pass = 0; pass < 2; ++pass) {
    for (size_t q = 0; q < params.size(); ++q) {
      bool trained = step_.updates.count(uint32_t(q)) != 0;
      if (trained != (pass == 0)) continue;
      offset_[q] = at;
      at += (params[q].ty.count() + 63) / 64 * 64;
    }
    if (pass == 0) trained_ = at;
  }
  total_ = std::max<int64_t>(at, 64);
  size_t floats = size_t(total_) * 4 + loss_capacity_ + 64;
  hip_check(hipMalloc(&state_mem_, floats * 4), "hipMalloc (parameter state)");
  hip_check(hipMemset(state_mem_, 0, floats * 4), "hipMemset (parameter state)");
  float* base = static_cast<float*>(state_mem_);
  param_ = base;
  grad_ = base + total_;
  m_ = base + 2 * total_;
  v_ = base + 3 * total_;
  losses_dev_ = base + 4 * total_;
  counter_ = reinterpret_cast<uint32_t*>(base + 4 * total_ + loss_capacity_);
  if (opt_.mixed) {
    hip_check(hipMalloc(&param16_, size_t(total_) * 2), "hipMalloc (f16 parameters)");
    hip_check(hipMemset(param16_, 0, size_t(total_) * 2), "hipMemset (f16 parameters)");
    stats_.device_bytes += size_t(total_) * 2;
    // The loss-scale state, in device memory for the whole run (read and written by the step).
    hip_check(hipMalloc(&scaler_, sizeof(hk::LossScaleState)), "hipMalloc (loss scale)");
    hk::LossScaleState init{opt_.loss_scale, 1.0f / opt_.loss_scale, 0, 0, 0, opt_.scale_window, 0, 0};
    hip_check(hipMemcpy(scaler_, &init, sizeof init, hipMemcpyHostToDevice), "hipMemcpy (loss scale)");
  }
  if (step_.has_optimizer) step_exec_ = std::make_unique<Executor>(*this, step_.program, true);
  fwd_exec_ = std::make_unique<Executor>(*this, forward_, false);
  stats_.device_bytes += floats * 4;
}

Session::~Session() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  if (side_) (void)hipStreamSynchronize(side_);
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  step_exec_.reset();
  fwd_exec_.reset();
  corpus_.reset();
  if (scaler_) (void)hipFree(scaler_);
  if (param16_) (void)hipFree(param16_);
  if (state_mem_) (void)hipFree(state_mem_);
  if (eval_mem_) (void)hipFree(eval_mem_);
  if (fork_) (void)hipEventDestroy(fork_);
  if (join_) (void)hipEventDestroy(join_);
  if (side_) (void)hipStreamDestroy(side_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

const std::vector<Launch>& Session::plan(bool step) const {
  if (step && !step_exec_) throw IrError("no training step is loaded");
  return step ? step_exec_->launches() : fwd_exec_->launches();
}

size_t Session::launches_per_step() const { return step_exec_ ? step_exec_->launches().size() : 0; }

const void* Session::forward_value(uint32_t id) const { return fwd_exec_->value(id); }
const void* Session::step_value(uint32_t id) const {
  if (!step_exec_) throw IrError("no training step is loaded");
  return step_exec_->value(id);
}

void Session::run_forward(const Batch& batch) {
  fwd_exec_->stage(batch);
  fwd_exec_->run(stream_);
  sync();
}

void Session::sync() { hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }

void Session::upload_params(const std::vector<std::vector<float>>& values) {
  const auto& params = step_.program.params;
  if (values.size() != params.size()) throw IrError("set_params: wrong number of parameters");
  sync();
  for (size_t q = 0; q < params.size(); ++q) {
    if (int64_t(values[q].size()) != params[q].ty.count()) throw IrError("set_params: `" + params[q].path + "` has the wrong size");
    hip_check(hipMemcpy(param_ + offset_[q], values[q].data(), values[q].size() * 4, hipMemcpyHostToDevice), "hipMemcpy (params)");
  }
  if (param16_) {
    hk::to_f16_rows(stream_, param_, total_, param16_, total_, 1, total_);
    sync();
  }
}

void Session::set_params(const std::vector<std::vector<float>>& values) {
  upload_params(values);
  hk::fill_zero(stream_, grad_, total_ * 4);
  hk::fill_zero(stream_, m_, total_ * 4);
  hk::fill_zero(stream_, v_, total_ * 4);
  hk::fill_zero(stream_, counter_, 64 * 4);
  sync();
  steps_since_reset_ = 0;
}

std::vector<std::vector<float>> Session::params() {
  sync();
  std::vector<std::vector<float>> out;
  for (size_t q = 0; q < step_.program.params.size(); ++q) {
    std::vector<float> v(size_t(step_.program.params[q].ty.count()));
    hip_check(hipMemcpy(v.data(), param_ + offset_[q], v.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy (read params)");
    out.push_back(std::move(v));
  }
  return out;
}

std::vector<std::vector<float>> Session::moments(char which) {
  sync();
  std::vector<std::vector<float>> out(step_.program.params.size());
  for (auto& [q, mo] : step_.moments) {
    std::vector<float> v(size_t(step_.program.params[q].ty.count()));
    float* src = (which == 'm' ? m_ : v_) + offset_[q];
    hip_check(hipMemcpy(v.data(), src, v.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy (read moments)");
    out[q] = std::move(v);
  }
  return out;
}

void Session::set_moments(const std::vector<std::vector<float>>& m, const std::vector<std::vector<float>>& v) {
  sync();
  for (auto& [q, mo] : step_.moments) {
    const size_t n = size_t(step_.program.params[q].ty.count());
    for (int k = 0; k < 2; ++k) {
      const auto& src = k == 0 ? m : v;
      if (q >= src.size() || src[q].size() != n)
        throw IrError(std::string("set_moments: `") + step_.program.params[q].path + "` needs " + (k ? "v" : "m") +
                      " of " + std::to_string(n) + " values");
      hip_check(hipMemcpy((k == 0 ? m_ : v_) + offset_[q], src[q].data(), n * 4, hipMemcpyHostToDevice),
                "hipMemcpy (moments)");
    }
  }
}

std::vector<float> Session::predict(const std::vector<std::vector<float>>& values, const Batch& batch) {
  upload_params(values);
  fwd_exec_->stage(batch);
  fwd_exec_->run(stream_);
  sync();
  std::vector<float> out(size_t(forward_.node(prediction_).ty.count()));
  hip_check(hipMemcpy(out.data(), fwd_exec_->value(prediction_), out.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy (prediction)");
  return out;
}

void Session::train_step(const StepInputs& in) {
  step_exec_->stage(in.batch);
  if (use_graph_) {
    if (!graph_exec_) {
      hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
      try {
        step_exec_->run(stream_);
      } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      hip_check(hipStreamEndCapture(stream_, &graph_), "hipStreamEndCapture");
      hip_check(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
      size_t nodes = 0;
      hip_check(hipGraphGetNodes(graph_, nullptr, &nodes), "hipGraphGetNodes");
      stats_.kernels_per_step = nodes;
    }
    hip_check(hipGraphLaunch(graph_exec_, stream_), "hipGraphLaunch");
    stats_.graph_launches += 1;
  } else {
    step_exec_->run(stream_);
  }
  stats_.steps += 1;
  steps_since_reset_ += 1;
}

// Each launch of one eager step between its own pair of events on the step's stream; a pure
// launch is then run kRepeats more times back to back between a second pair, and its time is
// their mean (one launch's events also hold the dispatch gap before it, a repeat run amortizes it).
std::vector<Session::Timed> Session::profile_step(const StepInputs& in) {
  constexpr int kRepeats = 10;
  step_exec_->stage(in.batch);
  const auto& ls = step_exec_->launches();
  std::vector<hipEvent_t> ev(4 * ls.size());
  for (auto& e : ev) hip_check(hipEventCreate(&e), "hipEventCreate");
  std::vector<std::vector<std::string>> kernels(ls.size());
  for (size_t i = 0; i < ls.size(); ++i) {
    hip_check(hipEventRecord(ev[4 * i], stream_), "hipEventRecord");
    hk::kernel_log(&kernels[i]);
    ls[i].run(stream_);
    hk::kernel_log(nullptr);
    hip_check(hipEventRecord(ev[4 * i + 1], stream_), "hipEventRecord");
    if (ls[i].pure) {
      hip_check(hipEventRecord(ev[4 * i + 2], stream_), "hipEventRecord");
      for (int r = 0; r < kRepeats; ++r) ls[i].run(stream_);
      hip_check(hipEventRecord(ev[4 * i + 3], stream_), "hipEventRecord");
    }
  }
  sync();
  std::vector<Timed> out;
  for (size_t i = 0; i < ls.size(); ++i) {
    float ms = 0;
    if (ls[i].pure) {
      hip_check(hipEventElapsedTime(&ms, ev[4 * i + 2], ev[4 * i + 3]), "hipEventElapsedTime");
      ms /= kRepeats;
    } else {
      hip_check(hipEventElapsedTime(&ms, ev[4 * i], ev[4 * i + 1]), "hipEventElapsedTime");
    }
    std::string names;
    for (auto& kname : kernels[i]) names += (names.empty() ? "" : "+") + kname;
    out.push_back({ls[i].what, ms, ls[i].flop, ls[i].bytes, names, ls[i].pure ? 1 + kRepeats : 1});
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  stats_.steps += 1;
  steps_since_reset_ += 1;
  return out;
}

float Session::final_loss(const Batch& batch) {
  fwd_exec_->stage(batch);
  fwd_exec_->run(stream_);
  sync();
  check_data_error();
  float loss = 0;
  hip_check(hipMemcpy(&loss, fwd_exec_->value(fwd_exec_->loss_value), 4, hipMemcpyDeviceToHost), "hipMemcpy (loss)");
  return loss;
}

HeldOutSums Session::held_out(const HeldOut& h) { return held_out_in(h, false); }

HeldOutSums Session::held_out_static(const HeldOut& h) { return held_out_in(h, true); }

HeldOutSums Session::held_out_in(const HeldOut& h, bool no_alloc) {
  h.check_labels();
  const Node* lab = forward_.input(h.labels_name());
  const Node* w = forward_.input(h.weights_name());
  const Node& pred = forward_.node(prediction_);
  if (!lab || !w || lab->ty.dtype != DType::I32 || w->ty.dtype != DType::F32 || pred.ty.rank() != 2 ||
      pred.ty.shape[1] != h.classes() || pred.ty.shape[0] != lab->ty.count() || w->ty.count() != lab->ty.count())
    throw IrError("held-out evaluation: the forward program's prediction, labels and weights do not match");
  const int64_t rows = lab->ty.count(), v = h.classes();
  // Row results first, the state at the next 256-byte boundary behind them.
  const size_t state_at = (size_t(rows) * 8 + 255) / 256 * 256;
  float* row_out = nullptr;
  hk::HeldOutState* state = nullptr;
  std::unique_lock<std::mutex> scratch_lock;
  if (no_alloc) {
    if (rows > kStaticEvalRows)
      throw IrError("held-out evaluation without allocation: a batch of " + std::to_string(rows) + " rows exceeds " +
                    std::to_string(kStaticEvalRows));
    StaticScratch& sc = static_scratch(device_);
    // Held until the sums are read back: no other call on this device uses the array meanwhile.
    scratch_lock = std::unique_lock<std::mutex>(sc.use);
    char* base = static_cast<char*>(sc.ptr);
    row_out = reinterpret_cast<float*>(base);
    state = reinterpret_cast<hk::HeldOutState*>(base + kStaticStateAt);
  } else if (rows > eval_rows_) {
    sync();
    if (eval_mem_) hip_check(hipFree(eval_mem_), "hipFree (held-out)");
    eval_mem_ = nullptr;
    eval_rows_ = 0;
    hip_check(hipMalloc(&eval_mem_, state_at + 256), "hipMalloc (held-out)");
    eval_rows_ = rows;
  }
  if (!no_alloc) {
    row_out = static_cast<float*>(eval_mem_);
    state = reinterpret_cast<hk::HeldOutState*>(static_cast<char*>(eval_mem_) + state_at);
  }
  hk::fill_zero(stream_, state, sizeof(hk::HeldOutState));
  for (auto& batch : h.batches()) {
    fwd_exec_->stage(batch);
    fwd_exec_->run(stream_);
    hk::held_out_rows(stream_, static_cast<const float*>(fwd_exec_->value(prediction_)),
                      static_cast<const int32_t*>(fwd_exec_->value(lab->id)), row_out, rows, v, v);
    hk::held_out_sum(stream_, row_out, static_cast<const float*>(fwd_exec_->value(w->id)), rows, state);
  }
  sync();
  check_data_error();
  hk::HeldOutState got{};
  hip_check(hipMemcpy(&got, state, sizeof(got), hipMemcpyDeviceToHost), "hipMemcpy (held-out state)");
  HeldOutSums out;
  out.numerator = got.numerator;
  out.correct = uint64_t(got.correct);
  out.denominator = got.denominator;
  out.selected = uint64_t(got.selected);
  out.has_totals = true;
  return out;
}

std::string Session::plan_text() const {
  std::string out;
  if (step_exec_) out += "plan step (" + std::to_string(step_exec_->launches().size()) + " launches)\n" + step_exec_->plan_text();
  out += "plan forward (" + std::to_string(fwd_exec_->launches().size()) + " launches)\n" + fwd_exec_->plan_text();
  return out;
}

std::vector<float> Session::losses() {
  sync();
  uint32_t count = 0;
  hip_check(hipMemcpy(&count, counter_, 4, hipMemcpyDeviceToHost), "hipMemcpy (loss counter)");
  check_data_error();
  count = std::min(count, loss_capacity_);
  std::vector<float> out(count);
  if (count) hip_check(hipMemcpy(out.data(), losses_dev_, count * 4, hipMemcpyDeviceToHost), "hipMemcpy (losses)");
  return out;
}

}  // namespace msx
