// TEST INFRASTRUCTURE — the CPU oracle's engine and its C API (liboracle.so). Loaded only by
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker.
//
// The engine runs a compiled training step the way crates/modelspec-runtime/src/train/optimizer.rs
// (PreparedStep::evaluate_with_ids, Evaluated::apply, lines 137-151 and 443-520) does: evaluate the
// step program on the inputs, parameters and moments, then take each update and next moment as the
// new state.
#include <chrono>
#include <cstring>
#include <memory>

#include "../modelspec_amd/csrc/host/runner.h"
#include "interp.h"

namespace {
thread_local std::string g_error;

class OracleEngine : public msx::Engine {
 public:
  explicit OracleEngine(const msx::Compiled& c) : c_(c) {}

  void set_params(const std::vector<std::vector<float>>& values) override {
    params_ = values;
    m_.clear();
    v_.clear();
    for (auto& [param, mo] : c_.step.moments) {
      m_[param].assign(values[param].size(), 0.0f);
      v_[param].assign(values[param].size(), 0.0f);
    }
    losses_.clear();
  }
  std::vector<std::vector<float>> params() override { return params_; }
  std::vector<std::vector<float>> moments(char which) override {
    std::vector<std::vector<float>> out(params_.size());
    for (auto& [param, v] : which == 'm' ? m_ : v_) out[param] = v;
    return out;
  }
  std::vector<float> predict(const std::vector<std::vector<float>>& values, const msx::Batch& b) override {
    oracle::Interpreter it(c_.forward, true, c_.config.seed);
    it.run(b.f32, b.i32, values);
    return it.value(c_.prediction);
  }
  void train_step(const msx::StepInputs& in) override {
    const msx::TrainingStep& s = c_.step;
    auto f32 = in.batch.f32;
    for (auto& [param, mo] : s.moments) {
      const std::string& path = s.program.params[param].path;
      f32[msx::moment_input('m', path)] = m_[param];
      f32[msx::moment_input('v', path)] = v_[param];
    }
    oracle::Interpreter it(s.program, true, c_.config.seed);
    it.run(f32, in.batch.i32, params_);
    losses_.push_back(it.value(s.loss)[0]);
    for (auto& [param, u] : s.updates) params_[param] = it.value(u);
    for (auto& [param, mo] : s.moments) {
      m_[param] = it.value(mo.m_next);
      v_[param] = it.value(mo.v_next);
    }
  }
  float final_loss(const msx::Batch& b) override {
    oracle::Interpreter it(c_.forward, true, c_.config.seed);
    it.run(b.f32, b.i32, params_);
    return it.value(c_.forward.outputs[0])[0];
  }
  std::vector<float> losses() override { return losses_; }
  msx::HeldOutSums held_out(const msx::HeldOut& h) override {
    tally = tally_of(h, params_);
    return {tally.numerator, tally.correct};
  }
  // The forward program over every held-out batch on `values`, tallied (eval.rs:263-287).
  oracle::HeldOutTally tally_of(const msx::HeldOut& h, const std::vector<std::vector<float>>& values) const {
    oracle::HeldOutTally t;
    size_t b = 0;
    for (auto& batch : h.batches()) {
      oracle::Interpreter it(c_.forward, true, c_.config.seed);
      it.run(batch.f32, batch.i32, values);
      const auto& labels = batch.i32.at(h.labels_name());
      if (!t.add(it.value(c_.prediction).data(), labels.data(), batch.f32.at(h.weights_name()).data(), labels.size(),
                 size_t(h.classes())))
        throw msx::HeldOutLabelError("held-out batch " + std::to_string(b) + ": a label is not below the classes");
      ++b;
    }
    return t;
  }
  oracle::HeldOutTally tally;  // of the last held_out call

 private:
  const msx::Compiled& c_;
  std::vector<std::vector<float>> params_;
  std::map<uint32_t, std::vector<float>> m_, v_;
  std::vector<float> losses_;
};

struct Prog {
  msx::Program program;
  std::unique_ptr<oracle::Interpreter> interp;
  bool has_seed;
  uint64_t seed;
};
}  // namespace

extern "C" {

const char* orc_last_error() { return g_error.c_str(); }

// The host draws the oracle interprets with, for known-answer tests.
void orc_philox(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]) {
  msx::Philox4 r = msx::philox4x32_10(counter, key);
  for (int i = 0; i < 4; ++i) out[i] = r.w[i];
}
void orc_blake3(const void* data, uint64_t len, uint8_t out[32]) { msx::blake3(data, size_t(len), out); }
uint64_t orc_canonical_id(const char* path) { return msx::canonical_id(path); }
uint64_t orc_dropout_id(const char* site, uint64_t step) { return msx::dropout_id(site, step); }
uint64_t orc_dropout_threshold(float p) { return msx::dropout_threshold(p); }
int orc_dropout_keeps(uint64_t seed, uint64_t id, uint32_t index, float p) { return msx::dropout_keeps(seed, id, index, p); }
void orc_adamw_scalars(float lr, uint64_t t, uint64_t steps, uint64_t warmup, float beta1, float beta2, float out[3]) {
  msx::AdamWConfig a;
  a.beta1 = beta1;
  a.beta2 = beta2;
  a.warmup_steps = warmup;
  msx::StepScalars s = msx::adamw_scalars(a, lr, t, steps);
  out[0] = s.lr_t;
  out[1] = s.c1;
  out[2] = s.c2;
}

// The inputs of training step `step` of a built-in config, one name per line with its dtype, for
// tests that feed the same step to both backends: names joined by '\n' into `names` (malloc'd),
// data concatenated into a malloc'd buffer of 4-byte words.
int orc_step_inputs(const char* config, int64_t steps, int64_t masked_rows, uint64_t step, char** names,
                    void** data, uint64_t* words) {
  try {
    msx::Compiled c = msx::compile_config(config, masked_rows, steps);
    msx::Feed feed(c);
    if (feed.needs_teacher()) {
      OracleEngine e(c);
      feed.set_target(e.predict(msx::initialize(c.forward, c.config.seed, msx::Stream::Teacher), feed.batch(0)));
    }
    msx::StepInputs in = msx::step_inputs(c, feed, step, c.config.steps);
    std::string text;
    std::vector<uint32_t> buf;
    for (auto& [name, v] : in.batch.f32) {
      text += name + "\tf32\t" + std::to_string(v.size()) + "\n";
      const uint32_t* w = reinterpret_cast<const uint32_t*>(v.data());
      buf.insert(buf.end(), w, w + v.size());
    }
    for (auto& [name, v] : in.batch.i32) {
      text += name + "\ti32\t" + std::to_string(v.size()) + "\n";
      const uint32_t* w = reinterpret_cast<const uint32_t*>(v.data());
      buf.insert(buf.end(), w, w + v.size());
    }
    *names = static_cast<char*>(std::malloc(text.size() + 1));
    std::memcpy(*names, text.c_str(), text.size() + 1);
    *data = std::malloc(std::max<size_t>(buf.size(), 1) * 4);
    std::memcpy(*data, buf.data(), buf.size() * 4);
    *words = buf.size();
    return 0;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}
void orc_free(void* p) { std::free(p); }

// The initial parameters of a built-in config (ParamId order, concatenated).
int orc_init_params(const char* config, float* out, uint64_t len) {
  try {
    msx::Compiled c = msx::compile_config(config, -1, -1);
    uint64_t off = 0;
    for (auto& p : msx::initialize(c.forward, c.config.seed, msx::Stream::Init)) {
      if (off + p.size() > len) { g_error = "buffer too small"; return -1; }
      std::memcpy(out + off, p.data(), p.size() * 4);
      off += p.size();
    }
    return 0;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

// Trains `config` for `steps` steps (negative: the config's own) and writes steps + 1 losses and
// the final parameters, concatenated in ParamId order. Returns 0, or -1 with orc_last_error().
int orc_train(const char* config, int64_t steps, int64_t masked_rows, float* losses, uint64_t losses_len,
              float* params_out, uint64_t params_len, double* train_seconds) {
  try {
    msx::Compiled c = msx::compile_config(config, masked_rows, steps);
    OracleEngine e(c);
    msx::RunResult r = msx::run(c, e, c.config.steps);
    if (r.nonfinite_step >= 0) { g_error = "E-TRAIN-001: non-finite loss at step " + std::to_string(r.nonfinite_step); return -1; }
    if (losses_len < r.losses.size()) { g_error = "losses buffer too small"; return -1; }
    std::memcpy(losses, r.losses.data(), r.losses.size() * sizeof(float));
    uint64_t off = 0;
    for (auto& p : r.params) {
      if (off + p.size() > params_len) { g_error = "params buffer too small"; return -1; }
      std::memcpy(params_out + off, p.data(), p.size() * sizeof(float));
      off += p.size();
    }
    if (train_seconds) *train_seconds = r.train_seconds;
    return 0;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

// A run of `config` with a held-out evaluation every `eval_every` steps over `eval_batches`
// batches: writes the evaluated steps and, per evaluation, [loss, accuracy] as the host finishes
// them from the sums (eval.rs:299-339) and [loss, accuracy] of the oracle's own tally
// (eval.rs:520-575) into metrics[4 * k ..]. Returns the number of evaluations, or -1.
int orc_train_eval(const char* config, int64_t steps, uint64_t eval_every, uint64_t eval_batches, uint64_t* eval_steps,
                   float* metrics, uint64_t evals_len) {
  try {
    msx::Compiled c = msx::compile_config(config, -1, steps);
    OracleEngine e(c);
    struct Both : msx::Engine {
      OracleEngine& e;
      std::vector<std::pair<float, float>> own;
      explicit Both(OracleEngine& x) : e(x) {}
      void set_params(const std::vector<std::vector<float>>& v) override { e.set_params(v); }
      std::vector<std::vector<float>> params() override { return e.params(); }
      std::vector<std::vector<float>> moments(char w) override { return e.moments(w); }
      std::vector<float> predict(const std::vector<std::vector<float>>& v, const msx::Batch& b) override { return e.predict(v, b); }
      void train_step(const msx::StepInputs& in) override { e.train_step(in); }
      float final_loss(const msx::Batch& b) override { return e.final_loss(b); }
      std::vector<float> losses() override { return e.losses(); }
      msx::HeldOutSums held_out(const msx::HeldOut& h) override {
        msx::HeldOutSums s = e.held_out(h);
        own.emplace_back(e.tally.loss(), e.tally.accuracy());
        return s;
      }
    } both(e);
    msx::RunResult r = msx::run(c, both, c.config.steps, eval_every, eval_batches);
    if (r.evals.size() > evals_len) { g_error = "evals buffer too small"; return -1; }
    for (size_t k = 0; k < r.evals.size(); ++k) {
      eval_steps[k] = r.evals[k].first;
      metrics[4 * k] = r.evals[k].second.loss;
      metrics[4 * k + 1] = r.evals[k].second.accuracy;
      metrics[4 * k + 2] = both.own[k].first;
      metrics[4 * k + 3] = both.own[k].second;
    }
    return int(r.evals.size());
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

// The held-out tally over explicit logits (eval.rs Tally): `batches` batches of `rows` rows of `v`
// logits each; out = [loss, accuracy, numerator, denominator, correct, selected]. Returns 0, or
// -1 for a label outside the classes.
int orc_held_out_tally(const float* logits, const int32_t* labels, const float* weights, uint64_t batches,
                       uint64_t rows, uint64_t v, double out[6]) {
  oracle::HeldOutTally t;
  for (uint64_t b = 0; b < batches; ++b)
    if (!t.add(logits + b * rows * v, labels + b * rows, weights + b * rows, rows, v)) {
      g_error = "label outside the classes";
      return -1;
    }
  out[0] = t.loss();
  out[1] = t.accuracy();
  out[2] = t.numerator;
  out[3] = t.denominator;
  out[4] = double(t.correct);
  out[5] = double(t.selected);
  return 0;
}

// Times `steps` training steps of `config` on this thread; writes seconds per step.
int orc_time_steps(const char* config, int64_t steps, int64_t masked_rows, double* seconds_per_step) {
  try {
    msx::Compiled c = msx::compile_config(config, masked_rows, -1);
    OracleEngine e(c);
    msx::Feed feed(c);
    if (feed.needs_teacher()) feed.set_target(e.predict(msx::initialize(c.forward, c.config.seed, msx::Stream::Teacher), feed.batch(0)));
    e.set_params(msx::initialize(c.forward, c.config.seed, msx::Stream::Init));
    std::vector<msx::StepInputs> ins;
    for (int64_t s = 0; s < steps; ++s) ins.push_back(msx::step_inputs(c, feed, uint64_t(s), c.config.steps));
    auto t0 = std::chrono::steady_clock::now();
    for (auto& in : ins) e.train_step(in);
    auto t1 = std::chrono::steady_clock::now();
    *seconds_per_step = std::chrono::duration<double>(t1 - t0).count() / double(steps);
    return 0;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

void* orc_prog_new(const char* program_text, int has_seed, uint64_t seed) {
  try {
    auto* p = new Prog;
    p->program = msx::parse_program(program_text);
    p->has_seed = has_seed != 0;
    p->seed = seed;
    return p;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return nullptr;
  }
}

void orc_prog_free(void* h) { delete static_cast<Prog*>(h); }

// dtypes: 0 = f32, 1 = i32. Params by ParamId.
int orc_prog_run(void* h, int n_in, const char** names, const int* dtypes, const void** data, const uint64_t* counts,
                 int n_params, const float** params, const uint64_t* pcounts) {
  try {
    auto* p = static_cast<Prog*>(h);
    std::map<std::string, std::vector<float>> f32;
    std::map<std::string, std::vector<int32_t>> i32;
    for (int k = 0; k < n_in; ++k) {
      if (dtypes[k] == 0) f32[names[k]].assign(static_cast<const float*>(data[k]), static_cast<const float*>(data[k]) + counts[k]);
      else i32[names[k]].assign(static_cast<const int32_t*>(data[k]), static_cast<const int32_t*>(data[k]) + counts[k]);
    }
    std::vector<std::vector<float>> ps;
    for (int k = 0; k < n_params; ++k) ps.emplace_back(params[k], params[k] + pcounts[k]);
    p->interp = std::make_unique<oracle::Interpreter>(p->program, p->has_seed, p->seed);
    p->interp->run(f32, i32, ps);
    return 0;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

int orc_prog_output(void* h, int k, float* out, uint64_t count) {
  try {
    auto* p = static_cast<Prog*>(h);
    const auto& v = p->interp->value(p->program.outputs.at(size_t(k)));
    if (v.size() != count) { g_error = "output size mismatch"; return -1; }
    std::memcpy(out, v.data(), count * sizeof(float));
    return 0;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

}  // extern "C"
