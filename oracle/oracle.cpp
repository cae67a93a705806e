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

#include "../modelspec_amd/csrc/host/checkpoint.h"
#include "../modelspec_amd/csrc/host/runner.h"
#include "interp.h"

namespace {
thread_local std::string g_error;

// The batch tensors of a corpus draw on the CPU: mlm_batch's rows (crates/modelspec-runtime/src/
// dataset/mlm.rs:761-788), each comparison of a Philox word made as the reference makes it, in
// f64 on uniform(w) = (w + 0.5) / 2^32; then, for a program with a masked-row gather, the gather
// of train/masked.rs:97-118 (rows of non-zero weight ascending, padding row 0 / label 0 / +0).
msx::Batch expand_draw(const msx::PackedCorpus& c, uint64_t seed, const msx::Batch& in, const msx::Program& p) {
  auto it = in.i32.find(msx::kDrawInput);
  if (it == in.i32.end()) return in;
  const std::vector<int32_t>& d = it->second;
  const bool held = d.at(0) != 0;
  const uint64_t draw_id = uint64_t(uint32_t(d[1])) | (uint64_t(uint32_t(d[2])) << 32);
  const std::vector<int32_t>& split = held ? c.heldout : c.train;
  const uint64_t S = c.seq_len, B = d.size() - 3, random_tokens = c.vocabulary_size - 5;
  msx::Batch out = in;
  out.i32.erase(msx::kDrawInput);
  std::vector<int32_t> ids, positions, labels;
  std::vector<float> key_mask(size_t(B * S), 1.0f), weights;
  for (uint64_t b = 0; b < B; ++b)
    for (uint64_t q = 0; q < S; ++q) {
      const uint32_t row = uint32_t(b * S + q);
      const int32_t label = split.at(size_t(uint64_t(uint32_t(d[3 + b])) * S + q));
      const msx::Philox4 w = msx::philox_block(seed, msx::Stream::Masking, draw_id, row);
      const bool selected = label >= 5 && msx::uniform_word(w.w[0]) < c.policy.selection_rate;
      int32_t id;
      if (!selected) id = label;
      else if (msx::uniform_word(w.w[1]) < c.policy.mask_fraction) id = 4;
      else if (msx::uniform_word(w.w[1]) < c.policy.mask_fraction + c.policy.random_fraction)
        id = int32_t(5 + ((uint64_t(w.w[2]) * random_tokens) >> 32));
      else id = label;
      ids.push_back(id);
      positions.push_back(int32_t(q));
      labels.push_back(label);
      weights.push_back(selected ? 1.0f : 0.0f);
    }
  out.i32["ids"] = ids;
  out.i32["positions"] = positions;
  out.i32["labels"] = labels;
  out.f32["key_mask"] = key_mask;
  out.f32["weights"] = weights;
  if (const msx::Node* rows_in = p.input(msx::kMaskedRowsInput)) {
    const size_t cap = size_t(rows_in->ty.count());
    std::vector<int32_t> rows, lab;
    std::vector<float> wts;
    for (size_t r = 0; r < weights.size(); ++r)
      if (weights[r] != 0.0f) {
        rows.push_back(int32_t(r));
        lab.push_back(labels[r]);
        wts.push_back(weights[r]);
      }
    if (rows.size() > cap)
      throw msx::IrError("E-DATA-012: the batch of draw " + std::to_string(draw_id) + " has " + std::to_string(rows.size()) +
                         " rows of non-zero weight, more than the " + std::to_string(cap) +
                         " rows the masked-row gather holds");
    rows.resize(cap, 0);
    lab.resize(cap, 0);
    wts.resize(cap, 0.0f);
    for (auto& x : p.nodes)
      if (x.op == msx::Op::Input) {
        if (x.name.rfind(msx::kMaskedLabelsPrefix, 0) == 0) out.i32[x.name] = lab;
        if (x.name.rfind(msx::kMaskedWeightsPrefix, 0) == 0) out.f32[x.name] = wts;
      }
    out.i32[msx::kMaskedRowsInput] = rows;
  }
  return out;
}

class OracleEngine : public msx::Engine {
 public:
  explicit OracleEngine(const msx::Compiled& c, const msx::PackedCorpus* corpus = nullptr) : c_(c), corpus_(corpus) {}
  msx::Batch expand(const msx::Batch& b, const msx::Program& p) const {
    return corpus_ ? expand_draw(*corpus_, c_.config.seed, b, p) : b;
  }

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
  void set_moments(const std::vector<std::vector<float>>& m, const std::vector<std::vector<float>>& v) override {
    for (auto& [param, mo] : c_.step.moments) {
      m_[param] = m.at(param);
      v_[param] = v.at(param);
    }
  }
  std::vector<float> predict(const std::vector<std::vector<float>>& values, const msx::Batch& b0) override {
    const msx::Batch b = expand(b0, c_.forward);
    oracle::Interpreter it(c_.forward, true, c_.config.seed);
    it.run(b.f32, b.i32, values);
    return it.value(c_.prediction);
  }
  void train_step(const msx::StepInputs& in0) override {
    const msx::TrainingStep& s = c_.step;
    msx::StepInputs in;
    in.batch = expand(in0.batch, s.program);
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
  float final_loss(const msx::Batch& b0) override {
    const msx::Batch b = expand(b0, c_.forward);
    oracle::Interpreter it(c_.forward, true, c_.config.seed);
    it.run(b.f32, b.i32, params_);
    return it.value(c_.forward.outputs[0])[0];
  }
  std::vector<float> losses() override { return losses_; }
  msx::HeldOutSums held_out(const msx::HeldOut& h) override {
    tally = tally_of(h, params_);
    msx::HeldOutSums out;
    out.numerator = tally.numerator;
    out.correct = tally.correct;
    out.denominator = tally.denominator;
    out.selected = tally.selected;
    out.has_totals = true;
    return out;
  }
  // The forward program over every held-out batch on `values`, tallied (eval.rs:263-287).
  oracle::HeldOutTally tally_of(const msx::HeldOut& h, const std::vector<std::vector<float>>& values) const {
    oracle::HeldOutTally t;
    size_t b = 0;
    for (auto& batch0 : h.batches()) {
      const msx::Batch batch = expand(batch0, c_.forward);
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
  const msx::PackedCorpus* corpus_;
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
    if (r.nonfinite_step >= 0) { g_error = "E-TRAIN-001: " + r.nonfinite_message; return -1; }
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

// A run of `config`, its batches synthetic or drawn from the packed directory `packed_dir`
// (may be null), with a held-out evaluation every `eval_every` steps (0: none) over
// `eval_batches` batches: writes the losses and final parameters (either may be null), the
// evaluated steps and, per evaluation, [loss, accuracy] as the host finishes them from the sums
// (eval.rs:299-339) and [loss, accuracy] of the oracle's own tally (eval.rs:520-575) into
// metrics[4 * k ..]. Returns the number of evaluations, or -1.
int orc_train_run(const char* config, const char* packed_dir, int64_t steps, uint64_t eval_every, uint64_t eval_batches,
                  float* losses, uint64_t losses_len, float* params_out, uint64_t params_len, uint64_t* eval_steps,
                  float* metrics, uint64_t evals_len) {
  try {
    msx::Compiled c = msx::compile_config(config, -1, steps);
    std::unique_ptr<msx::PackedCorpus> corpus;
    if (packed_dir) corpus = std::make_unique<msx::PackedCorpus>(msx::load_packed(packed_dir));
    OracleEngine e(c, corpus.get());
    struct Both : msx::Engine {
      OracleEngine& e;
      std::vector<std::pair<float, float>> own;
      explicit Both(OracleEngine& x) : e(x) {}
      void set_params(const std::vector<std::vector<float>>& v) override { e.set_params(v); }
      std::vector<std::vector<float>> params() override { return e.params(); }
      std::vector<std::vector<float>> moments(char w) override { return e.moments(w); }
      void set_moments(const std::vector<std::vector<float>>& m, const std::vector<std::vector<float>>& v) override {
        e.set_moments(m, v);
      }
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
    msx::RunResult r = msx::run(c, both, c.config.steps, eval_every, eval_batches, corpus.get());
    if (r.evals.size() > evals_len) { g_error = "evals buffer too small"; return -1; }
    if (losses) {
      if (losses_len < r.losses.size()) { g_error = "losses buffer too small"; return -1; }
      std::memcpy(losses, r.losses.data(), r.losses.size() * sizeof(float));
    }
    if (params_out) {
      uint64_t off = 0;
      for (auto& p : r.params) {
        if (off + p.size() > params_len) { g_error = "params buffer too small"; return -1; }
        std::memcpy(params_out + off, p.data(), p.size() * sizeof(float));
        off += p.size();
      }
    }
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

int orc_train_eval(const char* config, int64_t steps, uint64_t eval_every, uint64_t eval_batches, uint64_t* eval_steps,
                   float* metrics, uint64_t evals_len) {
  return orc_train_run(config, nullptr, steps, eval_every, eval_batches, nullptr, 0, nullptr, 0, eval_steps, metrics,
                       evals_len);
}

// The rows of one corpus draw on the CPU (the checker of the device's MlmBatch and MaskedGather):
// step `step` of split `role` (0 Train, 1 HeldOut) of the packed directory bound to `config`.
// Writes ids, positions, labels (i32 [B*S]), weights (f32 [B*S]) and, when the step program
// gathers, rows, labels and weights of the gather (i32/i32/f32 [C]) into caller buffers of the
// right sizes (any may be null). Returns B, or -1.
int64_t orc_corpus_draw(const char* config, const char* packed_dir, int role, uint64_t step, int32_t* ids,
                        int32_t* positions, int32_t* labels, float* weights, int32_t* g_rows, int32_t* g_labels,
                        float* g_weights) {
  try {
    msx::Compiled c = msx::compile_config(config, -1, -1);
    msx::PackedCorpus corpus = msx::load_packed(packed_dir);
    const uint64_t B = msx::bind_corpus(c.forward, corpus);
    msx::EpochOrders orders;
    const msx::SplitRole r = role ? msx::SplitRole::HeldOut : msx::SplitRole::Train;
    msx::Batch in;
    in.i32[msx::kDrawInput] = msx::draw_words(r, orders.draw(corpus, r, c.config.seed, step, B));
    msx::Batch b = expand_draw(corpus, c.config.seed, in, c.step.program);
    auto put_i = [&](int32_t* dst, const char* name) {
      if (dst && b.i32.count(name)) std::memcpy(dst, b.i32.at(name).data(), b.i32.at(name).size() * 4);
    };
    put_i(ids, "ids");
    put_i(positions, "positions");
    put_i(labels, "labels");
    if (weights) std::memcpy(weights, b.f32.at("weights").data(), b.f32.at("weights").size() * 4);
    if (b.i32.count(msx::kMaskedRowsInput)) {
      put_i(g_rows, msx::kMaskedRowsInput);
      for (auto& [name, v] : b.i32)
        if (g_labels && name.rfind(msx::kMaskedLabelsPrefix, 0) == 0) std::memcpy(g_labels, v.data(), v.size() * 4);
      for (auto& [name, v] : b.f32)
        if (g_weights && name.rfind(msx::kMaskedWeightsPrefix, 0) == 0) std::memcpy(g_weights, v.data(), v.size() * 4);
    }
    return int64_t(B);
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

// A run of `config` (on `packed_dir` when not null) that may resume from `resume` and write
// checkpoints as msx_train_checkpointed does. Writes the losses and final parameters; returns the
// start step, or -1.
int64_t orc_train_ckpt(const char* config, const char* packed_dir, int64_t steps, const char* resume,
                       uint64_t checkpoint_every, const char* checkpoint_path, float* losses, uint64_t losses_len,
                       float* params_out, uint64_t params_len) {
  try {
    msx::Compiled c = msx::compile_config(config, -1, -1);
    std::unique_ptr<msx::PackedCorpus> corpus;
    if (packed_dir) corpus = std::make_unique<msx::PackedCorpus>(msx::load_packed(packed_dir));
    std::unique_ptr<msx::ResumeState> from;
    if (resume) from = std::make_unique<msx::ResumeState>(msx::resume_into(msx::read_checkpoint(resume), c.step));
    const uint64_t n = steps >= 0 ? uint64_t(steps) : c.config.steps - (from ? std::min(from->step, c.config.steps) : 0);
    OracleEngine e(c, corpus.get());
    msx::RunOptions o;
    o.corpus = corpus.get();
    o.resume = from.get();
    o.checkpoint_every = checkpoint_every;
    if (checkpoint_path) o.checkpoint_path = checkpoint_path;
    msx::RunResult r = msx::run(c, e, n, o);
    if (r.nonfinite_step >= 0) {
      g_error = "E-TRAIN-001: " + r.nonfinite_message;
      return -1;
    }
    if (losses) {
      if (losses_len < r.losses.size()) { g_error = "losses buffer too small"; return -1; }
      std::memcpy(losses, r.losses.data(), r.losses.size() * sizeof(float));
    }
    if (params_out) {
      uint64_t off = 0;
      for (auto& p : r.params) {
        if (off + p.size() > params_len) { g_error = "params buffer too small"; return -1; }
        std::memcpy(params_out + off, p.data(), p.size() * sizeof(float));
        off += p.size();
      }
    }
    return int64_t(r.start_step);
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

// schema_hash (core/src/artifact.rs:169-193) of a config's step program, into out[65].
int orc_schema_hash(const char* config, char out[65]) {
  try {
    msx::Compiled c = msx::compile_config(config, -1, -1);
    std::string h = msx::schema_hash(c.step.program);
    std::memcpy(out, h.c_str(), 65);
    return 0;
  } catch (const std::exception& ex) {
    g_error = ex.what();
    return -1;
  }
}

// json_f64 of v into out[40].
void orc_json_f64(double v, char out[40]) {
  std::string s = msx::json_f64(v);
  std::memcpy(out, s.c_str(), s.size() + 1);
}

// uuid_of (dataset/mod.rs:212-227) of a 32-byte hash into out[37].
void orc_uuid_of(const uint8_t hash[32], char out[37]) {
  std::string u = msx::uuid_of(hash);
  std::memcpy(out, u.c_str(), u.size() + 1);
}

// binding_id (mlm.rs:161-185) into out[37]; returns 0, or -1 when an id is not a UUID.
int orc_binding_id(const char* dataset_id, const char* tokenizer_id, uint64_t seq_len, const double rates[4],
                   char out[37]) {
  msx::MaskingPolicy p;
  p.selection_rate = rates[0];
  p.mask_fraction = rates[1];
  p.random_fraction = rates[2];
  p.keep_fraction = rates[3];
  std::string id = msx::binding_id(dataset_id, tokenizer_id, seq_len, p);
  if (id.empty()) return -1;
  std::memcpy(out, id.c_str(), id.size() + 1);
  return 0;
}

// epoch_order (mlm.rs:665-680) into out[n].
void orc_epoch_order(uint64_t seed, uint64_t epoch, uint32_t n, uint32_t* out) {
  auto o = msx::epoch_order(seed, epoch, n);
  std::memcpy(out, o.data(), o.size() * 4);
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

// The wall-clock seconds of each of `steps` training steps of `config` on this thread, from the
// initial parameters, inputs made beforehand: out[k] is step k's. Returns 0, or -1 with
// orc_last_error().
int orc_step_times(const char* config, int64_t steps, int64_t masked_rows, double* out) {
  try {
    msx::Compiled c = msx::compile_config(config, masked_rows, -1);
    OracleEngine e(c);
    msx::Feed feed(c);
    if (feed.needs_teacher()) feed.set_target(e.predict(msx::initialize(c.forward, c.config.seed, msx::Stream::Teacher), feed.batch(0)));
    e.set_params(msx::initialize(c.forward, c.config.seed, msx::Stream::Init));
    std::vector<msx::StepInputs> ins;
    for (int64_t s = 0; s < steps; ++s) ins.push_back(msx::step_inputs(c, feed, uint64_t(s), c.config.steps));
    for (int64_t s = 0; s < steps; ++s) {
      auto t0 = std::chrono::steady_clock::now();
      e.train_step(ins[size_t(s)]);
      out[s] = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    }
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
