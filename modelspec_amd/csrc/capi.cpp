// The C ABI of libmsx.so (include/msx.h): status codes, no exception across the boundary.
#include <dlfcn.h>

#include <cstdlib>
#include <cstring>
#include <memory>

#include "../../include/msx.h"
#include "hip/runtime.h"
#include "host/models.h"
#include "host/artifact.h"
#include "host/checkpoint.h"
#include "host/packed.h"
#include "host/runner.h"

namespace {
thread_local std::string g_error;

int fail(int code, const std::string& what) {
  g_error = what;
  return code;
}

// Runs `f`, mapping the exceptions of the host and device layers to status codes.
template <class F>
int guarded(F&& f) {
  try {
    g_error.clear();
    return f();
  } catch (const msx::HipError& e) {
    return fail(MSX_E_DEVICE, e.what());
  } catch (const msx::HeldOutLabelError& e) {
    return fail(MSX_E_DATA, e.what());
  } catch (const msx::PackedError& e) {
    return fail(MSX_E_DATA, e.what());
  } catch (const msx::CheckpointError& e) {
    return fail(MSX_E_CHECKPOINT, e.what());
  } catch (const msx::ArtifactError& e) {
    return fail(e.code == "E-ARTIFACT-005" ? MSX_E_DEVICE : MSX_E_ARTIFACT, e.what());
  } catch (const msx::IrError& e) {
    std::string w = e.what();
    if (w.find("E-DATA-") != std::string::npos || w.find("key mask") != std::string::npos ||
        w.find("loss weight") != std::string::npos)
      return fail(MSX_E_DATA, w);
    if (w.find("no HIP kernel") != std::string::npos || w.find("not the AdamW/SGD template") != std::string::npos)
      return fail(MSX_E_UNSUPPORTED, w);
    return fail(MSX_E_INVALID, w);
  } catch (const std::exception& e) {
    std::string w = e.what();
    if (w.find("kernel launch refused") != std::string::npos) return fail(MSX_E_UNSUPPORTED, w);
    return fail(MSX_E_INVALID, w);
  }
}

char* dup(const std::string& s) {
  char* p = static_cast<char*>(std::malloc(s.size() + 1));
  std::memcpy(p, s.c_str(), s.size() + 1);
  return p;
}

// The smallest run length whose AdamW warmup stays shorter than the run.
uint64_t c_steps_floor(const char* config) {
  msx::Compiled c = msx::compile_config(config, -1, -1);
  return c.step.rule == msx::Rule::AdamW ? c.step.adamw.warmup_steps + 1 : 1;
}

msx::Batch batch_of(const msx_tensor* t, uint32_t n) {
  msx::Batch b;
  for (uint32_t i = 0; i < n; ++i) {
    if (!t[i].name) throw msx::IrError("an input has no name");
    if (t[i].dtype == 0) {
      auto* f = static_cast<const float*>(t[i].data);
      b.f32[t[i].name].assign(f, f + t[i].count);
    } else if (t[i].dtype == 1) {
      auto* v = static_cast<const int32_t*>(t[i].data);
      b.i32[t[i].name].assign(v, v + t[i].count);
    } else {
      throw msx::IrError(std::string("input `") + t[i].name + "` has an unknown dtype");
    }
  }
  return b;
}
}  // namespace

struct msx_ctx {
  int device = 0;
  std::unique_ptr<msx::Session> session;
  msx::TrainingStep step;
  msx::Program forward;
  uint32_t prediction = 0;  // the forward program's prediction value
  // A packed corpus msx_load_packed read; msx_load then draws every batch from it on the device.
  std::unique_ptr<msx::PackedCorpus> corpus;
  msx::EpochOrders orders;
  uint64_t seed = 0;
  msx::SessionOptions options;  // msx_set_precision, for the next msx_load
};

namespace {
// A built-in config's session: its own precision, the context's fusion choices (msx_set_fusion).
msx::SessionOptions config_options(const msx_ctx* ctx, const msx::Compiled& c) {
  msx::SessionOptions o;
  o.mixed = c.config.mixed;
  o.fuse_ce_head = ctx->options.fuse_ce_head;
  o.fuse_optimizer = ctx->options.fuse_optimizer;
  return o;
}

// With a corpus loaded, a batch that names `data.step` (i32 [low, high] of the step) is the
// corpus batch of that step: its sequences are drawn here and the device draws its rows.
void corpus_draw(msx_ctx* ctx, msx::Batch& b, msx::SplitRole role) {
  auto it = b.i32.find("data.step");
  if (it == b.i32.end()) return;
  if (!ctx->corpus || !ctx->session) throw msx::IrError("`data.step` names a corpus batch, and no corpus is loaded");
  if (it->second.size() != 2) throw msx::IrError("`data.step` is i32 [low, high]");
  const uint64_t step = uint64_t(uint32_t(it->second[0])) | (uint64_t(uint32_t(it->second[1])) << 32);
  b.i32.erase(it);
  b.i32[msx::kDrawInput] =
      msx::draw_words(role, ctx->orders.draw(*ctx->corpus, role, ctx->seed, step, ctx->session->corpus_batch()));
}
}  // namespace

struct msx_prog {
  std::unique_ptr<msx::Session> session;
  msx::Program program;
};

extern "C" {

const char* msx_last_error(void) { return g_error.c_str(); }

int msx_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int msx_compile_config(const char* config, int64_t masked_rows, int64_t steps, char** step_ir, char** forward_ir) {
  return guarded([&] {
    msx::Compiled c = msx::compile_config(config, masked_rows, steps);
    if (step_ir) *step_ir = dup(msx::print_step(c.step));
    if (forward_ir) *forward_ir = dup(msx::print_program(c.forward));
    return MSX_OK;
  });
}

int msx_config_steps(const char* config, uint64_t* steps, uint64_t* seed) {
  return guarded([&] {
    msx::Compiled c = msx::compile_config(config, -1, -1);
    if (steps) *steps = c.config.steps;
    if (seed) *seed = c.config.seed;
    return MSX_OK;
  });
}

void msx_free(void* p) { std::free(p); }

int msx_check_ir(const char* step_ir, char** normalized) {
  return guarded([&] {
    msx::TrainingStep t = msx::parse_step(step_ir);
    if (normalized) *normalized = dup(msx::print_step(t));
    return MSX_OK;
  });
}

int msx_open(int device, msx_ctx** out) {
  return guarded([&] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(MSX_E_DEVICE, "E-TARGET-002: no HIP device is visible");
    if (device < 0 || device >= n) return fail(MSX_E_DEVICE, "E-TARGET-003: no HIP device " + std::to_string(device));
    msx::hip_check(hipSetDevice(device), "hipSetDevice");
    auto* c = new msx_ctx;
    c->device = device;
    *out = c;
    return MSX_OK;
  });
}

void msx_close(msx_ctx* ctx) {
  try {
    delete ctx;
  } catch (...) {
  }
}

int msx_load(msx_ctx* ctx, const char* step_ir, const char* forward_ir, uint64_t seed, uint32_t prediction_output) {
  return guarded([&] {
    ctx->session.reset();
    ctx->step = msx::parse_step(step_ir);
    if (!ctx->step.has_optimizer) return fail(MSX_E_INVALID, "the step IR has no optimizer");
    ctx->forward = msx::parse_program(forward_ir);
    if (prediction_output >= ctx->forward.outputs.size()) return fail(MSX_E_INVALID, "no such forward output");
    ctx->prediction = ctx->forward.outputs[prediction_output];
    ctx->seed = seed;
    ctx->session = std::make_unique<msx::Session>(ctx->device, ctx->step, ctx->forward, seed,
                                                  ctx->forward.outputs[prediction_output], ctx->corpus.get(), ctx->options);
    return MSX_OK;
  });
}

int msx_plan(const char* step_ir, const char* forward_ir, uint32_t prediction_output, int32_t mixed, char** plan) {
  return guarded([&] {
    if (!step_ir || !forward_ir || !plan) return fail(MSX_E_INVALID, "null argument");
    msx::TrainingStep step = msx::parse_step(step_ir);
    if (!step.has_optimizer) return fail(MSX_E_INVALID, "the step IR has no optimizer");
    msx::Program forward = msx::parse_program(forward_ir);
    if (prediction_output >= forward.outputs.size()) return fail(MSX_E_INVALID, "no such forward output");
    msx::SessionOptions o;
    o.plan_only = true;
    o.mixed = mixed != 0;
    msx::Session s(0, step, forward, 0, forward.outputs[prediction_output], nullptr, o);
    *plan = dup(s.plan_text());
    return MSX_OK;
  });
}

int msx_set_params(msx_ctx* ctx, const float* const* values, const uint64_t* counts, uint32_t n) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    std::vector<std::vector<float>> v;
    for (uint32_t i = 0; i < n; ++i) v.emplace_back(values[i], values[i] + counts[i]);
    ctx->session->set_params(v);
    return MSX_OK;
  });
}

int msx_read_param(msx_ctx* ctx, uint32_t param, float* out, uint64_t count) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    auto all = ctx->session->params();
    if (param >= all.size() || all[param].size() != count) return fail(MSX_E_INVALID, "no such parameter or wrong count");
    std::memcpy(out, all[param].data(), count * 4);
    return MSX_OK;
  });
}

int msx_read_moment(msx_ctx* ctx, uint32_t param, int32_t which, float* out, uint64_t count) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    auto all = ctx->session->moments(char(which));
    if (param >= all.size() || all[param].size() != count) return fail(MSX_E_INVALID, "no such moment or wrong count");
    std::memcpy(out, all[param].data(), count * 4);
    return MSX_OK;
  });
}

int msx_run_steps(msx_ctx* ctx, uint32_t n, const msx_tensor* const* inputs, const uint32_t* n_inputs, float* losses_out) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    size_t before = ctx->session->losses().size();
    for (uint32_t i = 0; i < n; ++i) {
      msx::StepInputs in;
      in.batch = batch_of(inputs[i], n_inputs[i]);
      corpus_draw(ctx, in.batch, msx::SplitRole::Train);
      ctx->session->train_step(in);
    }
    auto all = ctx->session->losses();
    if (losses_out)
      for (uint32_t i = 0; i < n; ++i) losses_out[i] = all.at(before + i);
    for (uint32_t i = 0; i < n; ++i)
      if (!std::isfinite(all.at(before + i)))
        return fail(MSX_E_NONFINITE, "E-TRAIN-001: the loss of step " + std::to_string(before + i) + " is not finite");
    return MSX_OK;
  });
}

int msx_forward(msx_ctx* ctx, const msx_tensor* inputs, uint32_t n_inputs, float* loss_out, float* prediction_out,
                uint64_t prediction_count) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    msx::Batch b = batch_of(inputs, n_inputs);
    corpus_draw(ctx, b, msx::SplitRole::Train);
    float loss = ctx->session->final_loss(b);
    if (loss_out) *loss_out = loss;
    if (prediction_out) {
      const uint32_t pred = ctx->prediction;
      if (ctx->forward.node(pred).ty.count() != int64_t(prediction_count)) return fail(MSX_E_INVALID, "prediction count");
      msx::hip_check(hipMemcpy(prediction_out, ctx->session->forward_value(pred), prediction_count * 4, hipMemcpyDeviceToHost),
                     "hipMemcpy (prediction)");
    }
    return MSX_OK;
  });
}

int msx_read_input(msx_ctx* ctx, int32_t program, const char* name, void* out, uint64_t count) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    if (!name || !out) return fail(MSX_E_INVALID, "null argument");
    const msx::Program& p = program == 0 ? ctx->step.program : ctx->forward;
    const msx::Node* in = p.input(name);
    if (!in) return fail(MSX_E_INVALID, std::string("the program has no input `") + name + "`");
    if (in->ty.count() != int64_t(count)) return fail(MSX_E_INVALID, std::string("input `") + name + "` count");
    ctx->session->sync();
    const void* src = program == 0 ? ctx->session->step_value(in->id) : ctx->session->forward_value(in->id);
    msx::hip_check(hipMemcpy(out, src, count * 4, hipMemcpyDeviceToHost), "hipMemcpy (input)");
    return MSX_OK;
  });
}

int msx_set_fusion(msx_ctx* ctx, uint32_t flags) {
  return guarded([&] {
    if (flags & ~uint32_t(MSX_FUSE_CE_HEAD | MSX_FUSE_OPTIMIZER)) return fail(MSX_E_INVALID, "unknown fusion flags");
    ctx->options.fuse_ce_head = (flags & MSX_FUSE_CE_HEAD) != 0;
    ctx->options.fuse_optimizer = (flags & MSX_FUSE_OPTIMIZER) != 0;
    return MSX_OK;
  });
}

int msx_set_precision(msx_ctx* ctx, int32_t mixed, float loss_scale, uint32_t scale_window) {
  return guarded([&] {
    if (!(loss_scale >= 1.0f) || !std::isfinite(loss_scale) || scale_window == 0)
      return fail(MSX_E_INVALID, "a loss scale of at least 1 and a window of at least one step");
    ctx->options.mixed = mixed != 0;
    ctx->options.loss_scale = loss_scale;
    ctx->options.scale_window = scale_window;
    return MSX_OK;
  });
}

int msx_loss_scale(msx_ctx* ctx, float* scale, uint64_t* skipped) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    msx::hk::LossScaleState st = ctx->session->loss_scale();
    if (scale) *scale = ctx->session->mixed() ? st.scale : 1.0f;
    if (skipped) *skipped = ctx->session->mixed() ? st.skipped : 0;
    return MSX_OK;
  });
}

int msx_stats(msx_ctx* ctx, msx_run_stats* out) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    const auto& s = ctx->session->stats();
    out->steps = s.steps;
    out->graph_launches = s.graph_launches;
    out->kernels_per_step = s.kernels_per_step;
    out->bytes_uploaded = s.bytes_uploaded;
    out->device_bytes = s.device_bytes;
    return MSX_OK;
  });
}

namespace {
// The metrics of `sums` with the host's own sums of `h`'s weights beside them.
msx_heldout heldout_of(const msx::HeldOut& h, const msx::HeldOutSums& sums) {
  msx::HeldOutMetrics m = h.metrics_of_sums(sums);
  msx_heldout out{};
  out.loss = m.loss;
  out.accuracy = m.accuracy;
  out.numerator = sums.numerator;
  out.correct = sums.correct;
  bool host_weights = true;
  for (auto& b : h.batches()) host_weights = host_weights && b.f32.count(h.weights_name());
  if (!host_weights) {
    out.denominator = sums.denominator;
    out.selected = sums.selected;
    return out;
  }
  bool first = true;
  for (auto& b : h.batches())
    for (float w : b.f32.at(h.weights_name())) {
      out.denominator = first ? double(w) : out.denominator + double(w);
      first = false;
      if (w > 0.0f) ++out.selected;
    }
  return out;
}
}  // namespace

namespace {
int evaluate(msx_ctx* ctx, uint32_t n, const msx_tensor* const* inputs, const uint32_t* n_inputs, const char* labels,
             const char* weights, msx_heldout* out, bool no_alloc) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    if (!labels || !weights || !out || (n && (!inputs || !n_inputs))) return fail(MSX_E_INVALID, "null argument");
    std::vector<msx::Batch> batches;
    for (uint32_t i = 0; i < n; ++i) batches.push_back(batch_of(inputs[i], n_inputs[i]));
    if (n == 0 && ctx->corpus) {
      // Every whole batch of the corpus's HeldOut split, in stored order (eval.rs:6-12).
      const uint64_t B = ctx->session->corpus_batch(), whole = ctx->corpus->sequences(msx::SplitRole::HeldOut) / B;
      if (whole == 0) return fail(MSX_E_DATA, "the HeldOut split holds fewer sequences than one batch");
      for (uint64_t b = 0; b < whole; ++b) {
        msx::Batch x;
        x.i32[msx::kDrawInput] =
            msx::draw_words(msx::SplitRole::HeldOut, ctx->orders.draw(*ctx->corpus, msx::SplitRole::HeldOut, ctx->seed, b, B));
        batches.push_back(std::move(x));
      }
    }
    msx::HeldOut h(ctx->forward, ctx->prediction, labels, weights, std::move(batches));
    *out = heldout_of(h, no_alloc ? ctx->session->held_out_static(h) : ctx->session->held_out(h));
    return MSX_OK;
  });
}
}  // namespace

int msx_evaluate(msx_ctx* ctx, uint32_t n, const msx_tensor* const* inputs, const uint32_t* n_inputs,
                 const char* labels, const char* weights, msx_heldout* out) {
  return evaluate(ctx, n, inputs, n_inputs, labels, weights, out, false);
}

int msx_evaluate_static(msx_ctx* ctx, uint32_t n, const msx_tensor* const* inputs, const uint32_t* n_inputs,
                        const char* labels, const char* weights, msx_heldout* out) {
  return evaluate(ctx, n, inputs, n_inputs, labels, weights, out, true);
}

namespace {
// One run of a built-in config, its batches synthetic or drawn from `corpus`, with a held-out
// evaluation every `eval_every` steps (0: none).
int train_run(msx_ctx* ctx, const char* config, int64_t steps, uint64_t eval_every, uint64_t eval_batches,
              const msx::PackedCorpus* corpus, float* losses, uint64_t losses_len, float* params, uint64_t params_len,
              uint64_t* eval_steps, msx_heldout* evals, uint64_t evals_len, uint64_t* n_evals, double* train_seconds,
              double* eval_seconds) {
  msx::Compiled c = msx::compile_config(config, -1, steps);
  ctx->session.reset();
  ctx->step = c.step;
  ctx->forward = c.forward;
  ctx->prediction = c.prediction;
  ctx->seed = c.config.seed;
  ctx->session = std::make_unique<msx::Session>(ctx->device, ctx->step, ctx->forward, c.config.seed, c.prediction, corpus,
                                                config_options(ctx, c));
  // Each evaluation's metrics, finished with the host's weight sums as msx_evaluate does.
  struct Recording : msx::Engine {
    msx::Session& s;
    std::vector<msx_heldout> metrics;
    explicit Recording(msx::Session& x) : s(x) {}
    void set_params(const std::vector<std::vector<float>>& v) override { s.set_params(v); }
    std::vector<std::vector<float>> params() override { return s.params(); }
    std::vector<std::vector<float>> moments(char w) override { return s.moments(w); }
    void set_moments(const std::vector<std::vector<float>>& m, const std::vector<std::vector<float>>& v) override {
      s.set_moments(m, v);
    }
    std::vector<float> predict(const std::vector<std::vector<float>>& v, const msx::Batch& b) override { return s.predict(v, b); }
    void train_step(const msx::StepInputs& in) override { s.train_step(in); }
    float final_loss(const msx::Batch& b) override { return s.final_loss(b); }
    std::vector<float> losses() override { return s.losses(); }
    msx::HeldOutSums held_out(const msx::HeldOut& x) override {
      msx::HeldOutSums sums = s.held_out(x);
      metrics.push_back(heldout_of(x, sums));
      return sums;
    }
  } rec(*ctx->session);
  msx::RunResult r = msx::run(c, rec, c.config.steps, eval_every, eval_batches, corpus);
  if (losses_len < r.losses.size()) return fail(MSX_E_INVALID, "losses buffer too small");
  if (losses) std::memcpy(losses, r.losses.data(), r.losses.size() * 4);
  if (params) {
    uint64_t off = 0;
    for (auto& p : r.params) {
      if (off + p.size() > params_len) return fail(MSX_E_INVALID, "params buffer too small");
      std::memcpy(params + off, p.data(), p.size() * 4);
      off += p.size();
    }
  }
  if (r.evals.size() > evals_len) return fail(MSX_E_INVALID, "evals buffer too small");
  for (size_t k = 0; k < r.evals.size(); ++k) {
    if (eval_steps) eval_steps[k] = r.evals[k].first;
    if (evals) evals[k] = rec.metrics[k];
  }
  if (n_evals) *n_evals = r.evals.size();
  if (train_seconds) *train_seconds = r.train_seconds;
  if (eval_seconds) *eval_seconds = r.eval_seconds;
  if (r.nonfinite_step >= 0)
    return fail(MSX_E_NONFINITE, "E-TRAIN-001: " + r.nonfinite_message);
  return MSX_OK;
}
}  // namespace

int msx_train_config_eval(msx_ctx* ctx, const char* config, int64_t steps, uint64_t eval_every, uint64_t eval_batches,
                          float* losses, uint64_t losses_len, uint64_t* eval_steps, msx_heldout* evals,
                          uint64_t evals_len, uint64_t* n_evals, double* train_seconds, double* eval_seconds) {
  return guarded([&] {
    if (eval_every == 0) return fail(MSX_E_INVALID, "eval_every takes a step count of at least 1, not 0");
    return train_run(ctx, config, steps, eval_every, eval_batches, nullptr, losses, losses_len, nullptr, 0, eval_steps,
                     evals, evals_len, n_evals, train_seconds, eval_seconds);
  });
}

int msx_load_packed(msx_ctx* ctx, const char* dir) {
  return guarded([&] {
    ctx->session.reset();
    ctx->corpus.reset();
    if (!dir) return MSX_OK;
    ctx->corpus = std::make_unique<msx::PackedCorpus>(msx::load_packed(dir));
    ctx->orders = msx::EpochOrders();
    return MSX_OK;
  });
}

int msx_write_packed(const char* dir, const int32_t* train, uint64_t train_count, const int32_t* heldout,
                     uint64_t heldout_count, uint64_t seq_len, uint64_t vocabulary_size, const char* dataset_id,
                     const char* tokenizer_id, double selection_rate) {
  return guarded([&] {
    if (!dir || !train || !heldout || !dataset_id || !tokenizer_id) return fail(MSX_E_INVALID, "null argument");
    msx::MaskingPolicy policy;
    policy.selection_rate = selection_rate;
    msx::write_packed(dir, std::vector<int32_t>(train, train + train_count),
                      std::vector<int32_t>(heldout, heldout + heldout_count), seq_len, vocabulary_size, dataset_id,
                      tokenizer_id, policy);
    return MSX_OK;
  });
}

int msx_train_packed(msx_ctx* ctx, const char* config, const char* dir, int64_t steps, uint64_t eval_every,
                     uint64_t eval_batches, float* losses, uint64_t losses_len, float* params, uint64_t params_len,
                     uint64_t* eval_steps, msx_heldout* evals, uint64_t evals_len, uint64_t* n_evals,
                     double* train_seconds, double* eval_seconds) {
  return guarded([&] {
    if (!dir) return fail(MSX_E_INVALID, "null directory");
    ctx->session.reset();
    // The run's own corpus; the context's msx_load_packed binding is left as it was.
    auto corpus = std::make_unique<msx::PackedCorpus>(msx::load_packed(dir));
    const int rc = train_run(ctx, config, steps, eval_every, eval_batches, corpus.get(), losses, losses_len, params,
                             params_len, eval_steps, evals, evals_len, n_evals, train_seconds, eval_seconds);
    ctx->session.reset();  // its feed pointed at the run's corpus
    return rc;
  });
}

namespace {
// The directory of this library's gfx950 code objects: kernels/ beside libmsx.so.
std::string code_object_dir() {
  Dl_info info{};
  if (!dladdr(reinterpret_cast<void*>(&msx_device_count), &info) || !info.dli_fname)
    throw msx::IrError("cannot locate libmsx.so");
  std::string lib = info.dli_fname;
  const size_t slash = lib.find_last_of('/');
  return (slash == std::string::npos ? std::string(".") : lib.substr(0, slash)) + "/kernels";
}
}  // namespace

int msx_write_artifact(msx_ctx* ctx, const char* dir, const char* source_text, char* hash_out) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    if (!dir) return fail(MSX_E_INVALID, "null directory");
    msx::ArtifactSource src;
    src.step_ir = msx::print_step(ctx->step);
    src.forward_ir = msx::print_program(ctx->forward);
    src.source_text = source_text ? source_text : msx::print_program(ctx->forward);
    for (size_t k = 0; k < ctx->forward.outputs.size(); ++k)
      if (ctx->forward.outputs[k] == ctx->prediction) src.prediction_output = uint32_t(k);
    src.param_offsets = ctx->session->param_offsets();
    src.param_floats = ctx->session->param_floats();
    for (auto& l : ctx->session->plan(true)) src.plan.push_back({l.what, l.flop, l.bytes});
    for (auto& l : ctx->session->plan(false)) src.forward_plan.push_back({l.what, l.flop, l.bytes});
    src.code_objects = code_object_dir();
    src.compiler_version = "modelspec-hip 0.1 (hipcc, gfx950)";
    const std::string h = msx::write_artifact(dir, src);
    if (hash_out) std::memcpy(hash_out, h.c_str(), h.size() + 1);
    return MSX_OK;
  });
}

int msx_load_artifact(msx_ctx* ctx, const char* dir, uint64_t seed) {
  return guarded([&] {
    if (!dir) return fail(MSX_E_INVALID, "null directory");
    msx::HipArtifact a = msx::read_artifact(dir, code_object_dir());
    hipDeviceProp_t prop{};
    msx::hip_check(hipGetDeviceProperties(&prop, ctx->device), "hipGetDeviceProperties");
    const std::string arch = prop.gcnArchName;
    if (arch.substr(0, a.target.size()) != a.target || (arch.size() > a.target.size() && arch[a.target.size()] != ':'))
      throw msx::ArtifactError("E-ARTIFACT-005", "the artifact's code objects are for " + a.target + "; the device is " + arch);
    ctx->session.reset();
    ctx->step = msx::parse_step(a.step_ir);
    if (!ctx->step.has_optimizer) return fail(MSX_E_INVALID, "the artifact's step has no optimizer");
    ctx->forward = msx::parse_program(a.forward_ir);
    if (a.prediction_output >= ctx->forward.outputs.size()) return fail(MSX_E_INVALID, "no such forward output");
    ctx->prediction = ctx->forward.outputs[a.prediction_output];
    ctx->seed = seed;
    ctx->session = std::make_unique<msx::Session>(ctx->device, ctx->step, ctx->forward, seed, ctx->prediction, ctx->corpus.get(),
                                                  ctx->options);
    return MSX_OK;
  });
}

int msx_check_artifact(const char* dir, char* artifact_id_out) {
  return guarded([&] {
    if (!dir) return fail(MSX_E_INVALID, "null directory");
    msx::HipArtifact a = msx::read_artifact(dir, code_object_dir());
    if (artifact_id_out) std::memcpy(artifact_id_out, a.artifact_id.c_str(), a.artifact_id.size() + 1);
    return MSX_OK;
  });
}

int msx_checkpoint_write(msx_ctx* ctx, const char* path, uint64_t step) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    if (!path) return fail(MSX_E_INVALID, "null path");
    msx::Session& s = *ctx->session;
    msx::write_checkpoint(path, msx::checkpoint_of(ctx->step, ctx->seed, step, s.params(), s.moments('m'), s.moments('v')));
    return MSX_OK;
  });
}

int msx_checkpoint_read(msx_ctx* ctx, const char* path, int32_t resume, uint64_t* step) {
  return guarded([&] {
    if (!ctx->session) return fail(MSX_E_INVALID, "no step is loaded");
    if (!path) return fail(MSX_E_INVALID, "null path");
    msx::Checkpoint ck = msx::read_checkpoint(path);
    if (resume) {
      msx::ResumeState r = msx::resume_into(ck, ctx->step);
      ctx->session->set_params(r.values);
      if (ctx->step.rule == msx::Rule::AdamW) ctx->session->set_moments(r.m, r.v);
    } else {
      ctx->session->set_params(msx::parameters_for(ck, ctx->step));
    }
    if (step) *step = ck.step;
    return MSX_OK;
  });
}

int msx_train_checkpointed(msx_ctx* ctx, const char* config, const char* packed_dir, int64_t steps, const char* resume,
                           uint64_t checkpoint_every, const char* checkpoint_path, float* losses, uint64_t losses_len,
                           float* params, uint64_t params_len, uint64_t* start_step) {
  return guarded([&] {
    msx::Compiled c = msx::compile_config(config, -1, -1);
    std::unique_ptr<msx::PackedCorpus> corpus;
    if (packed_dir) corpus = std::make_unique<msx::PackedCorpus>(msx::load_packed(packed_dir));
    std::unique_ptr<msx::ResumeState> from;
    if (resume) from = std::make_unique<msx::ResumeState>(msx::resume_into(msx::read_checkpoint(resume), c.step));
    const uint64_t n = steps >= 0 ? uint64_t(steps) : c.config.steps - (from ? std::min(from->step, c.config.steps) : 0);
    ctx->session.reset();
    ctx->step = c.step;
    ctx->forward = c.forward;
    ctx->prediction = c.prediction;
    ctx->seed = c.config.seed;
    ctx->session =
        std::make_unique<msx::Session>(ctx->device, ctx->step, ctx->forward, c.config.seed, c.prediction, corpus.get(),
                                       config_options(ctx, c));
    msx::RunOptions o;
    o.corpus = corpus.get();
    o.resume = from.get();
    o.checkpoint_every = checkpoint_every;
    if (checkpoint_path) o.checkpoint_path = checkpoint_path;
    msx::RunResult r = msx::run(c, *ctx->session, n, o);
    if (corpus) ctx->session.reset();  // its feed pointed at this call's corpus
    if (losses_len < r.losses.size()) return fail(MSX_E_INVALID, "losses buffer too small");
    if (losses) std::memcpy(losses, r.losses.data(), r.losses.size() * 4);
    if (params) {
      uint64_t off = 0;
      for (auto& p : r.params) {
        if (off + p.size() > params_len) return fail(MSX_E_INVALID, "params buffer too small");
        std::memcpy(params + off, p.data(), p.size() * 4);
        off += p.size();
      }
    }
    if (start_step) *start_step = r.start_step;
    if (r.nonfinite_step >= 0)
      return fail(MSX_E_NONFINITE, "E-TRAIN-001: " + r.nonfinite_message);
    return MSX_OK;
  });
}

int msx_train_config(msx_ctx* ctx, const char* config, int64_t steps, int64_t masked_rows, float* losses,
                     uint64_t losses_len, float* params, uint64_t params_len, double* train_seconds) {
  return guarded([&] {
    msx::Compiled c = msx::compile_config(config, masked_rows, steps);
    ctx->session.reset();
    ctx->step = c.step;
    ctx->forward = c.forward;
    ctx->prediction = c.prediction;
    ctx->session = std::make_unique<msx::Session>(ctx->device, ctx->step, ctx->forward, c.config.seed, c.prediction, nullptr,
                                                  config_options(ctx, c));
    msx::RunResult r = msx::run(c, *ctx->session, c.config.steps);
    if (losses_len < r.losses.size()) return fail(MSX_E_INVALID, "losses buffer too small");
    std::memcpy(losses, r.losses.data(), r.losses.size() * 4);
    uint64_t off = 0;
    for (auto& p : r.params) {
      if (off + p.size() > params_len) return fail(MSX_E_INVALID, "params buffer too small");
      std::memcpy(params + off, p.data(), p.size() * 4);
      off += p.size();
    }
    if (train_seconds) *train_seconds = r.train_seconds;
    if (r.nonfinite_step >= 0)
      return fail(MSX_E_NONFINITE, "E-TRAIN-001: " + r.nonfinite_message);
    return MSX_OK;
  });
}

int msx_bench_config(msx_ctx* ctx, const char* config, int64_t masked_rows, uint32_t warmup, uint32_t steps,
                     double* ms_per_step, double* step_ms, float* last_loss, uint32_t profile_reps, char** profile) {
  return guarded([&] {
    uint64_t total = uint64_t(warmup) + steps + std::max<uint32_t>(1, profile_reps);
    msx::Compiled c = msx::compile_config(config, masked_rows, int64_t(std::max<uint64_t>(total, c_steps_floor(config))));
    ctx->session.reset();
    ctx->step = c.step;
    ctx->forward = c.forward;
    ctx->prediction = c.prediction;
    ctx->session = std::make_unique<msx::Session>(ctx->device, ctx->step, ctx->forward, c.config.seed, c.prediction, nullptr,
                                                  config_options(ctx, c));
    msx::Session& s = *ctx->session;
    msx::Feed feed(c);
    if (feed.needs_teacher())
      feed.set_target(s.predict(msx::initialize(c.forward, c.config.seed, msx::Stream::Teacher), feed.batch(0)));
    s.set_params(msx::initialize(c.forward, c.config.seed, msx::Stream::Init));
    const uint64_t end = c.config.steps;
    // Host inputs of every step are made before the timed region: it times the device's steps.
    std::vector<msx::StepInputs> ins;
    for (uint64_t k = 0; k < total; ++k) ins.push_back(msx::step_inputs(c, feed, k, end));
    for (uint32_t k = 0; k < warmup; ++k) s.train_step(ins[k]);
    s.sync();
    // One event after every step: the step times, whose median the benchmark reports.
    std::vector<hipEvent_t> ev(size_t(steps) + 1);
    for (auto& e : ev) msx::hip_check(hipEventCreate(&e), "hipEventCreate");
    msx::hip_check(hipEventRecord(ev[0], s.stream()), "hipEventRecord");
    for (uint32_t k = 0; k < steps; ++k) {
      s.train_step(ins[warmup + k]);
      msx::hip_check(hipEventRecord(ev[k + 1], s.stream()), "hipEventRecord");
    }
    s.sync();
    double total_ms = 0;
    for (uint32_t k = 0; k < steps; ++k) {
      float ms = 0;
      msx::hip_check(hipEventElapsedTime(&ms, ev[k], ev[k + 1]), "hipEventElapsedTime");
      if (step_ms) step_ms[k] = double(ms);
      total_ms += ms;
    }
    for (auto& e : ev) (void)hipEventDestroy(e);
    if (ms_per_step) *ms_per_step = steps ? total_ms / steps : 0.0;
    auto losses = s.losses();
    if (last_loss) *last_loss = losses.empty() ? 0.0f : losses.back();
    if (profile) {
      // Eager steps with an event pair around every launch; each launch's mean over the reps.
      std::vector<msx::Session::Timed> acc;
      uint32_t reps = std::max<uint32_t>(1, profile_reps);
      for (uint32_t r = 0; r < reps; ++r) {
        auto rows = s.profile_step(ins[warmup + steps + r]);
        if (acc.empty()) acc = rows;
        else for (size_t i = 0; i < rows.size(); ++i) acc[i].ms += rows[i].ms;
      }
      std::string text;
      for (auto& t : acc)
        text += t.what + "\t" + std::to_string(t.ms / reps) + "\t" + std::to_string(t.flop) + "\t" + std::to_string(t.bytes) +
                "\t" + t.kernels + "\t" + std::to_string(t.runs) + "\n";
      *profile = dup(text);
    }
    return MSX_OK;
  });
}

int msx_prog_new(msx_ctx* ctx, const char* program_text, uint64_t seed, msx_prog** out) {
  return guarded([&] {
    auto pr = std::make_unique<msx_prog>();
    pr->program = msx::parse_program(program_text);
    msx::TrainingStep none;
    none.program = pr->program;
    none.loss = pr->program.outputs.at(0);
    pr->session = std::make_unique<msx::Session>(ctx->device, none, pr->program, seed, pr->program.outputs.at(0), nullptr,
                                                 ctx->options);
    *out = pr.release();
    return MSX_OK;
  });
}

int msx_prog_run(msx_prog* prog, const msx_tensor* inputs, uint32_t n_inputs, const float* const* params,
                 const uint64_t* param_counts, uint32_t n_params) {
  return guarded([&] {
    std::vector<std::vector<float>> v;
    for (uint32_t i = 0; i < n_params; ++i) v.emplace_back(params[i], params[i] + param_counts[i]);
    prog->session->load_params(v);
    prog->session->run_forward(batch_of(inputs, n_inputs));
    return MSX_OK;
  });
}

int msx_prog_output(msx_prog* prog, uint32_t k, float* out, uint64_t count) {
  return guarded([&] {
    uint32_t v = prog->program.outputs.at(k);
    if (prog->program.node(v).ty.count() != int64_t(count)) return fail(MSX_E_INVALID, "output count");
    msx::hip_check(hipMemcpy(out, prog->session->forward_value(v), count * 4, hipMemcpyDeviceToHost), "hipMemcpy (output)");
    return MSX_OK;
  });
}

void msx_prog_free(msx_prog* prog) {
  try {
    delete prog;
  } catch (...) {
  }
}

}  // extern "C"
