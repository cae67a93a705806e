// Host side of a run. See runner.h.
#include "runner.h"

#include "checkpoint.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <memory>

namespace msx {

std::vector<std::vector<float>> initialize(const Program& p, uint64_t seed, Stream stream) {
  std::vector<std::vector<float>> out;
  for (auto& d : p.params) {
    int64_t n = d.ty.count();
    if (n > (int64_t(1) << 32)) throw IrError("`" + d.path + "` has more elements than a draw addresses");
    switch (d.init) {
      case Init::XavierUniform:
        if (d.ty.rank() != 2) throw IrError("`" + d.path + "`: xavier_uniform needs rank 2 [In, Out]");
        out.push_back(xavier_uniform(seed, stream, d.path, d.ty.shape[0], d.ty.shape[1]));
        break;
      case Init::Zeros: out.emplace_back(size_t(n), 0.0f); break;
      case Init::Ones: out.emplace_back(size_t(n), 1.0f); break;
    }
  }
  return out;
}

Feed::Feed(const Compiled& c) : cfg_(c.config) {
  const Program& fwd = c.forward;
  if (cfg_.feed == FeedKind::Teacher) {
    const Node* x = fwd.input(cfg_.x);
    const Node* y = fwd.input(cfg_.y);
    if (!x || !y) throw IrError("teacher data needs the input and the target");
    x_count_ = x->ty.count();
    y_count_ = y->ty.count();
    x_ = standard_normal(cfg_.seed, Stream::Data, cfg_.x, x_count_);
    target_.assign(size_t(y_count_), 0.0f);
  } else if (cfg_.feed == FeedKind::Classifier) {
    int64_t n = cfg_.batch * cfg_.features;
    uint64_t xid = canonical_id(cfg_.x), lid = canonical_id(cfg_.labels);
    x_.resize(size_t(n));
    for (int64_t i = 0; i < n; ++i)
      x_[size_t(i)] = float(uniform_word(philox_block(cfg_.seed, Stream::Data, xid, uint32_t(i)).w[0]));
    labels_.resize(size_t(cfg_.batch));
    for (int64_t i = 0; i < cfg_.batch; ++i) {
      uint64_t w = philox_block(cfg_.seed, Stream::Data, lid, uint32_t(i)).w[0];
      labels_[size_t(i)] = int32_t((w * uint64_t(cfg_.classes)) >> 32);
    }
  } else {
    // Zipf(s) over ranks 1..M, rank r -> token first_token + r - 1; the CDF summed ascending in f64.
    int64_t M = cfg_.vocab - cfg_.first_token;
    zipf_cdf_.resize(size_t(M));
    double acc = 0;
    for (int64_t r = 1; r <= M; ++r) {
      acc += std::pow(double(r), -cfg_.zipf_s);
      zipf_cdf_[size_t(r - 1)] = acc;
    }
    for (auto& v : zipf_cdf_) v /= acc;
    zipf_cdf_.back() = 1.0;
  }
}

int32_t Feed::zipf(uint64_t step, uint32_t row, uint64_t draw) const {
  (void)step;
  double u = uniform_word(philox_block(cfg_.seed, Stream::Data, draw, row).w[0]);
  auto it = std::lower_bound(zipf_cdf_.begin(), zipf_cdf_.end(), u);
  int64_t r = int64_t(it - zipf_cdf_.begin());
  if (r >= int64_t(zipf_cdf_.size())) r = int64_t(zipf_cdf_.size()) - 1;
  return int32_t(cfg_.first_token + r);
}

Feed::Feed(const Compiled& c, const PackedCorpus* corpus, uint64_t batch)
    : cfg_(c.config), corpus_(corpus), corpus_batch_(batch) {
  if (!corpus || batch == 0) throw IrError("a corpus feed needs a corpus and a batch of at least one sequence");
}

Batch Feed::held_out(uint64_t b) const {
  if (corpus_) {
    Batch out;
    out.i32[kDrawInput] = draw_words(SplitRole::HeldOut, orders_.draw(*corpus_, SplitRole::HeldOut, cfg_.seed, b, corpus_batch_));
    return out;
  }
  return batch((uint64_t(1) << 63) + b);
}

Batch Feed::batch(uint64_t step) const {
  Batch b;
  if (corpus_) {
    b.i32[kDrawInput] = draw_words(SplitRole::Train, orders_.draw(*corpus_, SplitRole::Train, cfg_.seed, step, corpus_batch_));
    return b;
  }
  switch (cfg_.feed) {
    case FeedKind::Teacher:
      b.f32[cfg_.x] = x_;
      b.f32[cfg_.y] = target_;
      break;
    case FeedKind::Classifier:
      b.f32[cfg_.x] = x_;
      b.i32[cfg_.labels] = labels_;
      b.f32[cfg_.weights].assign(size_t(cfg_.batch), 1.0f);
      break;
    case FeedKind::NextToken:
    case FeedKind::MaskedLm: {
      int64_t B = cfg_.batch, S = cfg_.seq, N = B * S;
      uint64_t draw = dropout_id(cfg_.ids, step);  // per-step draw id of the token stream
      std::vector<int32_t> tokens(static_cast<size_t>(N));
      for (int64_t r = 0; r < N; ++r) tokens[size_t(r)] = zipf(step, uint32_t(r), draw);
      std::vector<int32_t> ids(static_cast<size_t>(N)), positions(static_cast<size_t>(N)), labels(static_cast<size_t>(N));
      std::vector<float> weights(static_cast<size_t>(N)), mask(static_cast<size_t>(N), 1.0f);
      for (int64_t r = 0; r < N; ++r) positions[size_t(r)] = int32_t(r % S);
      if (cfg_.feed == FeedKind::NextToken) {
        for (int64_t r = 0; r < N; ++r) {
          ids[size_t(r)] = tokens[size_t(r)];
          bool last = (r % S) == S - 1;
          labels[size_t(r)] = last ? 0 : tokens[size_t(r + 1)];
          weights[size_t(r)] = last ? 0.0f : 1.0f;
        }
      } else {
        // dataset/mlm.rs:766-785 with MaskingPolicy::BERT (mlm.rs:67-72), [MASK] = 4, five specials.
        const double selection = 0.15, mask_fraction = 0.8, random_fraction = 0.1;
        const uint64_t specials = 5, random_tokens = uint64_t(cfg_.vocab) - specials;
        for (int64_t r = 0; r < N; ++r) {
          int32_t label = tokens[size_t(r)];
          Philox4 w = philox_block(cfg_.seed, Stream::Masking, step, uint32_t(r));
          bool selected = label >= int32_t(specials) && uniform_word(w.w[0]) < selection;
          int32_t id;
          if (!selected) id = label;
          else if (uniform_word(w.w[1]) < mask_fraction) id = 4;
          else if (uniform_word(w.w[1]) < mask_fraction + random_fraction)
            id = int32_t(specials + ((uint64_t(w.w[2]) * random_tokens) >> 32));
          else id = label;
          ids[size_t(r)] = id;
          labels[size_t(r)] = label;
          weights[size_t(r)] = selected ? 1.0f : 0.0f;
        }
      }
      b.i32[cfg_.ids] = ids;
      b.i32[cfg_.positions] = positions;
      b.f32[cfg_.key_mask] = mask;
      b.i32[cfg_.labels] = labels;
      b.f32[cfg_.weights] = weights;
      break;
    }
  }
  return b;
}

void masked_gather(const std::vector<int32_t>& labels, const std::vector<float>& weights, uint64_t capacity,
                   uint64_t step, std::vector<int32_t>& rows, std::vector<int32_t>& out_labels,
                   std::vector<float>& out_weights) {
  size_t selected = 0;
  for (float w : weights) selected += w != 0.0f;
  if (selected > capacity)
    throw IrError("E-DATA-012: the batch of step " + std::to_string(step) + " has " + std::to_string(selected) +
                  " rows of non-zero weight, more than the " + std::to_string(capacity) +
                  " rows the masked-row gather holds");
  rows.clear();
  out_labels.clear();
  out_weights.clear();
  for (size_t r = 0; r < weights.size(); ++r)
    if (weights[r] != 0.0f) {
      rows.push_back(int32_t(r));
      out_labels.push_back(r < labels.size() ? labels[r] : 0);
      out_weights.push_back(weights[r]);
    }
  rows.resize(capacity, 0);
  out_labels.resize(capacity, 0);
  out_weights.resize(capacity, 0.0f);
}

HeldOut::HeldOut(const Compiled& c, const Feed& feed, uint64_t batches)
    : labels_(c.config.labels), weights_(c.config.weights) {
  if (const PackedCorpus* corpus = feed.corpus()) {
    const uint64_t whole = corpus->sequences(SplitRole::HeldOut) / feed.corpus_batch();
    if (whole == 0)
      throw PackedError(corpus->dir + ": the HeldOut split holds " + std::to_string(corpus->sequences(SplitRole::HeldOut)) +
                        " sequences, fewer than the batch of " + std::to_string(feed.corpus_batch()) +
                        " that an evaluation reads");
    batches = batches == 0 ? whole : std::min(batches, whole);
  }
  if (batches == 0) throw IrError("held-out evaluation needs at least one batch");
  check_program(c.forward, c.prediction);
  batches_.reserve(size_t(batches));
  for (uint64_t b = 0; b < batches; ++b) batches_.push_back(feed.held_out(b));
}

HeldOut::HeldOut(const Program& forward, uint32_t prediction, std::string labels, std::string weights,
                 std::vector<Batch> batches)
    : batches_(std::move(batches)), labels_(std::move(labels)), weights_(std::move(weights)) {
  if (batches_.empty()) throw IrError("held-out evaluation needs at least one batch");
  check_program(forward, prediction);
  const int64_t rows = forward.input(labels_)->ty.count();
  for (size_t b = 0; b < batches_.size(); ++b) {
    if (batches_[b].i32.count(kDrawInput)) continue;  // drawn on the device
    auto l = batches_[b].i32.find(labels_);
    auto w = batches_[b].f32.find(weights_);
    if (l == batches_[b].i32.end() || w == batches_[b].f32.end() || int64_t(l->second.size()) != rows ||
        int64_t(w->second.size()) != rows)
      throw IrError("held-out batch " + std::to_string(b) + " lacks " + std::to_string(rows) + " labels `" + labels_ +
                    "` and weights `" + weights_ + "`");
  }
}

void HeldOut::check_program(const Program& forward, uint32_t prediction) {
  const Node& pred = forward.node(prediction);
  const Node* lab = forward.input(labels_);
  const Node* w = forward.input(weights_);
  if (labels_.empty() || weights_.empty() || !lab || !w || lab->ty.dtype != DType::I32 || w->ty.dtype != DType::F32)
    throw IrError("held-out evaluation reads the i32 labels and f32 weights of a cross-entropy loss");
  const int64_t rows = lab->ty.count();
  if (pred.ty.dtype != DType::F32 || pred.ty.rank() != 2 || pred.ty.shape[0] != rows || pred.ty.shape[1] <= 0 ||
      w->ty.count() != rows)
    throw IrError("held-out evaluation reads the prediction as f32 logits [" + std::to_string(rows) +
                  ", V], one row per position of the batch; the prediction is " + type_string(pred.ty));
  classes_ = pred.ty.shape[1];
}

void HeldOut::check_labels() const {
  for (size_t b = 0; b < batches_.size(); ++b) {
    auto it = batches_[b].i32.find(labels_);
    if (it == batches_[b].i32.end()) continue;  // drawn on the device from a checked corpus
    const auto& labels = it->second;
    for (size_t n = 0; n < labels.size(); ++n)
      if (labels[n] < 0 || labels[n] >= classes_)
        throw HeldOutLabelError("held-out batch " + std::to_string(b) + ", row " + std::to_string(n) + ": label " +
                                std::to_string(labels[n]) + " is not below the " + std::to_string(classes_) +
                                " classes");
  }
}

HeldOutMetrics HeldOut::metrics_of_sums(const HeldOutSums& sums) const {
  check_labels();
  // eval.rs:430-449: the denominator summed from its first term in batch and row order.
  double den = 0;
  bool first = true;
  uint64_t selected = 0;
  bool host_weights = true;
  for (auto& b : batches_) host_weights = host_weights && b.f32.count(weights_);
  if (!host_weights) {
    if (!sums.has_totals) throw IrError("held-out sums without the weight totals of batches drawn on the device");
    den = sums.denominator;
    selected = sums.selected;
  } else {
    for (auto& b : batches_)
      for (float w : b.f32.at(weights_)) {
        den = first ? double(w) : den + double(w);
        first = false;
        if (w > 0.0f) ++selected;
      }
  }
  HeldOutMetrics m;
  m.loss = den == 0.0 ? 0.0f : float(sums.numerator / den);
  m.accuracy = selected == 0 ? 0.0f : float(sums.correct) / float(selected);
  return m;
}

StepInputs step_inputs(const Compiled& c, const Feed& feed, uint64_t step, uint64_t end) {
  StepInputs in;
  in.batch = feed.batch(step);
  const Program& p = c.step.program;
  const bool on_device = in.batch.i32.count(kDrawInput) != 0;  // the device draws and gathers
  if (const Node* rows = on_device ? nullptr : p.input(kMaskedRowsInput)) {
    const auto& cfg = c.config;
    std::vector<int32_t> r, l;
    std::vector<float> w;
    masked_gather(in.batch.i32.at(cfg.labels), in.batch.f32.at(cfg.weights), uint64_t(rows->ty.count()), step, r, l, w);
    in.batch.i32[kMaskedRowsInput] = std::move(r);
    in.batch.i32[std::string(kMaskedLabelsPrefix) + cfg.labels] = std::move(l);
    in.batch.f32[std::string(kMaskedWeightsPrefix) + cfg.weights] = std::move(w);
  }
  for (auto& site : dropout_sites(p)) {
    int32_t t[2];
    dropout_token(site, step, t);
    in.batch.i32[site] = {t[0], t[1]};
  }
  if (c.step.rule == Rule::AdamW) {
    StepScalars s = adamw_scalars(c.step.adamw, c.step.lr, step + 1, end);
    in.batch.f32[kLrTInput] = {s.lr_t};
    in.batch.f32[kC1Input] = {s.c1};
    in.batch.f32[kC2Input] = {s.c2};
  }
  return in;
}

RunResult run(const Compiled& c, Engine& engine, uint64_t steps, uint64_t eval_every, uint64_t eval_batches,
              const PackedCorpus* corpus) {
  RunOptions o;
  o.eval_every = eval_every;
  o.eval_batches = eval_batches;
  o.corpus = corpus;
  return run(c, engine, steps, o);
}

std::string checkpoint_every_path(const std::string& path, uint64_t k) {
  const size_t slash = path.find_last_of('/');
  const size_t dot = path.find_last_of('.');
  const std::string stem = dot != std::string::npos && (slash == std::string::npos || dot > slash + 1)
                               ? path.substr(0, dot)
                               : path;
  return stem + "-" + std::to_string(k) + ".msckpt";
}

RunResult run(const Compiled& c, Engine& engine, uint64_t steps, const RunOptions& o) {
  RunResult out;
  const uint64_t start = o.resume ? o.resume->step : 0;
  const uint64_t end = start + steps;
  out.start_step = start;
  if (c.step.rule == Rule::AdamW && end > 0 && c.step.adamw.warmup_steps >= end)
    throw IrError("the warmup of " + std::to_string(c.step.adamw.warmup_steps) +
                  " steps is not shorter than the run of " + std::to_string(end) + " steps");
  out.initial = o.resume ? o.resume->values : initialize(c.forward, c.config.seed, Stream::Init);
  Feed feed = o.corpus ? Feed(c, o.corpus, bind_corpus(c.forward, *o.corpus)) : Feed(c);
  if (feed.needs_teacher()) {
    auto teacher = initialize(c.forward, c.config.seed, Stream::Teacher);
    feed.set_target(engine.predict(teacher, feed.batch(0)));
  }
  // Drawn once, before the first step, so a split the evaluation refuses stops the run first.
  std::unique_ptr<HeldOut> held_out;
  if (o.eval_every) {
    held_out = std::make_unique<HeldOut>(c, feed, o.eval_batches);
    held_out->check_labels();
  }
  double left_out = 0;  // evaluation and checkpoint time, outside the training clock
  auto evaluate = [&](uint64_t step) {
    auto e0 = std::chrono::steady_clock::now();
    out.evals.emplace_back(step, held_out->metrics_of_sums(engine.held_out(*held_out)));
    const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - e0).count();
    out.eval_seconds += dt;
    left_out += dt;
  };
  // The state after k updates (train.rs:1075, 1285: `<stem>-<k>.msckpt` every n updates before
  // the end, the checkpoint path itself at the end).
  // Losses stay on the device between read-backs, as the reference's Vulkan runner keeps them
  // (cli/src/train.rs:39-44): every loss so far, the parameters and the AdamW moments are checked
  // where they are read back, at each checkpoint and after the last step (runner.rs:156-227 checks
  // each step on the host). A non-finite loss names its own step; a non-finite parameter or moment
  // under finite losses names the step of the read-back that showed it. Returns false, with
  // out.nonfinite_step, out.nonfinite_message and the losses through that step set, on the first.
  auto finite_through = [&](uint64_t k, const std::vector<float>& losses, const std::vector<std::vector<float>>& params,
                            bool with_moments) {
    for (size_t i = 0; i < losses.size(); ++i)
      if (!std::isfinite(losses[i])) {
        out.nonfinite_step = int64_t(start + i);
        out.nonfinite_message = "the loss of step " + std::to_string(start + i) + " is not finite";
        out.losses.assign(losses.begin(), losses.begin() + i + 1);
        return false;
      }
    auto finite = [](const std::vector<float>& v) {
      for (float x : v)
        if (!std::isfinite(x)) return false;
      return true;
    };
    const auto& decls = c.step.program.params;
    std::vector<std::string> bad;
    for (size_t q = 0; q < params.size() && q < decls.size(); ++q)
      if (!finite(params[q])) bad.push_back("@" + decls[q].path);
    std::string what = "parameter";
    if (bad.empty() && with_moments && c.step.rule == Rule::AdamW) {
      const auto m = engine.moments('m'), v = engine.moments('v');
      std::vector<std::pair<std::string, char>> named;
      for (size_t q = 0; q < decls.size(); ++q) {
        if (q < m.size() && !finite(m[q])) named.emplace_back(decls[q].path, 'm');
        if (q < v.size() && !finite(v[q])) named.emplace_back(decls[q].path, 'v');
      }
      std::sort(named.begin(), named.end());
      for (auto& [path, mo] : named) bad.push_back(std::string(1, mo) + " @" + path);
      what = "optimizer moment";
    } else {
      std::sort(bad.begin(), bad.end());
    }
    if (bad.empty()) return true;
    std::string list;
    for (auto& b : bad) list += (list.empty() ? "" : ", ") + b;
    out.nonfinite_step = int64_t(k);
    out.nonfinite_message = "the update of step " + std::to_string(k) + " leaves " +
                            (what == "parameter" ? "a parameter" : "an optimizer moment") + " not finite: " + list;
    out.losses = losses;
    return false;
  };
  // Writes the state after k updates unless a loss or parameter read back is not finite; then
  // nothing is written and the run stops (returns false).
  auto checkpoint = [&](uint64_t k, const std::string& path) {
    auto w0 = std::chrono::steady_clock::now();
    std::vector<std::vector<float>> params = engine.params();
    if (!finite_through(k, engine.losses(), params, true)) return false;
    Checkpoint ck = checkpoint_of(c.step, c.config.seed, k, params, engine.moments('m'), engine.moments('v'));
    write_checkpoint(path, ck);
    out.checkpoints.push_back(path);
    left_out += std::chrono::duration<double>(std::chrono::steady_clock::now() - w0).count();
    return true;
  };
  engine.set_params(out.initial);
  if (o.resume && c.step.rule == Rule::AdamW) engine.set_moments(o.resume->m, o.resume->v);
  auto t0 = std::chrono::steady_clock::now();
  for (uint64_t step = start; step < end; ++step) {
    if (held_out && step % o.eval_every == 0) evaluate(step);
    if (o.checkpoint_every && step > start && step % o.checkpoint_every == 0 && !o.checkpoint_path.empty() &&
        !checkpoint(step, checkpoint_every_path(o.checkpoint_path, step)))
      return out;
    engine.train_step(step_inputs(c, feed, step, end));
  }
  out.losses = engine.losses();
  auto t1 = std::chrono::steady_clock::now();
  out.train_seconds = std::chrono::duration<double>(t1 - t0).count() - left_out;
  if (held_out) evaluate(end);
  Batch last = feed.batch(end);
  // The final batch is held to the gather's capacity as every trained batch is (runner.rs:462):
  // masked_gather throws E-DATA-012 on a batch the step's gather could not hold. Its rows are
  // not used: the final loss runs the forward program over every row.
  if (const Node* rows = last.i32.count(kDrawInput) ? nullptr : c.step.program.input(kMaskedRowsInput)) {
    std::vector<int32_t> r, l;
    std::vector<float> w;
    masked_gather(last.i32.at(c.config.labels), last.f32.at(c.config.weights), uint64_t(rows->ty.count()), end, r, l, w);
  }
  out.params = engine.params();
  if (!finite_through(end, out.losses, out.params, true)) return out;
  out.losses.push_back(engine.final_loss(last));
  if (!finite_through(end, out.losses, {}, false)) return out;
  if (!o.checkpoint_path.empty()) checkpoint(end, o.checkpoint_path);
  return out;
}

}  // namespace msx
