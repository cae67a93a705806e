// The host side of a training run: parameter initialization, the synthetic batches of each
// config, the per-step host inputs (dropout tokens, AdamW scalars, the masked-row gather) and the
// step loop, over an Engine that executes the compiled step.
//
// Restates crates/modelspec-runtime/src/train/runner.rs:365-470 (loop semantics: the loss of
// step k is the loss before update k; the final loss is the dropout-free forward program on the
// final parameters), train/init.rs:335-352 (initialize), train/data.rs:189-211 (teacher data),
// train/masked.rs:58-118 (host gather) and dataset/mlm.rs:717-788 (BERT masking rule).
#pragma once
#include <map>
#include <string>
#include <vector>

#include "models.h"
#include "packed.h"
#include "rng.h"

namespace msx {

struct Batch {
  std::map<std::string, std::vector<float>> f32;
  std::map<std::string, std::vector<int32_t>> i32;
};

// Initial parameter values by ParamId: xavier draws on `stream`, zeros, ones (init.rs:335-352).
std::vector<std::vector<float>> initialize(const Program& p, uint64_t seed, Stream stream);

// The synthetic batch source of a compiled config.
class Feed {
 public:
  explicit Feed(const Compiled& c);
  // Batches drawn from a packed corpus on the device: each batch is only kDrawInput, the step's
  // sequences of the epoch order (mlm.rs:717-760); `corpus` outlives the feed.
  Feed(const Compiled& c, const PackedCorpus* corpus, uint64_t batch);
  const PackedCorpus* corpus() const { return corpus_; }
  uint64_t corpus_batch() const { return corpus_batch_; }
  // The batch of step `step` (Teacher and Classifier data are the same every step).
  Batch batch(uint64_t step) const;
  // Batch `b` of the held-out split: the batch drawn at step id 2^63 + b, the id the reference
  // gives the masking of held-out batch b (train/eval.rs:6-10), so no training step draws it.
  Batch held_out(uint64_t b) const;
  // Teacher data: the input tensor and the (zero) target before set_target.
  void set_target(std::vector<float> y) { target_ = std::move(y); }
  bool needs_teacher() const { return cfg_.feed == FeedKind::Teacher; }

 private:
  TrainConfig cfg_;
  const PackedCorpus* corpus_ = nullptr;
  uint64_t corpus_batch_ = 0;
  mutable EpochOrders orders_;
  std::vector<double> zipf_cdf_;
  std::vector<float> x_, target_;
  std::vector<int32_t> labels_;
  int64_t x_count_ = 0, y_count_ = 0;
  int32_t zipf(uint64_t step, uint32_t row, uint64_t draw) const;
};

// The masked-row gather of one batch (train/masked.rs:97-118): rows of non-zero weight
// ascending, then padding rows 0 / label 0 / weight +0.0 up to `capacity`; more selected rows than
// the capacity is refused with an IrError naming E-DATA-012.
void masked_gather(const std::vector<int32_t>& labels, const std::vector<float>& weights, uint64_t capacity,
                   uint64_t step, std::vector<int32_t>& rows, std::vector<int32_t>& out_labels,
                   std::vector<float>& out_weights);

// Held-out evaluation (crates/modelspec-runtime/src/train/eval.rs): the forward program, the one
// without dropout, over every held-out batch; the loss is sum(w_n nll_n) / sum(w_n) over every row
// of every batch, both sums in f64, rounded to f32 once (0 when the weight sum is 0); the
// accuracy is correct / selected over the rows of positive weight, a row correct when the first
// largest logit of its row (lowest id among ties) is its label and the row holds no NaN.
struct HeldOutMetrics {
  float loss = 0, accuracy = 0;
};

// What a device reduces the logits of an evaluation to (eval.rs:299-339, metrics_of_sums): the
// weighted sum of the row losses and the count of correct rows of positive weight.
struct HeldOutSums {
  double numerator = 0;
  uint64_t correct = 0;
  // The weight sum and the rows of positive weight, when the reducer summed them too (batches
  // drawn on the device carry no weights on the host).
  double denominator = 0;
  uint64_t selected = 0;
  bool has_totals = false;
};

// The held-out batches of a run, drawn once (HeldOut::new, eval.rs:166-198): their labels and
// weights are what the reduction reads, by the config's input names.
class HeldOut {
 public:
  // Draws `batches` held-out batches of `feed` (of a corpus feed: 0 draws every whole batch of
  // the HeldOut split, eval.rs:6-12); the prediction must be f32 logits [rows, V] with one row per
  // label of a batch (eval.rs:148-163), else an IrError.
  HeldOut(const Compiled& c, const Feed& feed, uint64_t batches);
  // Batches the caller drew (HeldOut::batch hands the reference's own to a device, eval.rs:290),
  // with the labels and weights under the given input names of `forward`.
  HeldOut(const Program& forward, uint32_t prediction, std::string labels, std::string weights,
          std::vector<Batch> batches);
  const std::vector<Batch>& batches() const { return batches_; }
  const std::string& labels_name() const { return labels_; }
  const std::string& weights_name() const { return weights_; }
  int64_t classes() const { return classes_; }
  // The metrics of sums reduced elsewhere (eval.rs:299-339): the denominator and the selected
  // rows from the batches' own weights; a label outside [0, classes) is refused, the first in
  // batch and row order (DataError naming the batch and row).
  HeldOutMetrics metrics_of_sums(const HeldOutSums& sums) const;
  // The same label check alone, before any batch runs.
  void check_labels() const;

 private:
  std::vector<Batch> batches_;
  std::string labels_, weights_;
  int64_t classes_ = 0;
  void check_program(const Program& forward, uint32_t prediction);
};

// A held-out label outside the classes (EvalError::Label, eval.rs:84-91).
struct HeldOutLabelError : IrError {
  using IrError::IrError;
};

// Everything one training step reads besides parameters and moments.
struct StepInputs {
  Batch batch;  // declared data, gathered rows, dropout tokens, AdamW scalars, by input name
};

// Builds the inputs of training step `step` of a run ending at `end` (runner.rs:410-440).
StepInputs step_inputs(const Compiled& c, const Feed& feed, uint64_t step, uint64_t end);

// What executes the compiled step: the HIP device runtime, or the CPU oracle in tests.
class Engine {
 public:
  virtual ~Engine() = default;
  // Parameter values by ParamId; AdamW moments restart at zero.
  virtual void set_params(const std::vector<std::vector<float>>& values) = 0;
  virtual std::vector<std::vector<float>> params() = 0;
  // Moments by ParamId (empty for SGD): first then second.
  virtual std::vector<std::vector<float>> moments(char which) = 0;
  // The forward program's prediction under `values` on `batch` (synthetic teacher targets).
  virtual std::vector<float> predict(const std::vector<std::vector<float>>& values, const Batch& batch) = 0;
  // One training step: loss of the current parameters, then their update. The loss may be
  // collected later by losses().
  virtual void train_step(const StepInputs& in) = 0;
  // The forward program's loss on the current parameters, after every queued step.
  virtual float final_loss(const Batch& batch) = 0;
  // The losses of the train steps run since set_params, in order.
  virtual std::vector<float> losses() = 0;
  // The held-out sums of the forward program on the current parameters, after every queued step.
  virtual HeldOutSums held_out(const HeldOut& h) = 0;
  // AdamW moments by ParamId (empty entries: parameters without moments), after set_params.
  virtual void set_moments(const std::vector<std::vector<float>>& m, const std::vector<std::vector<float>>& v) = 0;
};

struct RunResult {
  std::vector<std::vector<float>> initial;
  std::vector<float> losses;  // steps + 1
  std::vector<std::vector<float>> params;
  double train_seconds = 0;   // wall clock of the step loop (runner.rs loop; train.rs:17-31 --clock)
  int64_t nonfinite_step = -1;  // the step whose loss was not finite (absolute step number)
  // With nonfinite_step: what was not finite, in the reference's words and order (runner.rs:156-
  // 227): the loss, else the parameters by canonical path ("@path", in path order), else the AdamW
  // moments ("m @path" / "v @path", in path order, m before v).
  std::string nonfinite_message;
  uint64_t start_step = 0;       // the step the run started at (a resumed run's checkpoint step)
  std::vector<std::string> checkpoints;  // paths written, in order
  // Held-out metrics at every step k with k % eval_every == 0 and at the last step, on the
  // parameters after k updates (crates/modelspec-cli/src/train.rs:1293-1312).
  std::vector<std::pair<uint64_t, HeldOutMetrics>> evals;
  double eval_seconds = 0;    // wall clock of the evaluations, outside train_seconds
};

struct ResumeState;

// What a run does besides training: held-out evaluation every `eval_every` steps over
// `eval_batches` batches, batches drawn from `corpus`, a start from a checkpoint's state
// (`resume`: `steps` then counts the steps of this invocation, which ends at resume->step +
// steps, train.rs:549-550), and checkpoints: `<stem>-<k>.msckpt` after every `checkpoint_every`
// updates before the end, `checkpoint_path` itself at the end (train.rs:538-542, 1075, 1285).
struct RunOptions {
  uint64_t eval_every = 0, eval_batches = 0;
  const PackedCorpus* corpus = nullptr;
  const ResumeState* resume = nullptr;
  uint64_t checkpoint_every = 0;
  std::string checkpoint_path;
};
RunResult run(const Compiled& c, Engine& engine, uint64_t steps, const RunOptions& options);
// The path of the checkpoint after k updates: `<stem>-<k>.msckpt` beside `path`.
std::string checkpoint_every_path(const std::string& path, uint64_t k);

// eval_every = 0: no evaluation; else `eval_batches` held-out batches (at least 1; 0 with a corpus:
// every whole batch of its HeldOut split). With `corpus`, the batches are drawn from it
// (mlm_batch, mlm.rs:717-788) instead of the config's synthetic data.
RunResult run(const Compiled& c, Engine& engine, uint64_t steps, uint64_t eval_every = 0, uint64_t eval_batches = 0,
              const PackedCorpus* corpus = nullptr);

}  // namespace msx
