// The HIP device runtime: executes a compiled training step (and its forward program) on one
// MI355X. It replaces the reference's Vulkan stepwise runner
// (crates/modelspec-runtime/src/vulkan/stepwise.rs:289-400, 975-1551): parameters and AdamW
// moments stay resident in HBM for the whole run, each step's host inputs are packed into one
// pinned staging slot and copied in one transfer, and the step's kernels are captured once into a
// hipGraph and relaunched every step.
#pragma once
#include <hip/hip_runtime.h>

#include <functional>
#include <map>
#include <set>
#include <memory>
#include <string>
#include <vector>

#include "../host/packed.h"
#include "../host/runner.h"
#include "kernels.h"

namespace msx {

struct HipError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void hip_check(hipError_t e, const char* what);

// One device allocation carved by a bump allocator; everything a plan needs is reserved when the
// plan is built, so a captured step never allocates.
class DeviceArena {
 public:
  ~DeviceArena();
  void* reserve(size_t bytes);  // 256-byte aligned, zero-initialized at commit()
  void commit();                // one hipMalloc of everything reserved
  void* at(void* token) const;  // device address of a reservation
  size_t bytes() const { return size_; }
  static size_t offset(void* token) { return reinterpret_cast<size_t>(token) - 1; }

 private:
  size_t size_ = 0;
  char* base_ = nullptr;
};

struct Launch {
  std::string what;  // op name and value, for profiles and errors
  std::function<void(hipStream_t)> run;
  // Algorithmic work of the node this launch completes, by the reference's counting rule
  // (crates/modelspec-core/src/ir/kernel.rs:1221, 1565): 2mnk for a matmul, 4 / 8 B heads L S d
  // for attention forward / backward, bytes of the values read and written otherwise.
  double flop = 0, bytes = 0;
  // A launch whose outputs only the optimizer reads (a weight gradient): in a step it runs on the
  // session's side stream, after work launched before it on the main stream, so that it overlaps
  // the rest of the backward; the main stream joins it before the optimizer.
  bool side = false;
  // A launch whose outputs are none of its inputs (a GEMM, attention): running it again recomputes
  // the same values, so a profile may time it over back-to-back repeats.
  bool pure = false;
};

struct RunStats {
  uint64_t steps = 0, graph_launches = 0, kernels_per_step = 0, bytes_uploaded = 0, device_bytes = 0;
};

class Executor;

// A loaded training run on one device.
// How a session computes: `mixed` runs every GEMM on the f16 MFMA (operands rounded to f16, f32
// accumulation, f32 values in HBM) with dynamic loss scaling of the gradients, starting at
// `loss_scale` and doubling after `scale_window` steps without an overflow.
struct SessionOptions {
  bool mixed = false;
  float loss_scale = 65536.0f;
  uint32_t scale_window = 2000;
  // Cross-entropy fused into its decoder head GEMMs (Executor::build).
  bool fuse_ce_head = false;
  bool fuse_optimizer = true;  // the deferred column finalize inside the AdamW launch
  // Plan only: the step and forward programs are planned (launches, fusions, buffer offsets) and
  // nothing touches a device; such a session can print its plans and cannot run.
  bool plan_only = false;
};

class Session : public Engine {
 public:
  // With `corpus`, the batch tensors of both programs (ids, positions, key_mask, labels, weights)
  // and the masked-row gather are drawn on the device from the corpus, resident in HBM; each
  // step then stages kDrawInput instead of its batch.
  Session(int device, const TrainingStep& step, const Program& forward, uint64_t seed, uint32_t prediction,
          const PackedCorpus* corpus = nullptr, SessionOptions options = SessionOptions());
  ~Session() override;

  void set_params(const std::vector<std::vector<float>>& values) override;
  std::vector<std::vector<float>> params() override;
  std::vector<std::vector<float>> moments(char which) override;
  void set_moments(const std::vector<std::vector<float>>& m, const std::vector<std::vector<float>>& v) override;
  std::vector<float> predict(const std::vector<std::vector<float>>& values, const Batch& batch) override;
  void train_step(const StepInputs& in) override;
  float final_loss(const Batch& batch) override;
  // The forward program over every held-out batch, each batch's logits reduced on the device to
  // the row losses and hits (held_out_rows) and added into one f64 sum and one count
  // (held_out_sum); one host wait at the end (vulkan/stepwise.rs:1635-1760 does the same with its
  // HeldOutRows / HeldOutSum modules).
  HeldOutSums held_out(const HeldOut& h) override;
  // held_out with the row results and the sums in the library's static device array instead of
  // a buffer of the session: no device memory is allocated. At most kStaticEvalRows rows a batch;
  // every call on one device shares the array, so calls that overlap on a device race.
  HeldOutSums held_out_static(const HeldOut& h);
  static constexpr int64_t kStaticEvalRows = 65536;
  std::vector<float> losses() override;
  // The plans of a plan-only (or any) session: the step's, then the forward program's.
  std::string plan_text() const;

  // Runs the step plan eagerly (no graph) with one event pair around every launch; returns the
  // launches and their milliseconds for the current inputs (the step's update is applied).
  // runs: how many times the profiled step ran the launch (1, or 1 + the repeats of a pure one).
  struct Timed { std::string what; float ms; double flop, bytes; std::string kernels; int runs; };
  std::vector<Timed> profile_step(const StepInputs& in);
  void use_graph(bool on) { use_graph_ = on; }
  void sync();
  hipStream_t stream() const { return stream_; }
  const RunStats& stats() const { return stats_; }
  size_t launches_per_step() const;
  // The forward program alone, on the current parameters (per-op tests, evaluation).
  void run_forward(const Batch& batch);
  const void* forward_value(uint32_t id) const;
  // A value of the step program (its inputs among them) as the last step left it.
  const void* step_value(uint32_t id) const;
  void load_params(const std::vector<std::vector<float>>& values) { upload_params(values); }
  // The launch plan of the step (or of the forward program): what each launch completes and its
  // algorithmic FLOP and bytes.
  const std::vector<Launch>& plan(bool step) const;
  const std::vector<int64_t>& param_offsets() const { return offset_; }
  int64_t param_floats() const { return total_; }
  // Sequences per step of the bound corpus (0 without one).
  uint64_t corpus_batch() const { return corpus_batch_; }
  // Throws the E-DATA-012 refusal a device gather recorded (after a wait on the stream).
  void check_data_error();
  // The loss-scale state of a mixed-precision session (zeros otherwise), after every queued step.
  hk::LossScaleState loss_scale();
  bool mixed() const { return opt_.mixed; }

 private:
  friend class Executor;
  int device_;
  hipStream_t stream_ = nullptr;
  hipStream_t side_ = nullptr;  // weight-gradient launches (default priority, like stream_)
  hipEvent_t fork_ = nullptr, join_ = nullptr;
  TrainingStep step_;
  Program forward_;
  uint64_t seed_;
  uint32_t prediction_;
  SessionOptions opt_;
  hk::LossScaleState* scaler_ = nullptr;  // device memory, mixed precision only
  bool use_graph_ = true;

  // Parameter, gradient and moment arenas share offsets: element i of each is the same element
  // of the same parameter. Parameters with a gradient come first, so the optimizer runs over one
  // prefix [0, trained_) of the arenas.
  std::vector<int64_t> offset_;  // per ParamId, in floats
  int64_t total_ = 0, trained_ = 0;
  float *param_ = nullptr, *grad_ = nullptr, *m_ = nullptr, *v_ = nullptr;
  // Mixed precision: the parameters rounded to f16 (the GEMMs' weight operands), refreshed after
  // every upload and every optimizer step.
  _Float16* param16_ = nullptr;
  float* losses_dev_ = nullptr;
  uint32_t* counter_ = nullptr;
  uint32_t loss_capacity_ = 1u << 20;
  void* state_mem_ = nullptr;
  // The packed corpus on the device: both splits, the masking constants and the gather's error
  // words.
  struct DeviceCorpus {
    hk::MlmCorpus c{};
    void* mem = nullptr;
    uint32_t* error = nullptr;
    ~DeviceCorpus();
  };
  std::unique_ptr<DeviceCorpus> corpus_;
  uint64_t corpus_batch_ = 0;
  // Whether the corpus writes input `name` of `p` (a batch tensor or a masked-row gather input).
  bool corpus_fed(const Program& p, const std::string& name) const;
  HeldOutSums held_out_in(const HeldOut& h, bool no_alloc);
  void* eval_mem_ = nullptr;     // held-out row results [rows, 2] and the HeldOutState behind them
  int64_t eval_rows_ = 0;

  std::unique_ptr<Executor> step_exec_, fwd_exec_;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  RunStats stats_;
  uint64_t steps_since_reset_ = 0;

  void upload_params(const std::vector<std::vector<float>>& values);
};

// Executes one Program: value storage, staged inputs, the fused launch list.
class Executor {
 public:
  Executor(Session& s, const Program& p, bool is_step);
  ~Executor();
  // Packs `batch` (and checks ids, labels and key masks) into the next pinned slot and enqueues
  // its copy to the device input block.
  void stage(const Batch& batch);
  void run(hipStream_t s);  // every launch, in order
  const std::vector<Launch>& launches() const { return launches_; }
  // The launch plan as text: one line a launch (its place, the values it completes, side stream,
  // algorithmic flop and bytes), then the buffer plan (every value's arena slice).
  std::string plan_text() const;
  const void* value(uint32_t id) const;
  uint32_t loss_value = 0;

 private:
  Session& s_;
  const Program& p_;
  bool is_step_;
  DeviceArena arena_;
  std::map<uint32_t, void*> token_;   // arena reservation per value
  std::map<uint32_t, void*> fixed_;   // values living in the session's arenas
  // Mixed precision: the f16 copy of a value GEMMs read as an operand, written by its producer.
  std::map<uint32_t, void*> token16_;
  std::map<uint32_t, _Float16*> fixed16_;  // parameters: their slice of the session's f16 copy
  std::set<uint32_t> only16_;               // values kept as their f16 copy alone (no f32 value written)
  _Float16* ptr16(uint32_t id) const;      // nullptr when the value has no f16 copy
  std::vector<Launch> launches_;
  size_t join_at_ = SIZE_MAX;  // the first launch after the backward (it waits for the side stream)
  // device: written on the device by the corpus prologue, never staged by the host.
  struct InputSlot { std::string name; DType dtype; int64_t count; size_t offset; uint32_t id; bool device; };
  std::vector<InputSlot> inputs_;
  // EmbeddingGrad plans of host-staged ids, made by the host in the input block (eg_plan_host).
  struct PlanSlot { std::string ids_name; uint32_t ids; int32_t n, rows; size_t offset; };
  std::vector<PlanSlot> plan_slots_;
  size_t input_bytes_ = 0, host_bytes_ = 0, draw_offset_ = 0;
  void* input_token_ = nullptr;
  static constexpr int kRing = 4;
  void* pinned_[kRing] = {};
  hipEvent_t slot_done_[kRing] = {};
  int next_slot_ = 0;
  // id checks before upload: input name -> rows it indexes (Embedding / EmbeddingGrad / labels)
  std::map<std::string, int64_t> id_bounds_;
  std::vector<std::string> key_masks_;
  void build();
  void* ptr(uint32_t id) const;
};

}  // namespace msx
