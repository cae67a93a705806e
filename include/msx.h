/* modelspec-hip: the C ABI of the MI355X training-step backend (libmsx.so).
 *
 * The reference host (crates/modelspec-cli/src/train.rs:1045-1200, Backend at :577-584) calls
 * its Vulkan runner through Rust functions; this header is the surface an `extern "C"` FFI crate
 * binds in their place for `train --backend hip`. Conventions: every function returns 0 or a
 * negative status (MSX_E_*), with msx_last_error() holding the message of the calling thread's
 * last failure; no exception crosses the ABI; every host pointer is caller-owned and read only
 * during the call; one context per thread.
 */
#ifndef MSX_H
#define MSX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSX_OK 0
#define MSX_E_INVALID -1     /* malformed IR, a shape or name the step does not declare */
#define MSX_E_DATA -2        /* E-DATA-011 / E-DATA-012: ids, labels, weights, masks, gather capacity */
#define MSX_E_DEVICE -3      /* E-TARGET-002/003: no HIP runtime or no such device */
#define MSX_E_NONFINITE -4   /* E-TRAIN-001: a loss stopped being finite */
#define MSX_E_UNSUPPORTED -5 /* a step op or shape this backend has no kernel for */
#define MSX_E_CHECKPOINT -6  /* E-CKPT-001..004: an unreadable, damaged or mismatched .msckpt */
#define MSX_E_ARTIFACT -7    /* E-ARTIFACT-001..004: an unreadable, altered or invalid artifact (005: MSX_E_DEVICE) */

typedef struct msx_ctx msx_ctx;

/* A named host tensor: dtype 0 = f32, 1 = i32; `count` elements at `data`. */
typedef struct {
  const char* name;
  int32_t dtype;
  const void* data;
  uint64_t count;
} msx_tensor;

typedef struct {
  uint64_t steps;
  uint64_t graph_launches;
  uint64_t kernels_per_step;
  uint64_t bytes_uploaded;
  uint64_t device_bytes;
} msx_run_stats;

/* The message of this thread's last failure ("" after a success). */
const char* msx_last_error(void);

/* Number of visible HIP devices (0 when the runtime finds none). */
int msx_device_count(void);

/* Compiles a built-in config (linear_regression, mlp_classifier, transformer_block, bert_tiny,
 * bert_cpu, bert_micro, block_micro, mlp_micro, ...) or, for a name ending in ".mspec", the source
 * file at that path (the front-end's subset of the reference language: a model of params and
 * functions and one train block) to the printed training step and forward program (ir/print.rs
 * text). masked_rows / steps < 0 take the config's own. Free both with msx_free. Every entry point
 * below that takes a config name takes such a path too. Replaces compile::compile_training_with,
 * crates/modelspec-core/src/compile.rs:85-118 (and, for a path, syntax::parse, types::check and
 * lower::lower before it, crates/modelspec-core/src/syntax/parser.rs, types.rs, lower.rs:95-160);
 * a refused source is MSX_E_INVALID with its E-SYNTAX-001 / E-NAME-001 / E-TYPE-001 / E-TRAIN-002
 * code and line:column in msx_last_error. */
int msx_compile_config(const char* config, int64_t masked_rows, int64_t steps, char** step_ir, char** forward_ir);

/* The `steps` and `seed` a config (or .mspec source) trains with. Replaces reading them off the
 * checked train block (crates/modelspec-core/src/hir.rs, HirTrain). */
int msx_config_steps(const char* config, uint64_t* steps, uint64_t* seed);
void msx_free(void* p);

/* Parses a printed training step and prints it back (msx_free the result): the validation
 * msx_load applies before planning, without a device. Replaces artifact::read's checks of the
 * plan it consumes (crates/modelspec-core/src/artifact.rs:426). */
int msx_check_ir(const char* step_ir, char** normalized);

/* Opens device `device`. Replaces vulkan::on_device (crates/modelspec-runtime/src/vulkan/mod.rs:216-552). */
int msx_open(int device, msx_ctx** out);
void msx_close(msx_ctx* ctx);

/* Loads a training step (the text of `modelspec ir --stage training` with its optimizer) and the
 * dropout-free forward program, plans them, and allocates every device buffer of the run.
 * `prediction_output` is the index in the forward program's outputs of the model prediction.
 * Replaces stepwise::train_stepwise_on_device's set-up (vulkan/stepwise.rs:289-400). */
int msx_load(msx_ctx* ctx, const char* step_ir, const char* forward_ir, uint64_t seed, uint32_t prediction_output);

/* Uploads every parameter (ParamId order, `n` arrays of counts[i] floats) and zeroes the AdamW
 * moments and the loss log. Replaces the parameter upload of vulkan/stepwise.rs:343-400. */
/* The launch plans this backend makes of a step and its forward program, without a device: for
 * each program one line a launch (the values it completes, whether it runs on the side stream, its
 * algorithmic flop and bytes), then its buffer plan (the arena size and each value's offset). The
 * counterpart of the reference's printed Kernel IR (crates/modelspec-core/src/ir/kernel.rs:1407,
 * the `*.kernel.ir` goldens): its fusion groups and buffers, as this backend plans them. The text
 * is freed with msx_free. */
int msx_plan(const char* step_ir, const char* forward_ir, uint32_t prediction_output, int32_t mixed, char** plan);

int msx_set_params(msx_ctx* ctx, const float* const* values, const uint64_t* counts, uint32_t n);
int msx_read_param(msx_ctx* ctx, uint32_t param, float* out, uint64_t count);
/* which = 'm' or 'v'. */
int msx_read_moment(msx_ctx* ctx, uint32_t param, int32_t which, float* out, uint64_t count);

/* Runs `n` training steps. Step i reads the n_inputs[i] tensors at inputs[i]: the batch, the
 * masked-row gather, one i32[2] token per dropout site and, under AdamW, optimizer.lr_t / c1 / c2
 * (the inputs the reference host feeds per step, vulkan/stepwise.rs:1454-1551). The losses of the
 * n steps are written to losses_out (may be null). */
int msx_run_steps(msx_ctx* ctx, uint32_t n, const msx_tensor* const* inputs, const uint32_t* n_inputs, float* losses_out);

/* The forward program on the current parameters: its loss, and the prediction if requested. */
int msx_forward(msx_ctx* ctx, const msx_tensor* inputs, uint32_t n_inputs, float* loss_out, float* prediction_out,
                uint64_t prediction_count);

int msx_stats(msx_ctx* ctx, msx_run_stats* out);

/* The precision of the next msx_load: mixed != 0 runs every GEMM on the f16 MFMA (operands
 * rounded to f16, f32 accumulation) with dynamic loss scaling: the loss gradient is seeded with the
 * scale (starting at loss_scale), the optimizer unscales the gradients and skips a step whose
 * gradients overflowed (halving the scale), and the scale doubles after scale_window clean steps.
 * No counterpart in the reference, which trains in f32 only. */
int msx_set_precision(msx_ctx* ctx, int32_t mixed, float loss_scale, uint32_t scale_window);

/* Optional fusions of the next msx_load, msx_prog_new or built-in config run (msx_train_config and
 * the other config entry points). MSX_FUSE_CE_HEAD: a cross-entropy whose
 * logits come from a GEMM and whose gradient only GEMMs read is folded into those GEMMs (the
 * forward leaves per-tile row partials, the gradient is formed from the logits as it is loaded and
 * never stored); off by default, as it measured slower on BERT-tiny. No counterpart in the
 * reference: a plan choice of this backend (the reference's own fusion groups are fixed by its
 * planner, crates/modelspec-core/src/ir/kernel.rs:1407). */
#define MSX_FUSE_CE_HEAD 1u
/* MSX_FUSE_OPTIMIZER (on by default): without loss scaling, the batched finalize of the reductions
 * only the optimizer reads (split-K weight gradients, LayerNorm gamma/beta sums) runs inside the
 * AdamW launch, each finished gradient updated by the block that sums it; results are identical to
 * the two launches'. A plan choice of this backend, no counterpart in the reference. */
#define MSX_FUSE_OPTIMIZER 2u
#define MSX_FUSE_DEFAULT MSX_FUSE_OPTIMIZER
int msx_set_fusion(msx_ctx* ctx, uint32_t flags);
/* The loaded step's current loss scale and the number of steps skipped for an overflow (1 and 0
 * without mixed precision). */
int msx_loss_scale(msx_ctx* ctx, float* scale, uint64_t* skipped);

/* The device copy of input `name` of the step program (program 0) or the forward program (1) as
 * the last step or forward pass read it: what the host staged, or what the device drew from a
 * packed corpus. `count` elements of 4 bytes. For tests and inspection; no counterpart in the
 * reference, whose host builds every input itself. */
int msx_read_input(msx_ctx* ctx, int32_t program, const char* name, void* out, uint64_t count);

/* Held-out metrics (crates/modelspec-runtime/src/train/eval.rs:27-39, HeldOutMetrics at :94-98):
 * loss = sum(w nll) / sum(w) over every row of every batch (f64 sums, rounded to f32 once, 0 when
 * the weight sum is 0); accuracy = correct / selected over the rows of positive weight. The
 * numerator and the correct count are the device's sums, the denominator and the selected count
 * the host's sums of the batches' weights (HeldOut::metrics_of_sums, eval.rs:299-339). */
typedef struct {
  float loss;
  float accuracy;
  double numerator;
  double denominator;
  uint64_t correct;
  uint64_t selected;
} msx_heldout;

/* Evaluates the loaded forward program on the current parameters (after every step run so far)
 * over `n` held-out batches: batch i is the n_inputs[i] tensors at inputs[i], its labels and
 * weights the inputs named `labels` and `weights`. The logits of each batch are reduced on the
 * device; one host wait. A label outside the classes is MSX_E_DATA. Replaces HeldOut::evaluate
 * (eval.rs:211-262) and the device reduction of vulkan/stepwise.rs:1635-1760. */
int msx_evaluate(msx_ctx* ctx, uint32_t n, const msx_tensor* const* inputs, const uint32_t* n_inputs,
                 const char* labels, const char* weights, msx_heldout* out);

/* msx_evaluate without device allocation. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (tight serving loops, harnesses that forbid hipMalloc). The row
 * results and sums live in one static device array of the library (512 KiB + 256 bytes a device,
 * held until the process ends) instead of a buffer the session allocates on its first
 * evaluation; the call makes no hipMalloc or hipFree. A batch of more than 65,536 rows (labels)
 * is MSX_E_INVALID. Calls on one device share the array: each holds a per-device lock from
 * clearing the sums to reading them back, so concurrent calls from several threads run one after
 * another. The call waits for the device and copies the sums to the host, so it cannot be
 * recorded under HIP graph capture. It leaves the calling thread's current device as it found
 * it. Results equal msx_evaluate's. */
int msx_evaluate_static(msx_ctx* ctx, uint32_t n, const msx_tensor* const* inputs, const uint32_t* n_inputs,
                        const char* labels, const char* weights, msx_heldout* out);

/* A whole run of a built-in config on the context's device: initial parameters from the seed,
 * synthetic batches, `steps` steps (negative: the config's own), the final loss. Writes steps + 1
 * losses and the final parameters concatenated in ParamId order. Replaces the device branch of
 * crates/modelspec-cli/src/train.rs:1045-1200 with runner::run_checked's loop semantics. */
int msx_train_config(msx_ctx* ctx, const char* config, int64_t steps, int64_t masked_rows, float* losses,
                     uint64_t losses_len, float* params, uint64_t params_len, double* train_seconds);

/* msx_train_config with held-out evaluation (`train --eval-every`, crates/modelspec-cli/src/
 * train.rs:1293-1312): before step k with k % eval_every == 0 and after the last step, the
 * forward program over `eval_batches` synthetic held-out batches (batch b drawn at step id
 * 2^63 + b). Writes the evaluated steps and their metrics (at most evals_len) and their count to
 * *n_evals; eval_seconds (may be null) is the evaluations' wall clock, which train_seconds
 * excludes. */
int msx_train_config_eval(msx_ctx* ctx, const char* config, int64_t steps, uint64_t eval_every, uint64_t eval_batches,
                          float* losses, uint64_t losses_len, uint64_t* eval_steps, msx_heldout* evals,
                          uint64_t evals_len, uint64_t* n_evals, double* train_seconds, double* eval_seconds);

/* Reads a packed masked-language-model directory (binding.json, packed.json, train.tokens,
 * heldout.tokens; crates/modelspec-runtime/src/dataset/mlm.rs:588-662, checks of
 * train/data.rs:1448-1640) into the context; the next msx_load binds it to the forward program's
 * batch tensors (ids, positions, key_mask, labels, weights; E-DATA-005/006 when they do not fit)
 * and keeps both splits in device memory. Every batch is then drawn on the device: a step's
 * inputs name `data.step` (i32 [low, high] of the step) in place of the batch and the masked-row
 * gather, and the library draws the step's sequences (epoch order, Philox tag 5), masks them
 * 80/10/10 (tag 3) and gathers the selected rows on the device (mlm_batch, mlm.rs:717-788;
 * train/masked.rs:58-118). msx_evaluate with n = 0 evaluates every whole batch of the HeldOut
 * split. A refused directory is MSX_E_DATA naming the file; a step that selects more rows than
 * the gather holds is MSX_E_DATA (E-DATA-012) at the next call that waits on the device.
 * dir = NULL unbinds the corpus: the next msx_load takes its batches from the host again. */
int msx_load_packed(msx_ctx* ctx, const char* dir);

/* Writes a packed directory of the given ids, whole sequences of seq_len, with the BERT masking
 * policy (its selection rate replaced by `selection_rate`; BERT's is 0.15) and the records pack()
 * writes (mlm.rs:395-535) for the dataset and tokenizer UUIDs given. No device is needed. */
int msx_write_packed(const char* dir, const int32_t* train, uint64_t train_count, const int32_t* heldout,
                     uint64_t heldout_count, uint64_t seq_len, uint64_t vocabulary_size, const char* dataset_id,
                     const char* tokenizer_id, double selection_rate);

/* A run of a built-in config on the packed directory `dir` (msx_load_packed): `steps` steps
 * (negative: the config's own), a held-out evaluation every `eval_every` steps (0: none) over
 * `eval_batches` batches (0: the whole HeldOut split). Writes steps + 1 losses, the final
 * parameters in ParamId order (params may be null), and the evaluations as
 * msx_train_config_eval does. Replaces `train --data <dir> --eval-every n`
 * (crates/modelspec-cli/src/train.rs:1084-1312). */
int msx_train_packed(msx_ctx* ctx, const char* config, const char* dir, int64_t steps, uint64_t eval_every,
                     uint64_t eval_batches, float* losses, uint64_t losses_len, float* params, uint64_t params_len,
                     uint64_t* eval_steps, msx_heldout* evals, uint64_t evals_len, uint64_t* n_evals,
                     double* train_seconds, double* eval_seconds);

/* Writes the loaded step as a compiled artifact of format 1 with the `Hip` backend
 * (crates/modelspec-core/src/artifact.rs:210-290): dir/artifact.json (the manifest keys of
 * format 1 in serde_json's pretty form, sealed by artifact_hash and artifact_id; the printed step
 * and forward program it was planned from; its launch plans) and dir/kernels/<id>.hsaco, the
 * gfx950 code objects of this library. `source_text` (may be NULL: the printed forward program)
 * is what source_hash hashes. Writes the 64-hex-digit artifact hash to hash_out[65] (may be
 * NULL). */
int msx_write_artifact(msx_ctx* ctx, const char* dir, const char* source_text, char* hash_out);

/* Reads and validates a Hip artifact in the reference's order (E-ARTIFACT-001 manifest, 004
 * module files, 002 module hashes / artifact hash / id, 003 invariants: AMDGPU code objects,
 * ir_hash, schema hash and parameters of the carried step), refuses code objects other than this
 * library's (E-ARTIFACT-002) and a device other than the artifact's target (E-ARTIFACT-005,
 * MSX_E_DEVICE), then loads its step and forward program as msx_load does (artifact::read_for_
 * device, artifact.rs:340-346). */
int msx_load_artifact(msx_ctx* ctx, const char* dir, uint64_t seed);

/* The checks of msx_load_artifact without a device or a load; writes the artifact id to
 * artifact_id_out[37] (may be NULL). */
int msx_check_artifact(const char* dir, char* artifact_id_out);

/* Writes the loaded step's current parameters (and, under AdamW, its moments as optimizer slots
 * "m" and "v") as a .msckpt v1 file recording `step` updates (crates/modelspec-runtime/src/train/
 * checkpoint.rs; the reference writes no moments and so refuses to resume AdamW). The same
 * state writes the same bytes. */
int msx_checkpoint_write(msx_ctx* ctx, const char* path, uint64_t step);

/* Reads a .msckpt v1 file, validated in the reference's order (E-CKPT-001/002/004 as
 * MSX_E_CHECKPOINT), matches it against the loaded step (paths, shapes, schema hash; with
 * `resume` the optimizer too: E-CKPT-003) and uploads its parameters; with `resume` under AdamW
 * its moments too (a checkpoint of step 0 may carry none). Writes the checkpoint's step. */
int msx_checkpoint_read(msx_ctx* ctx, const char* path, int32_t resume, uint64_t* step);

/* A run of a built-in config (on a packed directory when packed_dir is not NULL) that may start
 * from the checkpoint `resume` and write checkpoints: `<stem>-<k>.msckpt` beside
 * checkpoint_path after every checkpoint_every updates before the end, and checkpoint_path at the
 * end (train --resume / --checkpoint / --checkpoint-every, crates/modelspec-cli/src/train.rs:
 * 538-542, 829-835, 1075, 1285). `steps` counts this invocation's steps (negative: to the config's
 * end); a resumed run ends at its checkpoint's step + steps. Writes steps + 1 losses, the final
 * parameters and the start step. */
int msx_train_checkpointed(msx_ctx* ctx, const char* config, const char* packed_dir, int64_t steps, const char* resume,
                           uint64_t checkpoint_every, const char* checkpoint_path, float* losses, uint64_t losses_len,
                           float* params, uint64_t params_len, uint64_t* start_step);

/* Times `steps` graph-launched training steps of a built-in config after `warmup` (HIP events on
 * the run's stream after every step into step_ms[steps], may be null; host inputs made before the
 * timed region), then runs `profile_reps` more steps eagerly with an event pair around every
 * launch into `profile` ("launch\tms\tflop\tbytes\tkernels" lines, ms the mean over the reps,
 * flop and bytes the reference's algorithmic count, kernels the HIP kernels the launch dispatched
 * joined by '+'; free with msx_free). Replaces `train --clock
 * --profile` (crates/modelspec-cli/src/train.rs:17-31, vulkan/profile.rs:1-14). */
int msx_bench_config(msx_ctx* ctx, const char* config, int64_t masked_rows, uint32_t warmup, uint32_t steps,
                     double* ms_per_step, double* step_ms, float* last_loss, uint32_t profile_reps, char** profile);

/* One program (print.rs text of a Tensor IR program) on the device, for per-op tests: inputs by
 * name, parameters by ParamId; output k read back with msx_prog_output. */
typedef struct msx_prog msx_prog;
int msx_prog_new(msx_ctx* ctx, const char* program_text, uint64_t seed, msx_prog** out);
int msx_prog_run(msx_prog* prog, const msx_tensor* inputs, uint32_t n_inputs, const float* const* params,
                 const uint64_t* param_counts, uint32_t n_params);
int msx_prog_output(msx_prog* prog, uint32_t k, float* out, uint64_t count);
void msx_prog_free(msx_prog* prog);

#ifdef __cplusplus
}
#endif
#endif
