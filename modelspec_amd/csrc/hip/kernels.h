// Launchers of the CDNA4 (gfx950) kernels of the training step. Every launcher checks the shape
// assumptions of its kernel on the host before launching and enqueues on `s`.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

namespace msx::hk {

// Sets the launch attributes some kernels need (large dynamic LDS). Call once per process and
// device before launching, never during stream capture.
void prepare();

// While `log` is attached (non-null), the names of the kernels this thread dispatches are appended
// to it (profiling).
void kernel_log(std::vector<std::string>* log);

enum EwOp : int { EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_RELU, EW_RELU_GRAD, EW_GELU, EW_GELU_GRAD, EW_SQRT, EW_COPY };

// o[i] = op(a[a_scalar ? 0 : i], b[b_scalar ? 0 : i]) for i < n (binary ops), op(a[i]) for unary.
void elementwise(hipStream_t s, int op, const float* a, const float* b, float* o, int64_t n, bool a_scalar, bool b_scalar);
// o = (a op1 b) op2 s, or s op2 (a op1 b) when !inner_left; s a single value; each op rounded as
// elementwise rounds it.
void elementwise2(hipStream_t s, int op1, const float* a, const float* b, int op2, const float* sc, bool inner_left,
                  float* o, int64_t n);
void fill_from(hipStream_t s, const float* scalar, float* o, int64_t n);  // BroadcastScalar
void fill_zero(hipStream_t s, void* o, int64_t bytes);                     // kernel, not a memset
// y[r, c] = f16(x[r, c]) (round to nearest even) for r < rows, c < cols; rows ldx / ldy apart.
void to_f16_rows(hipStream_t s, const float* x, int64_t ldx, _Float16* y, int64_t ldy, int64_t rows, int64_t cols);
void copy(hipStream_t s, const float* a, float* o, int64_t n);

// C[M,N] = op(A) op(B) (+ bias[N]); A is [M,K] row-major with leading dimension lda, or [K,M]
// (read transposed) when ta; B is [K,N], or [N,K] when tb.
// `workspace` (gemm_workspace floats) takes split-K partials, summed in slice order. When
// `colsum` is non-null it receives the N column sums of op(B) over K as well, or with `sum_a` the
// M row sums of op(A) (a bias gradient beside its weight gradient). With `defer` the split-K sums
// are left to column_finalize jobs (gemm_deferred_jobs); the output must then be dense (ldc = n).
struct ColumnJob;
struct GemmArgs {
  const float* a; const float* b; float* c; const float* bias;
  int64_t m, n, k, lda, ldb, ldc;
  bool ta, tb;
  float* workspace; int64_t workspace_floats;
  float* colsum;
  bool sum_a, defer;
  // The operand's rows are zero from its contiguous extent up to its leading dimension (pad_c:
  // the output's rows are kept so).
  bool pad_a, pad_b, pad_c;
  // Mixed precision: operands rounded to f16 for the f16 MFMA, f32 accumulation and output.
  bool h16;
  // Epilogue after the bias: an activation (EPI_*: writing the pre-activation to pre_out when
  // non-null) or an activation gradient (pre_in the pre-activation), then addend + value.
  // addend, pre_in and pre_out share the output's leading dimension. pre16 (mixed precision), when
  // set, holds the pre-activation as f16 in place of pre_out (written) or pre_in (read).
  const float* addend;
  const float* pre_in;
  float* pre_out;
  _Float16* pre16;
  int act;
  // Then, with drop_token, the dropout gradient of the result: element (r, c) (index r ldc + c;
  // ldc == n) kept when Philox word 0 of (index, drop_token, drop_seed) >= drop_threshold, then
  // times drop_scale, else 0 (the dropout kernel's rule).
  const int32_t* drop_token;
  uint64_t drop_threshold;
  float drop_scale;
  uint64_t drop_seed;
  // Cross-entropy fused into a decoder head. ce_part (forward): each output row's (max, sum of
  // exp(v - max)) over each TN-column tile after the epilogue, [m][gemm_tile_n columns tiles] float2.
  // ce_operand 1 (A) or 2 (B): that operand is the loss gradient, formed from the logits it
  // reads: stored element (r, c) becomes ce_grad_of(x, ce_tab[r], c, ce_cols) (ce_head_rows).
  float* ce_part;
  const float4* ce_tab;
  int ce_operand;
  int64_t ce_cols;
  // Mixed precision with f16 operands in HBM: with both a16 and b16 set (the operands' f16 copies,
  // same layouts and leading dimensions as a and b), the GEMM reads them instead of a and b
  // (k_gemm_lds16: no rounding at load). c16, when set, receives the output (after the epilogue)
  // rounded to f16 as well, at ldc. An operand only its f16 copy holds (a or b null), or an output
  // kept only as its f16 copy (c null, c16 set), needs k_gemm_lds16 (gemm_lds16_fits): another
  // kernel refuses the problem.
  const _Float16* a16;
  const _Float16* b16;
  _Float16* c16;
  // K segments: with ksegs > 1 the product is the sum over s < ksegs of seg_a[s] seg_b[s], each
  // pair of the shape (m, k / ksegs, n) with a and b's transposes and leading dimensions, as one
  // contraction over k (a chain of like GEMMs added into one value); a and b are ignored then.
  int ksegs;
  const float* seg_a[4];
  const float* seg_b[4];
};
enum GemmAct : int { EPI_NONE, EPI_GELU, EPI_RELU, EPI_GELU_GRAD, EPI_RELU_GRAD };
struct GemmEpi {
  const float* bias; const float* addend; const float* pre_in; float* pre_out; int act;
  const int32_t* drop_token; uint64_t drop_threshold; float drop_scale; uint64_t drop_seed;
  _Float16* pre16;
};
// The pointers of each problem of a GEMM group (problems of one shape and configuration, one
// launch; block b works on problem b / tiles of the order).
constexpr int kGemmGroupMax = 4;
struct GemmPtrs {
  const float* a[kGemmGroupMax];
  const float* b[kGemmGroupMax];
  float* c[kGemmGroupMax];
  const _Float16* a16[kGemmGroupMax];
  const _Float16* b16[kGemmGroupMax];
  _Float16* c16[kGemmGroupMax];
  GemmEpi epi[kGemmGroupMax];
  float* ws[kGemmGroupMax];
  float* colsum[kGemmGroupMax];
  float* ce_part[kGemmGroupMax];
  const float4* ce_tab[kGemmGroupMax];
  int64_t ce_cols;
  int count;
  // K segments (GemmArgs::ksegs): one problem whose K tile at k0 reads a[k0 / kseg] and
  // b[k0 / kseg] at K offset k0 mod kseg.
  int ksegs;
  int64_t kseg;
};
// The output tile width of a GEMM of this shape (the column tiles of ce_part).
int64_t gemm_tile_n(int64_t m, int64_t n, int64_t k, bool defer = false, bool h16 = false);
// The split-K factor the launcher uses (with `defer` as in GemmArgs).
// ce: a cross-entropy head GEMM (GemmArgs ce_part or ce_operand), which takes the largest tile.
int gemm_split_for(int64_t m, int64_t n, int64_t k, bool defer = false, bool h16 = false, bool ce = false);
// Floats of workspace a gemm of this shape needs (0 without split-K): the slices' partial
// products, then the slices' column (row) sums when asked for.
int64_t gemm_workspace(int64_t m, int64_t n, int64_t k, bool colsum = false, bool sum_a = false, bool defer = false,
                       bool h16 = false, bool ce = false);
// The column_finalize jobs that finish a deferred split-K gemm (0, 1 or 2 written to jobs).
int gemm_deferred_jobs(const GemmArgs& g, ColumnJob* jobs);
// Whether a mixed-precision problem of this shape and layout runs on k_gemm_lds16 once its f16
// operand copies are given (16-byte aligned): no K segments or cross-entropy operand, whole
// 16-byte groups of f16 in its rows, K a multiple of 32 or zero-padded to one.
bool gemm_lds16_fits(const GemmArgs& g);
void gemm(hipStream_t s, const GemmArgs& g);
// `count` (1 .. kGemmGroupMax) independent GEMMs that differ only in their pointers, in one
// launch; split-K slices of a group are summed by deferral only.
void gemm_group(hipStream_t s, const GemmArgs* list, int count);

void transpose(hipStream_t s, const float* a, float* o, int64_t rows, int64_t cols);  // a [rows,cols] -> o [cols,rows]

void add_rows(hipStream_t s, const float* x, const float* bias, float* o, int64_t rows, int64_t h);
// Partial column sums of x [rows, h] (rows ld floats apart; ld < 0: h) into partial
// [column_partial_chunks, h], finished by column_finalize (a SumRows).
int64_t column_partial_chunks(int64_t rows, int64_t h);
void column_partial(hipStream_t s, const float* x, float* partial, int64_t rows, int64_t h, int64_t ld = -1);

// LayerNorm family, eps 1e-12. stats = [rows, 2] (mean, rstd).
void ln_stats(hipStream_t s, const float* x, float* stats, int64_t rows, int64_t h);
void layer_norm(hipStream_t s, const float* x, const float* gamma, const float* beta, float* y, float* stats,
                int64_t rows, int64_t h);
// LayerNorm with its neighbours: s = [a +] [dropout](b) (a may be null; din_token null: no
// dropout), y = LayerNorm(s; gamma, beta), yd = dropout(y) (dout_token non-null); each of s_out,
// y_out, stats, yd_out written when non-null. Dropout as `dropout` (threshold, scale, seed). With
// `gather` ([rows] ids into the src_rows rows of a and b), row r of s is the sum's row gather[r].
// With a_ids (b_ids), a (b) is a table of a_rows (b_rows) rows and its row r is the Embedding row
// a_ids[r] (0 for an id out of range); not combined with `gather` or an input dropout.
void ln_fused(hipStream_t s, const float* a, const float* b, const int32_t* din_token, uint64_t din_threshold,
              float din_scale, const float* gamma, const float* beta, float* s_out, float* y_out, float* stats,
              const int32_t* dout_token, uint64_t dout_threshold, float dout_scale, float* yd_out, int64_t rows,
              int64_t h, uint64_t seed, const int32_t* gather = nullptr, int64_t src_rows = 0,
              const int32_t* a_ids = nullptr, int64_t a_rows = 0, const int32_t* b_ids = nullptr, int64_t b_rows = 0,
              _Float16* y16 = nullptr, _Float16* yd16 = nullptr,  // f16 copies of y and yd
              const _Float16* b16 = nullptr);  // b read from its f16 copy instead (rows of 256..1024)

// LayerNorm backward in one pass: dx when non-null, and when `partial` is non-null the per-block
// partial sums [ln_backward_blocks, 2 h] of g * xhat (gamma gradient) then g (beta gradient), to be
// added by column_finalize. gamma may be null when dx is.
// dx2, when non-null, gets a function of dx on the way out: the dropout gradient (LNB_DROPOUT, with
// token, threshold, scale and seed as `dropout`) or the GELU / ReLU gradient with respect to
// pre-activation `pre` (LNB_GELU_GRAD / LNB_RELU_GRAD); dx itself may then be null.
enum LnbPost : int { LNB_DROPOUT, LNB_GELU_GRAD, LNB_RELU_GRAD };
int64_t ln_backward_blocks(int64_t rows, int64_t h);
void ln_backward(hipStream_t s, const float* x, const float* gamma, const float* g, const float* stats, float* dx,
                 float* partial, int64_t rows, int64_t h, float* dx2 = nullptr, int post = 0, const float* pre = nullptr,
                 const int32_t* token = nullptr, uint64_t threshold = 0, float scale = 1.0f, uint64_t seed = 0,
                 _Float16* dx16 = nullptr, _Float16* dx2_16 = nullptr);  // f16 copies of dx and dx2

// Sums of block partials [chunks, width] over the blocks, columns below `split` to out_lo and the
// rest to out_hi; up to kColumnJobs reductions a launch (`first` is set by column_finalize).
struct ColumnJob { const float* partial; float* out_lo; float* out_hi; int32_t chunks, width, split, first, parts; };
constexpr int kColumnJobs = 48;
struct ColumnJobs { ColumnJob job[kColumnJobs]; int32_t count; };
void column_finalize(hipStream_t s, const ColumnJob* jobs, int count);

void embedding(hipStream_t s, const float* table, const int32_t* ids, float* o, int64_t n, int64_t rows, int64_t h);
// Deterministic segmented scatter: e = 0; e[ids[k]] += g[k] in ascending k (no float atomics);
// out = e, or addend + e when addend is non-null.
void embedding_grad(hipStream_t s, const int32_t* ids, const float* g, float* out, int64_t n, int64_t rows,
                    int64_t h, const float* addend = nullptr);

// EmbeddingGrad as a sorted-segment scatter (segments.hip), bit-exact with embedding_grad: a plan
// per table (ids of at most 8192 positions made by eg_plan, 16384 by eg_plan_host) into a buffer of
// eg_plan_bytes, then eg_apply writes out = e (or addend + e) for up to kEgJobs tables a launch.
constexpr int kEgJobs = 3;
struct EgPlanJob { const int32_t* ids; int32_t* plan; int32_t n, rows, pos_bits, key_bits; };
struct EgPlanSet { EgPlanJob job[kEgJobs]; int32_t count; };
// With out2, the job also writes out2 = DropoutGrad(out) (dropout's rule: element i kept when
// Philox word 0 of (i, drop_token, seed) >= drop_threshold, then times drop_scale, else 0).
struct EgApplyJob {
  const int32_t* plan; const float* g; const float* addend; float* out;
  int32_t n, rows; int64_t h;
  float* out2; const int32_t* drop_token; uint64_t drop_threshold; float drop_scale; uint64_t seed;
  int32_t vec, blocks_short, blocks_long, blocks;  // set by eg_apply
};
struct EgApplySet { EgApplyJob job[kEgJobs]; int32_t count; };
bool eg_sorted_fits(int64_t n, int64_t rows);         // the apply (and a plan made by the host): n <= 16384
bool eg_device_plan_fits(int64_t n, int64_t rows);  // eg_plan on the device: n <= 8192
size_t eg_plan_bytes(int64_t n, int64_t rows);
void eg_plan(hipStream_t s, const EgPlanJob* jobs, int njobs);
// The same plan made on the host (ids in host memory, plan into host memory of eg_plan_bytes), for
// ids the host stages: it travels to the device with the step's inputs. Segments by ascending id,
// positions ascending within a segment; ids outside [0, rows) are left out, as eg_plan does.
void eg_plan_host(const int32_t* ids, int32_t n, int32_t rows, int32_t* plan);
void eg_apply(hipStream_t s, const EgApplyJob* jobs, int njobs);

void dropout(hipStream_t s, const float* x, float* o, int64_t n, const int32_t* token, uint64_t seed,
             uint64_t threshold, float scale);

// Attention over a key mask [B, S]; q [B*L, H], k/v [B*S, H] (attention.hip).
bool attention_fits(int64_t s, int64_t d);
bool attention_mfma(int64_t L, int64_t S, int64_t d);  // the MFMA path runs (else the scalar one)
// stats: [B*heads*L, 2] softmax maximum and sum per query (written when non-null; required by the
// MFMA backward).
// h16 (mixed precision): the MFMA path's contractions on the f16 MFMA with f32 accumulation.
void attention_fwd(hipStream_t s, const float* q, const float* k, const float* v, const float* mask, float* o,
                   float* stats, int64_t B, int64_t L, int64_t S, int64_t H, int64_t heads, bool h16 = false);
// Any of dk/dv may be null; the MFMA path needs dq, o (the forward's output), stats and dsum
// ([B*heads*L] scratch).
void attention_bwd(hipStream_t s, const float* q, const float* k, const float* v, const float* mask, const float* o,
                   const float* stats, const float* g, float* dq, float* dk, float* dv, float* dsum, int64_t B,
                   int64_t L, int64_t S, int64_t H, int64_t heads, bool h16 = false);
void prepare_attention();
// Mixed-precision attention of 64-wide heads on the f16 operand copies (flash16.hip), for query and
// key rows multiples of 128 (keys at most 4096): o and o16 (either may be null) the output in f32
// and f16, stats as attention_fwd's. The backward takes the f16 copies of the forward's output
// and of the output gradient, and qterms, 3 B heads L floats of scratch; any of the f32/f16
// gradient outputs may be null.
bool flash16_fits(int64_t L, int64_t S, int64_t d);
void prepare_flash16();
void flash16_fwd(hipStream_t s, const _Float16* q, const _Float16* k, const _Float16* v, const float* mask, float* o,
                 _Float16* o16, float* stats, int64_t B, int64_t L, int64_t S, int64_t H, int64_t heads);
void flash16_bwd(hipStream_t s, const _Float16* q, const _Float16* k, const _Float16* v, const float* mask,
                 const _Float16* o16, const _Float16* go16, const float* stats, float* qterms, float* dq, _Float16* dq16,
                 float* dk, _Float16* dk16, float* dv, _Float16* dv16, int64_t B, int64_t L, int64_t S, int64_t H,
                 int64_t heads);

// Cross-entropy over logits [rows, v] with row pitch ld (>= v): stats = [rows, 2] (max, total);
// den = [1] f32 weight sum rounded from f64; the gradient o has row pitch ld too.
void ce_stats(hipStream_t s, const float* logits, float* stats, int64_t rows, int64_t v, int64_t ld);
// The step's loss log: record_loss appends losses[counter] (when counter < capacity) and counts.
struct LossLog { float* losses = nullptr; uint32_t* counter = nullptr; uint32_t capacity = 0; };
// With rowloss non-null the per-row loss terms come from there (ce_rows) instead of stats and logits.
// With log.losses non-null the loss is also appended to the log, as record_loss would.
void ce_loss(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* stats,
             float* loss, float* den, int64_t rows, int64_t v, int64_t ld, const float* rowloss = nullptr,
             LossLog log = {});
// One pass per row: stats, the row loss terms (rowloss non-null) and the gradient (grad non-null,
// with the upstream gradient scalar g). Needs ce_rows_fits and 16-byte aligned logits and grad.
bool ce_rows_fits(int64_t v, int64_t ld);
// The rows of a cross-entropy whose logits came from a GEMM with ce_part: from the `tiles`
// column-tile partials of each row, its max and sum of exp (stats [rows, 2]), its loss term
// (rowloss) and its gradient entry tab[r] = (max, 1 / sum, g * w_r / sum(w), label; label -2 when
// sum(w) is 0) for the GEMMs that form the gradient from the logits.
void ce_head_rows(hipStream_t s, const float* part, int64_t tiles, const float* logits, int64_t ld, const int32_t* labels,
                  const float* w, const float* g, float* stats, float* rowloss, float4* tab, int64_t rows, int64_t v);
void ce_rows(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* g, float* stats,
             float* rowloss, float* grad, int64_t rows, int64_t v, int64_t ld);
void ce_grad(hipStream_t s, const float* logits, const int32_t* labels, const float* w, const float* stats,
             const float* den, const float* g, float* o, int64_t rows, int64_t v, int64_t ld);

// Held-out evaluation (train/eval.rs). held_out_rows: per row r of logits [rows, v] (row pitch
// ld), out[2r] = max + ln(sum exp(x - max)) - x[label] and out[2r + 1] = 1 when the row holds no
// NaN and its first largest logit (lowest id among ties) is its label, else 0. Labels must lie in
// [0, v) (the host checks them). held_out_sum: adds sum_r w_r out[2r] in f64, the count of rows
// with w_r > 0 and a hit, the weight sum in f64 and the count of rows with w_r > 0 to `state`
// (HeldOutState), which the caller zeroes before the first batch.
// A packed corpus resident on the device and the masking constants of its binding: the split
// ids (sequence after sequence), the sequence length, the run seed, the integer thresholds of the
// masking policy and V - 5 random tokens.
constexpr uint32_t kMlmSpecials = 5;
constexpr int32_t kMlmMask = 4;
struct MlmCorpus {
  const int32_t* train;
  const int32_t* heldout;
  int64_t seq_len;
  uint64_t seed;
  uint64_t select, mask, mask_or_random;
  uint64_t random_tokens;
};
// The batch of one step: `draw` is [split (0 Train, 1 HeldOut), draw id low, draw id high,
// sequence 0, ..., sequence batch-1] on the device. Any output may be null.
void mlm_rows(hipStream_t s, const MlmCorpus& c, const int32_t* draw, int64_t batch, int32_t* ids, int32_t* positions,
              float* key_mask, int32_t* labels, float* weights);
// The masked-row gather of `rows` rows into `capacity` slots; `error` (4 words, zeroed by the
// owner) records the first batch that selects more rows than the capacity: [1, count, draw id
// low, draw id high].
void masked_gather(hipStream_t s, const int32_t* labels, const float* weights, int64_t rows, int64_t capacity,
                   const int32_t* draw, int32_t* out_rows, int32_t* out_labels, float* out_weights, uint32_t* error);

struct HeldOutState {
  double numerator;
  unsigned long long correct;
  double denominator;            // sum of the weights
  unsigned long long selected;   // rows of positive weight
};
void held_out_rows(hipStream_t s, const float* logits, const int32_t* labels, float* out, int64_t rows, int64_t v,
                   int64_t ld);
void held_out_sum(hipStream_t s, const float* rows_in, const float* w, int64_t rows, HeldOutState* state);

void softmax(hipStream_t s, const float* x, float* o, int64_t rows, int64_t k);
void softmax_grad(hipStream_t s, const float* y, const float* g, float* o, int64_t rows, int64_t k);

// Whole-tensor sums in f64 (ReduceSum, ReduceMean, Mse), one deterministic block.
void reduce_sum(hipStream_t s, const float* a, float* o, int64_t n, bool mean);
void mse(hipStream_t s, const float* a, const float* b, float* o, int64_t n);

// The AdamW update of ir/training.rs:941-980 over one flat arena, in place.
struct AdamWConsts { float beta1, rest1, beta2, rest2, eps, decay; };
// Dynamic loss scaling of the mixed-precision step: the loss gradient is seeded with `scale`, the
// optimizer multiplies each gradient by `inv` (exact: a power of two) and makes no update when
// `overflow` is set; loss_scale_update then halves the scale on an overflow, doubles it after
// `window` clean steps, and clears the flag.
struct LossScaleState {
  float scale, inv;
  uint32_t good, overflow, skipped, window, pad0, pad1;
};
// ls may be null (no loss scaling). p16 (mixed precision), when set, receives the updated
// parameters rounded to f16 (left as they are when an overflowed step skips the update).
void adamw(hipStream_t s, float* p, const float* g, float* m, float* v, int64_t n, AdamWConsts k, const float* lr_t,
           const float* c1, const float* c2, const LossScaleState* ls = nullptr, _Float16* p16 = nullptr);
void sgd(hipStream_t s, float* p, const float* g, int64_t n, const float* lr, const LossScaleState* ls = nullptr);
// column_finalize and adamw in one launch, for a step without loss scaling whose deferred
// reductions are all gradients in the arena g[0, n): the blocks of the finalize jobs write each
// finished gradient and update its parameter and moments at once; the other blocks run the
// AdamW update over the rest of the arena. Results equal the two launches'.
// With `loss`, one more block of the launch does what ce_loss does with those arguments (a loss
// nothing in the step reads before the optimizer, logged at the step's end).
struct CeLossJob {
  const float* logits; const int32_t* labels; const float* w; const float* stats; float* loss; float* den;
  int64_t rows, v, ld; const float* rowloss; LossLog log;
};
void finalize_adamw(hipStream_t s, const ColumnJob* jobs, int count, float* p, float* g, float* m, float* v, int64_t n,
                    AdamWConsts k, const float* lr_t, const float* c1, const float* c2, const CeLossJob* loss = nullptr);
void grad_check(hipStream_t s, const float* g, int64_t n, LossScaleState* ls);
void loss_scale_update(hipStream_t s, LossScaleState* ls);

void record_loss(hipStream_t s, const float* loss, float* losses, uint32_t* counter, uint32_t capacity);

}  // namespace msx::hk
