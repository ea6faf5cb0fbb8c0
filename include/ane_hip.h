/*
 * ane_hip.h -- C-ABI of libane_hip.so, the MI355X (gfx950) engine for the
 * reference's `ane` transformer compute path (tmc/autoresearch-go-ane).
 *
 * Every entry point takes plain pointers and sizes.  Host buffers are
 * caller-owned and only read or written for the duration of the call;
 * device memory is owned by the engine from ane_open() to ane_close().
 * One engine = one HIP device + one HIP stream; an engine is not
 * thread-safe (the reference's Engine is not goroutine-safe either).
 *
 * Return value of every int entry point: ANE_OK (0) or a negative ANE_ERR_*
 * code; ane_last_error() then holds a message in the reference's wording
 * ("storiesane <op>: ...").  There is no silent fallback: a HIP failure is
 * returned, never replaced by a CPU computation.
 *
 * Layouts at the boundary follow the reference:
 *   - parameters: one flat fp32 vector in the canonical order of
 *     ane_param_layout() (nanochat: the order of writeModelGrad,
 *     ane/engine.go:811-840);
 *   - logits: vocab-major [vocab, seq] per sequence, as EvalLogits returns
 *     them (ane/engine.go:449-462, ane/stories/cpu.go:303-327);
 *   - tokens: uint16 ids.
 */
#ifndef ANE_HIP_H
#define ANE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  ANE_OK = 0,
  ANE_ERR_CLOSED = -1,  /* "storiesane <op>: engine is closed" */
  ANE_ERR_ARG = -2,     /* bad length / size / configuration */
  ANE_ERR_HIP = -3,     /* a HIP runtime call or kernel launch failed */
  ANE_ERR_NOMEM = -4,   /* device allocation failed */
  ANE_ERR_STATE = -5    /* call not valid in the engine's current state */
};

enum { ANE_ARCH_NANOCHAT = 0, ANE_ARCH_LLAMA2 = 1 };
enum { ANE_GRAD_COMPAT = 0, ANE_GRAD_TRUE = 1 };

/* Model shape.  The reference fixes these as package constants
 * (ane/stories/config.go:3-18: Dim 768, Hidden 2048, Heads 12, Layers 12,
 * Vocab 32000, SeqDefault 256) and RoPE theta 1e5 (ane/train_util.go:196).
 * arch NANOCHAT is the reference's CPU-path model; LLAMA2 is the SwiGLU /
 * gain-RMSNorm variant of the benchmark configs.  Constraints of the
 * kernels: dim == 64 * heads, dim, hidden, vocab multiples of 64, seq a
 * multiple of 64 and <= 512. */
typedef struct ane_model_cfg {
  int32_t dim, hidden, heads, layers, vocab, seq;
  int32_t arch;      /* ANE_ARCH_* */
  int32_t grad_mode; /* ANE_GRAD_*: COMPAT reproduces the reference backward */
  double rope_theta; /* 0 selects the arch default (1e5 nanochat, 1e4 llama2) */
} ane_model_cfg;

/* Options (ane/engine.go:14-40).  Zero fields take the reference defaults
 * applied in Open (ane/engine.go:185-240).  ModelPath / UseANE /
 * HybridBackward / CPUClassifierHead / GradTaskLimit have no meaning here:
 * weights arrive through ane_set_params, the device path is the only path.
 * max_batch sizes the device activation buffers (sequences per call). */
typedef struct ane_options {
  int32_t accum_steps;
  float lr;
  int64_t seed;
  float adam_beta1, adam_beta2, adam_eps, weight_decay, grad_clip, loss_scale;
  float embed_lr_mult, scalar_lr_mult, lambda_lr_mult;
  float lambda_beta1, lambda_beta2;
  int32_t max_batch;
  int32_t device;
} ane_options;

/* State (ane/engine.go:43-52). */
typedef struct ane_state {
  uint64_t token_pos;
  float last_loss;
  double cum_train_ms, cum_wall_ms;
  uint32_t cum_steps, cum_batches, adam_t, pending_steps;
} ane_state;

/* StepResult (ane/engine.go:55-69); durations in nanoseconds.  The ANE /
 * compile fields keep their names.  On this engine (device times from HIP
 * events on the engine's stream, host times from the wall clock):
 *   step_ns             host wall time of the call
 *   startup_compile_ns  one-time training set-up (buffers, transposed
 *                       shadows) when this call did it, else 0
 *   compile_ns          startup_compile_ns + weight_refresh_ns
 *   ane_eval_ns         device time of the forward and backward kernels
 *   weight_refresh_ns   device time of the fp16 shadow rebuild after an update
 *   final_head_ns       classifier, cross-entropy, dlogits, dy, classifier
 *                       weight gradient, final-norm backward
 *   embed_grad_ns       classifier weight gradient + embedding scatter-add
 *   rms_dw_ns           norm-gain gradient reductions (llama2; 0 for nanochat,
 *                       whose norms have no weights)
 *   dw_gemm_ns          weight-gradient GEMMs with their operand transposes
 *                       (these three: events around each kernel group cost
 *                       ~4 us of idle GPU apiece, so they are measured on the
 *                       first training call and every 16th after it --
 *                       ANE_PHASE_EVERY=n changes the period -- and the other
 *                       calls report the latest measurement, per window,
 *                       times their window count)
 *   dw_wait_ns          host time blocked until the queued device work ended
 *   adam_ns             clip + AdamW kernels when the call flushed
 *   cpu_work_ns         step_ns minus the set-up, refresh, eval and Adam times */
typedef struct ane_step_result {
  float loss;
  int64_t step_ns, compile_ns, startup_compile_ns, ane_eval_ns, cpu_work_ns, weight_refresh_ns,
      final_head_ns, embed_grad_ns, rms_dw_ns, dw_gemm_ns, dw_wait_ns, adam_ns;
} ane_step_result;

typedef struct ane_engine ane_engine;

/* ---- lifecycle ---------------------------------------------------------- */

/* Open (ane/engine.go:184-355): allocates device buffers for max_batch
 * sequences, zero-initialised weights and optimizer state. */
int ane_open(const ane_model_cfg *cfg, const ane_options *opts, ane_engine **out);
/* Close (ane/engine.go:567-644): frees all device memory; later calls
 * return ANE_ERR_CLOSED.  The handle itself stays valid until
 * ane_destroy(). */
void ane_close(ane_engine *e);
void ane_destroy(ane_engine *e);
const char *ane_last_error(const ane_engine *e);

/* Number of fp32 parameters, and the canonical segments (offset, size) in
 * order; returns the segment count (writes at most max entries). */
int64_t ane_param_count(const ane_model_cfg *cfg);
int ane_param_layout(const ane_model_cfg *cfg, int64_t *offsets, int64_t *sizes, int max);

/* Weight load / read-back: the device replacement of LoadPretrained /
 * LoadCheckpoint's weight copy (ane/stories/weights.go:73-153) and of the
 * per-update weight re-staging (refreshANERuntimeForWeights,
 * ane/runtime.go:25-69): fp32 masters live in HBM and the fp16 GEMM
 * shadows are rebuilt on the device. */
int ane_set_params(ane_engine *e, const float *params, int64_t n);
int ane_get_params(ane_engine *e, float *params, int64_t n);

/* Options.Tokens (ane/engine.go:17): the token stream the window sampler
 * draws from, copied once into HBM. */
int ane_set_tokens(ane_engine *e, const uint16_t *tokens, int64_t n);

/* ---- forward ------------------------------------------------------------ */

/* EvalLogits (ane/engine.go:449-462): one sequence of exactly seq tokens;
 * writes vocab*seq fp32 logits, vocab-major (after the 15*tanh softcap
 * for nanochat). */
int ane_eval_logits(ane_engine *e, const uint16_t *tokens, int64_t ntok, float *logits);

/* Batched forward + mean cross-entropy over nseq sequences (the loss of
 * runFinalHead / stories.CrossEntropyLoss, ane/train_full.go:480-508,
 * ane/stories/cpu.go:212-292, without the backward).  tokens/targets:
 * [nseq][seq] host arrays; targets >= vocab are excluded.  loss_per_seq
 * (optional): mean CE of each sequence; *mean_loss: mean over sequences. */
int ane_eval_loss(ane_engine *e, const uint16_t *tokens, const uint16_t *targets, int32_t nseq,
                  float *loss_per_seq, float *mean_loss);

/* Same, over windows of the resident token stream: sequence b is
 * tokens[pos[b] : pos[b]+seq], targets shifted by one (the window rule of
 * Step, ane/engine.go:395-405).  Inputs never leave HBM. */
int ane_eval_loss_windows(ane_engine *e, const uint64_t *positions, int32_t nseq, float *loss_per_seq,
                          float *mean_loss);

/* ---- training ------------------------------------------------------------ */

/* Step (ane/engine.go:381-442): draws one window from the resident token
 * stream with the drand48 sampler (seeded from Options.Seed, ane/engine.go:
 * 395-405, 873-880), runs forward + backward, accumulates the loss-scaled
 * gradients, and applies clipping + AdamW once AccumSteps windows are
 * pending (flushPending, ane/engine.go:646-682).  Errors: ANE_ERR_STATE with
 * "storiesane step: not enough tokens" when no stream is set.  Training
 * kernels support seq <= 256. */
int ane_step(ane_engine *e, ane_step_result *res);
/* nseq consecutive Steps fused into one batched forward/backward (same
 * windows, same update; no reference counterpart: the reference runs one
 * sequence per call).  res->loss is the mean over the nseq windows. */
int ane_train_batch(ane_engine *e, int32_t nseq, ane_step_result *res);
/* Flush (ane/engine.go:484-496): applies pending accumulated gradients;
 * *ns receives the weight-refresh duration (the device time of the fp16
 * shadow rebuild after the update; the reference returns its asynchronous
 * refresh time), which is also added to cum_train_ms / cum_wall_ms; 0 when
 * nothing was pending. */
int ane_flush(ane_engine *e, int64_t *ns);
/* LR / SetLR (ane/engine.go:358-376); SetLR rejects lr <= 0 with
 * "storiesane set lr: lr must be > 0". */
float ane_lr(const ane_engine *e);
int ane_set_lr(ane_engine *e, float lr);
/* State / LoadState (ane/engine.go:498-513). */
int ane_get_state(ane_engine *e, ane_state *out);
int ane_load_state(ane_engine *e, const ane_state *s);

/* Gradient of the mean loss over nseq explicit sequences (the flushed
 * gradient the reference's Adam would see for these windows: loss-scaled
 * sum divided by nseq * lossScale, before clipping).  Leaves weights and
 * optimizer state untouched; fails with ANE_ERR_STATE while steps are
 * pending.  No reference counterpart (parity / diagnostics). */
int ane_grads(ane_engine *e, const uint16_t *tokens, const uint16_t *targets, int32_t nseq, float *grads,
              float *mean_loss);
/* Replaces the accumulated (loss-scaled) gradient sum and the pending step
 * count, e.g. to apply an externally computed gradient with ane_flush().
 * No reference counterpart (optimizer parity tests). */
int ane_set_grads(ane_engine *e, const float *grads, int64_t n, uint32_t pending);
/* Reads the AdamW moments (OptimState, ane/stories/cpu.go:294-301). */
int ane_get_opt_state(ane_engine *e, float *m, float *v, int64_t n);

/* Checkpoint support (SaveCheckpoint / LoadCheckpoint, ane/engine.go:515-564,
 * the V5 file of ane/stories/ckpt.go:77-269 and the "SANE" trailer,
 * ane/engine.go:684-767; the file I/O lives with the host caller):
 * ane_set_opt_state restores the moments (NULL = zeros);
 * ane_get_accum_grads reads the pending loss-scaled gradient sum the trailer
 * stores (restored with ane_set_grads); ane_seed_sampler re-seeds the
 * window sampler the way LoadCheckpoint does (drand48Seed(seed + step),
 * ane/engine.go:560). */
int ane_set_opt_state(ane_engine *e, const float *m, const float *v, int64_t n);
int ane_get_accum_grads(ane_engine *e, float *grads, int64_t n);
int ane_seed_sampler(ane_engine *e, int64_t seed);

/* ---- diagnostics -------------------------------------------------------- */

/* Per-kernel-class device timing with HIP events on the engine's stream.
 * When enabled, every launch of the classes below is bracketed by events;
 * ane_profile_read() synchronises and returns, per class, the launch
 * count, summed milliseconds, and the algorithmic FLOPs and HBM bytes of
 * those launches.  Classes: 0 qkv-gemm, 1 wo-gemm, 2 ffn-up-gemm,
 * 3 ffn-down-gemm, 4 classifier-gemm, 5 attention, 6 rmsnorm, 7 other. */
enum { ANE_PROF_CLASSES = 8 };
typedef struct ane_prof_entry {
  int64_t launches;
  double ms;
  double flops;
  double bytes;
} ane_prof_entry;
int ane_profile_enable(ane_engine *e, int on);
int ane_profile_read(ane_engine *e, ane_prof_entry *out, int max, int reset);

/* Blocks until all queued device work of the engine has finished. */
int ane_sync(ane_engine *e);

/* Single-kernel entry points for unit tests (no counterpart in the
 * reference; they run one kernel on device 0 from host buffers).
 * ane_debug_gemm: C = A(m,k) B(n,k)^T with A stored [K, M] when a_t else
 * [M, K], B stored [K, N] when b_t else [N, K] (fp16 bit patterns); C is
 * [M, N] fp32 (epi 1) or fp16 (epi 0); bm/bn force a block tile (0 = auto);
 * nw: waves per block, 0 = default (4), 8 = two waves per SIMD (256x256);
 * ns: LDS pipeline stages, 0 = default (2), 3 (K-major operands only);
 * splits: split-K factor (K-major operands, 2-stage pipeline; <= 1: none).
 * ane_debug_attention: causal attention over qkv [nseq*S, 3*64*NH] (fp16,
 * q|k|v per row, pre-RoPE) with score scale `scale` (hilo: split-operand
 * scores) -> out [nseq*S, 64*NH] fp16 and lse [nseq*S, NH].
 * Messages: ane_debug_last_error(). */
int ane_debug_gemm(int a_t, int b_t, int epi, int M, int N, int K, const uint16_t *A, const uint16_t *B,
                   void *C, int bm, int bn, int nw, int ns, int splits);
/* One K-major GEMM (A [M, K], B [N, K]) with a fused forward epilogue on host
 * buffers (epi: 0 fp16 store, 1 fp32 store, 2 logits (softcap 15 when
 * seq < 0), 3 residual C = alpha R + acc + beta X0 (+ copy to C2), 4 SwiGLU
 * over 32-column interleaved W1|W3 (C fp16 [M, N/2], C2 fp16 h1|h3), 5
 * relu^2 (C2 = pre-activation), 6 smear (X0, seq; C2 = gate)).  Optional
 * operands may be NULL. */
int ane_debug_gemm_epi(int epi, int M, int N, int K, const uint16_t *A, const uint16_t *B, void *C, void *C2,
                       const float *X0, const float *R, float alpha, float beta, int seq, int bm, int bn, int nw);
/* The deferred-RMSNorm epilogues of the llama2 eval forward on one forced
 * tile (bm x bn, nw waves): epi 13: X [M, N] fp32 in/out (X += A B^T),
 * C [M, N] fp16 = X * gain[col], ssq [N/bn][M] = per-row sums of X^2 over
 * each block's bn columns; epi 14: C [M, N] fp16 = (A B^T) * rr[row]; epi 15:
 * C [M, N/2] fp16 = SwiGLU over 32-column interleaved W1|W3 of (A B^T) *
 * rr[row]; rr = 1 / sqrt(sum_{p < nparts} rr_part[p][row] / rr_dim + 1e-5)
 * (the RMSNorm of ane/stories/cpu.go applied after the projection). */
int ane_debug_gemm_norm(int epi, int M, int N, int K, const uint16_t *A, const uint16_t *B, float *X, uint16_t *C,
                        const float *gain, float *ssq, const float *rr_part, int nparts, int rr_dim, int bm, int bn,
                        int nw);
int ane_debug_attention(int nseq, int S, int NH, int qknorm, double theta, float scale, int hilo,
                        const uint16_t *qkv, uint16_t *out, float *lse);
/* Two fp16 transposes in one launch of the training step's transpose kernel:
 * out_a [Ca, Ra] = in_a [Ra, Ca]^T, and the same for b when in_b is not NULL
 * (rows and columns multiples of 64). */
int ane_debug_transpose2(int Ra, int Ca, const uint16_t *in_a, uint16_t *out_a, int Rb, int Cb,
                         const uint16_t *in_b, uint16_t *out_b);
/* The training step's RMSNorm backward (stories.RMSNormBackward,
 * ane/stories/cpu.go:191-210, gain on both terms as there) on host arrays,
 * gain form: out [T, D] = alpha * addend + RMSNorm-backward(dy; x, gain)
 * (addend may be NULL), out_h [T, D] its fp16 copy (may be NULL) and
 * dgain_part [ceil(T / 8), D] each 8-row block's sum of dy * x / rms.
 * general != 0 forces the general kernel (the one the nanochat terms use);
 * 0 takes the gain-form kernel the llama2 step runs.  D a multiple of 64,
 * at most 1024. */
int ane_debug_norm_bwd(int T, int D, const float *dy, const float *x, const float *gain, const float *addend,
                       float alpha, float *out, uint16_t *out_h, float *dgain_part, int general);
/* The classifier epilogues on one forced block tile (bm x bn, nw waves):
 * A [M, K] classifier rows, B [N, K] token rows (fp16), targets [N].
 * Cross-entropy partials (the loss path of runFinalHead /
 * stories.CrossEntropyLoss, ane/train_full.go:480-508, ane/stories/cpu.go:
 * 212-292): part_max / part_sum [M/bm][N] receive each block row's
 * (max, sum exp(v - max)) of every column (v = 15 tanh(acc/15) when
 * softcap), tgt_logit [N] the target's logit.  With lse [N] and colscale [N]
 * given, the dlogits epilogue then writes dl [M, N] (fp16, vocab-major:
 * (softmax - onehot) * colscale, rows >= vocab zero) and, if dl_t is not
 * NULL, the token-major copy [N, M]. */
int ane_debug_classifier(int M, int N, int K, const uint16_t *A, const uint16_t *B, const uint16_t *targets,
                         int softcap, int vocab, int bm, int bn, int nw, float *part_max, float *part_sum,
                         float *tgt_logit, const float *lse, const float *colscale, uint16_t *dl, uint16_t *dl_t);
/* Mean time of `iters` launches of one GEMM on device-resident operands
 * (arguments as ane_debug_gemm; A / B NULL: pseudo-random in [-0.5, 0.5)).
 * epi: 0 fp16 store, 1 fp32 store, 3 in-place residual add, 4 SwiGLU over
 * interleaved W1|W3 columns, 7 classifier cross-entropy partials, 13-16 the
 * deferred-RMSNorm forms (zero partials and gains, 12 partials per row). */
int ane_debug_gemm_bench(int a_t, int b_t, int epi, int M, int N, int K, int bm, int bn, int nw, int ns,
                         int splits, int iters, const uint16_t *A, const uint16_t *B, float *avg_ms);
const char *ane_debug_last_error(void);

/* ---- classifier-head loss on device buffers -------------------------------
 * The loss half of runFinalHead (ane/train_full.go:480-508) as a standalone
 * operation on caller-owned device memory: tied-classifier logits
 * embed . xn (ane/stories/cpu.go:303-327), the 15*tanh softcap when softcap
 * != 0 (ane/common.go:272-287), and stories.CrossEntropyLoss
 * (ane/stories/cpu.go:212-292): per token -log(max(p_target, 1e-10)),
 * averaged over the valid targets (< vocab) of each sequence (0 when a
 * sequence has none).  No logit is materialised.
 *   xn      [ntok][dim] fp16   normalised final hidden states (token-major)
 *   embed   [vocab][dim] fp16  classifier rows
 *   targets [ntok] uint16
 *   loss_seq [ntok/seq] fp32   per-sequence mean cross-entropy (output)
 *   lse      [ntok] fp32       per-token log-sum-exp (output; may be NULL)
 * ntok a multiple of seq and of 64; dim, vocab multiples of 64.  stream: a
 * hipStream_t (NULL: the default stream).  The call allocates its scratch
 * (cross-entropy partials) with hipMalloc, waits for the stream and frees
 * it.  Errors: ANE_ERR_ARG / ANE_ERR_NOMEM / ANE_ERR_HIP, message in
 * ane_op_last_error() (per thread).  No counterpart in the reference, whose
 * loss runs on host slices inside Step / EvalLogits. */
int ane_head_loss(const uint16_t *xn, const uint16_t *embed, const uint16_t *targets, int32_t ntok, int32_t dim,
                  int32_t vocab, int32_t seq, int32_t softcap, float *loss_seq, float *lse, void *stream);
const char *ane_op_last_error(void);
/* ane_head_loss without any allocation: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results; the scratch is a fixed 8 MiB array per GPU (vocab
 * 32000: up to 8192 tokens); larger requests fail with ANE_ERR_ARG.  The call is asynchronous on `stream` (it does not wait).
 * Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (other streams, other threads) race on it.  Calls no hipMalloc,
 * hipFree or allocating library routine. */
int ane_head_loss_noalloc(const uint16_t *xn, const uint16_t *embed, const uint16_t *targets, int32_t ntok,
                          int32_t dim, int32_t vocab, int32_t seq, int32_t softcap, float *loss_seq, float *lse,
                          void *stream);

/* ---- greedy KV-cache decoder (grouped-query attention) --------------------
 * No counterpart in the reference, which evaluates whole windows only
 * (ane/engine.go:954-1038).  Serves the decode benchmark's Llama2-style
 * model built from the reference's primitives: gain RMSNorm
 * (ane/stories/cpu.go:97-111), RoPE (ane/train_util.go:183-224), causal
 * softmax attention (ane/common.go:61-89) with kv_heads key/value heads
 * shared by heads/kv_heads query heads each, SwiGLU, tied classifier
 * (ane/stories/cpu.go:303-327), greedy = first index of the maximum logit.
 * Parameters: the flat LLAMA2 order of ane_param_layout() with Wk, Wv of
 * kv_heads*64 rows.  The fp16 KV cache holds max_ctx positions for each of
 * max_batch (<= 64) sequences. */
typedef struct {
  int32_t dim, hidden, heads, kv_heads, layers, vocab;
  int32_t max_batch; /* sequences decoded together, 1..64 */
  int32_t max_ctx;   /* cache positions per sequence: prefix + decode steps */
  double rope_theta;
  int32_t device;
} ane_decode_cfg;

typedef struct ane_decoder ane_decoder;

int ane_decode_open(const ane_decode_cfg *cfg, ane_decoder **out);
void ane_decode_destroy(ane_decoder *d);
const char *ane_decode_last_error(ane_decoder *d);
int64_t ane_decode_param_count(const ane_decode_cfg *cfg);
int ane_decode_set_params(ane_decoder *d, const float *params, int64_t n);
/* Runs the prefix [nseq][plen] (plen % 64 == 0, plen < max_ctx) into the
 * cache and returns the greedy token after it (next_tok [nseq]) and,
 * optionally, the fp32 logits of the last prefix position [nseq][vocab]. */
int ane_decode_prefill(ane_decoder *d, const uint16_t *prefix, int32_t nseq, int32_t plen, uint16_t *next_tok,
                       float *logits);
/* One decode step: feeds in_tok [nseq] (NULL: the previous greedy tokens)
 * at the next position; returns the greedy tokens and optional logits. */
int ane_decode_step(ane_decoder *d, const uint16_t *in_tok, uint16_t *next_tok, float *logits);
/* nsteps greedy steps without host round trips (replayed HIP graph of one
 * step); out_tok [nsteps][nseq] receives the tokens each step produced. */
int ane_decode_generate(ane_decoder *d, int32_t nsteps, uint16_t *out_tok);
/* current cache length (positions filled) of the active batch */
int32_t ane_decode_position(ane_decoder *d);
/* device time of the last ane_decode_generate call (ms, HIP events) */
double ane_decode_last_ms(ane_decoder *d);
/* Which form a step runs in (no reference counterpart; the decoder has
 * none): 1 the fused per-layer chain, 0 one launch per GEMM (chosen at open:
 * ANE_DEC_TAIL=0, or the chain's blocks do not all fit on the GPU at once),
 * 2 one launch per GEMM after a chain wait timed out.  The chain's waits
 * assume all of a launch's chain blocks resident at once and dispatched
 * before its attention blocks; when one times out (another process on the
 * GPU can break both) the decoder switches to one launch per GEMM for good
 * and redoes the call from its start, as the reference disables a failing
 * accelerator piece and carries on (ane/engine.go:887-894,
 * ane/train_full.go:356-368).  If the redo itself fails, the active batch is
 * dropped: Step / Generate then refuse until the next Prefill. */
int32_t ane_decode_fused_chain(ane_decoder *d);
/* Test-only (no reference counterpart): fills every byte of the KV cache
 * with `byte` (0xFF: fp16 NaN everywhere), so a test can show that no
 * position is read before it is written. */
int ane_decode_debug_fill_cache(ane_decoder *d, int byte);

/* ---- mixture-of-experts SwiGLU FFN layer ----------------------------------
 * No counterpart in the reference (its FFN is dense, ane/common.go:91-105
 * linearCF is the primitive reused).  Top-2 routing: router logits in fp32
 * with linearCF's operation order (bit-exact with a CPU evaluation of the
 * same order), the two largest logits (ties to the lower expert), weights =
 * softmax over those two; out[t] = w0 * FFN_e0(x[t]) + w1 * FFN_e1(x[t]),
 * FFN_e(x) = W2_e (silu(W1_e x) * W3_e x).  No capacity limit.  Parameters
 * (flat fp32): router [E][D], then per expert W1 [H][D], W3 [H][D],
 * W2 [D][H]. */
typedef struct {
  int32_t dim, hidden; /* multiples of 64 */
  int32_t experts;     /* 2, 4, 8 or 16 */
  int32_t top_k;       /* 2 */
  int32_t max_tokens;
  int32_t device;
} ane_moe_cfg;

typedef struct ane_moe ane_moe;

int ane_moe_open(const ane_moe_cfg *cfg, ane_moe **out);
void ane_moe_destroy(ane_moe *m);
const char *ane_moe_last_error(ane_moe *m);
int64_t ane_moe_param_count(const ane_moe_cfg *cfg);
int ane_moe_set_params(ane_moe *m, const float *params, int64_t n);
/* copies x [tokens][dim] fp32 to device memory; ane_moe_run then works on it */
int ane_moe_load_input(ane_moe *m, const float *x, int32_t tokens);
/* route, group, expert GEMMs, combine on the resident input (device time: ane_moe_last_ms) */
int ane_moe_run(ane_moe *m);
/* out [tokens][dim] fp32; experts / weights [tokens][2] (either may be NULL) */
int ane_moe_read_output(ane_moe *m, float *out, int32_t *experts, float *weights);
double ane_moe_last_ms(ane_moe *m);

#ifdef __cplusplus
}
#endif
#endif
