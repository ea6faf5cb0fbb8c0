/*
 * refcpu.h -- CPU oracle for the ane transformer path (TEST INFRASTRUCTURE).
 *
 * This is a plain-C restatement of the reference's non-darwin ("CPU path")
 * model math, used ONLY as the checker by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg.  The product (libane_hip.so) never links,
 * loads or calls it.
 *
 * Layout follows the reference: activations channel-first [C, seq] per
 * sequence, weights row-major [out, in], logits vocab-major [V, seq].
 *
 * Parameters travel as ONE flat fp32 vector in the canonical order below
 * (the same order the product's C-ABI uses):
 *   arch NANOCHAT (reference-exact, ane/engine.go:954-1038):
 *     per layer l: Wq[D*D] Wk[D*D] Wv[D*D] Wo[D*D] W1[H*D] W2[D*H]
 *                  (+ VEEmbed[V*D] VEGate[NH*12] when l is a VE layer)
 *     then Embed[V*D] ResidLambdas[L] X0Lambdas[L] SmearGate[D*D]
 *          SmearLambda[1] BackoutLambda[1]
 *     (order of ane/engine.go:811-840 writeModelGrad)
 *   arch LLAMA2 (built from the reference primitives):
 *     per layer l: Wq Wk Wv Wo W1[H*D] W2[D*H] W3[H*D] g_att[D] g_ffn[D]
 *     then Embed[V*D] g_final[D]
 */
#ifndef REFCPU_H
#define REFCPU_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_ARCH_NANOCHAT = 0, ORC_ARCH_LLAMA2 = 1 };
enum { ORC_GRAD_COMPAT = 0, ORC_GRAD_TRUE = 1 };

typedef struct {
  int32_t dim, hidden, heads, layers, vocab, seq;
  int32_t arch;       /* ORC_ARCH_* */
  int32_t grad_mode;  /* ORC_GRAD_*: compat reproduces the reference backward */
  double rope_theta;  /* 100000 (nanochat, ane/train_util.go:196) / 10000 */
} orc_cfg;

typedef struct {
  float lr, beta1, beta2, eps, weight_decay, grad_clip;
  float embed_lr_mult, scalar_lr_mult, lambda_lr_mult;
  float lambda_beta1, lambda_beta2;
} orc_adam;

/* threading knob: n worker threads for parallelFor-style loops (>=1). */
void orc_set_threads(int n);
/* when nonzero, linearCF-style GEMMs are split over output rows too
 * (bit-identical results; the reference runs them serially). */
void orc_set_parallel_linear(int on);

size_t orc_param_count(const orc_cfg *c);
/* fills offsets/sizes of the n-th canonical segment; returns #segments */
int orc_param_segments(const orc_cfg *c, int64_t *offsets, int64_t *sizes, int max);
int orc_is_ve_layer(const orc_cfg *c, int l);

/* Forward + loss over nseq independent sequences.
 * tokens/targets: [nseq][seq] uint16.  logits (optional, may be NULL):
 * [nseq][V][seq] vocab-major after softcap (nanochat).  loss_per_seq
 * (optional): mean CE per sequence.  Returns the mean over sequences. */
float orc_forward_loss(const orc_cfg *c, const float *params,
                       const uint16_t *tokens, const uint16_t *targets,
                       int nseq, float *logits, float *loss_per_seq);

/* Forward + backward over nseq sequences.  grads (size orc_param_count)
 * receives the mean over sequences of each sequence's gradient, after the
 * loss-scale round trip and before clipping (ane/train_full.go:822-945).
 * Returns the mean loss. */
float orc_grads(const orc_cfg *c, const float *params,
                const uint16_t *tokens, const uint16_t *targets, int nseq,
                float loss_scale, float *grads);

/* Global-norm clip + AdamW update with the reference's parameter groups
 * (ane/train_full.go:167-196, 1088-1150; ane/engine.go:646-682).
 * step is the 1-based Adam step t. grads are modified by clipping. */
void orc_adam_update(const orc_cfg *c, float *params, float *grads, float *m,
                     float *v, int step, const orc_adam *h);

/* --- single ops at the reference's signatures (channel-first) --------- */
void orc_linear_cf(float *out, const float *w, const float *in, int out_ch, int in_ch, int seq);
void orc_rmsnorm_noweight_cf(float *out, const float *x, int dim, int seq);
void orc_rmsnorm_cf(float *out, const float *x, const float *w, int dim, int seq);
void orc_causal_attention_cf(float *out, const float *q, const float *k, const float *v,
                             int heads, int head_dim, int seq);
void orc_build_rope(float *cos_t, float *sin_t, int seq, int head_dim, double theta);
void orc_apply_rope_cf(float *x, int heads, int head_dim, int seq, const float *cos_t,
                       const float *sin_t);
void orc_qknorm_cf(float *q, float *k, int dim, int heads, int seq);
float orc_cross_entropy(float *dlogits, const float *logits, const uint16_t *targets, int v, int s);
void orc_linear_bwd_dx_cf(float *dx, const float *w, const float *dy, int out_ch, int in_ch, int seq);
void orc_rmsnorm_noweight_bwd_cf(float *dx, const float *dy, const float *x, int dim, int seq);
/* scale: of the scores in the recomputed probabilities and in ds */
void orc_causal_attention_bwd_cf(float *dq, float *dk, float *dv, const float *dout, const float *q,
                                 const float *k, const float *v, int heads, int head_dim, int seq,
                                 float scale);
void orc_matmul_vocab_seq(float *logits, const float *embed, const float *x, int vocab, int dim, int seq);
void orc_matmul_embedT(float *dx, const float *embed, const float *dlogits, int vocab, int dim, int seq);
void orc_softmax_row(float *out, const float *in, int n);
void orc_softcap(float *x, size_t n);
uint64_t orc_drand48_seed(int64_t seed);
double orc_drand48_next(uint64_t *state);

/* --- the per-object accelerator seam (refseam.c) ------------------------
 * What the reference's Neural Engine programs compute for layerForward,
 * layerBackward and offload (not the CPU path's layer: no QK-norm,
 * residual lambdas or value embeddings; plain residuals). */
typedef struct {
  const float *wq, *wk, *wv, *wo, *w1, *w2;
} orc_seam_layer;
/* runWithTaps' layerCache taps; NULL fields are not written */
typedef struct {
  float *x_norm, *q, *k, *v, *att_out, *x2, *x2_norm, *h1, *gate;
} orc_seam_taps;
void orc_seam_layer_forward(const orc_seam_layer *w, int dim, int hidden, int heads, int seq, const float *x,
                            float *out, orc_seam_taps *taps);
void orc_seam_attention_backward(const orc_seam_layer *w, int dim, int heads, int seq, const float *q,
                                 const float *k, const float *v, const float *dx2, float *dx_norm, float *dq,
                                 float *dk, float *dv);
void orc_seam_ffn_backward(const orc_seam_layer *w, int dim, int hidden, int seq, const float *dffn,
                           const float *h1, float *dx_norm, float *dh1);
/* in place: softmax over the vocabulary of each position of [vocab, seq] */
void orc_seam_softmax_vocab(float *probs, int vocab, int seq);

/* --- greedy KV-cache decoding (refdecode.c) ----------------------------
 * Llama2-style model with grouped-query attention: kv_heads key/value
 * heads, each shared by heads/kv_heads query heads. */
typedef struct {
  int32_t dim, hidden, heads, kv_heads, layers, vocab;
  double rope_theta;
} orc_dec_cfg;

size_t orc_dec_param_count(const orc_dec_cfg *c);

/* prefix: [nseq][plen] ids.  Step i (0-based) feeds forced[b][i] when
 * forced is non-NULL ([nseq][nsteps]), else the previous greedy token, at
 * position plen + i.  tokens_out: [nseq][nsteps+1], entry 0 = argmax of the
 * logits at position plen-1, entry i+1 = argmax after step i.  logits_out
 * (optional): [nseq][nsteps+1][vocab].  Sequences run on `threads` threads. */
void orc_decode(const orc_dec_cfg *c, const float *params, const uint16_t *prefix, int nseq, int plen,
                const uint16_t *forced, int nsteps, int threads, uint16_t *tokens_out, float *logits_out);

/* --- mixture-of-experts FFN layer (refmoe.c) ---------------------------
 * params: router [E][D], then per expert W1 [H][D], W3 [H][D], W2 [D][H].
 * x, out: [T][D] fp32.  idx / wts: [T][2] (chosen experts, ties to the
 * lower index; weights = softmax over the two chosen logits). */
typedef struct {
  int32_t dim, hidden, experts;
} orc_moe_cfg;

size_t orc_moe_param_count(const orc_moe_cfg *c);
void orc_moe_route(const orc_moe_cfg *c, const float *params, const float *x, int T, int32_t *idx, float *wts);
void orc_moe_forward(const orc_moe_cfg *c, const float *params, const float *x, int T, int threads, float *out,
                     int32_t *idx, float *wts);

#ifdef __cplusplus
}
#endif
#endif
