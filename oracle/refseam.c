/*
 * refseam.c -- CPU oracle for the per-object accelerator seam (TEST
 * INFRASTRUCTURE ONLY; see refcpu.h): the functions the reference's Neural
 * Engine programs compute for layerForward, layerBackward and offload,
 * composed from the reference's CPU primitives (refcpu.c).
 *
 * Those programs compute a different layer from the CPU path's: no QK-norm,
 * no residual or x0 lambdas, no value embeddings, plain residuals
 * (ane/mil_stories.go:75-163,301-340; ane/layer_dynamic_darwin.go:381-404).
 * Each step below cites the program it restates; the primitives cite the
 * reference's CPU functions that compute the same arithmetic:
 *   parameterless RMSNorm   rmsNormNoWeightCF          ane/common.go:157-174
 *   projections             linearCF                   ane/common.go:91-105
 *   transposed projections  linearBackwardDXCF         ane/train_full.go:242-259
 *   RoPE, theta 100000      buildRoPEBlobsLocal         ane/layer_dynamic_darwin.go:858-893
 *                           (the same angles as buildRoPETables, applied as
 *                           applyRoPECFInPlace, ane/train_util.go:183-224)
 *   causal attention        causalAttentionCF          ane/common.go:61-89
 *   attention backward      causalAttentionBackwardCF  ane/train_full.go:261-316,
 *                           at the forward's score scale 1/sqrt(head_dim)
 *   relu^2                  reluSquared32              ane/common.go:146
 *   classifier              stories.MatMulVocabSeq / MatMulEmbedTScale
 *                                                      ane/stories/cpu.go:303-360
 *
 * The attention backward's second stage is the un-vendored
 * mil.GenSDPABackward2 of github.com/tmc/apple v0.3.5 (called at
 * ane/layer_dynamic_darwin.go:77); its first stage recomputes the
 * probabilities at scale 1/sqrt(head_dim) (ane/mil_stories.go:383-441).
 * This oracle takes the exact gradient of the forward at that scale, and
 * the tests pin it against automatic differentiation of the forward.
 */
#include "refcpu.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

static float *fbuf(size_t n) { return (float *)calloc(n, sizeof(float)); }

/* genStoriesSDPAForwardDynamicTaps (ane/mil_stories.go:75-163), then
 * genStoriesFFNForwardDynamicTaps (:301-340), with the taps
 * runDynamicWithTaps keeps (ane/layer_dynamic_darwin.go:367-422). */
void orc_seam_layer_forward(const orc_seam_layer *w, int dim, int hidden, int heads, int seq, const float *x,
                            float *out, orc_seam_taps *taps) {
  const size_t DS = (size_t)dim * seq, HS = (size_t)hidden * seq;
  const int hd = dim / heads;
  float *xn = fbuf(DS), *q = fbuf(DS), *k = fbuf(DS), *v = fbuf(DS), *att = fbuf(DS), *oo = fbuf(DS);
  float *x2 = fbuf(DS), *x2n = fbuf(DS), *h1 = fbuf(HS), *gate = fbuf(HS), *ff = fbuf(DS);
  float *cs = fbuf((size_t)seq * hd / 2), *sn = fbuf((size_t)seq * hd / 2);
  orc_build_rope(cs, sn, seq, hd, 100000.0);
  /* attention block: x2 = x + Wo attention(rope(Wq xn), rope(Wk xn), Wv xn) */
  orc_rmsnorm_noweight_cf(xn, x, dim, seq);
  orc_linear_cf(q, w->wq, xn, dim, dim, seq);
  orc_linear_cf(k, w->wk, xn, dim, dim, seq);
  orc_linear_cf(v, w->wv, xn, dim, dim, seq);
  orc_apply_rope_cf(q, heads, hd, seq, cs, sn);
  orc_apply_rope_cf(k, heads, hd, seq, cs, sn);
  orc_causal_attention_cf(att, q, k, v, heads, hd, seq);
  orc_linear_cf(oo, w->wo, att, dim, dim, seq);
  for (size_t i = 0; i < DS; i++) x2[i] = x[i] + oo[i];
  /* FFN block: out = x2 + W2 relu(W1 rms(x2))^2 */
  orc_rmsnorm_noweight_cf(x2n, x2, dim, seq);
  orc_linear_cf(h1, w->w1, x2n, hidden, dim, seq);
  for (size_t i = 0; i < HS; i++) gate[i] = h1[i] <= 0.f ? 0.f : h1[i] * h1[i];
  orc_linear_cf(ff, w->w2, gate, dim, hidden, seq);
  for (size_t i = 0; i < DS; i++) out[i] = x2[i] + ff[i];
  if (taps) {
    if (taps->x_norm) memcpy(taps->x_norm, xn, DS * 4);
    if (taps->q) memcpy(taps->q, q, DS * 4);
    if (taps->k) memcpy(taps->k, k, DS * 4);
    if (taps->v) memcpy(taps->v, v, DS * 4);
    if (taps->att_out) memcpy(taps->att_out, att, DS * 4);
    if (taps->x2) memcpy(taps->x2, x2, DS * 4);
    if (taps->x2_norm) memcpy(taps->x2_norm, x2n, DS * 4);
    if (taps->h1) memcpy(taps->h1, h1, HS * 4);
    if (taps->gate) memcpy(taps->gate, gate, HS * 4);
  }
  free(xn); free(q); free(k); free(v); free(att); free(oo);
  free(x2); free(x2n); free(h1); free(gate); free(ff); free(cs); free(sn);
}

/* runDynamicAttention (ane/layer_dynamic_darwin.go:511-598): da = Wo^T dx2
 * (the wot program), the attention backward at (q, k, v) as given (sdpa1,
 * ane/mil_stories.go:383-441, and sdpa2), dx = Wq^T dq + Wk^T dk + Wv^T dv
 * summed as genStoriesQKVBackwardDynamic does (:443-479). */
void orc_seam_attention_backward(const orc_seam_layer *w, int dim, int heads, int seq, const float *q,
                                 const float *k, const float *v, const float *dx2, float *dx_norm, float *dq,
                                 float *dk, float *dv) {
  const size_t DS = (size_t)dim * seq;
  const int hd = dim / heads;
  float *da = fbuf(DS), *tk = fbuf(DS), *tv = fbuf(DS);
  orc_linear_bwd_dx_cf(da, w->wo, dx2, dim, dim, seq);
  orc_causal_attention_bwd_cf(dq, dk, dv, da, q, k, v, heads, hd, seq, (float)(1.0 / sqrt((double)hd)));
  orc_linear_bwd_dx_cf(dx_norm, w->wq, dq, dim, dim, seq);
  orc_linear_bwd_dx_cf(tk, w->wk, dk, dim, dim, seq);
  orc_linear_bwd_dx_cf(tv, w->wv, dv, dim, dim, seq);
  for (size_t i = 0; i < DS; i++) dx_norm[i] = (dx_norm[i] + tk[i]) + tv[i];
  free(da); free(tk); free(tv);
}

/* runDynamicFFN (ane/layer_dynamic_darwin.go:470-509): dsilu = W2^T dffn
 * (the ffnW2 program), then genStoriesFFNBackwardTailDynamic
 * (ane/mil_stories.go:351-381): dh1 = dsilu * (2 relu(h1)), dx = W1^T dh1. */
void orc_seam_ffn_backward(const orc_seam_layer *w, int dim, int hidden, int seq, const float *dffn,
                           const float *h1, float *dx_norm, float *dh1) {
  const size_t HS = (size_t)hidden * seq;
  float *dsilu = fbuf(HS);
  orc_linear_bwd_dx_cf(dsilu, w->w2, dffn, dim, hidden, seq);
  for (size_t i = 0; i < HS; i++) {
    const float r2 = (h1[i] > 0.f ? h1[i] : 0.f) * 2.f;
    dh1[i] = dsilu[i] * r2;
  }
  orc_linear_bwd_dx_cf(dx_norm, w->w1, dh1, hidden, dim, seq);
  free(dsilu);
}

/* The softmax program over the vocabulary of each position
 * (compileSoftmaxKernel, ane/offload_darwin.go:225-234; its result is read
 * as probabilities by crossEntropyLossFromProbsUnscaled), with the CPU
 * path's row softmax (softmaxRowAccel, ane/accel_stub.go:31-48). */
void orc_seam_softmax_vocab(float *probs, int vocab, int seq) {
  float *col = fbuf((size_t)vocab), *res = fbuf((size_t)vocab);
  for (int t = 0; t < seq; t++) {
    for (int r = 0; r < vocab; r++) col[r] = probs[(size_t)r * seq + t];
    orc_softmax_row(res, col, vocab);
    for (int r = 0; r < vocab; r++) probs[(size_t)r * seq + t] = res[r];
  }
  free(col);
  free(res);
}
