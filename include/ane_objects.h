/*
 * ane_objects.h -- the reference's per-object accelerator seam on the GPU.
 *
 * The reference's Engine picks, per operation, an accelerator object or its
 * CPU function, and disables an object whose call fails and keeps going on
 * the CPU (ane/engine.go:887-894; ane/train_full.go:373-380,488-493,
 * 502-508,541-545).  Three object types fill that seam; the non-darwin
 * build stubs them as "unavailable" (ane/engine_other.go:15-89) and its
 * untagged callers also need refreshWeights on each and
 * layerBackward.runAttention (ane/runtime.go:34,149,176;
 * ane/train_full.go:621).  The entry points below are those objects, so a
 * Go host replaces the stubs with them and the Engine's own dispatch and
 * latch-to-CPU logic applies unchanged:
 *
 *   layerForward   ane_layer_forward_*    ane/layer_darwin.go:22-46,175-324
 *                                         (dynamic form: ane/layer_dynamic_darwin.go:367-468)
 *   layerBackward  ane_layer_backward_*   ane/backward_darwin.go:13-36,182-328
 *                                         (dynamic form: ane/layer_dynamic_darwin.go:470-598)
 *   offload        ane_offload_*          ane/offload_darwin.go:34-53,283-560
 *
 * Each object computes what the reference's accelerator programs compute
 * (not the CPU path, which differs from them: the layer programs have no
 * QK-norm, residual lambdas or value embeddings, and plain residuals,
 * ane/mil_stories.go:75-163,301-381,383-479), in fp16 operands with fp32
 * accumulation.  Activations cross the boundary as the reference's
 * channel-first fp32 slices [channels, seq] (element [c * seq + t]); the
 * objects keep their weights as fp16 copies on the device (refresh to
 * restage them, as refreshWeights does).
 *
 * Shapes: dim = 64 * heads, hidden and vocab multiples of 64, seq a multiple
 * of 64 with seq <= 512 (forward) or <= 256 (backward).  Weight matrices are
 * row-major [out, in] fp32 (stories.LayerWeights, ane/stories/weights.go:13-18):
 * wq, wk, wv, wo [dim, dim], w1 [hidden, dim], w2 [dim, hidden]; the
 * embedding [vocab, dim].
 *
 * Every int entry point returns ANE_OK or a negative ANE_ERR_* (ane_hip.h),
 * with the message in ane_seam_last_error() (per thread).  Calls on one
 * object are serialised by the caller (the reference's objects are not
 * safe for concurrent use either); each object owns a HIP stream and its
 * device buffers, on the device current when it was opened.
 */
#ifndef ANE_OBJECTS_H
#define ANE_OBJECTS_H

#include <stdint.h>

#include "ane_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* stories.LayerWeights without the value-embedding tables (ane/stories/weights.go:13-18;
 * layerForwardWeights, ane/layer_darwin.go:13-20). */
typedef struct ane_layer_weights {
  const float *wq, *wk, *wv, *wo;
  const float *w1;
  const float *w2;
} ane_layer_weights;

/* The taps runWithTaps fills in layerCache (ane/train_full.go:12-37), each
 * channel-first fp32: x_norm, q, k, v, att_out, x2, x2_norm [dim * seq];
 * h1, gate [hidden * seq].  q and k are after RoPE (the attention's
 * operands), x_norm and x2_norm the parameterless RMSNorms of the layer
 * input and of x2, gate = relu(h1)^2.  A NULL field is not written.  The
 * ready flags are set to 1 (attTapsReady / ffnTapsReady). */
typedef struct ane_layer_cache {
  float *x_norm, *q, *k, *v, *att_out, *x2, *x2_norm, *h1, *gate;
  int32_t att_taps_ready, ffn_taps_ready;
} ane_layer_cache;

/* Last error of a seam call on this thread. */
const char *ane_seam_last_error(void);

/* ---- layerForward ------------------------------------------------------ */
typedef struct ane_layer_fwd ane_layer_fwd;

/* compileStoriesLayerForward (ane/layer_darwin.go:50-62): stages one
 * layer's weights for sequences of `seq` tokens. */
int ane_layer_forward_open(int32_t dim, int32_t hidden, int32_t heads, int32_t seq, const ane_layer_weights *w,
                           ane_layer_fwd **out);
/* run (ane/layer_darwin.go:195-197; runDynamicInferenceOnly,
 * ane/layer_dynamic_darwin.go:427-468): out = x2 + W2 relu(W1 rms(x2))^2
 * with x2 = x + Wo attention(rope(Wq rms(x)), rope(Wk rms(x)), Wv rms(x));
 * x, out [dim * seq] (may alias). */
int ane_layer_forward_run(ane_layer_fwd *lf, float *out, const float *x);
/* runWithTaps (ane/layer_darwin.go:199-313; runDynamicWithTaps,
 * ane/layer_dynamic_darwin.go:367-422): run, and the taps into *cache
 * (NULL cache: run). */
int ane_layer_forward_run_taps(ane_layer_fwd *lf, float *out, const float *x, ane_layer_cache *cache);
/* refreshWeights (ane/layer_darwin.go:315-324; runtime.go:149). */
int ane_layer_forward_refresh(ane_layer_fwd *lf, const ane_layer_weights *w);
/* close (ane/layer_darwin.go:175-193): releases the device memory and the
 * stream; later calls fail with ANE_ERR_CLOSED ("layer is closed").  The
 * handle stays valid until destroy. */
void ane_layer_forward_close(ane_layer_fwd *lf);
void ane_layer_forward_destroy(ane_layer_fwd *lf);

/* ---- layerBackward ----------------------------------------------------- */
typedef struct ane_layer_bwd ane_layer_bwd;

/* compileStoriesLayerBackward (ane/backward_darwin.go:40-180). */
int ane_layer_backward_open(int32_t dim, int32_t hidden, int32_t heads, int32_t seq, const ane_layer_weights *w,
                            ane_layer_bwd **out);
/* runAttention (ane/backward_darwin.go:244-318; runDynamicAttention,
 * ane/layer_dynamic_darwin.go:511-598): da = Wo^T dx2; dq, dk, dv = the
 * causal attention's gradient at (q, k, v) as used (probabilities at scale
 * 1/sqrt(64)); dx_norm = Wq^T dq + Wk^T dk + Wv^T dv.  All [dim * seq]. */
int ane_layer_backward_run_attention(ane_layer_bwd *lb, float *dx_norm, float *dq, float *dk, float *dv,
                                     const float *q, const float *k, const float *v, const float *dx2);
/* runFFN (ane/backward_darwin.go:207-242; runDynamicFFN,
 * ane/layer_dynamic_darwin.go:470-509): dh1 = (W2^T dffn) * 2 relu(h1);
 * dx_norm = W1^T dh1.  dx_norm, dffn [dim * seq]; dh1, h1 [hidden * seq]. */
int ane_layer_backward_run_ffn(ane_layer_bwd *lb, float *dx_norm, float *dh1, const float *dffn, const float *h1);
/* refreshWeights (ane/backward_darwin.go:320-328; runtime.go:176). */
int ane_layer_backward_refresh(ane_layer_bwd *lb, const ane_layer_weights *w);
void ane_layer_backward_close(ane_layer_bwd *lb);
void ane_layer_backward_destroy(ane_layer_bwd *lb);

/* ---- offload ----------------------------------------------------------- */
typedef struct ane_offload ane_offload;

/* The pieces has* / disable* name (ane/offload_darwin.go:283-337). */
enum {
  ANE_OFF_RMS_FORWARD = 1,
  ANE_OFF_CLASSIFIER_FORWARD = 2,
  ANE_OFF_SOFTMAX = 4,
  ANE_OFF_CLASSIFIER_BACKWARD = 8,
  ANE_OFF_RMS_BACKWARD = 16
};

/* newOffload (ane/offload_darwin.go:55-203) for an enabled accelerator:
 * stages the tied embedding [vocab * dim].  cpu_classifier_head (Options.
 * CPUClassifierHead) leaves out the classifier and softmax pieces. */
int ane_offload_open(int32_t vocab, int32_t dim, int32_t seq, const float *embed, int32_t cpu_classifier_head,
                     ane_offload **out);
/* has* (1 or 0) for one piece; disable* drops it (ane/offload_darwin.go:283-337). */
int ane_offload_has(const ane_offload *o, int32_t piece);
void ane_offload_disable(ane_offload *o, int32_t piece);
/* runRMSForward (ane/offload_darwin.go:339-350): parameterless RMSNorm,
 * out, x [dim * seq]. */
int ane_offload_run_rms_forward(ane_offload *o, float *out, const float *x);
/* runClassifierForward (ane/offload_darwin.go:352-399): logits [vocab *
 * seq] (vocab-major) = Embed x_norm, x_norm [dim * seq]. */
int ane_offload_run_classifier_forward(ane_offload *o, float *logits, const float *x_norm);
/* runClassifierSoftmax (ane/offload_darwin.go:401-454): probs = softmax over
 * the vocabulary of each position of Embed x_norm. */
int ane_offload_run_classifier_softmax(ane_offload *o, float *probs, const float *x_norm);
/* runSoftmax (ane/offload_darwin.go:454-464): in place, over the
 * vocabulary of each position, probs [vocab * seq]. */
int ane_offload_run_softmax(ane_offload *o, float *probs);
/* runClassifierBackward (ane/offload_darwin.go:466-525): dy [dim * seq] =
 * Embed^T dlogits, dlogits [vocab * seq]. */
int ane_offload_run_classifier_backward(ane_offload *o, float *dy, const float *dlogits);
/* runRMSBackward (ane/offload_darwin.go:527-547): the parameterless
 * RMSNorm's input gradient, dx, dy, x [dim * seq]. */
int ane_offload_run_rms_backward(ane_offload *o, float *dx, const float *dy, const float *x);
/* refreshWeights (ane/offload_darwin.go:549-560; runtime.go:34): restages the embedding. */
int ane_offload_refresh(ane_offload *o, const float *embed);
void ane_offload_close(ane_offload *o);
void ane_offload_destroy(ane_offload *o);

#ifdef __cplusplus
}
#endif

#endif /* ANE_OBJECTS_H */
