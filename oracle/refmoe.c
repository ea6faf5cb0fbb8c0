/*
 * refmoe.c -- CPU oracle for the mixture-of-experts FFN layer (TEST
 * INFRASTRUCTURE ONLY; see refcpu.h).
 *
 * The reference has no MoE; this layer composes its primitives: every
 * projection is linearCF's fp32 sum in ascending input order
 * (ane/common.go:91-105, no fused multiply-add: the oracle is built with
 * -ffp-contract=off), SwiGLU is h1 * sigmoid(h1) * h3 as in the LLAMA2
 * forward of refcpu.c.  Routing (new, no reference counterpart):
 *   logits[t][e] = linearCF(router, x[t])             fp32, bit-exact target
 *   experts      = the two largest logits, ties to the lower expert index
 *   weights      = softmax over the two chosen logits (float64 exp)
 *   out[t]       = w0 * FFN_{e0}(x[t]) + w1 * FFN_{e1}(x[t])
 * No capacity limit: every token reaches both of its experts.
 */
#include "refcpu.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

size_t orc_moe_param_count(const orc_moe_cfg *c) {
  const size_t D = c->dim, H = c->hidden, E = c->experts;
  return E * D + E * (3 * H * D);
}

/* router logits for one token, linearCF order */
static void router_logits(float *lg, const float *wr, const float *x, int E, int D) {
  for (int e = 0; e < E; e++) {
    const float *w = wr + (size_t)e * D;
    float s = 0.f;
    for (int i = 0; i < D; i++) s += w[i] * x[i];
    lg[e] = s;
  }
}

void orc_moe_route(const orc_moe_cfg *c, const float *params, const float *x, int T, int32_t *idx, float *wts) {
  const int D = c->dim, E = c->experts;
  float lg[64];
  for (int t = 0; t < T; t++) {
    router_logits(lg, params, x + (size_t)t * D, E, D);
    int a = 0;
    for (int e = 1; e < E; e++)
      if (lg[e] > lg[a]) a = e;
    int b = a == 0 ? 1 : 0;
    for (int e = 0; e < E; e++)
      if (e != a && lg[e] > lg[b]) b = e;
    /* b is the first index of the largest logit among e != a: the scan
       starts at the lowest index and only a strictly larger value moves it */
    double eb = exp((double)lg[b] - (double)lg[a]);
    idx[2 * t] = a;
    idx[2 * t + 1] = b;
    wts[2 * t] = (float)(1.0 / (1.0 + eb));
    wts[2 * t + 1] = (float)(eb / (1.0 + eb));
  }
}

typedef struct {
  const orc_moe_cfg *c;
  const float *P, *x;
  const int32_t *idx;
  const float *wts;
  float *out;
  int T, next;
  pthread_mutex_t mu;
} moe_job;

static void moe_token(moe_job *J, int t, float *h1, float *h3, float *y) {
  const orc_moe_cfg *c = J->c;
  const int D = c->dim, H = c->hidden, E = c->experts;
  const float *x = J->x + (size_t)t * D;
  float *o = J->out + (size_t)t * D;
  for (int i = 0; i < D; i++) o[i] = 0.f;
  for (int k = 0; k < 2; k++) {
    const int e = J->idx[2 * t + k];
    const float *base = J->P + (size_t)E * D + (size_t)e * 3 * H * D;
    const float *w1 = base, *w3 = base + (size_t)H * D, *w2 = base + (size_t)2 * H * D;
    for (int j = 0; j < H; j++) {
      float s1 = 0.f, s3 = 0.f;
      for (int i = 0; i < D; i++) {
        s1 += w1[(size_t)j * D + i] * x[i];
        s3 += w3[(size_t)j * D + i] * x[i];
      }
      h1[j] = s1 * (1.0f / (1.0f + (float)exp((double)(-s1)))) * s3;
    }
    for (int i = 0; i < D; i++) {
      float s = 0.f;
      for (int j = 0; j < H; j++) s += w2[(size_t)i * H + j] * h1[j];
      y[i] = s;
    }
    const float w = J->wts[2 * t + k];
    for (int i = 0; i < D; i++) o[i] += w * y[i];
  }
  (void)h3;
}

static void *moe_worker(void *p) {
  moe_job *J = (moe_job *)p;
  const int D = J->c->dim, H = J->c->hidden;
  float *h1 = (float *)malloc(sizeof(float) * H), *h3 = (float *)malloc(sizeof(float) * H);
  float *y = (float *)malloc(sizeof(float) * D);
  for (;;) {
    pthread_mutex_lock(&J->mu);
    int t = J->next++;
    pthread_mutex_unlock(&J->mu);
    if (t >= J->T) break;
    moe_token(J, t, h1, h3, y);
  }
  free(h1);
  free(h3);
  free(y);
  return NULL;
}

void orc_moe_forward(const orc_moe_cfg *c, const float *params, const float *x, int T, int threads, float *out,
                     int32_t *idx, float *wts) {
  orc_moe_route(c, params, x, T, idx, wts);
  moe_job J = {c, params, x, idx, wts, out, T, 0, PTHREAD_MUTEX_INITIALIZER};
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  pthread_t th[64];
  for (int i = 1; i < threads; i++) pthread_create(&th[i], NULL, moe_worker, &J);
  moe_worker(&J);
  for (int i = 1; i < threads; i++) pthread_join(th[i], NULL);
}
