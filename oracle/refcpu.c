/*
 * refcpu.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see refcpu.h).
 *
 * A plain-C restatement of the reference's non-darwin CPU path.  Each
 * function cites the reference file:line it follows.  Loop orders that
 * decide fp32 rounding (the per-output summation order of linearCF and
 * friends) are kept; loops are interchanged only where that leaves every
 * output's operation sequence unchanged.  Build with -ffp-contract=off so
 * no multiply-add is fused (Go on amd64 does not fuse either).
 *
 * Deviations, all deliberate:
 *  - the VE lookup treats an out-of-range token as a zero row (the
 *    reference indexes out of bounds and panics, ane/train_full.go:1042).
 *  - arch LLAMA2 is not in the reference; it is composed from the
 *    reference's primitives (stories.RMSNorm / RMSNormBackward for gains,
 *    ane/stories/cpu.go:97-111,152-210; linearCF; causalAttentionCF) plus
 *    SwiGLU, with the true gradient.
 *  - grad_mode TRUE fixes the four quirks of the reference backward
 *    (attention scale, RoPE backward, QK-norm coefficient, x0 order).
 */
#include "refcpu.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* threading: parallelFor (ane/engine_other.go:93-123,                 */
/* ane/stories/cpu.go:9-39)                                            */
/* ------------------------------------------------------------------ */
static int g_threads = 1;
static int g_par_linear = 0;

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }
void orc_set_parallel_linear(int on) { g_par_linear = on; }

typedef void (*range_fn)(void *ctx, int start, int end);
typedef struct { range_fn fn; void *ctx; int start, end; } pf_job;

static void *pf_tramp(void *p) {
  pf_job *j = (pf_job *)p;
  j->fn(j->ctx, j->start, j->end);
  return NULL;
}

static void parallel_for_n(int workers, int n, range_fn fn, void *ctx) {
  if (n <= 0) return;
  if (workers < 2 || n < workers * 4) { fn(ctx, 0, n); return; }
  if (workers > n) workers = n;
  int chunk = (n + workers - 1) / workers;
  pthread_t th[256];
  pf_job jobs[256];
  int nj = 0;
  for (int w = 0; w < workers; w++) {
    int s = w * chunk;
    if (s >= n) break;
    int e = s + chunk > n ? n : s + chunk;
    jobs[nj] = (pf_job){fn, ctx, s, e};
    nj++;
  }
  for (int i = 1; i < nj; i++) pthread_create(&th[i], NULL, pf_tramp, &jobs[i]);
  pf_tramp(&jobs[0]);
  for (int i = 1; i < nj; i++) pthread_join(th[i], NULL);
}
static void parallel_for(int n, range_fn fn, void *ctx) { parallel_for_n(g_threads, n, fn, ctx); }
static void parallel_for_linear(int n, range_fn fn, void *ctx) {
  parallel_for_n(g_par_linear ? g_threads : 1, n, fn, ctx);
}

/* ------------------------------------------------------------------ */
/* parameter layout                                                    */
/* ------------------------------------------------------------------ */
#define VE_GATE_CH 12 /* ane/stories/weights.go:28 */

int orc_is_ve_layer(const orc_cfg *c, int l) {
  /* ane/stories/weights.go:22 */
  return c->arch == ORC_ARCH_NANOCHAT && (l % 2) == ((c->layers - 1) % 2);
}

typedef struct {
  int64_t wq, wk, wv, wo, w1, w2, w3, g_att, g_ffn, ve_embed, ve_gate;
} layer_off;
typedef struct {
  layer_off *L;
  int64_t embed, resid, x0l, smear_gate, smear_lambda, backout_lambda, g_final;
  int64_t total;
} param_map;

static void build_map(const orc_cfg *c, param_map *m) {
  int64_t D = c->dim, H = c->hidden, V = c->vocab, NH = c->heads;
  int64_t off = 0;
  m->L = (layer_off *)calloc((size_t)c->layers, sizeof(layer_off));
  for (int l = 0; l < c->layers; l++) {
    layer_off *o = &m->L[l];
    o->wq = off; off += D * D;
    o->wk = off; off += D * D;
    o->wv = off; off += D * D;
    o->wo = off; off += D * D;
    o->w1 = off; off += H * D;
    o->w2 = off; off += D * H;
    o->w3 = o->g_att = o->g_ffn = o->ve_embed = o->ve_gate = -1;
    if (c->arch == ORC_ARCH_LLAMA2) {
      o->w3 = off; off += H * D;
      o->g_att = off; off += D;
      o->g_ffn = off; off += D;
    } else if (orc_is_ve_layer(c, l)) {
      o->ve_embed = off; off += V * D;
      o->ve_gate = off; off += NH * VE_GATE_CH;
    }
  }
  m->embed = off; off += V * D;
  m->resid = m->x0l = m->smear_gate = m->smear_lambda = m->backout_lambda = m->g_final = -1;
  if (c->arch == ORC_ARCH_LLAMA2) {
    m->g_final = off; off += D;
  } else {
    m->resid = off; off += c->layers;
    m->x0l = off; off += c->layers;
    m->smear_gate = off; off += D * D;
    m->smear_lambda = off; off += 1;
    m->backout_lambda = off; off += 1;
  }
  m->total = off;
}

size_t orc_param_count(const orc_cfg *c) {
  param_map m;
  build_map(c, &m);
  free(m.L);
  return (size_t)m.total;
}

int orc_param_segments(const orc_cfg *c, int64_t *offsets, int64_t *sizes, int max) {
  param_map m;
  build_map(c, &m);
  int64_t D = c->dim, H = c->hidden, V = c->vocab, NH = c->heads;
  int n = 0;
#define SEG(o, s) do { if (n < max) { offsets[n] = (o); sizes[n] = (s); } n++; } while (0)
  for (int l = 0; l < c->layers; l++) {
    layer_off *o = &m.L[l];
    SEG(o->wq, D * D); SEG(o->wk, D * D); SEG(o->wv, D * D); SEG(o->wo, D * D);
    SEG(o->w1, H * D); SEG(o->w2, D * H);
    if (c->arch == ORC_ARCH_LLAMA2) { SEG(o->w3, H * D); SEG(o->g_att, D); SEG(o->g_ffn, D); }
    else if (o->ve_embed >= 0) { SEG(o->ve_embed, V * D); SEG(o->ve_gate, NH * VE_GATE_CH); }
  }
  SEG(m.embed, V * D);
  if (c->arch == ORC_ARCH_LLAMA2) SEG(m.g_final, D);
  else {
    SEG(m.resid, c->layers); SEG(m.x0l, c->layers); SEG(m.smear_gate, D * D);
    SEG(m.smear_lambda, 1); SEG(m.backout_lambda, 1);
  }
#undef SEG
  free(m.L);
  return n;
}

/* ------------------------------------------------------------------ */
/* primitives                                                          */
/* ------------------------------------------------------------------ */

/* linearCF (ane/common.go:91-105): out[o,t] = sum_i W[o,i]*in[i,t], the
 * sum over i ascending in fp32.  The t loop is innermost here, which
 * keeps each output's sequence of adds. */
typedef struct { float *out; const float *w, *in; int oc, ic, seq; } lin_ctx;
static void lin_range(void *p, int s, int e) {
  lin_ctx *c = (lin_ctx *)p;
  float *acc = (float *)malloc(sizeof(float) * (size_t)c->seq);
  for (int o = s; o < e; o++) {
    const float *row = c->w + (size_t)o * c->ic;
    for (int t = 0; t < c->seq; t++) acc[t] = 0.f;
    for (int i = 0; i < c->ic; i++) {
      float wv = row[i];
      const float *xi = c->in + (size_t)i * c->seq;
      for (int t = 0; t < c->seq; t++) acc[t] += wv * xi[t];
    }
    memcpy(c->out + (size_t)o * c->seq, acc, sizeof(float) * (size_t)c->seq);
  }
  free(acc);
}
void orc_linear_cf(float *out, const float *w, const float *in, int out_ch, int in_ch, int seq) {
  lin_ctx c = {out, w, in, out_ch, in_ch, seq};
  parallel_for_linear(out_ch, lin_range, &c);
}

/* linearBackwardDXCF (ane/train_full.go:242-259): dx[i,t] = sum_o W[o,i]*dy[o,t] */
typedef struct { float *dx; const float *w, *dy; int oc, ic, seq; } ldx_ctx;
static void ldx_range(void *p, int s, int e) {
  ldx_ctx *c = (ldx_ctx *)p;
  for (int i = s; i < e; i++) {
    float *row = c->dx + (size_t)i * c->seq;
    for (int t = 0; t < c->seq; t++) row[t] = 0.f;
    for (int o = 0; o < c->oc; o++) {
      float wv = c->w[(size_t)o * c->ic + i];
      const float *dyr = c->dy + (size_t)o * c->seq;
      for (int t = 0; t < c->seq; t++) row[t] += wv * dyr[t];
    }
  }
}
static void linear_bwd_dx(float *dx, const float *w, const float *dy, int oc, int ic, int seq) {
  ldx_ctx c = {dx, w, dy, oc, ic, seq};
  parallel_for_linear(ic, ldx_range, &c);
}

/* accumLinearGradCF (ane/train_full.go:213-229): dW[o,i] += sum_t dy[o,t]*x[i,t] */
typedef struct { float *dw; const float *dy, *x; int oc, ic, seq; } ldw_ctx;
static void ldw_range(void *p, int s, int e) {
  ldw_ctx *c = (ldw_ctx *)p;
  for (int o = s; o < e; o++) {
    float *row = c->dw + (size_t)o * c->ic;
    const float *dyr = c->dy + (size_t)o * c->seq;
    for (int i = 0; i < c->ic; i++) {
      const float *xr = c->x + (size_t)i * c->seq;
      float sum = 0.f;
      for (int t = 0; t < c->seq; t++) sum += dyr[t] * xr[t];
      row[i] += sum;
    }
  }
}
static void accum_linear_grad(float *dw, const float *dy, const float *x, int oc, int ic, int seq) {
  ldw_ctx c = {dw, dy, x, oc, ic, seq};
  parallel_for_linear(oc, ldw_range, &c);
}

/* rmsNormNoWeightCFWithRRMS (ane/common.go:157-174): fp32 scale, fp32 mul */
typedef struct { float *out; const float *x; const float *w; int dim, seq; } rn_ctx;
static void rn_cf_range(void *p, int s, int e) {
  rn_ctx *c = (rn_ctx *)p;
  for (int t = s; t < e; t++) {
    double sum = 0.0;
    for (int i = 0; i < c->dim; i++) { double v = c->x[(size_t)i * c->seq + t]; sum += v * v; }
    float scale = (float)(1.0 / sqrt(sum / (double)c->dim + 1e-5));
    for (int i = 0; i < c->dim; i++) {
      size_t idx = (size_t)i * c->seq + t;
      c->out[idx] = c->x[idx] * scale;
    }
  }
}
void orc_rmsnorm_noweight_cf(float *out, const float *x, int dim, int seq) {
  rn_ctx c = {out, x, NULL, dim, seq};
  parallel_for(seq, rn_cf_range, &c);
}

/* stories.RMSNormNoWeight (ane/stories/cpu.go:113-127): f64 scale */
static void rn_st_range(void *p, int s, int e) {
  rn_ctx *c = (rn_ctx *)p;
  for (int t = s; t < e; t++) {
    double sum = 0.0;
    for (int i = 0; i < c->dim; i++) { double v = c->x[(size_t)i * c->seq + t]; sum += v * v; }
    double scale = 1.0 / sqrt(sum / (double)c->dim + 1e-5);
    for (int i = 0; i < c->dim; i++) {
      size_t idx = (size_t)i * c->seq + t;
      c->out[idx] = (float)((double)c->x[idx] * scale);
    }
  }
}
static void rmsnorm_noweight_stories(float *out, const float *x, int dim, int seq) {
  rn_ctx c = {out, x, NULL, dim, seq};
  parallel_for(seq, rn_st_range, &c);
}

/* stories.RMSNorm (ane/stories/cpu.go:97-111): gain, all f64 */
static void rn_w_range(void *p, int s, int e) {
  rn_ctx *c = (rn_ctx *)p;
  for (int t = s; t < e; t++) {
    double sum = 0.0;
    for (int i = 0; i < c->dim; i++) { double v = c->x[(size_t)i * c->seq + t]; sum += v * v; }
    double rrms = 1.0 / sqrt(sum / (double)c->dim + 1e-5);
    for (int i = 0; i < c->dim; i++) {
      size_t idx = (size_t)i * c->seq + t;
      c->out[idx] = (float)((double)c->x[idx] * rrms * (double)c->w[i]);
    }
  }
}
void orc_rmsnorm_cf(float *out, const float *x, const float *w, int dim, int seq) {
  rn_ctx c = {out, x, w, dim, seq};
  parallel_for(seq, rn_w_range, &c);
}

/* rmsNormNoWeightBackwardCF (ane/common.go:176-197) and the identical
 * stories.RMSNormNoWeightBackward (ane/stories/cpu.go:129-150) */
typedef struct { float *dx; const float *dy, *x; int dim, seq; } rnb_ctx;
static void rnb_range(void *p, int s, int e) {
  rnb_ctx *c = (rnb_ctx *)p;
  double invD = 1.0 / (double)c->dim;
  for (int t = s; t < e; t++) {
    double sum = 0.0;
    for (int i = 0; i < c->dim; i++) { double v = c->x[(size_t)i * c->seq + t]; sum += v * v; }
    double rrms = 1.0 / sqrt(sum * invD + 1e-5);
    double dot = 0.0;
    for (int i = 0; i < c->dim; i++) {
      size_t idx = (size_t)i * c->seq + t;
      dot += (double)c->dy[idx] * (double)c->x[idx];
    }
    double coeff = dot * rrms * rrms * rrms * invD;
    for (int i = 0; i < c->dim; i++) {
      size_t idx = (size_t)i * c->seq + t;
      c->dx[idx] = (float)((double)c->dy[idx] * rrms - coeff * (double)c->x[idx]);
    }
  }
}
static void rmsnorm_noweight_bwd(float *dx, const float *dy, const float *x, int dim, int seq) {
  rnb_ctx c = {dx, dy, x, dim, seq};
  parallel_for(seq, rnb_range, &c);
}

/* stories.RMSNormBackward range (ane/stories/cpu.go:191-210), serial:
 * dx overwritten, dw accumulated. */
static void rmsnorm_bwd_gain(float *dx, float *dw, const float *dy, const float *x,
                             const float *w, int d, int s) {
  for (int t = 0; t < s; t++) {
    double sum = 0.0;
    for (int i = 0; i < d; i++) { double v = x[(size_t)i * s + t]; sum += v * v; }
    double rrms = 1.0 / sqrt(sum / (double)d + 1e-5);
    double rrms2InvD = (rrms * rrms) / (double)d;
    double dot = 0.0;
    for (int i = 0; i < d; i++) {
      size_t idx = (size_t)i * s + t;
      dot += (double)(dy[idx] * x[idx] * w[i]);
    }
    for (int i = 0; i < d; i++) {
      size_t idx = (size_t)i * s + t;
      double v = (double)dy[idx] - (double)x[idx] * dot * rrms2InvD;
      dx[idx] = (float)(v * rrms * (double)w[i]);
      dw[i] += (float)((double)(dy[idx] * x[idx]) * rrms);
    }
  }
}

static float relu_sq(float x) { return x <= 0.f ? 0.f : x * x; } /* ane/common.go:146 */
static float sigmoid32(float x) { return 1.0f / (1.0f + (float)exp((double)(-x))); } /* ane/common.go:301 */

/* softmaxRowAccel (ane/accel_stub.go:31-48) */
static void softmax_row(float *out, const float *in, int n) {
  float maxv = in[0];
  for (int i = 1; i < n; i++) if (in[i] > maxv) maxv = in[i];
  double sum = 0.0;
  for (int i = 0; i < n; i++) {
    double e = exp((double)(in[i] - maxv));
    out[i] = (float)e;
    sum += e;
  }
  float inv = (float)(1.0 / sum);
  for (int i = 0; i < n; i++) out[i] *= inv;
}

/* causalAttentionCF (ane/common.go:61-89) */
void orc_causal_attention_cf(float *out, const float *q, const float *k, const float *v,
                             int heads, int hd, int seq) {
  float *scores = (float *)malloc(sizeof(float) * (size_t)seq);
  float *probs = (float *)malloc(sizeof(float) * (size_t)seq);
  float scale = (float)(1.0 / sqrt((double)hd));
  for (int h = 0; h < heads; h++) {
    int base = h * hd;
    for (int t = 0; t < seq; t++) {
      for (int j = 0; j < seq; j++) {
        if (j > t) { scores[j] = -65504.f; continue; }
        float sum = 0.f;
        for (int i = 0; i < hd; i++) sum += q[(size_t)(base + i) * seq + t] * k[(size_t)(base + i) * seq + j];
        scores[j] = sum * scale;
      }
      softmax_row(probs, scores, seq);
      for (int i = 0; i < hd; i++) {
        float sum = 0.f;
        for (int j = 0; j < seq; j++) sum += probs[j] * v[(size_t)(base + i) * seq + j];
        out[(size_t)(base + i) * seq + t] = sum;
      }
    }
  }
  free(scores);
  free(probs);
}

/* causalAttentionBackwardCF (ane/train_full.go:261-316); `scale` is 1.0 in
 * the reference (compat) and 1/sqrt(hd) for the true gradient. */
static void causal_attention_bwd(float *dq, float *dk, float *dv, const float *dout, const float *q,
                                 const float *k, const float *v, int heads, int hd, int seq,
                                 float scale) {
  size_t n = (size_t)heads * hd * seq;
  memset(dq, 0, n * sizeof(float));
  memset(dk, 0, n * sizeof(float));
  memset(dv, 0, n * sizeof(float));
  float *scores = (float *)malloc(sizeof(float) * (size_t)seq);
  float *probs = (float *)malloc(sizeof(float) * (size_t)seq);
  float *dsc = (float *)malloc(sizeof(float) * (size_t)seq);
  for (int h = 0; h < heads; h++) {
    int base = h * hd;
    for (int t = 0; t < seq; t++) {
      float maxv = -INFINITY;
      for (int s = 0; s <= t; s++) {
        float sum = 0.f;
        for (int i = 0; i < hd; i++) sum += q[(size_t)(base + i) * seq + t] * k[(size_t)(base + i) * seq + s];
        scores[s] = sum * scale;
        if (scores[s] > maxv) maxv = scores[s];
      }
      double total = 0.0;
      for (int s = 0; s <= t; s++) {
        double e = exp((double)(scores[s] - maxv));
        probs[s] = (float)e;
        total += e;
      }
      float invTotal = (float)(1.0 / total);
      for (int s = 0; s <= t; s++) probs[s] *= invTotal;
      float dsSum = 0.f;
      for (int s = 0; s <= t; s++) {
        float dot = 0.f;
        for (int i = 0; i < hd; i++) dot += dout[(size_t)(base + i) * seq + t] * v[(size_t)(base + i) * seq + s];
        dsc[s] = dot;
        dsSum += probs[s] * dot;
      }
      for (int s = 0; s <= t; s++) {
        float ds = probs[s] * (dsc[s] - dsSum) * scale;
        for (int i = 0; i < hd; i++) {
          size_t qi = (size_t)(base + i) * seq;
          dq[qi + t] += ds * k[qi + s];
          dk[qi + s] += ds * q[qi + t];
          dv[qi + s] += probs[s] * dout[qi + t];
        }
      }
    }
  }
  free(scores);
  free(probs);
  free(dsc);
}

/* buildRoPETables (ane/train_util.go:183-202) with theta as a parameter */
void orc_build_rope(float *cos_t, float *sin_t, int seq, int hd, double theta) {
  int half = hd / 2;
  for (int pos = 0; pos < seq; pos++)
    for (int i = 0; i < half; i++) {
      double freq = (double)pos / pow(theta, (double)(2 * i) / (double)hd);
      cos_t[pos * half + i] = (float)cos(freq);
      sin_t[pos * half + i] = (float)sin(freq);
    }
}

/* applyRoPECFInPlace (ane/train_util.go:204-224): interleaved pairs */
void orc_apply_rope_cf(float *x, int heads, int hd, int seq, const float *cs, const float *sn) {
  int half = hd / 2;
  for (int h = 0; h < heads; h++)
    for (int i = 0; i < half; i++) {
      size_t even = (size_t)(h * hd + 2 * i) * seq, odd = even + seq;
      for (int t = 0; t < seq; t++) {
        float c = cs[t * half + i], s = sn[t * half + i];
        float e = x[even + t], o = x[odd + t];
        x[even + t] = e * c - o * s;
        x[odd + t] = o * c + e * s;
      }
    }
}
/* transpose of the rotation (true-gradient RoPE backward; the reference has none) */
static void rope_bwd_cf(float *dx, int heads, int hd, int seq, const float *cs, const float *sn) {
  int half = hd / 2;
  for (int h = 0; h < heads; h++)
    for (int i = 0; i < half; i++) {
      size_t even = (size_t)(h * hd + 2 * i) * seq, odd = even + seq;
      for (int t = 0; t < seq; t++) {
        float c = cs[t * half + i], s = sn[t * half + i];
        float e = dx[even + t], o = dx[odd + t];
        dx[even + t] = e * c + o * s;
        dx[odd + t] = o * c - e * s;
      }
    }
}

/* qkNormCF (ane/common.go:199-227) */
void orc_qknorm_cf(float *q, float *k, int dim, int heads, int seq) {
  int hd = dim / heads;
  const double qk = 1.2;
  for (int h = 0; h < heads; h++) {
    int base = h * hd;
    for (int t = 0; t < seq; t++) {
      double sq = 0.0;
      for (int i = 0; i < hd; i++) { double v = q[(size_t)(base + i) * seq + t]; sq += v * v; }
      float scq = (float)(qk / sqrt(sq / (double)hd + 1e-5));
      for (int i = 0; i < hd; i++) q[(size_t)(base + i) * seq + t] *= scq;
      double sk = 0.0;
      for (int i = 0; i < hd; i++) { double v = k[(size_t)(base + i) * seq + t]; sk += v * v; }
      float sck = (float)(qk / sqrt(sk / (double)hd + 1e-5));
      for (int i = 0; i < hd; i++) k[(size_t)(base + i) * seq + t] *= sck;
    }
  }
}

/* qkNormBackwardCF (ane/common.go:229-270); coef2 = qkScale^2 in the
 * reference (compat), qkScale for the true derivative. */
static void qknorm_bwd_one(float *d, const float *pre, int dim, int heads, int seq, double coef2) {
  int hd = dim / heads;
  const double qk = 1.2;
  double invHD = 1.0 / (double)hd;
  for (int h = 0; h < heads; h++) {
    int base = h * hd;
    for (int t = 0; t < seq; t++) {
      double sum = 0.0;
      for (int i = 0; i < hd; i++) { double v = pre[(size_t)(base + i) * seq + t]; sum += v * v; }
      double rr = 1.0 / sqrt(sum * invHD + 1e-5);
      double dot = 0.0;
      for (int i = 0; i < hd; i++) {
        size_t idx = (size_t)(base + i) * seq + t;
        dot += (double)d[idx] * (double)pre[idx];
      }
      double coeff = dot * rr * rr * rr * invHD * coef2;
      for (int i = 0; i < hd; i++) {
        size_t idx = (size_t)(base + i) * seq + t;
        d[idx] = (float)((double)d[idx] * rr * qk - coeff * (double)pre[idx]);
      }
    }
  }
}

/* logitSoftcap / logitSoftcapBackward (ane/common.go:272-287) */
void orc_softcap(float *x, size_t n) {
  const double invCap = 1.0 / 15.0;
  for (size_t i = 0; i < n; i++) x[i] = 15.0f * (float)tanh((double)x[i] * invCap);
}
static void softcap_bwd(float *g, const float *pre, size_t n) {
  const double invCap = 1.0 / 15.0;
  for (size_t i = 0; i < n; i++) {
    double t = tanh((double)pre[i] * invCap);
    g[i] = g[i] * (float)(1.0 - t * t);
  }
}

/* stories.EmbedLookup (ane/stories/cpu.go:41-72) */
static void embed_lookup(float *out, const float *embed, int vocab, const uint16_t *tok, int dim, int seq) {
  for (int t = 0; t < seq; t++) {
    int tk = tok[t];
    for (int d = 0; d < dim; d++)
      out[(size_t)d * seq + t] = (tk < vocab) ? embed[(size_t)tk * dim + d] : 0.f;
  }
}
/* stories.EmbedBackward (ane/stories/cpu.go:74-95) */
static void embed_backward(float *dembed, const float *dx, int vocab, const uint16_t *tok, int dim, int seq) {
  for (int t = 0; t < seq; t++) {
    int tk = tok[t];
    if (tk >= vocab) continue;
    for (int d = 0; d < dim; d++) dembed[(size_t)tk * dim + d] += dx[(size_t)d * seq + t];
  }
}

/* stories.MatMulVocabSeq (ane/stories/cpu.go:303-327) */
typedef struct { float *logits; const float *embed, *x; int vocab, dim, seq; } mvs_ctx;
static void mvs_range(void *p, int s, int e) {
  mvs_ctx *c = (mvs_ctx *)p;
  float *acc = (float *)malloc(sizeof(float) * (size_t)c->seq);
  for (int v = s; v < e; v++) {
    const float *eb = c->embed + (size_t)v * c->dim;
    for (int t = 0; t < c->seq; t++) acc[t] = 0.f;
    for (int d = 0; d < c->dim; d++) {
      float w = eb[d];
      const float *xd = c->x + (size_t)d * c->seq;
      for (int t = 0; t < c->seq; t++) acc[t] += w * xd[t];
    }
    memcpy(c->logits + (size_t)v * c->seq, acc, sizeof(float) * (size_t)c->seq);
  }
  free(acc);
}
static void matmul_vocab_seq(float *logits, const float *embed, const float *x, int vocab, int dim, int seq) {
  mvs_ctx c = {logits, embed, x, vocab, dim, seq};
  parallel_for(vocab, mvs_range, &c);
}

/* stories.MatMulEmbedTScale (ane/stories/cpu.go:333-360) */
typedef struct { float *dx; const float *embed, *dl; int vocab, dim, seq; float scale; } met_ctx;
static void met_range(void *p, int s, int e) {
  met_ctx *c = (met_ctx *)p;
  float *acc = (float *)malloc(sizeof(float) * (size_t)c->seq);
  for (int d = s; d < e; d++) {
    for (int t = 0; t < c->seq; t++) acc[t] = 0.f;
    for (int v = 0; v < c->vocab; v++) {
      float w = c->embed[(size_t)v * c->dim + d];
      const float *dlv = c->dl + (size_t)v * c->seq;
      for (int t = 0; t < c->seq; t++) acc[t] += w * dlv[t];
    }
    float *out = c->dx + (size_t)d * c->seq;
    for (int t = 0; t < c->seq; t++) out[t] = acc[t] * c->scale;
  }
  free(acc);
}
static void matmul_embedT_scale(float *dx, const float *embed, const float *dl, int vocab, int dim,
                                int seq, float scale) {
  if (scale == 0.f) { memset(dx, 0, sizeof(float) * (size_t)dim * seq); return; }
  met_ctx c = {dx, embed, dl, vocab, dim, seq, scale};
  parallel_for(dim, met_range, &c);
}

/* stories.MatMulGradEmbedScale (ane/stories/cpu.go:366-385): overwrite */
typedef struct { float *de; const float *dl, *x; int vocab, dim, seq; float scale; } mge_ctx;
static void mge_range(void *p, int s, int e) {
  mge_ctx *c = (mge_ctx *)p;
  for (int v = s; v < e; v++)
    for (int d = 0; d < c->dim; d++) {
      float sum = 0.f;
      const float *dlv = c->dl + (size_t)v * c->seq, *xd = c->x + (size_t)d * c->seq;
      for (int t = 0; t < c->seq; t++) sum += dlv[t] * xd[t];
      c->de[(size_t)v * c->dim + d] = sum * c->scale;
    }
}
static void matmul_grad_embed_scale(float *de, const float *dl, const float *x, int vocab, int dim,
                                    int seq, float scale) {
  if (scale == 0.f) { memset(de, 0, sizeof(float) * (size_t)vocab * dim); return; }
  mge_ctx c = {de, dl, x, vocab, dim, seq, scale};
  parallel_for(vocab, mge_range, &c);
}

/* stories.CrossEntropyLoss (ane/stories/cpu.go:212-292): dlogits and
 * logits may alias.  Loss shards are summed per parallelFor chunk. */
typedef struct {
  float *dl; const float *lg; const uint16_t *tg; int v, s;
  double *shard_loss; int *shard_valid; int nshards;
} ce_ctx;
static void ce_range(void *p, int start, int end) {
  ce_ctx *c = (ce_ctx *)p;
  int idx = (int)((long)start * c->nshards / c->s);
  double ll = 0.0;
  int lv = 0;
  for (int t = start; t < end; t++) {
    float mx = c->lg[t];
    for (int i = 1; i < c->v; i++) { float val = c->lg[(size_t)i * c->s + t]; if (val > mx) mx = val; }
    double sum = 0.0;
    for (int i = 0; i < c->v; i++) {
      float e = (float)exp((double)(c->lg[(size_t)i * c->s + t] - mx));
      c->dl[(size_t)i * c->s + t] = e;
      sum += (double)e;
    }
    float inv = (float)(1.0 / sum);
    int tgt = c->tg[t];
    for (int i = 0; i < c->v; i++) c->dl[(size_t)i * c->s + t] *= inv;
    if (tgt >= c->v) {
      for (int i = 0; i < c->v; i++) c->dl[(size_t)i * c->s + t] = 0.f;
      continue;
    }
    float pp = c->dl[(size_t)tgt * c->s + t];
    if (pp < 1e-10f) pp = 1e-10f;
    ll -= log((double)pp);
    c->dl[(size_t)tgt * c->s + t] -= 1.f;
    lv++;
  }
  /* the reference serialises these adds with a mutex */
  c->shard_loss[idx] += ll;
  c->shard_valid[idx] += lv;
}
typedef struct { float *dl; const uint16_t *tg; int v, s; float inv; } ces_ctx;
static void ces_range(void *p, int start, int end) {
  ces_ctx *c = (ces_ctx *)p;
  for (int t = start; t < end; t++) {
    if (c->tg[t] >= c->v) continue;
    for (int i = 0; i < c->v; i++) c->dl[(size_t)i * c->s + t] *= c->inv;
  }
}
float orc_cross_entropy(float *dl, const float *lg, const uint16_t *tg, int v, int s) {
  if (v <= 0 || s <= 0) return 0.f;
  int ns = g_threads;
  double *sl = (double *)calloc((size_t)ns, sizeof(double));
  int *sv = (int *)calloc((size_t)ns, sizeof(int));
  ce_ctx c = {dl, lg, tg, v, s, sl, sv, ns};
  /* shards are written by distinct chunks; with pthreads the mutex of the
   * reference is unnecessary because every chunk maps to its own index */
  parallel_for(s, ce_range, &c);
  double loss = 0.0;
  int valid = 0;
  for (int i = 0; i < ns; i++) { loss += sl[i]; valid += sv[i]; }
  free(sl);
  free(sv);
  if (valid == 0) return 0.f;
  ces_ctx cs = {dl, tg, v, s, (float)(1.0 / (double)valid)};
  parallel_for(s, ces_range, &cs);
  return (float)(loss / (double)valid);
}

/* veForwardCF (ane/train_full.go:1035-1059) */
static void ve_forward(float *v, float *ve, float *gact, const float *vemb, const float *vgate,
                       const float *x, const uint16_t *tok, int dim, int heads, int vocab, int seq) {
  int hd = dim / heads;
  for (int t = 0; t < seq; t++) {
    int tk = tok[t];
    for (int d = 0; d < dim; d++) ve[(size_t)d * seq + t] = tk < vocab ? vemb[(size_t)tk * dim + d] : 0.f;
    for (int h = 0; h < heads; h++) {
      float gp = 0.f;
      for (int c = 0; c < VE_GATE_CH; c++) gp += vgate[h * VE_GATE_CH + c] * x[(size_t)c * seq + t];
      float act = (float)(1.0 / (1.0 + exp(-(double)gp)));
      gact[(size_t)h * seq + t] = act;
      float gate = 3.0f * act;
      for (int d = h * hd; d < (h + 1) * hd; d++) v[(size_t)d * seq + t] += gate * ve[(size_t)d * seq + t];
    }
  }
}
/* veBackwardCF (ane/train_full.go:1062-1086) */
static void ve_backward(float *dvemb, float *dvgate, float *dprev, const float *dv, const float *ve,
                        const float *gact, const float *vgate, const float *x, const uint16_t *tok,
                        int dim, int heads, int vocab, int seq) {
  int hd = dim / heads;
  for (int t = 0; t < seq; t++) {
    int tk = tok[t];
    for (int h = 0; h < heads; h++) {
      float act = gact[(size_t)h * seq + t];
      float gate = 3.0f * act;
      float dg = 0.f;
      for (int d = h * hd; d < (h + 1) * hd; d++) {
        float dvdt = dv[(size_t)d * seq + t];
        if (tk < vocab) dvemb[(size_t)tk * dim + d] += dvdt * gate;
        dg += dvdt * ve[(size_t)d * seq + t];
      }
      float dgp = dg * 3.0f * act * (1.f - act);
      for (int c = 0; c < VE_GATE_CH; c++) {
        dvgate[h * VE_GATE_CH + c] += dgp * x[(size_t)c * seq + t];
        dprev[(size_t)c * seq + t] += dgp * vgate[h * VE_GATE_CH + c];
      }
    }
  }
}

/* smearForwardWithSaveCF (ane/common.go:324-339) */
static void smear_forward(float *x, float *xpre, const float *sg, float lam, float *gpre, float *shifted,
                          float *gact, int dim, int seq) {
  memcpy(xpre, x, sizeof(float) * (size_t)dim * seq);
  orc_linear_cf(gpre, sg, xpre, dim, dim, seq);
  for (int d = 0; d < dim; d++)
    for (int t = 0; t < seq; t++) {
      size_t i = (size_t)d * seq + t;
      gact[i] = sigmoid32(gpre[i]);
      shifted[i] = t == 0 ? 0.f : xpre[i - 1];
      x[i] += lam * gact[i] * shifted[i];
    }
}
/* smearBackwardCF (ane/common.go:343-382) */
static void smear_backward(float *dout, const float *xpre, const float *sg, float lam,
                           const float *shifted, const float *gact, float *gsg, float *glam,
                           int dim, int seq) {
  double dl = 0.0;
  float *dgp = (float *)malloc(sizeof(float) * (size_t)dim * seq);
  for (int d = 0; d < dim; d++)
    for (int t = 0; t < seq; t++) {
      size_t i = (size_t)d * seq + t;
      float g = gact[i], s = shifted[i], dy = dout[i];
      dl += (double)(dy * g * s);
      dgp[i] = dy * lam * s * g * (1.f - g);
      float dsh = dy * lam * g;
      if (t > 0) dout[i - 1] += dsh;
    }
  glam[0] += (float)dl;
  accum_linear_grad(gsg, dgp, xpre, dim, dim, seq);
  float *dxg = (float *)malloc(sizeof(float) * (size_t)dim * seq);
  linear_bwd_dx(dxg, sg, dgp, dim, dim, seq);
  for (size_t i = 0; i < (size_t)dim * seq; i++) dout[i] += dxg[i];
  free(dxg);
  free(dgp);
}

/* ------------------------------------------------------------------ */
/* model                                                               */
/* ------------------------------------------------------------------ */
typedef struct {
  float *x, *xn, *q, *k, *v, *att, *x2, *xn2, *h1, *h3, *gate, *qpre, *kpre, *ve, *gact;
} lcache;

typedef struct {
  const orc_cfg *c;
  param_map m;
  int D, H, NH, HD, L, V, S;
  float *rope_cos, *rope_sin;
  lcache *lc;
  float *x, *x0, *xpre_embnorm, *smear_xpre, *smear_gpre, *smear_shift, *smear_gact, *xmid;
  float *tmp, *xfinal, *xnorm, *logits, *logits_pre;
} model;

static float *fz(size_t n) { return (float *)calloc(n, sizeof(float)); }

static void model_init(model *M, const orc_cfg *c) {
  memset(M, 0, sizeof(*M));
  M->c = c;
  build_map(c, &M->m);
  M->D = c->dim; M->H = c->hidden; M->NH = c->heads; M->HD = c->dim / c->heads;
  M->L = c->layers; M->V = c->vocab; M->S = c->seq;
  size_t DS = (size_t)M->D * M->S, HS = (size_t)M->H * M->S;
  M->rope_cos = fz((size_t)M->S * M->HD / 2);
  M->rope_sin = fz((size_t)M->S * M->HD / 2);
  orc_build_rope(M->rope_cos, M->rope_sin, M->S, M->HD, c->rope_theta);
  M->lc = (lcache *)calloc((size_t)M->L, sizeof(lcache));
  for (int l = 0; l < M->L; l++) {
    lcache *a = &M->lc[l];
    a->x = fz(DS); a->xn = fz(DS); a->q = fz(DS); a->k = fz(DS); a->v = fz(DS); a->att = fz(DS);
    a->x2 = fz(DS); a->xn2 = fz(DS); a->h1 = fz(HS); a->h3 = fz(HS); a->gate = fz(HS);
    a->qpre = fz(DS); a->kpre = fz(DS); a->ve = fz(DS); a->gact = fz((size_t)M->NH * M->S);
  }
  M->x = fz(DS); M->x0 = fz(DS); M->xpre_embnorm = fz(DS); M->smear_xpre = fz(DS);
  M->smear_gpre = fz(DS); M->smear_shift = fz(DS); M->smear_gact = fz(DS); M->xmid = fz(DS);
  M->tmp = fz(DS); M->xfinal = fz(DS); M->xnorm = fz(DS);
  M->logits = fz((size_t)M->V * M->S); M->logits_pre = fz((size_t)M->V * M->S);
}

static void model_free(model *M) {
  for (int l = 0; l < M->L; l++) {
    lcache *a = &M->lc[l];
    free(a->x); free(a->xn); free(a->q); free(a->k); free(a->v); free(a->att); free(a->x2);
    free(a->xn2); free(a->h1); free(a->h3); free(a->gate); free(a->qpre); free(a->kpre);
    free(a->ve); free(a->gact);
  }
  free(M->lc); free(M->m.L); free(M->rope_cos); free(M->rope_sin);
  free(M->x); free(M->x0); free(M->xpre_embnorm); free(M->smear_xpre); free(M->smear_gpre);
  free(M->smear_shift); free(M->smear_gact); free(M->xmid); free(M->tmp); free(M->xfinal);
  free(M->xnorm); free(M->logits); free(M->logits_pre);
}

/* forwardTrainingCPU (ane/train_full.go:383-453) for NANOCHAT; the LLAMA2
 * variant swaps in gain RMSNorm, no QK-norm/VE/smear/lambdas/backout and
 * a SwiGLU FFN.  Leaves the final hidden state in M->xfinal. */
static void forward_body(model *M, const float *P, const uint16_t *tok) {
  const orc_cfg *c = M->c;
  int D = M->D, H = M->H, NH = M->NH, HD = M->HD, S = M->S;
  size_t DS = (size_t)D * S;
  int llama = c->arch == ORC_ARCH_LLAMA2;
  embed_lookup(M->x, P + M->m.embed, M->V, tok, D, S);
  if (!llama) {
    memcpy(M->xpre_embnorm, M->x, DS * sizeof(float));
    orc_rmsnorm_noweight_cf(M->x, M->x, D, S);
    memcpy(M->x0, M->x, DS * sizeof(float));
    smear_forward(M->x, M->smear_xpre, P + M->m.smear_gate, P[M->m.smear_lambda], M->smear_gpre,
                  M->smear_shift, M->smear_gact, D, S);
  }
  float *cur = M->x, *next = M->tmp;
  int mid = M->L / 2;
  for (int l = 0; l < M->L; l++) {
    layer_off *o = &M->m.L[l];
    lcache *a = &M->lc[l];
    memcpy(a->x, cur, DS * sizeof(float));
    if (llama) orc_rmsnorm_cf(a->xn, a->x, P + o->g_att, D, S);
    else orc_rmsnorm_noweight_cf(a->xn, a->x, D, S);
    orc_linear_cf(a->q, P + o->wq, a->xn, D, D, S);
    orc_linear_cf(a->k, P + o->wk, a->xn, D, D, S);
    orc_apply_rope_cf(a->q, NH, HD, S, M->rope_cos, M->rope_sin);
    orc_apply_rope_cf(a->k, NH, HD, S, M->rope_cos, M->rope_sin);
    if (!llama) {
      memcpy(a->qpre, a->q, DS * sizeof(float));
      memcpy(a->kpre, a->k, DS * sizeof(float));
      orc_qknorm_cf(a->q, a->k, D, NH, S);
    }
    orc_linear_cf(a->v, P + o->wv, a->xn, D, D, S);
    if (o->ve_embed >= 0)
      ve_forward(a->v, a->ve, a->gact, P + o->ve_embed, P + o->ve_gate, a->x, tok, D, NH, M->V, S);
    orc_causal_attention_cf(a->att, a->q, a->k, a->v, NH, HD, S);
    orc_linear_cf(next, P + o->wo, a->att, D, D, S);
    float rl = llama ? 1.f : P[M->m.resid + l];
    float xl = llama ? 0.f : P[M->m.x0l + l];
    for (size_t j = 0; j < DS; j++) a->x2[j] = rl * a->x[j] + next[j];
    if (xl != 0.f)
      for (size_t j = 0; j < DS; j++) a->x2[j] += xl * M->x0[j];
    if (llama) {
      orc_rmsnorm_cf(a->xn2, a->x2, P + o->g_ffn, D, S);
      orc_linear_cf(a->h1, P + o->w1, a->xn2, H, D, S);
      orc_linear_cf(a->h3, P + o->w3, a->xn2, H, D, S);
      for (size_t j = 0; j < (size_t)H * S; j++) a->gate[j] = a->h1[j] * sigmoid32(a->h1[j]) * a->h3[j];
    } else {
      orc_rmsnorm_noweight_cf(a->xn2, a->x2, D, S);
      orc_linear_cf(a->h1, P + o->w1, a->xn2, H, D, S);
      for (size_t j = 0; j < (size_t)H * S; j++) a->gate[j] = relu_sq(a->h1[j]);
    }
    orc_linear_cf(next, P + o->w2, a->gate, D, H, S);
    for (size_t j = 0; j < DS; j++) next[j] = rl * a->x2[j] + next[j];
    if (xl != 0.f)
      for (size_t j = 0; j < DS; j++) next[j] += xl * M->x0[j];
    float *t = cur; cur = next; next = t;
    if (!llama && l == mid - 1) memcpy(M->xmid, cur, DS * sizeof(float));
  }
  if (!llama) {
    float lb = P[M->m.backout_lambda];
    for (size_t i = 0; i < DS; i++) cur[i] -= lb * M->xmid[i]; /* backoutForwardCF */
  }
  memcpy(M->xfinal, cur, DS * sizeof(float));
}

/* classifier head forward: xnorm, logits (post-softcap) and logits_pre */
static void head_forward(model *M, const float *P) {
  int D = M->D, S = M->S, V = M->V;
  if (M->c->arch == ORC_ARCH_LLAMA2) orc_rmsnorm_cf(M->xnorm, M->xfinal, P + M->m.g_final, D, S);
  else rmsnorm_noweight_stories(M->xnorm, M->xfinal, D, S);
  matmul_vocab_seq(M->logits, P + M->m.embed, M->xnorm, V, D, S);
  memcpy(M->logits_pre, M->logits, sizeof(float) * (size_t)V * S);
  if (M->c->arch == ORC_ARCH_NANOCHAT) orc_softcap(M->logits, (size_t)V * S);
}

float orc_forward_loss(const orc_cfg *c, const float *P, const uint16_t *tokens, const uint16_t *targets,
                       int nseq, float *logits_out, float *loss_per_seq) {
  model M;
  model_init(&M, c);
  double total = 0.0;
  size_t VS = (size_t)c->vocab * c->seq;
  float *dl = fz(VS);
  for (int b = 0; b < nseq; b++) {
    forward_body(&M, P, tokens + (size_t)b * c->seq);
    head_forward(&M, P);
    if (logits_out) memcpy(logits_out + (size_t)b * VS, M.logits, VS * sizeof(float));
    float loss = orc_cross_entropy(dl, M.logits, targets + (size_t)b * c->seq, c->vocab, c->seq);
    if (loss_per_seq) loss_per_seq[b] = loss;
    total += loss;
  }
  free(dl);
  model_free(&M);
  return nseq > 0 ? (float)(total / nseq) : 0.f;
}

/* One sequence of backward, accumulating loss-scaled grads into G
 * (backwardAndAccumulate, ane/train_full.go:691-820, with the final head of
 * runFinalHead, ane/train_full.go:480-558).  Returns the loss. */
static float backward_one(model *M, const float *P, const uint16_t *tok, const uint16_t *tgt,
                          float loss_scale, float *G) {
  const orc_cfg *c = M->c;
  int D = M->D, H = M->H, NH = M->NH, HD = M->HD, S = M->S, V = M->V;
  size_t DS = (size_t)D * S, HS = (size_t)H * S, VS = (size_t)V * S;
  int llama = c->arch == ORC_ARCH_LLAMA2;
  int compat = c->grad_mode == ORC_GRAD_COMPAT && !llama;
  forward_body(M, P, tok);
  head_forward(M, P);

  /* --- head backward (runFinalHead) --- */
  float *dl = M->logits; /* CE writes dlogits in place */
  float loss = orc_cross_entropy(dl, M->logits, tgt, V, S);
  float grad_scale = loss_scale;
  if (!llama) softcap_bwd(dl, M->logits_pre, VS);
  float *gE = fz((size_t)V * D);
  matmul_grad_embed_scale(gE, dl, M->xnorm, V, D, S, grad_scale);
  float *dy = fz(DS), *dcur = fz(DS), *dprev = fz(DS);
  matmul_embedT_scale(dy, P + M->m.embed, dl, V, D, S, grad_scale);
  if (llama) rmsnorm_bwd_gain(dcur, G + M->m.g_final, dy, M->xfinal, P + M->m.g_final, D, S);
  else rmsnorm_noweight_bwd(dcur, dy, M->xfinal, D, S);

  float *gx0 = fz(DS), *ginj = fz(DS);
  float *gGate = fz(HS), *gH1 = fz(HS), *gH3 = fz(HS), *gXN = fz(DS), *gX2 = fz(DS), *gAtt = fz(DS);
  float *gQ = fz(DS), *gK = fz(DS), *gV = fz(DS);
  int mid = M->L / 2;
  if (!llama) {
    /* backoutBackwardCF (ane/common.go:393-403) then the injected grad */
    float lb = P[M->m.backout_lambda];
    double dlam = 0.0;
    for (size_t i = 0; i < DS; i++) dlam -= (double)(dcur[i] * M->xmid[i]);
    G[M->m.backout_lambda] += (float)dlam;
    for (size_t i = 0; i < DS; i++) ginj[i] = -lb * dcur[i];
  }
  for (int l = M->L - 1; l >= 0; l--) {
    layer_off *o = &M->m.L[l];
    lcache *a = &M->lc[l];
    float rl = llama ? 1.f : P[M->m.resid + l];
    float xl = llama ? 0.f : P[M->m.x0l + l];
    /* --- FFN (backwardFFNCPU, ane/train_full.go:592-601) --- */
    for (size_t i = 0; i < DS; i++) gX2[i] = rl * dcur[i];
    linear_bwd_dx(gGate, P + o->w2, dcur, D, H, S);
    if (llama) {
      for (size_t i = 0; i < HS; i++) {
        float h = a->h1[i], sg = sigmoid32(h);
        float silu = h * sg;
        gH3[i] = gGate[i] * silu;
        gH1[i] = gGate[i] * a->h3[i] * (sg + h * sg * (1.f - sg));
      }
      linear_bwd_dx(gXN, P + o->w1, gH1, H, D, S);
      linear_bwd_dx(dprev, P + o->w3, gH3, H, D, S);
      for (size_t i = 0; i < DS; i++) gXN[i] += dprev[i];
      rmsnorm_bwd_gain(dprev, G + o->g_ffn, gXN, a->x2, P + o->g_ffn, D, S);
    } else {
      for (size_t i = 0; i < HS; i++) { float r = a->h1[i] < 0.f ? 0.f : a->h1[i]; gH1[i] = gGate[i] * 2.f * r; }
      linear_bwd_dx(gXN, P + o->w1, gH1, H, D, S);
      rmsnorm_noweight_bwd(dprev, gXN, a->x2, D, S);
    }
    for (size_t i = 0; i < DS; i++) gX2[i] += dprev[i];
    accum_linear_grad(G + o->w2, dcur, a->gate, D, H, S);
    accum_linear_grad(G + o->w1, gH1, a->xn2, H, D, S);
    if (llama) accum_linear_grad(G + o->w3, gH3, a->xn2, H, D, S);
    double dRL = 0.0, dXL = 0.0;
    if (!llama) {
      for (size_t j = 0; j < DS; j++) dRL += (double)(dcur[j] * a->x2[j]);
      for (size_t j = 0; j < DS; j++) dXL += (double)(dcur[j] * M->x0[j]);
      for (size_t j = 0; j < DS; j++) gx0[j] += xl * dcur[j];
    }
    /* --- attention (backwardAttentionCPU, ane/train_full.go:644-675) --- */
    linear_bwd_dx(gAtt, P + o->wo, gX2, D, D, S);
    float ascale = compat ? 1.0f : (float)(1.0 / sqrt((double)HD));
    causal_attention_bwd(gQ, gK, gV, gAtt, a->q, a->k, a->v, NH, HD, S, ascale);
    if (!llama) {
      double coef2 = compat ? 1.2 * 1.2 : 1.2;
      qknorm_bwd_one(gQ, a->qpre, D, NH, S, coef2);
      qknorm_bwd_one(gK, a->kpre, D, NH, S, coef2);
    }
    if (!compat) {
      rope_bwd_cf(gQ, NH, HD, S, M->rope_cos, M->rope_sin);
      rope_bwd_cf(gK, NH, HD, S, M->rope_cos, M->rope_sin);
    }
    linear_bwd_dx(gXN, P + o->wq, gQ, D, D, S);
    linear_bwd_dx(dprev, P + o->wk, gK, D, D, S);
    for (size_t i = 0; i < DS; i++) gXN[i] += dprev[i];
    linear_bwd_dx(dprev, P + o->wv, gV, D, D, S);
    for (size_t i = 0; i < DS; i++) gXN[i] += dprev[i];
    if (llama) rmsnorm_bwd_gain(dprev, G + o->g_att, gXN, a->x, P + o->g_att, D, S);
    else rmsnorm_noweight_bwd(dprev, gXN, a->x, D, S);
    if (o->ve_embed >= 0)
      ve_backward(G + o->ve_embed, G + o->ve_gate, dprev, gV, a->ve, a->gact, P + o->ve_gate, a->x,
                  tok, D, NH, V, S);
    for (size_t i = 0; i < DS; i++) dprev[i] += rl * gX2[i];
    accum_linear_grad(G + o->wo, gX2, a->att, D, D, S);
    accum_linear_grad(G + o->wq, gQ, a->xn, D, D, S);
    accum_linear_grad(G + o->wk, gK, a->xn, D, D, S);
    accum_linear_grad(G + o->wv, gV, a->xn, D, D, S);
    if (!llama) {
      for (size_t j = 0; j < DS; j++) dRL += (double)(gX2[j] * a->x[j]);
      for (size_t j = 0; j < DS; j++) dXL += (double)(gX2[j] * M->x0[j]);
      for (size_t j = 0; j < DS; j++) gx0[j] += xl * gX2[j];
      G[M->m.resid + l] += (float)dRL;
      G[M->m.x0l + l] += (float)dXL;
    }
    float *t = dcur; dcur = dprev; dprev = t;
    if (!llama && l == mid)
      for (size_t i = 0; i < DS; i++) dcur[i] += ginj[i];
  }
  if (!llama) {
    if (compat) {
      /* x0 grad added before smear backward (ane/train_full.go:790-798) */
      for (size_t i = 0; i < DS; i++) dcur[i] += gx0[i];
      smear_backward(dcur, M->smear_xpre, P + M->m.smear_gate, P[M->m.smear_lambda], M->smear_shift,
                     M->smear_gact, G + M->m.smear_gate, G + M->m.smear_lambda, D, S);
    } else {
      smear_backward(dcur, M->smear_xpre, P + M->m.smear_gate, P[M->m.smear_lambda], M->smear_shift,
                     M->smear_gact, G + M->m.smear_gate, G + M->m.smear_lambda, D, S);
      for (size_t i = 0; i < DS; i++) dcur[i] += gx0[i];
    }
    rmsnorm_noweight_bwd(dprev, dcur, M->xpre_embnorm, D, S);
    memcpy(dcur, dprev, DS * sizeof(float));
  }
  embed_backward(gE, dcur, V, tok, D, S);
  float *Ge = G + M->m.embed;
  for (size_t i = 0; i < (size_t)V * D; i++) Ge[i] += gE[i];
  free(gE); free(dy); free(dcur); free(dprev); free(gx0); free(ginj); free(gGate); free(gH1);
  free(gH3); free(gXN); free(gX2); free(gAtt); free(gQ); free(gK); free(gV);
  return loss;
}

float orc_grads(const orc_cfg *c, const float *P, const uint16_t *tokens, const uint16_t *targets,
                int nseq, float loss_scale, float *G) {
  model M;
  model_init(&M, c);
  size_t n = (size_t)M.m.total;
  memset(G, 0, n * sizeof(float));
  if (loss_scale <= 0.f) loss_scale = 256.f;
  double total = 0.0;
  for (int b = 0; b < nseq; b++)
    total += backward_one(&M, P, tokens + (size_t)b * c->seq, targets + (size_t)b * c->seq, loss_scale, G);
  /* flushPending (ane/engine.go:650-654): scale = 1/n / lossScale */
  float scale = (float)(1.0 / (double)nseq);
  scale /= loss_scale;
  for (size_t i = 0; i < n; i++) G[i] *= scale;
  model_free(&M);
  return nseq > 0 ? (float)(total / nseq) : 0.f;
}

/* ------------------------------------------------------------------ */
/* optimizer                                                           */
/* ------------------------------------------------------------------ */
/* adamBiasCorrectionInv (ane/train_full.go:1107-1111) */
static void bias_inv(int t, float b1, float b2, float *i1, float *i2) {
  float bc1 = (float)(1.0 - pow((double)b1, (double)t));
  float bc2 = (float)(1.0 - pow((double)b2, (double)t));
  *i1 = 1.f / bc1;
  *i2 = 1.f / bc2;
}
/* adamUpdateCFWithInv (ane/train_full.go:1113-1150) */
static void adam_seg(float *w, const float *g, float *m, float *v, size_t n, float lr, float b1, float b2,
                     float eps, float wd, float i1, float i2) {
  for (size_t i = 0; i < n; i++) {
    m[i] = b1 * m[i] + (1.f - b1) * g[i];
    v[i] = b2 * v[i] + (1.f - b2) * g[i] * g[i];
    float mh = m[i] * i1, vh = v[i] * i2;
    float upd = mh / ((float)sqrt((double)vh) + eps);
    if (wd != 0.f) upd += wd * w[i];
    w[i] -= lr * upd;
  }
}
static double sumsq(const float *g, size_t n) {
  double s = 0.0;
  for (size_t i = 0; i < n; i++) { double f = g[i]; s += f * f; }
  return s;
}

void orc_adam_update(const orc_cfg *c, float *P, float *G, float *Mm, float *Vv, int step, const orc_adam *h) {
  param_map m;
  build_map(c, &m);
  int64_t D = c->dim, H = c->hidden, V = c->vocab, NH = c->heads;
  int llama = c->arch == ORC_ARCH_LLAMA2;
  /* clipLayerGradients (ane/train_full.go:167-196): layer grads + embed */
  if (h->grad_clip > 0.f) {
    double n2 = 0.0;
    for (int l = 0; l < c->layers; l++) {
      layer_off *o = &m.L[l];
      n2 += sumsq(G + o->wq, D * D) + sumsq(G + o->wk, D * D) + sumsq(G + o->wv, D * D) +
            sumsq(G + o->wo, D * D) + sumsq(G + o->w1, H * D) + sumsq(G + o->w2, D * H);
      if (llama) n2 += sumsq(G + o->w3, H * D) + sumsq(G + o->g_att, D) + sumsq(G + o->g_ffn, D);
      if (o->ve_embed >= 0) n2 += sumsq(G + o->ve_embed, V * D) + sumsq(G + o->ve_gate, NH * VE_GATE_CH);
    }
    n2 += sumsq(G + m.embed, V * D);
    if (n2 > 0.0) {
      float norm = (float)sqrt(n2);
      if (norm > h->grad_clip) {
        float sc = h->grad_clip / norm;
        for (int l = 0; l < c->layers; l++) {
          layer_off *o = &m.L[l];
          int64_t lo = o->wq, hi = (l + 1 < c->layers) ? m.L[l + 1].wq : m.embed;
          for (int64_t i = lo; i < hi; i++) G[i] *= sc;
        }
        for (int64_t i = 0; i < V * D; i++) G[m.embed + i] *= sc;
      }
    }
  }
  float lr = h->lr, embed_lr = h->lr * h->embed_lr_mult, scalar_lr = h->lr * h->scalar_lr_mult;
  float lambda_lr = h->lr * h->scalar_lr_mult * h->lambda_lr_mult;
  float b1 = h->beta1, b2 = h->beta2, eps = h->eps, wd = h->weight_decay;
  float i1, i2, l1, l2;
  bias_inv(step, b1, b2, &i1, &i2);
  bias_inv(step, h->lambda_beta1, h->lambda_beta2, &l1, &l2);
#define ADAM(off, n, LR, WD) adam_seg(P + (off), G + (off), Mm + (off), Vv + (off), (size_t)(n), LR, b1, b2, eps, WD, i1, i2)
  /* applyLayerAdam (ane/train_full.go:1088-1100) */
  for (int l = 0; l < c->layers; l++) {
    layer_off *o = &m.L[l];
    ADAM(o->wq, D * D, lr, wd); ADAM(o->wk, D * D, lr, wd); ADAM(o->wv, D * D, lr, wd);
    ADAM(o->wo, D * D, lr, wd); ADAM(o->w1, H * D, lr, wd); ADAM(o->w2, D * H, lr, wd);
    if (llama) {
      ADAM(o->w3, H * D, lr, wd);
      ADAM(o->g_att, D, scalar_lr, 0.f); ADAM(o->g_ffn, D, scalar_lr, 0.f);
    }
    if (o->ve_embed >= 0) {
      ADAM(o->ve_embed, V * D, embed_lr, 0.f);
      ADAM(o->ve_gate, NH * VE_GATE_CH, scalar_lr, 0.f);
    }
  }
  /* model-level groups (ane/engine.go:659-673) */
  if (!llama) ADAM(m.smear_gate, D * D, lr, wd);
  ADAM(m.embed, V * D, embed_lr, 0.f);
  if (llama) {
    ADAM(m.g_final, D, scalar_lr, 0.f);
  } else {
    ADAM(m.smear_lambda, 1, scalar_lr, 0.f);
    ADAM(m.backout_lambda, 1, scalar_lr, 0.f);
    adam_seg(P + m.resid, G + m.resid, Mm + m.resid, Vv + m.resid, (size_t)c->layers, lambda_lr,
             h->lambda_beta1, h->lambda_beta2, eps, 0.f, l1, l2);
    adam_seg(P + m.x0l, G + m.x0l, Mm + m.x0l, Vv + m.x0l, (size_t)c->layers, lambda_lr,
             h->lambda_beta1, h->lambda_beta2, eps, 0.f, l1, l2);
  }
#undef ADAM
  free(m.L);
}

/* drand48 stream of the window sampler (ane/engine.go:177-181,873-880) */
uint64_t orc_drand48_seed(int64_t seed) { return (((uint64_t)seed & 0xffffffffULL) << 16) | 0x330EULL; }
double orc_drand48_next(uint64_t *st) {
  *st = (0x5DEECE66DULL * *st + 0xBULL) & ((1ULL << 48) - 1);
  return (double)*st / (double)(1ULL << 48);
}

/* Single ops the seam oracle (refseam.c) composes, at the reference's
 * channel-first signatures. */
void orc_linear_bwd_dx_cf(float *dx, const float *w, const float *dy, int out_ch, int in_ch, int seq) {
  linear_bwd_dx(dx, w, dy, out_ch, in_ch, seq);
}
void orc_rmsnorm_noweight_bwd_cf(float *dx, const float *dy, const float *x, int dim, int seq) {
  rmsnorm_noweight_bwd(dx, dy, x, dim, seq);
}
void orc_causal_attention_bwd_cf(float *dq, float *dk, float *dv, const float *dout, const float *q,
                                 const float *k, const float *v, int heads, int head_dim, int seq,
                                 float scale) {
  causal_attention_bwd(dq, dk, dv, dout, q, k, v, heads, head_dim, seq, scale);
}
void orc_matmul_vocab_seq(float *logits, const float *embed, const float *x, int vocab, int dim, int seq) {
  matmul_vocab_seq(logits, embed, x, vocab, dim, seq);
}
void orc_matmul_embedT(float *dx, const float *embed, const float *dlogits, int vocab, int dim, int seq) {
  matmul_embedT_scale(dx, embed, dlogits, vocab, dim, seq, 1.f);
}
void orc_softmax_row(float *out, const float *in, int n) { softmax_row(out, in, n); }
