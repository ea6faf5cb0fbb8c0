/*
 * refdecode.c -- CPU oracle for greedy KV-cache decoding (TEST
 * INFRASTRUCTURE ONLY; see refcpu.h).
 *
 * The reference has no decode path: it evaluates whole 256-token windows
 * (ane/engine.go:954-1038).  This oracle composes the reference's own
 * primitives, token by token, for the Llama2-style model with grouped-query
 * attention that the decode benchmark names:
 *   embedding lookup      stories.EmbedLookup      ane/stories/cpu.go:41-72
 *   RMSNorm with gain     stories.RMSNorm          ane/stories/cpu.go:97-111
 *   projections           linearCF                 ane/common.go:91-105
 *   RoPE tables / apply   buildRoPETables, applyRoPECFInPlace
 *                                                  ane/train_util.go:183-224
 *   attention             causalAttentionCF        ane/common.go:61-89
 *                         + softmaxRowAccel        ane/accel_stub.go:31-48
 *   tied classifier       stories.MatMulVocabSeq   ane/stories/cpu.go:303-327
 * plus SwiGLU (h1 * sigmoid(h1) * h3) and grouped-query attention (query
 * head h reads key/value head h / (heads / kv_heads)), which the reference
 * does not have.
 *
 * Position t attends to keys 0..t only: the reference's -65504 fill of
 * future scores gives them probability exactly 0 in its float64 softmax,
 * so the cached, causal evaluation here is the same function as one
 * full-window forward pass.  Greedy choice = first index of the maximum.
 */
#include "refcpu.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  size_t wq, wk, wv, wo, w1, w2, w3, g_att, g_ffn;
} dec_layer_off;

/* parameter order: per layer Wq[D*D] Wk[KVD*D] Wv[KVD*D] Wo[D*D] W1[H*D]
 * W2[D*H] W3[H*D] g_att[D] g_ffn[D]; then Embed[V*D] g_final[D] (the
 * LLAMA2 order of refcpu.h with key/value projections of KVD rows) */
static size_t dec_map(const orc_dec_cfg *c, dec_layer_off *L, size_t *embed, size_t *g_final) {
  size_t D = c->dim, H = c->hidden, KVD = (size_t)c->kv_heads * (c->dim / c->heads), off = 0;
  for (int l = 0; l < c->layers; l++) {
    dec_layer_off o;
    o.wq = off; off += D * D;
    o.wk = off; off += KVD * D;
    o.wv = off; off += KVD * D;
    o.wo = off; off += D * D;
    o.w1 = off; off += H * D;
    o.w2 = off; off += D * H;
    o.w3 = off; off += H * D;
    o.g_att = off; off += D;
    o.g_ffn = off; off += D;
    if (L) L[l] = o;
  }
  if (embed) *embed = off;
  off += (size_t)c->vocab * D;
  if (g_final) *g_final = off;
  off += D;
  return off;
}

size_t orc_dec_param_count(const orc_dec_cfg *c) { return dec_map(c, NULL, NULL, NULL); }

/* linearCF for one token: out[o] = sum_i W[o,i] * in[i], fp32, i ascending */
static void matvec(float *out, const float *w, const float *in, int oc, int ic) {
  for (int o = 0; o < oc; o++) {
    const float *row = w + (size_t)o * ic;
    float s = 0.f;
    for (int i = 0; i < ic; i++) s += row[i] * in[i];
    out[o] = s;
  }
}

/* stories.RMSNorm for one token (f64 statistics and scaling) */
static void rmsnorm_gain(float *out, const float *x, const float *g, int d) {
  double sum = 0.0;
  for (int i = 0; i < d; i++) sum += (double)x[i] * (double)x[i];
  double rrms = 1.0 / sqrt(sum / (double)d + 1e-5);
  for (int i = 0; i < d; i++) out[i] = (float)((double)x[i] * rrms * (double)g[i]);
}

/* applyRoPECFInPlace for one token at position pos (interleaved pairs) */
static void rope_token(float *x, int heads, int hd, const float *cs, const float *sn, int pos) {
  int half = hd / 2;
  for (int h = 0; h < heads; h++)
    for (int i = 0; i < half; i++) {
      float c = cs[pos * half + i], s = sn[pos * half + i];
      float *p = x + h * hd + 2 * i;
      float e = p[0], o = p[1];
      p[0] = e * c - o * s;
      p[1] = o * c + e * s;
    }
}

static float sigmoid32(float x) { return 1.0f / (1.0f + (float)exp((double)(-x))); }

typedef struct {
  const orc_dec_cfg *c;
  const float *P;
  const uint16_t *prefix, *forced;
  int nseq, plen, nsteps;
  uint16_t *tokens_out;
  float *logits_out;
  int next;                 /* next sequence to take (under mu) */
  pthread_mutex_t mu;
} dec_job;

static void decode_one(dec_job *J, int b) {
  const orc_dec_cfg *c = J->c;
  const float *P = J->P;
  const int D = c->dim, H = c->hidden, NH = c->heads, NKV = c->kv_heads, HD = D / NH, V = c->vocab;
  const int KVD = NKV * HD, G = NH / NKV, ctx = J->plen + J->nsteps;
  dec_layer_off *L = (dec_layer_off *)malloc(sizeof(dec_layer_off) * (size_t)c->layers);
  size_t embed, g_final;
  dec_map(c, L, &embed, &g_final);
  float *cs = (float *)malloc(sizeof(float) * (size_t)ctx * HD / 2);
  float *sn = (float *)malloc(sizeof(float) * (size_t)ctx * HD / 2);
  orc_build_rope(cs, sn, ctx, HD, c->rope_theta);
  float *kc = (float *)calloc((size_t)c->layers * ctx * KVD, sizeof(float));
  float *vc = (float *)calloc((size_t)c->layers * ctx * KVD, sizeof(float));
  float *x = (float *)malloc(sizeof(float) * D), *xn = (float *)malloc(sizeof(float) * D);
  float *q = (float *)malloc(sizeof(float) * D), *att = (float *)malloc(sizeof(float) * D);
  float *tmp = (float *)malloc(sizeof(float) * D);
  float *h1 = (float *)malloc(sizeof(float) * H), *h3 = (float *)malloc(sizeof(float) * H);
  float *sc = (float *)malloc(sizeof(float) * ctx), *pr = (float *)malloc(sizeof(float) * ctx);
  float *logits = (float *)malloc(sizeof(float) * V);
  const float scale = (float)(1.0 / sqrt((double)HD));
  uint16_t prev = 0;
  for (int t = 0; t < ctx; t++) {
    uint16_t tok;
    if (t < J->plen) tok = J->prefix[(size_t)b * J->plen + t];
    else tok = J->forced ? J->forced[(size_t)b * J->nsteps + (t - J->plen)] : prev;
    if (tok < V) memcpy(x, P + embed + (size_t)tok * D, sizeof(float) * D);
    else memset(x, 0, sizeof(float) * D);
    for (int l = 0; l < c->layers; l++) {
      const dec_layer_off *o = &L[l];
      float *kt = kc + ((size_t)l * ctx + t) * KVD, *vt = vc + ((size_t)l * ctx + t) * KVD;
      rmsnorm_gain(xn, x, P + o->g_att, D);
      matvec(q, P + o->wq, xn, D, D);
      matvec(kt, P + o->wk, xn, KVD, D);
      matvec(vt, P + o->wv, xn, KVD, D);
      rope_token(q, NH, HD, cs, sn, t);
      rope_token(kt, NKV, HD, cs, sn, t);
      for (int h = 0; h < NH; h++) {
        const int kh = h / G;
        float maxv = -INFINITY;
        for (int j = 0; j <= t; j++) {
          const float *kj = kc + ((size_t)l * ctx + j) * KVD + kh * HD;
          float s = 0.f;
          for (int i = 0; i < HD; i++) s += q[h * HD + i] * kj[i];
          sc[j] = s * scale;
          if (sc[j] > maxv) maxv = sc[j];
        }
        double sum = 0.0;
        for (int j = 0; j <= t; j++) {
          double e = exp((double)(sc[j] - maxv));
          pr[j] = (float)e;
          sum += e;
        }
        float inv = (float)(1.0 / sum);
        for (int j = 0; j <= t; j++) pr[j] *= inv;
        for (int i = 0; i < HD; i++) {
          float s = 0.f;
          for (int j = 0; j <= t; j++) s += pr[j] * vc[((size_t)l * ctx + j) * KVD + kh * HD + i];
          att[h * HD + i] = s;
        }
      }
      matvec(tmp, P + o->wo, att, D, D);
      for (int i = 0; i < D; i++) x[i] += tmp[i];
      rmsnorm_gain(xn, x, P + o->g_ffn, D);
      matvec(h1, P + o->w1, xn, H, D);
      matvec(h3, P + o->w3, xn, H, D);
      for (int i = 0; i < H; i++) h1[i] = h1[i] * sigmoid32(h1[i]) * h3[i];
      matvec(tmp, P + o->w2, h1, D, H);
      for (int i = 0; i < D; i++) x[i] += tmp[i];
    }
    if (t < J->plen - 1) continue;  /* no logits needed inside the prefix */
    rmsnorm_gain(xn, x, P + g_final, D);
    matvec(logits, P + embed, xn, V, D);
    int best = 0;
    for (int v = 1; v < V; v++)
      if (logits[v] > logits[best]) best = v;
    const int step = t - (J->plen - 1);  /* 0: after the prefix, i: after decode step i */
    J->tokens_out[(size_t)b * (J->nsteps + 1) + step] = (uint16_t)best;
    if (J->logits_out) memcpy(J->logits_out + ((size_t)b * (J->nsteps + 1) + step) * V, logits, sizeof(float) * V);
    prev = (uint16_t)best;
  }
  free(L); free(cs); free(sn); free(kc); free(vc); free(x); free(xn); free(q); free(att); free(tmp);
  free(h1); free(h3); free(sc); free(pr); free(logits);
}

static void *dec_worker(void *p) {
  dec_job *J = (dec_job *)p;
  for (;;) {
    pthread_mutex_lock(&J->mu);
    int b = J->next++;
    pthread_mutex_unlock(&J->mu);
    if (b >= J->nseq) return NULL;
    decode_one(J, b);
  }
}

void orc_decode(const orc_dec_cfg *c, const float *params, const uint16_t *prefix, int nseq, int plen,
                const uint16_t *forced, int nsteps, int threads, uint16_t *tokens_out, float *logits_out) {
  if (nseq <= 0 || plen <= 0 || nsteps < 0 || c->heads % c->kv_heads) return;
  dec_job J = {c, params, prefix, forced, nseq, plen, nsteps, tokens_out, logits_out, 0,
               PTHREAD_MUTEX_INITIALIZER};
  if (threads < 1) threads = 1;
  if (threads > nseq) threads = nseq;
  pthread_t th[64];
  if (threads > 64) threads = 64;
  for (int i = 1; i < threads; i++) pthread_create(&th[i], NULL, dec_worker, &J);
  dec_worker(&J);
  for (int i = 1; i < threads; i++) pthread_join(th[i], NULL);
}
