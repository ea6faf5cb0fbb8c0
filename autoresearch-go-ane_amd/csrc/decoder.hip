// ane_decoder: greedy KV-cache decoding with grouped-query attention (the
// C-ABI declared in include/ane_hip.h).  No counterpart in the reference;
// see decode.h for the model and the kernels.
//
// Device layout (one HIP device, one stream):
//   P        fp32 parameters (flat LLAMA2 order, Wk/Wv of kv_heads*64 rows)
//   wqkv     fp16 [L][D + 2*KVD][D]   Wq | Wk | Wv rows
//   wo       fp16 [L][D][D]
//   w13      fp16 [L][2H][D]          W1 / W3 interleaved by 32 rows
//   w2       fp16 [L][D][H]
//   embed_h  fp16 [V][D]              tied classifier
//   f*       the same five in MFMA-fragment-major order (decode.h)
//   kc, vc   fp16 [L][max_batch][kv_heads][max_ctx][64]
//   decode rows (64 each): x fp32 [64][D], xn/q/att fp16 [64][D],
//   gate fp16 [64][H], split-K partials, attention partials, argmax partials
//   prefill chunk (<= 8192 tokens): px fp32, pxn/pqkv/patt/pgate fp16
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <cmath>
#include <string>
#include <algorithm>
#include <vector>

#include "../../include/ane_hip.h"
#include "decode.h"
#include "gemm.h"
#include "rowops.h"

using namespace ane;

namespace {

struct DecLayerOff {
  int64_t wq, wk, wv, wo, w1, w2, w3, g_att, g_ffn;
};

int64_t dec_layout(const ane_decode_cfg& c, std::vector<DecLayerOff>* L, int64_t* embed, int64_t* g_final) {
  const int64_t D = c.dim, H = c.hidden, KVD = (int64_t)c.kv_heads * 64;
  int64_t off = 0;
  for (int l = 0; l < c.layers; l++) {
    DecLayerOff o;
    o.wq = off; off += D * D;
    o.wk = off; off += KVD * D;
    o.wv = off; off += KVD * D;
    o.wo = off; off += D * D;
    o.w1 = off; off += H * D;
    o.w2 = off; off += D * H;
    o.w3 = off; off += H * D;
    o.g_att = off; off += D;
    o.g_ffn = off; off += D;
    if (L) L->push_back(o);
  }
  if (embed) *embed = off;
  off += (int64_t)c.vocab * D;
  if (g_final) *g_final = off;
  off += D;
  return off;
}

constexpr int kPrefillTokens = 8192;

}  // namespace

struct ane_decoder {
  ane_decode_cfg cfg{};
  int D = 0, H = 0, NH = 0, NKV = 0, KVD = 0, N1 = 0, L = 0, V = 0, B = 0, C = 0;
  std::string err;
  hipStream_t stream = nullptr;
  std::vector<void*> allocs;
  std::vector<DecLayerOff> off;
  int64_t off_embed = 0, off_gfinal = 0, nparams = 0;
  bool params_set = false;
  float* P = nullptr;
  half_t *wqkv = nullptr, *wo = nullptr, *w13 = nullptr, *w2 = nullptr, *embed_h = nullptr;
  // the same weights in MFMA-fragment-major order for the 64-row decode GEMMs
  half_t *fwqkv = nullptr, *fwo = nullptr, *fw13 = nullptr, *fw2 = nullptr, *fembed = nullptr;
  half_t *kc = nullptr, *vc = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  float* x = nullptr;
  half_t *xn = nullptr, *att = nullptr, *gate = nullptr;
  half_t* att2 = nullptr;  // the fused chain's odd layers' attention output (the next chain reads the other)
  bool fuse_att = true;    // the next layer's attention inside each chain launch (ANE_DEC_FUSE_ATT=0: its own launch)
  float* apart = nullptr;
  float* kpart = nullptr;  // split-K partials of the decode-step GEMMs
  size_t kpart_cap = 0;
  int nsplit = 0;
  int attn_form = 0;  // decode attention form: 0 by batch size; ANE_DEC_ATTN=wide (1) / split (2)
  float2* amax = nullptr;
  float* logits_d = nullptr;
  // the per-layer GEMM chain as one launch (decode_tail.hip); ANE_DEC_TAIL=0
  // keeps one launch per GEMM and finish
  bool use_tail = false;
  half_t *xg_att = nullptr, *xg_ffn = nullptr;  // fp16(x * gain) fragments
  float* rr_d = nullptr;                        // [64] 1 / rms of the current norm input
  float *ssq_wo = nullptr, *ssq_w2 = nullptr;
  unsigned* sync = nullptr;
  int* err_d = nullptr;
  int b_tail = 0;
  unsigned tail_spin = 0;
  bool tail_poll = false;      // the data-polling form of the chain (default; ANE_DEC_TAIL=1: done counters)
  char* tail_sets = nullptr;   // its two buffer sets, tail_set_bytes each
  size_t tail_set_sz = 0;
  uint16_t *tok_d = nullptr, *hist_d = nullptr, *prefix_d = nullptr;
  uint16_t* tok_save = nullptr;  // a call's input tokens, kept to redo it after a failed chain wait
  int chain_latched = 0;         // 1 once a failed chain wait switched the decoder to one launch per GEMM
  int* ctr_d = nullptr;
  int TC = 0;
  float* px = nullptr;
  half_t *pxn = nullptr, *pqkv = nullptr, *patt = nullptr, *pgate = nullptr;
  int nseq = 0, pos = 0;  // active batch, filled positions
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  int graph_nseq = 0;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double last_ms = 0.0;
};

namespace {

int dfail(ane_decoder* d, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (d) d->err = buf;
  return code;
}

#define DCHK(op, expr)                                                                                   \
  do {                                                                                                   \
    hipError_t _h = (expr);                                                                              \
    if (_h != hipSuccess)                                                                                \
      return dfail(d, ANE_ERR_HIP, "storiesane decode %s: %s: %s", op, #expr, hipGetErrorString(_h));    \
  } while (0)

template <typename T>
hipError_t dalloc(ane_decoder* d, T** p, size_t n) {
  void* q = nullptr;
  hipError_t e = hipMalloc(&q, n * sizeof(T) > 0 ? n * sizeof(T) : 16);
  if (e != hipSuccess) return e;
  d->allocs.push_back(q);
  *p = (T*)q;
  return hipSuccess;
}

void free_all(ane_decoder* d) {
  (void)hipSetDevice(d->cfg.device);
  if (d->stream) (void)hipStreamSynchronize(d->stream);
  if (d->gexec) (void)hipGraphExecDestroy(d->gexec);
  if (d->graph) (void)hipGraphDestroy(d->graph);
  d->gexec = nullptr;
  d->graph = nullptr;
  for (void* p : d->allocs) (void)hipFree(p);
  d->allocs.clear();
  if (d->ev0) (void)hipEventDestroy(d->ev0);
  if (d->ev1) (void)hipEventDestroy(d->ev1);
  d->ev0 = d->ev1 = nullptr;
  if (d->stream) (void)hipStreamDestroy(d->stream);
  d->stream = nullptr;
}

int validate(const ane_decode_cfg& c, std::string* why) {
  char buf[256];
  buf[0] = 0;
  if (c.heads <= 0 || c.kv_heads <= 0 || c.dim != 64 * c.heads)
    snprintf(buf, sizeof buf, "dim=%d must be 64 * heads (heads=%d)", c.dim, c.heads);
  else if (c.heads % c.kv_heads || c.heads / c.kv_heads > 4)
    snprintf(buf, sizeof buf, "heads=%d must be 1..4 times kv_heads=%d", c.heads, c.kv_heads);
  else if (c.dim > 1024)
    snprintf(buf, sizeof buf, "dim=%d exceeds 1024", c.dim);
  else if (c.hidden <= 0 || c.hidden % 64 || c.hidden > 2048)
    snprintf(buf, sizeof buf, "hidden=%d must be a multiple of 64 up to 2048", c.hidden);
  else if (c.vocab <= 0 || c.vocab % 32 || c.vocab > 65536)
    snprintf(buf, sizeof buf, "vocab=%d must be a multiple of 32 up to 65536", c.vocab);
  else if (c.layers <= 0)
    snprintf(buf, sizeof buf, "layers=%d", c.layers);
  else if (c.max_batch < 1 || c.max_batch > kDecRows)
    snprintf(buf, sizeof buf, "max_batch=%d must be 1..%d", c.max_batch, kDecRows);
  else if (c.max_ctx < 64 || c.max_ctx > 65536)
    snprintf(buf, sizeof buf, "max_ctx=%d must be 64..65536", c.max_ctx);
  if (buf[0]) {
    *why = buf;
    return ANE_ERR_ARG;
  }
  return ANE_OK;
}

int open_impl(ane_decoder* d) {
  const char* op = "open";
  const ane_decode_cfg& c = d->cfg;
  d->D = c.dim; d->H = c.hidden; d->NH = c.heads; d->NKV = c.kv_heads; d->KVD = c.kv_heads * 64;
  d->N1 = d->D + 2 * d->KVD; d->L = c.layers; d->V = c.vocab; d->B = c.max_batch; d->C = c.max_ctx;
  const int D = d->D, H = d->H, N1 = d->N1, L = d->L, V = d->V, B = d->B, C = d->C;
  d->nparams = dec_layout(c, &d->off, &d->off_embed, &d->off_gfinal);
  DCHK(op, hipSetDevice(c.device));
  DCHK(op, hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
  DCHK(op, hipEventCreate(&d->ev0));
  DCHK(op, hipEventCreate(&d->ev1));
  DCHK(op, dalloc(d, &d->P, (size_t)d->nparams));
  DCHK(op, dalloc(d, &d->wqkv, (size_t)L * N1 * D));
  DCHK(op, dalloc(d, &d->wo, (size_t)L * D * D));
  DCHK(op, dalloc(d, &d->w13, (size_t)L * 2 * H * D));
  DCHK(op, dalloc(d, &d->w2, (size_t)L * D * H));
  DCHK(op, dalloc(d, &d->embed_h, (size_t)V * D));
  DCHK(op, dalloc(d, &d->fwqkv, (size_t)L * N1 * D));
  DCHK(op, dalloc(d, &d->fwo, (size_t)L * D * D));
  DCHK(op, dalloc(d, &d->fw13, (size_t)L * 2 * H * D));
  DCHK(op, dalloc(d, &d->fw2, (size_t)L * D * H));
  DCHK(op, dalloc(d, &d->fembed, (size_t)V * D));
  const size_t cache = (size_t)L * B * d->NKV * C * 64;
  DCHK(op, dalloc(d, &d->kc, cache));
  DCHK(op, dalloc(d, &d->vc, cache));
  // RoPE tables (buildRoPETables, ane/train_util.go:183-202: f64 angle, fp32 cos/sin)
  {
    std::vector<float> cs((size_t)C * 32), sn((size_t)C * 32);
    for (int p = 0; p < C; p++)
      for (int i = 0; i < 32; i++) {
        const double f = (double)p / std::pow(c.rope_theta, (double)(2 * i) / 64.0);
        cs[(size_t)p * 32 + i] = (float)std::cos(f);
        sn[(size_t)p * 32 + i] = (float)std::sin(f);
      }
    DCHK(op, dalloc(d, &d->rope_cos, cs.size()));
    DCHK(op, dalloc(d, &d->rope_sin, sn.size()));
    DCHK(op, hipMemcpy(d->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    DCHK(op, hipMemcpy(d->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  }
  const int R = kDecRows;
  DCHK(op, dalloc(d, &d->x, (size_t)R * D));
  DCHK(op, dalloc(d, &d->xn, (size_t)R * D));
  DCHK(op, dalloc(d, &d->att, (size_t)R * D));
  DCHK(op, dalloc(d, &d->gate, (size_t)R * H));
  d->nsplit = (C + kDecChunk - 1) / kDecChunk;
  if (const char* f = getenv("ANE_DEC_ATTN")) d->attn_form = !strcmp(f, "wide") ? 1 : !strcmp(f, "split") ? 2 : 0;
  DCHK(op, dalloc(d, &d->apart, (size_t)B * d->NH * d->nsplit * 66));
  {
    const int NK[4][2] = {{N1, D}, {D, D}, {2 * H, D}, {D, H}};  // QKV, Wo, W1|W3, W2
    size_t cap = 0;
    for (const auto& nk : NK) {
      const int ks = skinny_splits(nk[0], nk[1]);
      if (ks <= 0) return dfail(d, ANE_ERR_ARG, "storiesane decode open: K=%d too long for the split-K GEMMs", nk[1]);
      cap = std::max(cap, (size_t)ks * kDecRows * nk[0]);
    }
    d->kpart_cap = cap;
    DCHK(op, dalloc(d, &d->kpart, cap));
  }
  DCHK(op, dalloc(d, &d->amax, (size_t)(V / 32) * R));
  DCHK(op, dalloc(d, &d->logits_d, (size_t)R * V));
  DCHK(op, dalloc(d, &d->tok_d, (size_t)R));
  DCHK(op, dalloc(d, &d->hist_d, (size_t)C * R));
  DCHK(op, dalloc(d, &d->prefix_d, (size_t)B * C));
  DCHK(op, dalloc(d, &d->tok_save, (size_t)R));
  DCHK(op, dalloc(d, &d->ctr_d, 3));
  d->TC = std::max(kPrefillTokens, (C + 63) / 64 * 64);
  DCHK(op, dalloc(d, &d->px, (size_t)d->TC * D));
  DCHK(op, dalloc(d, &d->pxn, (size_t)d->TC * D));
  DCHK(op, dalloc(d, &d->pqkv, (size_t)d->TC * N1));
  DCHK(op, dalloc(d, &d->patt, (size_t)d->TC * D));
  DCHK(op, dalloc(d, &d->pgate, (size_t)d->TC * H));
  // rows beyond the active batch feed the 64-row GEMMs: keep them finite
  DCHK(op, hipMemset(d->xn, 0, (size_t)R * D * 2));
  DCHK(op, hipMemset(d->att, 0, (size_t)R * D * 2));
  DCHK(op, hipMemset(d->gate, 0, (size_t)R * H * 2));
  DCHK(op, hipMemset(d->x, 0, (size_t)R * D * 4));
  DCHK(op, hipMemset(d->tok_d, 0, (size_t)R * 2));
  DCHK(op, hipMemset(d->ctr_d, 0, 12));
  // The fused GEMM chain: one block per column group of each phase, all
  // resident at once, or the chain keeps one launch per GEMM.
  {
    d->b_tail = D / 32 + H / 32 + D / 32 + N1 / 32 + 1;
    int ncu = 0;
    DCHK(op, hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, c.device));
    const int per_cu = dec_tail_blocks_per_cu();
    d->use_tail = per_cu > 0 && (long)per_cu * ncu >= d->b_tail;
    // ANE_DEC_TAIL: 0 one launch per GEMM; 1 the chain with done counters;
    // 2 (default) the chain whose consumers poll the data itself
    int tail_form = 2;
    if (const char* f = getenv("ANE_DEC_TAIL")) tail_form = atoi(f);
    d->use_tail = d->use_tail && tail_form != 0;
    d->tail_poll = tail_form != 1;
    if (const char* f = getenv("ANE_DEC_FUSE_ATT")) d->fuse_att = atoi(f) != 0;
    // ANE_DEC_TAIL_SPIN: polls before a dependency wait times out (0: every
    // wait fails at once; for tests of the timeout path)
    d->tail_spin = kDecTailSpin;
    if (const char* f = getenv("ANE_DEC_TAIL_SPIN")) d->tail_spin = (unsigned)strtoul(f, nullptr, 10);
    if (d->use_tail) {
      DCHK(op, dalloc(d, &d->xg_att, (size_t)R * D));
      DCHK(op, dalloc(d, &d->xg_ffn, (size_t)R * D));
      DCHK(op, dalloc(d, &d->rr_d, (size_t)R));
      DCHK(op, dalloc(d, &d->ssq_wo, (size_t)(D / 32) * R));
      DCHK(op, dalloc(d, &d->ssq_w2, (size_t)(D / 32) * R));
      DCHK(op, dalloc(d, &d->sync, (size_t)kDecTailSync));
      DCHK(op, dalloc(d, &d->err_d, 1));
      DCHK(op, hipMemset(d->xg_att, 0, (size_t)R * D * 2));
      DCHK(op, hipMemset(d->xg_ffn, 0, (size_t)R * D * 2));
      DCHK(op, hipMemset(d->rr_d, 0, (size_t)R * 4));
      DCHK(op, hipMemset(d->sync, 0, (size_t)kDecTailSync * 4));
      DCHK(op, hipMemset(d->err_d, 0, 4));
      if (d->tail_poll) {
        d->tail_set_sz = (tail_set_bytes(D, H, N1) + 255) & ~(size_t)255;
        DCHK(op, dalloc(d, &d->tail_sets, 2 * d->tail_set_sz));
        DCHK(op, hipMemset(d->tail_sets, 0xff, 2 * d->tail_set_sz));  // every dword kTailStale
        DCHK(op, dalloc(d, &d->att2, (size_t)R * D));
        DCHK(op, hipMemset(d->att2, 0, (size_t)R * D * 2));
      }
    }
  }
  DCHK(op, hipDeviceSynchronize());
  return ANE_OK;
}

hipError_t gemm(ane_decoder* d, const half_t* A, const half_t* Bw, int M, int N, int K, int epi, const EpiParams& p) {
  GemmArgs g;
  g.A = A; g.B = Bw; g.lda = K; g.ldb = K; g.M = M; g.N = N; g.K = K; g.a_t = false; g.b_t = false;
  return gemm_run(g, epi, p, d->stream);
}

// One decode step for the active batch; every position/step index is read
// from ctr_d on the device, so the same launches replay as a graph.
int enqueue_step_tail(ane_decoder* d, float* logits, uint16_t* hist);
int generate_run(ane_decoder* d, const char* op, int nsteps, uint16_t* out_tok);

int enqueue_step(ane_decoder* d, float* logits, uint16_t* hist) {
  if (d->use_tail) return enqueue_step_tail(d, logits, hist);
  const char* op = "step";
  const int D = d->D, H = d->H, N1 = d->N1, nb = d->nseq;
  const hipStream_t st = d->stream;
  DCHK(op, dec_embed_norm(d->x, d->xn, d->P + d->off_embed, d->tok_d, d->P + d->off[0].g_att, nb, D, d->V, st));
  for (int l = 0; l < d->L; l++) {
    const DecLayerOff& o = d->off[l];
    half_t* kcl = d->kc + (size_t)l * d->B * d->NKV * d->C * 64;
    half_t* vcl = d->vc + (size_t)l * d->B * d->NKV * d->C * 64;
    // each GEMM: split-K partials from (N/32) x ks one-wave blocks, then a
    // per-row finish that sums the splits and applies the epilogue (the QKV
    // partials are finished by the attention kernel)
    DCHK(op, skinny_partials(d->xn, d->fwqkv + (size_t)l * N1 * D, d->kpart, d->kpart_cap, N1, D, st));
    DecAttnArgs aa;
    aa.qkv_part = d->kpart; aa.qkv_ks = skinny_splits(N1, D); aa.rope_cos = d->rope_cos; aa.rope_sin = d->rope_sin;
    aa.kc = kcl; aa.vc = vcl; aa.ctr = d->ctr_d; aa.part = d->apart; aa.att = d->att; aa.nb = nb;
    aa.NH = d->NH; aa.NKV = d->NKV; aa.max_ctx = d->C; aa.nsplit = d->nsplit; aa.scale = 0.125f;
    aa.form = d->attn_form;
    DCHK(op, dec_attention(aa, st));
    DCHK(op, skinny_partials(d->att, d->fwo + (size_t)l * D * D, d->kpart, d->kpart_cap, D, D, st));
    DCHK(op, skinny_finish_resid_norm(d->kpart, D, D, d->x, d->xn, d->P + o.g_ffn, nb, st));
    DCHK(op, skinny_partials(d->xn, d->fw13 + (size_t)l * 2 * H * D, d->kpart, d->kpart_cap, 2 * H, D, st));
    DCHK(op, skinny_finish_swiglu(d->kpart, 2 * H, D, d->gate, nb, st));
    DCHK(op, skinny_partials(d->gate, d->fw2 + (size_t)l * D * H, d->kpart, d->kpart_cap, D, H, st));
    const float* gnext = l + 1 < d->L ? d->P + d->off[l + 1].g_att : d->P + d->off_gfinal;
    DCHK(op, skinny_finish_resid_norm(d->kpart, D, H, d->x, d->xn, gnext, nb, st));
  }
  SkinnyArgs s;
  memset(&s, 0, sizeof s);
  s.nb = nb;
  s.X = d->xn; s.W = d->fembed; s.N = d->V; s.K = D; s.amax = d->amax;
  s.logits = logits; s.nvalid = d->V;
  DCHK(op, classifier_argmax(s, st));
  DCHK(op, argmax_reduce(d->tok_d, hist, d->ctr_d + 1, d->amax, d->V / 32, nb, st));
  DCHK(op, dec_advance(d->ctr_d, st));
  return ANE_OK;
}

// The same step with each layer's GEMM chain fused into one launch
// (decode_tail.hip): per layer the attention kernel, then the tail kernel
// (Wo, W1|W3, W2 and the next layer's QKV partials).  Norm inputs are
// fp16(x * gain) with the 1 / rms applied to the GEMM outputs.
int enqueue_step_tail(ane_decoder* d, float* logits, uint16_t* hist) {
  const char* op = "step";
  const int D = d->D, H = d->H, N1 = d->N1, nb = d->nseq, L = d->L;
  const hipStream_t st = d->stream;
  DCHK(op, dec_row_xg(d->x, d->xg_att, d->rr_d, d->P + d->off_embed, d->tok_d, d->P + d->off[0].g_att, nb, D, d->V,
                      st));
  DCHK(op, skinny_partials(d->xg_att, d->fwqkv, d->kpart, d->kpart_cap, N1, D, st));
  auto attn_args = [&](int l, half_t* out) {
    DecAttnArgs aa;
    aa.qkv_part = d->kpart; aa.qkv_ks = l == 0 ? skinny_splits(N1, D) : 1; aa.rr = d->rr_d;
    aa.rope_cos = d->rope_cos; aa.rope_sin = d->rope_sin;
    aa.kc = d->kc + (size_t)l * d->B * d->NKV * d->C * 64;
    aa.vc = d->vc + (size_t)l * d->B * d->NKV * d->C * 64;
    aa.ctr = d->ctr_d; aa.part = d->apart; aa.att = out; aa.nb = nb;
    aa.NH = d->NH; aa.NKV = d->NKV; aa.max_ctx = d->C; aa.nsplit = d->nsplit; aa.scale = 0.125f;
    aa.form = d->attn_form;
    return aa;
  };
  // With the data-polling chain, the next layer's attention (wide form, one
  // split) runs inside each chain launch; its output alternates between att
  // and att2 so that a launch never writes what its own Wo blocks read.
  const bool fuse = d->tail_poll && d->fuse_att && d->att2 && dec_attention_fusable(attn_args(1 < L ? 1 : 0, d->att));
  auto att_of = [&](int l) { return fuse && (l & 1) ? d->att2 : d->att; };
  DCHK(op, dec_attention(attn_args(0, att_of(0)), st));
  for (int l = 0; l < L; l++) {
    const DecLayerOff& o = d->off[l];
    const bool last = l + 1 == L;
    TailArgs t;
    t.att = att_of(l); t.x = d->x;
    t.wo = d->fwo + (size_t)l * D * D; t.w13 = d->fw13 + (size_t)l * 2 * H * D; t.w2 = d->fw2 + (size_t)l * D * H;
    t.wqkv_next = last ? nullptr : d->fwqkv + (size_t)(l + 1) * N1 * D;
    t.g_ffn = d->P + o.g_ffn;
    t.g_next = last ? d->P + d->off_gfinal : d->P + d->off[l + 1].g_att;
    t.xg_ffn = d->xg_ffn; t.gate = d->gate; t.xg_next = d->xg_att; t.rr_next = d->rr_d;
    t.p_q = d->kpart;
    t.ssq_wo = d->ssq_wo; t.ssq_w2 = d->ssq_w2; t.sync = d->sync; t.gstep = d->ctr_d + 2; t.err = d->err_d;
    t.spin_limit = d->tail_spin;
    t.D = D; t.H = H; t.N1 = N1; t.layer = l; t.L = L;
    t.b_wo = D / 32; t.b_13 = H / 32; t.b_w2 = D / 32; t.b_q = last ? 0 : N1 / 32;
    t.poll = d->tail_poll ? 1 : 0;
    t.sets[0] = d->tail_sets;
    t.sets[1] = d->tail_poll ? d->tail_sets + d->tail_set_sz : nullptr;
    if (fuse && !last) {
      t.att_next = attn_args(l + 1, att_of(l + 1));
      t.att_next.nsplit = 1;
      t.b_att = nb * d->NKV;
    }
    DCHK(op, dec_tail(t, st));
    if (!fuse && !last) DCHK(op, dec_attention(attn_args(l + 1, d->att), st));
  }
  SkinnyArgs s;
  memset(&s, 0, sizeof s);
  s.nb = nb;
  s.X = d->xg_att; s.W = d->fembed; s.N = d->V; s.K = D; s.amax = d->amax;
  s.logits = logits; s.nvalid = d->V; s.rr = d->rr_d;
  DCHK(op, classifier_argmax(s, st));
  DCHK(op, argmax_reduce(d->tok_d, hist, d->ctr_d + 1, d->amax, d->V / 32, nb, st));
  DCHK(op, dec_advance(d->ctr_d, st));
  return ANE_OK;
}

// After a synchronised call: a dependency wait of the fused chain that timed
// out leaves *err set (every later launch of the chain exits at once, the
// other kernels of the step still run on what it left).  Clears the chain's
// state (epoch counters, buffer sets, error flag) and reports the failure in
// *failed; the call's outputs and the cache rows it wrote are then invalid.
int tail_failed(ane_decoder* d, const char* op, bool* failed) {
  *failed = false;
  if (!d->use_tail) return ANE_OK;
  int err = 0;
  DCHK(op, hipMemcpy(&err, d->err_d, 4, hipMemcpyDeviceToHost));
  if (!err) return ANE_OK;
  DCHK(op, hipMemset(d->sync, 0, (size_t)kDecTailSync * 4));
  DCHK(op, hipMemset(d->ctr_d + 2, 0, 4));
  DCHK(op, hipMemset(d->err_d, 0, 4));
  if (d->tail_poll) DCHK(op, hipMemset(d->tail_sets, 0xff, 2 * d->tail_set_sz));  // a failed launch left sets half-used
  DCHK(op, hipDeviceSynchronize());
  *failed = true;
  return ANE_OK;
}

// A failed chain wait means the chain's two assumptions did not hold on this
// GPU (all of a launch's chain blocks resident at once, and dispatched before
// its attention blocks: another process on the GPU can break both).  As the
// reference disables a failing accelerator piece and carries on with its
// other path (ane/engine.go:887-894, ane/train_full.go:356-368), the decoder
// switches for good to one launch per GEMM, which has no inter-block waits,
// and the caller redoes the call from its saved start.
void latch_per_gemm(ane_decoder* d) {
  d->use_tail = false;
  d->chain_latched = 1;
  if (d->gexec) (void)hipGraphExecDestroy(d->gexec);
  if (d->graph) (void)hipGraphDestroy(d->graph);
  d->gexec = nullptr;
  d->graph = nullptr;
}

// The start of a step / generate call, kept so that the call can be redone:
// the input tokens (the device copy the first step reads) and the position.
int save_start(ane_decoder* d, const char* op) {
  DCHK(op, hipMemcpyAsync(d->tok_save, d->tok_d, (size_t)d->nseq * 2, hipMemcpyDeviceToDevice, d->stream));
  return ANE_OK;
}

// Rewinds to a saved start: the tokens and the device counters of position
// pos0 (cache rows from pos0 on are rewritten by the redo before any read).
int restore_start(ane_decoder* d, const char* op, int pos0) {
  DCHK(op, hipMemcpyAsync(d->tok_d, d->tok_save, (size_t)d->nseq * 2, hipMemcpyDeviceToDevice, d->stream));
  DCHK(op, dec_set_ctr(d->ctr_d, pos0, 0, d->stream));
  return ANE_OK;
}

int copy_out(ane_decoder* d, uint16_t* next_tok, float* logits) {
  const char* op = "copy out";
  if (next_tok) DCHK(op, hipMemcpyAsync(next_tok, d->tok_d, (size_t)d->nseq * 2, hipMemcpyDeviceToHost, d->stream));
  if (logits)
    DCHK(op, hipMemcpyAsync(logits, d->logits_d, (size_t)d->nseq * d->V * 4, hipMemcpyDeviceToHost, d->stream));
  DCHK(op, hipStreamSynchronize(d->stream));
  return ANE_OK;
}

// A failure that the redo cannot repair leaves the cache inconsistent: the
// active batch is dropped so that Step / Generate refuse until a new Prefill.
int drop_batch(ane_decoder* d, int rc) {
  d->nseq = 0;
  return rc;
}

}  // namespace

extern "C" int64_t ane_decode_param_count(const ane_decode_cfg* cfg) {
  if (!cfg) return -1;
  return dec_layout(*cfg, nullptr, nullptr, nullptr);
}

extern "C" int ane_decode_open(const ane_decode_cfg* cfg, ane_decoder** out) {
  if (!out) return ANE_ERR_ARG;
  *out = nullptr;
  ane_decoder* d = new ane_decoder();
  *out = d;
  if (!cfg) return dfail(d, ANE_ERR_ARG, "storiesane decode open: no config");
  d->cfg = *cfg;
  std::string why;
  if (validate(*cfg, &why) != ANE_OK) return dfail(d, ANE_ERR_ARG, "storiesane decode open: %s", why.c_str());
  int rc = open_impl(d);
  if (rc != ANE_OK) free_all(d);
  return rc;
}

extern "C" void ane_decode_destroy(ane_decoder* d) {
  if (!d) return;
  free_all(d);
  delete d;
}

extern "C" const char* ane_decode_last_error(ane_decoder* d) { return d ? d->err.c_str() : "no decoder"; }

extern "C" int ane_decode_set_params(ane_decoder* d, const float* params, int64_t n) {
  const char* op = "set params";
  if (!d || !d->stream) return ANE_ERR_STATE;
  if (!params || n != d->nparams)
    return dfail(d, ANE_ERR_ARG, "storiesane decode set params: len=%lld want=%lld", (long long)n,
                 (long long)d->nparams);
  const int D = d->D, H = d->H, KVD = d->KVD, N1 = d->N1;
  const hipStream_t st = d->stream;
  DCHK(op, hipSetDevice(d->cfg.device));
  DCHK(op, hipMemcpyAsync(d->P, params, (size_t)n * 4, hipMemcpyHostToDevice, st));
  for (int l = 0; l < d->L; l++) {
    const DecLayerOff& o = d->off[l];
    half_t* q = d->wqkv + (size_t)l * N1 * D;
    DCHK(op, f32_to_f16(q, d->P + o.wq, (size_t)D * D, st));
    DCHK(op, f32_to_f16(q + (size_t)D * D, d->P + o.wk, (size_t)KVD * D, st));
    DCHK(op, f32_to_f16(q + (size_t)(D + KVD) * D, d->P + o.wv, (size_t)KVD * D, st));
    DCHK(op, f32_to_f16(d->wo + (size_t)l * D * D, d->P + o.wo, (size_t)D * D, st));
    DCHK(op, interleave_w13(d->w13 + (size_t)l * 2 * H * D, d->P + o.w1, d->P + o.w3, H, D, st));
    DCHK(op, f32_to_f16(d->w2 + (size_t)l * D * H, d->P + o.w2, (size_t)D * H, st));
  }
  DCHK(op, f32_to_f16(d->embed_h, d->P + d->off_embed, (size_t)d->V * D, st));
  for (int l = 0; l < d->L; l++) {
    DCHK(op, weight_to_frag(d->fwqkv + (size_t)l * N1 * D, d->wqkv + (size_t)l * N1 * D, N1, D, st));
    DCHK(op, weight_to_frag(d->fwo + (size_t)l * D * D, d->wo + (size_t)l * D * D, D, D, st));
    DCHK(op, weight_to_frag(d->fw13 + (size_t)l * 2 * H * D, d->w13 + (size_t)l * 2 * H * D, 2 * H, D, st));
    DCHK(op, weight_to_frag(d->fw2 + (size_t)l * D * H, d->w2 + (size_t)l * D * H, D, H, st));
  }
  DCHK(op, weight_to_frag(d->fembed, d->embed_h, d->V, D, st));
  DCHK(op, hipStreamSynchronize(st));
  d->params_set = true;
  return ANE_OK;
}

extern "C" int ane_decode_prefill(ane_decoder* d, const uint16_t* prefix, int32_t nseq, int32_t plen,
                                  uint16_t* next_tok, float* logits) {
  const char* op = "prefill";
  if (!d || !d->stream) return ANE_ERR_STATE;
  if (!d->params_set) return dfail(d, ANE_ERR_STATE, "storiesane decode prefill: parameters not set");
  if (!prefix || nseq < 1 || nseq > d->B)
    return dfail(d, ANE_ERR_ARG, "storiesane decode prefill: nseq=%d want 1..%d", nseq, d->B);
  if (plen < 64 || plen % 64 || plen >= d->C)
    return dfail(d, ANE_ERR_ARG, "storiesane decode prefill: plen=%d must be a multiple of 64 below max_ctx=%d",
                 plen, d->C);
  const int D = d->D, H = d->H, N1 = d->N1;
  const hipStream_t st = d->stream;
  DCHK(op, hipSetDevice(d->cfg.device));
  DCHK(op, hipMemcpyAsync(d->prefix_d, prefix, (size_t)nseq * plen * 2, hipMemcpyHostToDevice, st));
  const int per = std::max(1, d->TC / plen);
  for (int s0 = 0; s0 < nseq; s0 += per) {
    const int n = std::min(per, nseq - s0), T = n * plen;
    DCHK(op, embed_lookup(d->px, d->P + d->off_embed, d->prefix_d + (size_t)s0 * plen, T, D, d->V, st));
    for (int l = 0; l < d->L; l++) {
      const DecLayerOff& o = d->off[l];
      half_t* kcl = d->kc + (size_t)l * d->B * d->NKV * d->C * 64;
      half_t* vcl = d->vc + (size_t)l * d->B * d->NKV * d->C * 64;
      DCHK(op, rmsnorm_f16(d->pxn, d->px, nullptr, nullptr, d->P + o.g_att, T, D, st));
      {
        EpiParams p;
        p.C = d->pqkv; p.ldc = N1;
        DCHK(op, gemm(d, d->pxn, d->wqkv + (size_t)l * N1 * D, T, N1, D, EPI_STORE_H, p));
      }
      DCHK(op, prefill_kv_write(d->pqkv, kcl, vcl, d->rope_cos, d->rope_sin, s0, n, plen, d->NH, d->NKV, d->C, st));
      {
        PrefillAttnArgs a;
        a.qkv = d->pqkv; a.ldq = N1; a.kc = kcl; a.vc = vcl; a.out = d->patt; a.seq0 = s0; a.nseq = n; a.S = plen;
        a.NH = d->NH; a.NKV = d->NKV; a.max_ctx = d->C; a.scale = 0.125f;
        DCHK(op, prefill_attention(a, st));
      }
      {
        EpiParams p;
        p.C = d->px; p.ldc = D; p.R = d->px;
        DCHK(op, gemm(d, d->patt, d->wo + (size_t)l * D * D, T, D, D, EPI_RESID, p));
      }
      DCHK(op, rmsnorm_f16(d->pxn, d->px, nullptr, nullptr, d->P + o.g_ffn, T, D, st));
      {
        EpiParams p;
        p.C = d->pgate; p.ldc = H;
        DCHK(op, gemm(d, d->pxn, d->w13 + (size_t)l * 2 * H * D, T, 2 * H, D, EPI_SWIGLU, p));
      }
      {
        EpiParams p;
        p.C = d->px; p.ldc = D; p.R = d->px;
        DCHK(op, gemm(d, d->pgate, d->w2 + (size_t)l * D * H, T, D, H, EPI_RESID, p));
      }
    }
    DCHK(op, gather_last_rows(d->x + (size_t)s0 * D, d->px, n, plen, D, st));
  }
  d->nseq = nseq;
  DCHK(op, dec_norm(d->x, d->xn, d->P + d->off_gfinal, nseq, D, st));
  SkinnyArgs s;
  memset(&s, 0, sizeof s);
  s.nb = nseq;
  s.X = d->xn; s.W = d->fembed; s.N = d->V; s.K = D; s.amax = d->amax;
  s.logits = logits ? d->logits_d : nullptr; s.nvalid = d->V;
  DCHK(op, classifier_argmax(s, st));
  DCHK(op, argmax_reduce(d->tok_d, nullptr, nullptr, d->amax, d->V / 32, nseq, st));
  DCHK(op, dec_set_ctr(d->ctr_d, plen, 0, st));
  d->pos = plen;
  return copy_out(d, next_tok, logits);  // prefill launches no chain kernel: nothing to check
}

extern "C" int ane_decode_step(ane_decoder* d, const uint16_t* in_tok, uint16_t* next_tok, float* logits) {
  const char* op = "step";
  if (!d || !d->stream) return ANE_ERR_STATE;
  if (d->nseq == 0) return dfail(d, ANE_ERR_STATE, "storiesane decode step: no prefill");
  if (d->pos >= d->C) return dfail(d, ANE_ERR_ARG, "storiesane decode step: cache full (max_ctx=%d)", d->C);
  DCHK(op, hipSetDevice(d->cfg.device));
  if (in_tok) DCHK(op, hipMemcpyAsync(d->tok_d, in_tok, (size_t)d->nseq * 2, hipMemcpyHostToDevice, d->stream));
  const int pos0 = d->pos;
  int rc = d->use_tail ? save_start(d, op) : ANE_OK;
  if (rc == ANE_OK) rc = enqueue_step(d, logits ? d->logits_d : nullptr, nullptr);
  if (rc == ANE_OK) rc = copy_out(d, next_tok, logits);
  bool failed = false;
  if (rc == ANE_OK) rc = tail_failed(d, op, &failed);
  if (rc == ANE_OK && failed) {
    latch_per_gemm(d);
    rc = restore_start(d, op, pos0);
    if (rc == ANE_OK) rc = enqueue_step(d, logits ? d->logits_d : nullptr, nullptr);
    if (rc == ANE_OK) rc = copy_out(d, next_tok, logits);
  }
  if (rc != ANE_OK) return drop_batch(d, rc);
  d->pos = pos0 + 1;
  return ANE_OK;
}

extern "C" int ane_decode_generate(ane_decoder* d, int32_t nsteps, uint16_t* out_tok) {
  const char* op = "generate";
  if (!d || !d->stream) return ANE_ERR_STATE;
  if (d->nseq == 0) return dfail(d, ANE_ERR_STATE, "storiesane decode generate: no prefill");
  if (nsteps < 0 || d->pos + nsteps > d->C)
    return dfail(d, ANE_ERR_ARG, "storiesane decode generate: %d steps from position %d exceed max_ctx=%d", nsteps,
                 d->pos, d->C);
  if (nsteps == 0) return ANE_OK;
  DCHK(op, hipSetDevice(d->cfg.device));
  const int pos0 = d->pos;
  int rc = d->use_tail ? save_start(d, op) : ANE_OK;
  if (rc == ANE_OK) rc = generate_run(d, op, nsteps, out_tok);
  bool failed = false;
  if (rc == ANE_OK) rc = tail_failed(d, op, &failed);
  if (rc == ANE_OK && failed) {
    latch_per_gemm(d);
    rc = restore_start(d, op, pos0);
    if (rc == ANE_OK) rc = generate_run(d, op, nsteps, out_tok);
  }
  if (rc != ANE_OK) return drop_batch(d, rc);
  d->pos = pos0 + nsteps;
  return ANE_OK;
}

namespace {

// nsteps replays of the step graph (captured on first use, and again after
// the batch size or the step's form changed), from position d->pos.
int generate_run(ane_decoder* d, const char* op, int nsteps, uint16_t* out_tok) {
  const hipStream_t st = d->stream;
  if (!d->gexec || d->graph_nseq != d->nseq) {
    if (d->gexec) (void)hipGraphExecDestroy(d->gexec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    d->gexec = nullptr;
    d->graph = nullptr;
    DCHK(op, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(d, nullptr, d->hist_d);
    hipGraph_t g = nullptr;
    hipError_t ce = hipStreamEndCapture(st, &g);
    if (rc != ANE_OK) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    DCHK(op, ce);
    d->graph = g;
    DCHK(op, hipGraphInstantiate(&d->gexec, g, nullptr, nullptr, 0));
    d->graph_nseq = d->nseq;
  }
  DCHK(op, dec_set_ctr(d->ctr_d, d->pos, 0, st));  // history rows count from 0 for this call
  DCHK(op, hipEventRecord(d->ev0, st));
  for (int i = 0; i < nsteps; i++) DCHK(op, hipGraphLaunch(d->gexec, st));
  DCHK(op, hipEventRecord(d->ev1, st));
  if (out_tok)
    DCHK(op, hipMemcpyAsync(out_tok, d->hist_d, (size_t)nsteps * d->nseq * 2, hipMemcpyDeviceToHost, st));
  DCHK(op, hipStreamSynchronize(st));
  float ms = 0.f;
  DCHK(op, hipEventElapsedTime(&ms, d->ev0, d->ev1));
  d->last_ms = ms;
  return ANE_OK;
}

}  // namespace

extern "C" int32_t ane_decode_fused_chain(ane_decoder* d) {
  if (!d) return -1;
  return d->chain_latched ? 2 : d->use_tail ? 1 : 0;
}

extern "C" int32_t ane_decode_position(ane_decoder* d) { return d ? d->pos : -1; }

extern "C" double ane_decode_last_ms(ane_decoder* d) { return d ? d->last_ms : 0.0; }

extern "C" int ane_decode_debug_fill_cache(ane_decoder* d, int byte) {
  const char* op = "debug fill cache";
  if (!d || !d->stream) return ANE_ERR_STATE;
  const size_t bytes = (size_t)d->L * d->B * d->NKV * d->C * 64 * sizeof(half_t);
  DCHK(op, hipSetDevice(d->cfg.device));
  DCHK(op, hipMemsetAsync(d->kc, byte & 0xff, bytes, d->stream));
  DCHK(op, hipMemsetAsync(d->vc, byte & 0xff, bytes, d->stream));
  DCHK(op, hipStreamSynchronize(d->stream));
  return ANE_OK;
}
