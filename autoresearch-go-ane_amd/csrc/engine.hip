// Engine: device state and the C-ABI entry points of libane_hip.so.
//
// This replaces the reference's accelerator objects (layerForward /
// offload / refreshANERuntimeForWeights: ane/layer_darwin.go,
// ane/offload_darwin.go, ane/runtime.go) with one device-resident model:
// fp32 master weights and their fp16 GEMM shadows live in HBM, activations
// never round-trip to the host between layers, and every stage runs on the
// engine's single HIP stream in order (which also removes the reference's
// eval-vs-refresh race, ane/engine.go:449 vs ane/runtime.go:74).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <string>
#include <algorithm>
#include <vector>

#include "../../include/ane_hip.h"
#include "../../include/ane_kernels.h"
#include "attention.h"
#include "engine_internal.h"
#include "gemm.h"
#include "rowops.h"
#include "train_ops.h"

using namespace ane;

// ---------------------------------------------------------------------------
// canonical parameter layout (one flat fp32 vector)
// ---------------------------------------------------------------------------
static constexpr int kVEGateCh = 12;  // ane/stories/weights.go:28

static bool cfg_is_ve_layer(const ane_model_cfg& c, int l) {
  // ane/stories/weights.go:22: value embeddings on layers with the parity of the last layer
  return c.arch == ANE_ARCH_NANOCHAT && (l % 2) == ((c.layers - 1) % 2);
}

void build_param_map(const ane_model_cfg& c, ParamMap* m) {
  const int64_t D = c.dim, H = c.hidden, V = c.vocab, NH = c.heads;
  int64_t off = 0;
  m->L.assign(c.layers, LayerOff());
  for (int l = 0; l < c.layers; l++) {
    LayerOff& o = m->L[l];
    o.wq = off; off += D * D;
    o.wk = off; off += D * D;
    o.wv = off; off += D * D;
    o.wo = off; off += D * D;
    o.w1 = off; off += H * D;
    o.w2 = off; off += D * H;
    if (c.arch == ANE_ARCH_LLAMA2) {
      o.w3 = off; off += H * D;
      o.g_att = off; off += D;
      o.g_ffn = off; off += D;
    } else if (cfg_is_ve_layer(c, l)) {
      o.ve_embed = off; off += V * D;
      o.ve_gate = off; off += NH * kVEGateCh;
    }
  }
  m->embed = off; off += V * D;
  if (c.arch == ANE_ARCH_LLAMA2) {
    m->g_final = off; off += D;
  } else {
    m->resid = off; off += c.layers;
    m->x0l = off; off += c.layers;
    m->smear_gate = off; off += D * D;
    m->smear_lambda = off; off += 1;
    m->backout_lambda = off; off += 1;
  }
  m->total = off;
}

static void param_segments(const ane_model_cfg& c, std::vector<std::pair<int64_t, int64_t>>* segs) {
  ParamMap m;
  build_param_map(c, &m);
  const int64_t D = c.dim, H = c.hidden, V = c.vocab, NH = c.heads;
  segs->clear();
  for (int l = 0; l < c.layers; l++) {
    const LayerOff& o = m.L[l];
    segs->push_back({o.wq, D * D});
    segs->push_back({o.wk, D * D});
    segs->push_back({o.wv, D * D});
    segs->push_back({o.wo, D * D});
    segs->push_back({o.w1, H * D});
    segs->push_back({o.w2, D * H});
    if (c.arch == ANE_ARCH_LLAMA2) {
      segs->push_back({o.w3, H * D});
      segs->push_back({o.g_att, D});
      segs->push_back({o.g_ffn, D});
    } else if (o.ve_embed >= 0) {
      segs->push_back({o.ve_embed, V * D});
      segs->push_back({o.ve_gate, NH * kVEGateCh});
    }
  }
  segs->push_back({m.embed, V * D});
  if (c.arch == ANE_ARCH_LLAMA2) {
    segs->push_back({m.g_final, D});
  } else {
    segs->push_back({m.resid, c.layers});
    segs->push_back({m.x0l, c.layers});
    segs->push_back({m.smear_gate, D * D});
    segs->push_back({m.smear_lambda, 1});
    segs->push_back({m.backout_lambda, 1});
  }
}

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
int eng_fail(ane_engine* e, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (e) e->err = buf;
  return code;
}


// ---------------------------------------------------------------------------
// profiling (HIP events bracketing tracked launches)
// ---------------------------------------------------------------------------
void prof_begin(ane_engine* e, int cls, hipStream_t s) {
  if (!e->prof_on) return;
  if (e->prof_next >= e->prof_events.size()) {
    ProfEvent pe;
    (void)hipEventCreate(&pe.a);
    (void)hipEventCreate(&pe.b);
    e->prof_events.push_back(pe);
  }
  ProfEvent& pe = e->prof_events[e->prof_next];
  pe.cls = cls;
  (void)hipEventRecord(pe.a, s ? s : e->stream);
}
void prof_end(ane_engine* e, double flops, double bytes, hipStream_t s) {
  if (!e->prof_on) return;
  ProfEvent& pe = e->prof_events[e->prof_next];
  pe.flops = flops;
  pe.bytes = bytes;
  (void)hipEventRecord(pe.b, s ? s : e->stream);
  e->prof_next++;
}

// Phase timers: a pair of events per kernel group of one training call.
// The pool only grows (hipEventCreate on the host; training never runs
// under graph capture); a failed create or record leaves the phase untimed.
void phase_reset(ane_engine* e) {
  e->ph_used = 0;
  e->ph_open = false;
  e->ph_cls.clear();
}

void phase_begin(ane_engine* e, int phase, hipStream_t s) {
  e->ph_open = false;
  if (!e->ph_sample && phase != PH_REFRESH) return;
  while ((int)e->ph_ev.size() < e->ph_used + 2) {
    hipEvent_t ev = nullptr;
    if (hipEventCreate(&ev) != hipSuccess) return;
    e->ph_ev.push_back(ev);
  }
  if (hipEventRecord(e->ph_ev[e->ph_used], s ? s : e->stream) != hipSuccess) return;
  e->ph_cls.push_back(phase);
  e->ph_used += 2;
  e->ph_open = true;
}

void phase_end(ane_engine* e, hipStream_t s) {
  if (!e->ph_open) return;
  e->ph_open = false;
  if (hipEventRecord(e->ph_ev[e->ph_used - 1], s ? s : e->stream) != hipSuccess) e->ph_cls.back() = -1;
}

void phase_sum(ane_engine* e, double ms[PH_COUNT]) {
  for (int p = 0; p < PH_COUNT; p++) ms[p] = 0.0;
  for (size_t i = 0; i < e->ph_cls.size(); i++) {
    const int p = e->ph_cls[i];
    float t = 0.f;
    if (p >= 0 && p < PH_COUNT && hipEventElapsedTime(&t, e->ph_ev[2 * i], e->ph_ev[2 * i + 1]) == hipSuccess)
      ms[p] += t;
  }
}

hipError_t eng_gemm(ane_engine* e, int cls, const half_t* A, int lda, bool at, const half_t* B, int ldb, bool bt,
                    int M, int N, int K, int epi, const EpiParams& p, int bm, int bn, bool side, const void* pf,
                    size_t pf_bytes) {
  if (side && (!e->dw_stream || !e->tr.splitk_ws2)) return hipErrorInvalidValue;
  hipStream_t s = side ? e->dw_stream : e->stream;
  float* ws = side ? e->tr.splitk_ws2 : e->tr.splitk_ws;
  GemmArgs g;
  g.A = A; g.B = B; g.lda = lda; g.ldb = ldb; g.M = M; g.N = N; g.K = K; g.a_t = at; g.b_t = bt;
  if (pf && pf_bytes && !at && !bt) {
    g.pf = pf;
    g.pf_bytes = pf_bytes;
  }
  // training: GEMMs whose output is too small to fill the chip split K
  // (K-major operands, or M-major ones as the weight gradients read them)
  if (!(at && !bt) && ws && bm == 0 && bn == 0) {
    int sp = 1;
    gemm_pick_split(M, N, K, epi, e->tr.splitk_cap, &bm, &bn, &sp);
    if (sp > 1) {
      g.splits = sp;
      g.ws = ws;
    }
  }
  prof_begin(e, cls, s);
  hipError_t r = gemm_run(g, epi, p, s, bm, bn);
  prof_end(e, 2.0 * M * N * K, 2.0 * ((double)M * K + (double)N * K), s);
  return r;
}

// ---------------------------------------------------------------------------
// allocation
// ---------------------------------------------------------------------------
static void free_all(ane_engine* e) {
  if (e->dev_set) (void)hipSetDevice(e->device);
  if (e->dw_stream) (void)hipStreamSynchronize(e->dw_stream);
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  for (void* p : e->allocs) (void)hipFree(p);
  e->allocs.clear();
  if (e->loss_host) (void)hipHostFree(e->loss_host);
  e->loss_host = nullptr;
  for (ProfEvent& pe : e->prof_events) {
    (void)hipEventDestroy(pe.a);
    (void)hipEventDestroy(pe.b);
  }
  e->prof_events.clear();
  for (hipEvent_t& ev : e->step_ev)
    if (ev) {
      (void)hipEventDestroy(ev);
      ev = nullptr;
    }
  for (hipEvent_t ev : e->ph_ev) (void)hipEventDestroy(ev);
  e->ph_ev.clear();
  e->ph_cls.clear();
  e->ph_used = 0;
  e->train_ready = false;
  e->tr = TrainBufs();
  e->ls.clear();
  e->embed_h = e->smear_h = e->embed_t = e->smear_t = nullptr;
  e->shadow_jobs = nullptr;
  e->n_shadow_jobs = e->n_shadow_tiles = 0;
  e->shadow_jobs_t = false;
  drop_fwd_graph(e);
  for (hipEvent_t& ev : e->refresh_ev)
    if (ev) {
      (void)hipEventDestroy(ev);
      ev = nullptr;
    }
  e->refresh_pending = false;
  for (hipEvent_t ev : e->upd_ev) (void)hipEventDestroy(ev);
  e->upd_ev.clear();
  e->upd_pending = false;
  e->adam_unread = false;
  for (hipEvent_t ev : e->xev) (void)hipEventDestroy(ev);
  e->xev.clear();
  e->xev_next = 0;
  if (e->dw_stream) (void)hipStreamDestroy(e->dw_stream);
  e->dw_stream = nullptr;
  if (e->stream) (void)hipStreamDestroy(e->stream);
  e->stream = nullptr;
}

static int validate_cfg(ane_engine* e, const ane_model_cfg& c) {
  if (c.arch != ANE_ARCH_NANOCHAT && c.arch != ANE_ARCH_LLAMA2)
    return eng_fail(e, ANE_ERR_ARG, "storiesane open: unknown arch %d", c.arch);
  if (c.heads <= 0 || c.dim != 64 * c.heads)
    return eng_fail(e, ANE_ERR_ARG, "storiesane open: dim=%d must be 64*heads (heads=%d)", c.dim, c.heads);
  if (c.dim % 64 || c.hidden <= 0 || c.hidden % 64 || c.vocab <= 0 || c.vocab % 64 || c.layers <= 0)
    return eng_fail(e, ANE_ERR_ARG, "storiesane open: dim/hidden/vocab must be positive multiples of 64");
  if (c.seq <= 0 || c.seq % 64 || c.seq > 512)
    return eng_fail(e, ANE_ERR_ARG, "storiesane open: seq=%d must be a multiple of 64 and <= 512", c.seq);
  if (c.arch == ANE_ARCH_NANOCHAT && c.layers < 2)
    return eng_fail(e, ANE_ERR_ARG, "storiesane open: nanochat needs >= 2 layers (backout)");
  return ANE_OK;
}

// ---------------------------------------------------------------------------
// lifecycle
// ---------------------------------------------------------------------------
extern "C" int64_t ane_param_count(const ane_model_cfg* cfg) {
  if (!cfg) return -1;
  ParamMap m;
  build_param_map(*cfg, &m);
  return m.total;
}

extern "C" int ane_param_layout(const ane_model_cfg* cfg, int64_t* offsets, int64_t* sizes, int max) {
  if (!cfg) return ANE_ERR_ARG;
  std::vector<std::pair<int64_t, int64_t>> segs;
  param_segments(*cfg, &segs);
  for (int i = 0; i < (int)segs.size() && i < max; i++) {
    if (offsets) offsets[i] = segs[i].first;
    if (sizes) sizes[i] = segs[i].second;
  }
  return (int)segs.size();
}

extern "C" const char* ane_last_error(const ane_engine* e) { return e ? e->err.c_str() : "storiesane: null engine"; }

static void apply_option_defaults(ane_options* o) {
  // ane/engine.go:185-240
  if (o->lr <= 0) o->lr = 3e-4f;
  if (o->accum_steps <= 0) o->accum_steps = 1;
  if (o->seed == 0) o->seed = 42;
  if (o->adam_beta1 <= 0) o->adam_beta1 = 0.9f;
  if (o->adam_beta2 <= 0) o->adam_beta2 = 0.999f;
  if (o->adam_eps <= 0) o->adam_eps = 1e-8f;
  if (o->grad_clip < 0) o->grad_clip = 0;
  if (o->loss_scale <= 0) o->loss_scale = 256;
  if (o->embed_lr_mult <= 0) o->embed_lr_mult = 1.0f;
  if (o->scalar_lr_mult <= 0) o->scalar_lr_mult = 1.0f;
  if (o->lambda_lr_mult <= 0) o->lambda_lr_mult = 0.01f;
  if (o->lambda_beta1 <= 0) o->lambda_beta1 = o->adam_beta1;
  if (o->lambda_beta2 <= 0) o->lambda_beta2 = o->adam_beta2;
  if (o->max_batch <= 0) o->max_batch = 1;
}

static int open_impl(ane_engine* e) {
  const char* op = "open";
  const ane_model_cfg& c = e->cfg;
  const int D = c.dim, H = c.hidden, V = c.vocab, S = c.seq, NH = c.heads, L = c.layers;
  const size_t T = (size_t)e->opt.max_batch * S;
  HIPCHK(op, hipSetDevice(e->device));
  e->dev_set = true;
  HIPCHK(op, hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
  build_param_map(c, &e->pm);
  const size_t P = (size_t)e->pm.total;
  HIPCHK(op, dalloc(e, &e->P, P));
  HIPCHK(op, hipMemsetAsync(e->P, 0, P * sizeof(float), e->stream));

  // fp16 shadows
  size_t nsh = 0;
  const bool llama = c.arch == ANE_ARCH_LLAMA2;
  const size_t per_layer = (size_t)3 * D * D + (size_t)D * D + (size_t)(llama ? 2 : 1) * H * D + (size_t)D * H;
  nsh = per_layer * L + (size_t)V * D + (llama ? 0 : (size_t)D * D);
  HIPCHK(op, dalloc(e, &e->shadow, nsh));
  e->ls.assign(L, LayerShadow());
  half_t* q = e->shadow;
  for (int l = 0; l < L; l++) {
    LayerShadow& s = e->ls[l];
    s.wqkv = q; q += (size_t)3 * D * D;
    s.wo = q; q += (size_t)D * D;
    s.w13 = q; q += (size_t)(llama ? 2 : 1) * H * D;
    s.w2 = q; q += (size_t)D * H;
  }
  e->embed_h = q; q += (size_t)V * D;
  if (!llama) { e->smear_h = q; q += (size_t)D * D; }

  // RoPE tables: buildRoPETables (ane/train_util.go:183-202), theta as configured
  {
    const int half = 32;
    std::vector<float> cs((size_t)S * half), sn((size_t)S * half);
    for (int pos = 0; pos < S; pos++)
      for (int i = 0; i < half; i++) {
        double freq = (double)pos / pow(c.rope_theta, (double)(2 * i) / 64.0);
        cs[(size_t)pos * half + i] = (float)cos(freq);
        sn[(size_t)pos * half + i] = (float)sin(freq);
      }
    HIPCHK(op, dalloc(e, &e->rope_cos, cs.size()));
    HIPCHK(op, dalloc(e, &e->rope_sin, sn.size()));
    HIPCHK(op, hipMemcpy(e->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    HIPCHK(op, hipMemcpy(e->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  }

  // activations
  HIPCHK(op, dalloc(e, &e->tok, T));
  HIPCHK(op, dalloc(e, &e->tgt, T));
  HIPCHK(op, dalloc(e, &e->pos_d, (size_t)e->opt.max_batch));
  HIPCHK(op, dalloc(e, &e->x, T * D));
  if (!llama) {
    HIPCHK(op, dalloc(e, &e->x0, T * D));
    HIPCHK(op, dalloc(e, &e->xpre, T * D));
    HIPCHK(op, dalloc(e, &e->xmid, T * D));
  }
  HIPCHK(op, dalloc(e, &e->xh, T * D));
  if (llama) HIPCHK(op, dalloc(e, &e->ssq_part, (size_t)kRrMaxParts * T));
  HIPCHK(op, dalloc(e, &e->qkv, T * 3 * D));
  HIPCHK(op, dalloc(e, &e->att, T * D));
  HIPCHK(op, dalloc(e, &e->gate, T * H));
  // classifier block rows: one (max, sumexp) partial per block row and token
  e->ce_bm = (V % 128 == 0) ? 128 : 64;
  e->ce_np = V / e->ce_bm;
  HIPCHK(op, dalloc(e, &e->partial, (size_t)e->ce_np * T));
  HIPCHK(op, dalloc(e, &e->tgt_logit, T));
  HIPCHK(op, dalloc(e, &e->lse, T));
  HIPCHK(op, dalloc(e, &e->tok_loss, T));
  HIPCHK(op, dalloc(e, &e->loss_seq, (size_t)e->opt.max_batch));
  HIPCHK(op, hipHostMalloc((void**)&e->loss_host, (size_t)e->opt.max_batch * sizeof(float), hipHostMallocDefault));
  HIPCHK(op, dalloc(e, &e->logits, (size_t)V * S));
  (void)NH;
  HIPCHK(op, hipStreamSynchronize(e->stream));
  return ANE_OK;
}

extern "C" int ane_open(const ane_model_cfg* cfg, const ane_options* opts, ane_engine** out) {
  if (!out || !cfg) return ANE_ERR_ARG;
  *out = nullptr;
  ane_engine* e = new ane_engine();
  e->cfg = *cfg;
  if (e->cfg.rope_theta <= 0) e->cfg.rope_theta = e->cfg.arch == ANE_ARCH_LLAMA2 ? 10000.0 : 100000.0;
  if (opts) e->opt = *opts;
  apply_option_defaults(&e->opt);
  e->device = e->opt.device;
  if (const char* g = getenv("ANE_GRAPHS")) e->use_graph = atoi(g) != 0;
  // ANE_FUSED_NORM=1: the llama2 eval forward defers each RMSNorm into the
  // GEMMs around it instead of launching it
  if (const char* g = getenv("ANE_FUSED_NORM")) e->fused_norm = atoi(g) != 0;
  if (const char* g = getenv("ANE_FUSED_PF")) e->fused_pf = atoi(g) != 0;
  if (const char* g = getenv("ANE_GEMM_SELFPF")) e->gemm_selfpf = atoi(g) != 0;
  if (const char* g = getenv("ANE_TR_DW")) e->tr_dw = atoi(g) != 0;
  if (const char* g = getenv("ANE_DW_ASYNC")) e->dw_async = atoi(g) != 0;
  if (const char* g = getenv("ANE_BWD_PREFETCH")) e->bwd_prefetch = atoi(g) != 0;
  if (const char* g = getenv("ANE_FUSED_ADAM")) e->fused_adam = atoi(g) != 0;
  if (const char* g = getenv("ANE_ASYNC_UPDATE")) e->async_update = atoi(g) != 0;
  if (const char* g = getenv("ANE_PHASE_EVERY")) e->ph_period = atoi(g) > 0 ? atoi(g) : 1;
  e->lr = e->opt.lr;
  int rc = validate_cfg(e, e->cfg);
  if (rc == ANE_OK) rc = open_impl(e);
  if (rc != ANE_OK) {
    free_all(e);
    e->closed = true;
  } else {
    e->rng = drand48_seed(e->opt.seed);
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    e->start_s = (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
  }
  *out = e;
  return rc;
}

extern "C" void ane_close(ane_engine* e) {
  if (!e || e->closed) return;
  free_all(e);
  e->closed = true;
}

extern "C" void ane_destroy(ane_engine* e) {
  if (!e) return;
  ane_close(e);
  delete e;
}

extern "C" int ane_sync(ane_engine* e) {
  CLOSED_CHECK("sync");
  HIPCHK("sync", join_update(e));  // an asynchronous update still running
  HIPCHK("sync", hipStreamSynchronize(e->stream));
  if (e->dw_stream) HIPCHK("sync", hipStreamSynchronize(e->dw_stream));
  return ANE_OK;
}

// ---------------------------------------------------------------------------
// weights
// ---------------------------------------------------------------------------
// Job table of shadow_refresh: every fp16 shadow (and, once training has
// allocated them, its transpose) from the fp32 masters in one launch.
static int build_shadow_jobs(ane_engine* e) {
  const char* op = "refresh weights";
  const ane_model_cfg& c = e->cfg;
  const int D = c.dim, H = c.hidden, V = c.vocab;
  const bool llama = c.arch == ANE_ARCH_LLAMA2;
  std::vector<ShadowJob> jobs;
  int tiles = 0;
  auto add = [&](const float* src, half_t* dst, half_t* dst_t, int R, int C, int stride, int off, int ldt) {
    ShadowJob j;
    j.src = src; j.dst = dst; j.dst_t = dst_t; j.R = R; j.C = C; j.blk_stride = stride; j.blk_off = off;
    j.ldt = ldt; j.tile0 = tiles;
    tiles += (R / 64) * (C / 64);
    jobs.push_back(j);
  };
  for (int l = 0; l < c.layers; l++) {
    const LayerOff& o = e->pm.L[l];
    const LayerShadow& s = e->ls[l];
    add(e->P + o.wq, s.wqkv, s.wqkv_t, 3 * D, D, 32, 0, 3 * D);  // Wq|Wk|Wv are adjacent
    add(e->P + o.wo, s.wo, s.wo_t, D, D, 32, 0, D);
    if (llama) {  // W1 / W3 rows interleaved by 32
      add(e->P + o.w1, s.w13, s.w13_t, H, D, 64, 0, 2 * H);
      add(e->P + o.w3, s.w13, s.w13_t, H, D, 64, 32, 2 * H);
    } else {
      add(e->P + o.w1, s.w13, s.w13_t, H, D, 32, 0, H);
    }
    add(e->P + o.w2, s.w2, s.w2_t, D, H, 32, 0, D);
  }
  add(e->P + e->pm.embed, e->embed_h, e->embed_t, V, D, 32, 0, V);
  if (!llama) add(e->P + e->pm.smear_gate, e->smear_h, e->smear_t, D, D, 32, 0, D);
  if (!e->shadow_jobs || (int)jobs.size() > e->n_shadow_jobs) {
    // sized once for the largest table this engine builds (same count with or without transposes)
    HIPCHK(op, dalloc(e, &e->shadow_jobs, jobs.size()));
  }
  HIPCHK(op, hipStreamSynchronize(e->stream));  // no launch still reads the old table
  HIPCHK(op, hipMemcpy(e->shadow_jobs, jobs.data(), jobs.size() * sizeof(ShadowJob), hipMemcpyHostToDevice));
  e->shadow_jobs_h = jobs;
  e->upd_sig.clear();  // update jobs point at these shadows
  e->n_shadow_jobs = (int)jobs.size();
  e->n_shadow_tiles = tiles;
  e->shadow_jobs_t = e->embed_t != nullptr;
  return ANE_OK;
}

int ensure_update_jobs(ane_engine* e, const AdamArgs& a) {
  const char* op = "flush";
  std::vector<int64_t> sig;
  for (int i = 0; i < a.nseg; i++) {
    sig.push_back(a.seg[i].off);
    sig.push_back(a.seg[i].len);
    sig.push_back(a.seg[i].chunk);
  }
  if (e->upd_jobs && sig == e->upd_sig) return ANE_OK;
  // segments in parameter order, each cut at the matrices with a shadow
  std::vector<int> order(a.nseg);
  for (int i = 0; i < a.nseg; i++) order[i] = i;
  std::sort(order.begin(), order.end(), [&](int x, int y) { return a.seg[x].off < a.seg[y].off; });
  std::vector<const ShadowJob*> sj;
  for (const ShadowJob& j : e->shadow_jobs_h) sj.push_back(&j);
  std::sort(sj.begin(), sj.end(), [](const ShadowJob* x, const ShadowJob* y) { return x->src < y->src; });
  std::vector<UpdateJob> jobs;
  int blocks = 0;
  auto emit = [&](int64_t off, int64_t len, const ShadowJob* sh, int seg) {
    UpdateJob u;
    u.off = off; u.len = len; u.sh = sh ? sh->dst : nullptr;
    u.C = sh ? sh->C : 0; u.blk_stride = sh ? sh->blk_stride : 0; u.blk_off = sh ? sh->blk_off : 0;
    u.seg = seg; u.blk0 = blocks; u.vec = (off % 4 == 0 && len % 4 == 0) ? 1 : 0;
    blocks += (int)((len + kUpdateChunk - 1) / kUpdateChunk);
    jobs.push_back(u);
    return !sh || (u.vec && u.C % 4 == 0);
  };
  int64_t covered = 0;
  for (int si : order) {
    const AdamSeg& sg = a.seg[si];
    if (sg.off != covered)
      return eng_fail(e, ANE_ERR_STATE, "storiesane flush: parameter groups leave [%lld, %lld) uncovered",
                      (long long)covered, (long long)sg.off);
    int64_t cur = sg.off;
    const int64_t end = sg.off + sg.len;
    for (const ShadowJob* j : sj) {
      const int64_t jo = j->src - e->P, je = jo + (int64_t)j->R * j->C;
      if (je <= sg.off || jo >= end) continue;
      if (jo < sg.off || je > end)
        return eng_fail(e, ANE_ERR_STATE, "storiesane flush: a shadowed matrix straddles a parameter group");
      if (cur < jo && !emit(cur, jo - cur, nullptr, si)) return eng_fail(e, ANE_ERR_STATE, "storiesane flush: job");
      if (!emit(jo, je - jo, j, si))
        return eng_fail(e, ANE_ERR_STATE, "storiesane flush: shadowed matrix not 16-byte aligned");
      cur = je;
    }
    if (cur < end && !emit(cur, end - cur, nullptr, si)) return eng_fail(e, ANE_ERR_STATE, "storiesane flush: job");
    covered = end;
  }
  if (covered != e->pm.total)
    return eng_fail(e, ANE_ERR_STATE, "storiesane flush: parameter groups cover %lld of %lld",
                    (long long)covered, (long long)e->pm.total);
  // chunk order (parameter order within a chunk), blocks renumbered to match
  const int nch = 1 + e->cfg.layers;
  std::vector<UpdateJob> by;
  e->upd_j0.assign(nch, 0);
  e->upd_nj.assign(nch, 0);
  e->upd_b0.assign(nch, 0);
  e->upd_nb.assign(nch, 0);
  int nb = 0;
  for (int c = 0; c < nch; c++) {
    e->upd_j0[c] = (int)by.size();
    e->upd_b0[c] = nb;
    for (UpdateJob u : jobs) {
      if (a.seg[u.seg].chunk != c) continue;
      u.blk0 = nb;
      nb += (int)((u.len + kUpdateChunk - 1) / kUpdateChunk);
      by.push_back(u);
    }
    e->upd_nj[c] = (int)by.size() - e->upd_j0[c];
    e->upd_nb[c] = nb - e->upd_b0[c];
  }
  if (by.size() != jobs.size() || nb != blocks)
    return eng_fail(e, ANE_ERR_STATE, "storiesane flush: a parameter group has no update chunk");
  if ((int)by.size() > e->upd_cap) {
    HIPCHK(op, dalloc(e, &e->upd_jobs, by.size()));
    e->upd_cap = (int)by.size();
  }
  // no launch still reads the old table (an asynchronous update reads it on the dW stream)
  HIPCHK(op, hipStreamSynchronize(e->stream));
  if (e->dw_stream) HIPCHK(op, hipStreamSynchronize(e->dw_stream));
  HIPCHK(op, hipMemcpy(e->upd_jobs, by.data(), by.size() * sizeof(UpdateJob), hipMemcpyHostToDevice));
  e->n_upd_jobs = (int)by.size();
  e->n_upd_blocks = nb;
  e->upd_sig = sig;
  return ANE_OK;
}

hipError_t join_update(ane_engine* e) {
  if (!e->upd_pending) return hipSuccess;
  e->upd_pending = false;
  return hipStreamWaitEvent(e->stream, e->upd_ev.back(), 0);
}

hipError_t wait_update(ane_engine* e, int chunk) {
  if (!e->upd_pending) return hipSuccess;
  return hipStreamWaitEvent(e->stream, e->upd_ev[chunk], 0);
}

int refresh_shadows(ane_engine* e) {
  const char* op = "refresh weights";
  // an asynchronous refresh still reading the plain shadows and the table
  if (e->refresh_pending) HIPCHK(op, hipEventSynchronize(e->refresh_ev[1]));
  if (!e->shadow_jobs || e->shadow_jobs_t != (e->embed_t != nullptr)) {
    int rc = build_shadow_jobs(e);
    if (rc) return rc;
  }
  HIPCHK(op, shadow_refresh(e->shadow_jobs, e->n_shadow_jobs, e->n_shadow_tiles, e->stream));
  return ANE_OK;
}

extern "C" int ane_set_params(ane_engine* e, const float* params, int64_t n) {
  CLOSED_CHECK("set params");
  HIPCHK("set params", join_update(e));  // an asynchronous update still running
  if (!params || n != e->pm.total)
    return eng_fail(e, ANE_ERR_ARG, "storiesane set params: len=%lld want=%lld", (long long)n,
                    (long long)e->pm.total);
  HIPCHK("set params", hipMemcpyAsync(e->P, params, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
  int rc = refresh_shadows(e);
  if (rc) return rc;
  HIPCHK("set params", hipStreamSynchronize(e->stream));
  return ANE_OK;
}

extern "C" int ane_get_params(ane_engine* e, float* params, int64_t n) {
  CLOSED_CHECK("get params");
  HIPCHK("get params", join_update(e));  // an asynchronous update still running
  if (!params || n != e->pm.total)
    return eng_fail(e, ANE_ERR_ARG, "storiesane get params: len=%lld want=%lld", (long long)n,
                    (long long)e->pm.total);
  HIPCHK("get params", hipMemcpyAsync(params, e->P, (size_t)n * 4, hipMemcpyDeviceToHost, e->stream));
  HIPCHK("get params", hipStreamSynchronize(e->stream));
  return ANE_OK;
}

extern "C" int ane_set_tokens(ane_engine* e, const uint16_t* tokens, int64_t n) {
  CLOSED_CHECK("set tokens");
  if (n > 0 && n < (int64_t)e->cfg.seq + 1)
    return eng_fail(e, ANE_ERR_ARG, "storiesane open: not enough tokens for seq=%d", e->cfg.seq);
  if (e->data) {
    HIPCHK("set tokens", hipStreamSynchronize(e->stream));
    HIPCHK("set tokens", hipFree(e->data));
    for (auto it = e->allocs.begin(); it != e->allocs.end(); ++it)
      if (*it == (void*)e->data) { e->allocs.erase(it); break; }
    e->data = nullptr;
    e->ndata = 0;
  }
  if (n <= 0) return ANE_OK;
  HIPCHK("set tokens", dalloc(e, &e->data, (size_t)n));
  HIPCHK("set tokens", hipMemcpy(e->data, tokens, (size_t)n * 2, hipMemcpyHostToDevice));
  e->ndata = n;
  return ANE_OK;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// One pass of the layer stack over T = nseq * seq tokens already in e->tok.
// Leaves fp16 final-normed hidden states in e->xh.  Mirrors
// forwardTrainingCPU (ane/train_full.go:383-453) and evalLogitsCPUInto
// (ane/engine.go:954-1038) for nanochat; llama2 uses gain RMSNorm, SwiGLU,
// plain residuals and no QK-norm / VE / smear / backout.
// In training mode (train != 0, buffers of ensure_train) every layer keeps
// its activations: the residual GEMMs write out-of-place into the next
// layer's input buffer, so nothing is copied.
//
// defer_norm (llama2 eval forward; ANE_FUSED_NORM=0 keeps the norm
// launches): no RMSNorm launch.  Each norm's input x comes with xh =
// fp16(x * gain) and per-row partial sums of x^2 (from the embedding, or
// from the residual GEMM's epilogue, one partial per column block); the GEMM
// that consumes xh scales its (linear) output rows by rr = 1 / rms(x) in its
// epilogue.  The final norm is left to the classifier (e->fwd_rr_nparts > 0).
// The norm launches also streamed the next GEMM's weights through the
// caches; without them each GEMM's blocks would wait on HBM for the same
// cold weight tile at every k-step, so the QKV, W1|W3 and W2 GEMMs' first
// blocks stream their own weights with their prologue loads (GemmArgs::pf;
// Wo's are streamed by attention, the classifier's by a prefetch launch).
// B32, back to back on one box: 2.770 ms per forward against 2.844 with the
// norm launches, 2.795 with a prefetch launch before each GEMM instead.
int forward_body(ane_engine* e, int nseq, int train, bool defer_norm) {
  const char* op = "forward";
  const ane_model_cfg& c = e->cfg;
  const int D = c.dim, H = c.hidden, V = c.vocab, S = c.seq, NH = c.heads, L = c.layers;
  const int T = nseq * S;
  const bool llama = c.arch == ANE_ARCH_LLAMA2;
  const float* P = e->P;
  hipStream_t st = e->stream;
  TrainBufs& tb = e->tr;
  const bool fused = defer_norm && !train && llama && e->fused_norm && e->ssq_part;
  e->fwd_rr_nparts = 0;
  // the residual GEMMs' tile fixes how many partials each norm has
  int res_bm = 0, res_bn = 0;
  if (fused) {
    gemm_pick_tile(T, D, H, EPI_RESID_NORM, &res_bm, &res_bn);
    if (!res_bn || D / res_bn > kRrMaxParts)
      return eng_fail(e, ANE_ERR_ARG, "storiesane forward: no residual tile for dim=%d", D);
  }
  // RR epilogue parameters over the current partials
  auto rr = [&](EpiParams& p, int nparts) {
    p.rr_part = e->ssq_part; p.rr_ld = T; p.rr_nparts = nparts; p.rr_dim = D;
  };
  int nparts = 1;

  float* x_first = train ? tb.L[0].xin : e->x;
  // a training forward behind an asynchronous update: each part starts once
  // the update chunk of the weights it reads is done (every other caller
  // has waited for the whole update at its entry point)
  if (train) HIPCHK(op, wait_update(e, 0));
  if (llama && fused) {
    prof_begin(e, 7);
    HIPCHK(op, embed_xg(x_first, e->xh, e->ssq_part, P + e->pm.embed, e->tok, P + e->pm.L[0].g_att, T, D, V, st,
                        e->ls[0].wqkv, (size_t)3 * D * D * sizeof(half_t)));
    prof_end(e, 0, (double)T * D * 10);
  } else if (llama) {
    prof_begin(e, 7);
    HIPCHK(op, embed_lookup(x_first, P + e->pm.embed, e->tok, T, D, V, st));
    prof_end(e, 0, (double)T * D * 8);
  } else {
    half_t* x0h = train ? tb.x0h : e->xh;
    prof_begin(e, 7);
    HIPCHK(op, embed_norm(e->xpre, e->x0, x0h, P + e->pm.embed, e->tok, T, D, V, st));
    prof_end(e, 0, (double)T * D * 14);
    // smear (ane/common.go:324-339): x = x0 + lambda * sigmoid(SmearGate x0)[t] * x0[t-1]
    EpiParams p;
    p.C = x_first; p.ldc = D; p.X0 = e->x0; p.alpha_ptr = P + e->pm.smear_lambda; p.seq = S;
    if (train) p.C2 = tb.sg_act;
    HIPCHK(op, eng_gemm(e, 7, x0h, D, false, e->smear_h, D, false, T, D, D, EPI_SMEAR, p));
  }
  for (int l = 0; l < L; l++) {
    const LayerOff& o = e->pm.L[l];
    const LayerShadow& s = e->ls[l];
    LayerActs A;
    if (train) {
      A = tb.L[l];
    } else {
      A.xin = e->x; A.x2 = e->x; A.xn = e->xh; A.xn2 = e->xh; A.qkv = e->qkv; A.att = e->att; A.gate = e->gate;
    }
    float* xout = train ? (l + 1 < L ? tb.L[l + 1].xin : tb.xlast) : e->x;
    if (train) HIPCHK(op, wait_update(e, 1 + l));
    if (!fused) {
      prof_begin(e, 6);
      // each memory-bound kernel also streams the next GEMM's weights through
      // the caches (prefetch_slice): QKV here, Wo in attention, W1|W3 + W2 in
      // the FFN norm, the classifier in the final norm
      HIPCHK(op, rmsnorm_f16(A.xn, A.xin, nullptr, nullptr, llama ? P + o.g_att : nullptr, T, D, st, s.wqkv,
                             (size_t)3 * D * D * sizeof(half_t)));
      prof_end(e, 0, (double)T * D * 6);
    }
    if (fused && l > 0 && e->fused_pf && !e->gemm_selfpf) {
      prof_begin(e, 6);
      HIPCHK(op, prefetch_weights(s.wqkv, (size_t)3 * D * D * sizeof(half_t), st));
      prof_end(e, 0, (double)3 * D * D * 2);
    }
    {
      EpiParams p;
      p.C = A.qkv; p.ldc = 3 * D;
      if (fused) rr(p, nparts);
      // its weights were streamed by the previous layer's W2 GEMM (layer 0: by the embedding)
      HIPCHK(op, eng_gemm(e, 0, A.xn, D, false, s.wqkv, D, false, T, 3 * D, D, fused ? EPI_STORE_H_RR : EPI_STORE_H,
                          p));
    }
    {
      AttnArgs a;
      memset(&a, 0, sizeof a);
      a.qkv = A.qkv; a.out = A.att; a.lse = A.lse; a.qkvt = A.qkvt; a.qkvt_lo = A.qk_lo;
      a.rope_cos = e->rope_cos; a.rope_sin = e->rope_sin;
      a.nseq = nseq; a.S = S; a.NH = NH;
      a.qknorm = llama ? 0 : 1;
      a.scale = 0.125f;
      a.pf = s.wo; a.pf_bytes = (size_t)D * D * sizeof(half_t);
      if (o.ve_embed >= 0) {
        a.ve_x = A.xin; a.ve_gate = P + o.ve_gate; a.ve_embed = P + o.ve_embed; a.tokens = e->tok; a.vocab = V;
      }
      prof_begin(e, 5);
      HIPCHK(op, attention_fwd(a, st));
      // causal FLOPs: QK^T and PV over the lower triangle
      prof_end(e, 4.0 * 64 * NH * (double)nseq * ((double)S * (S + 1) / 2), (double)T * D * 2 * 4);
    }
    {
      EpiParams p;
      p.C = A.x2; p.ldc = D; p.R = A.xin;
      if (!llama) { p.alpha_ptr = P + e->pm.resid + l; p.X0 = e->x0; p.beta_ptr = P + e->pm.x0l + l; }
      if (fused) {
        p.C2 = A.xn2; p.ldc2 = D; p.gain = P + o.g_ffn; p.ssq_part = e->ssq_part; p.ssq_ld = T;
        HIPCHK(op, eng_gemm(e, 1, A.att, D, false, s.wo, D, false, T, D, D, EPI_RESID_NORM, p, res_bm, res_bn));
        nparts = D / res_bn;
      } else {
        HIPCHK(op, eng_gemm(e, 1, A.att, D, false, s.wo, D, false, T, D, D, EPI_RESID, p));
      }
    }
    if (!fused) {
      prof_begin(e, 6);
      HIPCHK(op, rmsnorm_f16(A.xn2, A.x2, nullptr, nullptr, llama ? P + o.g_ffn : nullptr, T, D, st, s.w13,
                             ((size_t)(llama ? 2 : 1) * H * D + (size_t)D * H) * sizeof(half_t)));  // W1|W3, W2
      prof_end(e, 0, (double)T * D * 6);
    }
    {
      EpiParams p;
      p.C = A.gate; p.ldc = H;
      p.C2 = A.h13; p.ldc2 = llama ? 2 * H : H;
      if (fused) {
        if (e->fused_pf && !e->gemm_selfpf) {
          prof_begin(e, 6);
          HIPCHK(op, prefetch_weights(s.w13, ((size_t)2 * H * D + (size_t)D * H) * sizeof(half_t), st));  // W1|W3, W2
          prof_end(e, 0, (double)3 * H * D * 2);
        }
        rr(p, nparts);
        // streams its own weights and W2's (adjacent shadows)
        HIPCHK(op, eng_gemm(e, 2, A.xn2, D, false, s.w13, D, false, T, 2 * H, D, EPI_SWIGLU_RR, p, 0, 0, false,
                            e->gemm_selfpf ? s.w13 : nullptr, ((size_t)2 * H * D + (size_t)D * H) * sizeof(half_t)));
      } else if (llama) {
        HIPCHK(op, eng_gemm(e, 2, A.xn2, D, false, s.w13, D, false, T, 2 * H, D, EPI_SWIGLU, p));
      } else {
        HIPCHK(op, eng_gemm(e, 2, A.xn2, D, false, s.w13, D, false, T, H, D, EPI_RELU2, p));
      }
    }
    {
      EpiParams p;
      p.C = xout; p.ldc = D; p.R = A.x2;
      if (!llama) {
        p.alpha_ptr = P + e->pm.resid + l; p.X0 = e->x0; p.beta_ptr = P + e->pm.x0l + l;
        if (l == L / 2 - 1) p.C2 = e->xmid;  // backout snapshot (ane/train_full.go:447-449)
      }
      if (fused) {
        // the next norm's inputs: the next layer's attention norm, or the final norm
        p.C2 = A.xn; p.ldc2 = D; p.gain = P + (l + 1 < L ? e->pm.L[l + 1].g_att : e->pm.g_final);
        p.ssq_part = e->ssq_part; p.ssq_ld = T;
        // streams the next layer's Wq|Wk|Wv (the classifier's come by a prefetch launch)
        const void* pf2 = e->gemm_selfpf && l + 1 < L ? (const void*)e->ls[l + 1].wqkv : nullptr;
        HIPCHK(op, eng_gemm(e, 3, A.gate, H, false, s.w2, H, false, T, D, H, EPI_RESID_NORM, p, res_bm, res_bn, false,
                            pf2, (size_t)3 * D * D * sizeof(half_t)));
        nparts = D / res_bn;
      } else {
        HIPCHK(op, eng_gemm(e, 3, A.gate, H, false, s.w2, H, false, T, D, H, EPI_RESID, p));
      }
    }
  }
  if (train) e->upd_pending = false;  // the main stream now follows every chunk
  if (fused) {  // xh = fp16(x * g_final); the classifier applies 1 / rms
    if (e->fused_pf) {
      prof_begin(e, 6);
      HIPCHK(op, prefetch_weights(e->embed_h, (size_t)V * D * sizeof(half_t), st));
      prof_end(e, 0, (double)V * D * 2);
    }
    e->fwd_rr_nparts = nparts;
    return ANE_OK;
  }
  // final norm (backout first for nanochat, ane/common.go:385-389)
  float* xl = train ? tb.xlast : e->x;
  prof_begin(e, 6);
  if (llama) {
    HIPCHK(op, rmsnorm_f16(e->xh, xl, nullptr, nullptr, P + e->pm.g_final, T, D, st, e->embed_h,
                           (size_t)V * D * sizeof(half_t)));
  } else if (train) {
    // keep the post-backout state for the final norm's backward
    HIPCHK(op, backout_fwd(tb.xfinal, xl, e->xmid, P + e->pm.backout_lambda, (size_t)T * D, st));
    HIPCHK(op, rmsnorm_f16(e->xh, tb.xfinal, nullptr, nullptr, nullptr, T, D, st, e->embed_h,
                           (size_t)V * D * sizeof(half_t)));
  } else {
    HIPCHK(op, rmsnorm_f16(e->xh, xl, e->xmid, P + e->pm.backout_lambda, nullptr, T, D, st, e->embed_h,
                           (size_t)V * D * sizeof(half_t)));
  }
  prof_end(e, 0, (double)T * D * (llama ? 6 : 10));
  return ANE_OK;
}

// classifier + softcap + cross-entropy partials, then the per-sequence mean
int head_loss(ane_engine* e, int nseq, float* colscale, float dscale) {
  const char* op = "final head";
  const ane_model_cfg& c = e->cfg;
  const int D = c.dim, V = c.vocab, S = c.seq;
  const int T = nseq * S;
  EpiParams p;
  p.targets = e->tgt; p.partial = e->partial; p.tgt_logit = e->tgt_logit;
  p.softcap = c.arch == ANE_ARCH_NANOCHAT; p.cap = 15.f; p.vocab = V;
  // block rows: 256 (8-wave 256x256 tiles) once that still gives >= 512
  // blocks, else the open-time size; the partial buffer holds V / ce_bm rows
  int bm = e->ce_bm, bn = 0;
  if (V % 256 == 0 && T % 256 == 0 && (long)(V / 256) * (T / 256) >= 512) bm = bn = 256;
  const int np = V / bm;
  if (e->fwd_rr_nparts > 0) {  // the final norm deferred into the classifier
    p.rr_part = e->ssq_part; p.rr_ld = T; p.rr_nparts = e->fwd_rr_nparts; p.rr_dim = D;
    HIPCHK(op, eng_gemm(e, 4, e->embed_h, D, false, e->xh, D, false, V, T, D, EPI_CE_RR, p, bm, bn));
  } else {
    HIPCHK(op, eng_gemm(e, 4, e->embed_h, D, false, e->xh, D, false, V, T, D, EPI_CE, p, bm, bn));
  }
  prof_begin(e, 7);
  HIPCHK(op, ce_reduce(e->loss_seq, e->lse, e->tok_loss, colscale, dscale, e->partial, np, e->tgt_logit, e->tgt, V, nseq,
                       S, e->stream));
  prof_end(e, 0, (double)np * T * 8);
  return ANE_OK;
}

void drop_fwd_graph(ane_engine* e) {
  if (e->fwd_exec) (void)hipGraphExecDestroy(e->fwd_exec);
  e->fwd_exec = nullptr;
  e->fwd_graph_nseq = 0;
}

// Eval forward + classifier loss of nseq sequences whose tokens and targets
// are already in e->tok / e->tgt.  The ~90 launches of one call are captured
// once per batch size and replayed as a graph, which removes their host-side
// launch cost and the gaps it leaves between dependent kernels.  Profiling
// (events between the kernels) runs eagerly.
static int fwd_loss(ane_engine* e, int nseq) {
  const char* op = "eval loss";
  if (!e->use_graph || e->prof_on) {
    int rc = forward_body(e, nseq, 0, true);
    if (!rc) rc = head_loss(e, nseq, nullptr, 0.f);
    return rc;
  }
  if (!e->fwd_exec || e->fwd_graph_nseq != nseq) {
    drop_fwd_graph(e);
    HIPCHK(op, hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    int rc = forward_body(e, nseq, 0, true);
    if (!rc) rc = head_loss(e, nseq, nullptr, 0.f);
    hipGraph_t g = nullptr;
    const hipError_t h = hipStreamEndCapture(e->stream, &g);  // always leaves capture mode
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    HIPCHK(op, h);
    const hipError_t hi = hipGraphInstantiate(&e->fwd_exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (hi != hipSuccess) e->fwd_exec = nullptr;
    HIPCHK(op, hi);
    e->fwd_graph_nseq = nseq;
  }
  HIPCHK(op, hipGraphLaunch(e->fwd_exec, e->stream));
  return ANE_OK;
}

static int finish_loss(ane_engine* e, int nseq, float* loss_per_seq, float* mean_loss) {
  const char* op = "eval loss";
  const float* ls = e->loss_host;
  HIPCHK(op, hipMemcpyAsync(e->loss_host, e->loss_seq, (size_t)nseq * 4, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(op, stream_wait(e->stream));
  double tot = 0;
  for (int b = 0; b < nseq; b++) {
    tot += ls[b];
    if (loss_per_seq) loss_per_seq[b] = ls[b];
  }
  if (mean_loss) *mean_loss = nseq > 0 ? (float)(tot / nseq) : 0.f;
  return ANE_OK;
}

extern "C" int ane_eval_loss(ane_engine* e, const uint16_t* tokens, const uint16_t* targets, int32_t nseq,
                             float* loss_per_seq, float* mean_loss) {
  CLOSED_CHECK("eval loss");
  HIPCHK("eval loss", join_update(e));  // an asynchronous update still running
  if (nseq <= 0 || nseq > e->opt.max_batch || !tokens || !targets)
    return eng_fail(e, ANE_ERR_ARG, "storiesane eval loss: nseq=%d must be in [1, %d]", nseq, e->opt.max_batch);
  const size_t T = (size_t)nseq * e->cfg.seq;
  HIPCHK("eval loss", hipMemcpyAsync(e->tok, tokens, T * 2, hipMemcpyHostToDevice, e->stream));
  HIPCHK("eval loss", hipMemcpyAsync(e->tgt, targets, T * 2, hipMemcpyHostToDevice, e->stream));
  int rc = fwd_loss(e, nseq);
  if (!rc) rc = finish_loss(e, nseq, loss_per_seq, mean_loss);
  return rc;
}

int load_windows(ane_engine* e, const uint64_t* positions, int nseq) {
  const char* op = "eval loss";
  if (!e->data) return eng_fail(e, ANE_ERR_STATE, "storiesane step: not enough tokens");
  const uint64_t S = (uint64_t)e->cfg.seq;
  for (int b = 0; b < nseq; b++)
    if (positions[b] + S + 1 > (uint64_t)e->ndata)
      return eng_fail(e, ANE_ERR_ARG, "storiesane eval loss: window %d at %llu exceeds %lld tokens", b,
                      (unsigned long long)positions[b], (long long)e->ndata);
  if (nseq <= kArgWindows) {
    HIPCHK(op, gather_windows_args(e->tok, e->tgt, e->data, positions, nseq, e->cfg.seq, e->stream));
  } else {
    HIPCHK(op, hipMemcpyAsync(e->pos_d, positions, (size_t)nseq * 8, hipMemcpyHostToDevice, e->stream));
    HIPCHK(op, gather_windows(e->tok, e->tgt, e->data, e->pos_d, nseq, e->cfg.seq, e->stream));
  }
  return ANE_OK;
}

extern "C" int ane_eval_loss_windows(ane_engine* e, const uint64_t* positions, int32_t nseq, float* loss_per_seq,
                                     float* mean_loss) {
  CLOSED_CHECK("eval loss");
  HIPCHK("eval loss", join_update(e));  // an asynchronous update still running
  if (nseq <= 0 || nseq > e->opt.max_batch || !positions)
    return eng_fail(e, ANE_ERR_ARG, "storiesane eval loss: nseq=%d must be in [1, %d]", nseq, e->opt.max_batch);
  int rc = load_windows(e, positions, nseq);
  if (!rc) rc = fwd_loss(e, nseq);
  if (!rc) rc = finish_loss(e, nseq, loss_per_seq, mean_loss);
  return rc;
}

extern "C" int ane_eval_logits(ane_engine* e, const uint16_t* tokens, int64_t ntok, float* logits) {
  CLOSED_CHECK("eval logits");
  HIPCHK("eval logits", join_update(e));  // an asynchronous update still running
  if (ntok != e->cfg.seq || !tokens)
    return eng_fail(e, ANE_ERR_ARG, "storiesane eval logits: token len=%lld want=%d", (long long)ntok, e->cfg.seq);
  if (!logits) return eng_fail(e, ANE_ERR_ARG, "storiesane eval logits: null output");
  const char* op = "eval logits";
  const ane_model_cfg& c = e->cfg;
  const int D = c.dim, V = c.vocab, S = c.seq;
  HIPCHK(op, hipMemcpyAsync(e->tok, tokens, (size_t)S * 2, hipMemcpyHostToDevice, e->stream));
  int rc = forward_body(e, 1, 0);
  if (rc) return rc;
  EpiParams p;
  p.C = e->logits; p.ldc = S; p.softcap = c.arch == ANE_ARCH_NANOCHAT; p.cap = 15.f;
  HIPCHK(op, eng_gemm(e, 4, e->embed_h, D, false, e->xh, D, false, V, S, D, EPI_LOGITS, p));
  HIPCHK(op, hipMemcpyAsync(logits, e->logits, (size_t)V * S * 4, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(op, stream_wait(e->stream));
  return ANE_OK;
}

// ---------------------------------------------------------------------------
// profiling API
// ---------------------------------------------------------------------------
extern "C" int ane_profile_enable(ane_engine* e, int on) {
  CLOSED_CHECK("profile");
  e->prof_on = on != 0;
  return ANE_OK;
}

extern "C" int ane_profile_read(ane_engine* e, ane_prof_entry* out, int max, int reset) {
  CLOSED_CHECK("profile");
  HIPCHK("profile", hipStreamSynchronize(e->stream));
  for (size_t i = 0; i < e->prof_next; i++) {
    ProfEvent& pe = e->prof_events[i];
    float ms = 0.f;
    HIPCHK("profile", hipEventElapsedTime(&ms, pe.a, pe.b));
    ane_prof_entry& a = e->prof_acc[pe.cls];
    a.launches++;
    a.ms += ms;
    a.flops += pe.flops;
    a.bytes += pe.bytes;
  }
  e->prof_next = 0;
  for (int i = 0; i < max && i < ANE_PROF_CLASSES; i++) out[i] = e->prof_acc[i];
  if (reset)
    for (int i = 0; i < ANE_PROF_CLASSES; i++) e->prof_acc[i] = ane_prof_entry{0, 0, 0, 0};
  return ANE_OK;
}

// ---------------------------------------------------------------------------
// kernel-level diagnostics (unit tests of single kernels; no engine)
// ---------------------------------------------------------------------------
static std::string g_debug_err;

static int debug_fail(const char* what, hipError_t h) {
  g_debug_err = std::string("storiesane debug: ") + what + ": " + hipGetErrorString(h);
  return ANE_ERR_HIP;
}

#define DBGCHK(expr)                                  \
  do {                                                \
    hipError_t _h = (expr);                           \
    if (_h != hipSuccess) { rc = debug_fail(#expr, _h); goto done; } \
  } while (0)

extern "C" const char* ane_debug_last_error(void) { return g_debug_err.c_str(); }

// The argument structs of the code objects' kernels as compiled here (the C
// mirrors of ane_kernels.h are checked against them where the kernels are).
extern "C" int ane_kernel_abi(const char* name, int64_t* size, int64_t* offsets, int max) {
  if (!name || !size) return -1;
  std::vector<int64_t> off;
#define ANE_FIELD(T, f) off.push_back((int64_t)offsetof(T, f))
  if (!strcmp(name, "AneGemmArgs")) {
    *size = (int64_t)sizeof(GemmArgs);
    ANE_FIELD(GemmArgs, A); ANE_FIELD(GemmArgs, B); ANE_FIELD(GemmArgs, lda); ANE_FIELD(GemmArgs, ldb);
    ANE_FIELD(GemmArgs, M); ANE_FIELD(GemmArgs, N); ANE_FIELD(GemmArgs, K); ANE_FIELD(GemmArgs, a_t);
    ANE_FIELD(GemmArgs, b_t); ANE_FIELD(GemmArgs, grp); ANE_FIELD(GemmArgs, b_group_stride);
    ANE_FIELD(GemmArgs, splits); ANE_FIELD(GemmArgs, ws); ANE_FIELD(GemmArgs, pf); ANE_FIELD(GemmArgs, pf_bytes);
  } else if (!strcmp(name, "AneEpiParams")) {
    *size = (int64_t)sizeof(EpiParams);
    ANE_FIELD(EpiParams, C); ANE_FIELD(EpiParams, ldc); ANE_FIELD(EpiParams, C2); ANE_FIELD(EpiParams, ldc2);
    ANE_FIELD(EpiParams, R); ANE_FIELD(EpiParams, X0); ANE_FIELD(EpiParams, alpha); ANE_FIELD(EpiParams, beta);
    ANE_FIELD(EpiParams, scale); ANE_FIELD(EpiParams, alpha_ptr); ANE_FIELD(EpiParams, beta_ptr);
    ANE_FIELD(EpiParams, accumulate); ANE_FIELD(EpiParams, seq); ANE_FIELD(EpiParams, targets);
    ANE_FIELD(EpiParams, partial); ANE_FIELD(EpiParams, tgt_logit); ANE_FIELD(EpiParams, lse);
    ANE_FIELD(EpiParams, colscale); ANE_FIELD(EpiParams, softcap); ANE_FIELD(EpiParams, cap);
    ANE_FIELD(EpiParams, vocab); ANE_FIELD(EpiParams, C3); ANE_FIELD(EpiParams, rowscale); ANE_FIELD(EpiParams, gain);
    ANE_FIELD(EpiParams, ssq_part); ANE_FIELD(EpiParams, ssq_ld); ANE_FIELD(EpiParams, rr_part);
    ANE_FIELD(EpiParams, rr_ld); ANE_FIELD(EpiParams, rr_nparts); ANE_FIELD(EpiParams, rr_dim);
  } else if (!strcmp(name, "AneAttnArgs")) {
    *size = (int64_t)sizeof(AttnArgs);
    ANE_FIELD(AttnArgs, qkv); ANE_FIELD(AttnArgs, out); ANE_FIELD(AttnArgs, lse); ANE_FIELD(AttnArgs, rope_cos);
    ANE_FIELD(AttnArgs, rope_sin); ANE_FIELD(AttnArgs, nseq); ANE_FIELD(AttnArgs, S); ANE_FIELD(AttnArgs, NH);
    ANE_FIELD(AttnArgs, qknorm); ANE_FIELD(AttnArgs, scale); ANE_FIELD(AttnArgs, ve_x); ANE_FIELD(AttnArgs, ve_gate);
    ANE_FIELD(AttnArgs, ve_embed); ANE_FIELD(AttnArgs, tokens); ANE_FIELD(AttnArgs, vocab); ANE_FIELD(AttnArgs, qkvt);
    ANE_FIELD(AttnArgs, qkvt_lo); ANE_FIELD(AttnArgs, hilo); ANE_FIELD(AttnArgs, pf); ANE_FIELD(AttnArgs, pf_bytes);
    ANE_FIELD(AttnArgs, split_from);
  } else {
    return -1;
  }
#undef ANE_FIELD
  for (int i = 0; i < (int)off.size() && i < max && offsets; i++) offsets[i] = off[i];
  return (int)off.size();
}

extern "C" int ane_debug_gemm(int a_t, int b_t, int epi, int M, int N, int K, const uint16_t* A, const uint16_t* B,
                              void* C, int bm, int bn, int nw, int ns, int splits) {
  if (epi != EPI_STORE_F && epi != EPI_STORE_H) {
    g_debug_err = "storiesane debug: epilogue must be STORE_F or STORE_H";
    return ANE_ERR_ARG;
  }
  int rc = ANE_OK;
  void *dA = nullptr, *dB = nullptr, *dC = nullptr, *dW = nullptr;
  const size_t esz = epi == EPI_STORE_F ? 4 : 2;
  GemmArgs g;
  EpiParams p;
  if (splits < 1) splits = 1;
  DBGCHK(hipMalloc(&dA, (size_t)M * K * 2));
  DBGCHK(hipMalloc(&dB, (size_t)N * K * 2));
  DBGCHK(hipMalloc(&dC, (size_t)M * N * esz));
  if (splits > 1) DBGCHK(hipMalloc(&dW, (size_t)splits * M * N * 4));
  g.splits = splits;
  g.ws = (float*)dW;
  DBGCHK(hipMemcpy(dA, A, (size_t)M * K * 2, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dB, B, (size_t)N * K * 2, hipMemcpyHostToDevice));
  g.A = (const half_t*)dA; g.B = (const half_t*)dB;
  g.lda = a_t ? M : K; g.ldb = b_t ? N : K;
  g.M = M; g.N = N; g.K = K; g.a_t = a_t != 0; g.b_t = b_t != 0;
  p.C = dC; p.ldc = N;
  DBGCHK(gemm_run(g, epi, p, nullptr, bm, bn, nw, ns));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipMemcpy(C, dC, (size_t)M * N * esz, hipMemcpyDeviceToHost));
done:
  if (dA) (void)hipFree(dA);
  if (dB) (void)hipFree(dB);
  if (dC) (void)hipFree(dC);
  if (dW) (void)hipFree(dW);
  return rc;
}

// One K-major GEMM (A [M, K], B [N, K]) with a fused forward epilogue on
// host buffers.  Element types and shapes by epilogue:
//   STORE_H, RELU2: C fp16 [M, N];  RELU2: C2 fp16 [M, N] (pre-activation)
//   SWIGLU: C fp16 [M, N/2] over 32-column interleaved W1|W3, C2 fp16 [M, N]
//   STORE_F, LOGITS (softcap = 15 when seq < 0), RESID, SMEAR: C fp32 [M, N]
//   RESID: R fp32 [M, N] (C = alpha R + acc + beta X0; X0 optional; C2 fp32
//          copy optional);  SMEAR: X0 fp32 [M, N], rows t with t % seq == 0
//          have no predecessor, C2 fp32 gate
// C2 / X0 / R may be NULL where optional.
extern "C" int ane_debug_gemm_epi(int epi, int M, int N, int K, const uint16_t* A, const uint16_t* B, void* C,
                                  void* C2, const float* X0, const float* R, float alpha, float beta, int seq, int bm,
                                  int bn, int nw) {
  const bool f32 = epi == EPI_STORE_F || epi == EPI_LOGITS || epi == EPI_RESID || epi == EPI_SMEAR;
  if (!f32 && epi != EPI_STORE_H && epi != EPI_RELU2 && epi != EPI_SWIGLU) {
    g_debug_err = "storiesane debug: unsupported epilogue";
    return ANE_ERR_ARG;
  }
  if ((epi == EPI_RESID && !R) || (epi == EPI_SMEAR && (!X0 || seq <= 0))) {
    g_debug_err = "storiesane debug: missing epilogue operand";
    return ANE_ERR_ARG;
  }
  int rc = ANE_OK;
  void *dA = nullptr, *dB = nullptr, *dC = nullptr, *dC2 = nullptr, *dX0 = nullptr, *dR = nullptr;
  const size_t MN = (size_t)M * N;
  const size_t cbytes = epi == EPI_SWIGLU ? MN : (f32 ? MN * 4 : MN * 2);
  const size_t c2bytes = (epi == EPI_RESID || epi == EPI_SMEAR) ? MN * 4 : MN * 2;
  GemmArgs g;
  EpiParams p;
  DBGCHK(hipMalloc(&dA, (size_t)M * K * 2));
  DBGCHK(hipMalloc(&dB, (size_t)N * K * 2));
  DBGCHK(hipMalloc(&dC, cbytes));
  DBGCHK(hipMemcpy(dA, A, (size_t)M * K * 2, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dB, B, (size_t)N * K * 2, hipMemcpyHostToDevice));
  if (C2) DBGCHK(hipMalloc(&dC2, c2bytes));
  if (X0) {
    DBGCHK(hipMalloc(&dX0, MN * 4));
    DBGCHK(hipMemcpy(dX0, X0, MN * 4, hipMemcpyHostToDevice));
  }
  if (R) {
    DBGCHK(hipMalloc(&dR, MN * 4));
    DBGCHK(hipMemcpy(dR, R, MN * 4, hipMemcpyHostToDevice));
  }
  g.A = (const half_t*)dA; g.B = (const half_t*)dB;
  g.lda = K; g.ldb = K; g.M = M; g.N = N; g.K = K; g.a_t = false; g.b_t = false;
  p.C = dC; p.ldc = epi == EPI_SWIGLU ? N / 2 : N;
  p.C2 = dC2; p.ldc2 = N;
  p.X0 = (const float*)dX0; p.R = (const float*)dR;
  p.alpha = alpha; p.beta = beta; p.seq = seq;
  if (epi == EPI_LOGITS && seq < 0) { p.softcap = 1; p.cap = 15.f; }
  DBGCHK(gemm_run(g, epi, p, nullptr, bm, bn, nw, 0));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipMemcpy(C, dC, cbytes, hipMemcpyDeviceToHost));
  if (C2) DBGCHK(hipMemcpy(C2, dC2, c2bytes, hipMemcpyDeviceToHost));
done:
  for (void* q : {dA, dB, dC, dC2, dX0, dR})
    if (q) (void)hipFree(q);
  return rc;
}

// The deferred-RMSNorm epilogues on one forced tile (host buffers).
// epi 13 (EPI_RESID_NORM): X [M, N] fp32 in/out (X += acc), C [M, N] fp16 =
// X * gain[col], ssq [N / bn][M] = per-row sums of X^2 over each block's bn
// columns.  epi 14 (EPI_STORE_H_RR): C [M, N] fp16 = acc * rr[row]; epi 15
// (EPI_SWIGLU_RR): C [M, N / 2] fp16 = SwiGLU of the interleaved W1|W3
// columns of acc * rr[row]; rr = 1 / sqrt(sum of rr_part[p][row] over
// p < nparts / rr_dim + 1e-5).
extern "C" int ane_debug_gemm_norm(int epi, int M, int N, int K, const uint16_t* A, const uint16_t* B, float* X,
                                   uint16_t* C, const float* gain, float* ssq, const float* rr_part, int nparts,
                                   int rr_dim, int bm, int bn, int nw) {
  if ((epi != EPI_RESID_NORM && epi != EPI_STORE_H_RR && epi != EPI_SWIGLU_RR) || bm <= 0 || bn <= 0 ||
      (epi == EPI_RESID_NORM && (!X || !gain || !ssq)) || (epi != EPI_RESID_NORM && (!rr_part || nparts < 1))) {
    g_debug_err = "storiesane debug: unsupported deferred-norm epilogue or missing operand";
    return ANE_ERR_ARG;
  }
  int rc = ANE_OK;
  void *dA = nullptr, *dB = nullptr, *dC = nullptr, *dX = nullptr, *dG = nullptr, *dS = nullptr, *dP = nullptr;
  const size_t MN = (size_t)M * N;
  const size_t cbytes = epi == EPI_SWIGLU_RR ? MN : MN * 2;
  const size_t sbytes = (size_t)(N / bn) * M * 4;
  GemmArgs g;
  EpiParams p;
  DBGCHK(hipMalloc(&dA, (size_t)M * K * 2));
  DBGCHK(hipMalloc(&dB, (size_t)N * K * 2));
  DBGCHK(hipMalloc(&dC, cbytes));
  DBGCHK(hipMemcpy(dA, A, (size_t)M * K * 2, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dB, B, (size_t)N * K * 2, hipMemcpyHostToDevice));
  if (epi == EPI_RESID_NORM) {
    DBGCHK(hipMalloc(&dX, MN * 4));
    DBGCHK(hipMalloc(&dG, (size_t)N * 4));
    DBGCHK(hipMalloc(&dS, sbytes));
    DBGCHK(hipMemcpy(dX, X, MN * 4, hipMemcpyHostToDevice));
    DBGCHK(hipMemcpy(dG, gain, (size_t)N * 4, hipMemcpyHostToDevice));
    p.C = dX; p.ldc = N; p.R = (const float*)dX; p.C2 = dC; p.ldc2 = N; p.gain = (const float*)dG;
    p.ssq_part = (float*)dS; p.ssq_ld = M;
  } else {
    DBGCHK(hipMalloc(&dP, (size_t)nparts * M * 4));
    DBGCHK(hipMemcpy(dP, rr_part, (size_t)nparts * M * 4, hipMemcpyHostToDevice));
    p.C = dC; p.ldc = epi == EPI_SWIGLU_RR ? N / 2 : N;
    p.rr_part = (const float*)dP; p.rr_ld = M; p.rr_nparts = nparts; p.rr_dim = rr_dim;
  }
  g.A = (const half_t*)dA; g.B = (const half_t*)dB;
  g.lda = K; g.ldb = K; g.M = M; g.N = N; g.K = K; g.a_t = false; g.b_t = false;
  DBGCHK(gemm_run(g, epi, p, nullptr, bm, bn, nw, 0));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipMemcpy(C, dC, cbytes, hipMemcpyDeviceToHost));
  if (epi == EPI_RESID_NORM) {
    DBGCHK(hipMemcpy(X, dX, MN * 4, hipMemcpyDeviceToHost));
    DBGCHK(hipMemcpy(ssq, dS, sbytes, hipMemcpyDeviceToHost));
  }
done:
  for (void* q : {dA, dB, dC, dX, dG, dS, dP})
    if (q) (void)hipFree(q);
  return rc;
}

// The classifier epilogues on one forced tile (host buffers): EPI_CE writes
// per-(block row, column) partials (max, sum exp(v - max)) and the target
// logit of every column; with lse given, EPI_DLOGITS then writes the
// vocab-major dlogits dl [M, N] and, when dl_t is given, the token-major
// copy [N, M].  A [M, K] = classifier rows (vocabulary), B [N, K] = tokens.
extern "C" int ane_debug_classifier(int M, int N, int K, const uint16_t* A, const uint16_t* B,
                                    const uint16_t* targets, int softcap, int vocab, int bm, int bn, int nw,
                                    float* part_max, float* part_sum, float* tgt_logit, const float* lse,
                                    const float* colscale, uint16_t* dl, uint16_t* dl_t) {
  if (bm <= 0 || bn <= 0 || M % bm || N % bn || !A || !B || !targets || !part_max || !part_sum || !tgt_logit ||
      (lse && (!colscale || !dl))) {
    g_debug_err = "storiesane debug classifier: tile must divide M, N; operands missing";
    return ANE_ERR_ARG;
  }
  int rc = ANE_OK;
  const size_t MN = (size_t)M * N, np = (size_t)(M / bm) * N;
  void *dA = nullptr, *dB = nullptr, *dT = nullptr, *dP = nullptr, *dTL = nullptr, *dL = nullptr, *dS = nullptr,
       *dC = nullptr, *dC2 = nullptr;
  std::vector<float2> part(np);
  GemmArgs g;
  EpiParams p;
  DBGCHK(hipMalloc(&dA, (size_t)M * K * 2));
  DBGCHK(hipMalloc(&dB, (size_t)N * K * 2));
  DBGCHK(hipMalloc(&dT, (size_t)N * 2));
  DBGCHK(hipMalloc(&dP, np * sizeof(float2)));
  DBGCHK(hipMalloc(&dTL, (size_t)N * 4));
  DBGCHK(hipMemcpy(dA, A, (size_t)M * K * 2, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dB, B, (size_t)N * K * 2, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dT, targets, (size_t)N * 2, hipMemcpyHostToDevice));
  DBGCHK(hipMemset(dTL, 0xff, (size_t)N * 4));  // NaN: a column whose target no lane claimed stays NaN
  g.A = (const half_t*)dA; g.B = (const half_t*)dB;
  g.lda = K; g.ldb = K; g.M = M; g.N = N; g.K = K; g.a_t = false; g.b_t = false;
  p.targets = (const uint16_t*)dT; p.partial = (float2*)dP; p.tgt_logit = (float*)dTL;
  p.softcap = softcap != 0; p.cap = 15.f; p.vocab = vocab;
  DBGCHK(gemm_run(g, EPI_CE, p, nullptr, bm, bn, nw, 0));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipMemcpy(part.data(), dP, np * sizeof(float2), hipMemcpyDeviceToHost));
  DBGCHK(hipMemcpy(tgt_logit, dTL, (size_t)N * 4, hipMemcpyDeviceToHost));
  for (size_t i = 0; i < np; i++) {
    part_max[i] = part[i].x;
    part_sum[i] = part[i].y;
  }
  if (lse) {
    DBGCHK(hipMalloc(&dL, (size_t)N * 4));
    DBGCHK(hipMalloc(&dS, (size_t)N * 4));
    DBGCHK(hipMalloc(&dC, MN * 2));
    if (dl_t) DBGCHK(hipMalloc(&dC2, MN * 2));
    DBGCHK(hipMemcpy(dL, lse, (size_t)N * 4, hipMemcpyHostToDevice));
    DBGCHK(hipMemcpy(dS, colscale, (size_t)N * 4, hipMemcpyHostToDevice));
    EpiParams q;
    q.targets = (const uint16_t*)dT; q.lse = (const float*)dL; q.colscale = (const float*)dS;
    q.softcap = softcap != 0; q.cap = 15.f; q.vocab = vocab;
    q.C = dC; q.ldc = N; q.C2 = dC2; q.ldc2 = M;
    DBGCHK(gemm_run(g, EPI_DLOGITS, q, nullptr, bm, bn, nw, 0));
    DBGCHK(hipDeviceSynchronize());
    DBGCHK(hipMemcpy(dl, dC, MN * 2, hipMemcpyDeviceToHost));
    if (dl_t) DBGCHK(hipMemcpy(dl_t, dC2, MN * 2, hipMemcpyDeviceToHost));
  }
done:
  for (void* q : {dA, dB, dT, dP, dTL, dL, dS, dC, dC2})
    if (q) (void)hipFree(q);
  return rc;
}

__global__ void debug_fill_kernel(half_t* p, size_t n, uint32_t seed) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint32_t x = (uint32_t)i * 2654435761u ^ seed;
    x ^= x >> 15; x *= 2246822519u; x ^= x >> 13;
    p[i] = (half_t)(((float)(x & 0xffff) / 65536.0f - 0.5f));
  }
}

// Times `iters` launches of one GEMM with HIP events; *avg_ms receives the
// mean launch time.  Operands: the host arrays A, B (stored as for
// ane_debug_gemm) when given, else pseudo-random values in [-0.5, 0.5).
extern "C" int ane_debug_gemm_bench(int a_t, int b_t, int epi, int M, int N, int K, int bm, int bn, int nw,
                                    int ns, int splits, int iters, const uint16_t* A, const uint16_t* B,
                                    float* avg_ms) {
  if (epi != EPI_STORE_F && epi != EPI_STORE_H && epi != EPI_RESID && epi != EPI_SWIGLU && epi != EPI_CE &&
      epi != EPI_RESID_NORM && !epi_rr(epi)) {
    g_debug_err = "storiesane debug: epilogue must be STORE_F, STORE_H, RESID, SWIGLU, CE or a deferred-norm form";
    return ANE_ERR_ARG;
  }
  int rc = ANE_OK;
  void *dA = nullptr, *dB = nullptr, *dC = nullptr, *dX = nullptr, *dW = nullptr, *dN = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  GemmArgs g;
  EpiParams p;
  float ms = 0.f;
  if (splits < 1) splits = 1;
  DBGCHK(hipMalloc(&dA, (size_t)M * K * 2));
  DBGCHK(hipMalloc(&dB, (size_t)N * K * 2));
  DBGCHK(hipMalloc(&dC, (size_t)M * N * 4));
  if (splits > 1) DBGCHK(hipMalloc(&dW, (size_t)splits * M * N * 4));
  g.splits = splits;
  g.ws = (float*)dW;
  // CE side buffers: targets (zeros), per-64-row-block partials, target logits
  if (epi == EPI_CE || epi == EPI_CE_RR) {
    DBGCHK(hipMalloc(&dX, (size_t)N * 2 + (size_t)(M / 64) * N * sizeof(float2) + (size_t)N * 4 + 256));
    DBGCHK(hipMemset(dX, 0, (size_t)N * 2));
  }
  // deferred-norm side buffers (zeros): partials [16][max(M, N)], gain [N], ssq [16][M], fp16 copy [M, N]
  if (epi == EPI_RESID_NORM || epi_rr(epi)) {
    const size_t nside = (size_t)kRrMaxParts * (M > N ? M : N) + (size_t)N + (size_t)kRrMaxParts * M + (size_t)M * N;
    DBGCHK(hipMalloc(&dN, nside * 4));
    DBGCHK(hipMemset(dN, 0, nside * 4));
  }
  if (A) DBGCHK(hipMemcpy(dA, A, (size_t)M * K * 2, hipMemcpyHostToDevice));
  else hipLaunchKernelGGL(debug_fill_kernel, dim3(1024), dim3(256), 0, nullptr, (half_t*)dA, (size_t)M * K, 1u);
  if (B) DBGCHK(hipMemcpy(dB, B, (size_t)N * K * 2, hipMemcpyHostToDevice));
  else hipLaunchKernelGGL(debug_fill_kernel, dim3(1024), dim3(256), 0, nullptr, (half_t*)dB, (size_t)N * K, 2u);
  DBGCHK(hipGetLastError());
  DBGCHK(hipEventCreate(&e0));
  DBGCHK(hipEventCreate(&e1));
  g.A = (const half_t*)dA; g.B = (const half_t*)dB;
  g.lda = a_t ? M : K; g.ldb = b_t ? N : K;
  g.M = M; g.N = N; g.K = K; g.a_t = a_t != 0; g.b_t = b_t != 0;
  p.C = dC; p.ldc = N;
  if (epi == EPI_RESID || epi == EPI_RESID_NORM) p.R = (const float*)dC;
  if (epi == EPI_SWIGLU || epi == EPI_SWIGLU_RR) p.ldc = N / 2;
  if (dN) {
    float* f = (float*)dN;
    p.rr_part = f; p.rr_ld = M > N ? M : N; p.rr_nparts = 12; p.rr_dim = 768;
    f += (size_t)kRrMaxParts * p.rr_ld;
    p.gain = f;
    f += N;
    p.ssq_part = f; p.ssq_ld = M;
    f += (size_t)kRrMaxParts * M;
    if (epi == EPI_RESID_NORM) {  // its fp16 x * gain output (the rr forms have no second output here)
      p.C2 = f;
      p.ldc2 = N;
    }
  }
  if (epi == EPI_CE || epi == EPI_CE_RR) {
    char* x = (char*)dX;
    p.targets = (const uint16_t*)x;
    p.partial = (float2*)(x + (((size_t)N * 2 + 255) & ~(size_t)255));
    p.tgt_logit = (float*)((char*)p.partial + (size_t)(M / 64) * N * sizeof(float2));
    p.vocab = M;
  }
  DBGCHK(gemm_run(g, epi, p, nullptr, bm, bn, nw, ns));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipEventRecord(e0, nullptr));
  for (int i = 0; i < iters; i++) DBGCHK(gemm_run(g, epi, p, nullptr, bm, bn, nw, ns));
  DBGCHK(hipEventRecord(e1, nullptr));
  DBGCHK(hipEventSynchronize(e1));
  DBGCHK(hipEventElapsedTime(&ms, e0, e1));
  *avg_ms = ms / (float)(iters > 0 ? iters : 1);
done:
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (dA) (void)hipFree(dA);
  if (dB) (void)hipFree(dB);
  if (dC) (void)hipFree(dC);
  if (dX) (void)hipFree(dX);
  if (dW) (void)hipFree(dW);
  if (dN) (void)hipFree(dN);
  return rc;
}

extern "C" int ane_debug_transpose2(int Ra, int Ca, const uint16_t* in_a, uint16_t* out_a, int Rb, int Cb,
                                    const uint16_t* in_b, uint16_t* out_b) {
  int rc = ANE_OK;
  const size_t na = (size_t)Ra * Ca, nb = in_b ? (size_t)Rb * Cb : 0;
  void *dia = nullptr, *doa = nullptr, *dib = nullptr, *dob = nullptr;
  if (Ra <= 0 || Ca <= 0 || Ra % 64 || Ca % 64 || !in_a || !out_a ||
      (in_b && (Rb <= 0 || Cb <= 0 || Rb % 64 || Cb % 64 || !out_b)))
    return debug_fail("transpose2: shapes must be positive multiples of 64", hipErrorInvalidValue);
  DBGCHK(hipMalloc(&dia, na * 2));
  DBGCHK(hipMalloc(&doa, na * 2));
  DBGCHK(hipMemcpy(dia, in_a, na * 2, hipMemcpyHostToDevice));
  if (nb) {
    DBGCHK(hipMalloc(&dib, nb * 2));
    DBGCHK(hipMalloc(&dob, nb * 2));
    DBGCHK(hipMemcpy(dib, in_b, nb * 2, hipMemcpyHostToDevice));
  }
  DBGCHK(transpose2_h((half_t*)doa, (const half_t*)dia, Ra, Ca, Ca, Ra, (half_t*)dob, (const half_t*)dib, Rb, Cb, Cb,
                      Rb, nullptr));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipMemcpy(out_a, doa, na * 2, hipMemcpyDeviceToHost));
  if (nb) DBGCHK(hipMemcpy(out_b, dob, nb * 2, hipMemcpyDeviceToHost));
done:
  if (dia) (void)hipFree(dia);
  if (doa) (void)hipFree(doa);
  if (dib) (void)hipFree(dib);
  if (dob) (void)hipFree(dob);
  return rc;
}

extern "C" int ane_debug_norm_bwd(int T, int D, const float* dy, const float* x, const float* gain,
                                  const float* addend, float alpha, float* out, uint16_t* out_h, float* dgain_part,
                                  int general) {
  int rc = ANE_OK;
  if (T <= 0 || D <= 0 || D % 64 || D > 1024 || !dy || !x || !gain || !out || !dgain_part)
    return debug_fail("norm_bwd: T > 0, D a multiple of 64 up to 1024, dy / x / gain / out / dgain_part given",
                      hipErrorInvalidValue);
  const size_t n = (size_t)T * D, nb = (size_t)norm_bwd_blocks(T);
  float *ddy = nullptr, *dx = nullptr, *dg = nullptr, *dad = nullptr, *dout = nullptr, *dpart = nullptr;
  half_t* douth = nullptr;
  NormBwdArgs a;
  DBGCHK(hipMalloc(&ddy, n * 4));
  DBGCHK(hipMalloc(&dx, n * 4));
  DBGCHK(hipMalloc(&dg, (size_t)D * 4));
  DBGCHK(hipMalloc(&dout, n * 4));
  DBGCHK(hipMalloc(&dpart, nb * D * 4));
  DBGCHK(hipMemcpy(ddy, dy, n * 4, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dx, x, n * 4, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dg, gain, (size_t)D * 4, hipMemcpyHostToDevice));
  if (addend) {
    DBGCHK(hipMalloc(&dad, n * 4));
    DBGCHK(hipMemcpy(dad, addend, n * 4, hipMemcpyHostToDevice));
  }
  if (out_h) DBGCHK(hipMalloc(&douth, n * 2));
  a.dy = ddy; a.x = dx; a.gain = dg; a.dgain_part = dpart; a.addend = dad; a.alpha = alpha;
  a.out = dout; a.out_h = douth; a.T = T; a.D = D; a.general = general;
  DBGCHK(norm_bwd(a, nullptr));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipMemcpy(out, dout, n * 4, hipMemcpyDeviceToHost));
  DBGCHK(hipMemcpy(dgain_part, dpart, nb * D * 4, hipMemcpyDeviceToHost));
  if (out_h) DBGCHK(hipMemcpy(out_h, douth, n * 2, hipMemcpyDeviceToHost));
done:
  for (void* p : {(void*)ddy, (void*)dx, (void*)dg, (void*)dad, (void*)dout, (void*)dpart, (void*)douth})
    if (p) (void)hipFree(p);
  return rc;
}

extern "C" int ane_debug_attention(int nseq, int S, int NH, int qknorm, double theta, float scale, int hilo,
                                   const uint16_t* qkv, uint16_t* out, float* lse) {
  int rc = ANE_OK;
  const int D = 64 * NH;
  const size_t T = (size_t)nseq * S;
  void *dq = nullptr, *dout = nullptr, *dc = nullptr, *ds = nullptr, *dl = nullptr;
  std::vector<float> cs((size_t)S * 32), sn((size_t)S * 32);
  AttnArgs a;
  memset(&a, 0, sizeof a);
  for (int pos = 0; pos < S; pos++)
    for (int i = 0; i < 32; i++) {
      double f = (double)pos / pow(theta, (double)(2 * i) / 64.0);
      cs[(size_t)pos * 32 + i] = (float)cos(f);
      sn[(size_t)pos * 32 + i] = (float)sin(f);
    }
  DBGCHK(hipMalloc(&dq, T * 3 * D * 2));
  DBGCHK(hipMalloc(&dout, T * D * 2));
  DBGCHK(hipMalloc(&dc, cs.size() * 4));
  DBGCHK(hipMalloc(&ds, sn.size() * 4));
  DBGCHK(hipMalloc(&dl, T * NH * 4));
  DBGCHK(hipMemcpy(dq, qkv, T * 3 * D * 2, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(dc, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  DBGCHK(hipMemcpy(ds, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  a.qkv = (const half_t*)dq; a.out = (half_t*)dout; a.lse = (float*)dl;
  a.rope_cos = (const float*)dc; a.rope_sin = (const float*)ds;
  a.nseq = nseq; a.S = S; a.NH = NH; a.qknorm = qknorm; a.scale = scale; a.hilo = hilo;
  DBGCHK(attention_fwd(a, nullptr));
  DBGCHK(hipDeviceSynchronize());
  DBGCHK(hipMemcpy(out, dout, T * D * 2, hipMemcpyDeviceToHost));
  if (lse) DBGCHK(hipMemcpy(lse, dl, T * NH * 4, hipMemcpyDeviceToHost));
done:
  if (dq) (void)hipFree(dq);
  if (dout) (void)hipFree(dout);
  if (dc) (void)hipFree(dc);
  if (ds) (void)hipFree(ds);
  if (dl) (void)hipFree(dl);
  return rc;
}
