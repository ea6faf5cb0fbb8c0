// Engine state shared by the host-side translation units of libane_hip.
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/ane_hip.h"
#include "gemm.h"
#include "train_ops.h"

struct LayerOff {
  int64_t wq = -1, wk = -1, wv = -1, wo = -1, w1 = -1, w2 = -1, w3 = -1, g_att = -1, g_ffn = -1, ve_embed = -1,
          ve_gate = -1;
};
struct ParamMap {
  std::vector<LayerOff> L;
  int64_t embed = -1, resid = -1, x0l = -1, smear_gate = -1, smear_lambda = -1, backout_lambda = -1,
          g_final = -1, total = 0;
};
void build_param_map(const ane_model_cfg& c, ParamMap* m);

struct LayerShadow {
  ane::half_t* wqkv = nullptr;  // [3D, D]: Wq | Wk | Wv
  ane::half_t* wo = nullptr;    // [D, D]
  ane::half_t* w13 = nullptr;   // llama2: [2H, D] W1/W3 interleaved by 32 rows; nanochat: W1 [H, D]
  ane::half_t* w2 = nullptr;    // [D, H]
  // transposes for the backward's dX GEMMs (training only): B operands
  // read K-major with K = the forward's output dimension
  ane::half_t* wqkv_t = nullptr;  // [D, 3D]
  ane::half_t* wo_t = nullptr;    // [D, D]
  ane::half_t* w13_t = nullptr;   // [D, 2H] (columns in the interleaved W1|W3 order) or [D, H]
  ane::half_t* w2_t = nullptr;    // [H, D]
};

// activations one layer keeps for its backward ([T, C] token-major)
struct LayerActs {
  float* xin = nullptr;         // layer input (fp32 residual stream)
  ane::half_t* xn = nullptr;    // RMSNorm(xin), QKV GEMM operand
  ane::half_t* qkv = nullptr;   // [T, 3D] projections (pre-RoPE)
  ane::half_t* qkvt = nullptr;  // [T, 3D] q, k after RoPE / QK-norm, v after VE
  ane::half_t* qk_lo = nullptr; // [T, 2D] fp16 residuals of those q, k (reference-compat backward)
  ane::half_t* att = nullptr;   // attention output
  float* lse = nullptr;         // [T, NH]
  float* x2 = nullptr;          // residual after attention
  ane::half_t* xn2 = nullptr;   // RMSNorm(x2)
  ane::half_t* h13 = nullptr;   // FFN pre-activations ([T, 2H] interleaved W1|W3, or [T, H])
  ane::half_t* gate = nullptr;  // FFN activation, W2 operand
};

struct TrainBufs {
  std::vector<LayerActs> L;
  float* xlast = nullptr;   // output of the last layer
  float* xfinal = nullptr;  // nanochat: after backout
  float* sg_act = nullptr;  // nanochat: smear gate sigmoid
  ane::half_t* x0h = nullptr;
  // gradients and optimizer state (canonical layout)
  float* G = nullptr;
  float* M = nullptr;
  float* Vv = nullptr;
  // backward scratch
  float* dcur = nullptr;
  ane::half_t* dcur_h = nullptr;
  float* dx2 = nullptr;
  ane::half_t* dx2_h = nullptr;
  float* dxn = nullptr;
  ane::half_t* dh13 = nullptr;
  ane::half_t* datt = nullptr;
  ane::half_t* dqkv = nullptr;
  float* delta = nullptr;
  ane::half_t* att1 = nullptr;  // compat: scale-1 attention output
  float* lse1 = nullptr;
  ane::half_t* dl = nullptr;    // [V, T] dlogits
  ane::half_t* dl_t = nullptr;  // [T, V] the same, token-major
  // transposed GEMM operands of the weight gradients ([C, T], K = T)
  ane::half_t* op_a = nullptr;  // [max(2H, 3D), T]
  ane::half_t* op_b = nullptr;  // [max(H, D), T]
  float* splitk_ws = nullptr;   // split-K partials of the backward GEMMs
  size_t splitk_cap = 0;        // floats
  // weight gradients on the dW stream: its own split-K workspace, and a
  // second copy of each activation gradient they read, so that layer l and
  // layer l - 1 use different buffers (index = layer parity)
  float* splitk_ws2 = nullptr;
  ane::half_t* dcur_h2 = nullptr;
  ane::half_t* dh13_2 = nullptr;
  ane::half_t* dx2_h2 = nullptr;
  ane::half_t* dqkv2 = nullptr;
  float* colscale = nullptr;
  float* gx0 = nullptr;
  float* ginj = nullptr;
  float* ve_dx = nullptr;
  ane::half_t* dgp = nullptr;
  float* dgain_part = nullptr;
  // llama2: per-layer gain-gradient partials [2 L][nblocks][D] (FFN norm
  // 2 l, attention norm 2 l + 1), so their reductions can run on the dW
  // stream while the main stream's next norms write other partials
  float* dgain_parts = nullptr;
  double* dot_part = nullptr;
  double* sumsq = nullptr;
  double* sumsq_part = nullptr;
};

struct ProfEvent {
  hipEvent_t a = nullptr, b = nullptr;
  int cls = 0;
  double flops = 0, bytes = 0;
};

// drand48 (ane/engine.go:177-181, 873-880)
inline uint64_t drand48_seed(int64_t seed) { return (((uint64_t)seed & 0xffffffffULL) << 16) | 0x330EULL; }
inline double drand48_next(uint64_t* st) {
  *st = (0x5DEECE66DULL * *st + 0xBULL) & ((1ULL << 48) - 1);
  return (double)*st / (double)(1ULL << 48);
}

struct ane_engine {
  ane_model_cfg cfg{};
  ane_options opt{};
  int device = 0;
  bool dev_set = false;
  bool closed = false;
  std::string err;
  hipStream_t stream = nullptr;
  std::vector<void*> allocs;
  ParamMap pm;

  // weights
  float* P = nullptr;  // fp32 masters, canonical layout
  ane::half_t* shadow = nullptr;
  std::vector<LayerShadow> ls;
  ane::half_t* embed_h = nullptr;  // [V, D]
  ane::half_t* smear_h = nullptr;  // [D, D]
  ane::half_t* embed_t = nullptr;  // [D, V] (training)
  ane::half_t* smear_t = nullptr;  // [D, D] (training)
  // shadow refresh job table (device), rebuilt when the transposes appear
  ane::ShadowJob* shadow_jobs = nullptr;
  int n_shadow_jobs = 0, n_shadow_tiles = 0;
  std::vector<ane::ShadowJob> shadow_jobs_h;  // host copy of the table
  // the flush's fused AdamW + shadow update (ANE_FUSED_ADAM=0: AdamW, then
  // the fp32 -> fp16 refresh, then a fill of the gradient): job table on the
  // device, built for the segment list in upd_sig
  bool fused_adam = true;
  ane::UpdateJob* upd_jobs = nullptr;
  int n_upd_jobs = 0, n_upd_blocks = 0, upd_cap = 0;
  std::vector<int64_t> upd_sig;
  // The table is ordered by update chunk: chunk 0 = the model-level groups
  // (embedding, final gain; nanochat's smear and residual scalars), chunk
  // 1 + l = layer l's groups; chunk c is jobs [upd_j0[c], upd_j0[c] + upd_nj[c])
  // and blocks [upd_b0[c], upd_b0[c] + upd_nb[c]).
  std::vector<int> upd_j0, upd_nj, upd_b0, upd_nb;
  // Asynchronous update (accumulate-mode flushes with the dW stream;
  // ANE_ASYNC_UPDATE=0: in line on the main stream): the gradient norm and
  // the chunks run on the dW stream behind the backward, upd_ev[c] marking
  // chunk c done, while the call returns once the losses are in.  The next
  // training forward waits on the GPU for chunk 0 before the embedding and
  // for chunk 1 + l before layer l; every other entry point that launches
  // work waits for the whole update first (join_update).
  bool async_update = true;
  std::vector<hipEvent_t> upd_ev;
  bool upd_pending = false;
  // StepResult.AdamDuration of an asynchronous update: the step_ev pair is
  // read once complete (adam_unread until then); adam_ns_last keeps the
  // latest completed update's duration
  bool adam_unread = false;
  int64_t adam_ns_last = 0;
  bool shadow_jobs_t = false;
  float* rope_cos = nullptr;
  float* rope_sin = nullptr;

  // token stream (Options.Tokens) and per-call windows
  uint16_t* data = nullptr;
  int64_t ndata = 0;
  uint16_t* tok = nullptr;
  uint16_t* tgt = nullptr;
  uint64_t* pos_d = nullptr;

  // activations ([T, C] token-major)
  float* x = nullptr;
  float* x0 = nullptr;
  float* xpre = nullptr;
  float* xmid = nullptr;
  ane::half_t* xh = nullptr;
  ane::half_t* qkv = nullptr;
  ane::half_t* att = nullptr;
  ane::half_t* gate = nullptr;
  // deferred RMSNorm of the llama2 eval forward (default; ANE_FUSED_NORM=0
  // runs the norm launches, see forward_body): per-row partial sums of
  // squares [kRrMaxParts][T] behind xh = fp16(x * gain); fwd_rr_nparts > 0
  // when the last forward left its final norm to the classifier this way
  float* ssq_part = nullptr;
  bool fused_norm = true;
  // the classifier's weights by a prefetch launch before it (ANE_FUSED_PF=1;
  // off: 2.643-2.653 against 2.650-2.657 ms per B32 forward, seven
  // alternating pairs, since the self-prefetching GEMMs and the 1.5-head
  // attention)
  bool fused_pf = false;
  // the deferred-norm forward's GEMMs stream weights from their first
  // blocks (GemmArgs::pf): W1|W3 its own and W2's, W2 the next layer's
  // Wq|Wk|Wv (ANE_GEMM_SELFPF=0: a prefetch launch before QKV and W1|W3)
  bool gemm_selfpf = true;
  bool tr_dw = true;  // weight gradients read token-major operands directly (ANE_TR_DW=0: transposes)
  // The backward's weight-gradient GEMMs run on a second stream beside the
  // activation-gradient chain (ANE_DW_ASYNC=0: all on one stream).  Events
  // order the two: the dW stream waits for the producer of each dY, and the
  // main stream waits, once per layer, for the dW work of the layer above
  // before it overwrites a buffer that work reads.
  bool dw_async = true;
  bool bwd_prefetch = true;  // ANE_BWD_PREFETCH=0: no prefetch of the backward's GEMM operands
  hipStream_t dw_stream = nullptr;
  // asynchronous weight refresh of an accumulate-mode flush (the transposed
  // shadows, on the dW stream; startAsyncRefresh, ane/runtime.go:71-83): the
  // next backward waits for refresh_ev[1] on the GPU, Flush on the host,
  // returning its duration (waitAsyncRefresh, ane/runtime.go:85-94)
  hipEvent_t refresh_ev[2] = {};
  bool refresh_pending = false;
  std::vector<hipEvent_t> xev;  // fork / join events (timing disabled), reused per call
  size_t xev_next = 0;
  int fwd_rr_nparts = 0;
  int ce_bm = 256, ce_np = 0;  // smallest classifier block row and the partial rows it needs
  float2* partial = nullptr;
  float* tgt_logit = nullptr;
  float* lse = nullptr;
  float* tok_loss = nullptr;
  float* loss_seq = nullptr;
  float* loss_host = nullptr;  // pinned copy of loss_seq: the read-back is one queued copy and one wait
  float* logits = nullptr;  // [V, S]

  // host-side engine state (ane/engine.go:76-175)
  ane_state state{};
  uint64_t rng = 0;
  float lr = 0.f;
  bool train_ready = false;
  TrainBufs tr;
  double start_s = 0.0;  // wall clock at open (CumWallMS)
  // step start, final head start / end, end of the backward, Adam start / end
  enum { EV_STEP0 = 0, EV_HEAD0, EV_HEAD1, EV_BWD1, EV_ADAM0, EV_ADAM1, EV_COUNT };
  hipEvent_t step_ev[EV_COUNT] = {};
  bool flushed = false;
  // phase timers of one training call (StepResult, ane/engine.go:55-69):
  // event pairs around kernel groups, summed per phase after the call
  std::vector<hipEvent_t> ph_ev;  // pool, grown on the host outside any graph capture
  std::vector<int> ph_cls;        // phase of each recorded pair
  int ph_used = 0;
  bool ph_open = false;
  // An event recorded between kernels costs ~4 us of idle GPU (0.47 ms on an
  // 8.4 ms B16 step), so the kernel-group phases are timed on the first
  // training call and every ph_period-th after it (ANE_PHASE_EVERY, default
  // 16); the other calls report the latest measurement.  The weight refresh
  // (one pair per update) is timed on every call.
  bool ph_sample = false;
  int ph_period = 16;
  uint64_t ph_calls = 0;
  int64_t ph_last_ns[4] = {0, 0, 0, 0};  // latest embed_grad, rms_dw, dw_gemm, per window
  int64_t startup_ns = 0;  // host time of this call's one-time training set-up

  // eval forward + loss replayed as one HIP graph per batch size with
  // ANE_GRAPHS=1 (the kernels read only buffers fixed at open); by default
  // they are launched eagerly, which measured as fast (B32, same box: 2.456
  // against 2.470 ms per call) and is the form rocprofv3 traces cleanly
  bool use_graph = false;
  hipGraphExec_t fwd_exec = nullptr;
  int fwd_graph_nseq = 0;

  // profiling
  bool prof_on = false;
  std::vector<ProfEvent> prof_events;
  size_t prof_next = 0;
  ane_prof_entry prof_acc[ANE_PROF_CLASSES] = {};
};

int eng_fail(ane_engine* e, int code, const char* fmt, ...);

#define HIPCHK(op, expr)                                                                             \
  do {                                                                                               \
    hipError_t _h = (expr);                                                                          \
    if (_h != hipSuccess) return eng_fail(e, ANE_ERR_HIP, "storiesane %s: %s: %s", op, #expr,        \
                                          hipGetErrorString(_h));                                    \
  } while (0)

#define CLOSED_CHECK(op)                                                                          \
  do {                                                                                            \
    if (!e) return ANE_ERR_CLOSED;                                                                \
    if (e->closed) return eng_fail(e, ANE_ERR_CLOSED, "storiesane %s: engine is closed", op);     \
  } while (0)
void prof_begin(ane_engine* e, int cls, hipStream_t s = nullptr);
void prof_end(ane_engine* e, double flops, double bytes, hipStream_t s = nullptr);
// side = run on the dW stream with its own split-K workspace; pf / pf_bytes:
// bytes the GEMM's first blocks stream through the caches with their
// prologue loads (GemmArgs::pf; ignored past its limit)
hipError_t eng_gemm(ane_engine* e, int cls, const ane::half_t* A, int lda, bool at, const ane::half_t* B, int ldb,
                    bool bt, int M, int N, int K, int epi, const ane::EpiParams& p, int bm = 0, int bn = 0,
                    bool side = false, const void* pf = nullptr, size_t pf_bytes = 0);
int refresh_shadows(ane_engine* e);
// the update job table of adam_fused_update for the segments of a (cached),
// in chunk order (AdamSeg::chunk)
int ensure_update_jobs(ane_engine* e, const ane::AdamArgs& a);
// An asynchronous update still pending: the main stream waits for all of it
// (join_update) or for chunk c (wait_update); both are no-ops otherwise.
hipError_t join_update(ane_engine* e);
hipError_t wait_update(ane_engine* e, int chunk);
int forward_body(ane_engine* e, int nseq, int train, bool defer_norm = false);
void drop_fwd_graph(ane_engine* e);
template <class T>
hipError_t dalloc(ane_engine* e, T** p, size_t n) {
  void* q = nullptr;
  hipError_t r = hipMalloc(&q, n * sizeof(T) > 0 ? n * sizeof(T) : 16);
  if (r == hipSuccess) {
    e->allocs.push_back(q);
    *p = (T*)q;
  }
  return r;
}
int head_loss(ane_engine* e, int nseq, float* colscale, float dscale);
enum StepPhase { PH_EMBED_GRAD = 0, PH_RMS_DW, PH_DW_GEMM, PH_REFRESH, PH_COUNT };
void phase_reset(ane_engine* e);
void phase_begin(ane_engine* e, int phase, hipStream_t s = nullptr);
void phase_end(ane_engine* e, hipStream_t s = nullptr);
// after the stream has drained: milliseconds per phase
void phase_sum(ane_engine* e, double ms[PH_COUNT]);
int load_windows(ane_engine* e, const uint64_t* positions, int nseq);
