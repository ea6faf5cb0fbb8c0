// Training: backward pass, gradient accumulation, clipping and AdamW, and
// the Step / Flush / SetLR / State entry points of the C-ABI.
//
// Follows the reference's CPU path (backwardAndAccumulate / backwardAndApply,
// ane/train_full.go:691-967; runFinalHead, :480-558; flushPending,
// ane/engine.go:646-682) on the device:
//  * the loss seed is dlogits = (softmax - onehot) * lossScale / valid per
//    sequence (times the softcap derivative for nanochat), so every
//    activation gradient carries the loss scale, as in the reference;
//  * weight gradients are summed over all sequences of a call by the dW
//    GEMMs (reduction over T = nseq * seq) and accumulate into one fp32
//    gradient vector in the canonical parameter layout;
//  * a flush scales by 1 / (pending * lossScale), clips the global L2 norm of
//    the layer + embedding gradients, and applies AdamW with the reference's
//    parameter groups, then rebuilds the fp16 weight shadows.
// dlogits are stored fp16 times kDlScale (so probabilities ~1e-5 stay
// normal fp16 numbers); the two GEMMs that consume them divide it out.
#include <math.h>
#include <string.h>
#include <time.h>

#include <initializer_list>
#include <utility>
#include <vector>

#include "attention.h"
#include "engine_internal.h"
#include "gemm.h"
#include "rowops.h"
#include "train_ops.h"

using namespace ane;

namespace {

constexpr float kDlScale = 64.f;

double now_s() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int ensure_train(ane_engine* e, const char* op) {
  if (e->train_ready) return ANE_OK;
  const double t_start = now_s();
  drop_fwd_graph(e);  // eng_gemm may pick other shapes once the split-K workspace exists
  const ane_model_cfg& c = e->cfg;
  const bool llama = c.arch == ANE_ARCH_LLAMA2;
  const size_t D = c.dim, H = c.hidden, V = c.vocab, NH = c.heads;
  const size_t T = (size_t)e->opt.max_batch * c.seq;
  const size_t KH = llama ? 2 * H : H;
  if (c.seq > 256)
    return eng_fail(e, ANE_ERR_ARG, "storiesane %s: training supports seq <= 256 (got %d)", op, c.seq);
  TrainBufs& tb = e->tr;
  tb.L.assign(c.layers, LayerActs());
  for (int l = 0; l < c.layers; l++) {
    LayerActs& A = tb.L[l];
    HIPCHK(op, dalloc(e, &A.xin, T * D));
    HIPCHK(op, dalloc(e, &A.xn, T * D));
    HIPCHK(op, dalloc(e, &A.qkv, T * 3 * D));
    HIPCHK(op, dalloc(e, &A.qkvt, T * 3 * D));
    if (!llama && c.grad_mode == ANE_GRAD_COMPAT) HIPCHK(op, dalloc(e, &A.qk_lo, T * 2 * D));
    HIPCHK(op, dalloc(e, &A.att, T * D));
    HIPCHK(op, dalloc(e, &A.lse, T * NH));
    HIPCHK(op, dalloc(e, &A.x2, T * D));
    HIPCHK(op, dalloc(e, &A.xn2, T * D));
    HIPCHK(op, dalloc(e, &A.h13, T * KH));
    HIPCHK(op, dalloc(e, &A.gate, T * H));
  }
  HIPCHK(op, dalloc(e, &tb.xlast, T * D));
  if (!llama) {
    HIPCHK(op, dalloc(e, &tb.xfinal, T * D));
    HIPCHK(op, dalloc(e, &tb.sg_act, T * D));
    HIPCHK(op, dalloc(e, &tb.x0h, T * D));
    HIPCHK(op, dalloc(e, &tb.gx0, T * D));
    HIPCHK(op, dalloc(e, &tb.ginj, T * D));
    HIPCHK(op, dalloc(e, &tb.ve_dx, T * 12));
    HIPCHK(op, dalloc(e, &tb.dgp, T * D));
    HIPCHK(op, dalloc(e, &tb.att1, T * D));
    HIPCHK(op, dalloc(e, &tb.lse1, T * NH));
  }
  const size_t P = (size_t)e->pm.total;
  HIPCHK(op, dalloc(e, &tb.G, P));
  HIPCHK(op, dalloc(e, &tb.M, P));
  HIPCHK(op, dalloc(e, &tb.Vv, P));
  HIPCHK(op, fill_f32(tb.G, P, 0.f, e->stream));
  HIPCHK(op, fill_f32(tb.M, P, 0.f, e->stream));
  HIPCHK(op, fill_f32(tb.Vv, P, 0.f, e->stream));
  HIPCHK(op, dalloc(e, &tb.dcur, T * D));
  HIPCHK(op, dalloc(e, &tb.dcur_h, T * D));
  HIPCHK(op, dalloc(e, &tb.dx2, T * D));
  HIPCHK(op, dalloc(e, &tb.dx2_h, T * D));
  HIPCHK(op, dalloc(e, &tb.dxn, T * D));
  HIPCHK(op, dalloc(e, &tb.dh13, T * KH));
  HIPCHK(op, dalloc(e, &tb.datt, T * D));
  HIPCHK(op, dalloc(e, &tb.dqkv, T * 3 * D));
  HIPCHK(op, dalloc(e, &tb.delta, T * NH));
  HIPCHK(op, dalloc(e, &tb.dl, V * T));
  HIPCHK(op, dalloc(e, &tb.dl_t, V * T));
  {
    const size_t ca = KH > 3 * D ? KH : 3 * D, cb = H > D ? H : D;
    HIPCHK(op, dalloc(e, &tb.op_a, ca * T));
    HIPCHK(op, dalloc(e, &tb.op_b, cb * T));
    // split-K workspace: 8 slices of the largest backward output
    size_t mx = T * D;
    for (size_t v : {(size_t)D * H, (size_t)KH * D, (size_t)3 * D * D}) mx = v > mx ? v : mx;
    tb.splitk_cap = 8 * mx;
    HIPCHK(op, dalloc(e, &tb.splitk_ws, tb.splitk_cap));
  }
  if (e->dw_async && e->tr_dw) {
    // default priority, like the main stream
    if (!e->dw_stream) HIPCHK(op, hipStreamCreateWithFlags(&e->dw_stream, hipStreamNonBlocking));
    for (hipEvent_t& ev : e->refresh_ev)
      if (!ev) HIPCHK(op, hipEventCreate(&ev));
    // update chunk events: ordering between the two streams only
    while ((int)e->upd_ev.size() < 1 + c.layers) {
      hipEvent_t x = nullptr;
      HIPCHK(op, hipEventCreateWithFlags(&x, hipEventDisableTiming | hipEventDisableSystemFence));
      e->upd_ev.push_back(x);
    }
    HIPCHK(op, dalloc(e, &tb.splitk_ws2, tb.splitk_cap));
    HIPCHK(op, dalloc(e, &tb.dcur_h2, T * D));
    HIPCHK(op, dalloc(e, &tb.dh13_2, T * KH));
    HIPCHK(op, dalloc(e, &tb.dx2_h2, T * D));
    HIPCHK(op, dalloc(e, &tb.dqkv2, T * 3 * D));
  }
  // transposed weight shadows, filled by the refresh below
  for (int l = 0; l < c.layers; l++) {
    LayerShadow& s = e->ls[l];
    HIPCHK(op, dalloc(e, &s.wqkv_t, 3 * D * D));
    HIPCHK(op, dalloc(e, &s.wo_t, D * D));
    HIPCHK(op, dalloc(e, &s.w13_t, KH * D));
    HIPCHK(op, dalloc(e, &s.w2_t, H * D));
  }
  if (!llama) HIPCHK(op, dalloc(e, &e->smear_t, D * D));
  HIPCHK(op, dalloc(e, &e->embed_t, V * D));
  HIPCHK(op, dalloc(e, &tb.colscale, T));
  const size_t nblk = (size_t)norm_bwd_blocks((int)T);
  HIPCHK(op, dalloc(e, &tb.dgain_part, nblk * D));
  if (llama) HIPCHK(op, dalloc(e, &tb.dgain_parts, 2 * (size_t)c.layers * nblk * D));
  HIPCHK(op, dalloc(e, &tb.dot_part, (nblk > 256 ? nblk : 256) * 2));
  HIPCHK(op, dalloc(e, &tb.sumsq, 1));
  HIPCHK(op, dalloc(e, &tb.sumsq_part, kSumsqBlocks));
  for (hipEvent_t& ev : e->step_ev) HIPCHK(op, hipEventCreate(&ev));
  int rc = refresh_shadows(e);
  if (rc) return rc;
  HIPCHK(op, hipStreamSynchronize(e->stream));
  e->train_ready = true;
  // the one-time set-up the reference's Prepare() does (StartupCompileDuration)
  e->startup_ns += (int64_t)((now_s() - t_start) * 1e9);
  return ANE_OK;
}

// Forward + backward of the nseq sequences in e->tok / e->tgt; ADDS the
// loss-scaled gradient sum to tr.G and leaves per-sequence losses in
// e->loss_seq.
// Weight gradient dW += dY^T X over the T tokens of the step, dY [T][M] and
// X [T][N] token-major as the backward leaves them.  By default the GEMM
// reads them as they are (M-major operands through transposing LDS reads);
// with ANE_TR_DW=0 both are first transposed into K-major staging buffers
// and the K-major kernel runs (the same products; measured slower by the
// transposes' HBM round trip).
hipError_t dw_gemm(ane_engine* e, int cls, const half_t* dY, int M, const half_t* X, int N, int T, int epi,
                   const EpiParams& p, bool side = false) {
  TrainBufs& tb = e->tr;
  if (e->tr_dw) return eng_gemm(e, cls, dY, M, true, X, N, true, M, N, T, epi, p, 0, 0, side);
  if (side) return hipErrorInvalidValue;  // the staging buffers belong to the main stream
  hipError_t h = transpose2_h(tb.op_a, dY, T, M, M, T, tb.op_b, X, T, N, N, T, e->stream);
  if (h != hipSuccess) return h;
  return eng_gemm(e, cls, tb.op_a, T, false, tb.op_b, T, false, M, N, T, epi, p);
}

// An event of the fork / join pool: created on first use (on the host,
// never under capture), handed out in order and reused by the next call.
hipError_t next_xev(ane_engine* e, hipEvent_t* ev) {
  if (e->xev_next >= e->xev.size()) {
    hipEvent_t x = nullptr;
    // ordering between two streams of one device only: no system-scope
    // fence (each kernel's own release / acquire makes its results visible;
    // the fence costs ~3 us of idle GPU per record, 0.14 ms per B16 step)
    hipError_t h = hipEventCreateWithFlags(&x, hipEventDisableTiming | hipEventDisableSystemFence);
    if (h != hipSuccess) return h;
    e->xev.push_back(x);
  }
  *ev = e->xev[e->xev_next++];
  return hipSuccess;
}

// Marks the work given to stream `s` so far; *ev (if given) receives the
// event so that another stream can wait for it later.
hipError_t mark(ane_engine* e, hipStream_t s, hipEvent_t* ev) {
  hipEvent_t x = nullptr;
  hipError_t h = next_xev(e, &x);
  if (h == hipSuccess) h = hipEventRecord(x, s);
  if (h == hipSuccess && ev) *ev = x;
  return h;
}

// Stream `to` runs its later work after what `from` has been given so far.
hipError_t stream_after(ane_engine* e, hipStream_t to, hipStream_t from) {
  hipEvent_t x = nullptr;
  hipError_t h = mark(e, from, &x);
  return h == hipSuccess ? hipStreamWaitEvent(to, x, 0) : h;
}

int backward_body(ane_engine* e, int nseq, bool async);

// The backward with the weight gradients on the dW stream when enabled: the
// main stream waits for all of them before it returns, also on an error
// return, so that no later launch overwrites what they still read.
int backward_pass(ane_engine* e, int nseq) {
  const bool async = e->dw_async && e->tr_dw && e->dw_stream && e->tr.splitk_ws2;
  e->xev_next = 0;
  int rc = backward_body(e, nseq, async);
  if (async) {
    const hipError_t h = stream_after(e, e->stream, e->dw_stream);
    if (h != hipSuccess && rc == ANE_OK)
      rc = eng_fail(e, ANE_ERR_HIP, "storiesane step: dW stream join: %s", hipGetErrorString(h));
  }
  return rc;
}

int backward_body(ane_engine* e, int nseq, bool async) {
  const char* op = "step";
  const ane_model_cfg& c = e->cfg;
  const bool llama = c.arch == ANE_ARCH_LLAMA2;
  const bool compat = !llama && c.grad_mode == ANE_GRAD_COMPAT;
  const int D = c.dim, H = c.hidden, V = c.vocab, S = c.seq, NH = c.heads, L = c.layers;
  const int T = nseq * S, KH = llama ? 2 * H : H;
  const int nblk = norm_bwd_blocks(T);
  TrainBufs& tb = e->tr;
  const float* P = e->P;
  float* G = tb.G;
  hipStream_t st = e->stream;
  // weight gradients: on the dW stream (ds) or in line on the main stream
  hipStream_t ds = async ? e->dw_stream : st;
  const ParamMap& pm = e->pm;
  // activation gradients the dW GEMMs read: layer l uses copy (l & 1), so the
  // main stream may write layer l - 1's while layer l's dW GEMMs still run;
  // dcur_h(l) is the dY that enters layer l from above
  auto by_parity = [&](half_t* a, half_t* b, int l) { return async && (l & 1) ? b : a; };
  auto dcur_h_of = [&](int l) { return by_parity(tb.dcur_h, tb.dcur_h2, l); };
  auto gpart = [&](int i) { return tb.dgain_parts + (size_t)i * nblk * D; };
  // llama2, first backward of an accumulation window: every gradient writer
  // (the dW GEMMs, the classifier's gEmbed GEMM, the gain reductions)
  // overwrites its region instead of adding to it, so the flush's update need
  // not clear the gradient (nanochat's VE tables take atomic adds and keep
  // the clear)
  const bool fresh = llama && e->state.pending_steps == 0;
  const int acc = fresh ? 0 : 1;

  // Cold GEMM operands streamed into the caches by a prefetch kernel on the
  // dW stream at each fork: the weight shadow of the dX GEMM that the main
  // stream starts at the same time (the prefetch runs ahead of that GEMM's
  // k loop) and the saved activations of the dW GEMMs queued behind it.
  // Both were last read a step or a forward ago; with them cold, 64 blocks
  // meet each B panel at once and a 64x64-tile GEMM pays ~10 us (W1|W3 dX
  // and dW at B16).  A prefetch issued a few kernels earlier does not help:
  // the data in between evicts it.
  auto prefetch = [&](hipStream_t s, std::initializer_list<std::pair<const void*, size_t>> regions) -> hipError_t {
    if (!e->bwd_prefetch) return hipSuccess;
    PrefetchList pl;
    for (const auto& r : regions) pl.add(r.first, r.second);
    return prefetch_list(pl, s);
  };
  const size_t TD2 = (size_t)T * D * 2;

  int rc = forward_body(e, nseq, 1);
  if (rc) return rc;
  // the transposed shadows of an asynchronous refresh (waitAsyncRefresh at
  // the next step, ane/train_full.go:370-372): waited for on the GPU
  if (e->refresh_pending) {
    HIPCHK(op, hipStreamWaitEvent(st, e->refresh_ev[1], 0));
    e->refresh_pending = false;
  }

  // ---- final head (runFinalHead, ane/train_full.go:480-558) ----------------
  (void)hipEventRecord(e->step_ev[ane_engine::EV_HEAD0], st);
  rc = head_loss(e, nseq, tb.colscale, e->opt.loss_scale * kDlScale);
  if (rc) return rc;
  {
    // token-major dl_t for the dy GEMM (K = vocab); the vocab-major copy only
    // for the K-major embedding-gradient GEMM of ANE_TR_DW=0
    EpiParams p;
    p.C = e->tr_dw ? nullptr : tb.dl; p.ldc = T; p.C2 = tb.dl_t; p.ldc2 = V;
    p.targets = e->tgt; p.lse = e->lse; p.colscale = tb.colscale;
    p.softcap = !llama; p.cap = 15.f; p.vocab = V;
    HIPCHK(op, eng_gemm(e, 4, e->embed_h, D, false, e->xh, D, false, V, T, D, EPI_DLOGITS, p));
  }
  if (async) HIPCHK(op, stream_after(e, ds, st));  // dl, dl_t written
  {  // dy = Embed^T dlogits (MatMulEmbedTScale, ane/stories/cpu.go:333-360)
    EpiParams p;
    p.C = tb.dxn; p.ldc = D; p.scale = 1.f / kDlScale;
    HIPCHK(op, eng_gemm(e, 7, tb.dl_t, V, false, e->embed_t, V, false, T, D, V, EPI_STORE_F, p));
  }
  {  // classifier part of the embedding gradient (MatMulGradEmbedScale, ane/stories/cpu.go:366-385)
    EpiParams p;
    p.C = G + pm.embed; p.ldc = D; p.scale = 1.f / kDlScale; p.accumulate = acc;
    phase_begin(e, PH_EMBED_GRAD, ds);
    if (e->tr_dw) {  // dl_t and xh token-major, both read through transposing LDS loads
      HIPCHK(op, eng_gemm(e, 7, tb.dl_t, V, true, e->xh, D, true, V, D, T, EPI_STORE_F, p, 0, 0, async));
    } else {
      HIPCHK(op, transpose_h(tb.op_b, e->xh, T, D, D, T, st));
      HIPCHK(op, eng_gemm(e, 7, tb.dl, T, false, tb.op_b, T, false, V, D, T, EPI_STORE_F, p));
    }
    phase_end(e, ds);
  }
  {  // final RMSNorm backward (+ backout backward for nanochat)
    NormBwdArgs a;
    a.dy = tb.dxn; a.T = T; a.D = D; a.out = tb.dcur; a.out_h = dcur_h_of(L - 1);
    if (llama) {
      a.x = tb.xlast; a.gain = P + pm.g_final; a.dgain_part = tb.dgain_part;
    } else {
      a.x = tb.xfinal;
    }
    HIPCHK(op, norm_bwd(a, st));
    if (llama) {
      phase_begin(e, PH_RMS_DW);
      HIPCHK(op, reduce_partials_add(G + pm.g_final, tb.dgain_part, nblk, D, st, fresh));
      phase_end(e);
    } else {
      HIPCHK(op, backout_bwd(tb.ginj, tb.dot_part, tb.dcur, e->xmid, P + pm.backout_lambda, T, D, st));
      HIPCHK(op, reduce_dots_add(G + pm.backout_lambda, nullptr, tb.dot_part, 256, -1.f, st));
      HIPCHK(op, fill_f32(tb.gx0, (size_t)T * D, 0.f, st));
    }
  }
  (void)hipEventRecord(e->step_ev[ane_engine::EV_HEAD1], st);
  HIPCHK(op, prefetch(st, {{e->ls[L - 1].w2_t, (size_t)H * D * 2}}));

  // ---- layers, last to first ------------------------------------------------
  // dW stream order per layer: dW2 (after the SwiGLU-backward GEMM), dWo and
  // dW13 (after the FFN norm backward), dWqkv (after the attention backward);
  // above_done marks the end of the layer above's dW work
  hipEvent_t above_done = nullptr;
  int att_gain_layer = -1;
  for (int l = L - 1; l >= 0; l--) {
    const LayerOff& o = pm.L[l];
    const LayerShadow& s = e->ls[l];
    const LayerActs& A = tb.L[l];
    const float* rl_p = llama ? nullptr : P + pm.resid + l;
    const float* xl_p = llama ? nullptr : P + pm.x0l + l;
    half_t* dcur_in = dcur_h_of(l);
    half_t* dcur_out = dcur_h_of(l - 1);
    half_t* dh13 = by_parity(tb.dh13, tb.dh13_2, l);
    half_t* dx2_h = by_parity(tb.dx2_h, tb.dx2_h2, l);
    half_t* dqkv = by_parity(tb.dqkv, tb.dqkv2, l);
    // FFN (backwardFFNCPU, ane/train_full.go:592-601)
    {
      EpiParams p;
      p.C = dh13; p.ldc = KH; p.C2 = A.h13; p.ldc2 = KH;
      HIPCHK(op, eng_gemm(e, 3, dcur_in, D, false, s.w2_t, D, false, T, H, D,
                          llama ? EPI_SWIGLU_BWD : EPI_RELU2_BWD, p));
    }
    if (async) HIPCHK(op, stream_after(e, ds, st));  // dcur_in, dh13 written
    HIPCHK(op, prefetch(ds, {{s.w13_t, (size_t)KH * D * 2}, {A.xn2, TD2}, {A.gate, (size_t)T * H * 2}}));
    if (att_gain_layer >= 0) {  // the attention-norm gain of the layer above
      phase_begin(e, PH_RMS_DW, ds);
      HIPCHK(op, reduce_partials_add(G + pm.L[att_gain_layer].g_att, gpart(2 * att_gain_layer + 1), nblk, D, ds,
                                     fresh));
      phase_end(e, ds);
      att_gain_layer = -1;
    }
    auto dw2 = [&]() -> int {  // dW2 += dOut gate^T
      EpiParams p;
      p.C = G + o.w2; p.ldc = H; p.accumulate = acc;
      phase_begin(e, PH_DW_GEMM, ds);
      HIPCHK(op, dw_gemm(e, 3, dcur_in, D, A.gate, H, T, EPI_STORE_F, p, async));
      phase_end(e, ds);
      return ANE_OK;
    };
    auto dw13 = [&]() -> int {  // dW1 (| dW3) += dh x2Norm^T
      EpiParams p;
      p.C = G + o.w1; p.ldc = D; p.accumulate = acc;
      if (llama) p.C3 = G + o.w3;
      phase_begin(e, PH_DW_GEMM, ds);
      HIPCHK(op, dw_gemm(e, 2, dh13, KH, A.xn2, D, T, llama ? EPI_STORE_W13 : EPI_STORE_F, p, async));
      phase_end(e, ds);
      return ANE_OK;
    };
    if ((rc = dw2())) return rc;
    {
      EpiParams p;
      p.C = tb.dxn; p.ldc = D;
      HIPCHK(op, eng_gemm(e, 2, dh13, KH, false, s.w13_t, KH, false, T, D, KH, EPI_STORE_F, p));
    }
    {  // dx2 = rl * dOut + RMSNorm-backward(dxn2; x2)
      NormBwdArgs a;
      a.dy = tb.dxn; a.x = A.x2; a.T = T; a.D = D; a.addend = tb.dcur; a.alpha_p = rl_p;
      a.out = tb.dx2; a.out_h = dx2_h;
      if (llama) {
        a.gain = P + o.g_ffn; a.dgain_part = gpart(2 * l);
      } else {
        a.lam_x = A.x2; a.lam_x0 = e->x0; a.lam_part = tb.dot_part; a.gx0 = tb.gx0; a.xl_p = xl_p;
      }
      HIPCHK(op, norm_bwd(a, st));
      if (async) HIPCHK(op, stream_after(e, ds, st));  // dx2_h and the FFN gain partials written
      HIPCHK(op, prefetch(ds, {{s.wo_t, (size_t)D * D * 2}, {A.att, TD2}}));
      if (llama) {
        phase_begin(e, PH_RMS_DW, ds);
        HIPCHK(op, reduce_partials_add(G + o.g_ffn, gpart(2 * l), nblk, D, ds, fresh));
        phase_end(e, ds);
      } else
        HIPCHK(op, reduce_dots_add(G + pm.resid + l, G + pm.x0l + l, tb.dot_part, nblk, 1.f, st));
    }
    // attention (backwardAttentionCPU, ane/train_full.go:644-675)
    {
      EpiParams p;
      p.C = G + o.wo; p.ldc = D; p.accumulate = acc;
      phase_begin(e, PH_DW_GEMM, ds);
      HIPCHK(op, dw_gemm(e, 1, dx2_h, D, A.att, D, T, EPI_STORE_F, p, async));
      phase_end(e, ds);
    }
    // dW1|3 behind dWo: beside the Wo dX GEMM and the attention backward
    // rather than the W1|W3 dX GEMM (6.55-6.58 against 6.60-6.63 ms per B16
    // step with it at the first fork)
    if ((rc = dw13())) return rc;
    {
      EpiParams p;
      p.C = tb.datt; p.ldc = D;
      HIPCHK(op, eng_gemm(e, 1, dx2_h, D, false, s.wo_t, D, false, T, D, D, EPI_STORE_H, p));
    }
    {
      AttnBwdArgs b;
      memset(&b, 0, sizeof b);
      b.qkv = A.qkv; b.qkvt = A.qkvt; b.dout = tb.datt; b.delta = tb.delta; b.dqkv = dqkv;
      b.rope_cos = e->rope_cos; b.rope_sin = e->rope_sin; b.nseq = nseq; b.S = S; b.NH = NH;
      b.qknorm = llama ? 0 : 1;
      if (compat) {
        // the reference's backward recomputes the probabilities with scale
        // 1.0 (ane/train_full.go:268-269): its O and lse come from a scale-1 forward
        AttnArgs f;
        memset(&f, 0, sizeof f);
        f.qkv = A.qkv; f.out = tb.att1; f.lse = tb.lse1; f.rope_cos = e->rope_cos; f.rope_sin = e->rope_sin;
        f.nseq = nseq; f.S = S; f.NH = NH; f.qknorm = 1; f.scale = 1.0f;
        // scale-1 scores reach |q.k| ~ 1.44 * 64: fp16 rounding of q and k
        // would move them by ~0.05, so both passes use split operands
        f.hilo = 1;
        if (o.ve_embed >= 0) {
          f.ve_x = A.xin; f.ve_gate = P + o.ve_gate; f.ve_embed = P + o.ve_embed; f.tokens = e->tok; f.vocab = V;
        }
        prof_begin(e, 5);
        HIPCHK(op, attention_fwd(f, st));
        prof_end(e, 0, 0);
        b.o = tb.att1; b.lse = tb.lse1; b.scale_p = 1.f; b.scale_ds = 1.f; b.qk_coef2 = 1.2f * 1.2f; b.rope_bwd = 0;
        b.qkvt_lo = A.qk_lo; b.hilo = 1;
      } else {
        b.o = A.att; b.lse = A.lse; b.scale_p = 0.125f; b.scale_ds = 0.125f; b.qk_coef2 = 1.2f; b.rope_bwd = 1;
      }
      prof_begin(e, 5);
      HIPCHK(op, attention_bwd(b, st));
      prof_end(e, 2.5 * 4.0 * 64 * NH * (double)nseq * ((double)S * (S + 1) / 2), 0);
    }
    if (async) HIPCHK(op, stream_after(e, ds, st));  // dqkv written
    HIPCHK(op, prefetch(ds, {{s.wqkv_t, (size_t)3 * D * D * 2}, {A.xn, TD2}}));
    {  // dWq | dWk | dWv += dqkv xNorm^T
      EpiParams p;
      p.C = G + o.wq; p.ldc = D; p.accumulate = acc;
      phase_begin(e, PH_DW_GEMM, ds);
      HIPCHK(op, dw_gemm(e, 0, dqkv, 3 * D, A.xn, D, T, EPI_STORE_F, p, async));
      phase_end(e, ds);
    }
    hipEvent_t this_done = nullptr;
    if (async) HIPCHK(op, mark(e, ds, &this_done));
    if (o.ve_embed >= 0)
      HIPCHK(op, ve_bwd(G + o.ve_embed, G + o.ve_gate, tb.ve_dx, dqkv + 2 * D, 3 * D, A.xin, P + o.ve_embed,
                        P + o.ve_gate, e->tok, T, D, NH, V, st));
    {
      EpiParams p;
      p.C = tb.dxn; p.ldc = D;
      HIPCHK(op, eng_gemm(e, 0, dqkv, 3 * D, false, s.wqkv_t, 3 * D, false, T, D, 3 * D, EPI_STORE_F, p));
    }
    // dcur_out is the copy the layer above's dW2 read: wait for that layer's
    // dW work (which also covers its dh13, dx2_h and dqkv copies, written
    // again by the layer below)
    if (above_done) HIPCHK(op, hipStreamWaitEvent(st, above_done, 0));
    above_done = this_done;
    {  // dPrev = rl * dx2 + RMSNorm-backward(dxn; x) (+ VE gate grads, + backout injection)
      NormBwdArgs a;
      a.dy = tb.dxn; a.x = A.xin; a.T = T; a.D = D; a.addend = tb.dx2; a.alpha_p = rl_p;
      a.out = tb.dcur; a.out_h = dcur_out;
      if (llama) {
        a.gain = P + o.g_att; a.dgain_part = gpart(2 * l + 1);
      } else {
        a.lam_x = A.xin; a.lam_x0 = e->x0; a.lam_part = tb.dot_part; a.gx0 = tb.gx0; a.xl_p = xl_p;
        if (o.ve_embed >= 0) a.ve_dx = tb.ve_dx;
        if (l == L / 2) a.addend2 = tb.ginj;  // ane/train_full.go:784-787
      }
      HIPCHK(op, norm_bwd(a, st));
      if (llama && async && l > 0) {
        att_gain_layer = l;  // reduced on the dW stream after the next fork
      } else if (llama) {
        phase_begin(e, PH_RMS_DW);
        HIPCHK(op, reduce_partials_add(G + o.g_att, gpart(2 * l + 1), nblk, D, st, fresh));
        phase_end(e);
      } else
        HIPCHK(op, reduce_dots_add(G + pm.resid + l, G + pm.x0l + l, tb.dot_part, nblk, 1.f, st));
    }
  }
  // every dW launch is done before the embedding side (embed_bwd adds into
  // the embedding gradient the classifier's dW GEMM wrote)
  if (async) HIPCHK(op, stream_after(e, st, ds));

  // ---- embedding side ---------------------------------------------------------
  if (!llama) {
    // compat: the x0 gradient joins before the smear backward
    // (ane/train_full.go:790-798); exact: after it (x0 is pre-smear)
    if (compat) HIPCHK(op, axpy_inplace(tb.dcur, tb.gx0, nullptr, (size_t)T * D, st));
    HIPCHK(op, smear_bwd_prep(tb.dgp, tb.dx2, tb.dot_part, tb.dcur, tb.sg_act, e->x0, P + pm.smear_lambda, T, D, S,
                              st));
    HIPCHK(op, reduce_dots_add(G + pm.smear_lambda, nullptr, tb.dot_part, 256, 1.f, st));
    {
      EpiParams p;
      p.C = G + pm.smear_gate; p.ldc = D; p.accumulate = 1;
      phase_begin(e, PH_DW_GEMM);
      HIPCHK(op, dw_gemm(e, 7, tb.dgp, D, tb.x0h, D, T, EPI_STORE_F, p));
      phase_end(e);
    }
    {
      EpiParams p;
      p.C = tb.dx2; p.ldc = D; p.accumulate = 1;
      HIPCHK(op, eng_gemm(e, 7, tb.dgp, D, false, e->smear_t, D, false, T, D, D, EPI_STORE_F, p));
    }
    if (!compat) HIPCHK(op, axpy_inplace(tb.dx2, tb.gx0, nullptr, (size_t)T * D, st));
    NormBwdArgs a;  // embedding RMSNorm backward (ane/train_full.go:921-925)
    a.dy = tb.dx2; a.x = e->xpre; a.T = T; a.D = D; a.out = tb.dcur;
    HIPCHK(op, norm_bwd(a, st));
  }
  phase_begin(e, PH_EMBED_GRAD);  // EmbedBackward (ane/train_full.go:930-933)
  HIPCHK(op, embed_bwd(G + pm.embed, tb.dcur, e->tok, T, D, V, st));
  phase_end(e);
  (void)hipEventRecord(e->step_ev[ane_engine::EV_BWD1], st);
  return ANE_OK;
}

void bias_inv(int t, float b1, float b2, float* i1, float* i2) {
  // adamBiasCorrectionInv (ane/train_full.go:1107-1111)
  const float bc1 = (float)(1.0 - pow((double)b1, (double)t));
  const float bc2 = (float)(1.0 - pow((double)b2, (double)t));
  *i1 = 1.f / bc1;
  *i2 = 1.f / bc2;
}

void add_seg(AdamArgs& a, int64_t off, int64_t len, float lr, float wd, float b1, float b2, float i1, float i2,
             int clip, int chunk) {
  AdamSeg& s = a.seg[a.nseg++];
  s.off = off; s.len = len; s.lr = lr; s.wd = wd; s.b1 = b1; s.b2 = b2; s.i1 = i1; s.i2 = i2; s.clip = clip;
  s.chunk = chunk;
}

// The duration of the last asynchronous update into adam_ns_last once its
// end event has completed (no wait).
void read_adam_ns(ane_engine* e) {
  if (!e->adam_unread || hipEventQuery(e->step_ev[ane_engine::EV_ADAM1]) != hipSuccess) return;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, e->step_ev[ane_engine::EV_ADAM0], e->step_ev[ane_engine::EV_ADAM1]) == hipSuccess)
    e->adam_ns_last = (int64_t)((double)ms * 1e6);
  e->adam_unread = false;
}

// flushPending (ane/engine.go:646-682)
int flush_pending(ane_engine* e) {
  const char* op = "flush";
  if (!e->train_ready || e->state.pending_steps == 0) return ANE_OK;
  const ane_model_cfg& c = e->cfg;
  const bool llama = c.arch == ANE_ARCH_LLAMA2;
  const int64_t D = c.dim, H = c.hidden, V = c.vocab, NH = c.heads, L = c.layers;
  const ParamMap& pm = e->pm;
  TrainBufs& tb = e->tr;
  const ane_options& O = e->opt;
  hipStream_t st = e->stream;
  // accumulate mode with the dW stream: the update runs there behind the
  // backward, in chunks the next training forward waits for one at a time
  const bool async_upd = e->async_update && e->fused_adam && e->shadow_jobs && e->shadow_jobs_t &&
                         O.accum_steps > 1 && e->dw_stream && e->refresh_ev[1] &&
                         (int)e->upd_ev.size() == 1 + (int)L;
  hipStream_t us = async_upd ? e->dw_stream : st;
  // the previous asynchronous update's duration, before its events are reused
  if (e->adam_unread) HIPCHK(op, hipEventSynchronize(e->step_ev[ane_engine::EV_ADAM1]));
  read_adam_ns(e);
  HIPCHK(op, join_update(e));
  if (async_upd) HIPCHK(op, stream_after(e, us, st));

  float gscale = (float)(1.0 / (double)e->state.pending_steps);
  gscale /= O.loss_scale;
  // the norm only feeds the clip: clipLayerGradients returns before it
  // without one (ane/train_full.go:168)
  if (O.grad_clip > 0.f) HIPCHK(op, sumsq(tb.sumsq, tb.sumsq_part, tb.G, (size_t)(pm.embed + V * D), us));
  e->state.adam_t++;
  const int t = (int)e->state.adam_t;
  float i1, i2, l1, l2;
  bias_inv(t, O.adam_beta1, O.adam_beta2, &i1, &i2);
  bias_inv(t, O.lambda_beta1, O.lambda_beta2, &l1, &l2);
  const float lr = e->lr, embed_lr = e->lr * O.embed_lr_mult, scalar_lr = e->lr * O.scalar_lr_mult;
  const float lambda_lr = e->lr * O.scalar_lr_mult * O.lambda_lr_mult;
  const float b1 = O.adam_beta1, b2 = O.adam_beta2, wd = O.weight_decay;
  AdamArgs a;
  memset(&a, 0, sizeof a);
  a.w = e->P; a.g = tb.G; a.m = tb.M; a.v = tb.Vv; a.sumsq = tb.sumsq;
  a.gscale = gscale; a.clip = O.grad_clip; a.eps = O.adam_eps;
  a.zero_g = llama ? 0 : 1;  // llama2's next backward overwrites the gradient (backward_body)
  // applyLayerAdam (ane/train_full.go:1088-1100): matrices with lr + wd; gains
  // and VE gate with the scalar lr, VE table with the embedding lr, no wd
  for (int l = 0; l < L; l++) {
    const LayerOff& o = pm.L[l];
    const int ch = 1 + l;
    add_seg(a, o.wq, o.w2 + D * H - o.wq, lr, wd, b1, b2, i1, i2, 1, ch);
    if (llama) {
      add_seg(a, o.w3, H * D, lr, wd, b1, b2, i1, i2, 1, ch);
      add_seg(a, o.g_att, 2 * D, scalar_lr, 0.f, b1, b2, i1, i2, 1, ch);
    } else if (o.ve_embed >= 0) {
      add_seg(a, o.ve_embed, V * D, embed_lr, 0.f, b1, b2, i1, i2, 1, ch);
      add_seg(a, o.ve_gate, NH * 12, scalar_lr, 0.f, b1, b2, i1, i2, 1, ch);
    }
  }
  // model-level groups (ane/engine.go:659-673)
  add_seg(a, pm.embed, V * D, embed_lr, 0.f, b1, b2, i1, i2, 1, 0);
  if (llama) {
    add_seg(a, pm.g_final, D, scalar_lr, 0.f, b1, b2, i1, i2, 0, 0);
  } else {
    add_seg(a, pm.smear_gate, D * D, lr, wd, b1, b2, i1, i2, 0, 0);
    add_seg(a, pm.smear_lambda, 2, scalar_lr, 0.f, b1, b2, i1, i2, 0, 0);
    add_seg(a, pm.resid, 2 * L, lambda_lr, 0.f, O.lambda_beta1, O.lambda_beta2, l1, l2, 0, 0);
  }
  if (a.nseg > kMaxAdamSegs) return eng_fail(e, ANE_ERR_ARG, "storiesane flush: too many parameter groups");
  // the fp16 shadows the next forward and backward read: the weight refresh
  // (refreshANERuntimeForWeights, ane/runtime.go:25-69)
  if (e->fused_adam && e->shadow_jobs && e->shadow_jobs_t) {
    // one pass: AdamW, the plain shadows and (nanochat) the gradient
    // cleared; then the refresh proper is the transposed shadows, read from
    // the plain ones
    int rc = ensure_update_jobs(e, a);
    if (rc) return rc;
    (void)hipEventRecord(e->step_ev[ane_engine::EV_ADAM0], us);
    if (async_upd) {
      for (int c = 0; c <= (int)L; c++) {
        HIPCHK(op, adam_fused_update(a, e->upd_jobs + e->upd_j0[c], e->upd_nj[c], e->upd_nb[c], e->upd_b0[c], us));
        HIPCHK(op, hipEventRecord(e->upd_ev[c], us));
      }
      e->upd_pending = true;
      e->adam_unread = true;
    } else {
      HIPCHK(op, adam_fused_update(a, e->upd_jobs, e->n_upd_jobs, e->n_upd_blocks, 0, us));
    }
    (void)hipEventRecord(e->step_ev[ane_engine::EV_ADAM1], us);
    if (e->opt.accum_steps > 1 && e->dw_stream && e->refresh_ev[1]) {
      // accumulate mode: the refresh runs asynchronously (flushPending,
      // ane/engine.go:674-677), beside the next step's forward, which
      // reads only the plain shadows
      if (!async_upd) HIPCHK(op, stream_after(e, e->dw_stream, st));
      HIPCHK(op, hipEventRecord(e->refresh_ev[0], e->dw_stream));
      HIPCHK(op, shadow_transpose(e->shadow_jobs, e->n_shadow_jobs, e->n_shadow_tiles, e->dw_stream));
      HIPCHK(op, hipEventRecord(e->refresh_ev[1], e->dw_stream));
      e->refresh_pending = true;
    } else {
      phase_begin(e, PH_REFRESH);
      HIPCHK(op, shadow_transpose(e->shadow_jobs, e->n_shadow_jobs, e->n_shadow_tiles, st));
      phase_end(e);
    }
  } else {
    (void)hipEventRecord(e->step_ev[ane_engine::EV_ADAM0], st);
    HIPCHK(op, adam_update(a, st));
    (void)hipEventRecord(e->step_ev[ane_engine::EV_ADAM1], st);
    phase_begin(e, PH_REFRESH);
    int rc = refresh_shadows(e);
    phase_end(e);
    if (rc) return rc;
    HIPCHK(op, fill_f32(tb.G, (size_t)pm.total, 0.f, st));
  }
  e->state.pending_steps = 0;
  e->state.cum_batches++;
  e->flushed = true;
  return ANE_OK;
}

// *wait_s (optional): host time spent blocked until the queued device work
// (forward, backward, weight-gradient GEMMs, update) had finished
int read_losses(ane_engine* e, int nseq, float* per, double* mean, double* wait_s = nullptr) {
  const char* op = "step";
  const float* ls = e->loss_host;
  HIPCHK(op, hipMemcpyAsync(e->loss_host, e->loss_seq, (size_t)nseq * 4, hipMemcpyDeviceToHost, e->stream));
  const double t0 = now_s();
  HIPCHK(op, stream_wait(e->stream));
  if (wait_s) *wait_s = now_s() - t0;
  double tot = 0;
  for (int b = 0; b < nseq; b++) {
    tot += ls[b];
    if (per) per[b] = ls[b];
  }
  *mean = nseq > 0 ? tot / nseq : 0.0;
  return ANE_OK;
}

// nseq windows drawn from the drand48 stream, one fused forward/backward,
// pending += nseq, flush when pending >= AccumSteps: the same update as
// nseq consecutive reference Steps (ane/engine.go:381-442).
int train_windows(ane_engine* e, int nseq, ane_step_result* res) {
  const char* op = "step";
  const double t0 = now_s();
  if (!e->data || e->ndata < (int64_t)e->cfg.seq + 1) return eng_fail(e, ANE_ERR_STATE, "storiesane step: not enough tokens");
  if (nseq <= 0 || nseq > e->opt.max_batch)
    return eng_fail(e, ANE_ERR_ARG, "storiesane step: nseq=%d must be in [1, %d]", nseq, e->opt.max_batch);
  e->startup_ns = 0;
  int rc = ensure_train(e, op);
  if (rc) return rc;
  phase_reset(e);
  e->ph_sample = e->ph_calls++ % (uint64_t)e->ph_period == 0;
  const uint64_t S = (uint64_t)e->cfg.seq;
  const uint64_t limit = (uint64_t)e->ndata - S - 1;
  std::vector<uint64_t> pos(nseq);
  for (int b = 0; b < nseq; b++) {
    uint64_t p = 0;
    if (limit > 0) {
      p = (uint64_t)(drand48_next(&e->rng) * (double)limit);
      if (p >= limit) p = limit - 1;
    }
    pos[b] = p;
    e->state.token_pos = p + S;
  }
  rc = load_windows(e, pos.data(), nseq);
  if (rc) return rc;
  e->flushed = false;
  (void)hipEventRecord(e->step_ev[ane_engine::EV_STEP0], e->stream);
  rc = backward_pass(e, nseq);
  if (rc) return rc;
  e->state.pending_steps += (uint32_t)nseq;
  if ((int)e->state.pending_steps >= e->opt.accum_steps) {
    rc = flush_pending(e);
    if (rc) return rc;
  }
  double mean = 0, wait_s = 0;
  rc = read_losses(e, nseq, nullptr, &mean, &wait_s);
  if (rc) return rc;
  const double dt = now_s() - t0;
  e->state.last_loss = (float)mean;
  e->state.cum_steps += (uint32_t)nseq;
  e->state.cum_train_ms += dt * 1e3;
  e->state.cum_wall_ms = (now_s() - e->start_s) * 1e3;
  if (res) {
    // StepResult (ane/engine.go:416-441): device phases from HIP events,
    // host durations from the wall clock
    memset(res, 0, sizeof *res);
    auto ev_ns = [&](int a, int b) -> int64_t {
      float ms = 0.f;
      return hipEventElapsedTime(&ms, e->step_ev[a], e->step_ev[b]) == hipSuccess ? (int64_t)((double)ms * 1e6) : 0;
    };
    double ph[PH_COUNT];
    phase_sum(e, ph);
    res->loss = (float)mean;
    res->step_ns = (int64_t)(dt * 1e9);
    res->startup_compile_ns = e->startup_ns;
    res->ane_eval_ns = ev_ns(ane_engine::EV_STEP0, ane_engine::EV_BWD1);  // forward + backward kernels
    res->final_head_ns = ev_ns(ane_engine::EV_HEAD0, ane_engine::EV_HEAD1);
    if (e->ph_sample) {  // this call's kernel-group phases were timed; per window
      e->ph_last_ns[PH_EMBED_GRAD] = (int64_t)(ph[PH_EMBED_GRAD] * 1e6 / nseq);
      e->ph_last_ns[PH_RMS_DW] = (int64_t)(ph[PH_RMS_DW] * 1e6 / nseq);
      e->ph_last_ns[PH_DW_GEMM] = (int64_t)(ph[PH_DW_GEMM] * 1e6 / nseq);
    }
    res->embed_grad_ns = e->ph_last_ns[PH_EMBED_GRAD] * nseq;
    res->rms_dw_ns = e->ph_last_ns[PH_RMS_DW] * nseq;
    res->dw_gemm_ns = e->ph_last_ns[PH_DW_GEMM] * nseq;
    res->dw_wait_ns = (int64_t)(wait_s * 1e9);
    if (e->flushed) {
      // an asynchronous update is still running: the latest completed one's
      if (e->adam_unread) {
        read_adam_ns(e);
        res->adam_ns = e->adam_ns_last;
      } else {
        res->adam_ns = ev_ns(ane_engine::EV_ADAM0, ane_engine::EV_ADAM1);
      }
      res->weight_refresh_ns = (int64_t)(ph[PH_REFRESH] * 1e6);
    }
    res->compile_ns = res->startup_compile_ns + res->weight_refresh_ns;
    res->cpu_work_ns = res->step_ns - res->startup_compile_ns - res->weight_refresh_ns - res->ane_eval_ns -
                       res->adam_ns;
    if (res->cpu_work_ns < 0) res->cpu_work_ns = 0;
  }
  return ANE_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
extern "C" int ane_step(ane_engine* e, ane_step_result* res) {
  CLOSED_CHECK("step");
  return train_windows(e, 1, res);
}

extern "C" int ane_train_batch(ane_engine* e, int32_t nseq, ane_step_result* res) {
  CLOSED_CHECK("step");
  return train_windows(e, nseq, res);
}

// Flush (ane/engine.go:484-496): returns the weight-refresh duration (the
// reference's waitAsyncRefresh) and adds it to CumTrainMS / CumWallMS.
extern "C" int ane_flush(ane_engine* e, int64_t* ns) {
  CLOSED_CHECK("flush");
  HIPCHK("flush", join_update(e));  // an asynchronous update still running
  phase_reset(e);
  int rc = flush_pending(e);
  if (rc) return rc;
  HIPCHK("flush", join_update(e));
  HIPCHK("flush", hipStreamSynchronize(e->stream));
  double ph[PH_COUNT];
  phase_sum(e, ph);
  int64_t refresh_ns = (int64_t)(ph[PH_REFRESH] * 1e6);
  if (e->refresh_pending) {  // waitAsyncRefresh (ane/engine.go:489)
    HIPCHK("flush", hipEventSynchronize(e->refresh_ev[1]));
    float ms = 0.f;
    HIPCHK("flush", hipEventElapsedTime(&ms, e->refresh_ev[0], e->refresh_ev[1]));
    refresh_ns = (int64_t)((double)ms * 1e6);
    e->refresh_pending = false;
  }
  if (refresh_ns > 0) {
    e->state.cum_train_ms += (double)refresh_ns / 1e6;
    e->state.cum_wall_ms = (now_s() - e->start_s) * 1e3;
  }
  if (ns) *ns = refresh_ns;
  return ANE_OK;
}

extern "C" int ane_grads(ane_engine* e, const uint16_t* tokens, const uint16_t* targets, int32_t nseq, float* grads,
                         float* mean_loss) {
  CLOSED_CHECK("grads");
  HIPCHK("grads", join_update(e));  // an asynchronous update still running
  const char* op = "grads";
  if (nseq <= 0 || nseq > e->opt.max_batch || !tokens || !targets || !grads)
    return eng_fail(e, ANE_ERR_ARG, "storiesane grads: nseq=%d must be in [1, %d]", nseq, e->opt.max_batch);
  int rc = ensure_train(e, op);
  if (rc) return rc;
  if (e->state.pending_steps)
    return eng_fail(e, ANE_ERR_STATE, "storiesane grads: %u accumulated steps pending; Flush first",
                    e->state.pending_steps);
  const size_t T = (size_t)nseq * e->cfg.seq, P = (size_t)e->pm.total;
  HIPCHK(op, hipMemcpyAsync(e->tok, tokens, T * 2, hipMemcpyHostToDevice, e->stream));
  HIPCHK(op, hipMemcpyAsync(e->tgt, targets, T * 2, hipMemcpyHostToDevice, e->stream));
  HIPCHK(op, fill_f32(e->tr.G, P, 0.f, e->stream));
  rc = backward_pass(e, nseq);
  if (rc) return rc;
  HIPCHK(op, hipMemcpyAsync(grads, e->tr.G, P * 4, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(op, fill_f32(e->tr.G, P, 0.f, e->stream));
  double mean = 0;
  rc = read_losses(e, nseq, nullptr, &mean);
  if (rc) return rc;
  // the reference's flush scale: 1 / n, then / lossScale (ane/engine.go:650-654)
  float sc = (float)(1.0 / (double)nseq);
  sc /= e->opt.loss_scale;
  for (size_t i = 0; i < P; i++) grads[i] *= sc;
  if (mean_loss) *mean_loss = (float)mean;
  return ANE_OK;
}

extern "C" int ane_set_grads(ane_engine* e, const float* grads, int64_t n, uint32_t pending) {
  CLOSED_CHECK("set grads");
  HIPCHK("set grads", join_update(e));  // an asynchronous update still running
  const char* op = "set grads";
  if (!grads || n != e->pm.total)
    return eng_fail(e, ANE_ERR_ARG, "storiesane set grads: len=%lld want=%lld", (long long)n, (long long)e->pm.total);
  int rc = ensure_train(e, op);
  if (rc) return rc;
  HIPCHK(op, hipMemcpyAsync(e->tr.G, grads, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
  HIPCHK(op, hipStreamSynchronize(e->stream));
  e->state.pending_steps = pending;
  return ANE_OK;
}

extern "C" int ane_get_opt_state(ane_engine* e, float* m, float* v, int64_t n) {
  CLOSED_CHECK("optimizer state");
  HIPCHK("optimizer state", join_update(e));  // an asynchronous update still running
  const char* op = "optimizer state";
  if (n != e->pm.total)
    return eng_fail(e, ANE_ERR_ARG, "storiesane optimizer state: len=%lld want=%lld", (long long)n,
                    (long long)e->pm.total);
  int rc = ensure_train(e, op);
  if (rc) return rc;
  if (m) HIPCHK(op, hipMemcpyAsync(m, e->tr.M, (size_t)n * 4, hipMemcpyDeviceToHost, e->stream));
  if (v) HIPCHK(op, hipMemcpyAsync(v, e->tr.Vv, (size_t)n * 4, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(op, hipStreamSynchronize(e->stream));
  return ANE_OK;
}

extern "C" int ane_set_opt_state(ane_engine* e, const float* m, const float* v, int64_t n) {
  CLOSED_CHECK("set optimizer state");
  HIPCHK("set optimizer state", join_update(e));  // an asynchronous update still running
  const char* op = "set optimizer state";
  if (n != e->pm.total)
    return eng_fail(e, ANE_ERR_ARG, "storiesane set optimizer state: len=%lld want=%lld", (long long)n,
                    (long long)e->pm.total);
  int rc = ensure_train(e, op);
  if (rc) return rc;
  if (m) HIPCHK(op, hipMemcpyAsync(e->tr.M, m, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
  else HIPCHK(op, hipMemsetAsync(e->tr.M, 0, (size_t)n * 4, e->stream));
  if (v) HIPCHK(op, hipMemcpyAsync(e->tr.Vv, v, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
  else HIPCHK(op, hipMemsetAsync(e->tr.Vv, 0, (size_t)n * 4, e->stream));
  HIPCHK(op, hipStreamSynchronize(e->stream));
  return ANE_OK;
}

extern "C" int ane_get_accum_grads(ane_engine* e, float* grads, int64_t n) {
  CLOSED_CHECK("accumulated grads");
  HIPCHK("accumulated grads", join_update(e));  // an asynchronous update still running
  const char* op = "accumulated grads";
  if (!grads || n != e->pm.total)
    return eng_fail(e, ANE_ERR_ARG, "storiesane accumulated grads: len=%lld want=%lld", (long long)n,
                    (long long)e->pm.total);
  int rc = ensure_train(e, op);
  if (rc) return rc;
  if (e->state.pending_steps == 0) {  // nothing accumulated (the buffer may hold a finished window's sums)
    memset(grads, 0, (size_t)n * 4);
    return ANE_OK;
  }
  HIPCHK(op, hipMemcpyAsync(grads, e->tr.G, (size_t)n * 4, hipMemcpyDeviceToHost, e->stream));
  HIPCHK(op, hipStreamSynchronize(e->stream));
  return ANE_OK;
}

extern "C" int ane_seed_sampler(ane_engine* e, int64_t seed) {
  CLOSED_CHECK("seed sampler");
  e->rng = drand48_seed(seed);
  return ANE_OK;
}

extern "C" float ane_lr(const ane_engine* e) { return (e && !e->closed) ? e->lr : 0.f; }

extern "C" int ane_set_lr(ane_engine* e, float lr) {
  CLOSED_CHECK("set lr");
  if (!(lr > 0.f)) return eng_fail(e, ANE_ERR_ARG, "storiesane set lr: lr must be > 0");
  e->lr = lr;
  return ANE_OK;
}

extern "C" int ane_get_state(ane_engine* e, ane_state* out) {
  if (!e || !out) return ANE_ERR_ARG;
  *out = e->closed ? ane_state{} : e->state;
  return ANE_OK;
}

extern "C" int ane_load_state(ane_engine* e, const ane_state* s) {
  CLOSED_CHECK("load state");
  if (!s) return eng_fail(e, ANE_ERR_ARG, "storiesane load state: null state");
  e->state = *s;
  return ANE_OK;
}
