// Classifier-head cross-entropy on caller-owned device buffers: the loss
// half of runFinalHead (ane/train_full.go:480-508) -- tied classifier
// logits = Embed . xn (ane/stories/cpu.go:303-327), the optional 15*tanh
// softcap (ane/common.go:272-287) and stories.CrossEntropyLoss's per-token
// -log(max(p_target, 1e-10)) averaged over the valid targets of each
// sequence (ane/stories/cpu.go:212-292) -- without materialising a logit.
//
// Kernels: the classifier GEMM with the cross-entropy epilogue (one
// (max, sum exp) partial per block row and token, plus the target logit),
// then the per-token merge and the per-sequence mean (ce_reduce).  Their
// scratch -- partials, target logits, per-token losses and, when the caller
// passes no lse buffer, the log-sum-exps -- is allocated by the library for
// the duration of the call (ane_head_loss), or is a fixed array in device
// global memory (ane_head_loss_noalloc, for callers that cannot allocate).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "../../include/ane_hip.h"
#include "gemm.h"
#include "rowops.h"

using namespace ane;

namespace {

thread_local std::string g_op_err;

int op_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_op_err = buf;
  return code;
}

constexpr size_t kAlign = 256;
size_t up(size_t n) { return (n + kAlign - 1) & ~(kAlign - 1); }

// Tile of the classifier GEMM (rows = vocabulary, columns = tokens) and the
// scratch layout: partials [V / bm][T] float2 | tgt_logit [T] | tok_loss [T]
// | lse [T] (used when the caller passes none).
struct HeadPlan {
  int bm = 0, bn = 0, np = 0;
  size_t off_tl = 0, off_tok = 0, off_lse = 0, bytes = 0;
};

int head_plan(const char* op, int T, int D, int V, int S, HeadPlan* p) {
  if (T <= 0 || D <= 0 || V <= 0 || S <= 0 || T % S || D % 64 || V % 64 || T % 64 || V > 65535)
    return op_fail(ANE_ERR_ARG,
                   "storiesane %s: ntok=%d dim=%d vocab=%d seq=%d (ntok a multiple of seq and of 64; dim and vocab "
                   "multiples of 64; vocab < 65536)",
                   op, T, D, V, S);
  int bm = 0, bn = 0;
  gemm_pick_tile(V, T, D, EPI_CE, &bm, &bn);
  if (!bm || !bn) return op_fail(ANE_ERR_ARG, "storiesane %s: no classifier tile fits vocab=%d ntok=%d", op, V, T);
  p->bm = bm;
  p->bn = bn;
  p->np = V / bm;
  size_t o = up((size_t)p->np * T * sizeof(float2));
  p->off_tl = o;
  o += up((size_t)T * 4);
  p->off_tok = o;
  o += up((size_t)T * 4);
  p->off_lse = o;
  o += up((size_t)T * 4);
  p->bytes = o;
  return ANE_OK;
}

// ws: at least plan.bytes of device memory, 256-byte aligned.  Every scratch
// element the kernels read was written earlier in the same call (each
// partial by its block, each valid target's logit by the one lane holding
// it; invalid targets' logits are never read), so nothing needs clearing.
hipError_t head_run(const HeadPlan& pl, const uint16_t* xn, const uint16_t* embed, const uint16_t* targets, int T,
                    int D, int V, int S, int softcap, float* loss_seq, float* lse, char* ws, hipStream_t st) {
  GemmArgs g;
  g.A = (const half_t*)embed; g.B = (const half_t*)xn;
  g.lda = D; g.ldb = D; g.M = V; g.N = T; g.K = D; g.a_t = false; g.b_t = false;
  EpiParams p;
  p.targets = targets;
  p.partial = (float2*)ws;
  p.tgt_logit = (float*)(ws + pl.off_tl);
  p.softcap = softcap != 0;
  p.cap = 15.f;
  p.vocab = V;
  hipError_t h = gemm_run(g, EPI_CE, p, st, pl.bm, pl.bn);
  if (h != hipSuccess) return h;
  return ce_reduce(loss_seq, lse ? lse : (float*)(ws + pl.off_lse), (float*)(ws + pl.off_tok), nullptr, 0.f,
                   (const float2*)ws, pl.np, (const float*)(ws + pl.off_tl), targets, V, T / S, S, st);
}

}  // namespace

extern "C" const char* ane_op_last_error(void) { return g_op_err.c_str(); }

extern "C" int ane_head_loss(const uint16_t* xn, const uint16_t* embed, const uint16_t* targets, int32_t ntok,
                             int32_t dim, int32_t vocab, int32_t seq, int32_t softcap, float* loss_seq, float* lse,
                             void* stream) {
  const char* op = "head loss";
  if (!xn || !embed || !targets || !loss_seq) return op_fail(ANE_ERR_ARG, "storiesane %s: null buffer", op);
  HeadPlan pl;
  int rc = head_plan(op, ntok, dim, vocab, seq, &pl);
  if (rc) return rc;
  const hipStream_t st = (hipStream_t)stream;
  void* ws = nullptr;
  hipError_t h = hipMalloc(&ws, pl.bytes);
  if (h != hipSuccess) return op_fail(ANE_ERR_NOMEM, "storiesane %s: hipMalloc(%zu): %s", op, pl.bytes,
                                      hipGetErrorString(h));
  h = head_run(pl, xn, embed, targets, ntok, dim, vocab, seq, softcap, loss_seq, lse, (char*)ws, st);
  const hipError_t hs = hipStreamSynchronize(st);  // the workspace is freed below
  (void)hipFree(ws);
  if (h == hipSuccess) h = hs;
  if (h != hipSuccess) return op_fail(ANE_ERR_HIP, "storiesane %s: %s", op, hipGetErrorString(h));
  return ANE_OK;
}

// ---- allocation-free variant --------------------------------------------------
// The scratch of ane_head_loss_noalloc: a fixed array in this library's code
// object, one copy per GPU (each device that loads the library holds it
// until the process ends).  8 MiB holds the stories110M head (vocabulary
// 32000) at up to 8192 tokens when the classifier runs 256-row blocks
// (from 1024 tokens on), up to 4096 with the 128-row blocks of fewer tokens.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

// The array's name is a host-side stand-in, not a device address: each
// device's address comes from hipGetSymbolAddress, taken once per device on
// its first call with that device current, and only that address reaches a
// kernel.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

int scratch_address(const char* op, void** out) {
  int dev = -1;
  hipError_t h = hipGetDevice(&dev);
  if (h != hipSuccess) return op_fail(ANE_ERR_HIP, "storiesane %s: hipGetDevice: %s", op, hipGetErrorString(h));
  if (dev < 0 || dev >= kMaxDevices) return op_fail(ANE_ERR_ARG, "storiesane %s: device %d out of range", op, dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    h = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (h != hipSuccess || !p)
      return op_fail(ANE_ERR_HIP, "storiesane %s: hipGetSymbolAddress(scratch) on device %d: %s", op, dev,
                     hipGetErrorString(h));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return ANE_OK;
}

}  // namespace

extern "C" int ane_head_loss_noalloc(const uint16_t* xn, const uint16_t* embed, const uint16_t* targets,
                                     int32_t ntok, int32_t dim, int32_t vocab, int32_t seq, int32_t softcap,
                                     float* loss_seq, float* lse, void* stream) {
  const char* op = "head loss noalloc";
  if (!xn || !embed || !targets || !loss_seq) return op_fail(ANE_ERR_ARG, "storiesane %s: null buffer", op);
  HeadPlan pl;
  int rc = head_plan(op, ntok, dim, vocab, seq, &pl);
  if (rc) return rc;
  if (pl.bytes > kNoAllocScratchBytes)
    return op_fail(ANE_ERR_ARG,
                   "storiesane %s: ntok=%d vocab=%d needs %zu bytes of scratch; this entry point holds %zu "
                   "(use ane_head_loss)",
                   op, ntok, vocab, pl.bytes, kNoAllocScratchBytes);
  void* ws = nullptr;
  rc = scratch_address(op, &ws);
  if (rc) return rc;
  const hipError_t h = head_run(pl, xn, embed, targets, ntok, dim, vocab, seq, softcap, loss_seq, lse, (char*)ws,
                                (hipStream_t)stream);
  if (h != hipSuccess) return op_fail(ANE_ERR_HIP, "storiesane %s: %s", op, hipGetErrorString(h));
  return ANE_OK;
}
