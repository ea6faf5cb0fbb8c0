// Row-wise (per token) and elementwise kernels: embedding, RMSNorm,
// cross-entropy reduction, window gather, weight shadow conversion.
#pragma once
#include "hip_common.h"

namespace ane {

// x[t, :] = embed[tok_t, :] (zero row for tok_t >= vocab)      ane/stories/cpu.go:41-72
hipError_t embed_lookup(float* x, const float* embed, const uint16_t* tok, int T, int D, int V,
                        hipStream_t s);
// Streams [p, p + bytes) through the cache hierarchy (prefetch_slice over up
// to 1024 blocks): the weights of the GEMM that runs next.
hipError_t prefetch_weights(const void* p, size_t bytes, hipStream_t s);
// The same for up to kPrefetchRegions regions in one launch (null or empty
// regions are skipped): brings the operands of GEMMs a few kernels ahead
// into the device's last-level cache.
constexpr int kPrefetchRegions = 6;
struct PrefetchList {
  const void* p[kPrefetchRegions] = {};
  size_t bytes[kPrefetchRegions] = {};
  int n = 0;
  void add(const void* q, size_t b) {
    if (q && b >= 16 && n < kPrefetchRegions) {
      p[n] = q;
      bytes[n++] = b;
    }
  }
};
hipError_t prefetch_list(const PrefetchList& l, hipStream_t s);
// x = embed[tok] (0 for tok >= V), xg = fp16(x * gain) and ssq[t] = sum of
// x[t]^2: the inputs of a GEMM that applies the RMSNorm after its product
// (EPI_*_RR with one partial per row); pf: weights streamed alongside.
hipError_t embed_xg(float* x, half_t* xg, float* ssq, const float* embed, const uint16_t* tok, const float* gain,
                    int T, int D, int V, hipStream_t s, const void* pf = nullptr, size_t pf_bytes = 0);

// nanochat entry: xpre = embed[tok]; x0 = xpre / rms(xpre) (fp32 scale);
// xh = fp16(x0)                      ane/train_full.go:386-390, ane/common.go:157-174
hipError_t embed_norm(float* xpre, float* x0, half_t* xh, const float* embed, const uint16_t* tok, int T,
                      int D, int V, hipStream_t s);

// out = fp16((x - *lam * xsub) / rms(x - lam * xsub) * gain); xsub, gain optional.
// Gain-free form: rmsNormNoWeightCF (ane/common.go:157-174); gain form:
// stories.RMSNorm (ane/stories/cpu.go:97-111); backout: ane/common.go:385-389.
// pf / pf_bytes: weights of the GEMM that follows, streamed through the
// caches alongside (prefetch_slice); NULL for none.
hipError_t rmsnorm_f16(half_t* out, const float* x, const float* xsub, const float* lam, const float* gain,
                       int T, int D, hipStream_t s, const void* pf = nullptr, size_t pf_bytes = 0);

// tok[b*S + t] = data[pos[b] + t]; tgt[b*S + t] = data[pos[b] + t + 1]   ane/engine.go:403-404
hipError_t gather_windows(uint16_t* tok, uint16_t* tgt, const uint16_t* data, const uint64_t* pos, int nseq,
                          int S, hipStream_t s);
// the same with host-side window starts passed as kernel arguments (nseq <=
// kArgWindows): no copy, so nothing waits on the host before the launch
constexpr int kArgWindows = 64;
struct WindowStarts {
  uint64_t p[kArgWindows];
};
hipError_t gather_windows_args(uint16_t* tok, uint16_t* tgt, const uint16_t* data, const uint64_t* pos_host, int nseq,
                               int S, hipStream_t s);

// Merges the classifier's per-block (max, sumexp) partials into per-token
// log-sum-exp and the per-sequence mean cross-entropy over valid targets
// (stories.CrossEntropyLoss, ane/stories/cpu.go:212-292).  colscale (optional)
// receives dscale / valid_b for valid tokens and 0 otherwise.
// lse and tok_loss ([T] each) are required scratch/outputs.
hipError_t ce_reduce(float* loss_seq, float* lse, float* tok_loss, float* colscale, float dscale,
                     const float2* partial, int np, const float* tgt_logit, const uint16_t* tgt, int V, int nseq, int S,
                     hipStream_t s);

hipError_t f32_to_f16(half_t* dst, const float* src, size_t n, hipStream_t s);
// dst [2H, D] with 32-row blocks alternating W1 / W3 rows
hipError_t interleave_w13(half_t* dst, const float* w1, const float* w3, int H, int D, hipStream_t s);

}  // namespace ane
