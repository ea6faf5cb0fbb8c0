// Row-wise and elementwise kernels of the backward pass and the optimizer.
#pragma once
#include "hip_common.h"

namespace ane {

constexpr int kNormBwdRows = 8;  // rows per block of norm_bwd (4 waves x 2 rows)

// out = alpha * addend + addend2 + RMSNorm-backward(dy; x, gain) (+ ve_dx on
// channels 0..11), fp32 and optionally fp16.  Gain-free form:
// rmsNormNoWeightBackwardCF (ane/common.go:176-197); gain form:
// stories.RMSNormBackward (ane/stories/cpu.go:191-210, gain on both terms
// as there).  Per block of kNormBwdRows rows it also writes partials of
// dgain (sum dy*x*rrms) and of the two lambda dots (addend.lam_x,
// addend.lam_x0, in double), and accumulates gx0 += xl * addend.
struct NormBwdArgs {
  const float* dy = nullptr;
  const float* x = nullptr;
  const float* gain = nullptr;
  float* dgain_part = nullptr;      // [nblocks][D]
  const float* addend = nullptr;
  const float* alpha_p = nullptr;   // device scalar (else alpha)
  float alpha = 1.f;
  const float* addend2 = nullptr;
  const float* ve_dx = nullptr;     // [T][12]
  float* out = nullptr;
  half_t* out_h = nullptr;
  const float* lam_x = nullptr;
  const float* lam_x0 = nullptr;
  double* lam_part = nullptr;       // [nblocks][2]
  float* gx0 = nullptr;
  const float* xl_p = nullptr;
  int T = 0, D = 0;
  int general = 0;                  // host: take the general kernel even for the gain form
};
hipError_t norm_bwd(const NormBwdArgs& a, hipStream_t s);
inline int norm_bwd_blocks(int T) { return (T + kNormBwdRows - 1) / kNormBwdRows; }

// dst[i] += sum over blocks of part[b][i]  (i < n)
// (overwrite: dst[i] = the sum, the first gradient of an accumulation window)
hipError_t reduce_partials_add(float* dst, const float* part, int nblocks, int n, hipStream_t s,
                               bool overwrite = false);
// dst[k] += (float)(sign * sum over blocks of part[b][k])  for k < 2 (lambda grads)
hipError_t reduce_dots_add(float* dst0, float* dst1, const double* part, int nblocks, float sign, hipStream_t s);

// backoutBackwardCF (ane/common.go:393-403): part[b] = partial sum of d * xmid
// (double), ginj = -lambda * d
hipError_t backout_bwd(float* ginj, double* part, const float* d, const float* xmid, const float* lam_p, int T,
                       int D, hipStream_t s);

// backoutForwardCF (ane/common.go:385-389), out of place: out = x - lambda * xmid
hipError_t backout_fwd(float* out, const float* x, const float* xmid, const float* lam_p, size_t n, hipStream_t s);

// y += x (n floats); with out_h, also writes fp16(y)
hipError_t axpy_inplace(float* y, const float* x, half_t* out_h, size_t n, hipStream_t s);

// smearBackwardCF first half (ane/common.go:343-382):
// dgp = dy*lam*s*g*(1-g) (fp16), dout2[t] = dy[t] + dy[t+1]*lam*g[t+1]
// (same sequence), part = partial sums of dy*g*s (double); s = x0[t-1].
hipError_t smear_bwd_prep(half_t* dgp, float* dout2, double* part, const float* dy, const float* gact,
                          const float* x0, const float* lam_p, int T, int D, int seq, hipStream_t s);

// stories.EmbedBackward (ane/stories/cpu.go:74-95): G[tok_t, :] += dx[t, :]
hipError_t embed_bwd(float* gembed, const float* dx, const uint16_t* tok, int T, int D, int V, hipStream_t s);

// veBackwardCF (ane/train_full.go:1062-1086) for one VE layer.
hipError_t ve_bwd(float* gve_embed, float* gve_gate, float* ve_dx, const half_t* dv, int ldv, const float* x,
                  const float* ve_embed, const float* ve_gate, const uint16_t* tok, int T, int D, int NH, int V,
                  hipStream_t s);

hipError_t fill_f32(float* p, size_t n, float v, hipStream_t s);

// out[c * ldo + r] = in[r * ldi + c] for r < R, c < C (fp16); R and C
// multiples of 64.  Turns a token-major [T, C] operand into the [C, T]
// form the weight-gradient GEMMs read K-major (K = T).
hipError_t transpose_h(half_t* out, const half_t* in, int R, int C, int ldi, int ldo, hipStream_t s);
// Two independent transposes in one launch (out_b == nullptr: only the first).
hipError_t transpose2_h(half_t* out_a, const half_t* in_a, int Ra, int Ca, int ldi_a, int ldo_a, half_t* out_b,
                        const half_t* in_b, int Rb, int Cb, int ldi_b, int ldo_b, hipStream_t s);

// fp16 weight shadows from the fp32 masters in one launch.  Job j converts
// src [R, C] (row-major fp32) into dst row dr(r) = (r / 32) * blk_stride +
// blk_off + r % 32 of a row-major [*, C] fp16 matrix and, when dst_t is set,
// into column dr(r) of its transpose dst_t [C, ldt].  R and C are multiples
// of 64; tile0 = the job's first 64x64 tile in the launch's tile numbering.
struct ShadowJob {
  const float* src;
  half_t* dst;
  half_t* dst_t;
  int R, C, blk_stride, blk_off, ldt, tile0;
};
hipError_t shadow_refresh(const ShadowJob* jobs_dev, int njobs, int ntiles, hipStream_t s);

// sum of squares of g[0, n) in double -> *out (two passes through part[kSumsqBlocks])
constexpr int kSumsqBlocks = 1024;
hipError_t sumsq(double* out, double* part, const float* g, size_t n, hipStream_t s);

// AdamW over parameter segments (adamUpdateCFWithInv, ane/train_full.go:1113-1150):
// g' = g * gscale * (clip segment ? clip factor : 1), clip factor =
// clip / ||g * gscale||_(clip segments) when that norm exceeds clip
// (clipLayerGradients, ane/train_full.go:167-196).
struct AdamSeg {
  int64_t off, len;
  float lr, wd, b1, b2, i1, i2;
  int clip;
  int chunk;  // update chunk the host launches it in (scheduling only; the kernels ignore it)
};
constexpr int kMaxAdamSegs = 64;
struct AdamArgs {
  float* w;
  float* g;  // read by adam_update; read (and zeroed when zero_g) by adam_fused_update
  float* m;
  float* v;
  const double* sumsq;  // device: sum of squares of the raw clip-segment grads
  float gscale, clip, eps;
  int nseg;
  int zero_g;  // adam_fused_update: clear the gradient (unless the next backward overwrites it)
  AdamSeg seg[kMaxAdamSegs];
};
hipError_t adam_update(const AdamArgs& a, hipStream_t s);

// The flush's fused update: the AdamW of adam_update (same arithmetic), the
// gradient zeroed for the next accumulation, and the fp16 shadow of every
// updated weight matrix written (rows placed as ShadowJob's blk_stride /
// blk_off mapping), in one pass.  Jobs are the segments cut where a matrix
// with a shadow starts or ends; a block updates kUpdateChunk elements of one
// job (4 per thread and pass when vec: offset and length multiples of 4).
constexpr int kUpdateChunk = 4096;
struct UpdateJob {
  int64_t off, len;
  half_t* sh;                  // plain fp16 shadow, [rows][C] (null: none)
  int C, blk_stride, blk_off;  // shadow row of source row r: (r / 32) * blk_stride + blk_off + r % 32
  int seg;                     // AdamArgs segment: hyperparameters
  int blk0;                    // first block of the job (counted over the whole table)
  int vec;
};
// One launch covers jobs_dev[0, njobs), whose blocks are [blk_base, blk_base + nblocks)
// of the table: the whole table, or the jobs of one chunk (kept together).
hipError_t adam_fused_update(const AdamArgs& a, const UpdateJob* jobs_dev, int njobs, int nblocks, int blk_base,
                             hipStream_t s);
// the transposed shadows (dst_t) of every job, read from the plain fp16 shadows
hipError_t shadow_transpose(const ShadowJob* jobs_dev, int njobs, int ntiles, hipStream_t s);

}  // namespace ane
