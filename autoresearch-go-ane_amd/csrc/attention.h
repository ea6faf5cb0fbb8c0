// Fused causal attention (forward) for head_dim 64 on gfx950.
#pragma once
#include "hip_common.h"

namespace ane {

struct AttnArgs {
  const half_t* qkv;      // [T, 3*D] rows: q | k | v (pre-RoPE), T = nseq * S
  half_t* out;            // [T, D]
  float* lse;             // [T, NH] log-sum-exp of the scaled scores (optional)
  const float* rope_cos;  // [S, 32]
  const float* rope_sin;  // [S, 32]
  int nseq, S, NH;
  int qknorm;             // nanochat: q,k <- 1.2 * q / rms(q) per head after RoPE
  float scale;            // score scale (1/8)
  // value embeddings (nanochat VE layers): v += 3 * sigmoid(gate_h . x[t, 0:12]) * ve_embed[tok_t, h*64 + d]
  const float* ve_x;      // [T, D] layer input before its RMSNorm; null disables VE
  const float* ve_gate;   // [NH * 12]
  const float* ve_embed;  // [V, D]
  const uint16_t* tokens; // [T]
  int vocab;
  half_t* qkvt;           // optional [T, 3*D]: q, k after RoPE (+ QK-norm) and v after VE, as used
  half_t* qkvt_lo;        // optional [T, 2*D]: fp16 residuals q - q_hi | k - k_hi of those q, k
  int hilo;               // scores from hi+lo split operands (~fp32); S <= 256
  const void* pf;         // optional: weights of the next GEMM, streamed through the caches
  size_t pf_bytes;
  int split_from;         // set by attention_fwd (block decomposition)
};

hipError_t attention_fwd(const AttnArgs& a, hipStream_t stream);

// Backward of the fused attention (ane/train_full.go:261-316 for the
// probabilities / ds recurrences, ane/common.go:229-270 for QK-norm).
struct AttnBwdArgs {
  const half_t* qkv;      // [T, 3D] pre-RoPE projections (QK-norm / RoPE backward recompute from it)
  const half_t* qkvt;     // [T, 3D] q, k, v as used by the forward (AttnArgs.qkvt)
  const half_t* o;        // [T, D] attention output whose probabilities P uses (for delta = rowsum(dO * O))
  const half_t* dout;     // [T, D] gradient of the attention output
  const float* lse;       // [T, NH] log-sum-exp of the scale_p-scaled scores
  float* delta;           // [T, NH] scratch: written by the dQ pass, read by the dK/dV pass
  half_t* dqkv;           // [T, 3D] out: dq | dk w.r.t. the projections, dv w.r.t. v as used
  const float* rope_cos;  // [S, 32]
  const float* rope_sin;
  int nseq, S, NH;
  int qknorm;             // apply the QK-norm backward
  float qk_coef2;         // coefficient of its projection term: 1.2^2 (reference) or 1.2 (exact)
  int rope_bwd;           // apply the transposed rotation (the reference has none)
  float scale_p;          // P = exp(scale_p * q.k - lse)
  float scale_ds;         // dS = P * (dP - delta) * scale_ds
  const half_t* qkvt_lo;  // [T, 2D] q | k fp16 residuals (AttnArgs.qkvt_lo), used when hilo
  int hilo;               // recompute the scores from split operands (~fp32)
};

// seq <= 256 (the whole sequence is staged in LDS twice).
hipError_t attention_bwd(const AttnBwdArgs& a, hipStream_t stream);

}  // namespace ane
