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
};

hipError_t attention_fwd(const AttnArgs& a, hipStream_t stream);

}  // namespace ane
