// Fused causal attention backward, head_dim 64, seq <= 256.
//
// The reference computes, per head and query t (causalAttentionBackwardCF,
// ane/train_full.go:261-316):  p = softmax(scale * q_t.k), dP_s = dO_t.v_s,
// ds = p * (dP - sum_s p dP) * scale, dq_t += ds k_s, dk_s += ds q_t,
// dv_s += p dO_t.  With delta_t = sum_s p_s dP_s = dO_t . O_t (O the output
// of those probabilities) this is the flash-attention backward; scale is a
// parameter because the reference recomputes the probabilities with scale
// 1.0 although its forward uses 1/8 (its backward is therefore the gradient
// of the scale-1 attention, which the engine reproduces by passing the
// scale-1 forward's O and lse).
//
// Two kernels per (sequence, head), both keeping P and dS in registers:
//  * dQ pass: lanes own queries; S^T = K Q^T and dP^T = V dO^T leave each
//    lane with 16 keys of one query, which is the B-operand layout of
//    dQ^T = K^T dS^T.  It also writes delta for the second pass.
//  * dK/dV pass: lanes own keys; S = Q K^T and dP = dO V^T leave each lane
//    with 16 queries of one key, the B-operand layout of dV^T = dO^T P and
//    dK^T = Q^T dS.
// Operands that are contracted over the sequence (K^T, Q^T, dO^T) are staged
// transposed in LDS by 8x8 register transposes.  The epilogues apply the
// QK-norm backward (qkNormBackwardCF, ane/common.go:229-270, with the
// reference's 1.2^2 coefficient or the exact 1.2) and, for the exact
// gradient, the transposed RoPE rotation (the reference applies none,
// ane/train_full.go:646-665), each on the 64 dims a lane pair holds.
#include <stdlib.h>

#include "attention.h"

namespace ane {

namespace {

constexpr int HD = 64;
constexpr float kL2E = 1.4426950408889634f;

// rows [0, S) of a [*, ld] fp16 matrix (64 columns at src) -> swizzled [S][64];
// batches of 8 chunks per thread, all loads of a batch issued before its stores
__device__ __forceinline__ void stage_rows(half_t* dst, const half_t* src, size_t ld, int S, int tid, int nthr) {
  constexpr int KB = 8;
  for (int c0 = tid; c0 < S * 8; c0 += KB * nthr) {
    half8 v[KB];
#pragma unroll
    for (int u = 0; u < KB; u++) {
      const int c = c0 + u * nthr;
      if (c < S * 8) v[u] = ld_h8(src + (size_t)(c >> 3) * ld + (c & 7) * 8);
    }
#pragma unroll
    for (int u = 0; u < KB; u++) {
      const int c = c0 + u * nthr;
      if (c < S * 8) st_h8(dst + (c >> 3) * HD + swz(c >> 3, c & 7) * 8, v[u]);
    }
  }
}

// rows [0, S) of a [*, ld] fp16 matrix (64 columns at src) -> transposed
// [64][ST] (row = column of src, sequence index contiguous), via 8x8 blocks
__device__ __forceinline__ void stage_T(half_t* dst, int ST, const half_t* src, size_t ld, int S, int tid,
                                        int nthr) {
  const int nrc = S / 8;
  for (int blk = tid; blk < S; blk += nthr) {
    const int rc = blk % nrc, cc = blk / nrc;
    half8 v[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) v[jj] = ld_h8(src + (size_t)(rc * 8 + jj) * ld + cc * 8);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      half4 lo, hi;
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        lo[jj] = v[jj][i];
        hi[jj] = v[jj + 4][i];
      }
      half_t* d = dst + (cc * 8 + i) * ST + rc * 8;
      *reinterpret_cast<half4*>(d) = lo;
      *reinterpret_cast<half4*>(d + 4) = hi;
    }
  }
}

// 8 values of a transposed tile: positions p0..p0+3 and p0+8..p0+11 of row d
__device__ __forceinline__ half8 ld_t8(const half_t* Tt, int ST, int d, int p0) {
  const half4 x = *reinterpret_cast<const half4*>(Tt + d * ST + p0);
  const half4 y = *reinterpret_cast<const half4*>(Tt + d * ST + p0 + 8);
  half8 r;
#pragma unroll
  for (int u = 0; u < 4; u++) {
    r[u] = x[u];
    r[u + 4] = y[u];
  }
  return r;
}

// Gradient w.r.t. the transformed q (or k) -> w.r.t. the projection.  A lane
// holds dims dt*32 + 8*(r/4) + 4g + r%4 (dt = 0,1; r = 0..15) of one row;
// its partner lane (l ^ 32) holds the other 32 dims.
__device__ __forceinline__ void qk_post(float (&dv)[2][16], const half_t* raw, int pos, int g,
                                        const AttnBwdArgs& a) {
  if (a.qknorm) {
    float pre[2][16];
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
      for (int rq = 0; rq < 4; rq++) {
        const int d0 = dt * 32 + 8 * rq + 4 * g;
        const half4 hv = *reinterpret_cast<const half4*>(raw + d0);
#pragma unroll
        for (int p = 0; p < 2; p++) {
          const int i = d0 / 2 + p;
          const float cs = a.rope_cos[pos * 32 + i], sn = a.rope_sin[pos * 32 + i];
          const float e = (float)hv[2 * p], o = (float)hv[2 * p + 1];
          pre[dt][4 * rq + 2 * p] = e * cs - o * sn;
          pre[dt][4 * rq + 2 * p + 1] = o * cs + e * sn;
        }
      }
    float ss = 0.f, dot = 0.f;
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        ss += pre[dt][r] * pre[dt][r];
        dot += dv[dt][r] * pre[dt][r];
      }
    ss += __shfl_xor(ss, 32, 64);
    dot += __shfl_xor(dot, 32, 64);
    const float rr = 1.0f / sqrtf(ss * (1.0f / HD) + 1e-5f);
    const float coeff = dot * rr * rr * rr * (1.0f / HD) * a.qk_coef2;
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
      for (int r = 0; r < 16; r++) dv[dt][r] = dv[dt][r] * rr * 1.2f - coeff * pre[dt][r];
  }
  if (a.rope_bwd) {
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
      for (int rq = 0; rq < 4; rq++) {
        const int d0 = dt * 32 + 8 * rq + 4 * g;
#pragma unroll
        for (int p = 0; p < 2; p++) {
          const int i = d0 / 2 + p;
          const float cs = a.rope_cos[pos * 32 + i], sn = a.rope_sin[pos * 32 + i];
          const float e = dv[dt][4 * rq + 2 * p], o = dv[dt][4 * rq + 2 * p + 1];
          dv[dt][4 * rq + 2 * p] = e * cs + o * sn;
          dv[dt][4 * rq + 2 * p + 1] = o * cs - e * sn;
        }
      }
  }
}

__device__ __forceinline__ void store_row(half_t* dst, const float (&dv)[2][16], int g) {
#pragma unroll
  for (int dt = 0; dt < 2; dt++)
#pragma unroll
    for (int rq = 0; rq < 4; rq++) {
      half4 w;
#pragma unroll
      for (int u = 0; u < 4; u++) w[u] = (half_t)dv[dt][4 * rq + u];
      *reinterpret_cast<half4*>(dst + dt * 32 + 8 * rq + 4 * g) = w;
    }
}

// HILO: the scores are recomputed from split fp16 operands (hi + lo,
// ~fp32 accuracy), matching a forward that used them (AttnArgs.hilo).
// PERQ: one q block (dQ pass) or key block (dK/dV pass) per wave, 8 waves
// per block, so two waves share each SIMD instead of one wave walking a
// pair of blocks in turn (wave w takes the first block of pair w % (waves / 2)
// if w < waves / 2, else the second).
template <int SMAX, bool HILO, bool PERQ>
__global__ __launch_bounds__(PERQ ? 512 : 256) void attn_bwd_dq_kernel(AttnBwdArgs a) {
  constexpr int ST = SMAX + 4;
  __shared__ __attribute__((aligned(16))) half_t Ks[SMAX * HD];
  __shared__ __attribute__((aligned(16))) half_t Ks_lo[HILO ? SMAX * HD : 8];
  __shared__ __attribute__((aligned(16))) half_t Kt[HD * ST];
  __shared__ __attribute__((aligned(16))) half_t Vs[SMAX * HD];
  const int S = a.S, NH = a.NH, D = NH * HD, D3 = 3 * D;
  const int h = blockIdx.y, b = blockIdx.z, nthr = blockDim.x, tid = threadIdx.x;
  const size_t tok0 = (size_t)b * S;
  const half_t* base = a.qkvt + tok0 * D3;
  stage_rows(Ks, base + D + h * HD, D3, S, tid, nthr);
  if constexpr (HILO) stage_rows(Ks_lo, a.qkvt_lo + tok0 * 2 * D + D + h * HD, 2 * D, S, tid, nthr);
  stage_T(Kt, ST, base + D + h * HD, D3, S, tid, nthr);
  stage_rows(Vs, base + 2 * D + h * HD, D3, S, tid, nthr);
  __syncthreads();

  const int lane = tid & 63, wave = tid >> 6, nw = nthr >> 6;
  const int nqb = S / 32, npairs = nqb / 2;
  const int slots = PERQ ? nw / 2 : nw, slot = PERQ ? wave % slots : wave;
  const int pair = blockIdx.x * slots + slot;
  if (pair >= npairs) return;
  const int g = lane >> 5, ql = lane & 31;
  const float sp = a.scale_p * kL2E;
  const int which0 = PERQ ? wave / slots : 0, which1 = PERQ ? which0 + 1 : 2;

  for (int which = which0; which < which1; which++) {
    const int qb = which == 0 ? pair : nqb - 1 - pair;
    const int q = qb * 32 + ql;
    const size_t t = tok0 + q;
    half8 qf[4], qlo[4], df[4];
    float dd = 0.f;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int d0 = s * 16 + g * 8;
      qf[s] = ld_h8(base + (size_t)q * D3 + h * HD + d0);
      if constexpr (HILO) qlo[s] = ld_h8(a.qkvt_lo + t * 2 * D + h * HD + d0);
      df[s] = ld_h8(a.dout + t * D + h * HD + d0);
      const half8 ov = ld_h8(a.o + t * D + h * HD + d0);
#pragma unroll
      for (int p = 0; p < 8; p++) dd += (float)df[s][p] * (float)ov[p];
    }
    dd += __shfl_xor(dd, 32, 64);
    if (g == 0) a.delta[t * NH + h] = dd;
    const float lse2 = a.lse[t * NH + h] * kL2E;

    floatx16 dq0, dq1;
#pragma unroll
    for (int r = 0; r < 16; r++) { dq0[r] = 0.f; dq1[r] = 0.f; }
    for (int kb = 0; kb <= qb; kb++) {
      floatx16 sacc, dpacc;
#pragma unroll
      for (int r = 0; r < 16; r++) { sacc[r] = 0.f; dpacc[r] = 0.f; }
      const int krow = kb * 32 + ql;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const int off = krow * HD + swz(krow, s * 2 + g) * 8;
        const half8 kf = ld_h8(Ks + off);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], sacc, 0, 0, 0);
        if constexpr (HILO) {
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_h8(Ks_lo + off), qf[s], sacc, 0, 0, 0);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qlo[s], sacc, 0, 0, 0);
        }
        dpacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_h8(Vs + off), df[s], dpacc, 0, 0, 0);
      }
      // sacc[r] / dpacc[r]: key kb*32 + 8*(r/4) + 4g + r%4, query q
      float ds[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const bool masked = kb == qb && (8 * (r >> 2) + 4 * g + (r & 3)) > ql;
        const float p = masked ? 0.f : __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], sp, -lse2));
        ds[r] = p * (dpacc[r] - dd) * a.scale_ds;
      }
#pragma unroll
      for (int jh = 0; jh < 2; jh++) {
        half8 bf;
#pragma unroll
        for (int u = 0; u < 8; u++) bf[u] = (half_t)ds[8 * jh + u];
        const int k0 = kb * 32 + 16 * jh + 4 * g;
        dq0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_t8(Kt, ST, ql, k0), bf, dq0, 0, 0, 0);
        dq1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_t8(Kt, ST, 32 + ql, k0), bf, dq1, 0, 0, 0);
      }
    }
    float dv[2][16];
#pragma unroll
    for (int r = 0; r < 16; r++) { dv[0][r] = dq0[r]; dv[1][r] = dq1[r]; }
    qk_post(dv, a.qkv + t * D3 + h * HD, q, g, a);
    store_row(a.dqkv + t * D3 + h * HD, dv, g);
  }
}

template <int SMAX, bool HILO, bool PERQ>
__global__ __launch_bounds__(PERQ ? 512 : 256) void attn_bwd_dkdv_kernel(AttnBwdArgs a) {
  constexpr int ST = SMAX + 4;
  __shared__ __attribute__((aligned(16))) half_t Qs[SMAX * HD];
  __shared__ __attribute__((aligned(16))) half_t Qt[HD * ST];
  __shared__ __attribute__((aligned(16))) half_t dOs[SMAX * HD];
  __shared__ __attribute__((aligned(16))) half_t dOt[HD * ST];
  __shared__ __attribute__((aligned(16))) float lse_s[SMAX];
  __shared__ __attribute__((aligned(16))) float dl_s[SMAX];
  const int S = a.S, NH = a.NH, D = NH * HD, D3 = 3 * D;
  const int h = blockIdx.y, b = blockIdx.z, nthr = blockDim.x, tid = threadIdx.x;
  const size_t tok0 = (size_t)b * S;
  const half_t* base = a.qkvt + tok0 * D3;
  stage_rows(Qs, base + h * HD, D3, S, tid, nthr);
  stage_T(Qt, ST, base + h * HD, D3, S, tid, nthr);
  stage_rows(dOs, a.dout + tok0 * D + h * HD, D, S, tid, nthr);
  stage_T(dOt, ST, a.dout + tok0 * D + h * HD, D, S, tid, nthr);
  for (int j = tid; j < S; j += nthr) {
    lse_s[j] = a.lse[(tok0 + j) * NH + h] * kL2E;
    dl_s[j] = a.delta[(tok0 + j) * NH + h];
  }
  __syncthreads();

  const int lane = tid & 63, wave = tid >> 6, nw = nthr >> 6;
  const int nkb = S / 32, npairs = nkb / 2;
  const int slots = PERQ ? nw / 2 : nw, slot = PERQ ? wave % slots : wave;
  const int pair = blockIdx.x * slots + slot;
  if (pair >= npairs) return;
  const int g = lane >> 5, kl = lane & 31;
  const float sp = a.scale_p * kL2E;
  const int which0 = PERQ ? wave / slots : 0, which1 = PERQ ? which0 + 1 : 2;

  for (int which = which0; which < which1; which++) {
    const int kb = which == 0 ? pair : nkb - 1 - pair;
    const int key = kb * 32 + kl;
    const size_t t = tok0 + key;
    half8 kf[4], klo[4], vf[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int d0 = s * 16 + g * 8;
      kf[s] = ld_h8(base + (size_t)key * D3 + D + h * HD + d0);
      if constexpr (HILO) klo[s] = ld_h8(a.qkvt_lo + t * 2 * D + D + h * HD + d0);
      vf[s] = ld_h8(base + (size_t)key * D3 + 2 * D + h * HD + d0);
    }
    floatx16 dk0, dk1, dv0, dv1;
#pragma unroll
    for (int r = 0; r < 16; r++) { dk0[r] = 0.f; dk1[r] = 0.f; dv0[r] = 0.f; dv1[r] = 0.f; }
    for (int qb = kb; qb < nkb; qb++) {
      floatx16 sacc, dpacc;
#pragma unroll
      for (int r = 0; r < 16; r++) { sacc[r] = 0.f; dpacc[r] = 0.f; }
      const int qrow = qb * 32 + kl;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const int off = qrow * HD + swz(qrow, s * 2 + g) * 8;
        const half8 qv = ld_h8(Qs + off);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qv, kf[s], sacc, 0, 0, 0);
        if constexpr (HILO) {
          const half8 ql = ld_h8(a.qkvt_lo + (tok0 + qrow) * 2 * D + h * HD + s * 16 + g * 8);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ql, kf[s], sacc, 0, 0, 0);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qv, klo[s], sacc, 0, 0, 0);
        }
        dpacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_h8(dOs + off), vf[s], dpacc, 0, 0, 0);
      }
      // sacc[r] / dpacc[r]: query qb*32 + 8*(r/4) + 4g + r%4, key `key`
      float pr[16], ds[16];
#pragma unroll
      for (int rq = 0; rq < 4; rq++) {
        const int q0 = qb * 32 + 8 * rq + 4 * g;
        const float4 l4 = *reinterpret_cast<const float4*>(lse_s + q0);
        const float4 d4 = *reinterpret_cast<const float4*>(dl_s + q0);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dl[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int r = 4 * rq + u;
          const bool masked = qb == kb && kl > (8 * rq + 4 * g + u);
          const float p = masked ? 0.f : __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], sp, -lv[u]));
          pr[r] = p;
          ds[r] = p * (dpacc[r] - dl[u]) * a.scale_ds;
        }
      }
#pragma unroll
      for (int jh = 0; jh < 2; jh++) {
        half8 pf, sf;
#pragma unroll
        for (int u = 0; u < 8; u++) {
          pf[u] = (half_t)pr[8 * jh + u];
          sf[u] = (half_t)ds[8 * jh + u];
        }
        const int q0 = qb * 32 + 16 * jh + 4 * g;
        dv0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_t8(dOt, ST, kl, q0), pf, dv0, 0, 0, 0);
        dv1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_t8(dOt, ST, 32 + kl, q0), pf, dv1, 0, 0, 0);
        dk0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_t8(Qt, ST, kl, q0), sf, dk0, 0, 0, 0);
        dk1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_t8(Qt, ST, 32 + kl, q0), sf, dk1, 0, 0, 0);
      }
    }
    float dkv[2][16], dvv[2][16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      dkv[0][r] = dk0[r]; dkv[1][r] = dk1[r];
      dvv[0][r] = dv0[r]; dvv[1][r] = dv1[r];
    }
    qk_post(dkv, a.qkv + t * D3 + D + h * HD, key, g, a);
    store_row(a.dqkv + t * D3 + D + h * HD, dkv, g);
    store_row(a.dqkv + t * D3 + 2 * D + h * HD, dvv, g);
  }
}

}  // namespace

hipError_t attention_bwd(const AttnBwdArgs& a, hipStream_t stream) {
  if (a.S <= 0 || a.S % 64 != 0 || a.S > 256 || a.NH <= 0 || a.nseq <= 0) return hipErrorInvalidValue;
  const int npairs = a.S / 64;
  const int nw = npairs < 4 ? npairs : 4;
  dim3 grid((npairs + nw - 1) / nw, a.NH, a.nseq);
  // ANE_ATT_BWD_PERQ=0: one wave per pair of blocks (4-wave blocks)
  static const bool perq = [] {
    const char* f = getenv("ANE_ATT_BWD_PERQ");
    return !f || atoi(f) != 0;
  }();
  if (a.hilo) {
    if (!a.qkvt_lo) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_bwd_dq_kernel<256, true, false>), grid, dim3(64 * nw), 0, stream, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<256, true, false>), grid, dim3(64 * nw), 0, stream, a);
  } else if (perq) {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<256, false, true>), grid, dim3(128 * nw), 0, stream, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<256, false, true>), grid, dim3(128 * nw), 0, stream, a);
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<256, false, false>), grid, dim3(64 * nw), 0, stream, a);
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<256, false, false>), grid, dim3(64 * nw), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace ane
