// Fused causal attention forward, head_dim 64 (reference: causalAttentionCF,
// ane/common.go:61-89, with RoPE ane/train_util.go:204-224 and QK-norm
// ane/common.go:199-227 applied in-kernel; value embeddings
// ane/train_full.go:1035-1059 added while V is staged).
//
// One workgroup per (sequence, head, group of q-block pairs).  The whole
// sequence's K (after RoPE / QK-norm) and V^T are staged once in LDS; each
// wave then owns two 32-row q-blocks (i, nqb-1-i) so every wave walks the
// same number of causal key blocks.  Scores are computed transposed,
// S^T = K Q^T, which leaves each lane holding 16 keys of ONE query: the
// online-softmax statistics are per lane (plus one xor-32 exchange), and
// the probabilities are already in the B-operand layout of O^T = V^T P^T,
// so P never leaves registers.
//
// The reference fills masked scores with -65504 and takes exp in float64,
// which yields exactly 0 for every masked key; skipping masked keys is the
// same function.
#include <type_traits>

#include "attention.h"

namespace ane {

namespace {

constexpr int HD = 64;

// One key chunk (dims 8 ch .. 8 ch + 7 of key row j) from its fp16 load and
// angles: RoPE (+ QK-norm: the 8 consecutive lanes that hold one row's
// chunks combine their sums of squares), fp16 (+ the fp16 residual with
// HILO) into the row's swizzled LDS slot, and, from the block that writes
// them (wt), the training copies (qkvt / qkvt_lo) of token tok0 + j, head h.
template <bool HILO>
__device__ __forceinline__ void k_chunk_store(const AttnArgs& a, const half8& raw, const float4& cs4, const float4& sn4,
                                              int j, int ch, half_t* Ks, half_t* Ks_lo, size_t tok0, int h, bool wt) {
  const int D = a.NH * HD, D3 = 3 * D;
  const float csv[4] = {cs4.x, cs4.y, cs4.z, cs4.w};
  const float snv[4] = {sn4.x, sn4.y, sn4.z, sn4.w};
  float f[8];
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const float e = (float)raw[2 * p], o = (float)raw[2 * p + 1];
    f[2 * p] = e * csv[p] - o * snv[p];
    f[2 * p + 1] = o * csv[p] + e * snv[p];
  }
  if (a.qknorm) {
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < 8; p++) ss += f[p] * f[p];
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    ss += __shfl_xor(ss, 4, 64);
    const float sc = 1.2f / sqrtf(ss * (1.0f / HD) + 1e-5f);
#pragma unroll
    for (int p = 0; p < 8; p++) f[p] *= sc;
  }
  half8 w, wl;
#pragma unroll
  for (int p = 0; p < 8; p++) {
    w[p] = (half_t)f[p];
    wl[p] = (half_t)(f[p] - (float)w[p]);
  }
  st_h8(Ks + j * HD + swz(j, ch) * 8, w);
  if constexpr (HILO) st_h8(Ks_lo + j * HD + swz(j, ch) * 8, wl);
  if (a.qkvt && wt) st_h8(a.qkvt + (tok0 + j) * D3 + D + h * HD + ch * 8, w);
  if (a.qkvt_lo && wt) st_h8(a.qkvt_lo + (tok0 + j) * 2 * D + D + h * HD + ch * 8, wl);
}

// One V block (keys 8 kc .. 8 kc + 7, dims 8 dc .. 8 dc + 7) from its 8 row
// loads: value embeddings added (VE layers), transposed into V^T rows of
// stride VST, and, from the block that writes it (wt), the training copy of v.
__device__ __forceinline__ void v_block_store(const AttnArgs& a, half8 (&raw)[8], int kc, int dc, int h, size_t tok0,
                                              half_t* Vt, int VST, bool wt) {
  const int D = a.NH * HD, D3 = 3 * D;
  if (a.ve_x) {
    float v[8][8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      const int j = kc * 8 + jj;
#pragma unroll
      for (int i = 0; i < 8; i++) v[jj][i] = (float)raw[jj][i];
      const float* xr = a.ve_x + (tok0 + j) * D;
      float gp = 0.f;
#pragma unroll
      for (int c2 = 0; c2 < 12; c2++) gp += a.ve_gate[h * 12 + c2] * xr[c2];
      const float gate = 3.0f / (1.0f + __expf(-gp));
      const int tk = a.tokens[tok0 + j];
      if (tk < a.vocab) {
        const float* er = a.ve_embed + (size_t)tk * D + h * HD + dc * 8;
#pragma unroll
        for (int i = 0; i < 8; i++) v[jj][i] += gate * er[i];
      }
#pragma unroll
      for (int i = 0; i < 8; i++) raw[jj][i] = (half_t)v[jj][i];
    }
  }
  // 8 x 8 transpose of fp16 values (no conversion without value embeddings)
#pragma unroll
  for (int i = 0; i < 8; i++) {
    half4 lo, hi;
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      lo[jj] = raw[jj][i];
      hi[jj] = raw[jj + 4][i];
    }
    half_t* dst = Vt + (dc * 8 + i) * VST + kc * 8;
    *reinterpret_cast<half4*>(dst) = lo;
    *reinterpret_cast<half4*>(dst + 4) = hi;
  }
  if (a.qkvt && wt) {
#pragma unroll
    for (int jj = 0; jj < 8; jj++) st_h8(a.qkvt + (tok0 + kc * 8 + jj) * D3 + 2 * D + h * HD + dc * 8, raw[jj]);
  }
}

// One wave: the 32 queries of q block qb of one (sequence, head) against
// keys 0 .. 32 qb + 31 staged in LDS (Ks rows, V^T rows of stride SMAX + 4).
// RSUM: the probabilities' row sum is taken by the matrix core, as a third
// P.V product against a constant tile whose row 0 is ones (two MFMAs per
// key block, 20 VGPRs), instead of 16 adds per key block; it then sums the
// fp16 probabilities P.V multiplies.
template <int SMAX, bool HILO, bool RSUM = false>
__device__ __forceinline__ void q_block(const AttnArgs& a, const half_t* base, size_t tok0, int h, int qb,
                                        const half_t* Ks, const half_t* Ks_lo, const half_t* Vt) {
  constexpr int VST = SMAX + 4;
  const int NH = a.NH, D = NH * HD, D3 = 3 * D;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 5, ql = lane & 31;
  const float l2e = 1.4426950408889634f;
  const float sl2 = a.scale * l2e;
  const int q = qb * 32 + ql;
  // Q fragment (B operand of S^T = K Q^T): dims s*16 + 8g + [0..7]
  float qf[4][8];
  const half_t* qrow = base + (size_t)q * D3 + h * HD;
  half8 qraw[4];
  float4 qcs[4], qsn[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {  // all loads first
    const int d0 = s * 16 + g * 8;
    qraw[s] = ld_h8(qrow + d0);
    qcs[s] = *reinterpret_cast<const float4*>(a.rope_cos + q * 32 + d0 / 2);
    qsn[s] = *reinterpret_cast<const float4*>(a.rope_sin + q * 32 + d0 / 2);
  }
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const float csv[4] = {qcs[s].x, qcs[s].y, qcs[s].z, qcs[s].w};
    const float snv[4] = {qsn[s].x, qsn[s].y, qsn[s].z, qsn[s].w};
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const float e = (float)qraw[s][2 * p], o = (float)qraw[s][2 * p + 1];
      qf[s][2 * p] = e * csv[p] - o * snv[p];
      qf[s][2 * p + 1] = o * csv[p] + e * snv[p];
    }
  }
  if (a.qknorm) {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int p = 0; p < 8; p++) ss += qf[s][p] * qf[s][p];
    ss += __shfl_xor(ss, 32, 64);
    const float sc = 1.2f / sqrtf(ss * (1.0f / HD) + 1e-5f);
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int p = 0; p < 8; p++) qf[s][p] *= sc;
  }
  half8 qfrag[4], qlo[4];
#pragma unroll
  for (int s = 0; s < 4; s++)
#pragma unroll
    for (int p = 0; p < 8; p++) {
      qfrag[s][p] = (half_t)qf[s][p];
      qlo[s][p] = (half_t)(qf[s][p] - (float)qfrag[s][p]);
    }
  if (a.qkvt) {
#pragma unroll
    for (int s = 0; s < 4; s++) st_h8(a.qkvt + (tok0 + q) * D3 + h * HD + s * 16 + g * 8, qfrag[s]);
  }
  if (a.qkvt_lo) {
#pragma unroll
    for (int s = 0; s < 4; s++) st_h8(a.qkvt_lo + (tok0 + q) * 2 * D + h * HD + s * 16 + g * 8, qlo[s]);
  }

  floatx16 o0, o1, o2;
#pragma unroll
  for (int r = 0; r < 16; r++) { o0[r] = 0.f; o1[r] = 0.f; o2[r] = 0.f; }
  half8 ones_row;  // A operand [32 rows][16 k]: row 0 ones, the rest zero
#pragma unroll
  for (int u = 0; u < 8; u++) ones_row[u] = (half_t)(ql == 0 ? 1.f : 0.f);
  // m: the reference maximum (scaled, log2 units) of the exponentials in
  // lsum and o.  It is raised only when a block's maximum exceeds it by
  // more than kRescale (or on the first block), so o is rescaled rarely;
  // in between the exponentials stay below 2^kRescale.  Any m gives the
  // same o / lsum; the final lse uses the m actually applied.
  constexpr float kRescale = 8.f;
  float m = -INFINITY, lsum = 0.f;

  // K fragments are read one key block ahead (issued before the softmax
  // of the current block) and V fragments right after the score MFMAs, so
  // the LDS latency hides behind the softmax instead of stalling the MFMAs.
  half8 kf[4];
  auto load_k = [&](int kb) {
    const int krow = kb * 32 + ql;
#pragma unroll
    for (int s = 0; s < 4; s++) kf[s] = ld_h8(Ks + krow * HD + swz(krow, s * 2 + g) * 8);
  };
  auto block = [&](auto diag_c, int kb) {
    constexpr bool DIAG = decltype(diag_c)::value;
    floatx16 sacc;
#pragma unroll
    for (int r = 0; r < 16; r++) sacc[r] = 0.f;
    const int krow = kb * 32 + ql;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[s], qfrag[s], sacc, 0, 0, 0);
      if constexpr (HILO) {
        const int off = krow * HD + swz(krow, s * 2 + g) * 8;
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld_h8(Ks_lo + off), qfrag[s], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[s], qlo[s], sacc, 0, 0, 0);
      }
    }
    half8 v0[2], v1[2];
#pragma unroll
    for (int jh = 0; jh < 2; jh++) {
      const int k0 = kb * 32 + 16 * jh + 4 * g;
      const half_t* r0 = Vt + ql * VST + k0;
      const half_t* r1 = Vt + (32 + ql) * VST + k0;
      const half4 a0 = *reinterpret_cast<const half4*>(r0), a1 = *reinterpret_cast<const half4*>(r0 + 8);
      const half4 b0 = *reinterpret_cast<const half4*>(r1), b1 = *reinterpret_cast<const half4*>(r1 + 8);
#pragma unroll
      for (int u = 0; u < 4; u++) {
        v0[jh][u] = a0[u]; v0[jh][u + 4] = a1[u];
        v1[jh][u] = b0[u]; v1[jh][u + 4] = b1[u];
      }
    }
    if constexpr (!DIAG) load_k(kb + 1);  // kb < qb: the next block exists
    // sacc[r]: raw score of key kb*32 + 8*(r/4) + 4g + r%4, query q; the
    // diagonal block masks keys after q (their exponentials are exactly 0,
    // as the reference's -65504 fill gives after its float64 exp)
    if constexpr (DIAG) {
#pragma unroll
      for (int r = 0; r < 16; r++)
        if ((8 * (r >> 2) + 4 * g + (r & 3)) > ql) sacc[r] = -INFINITY;
    }
    float mloc = sacc[0];
#pragma unroll
    for (int r = 1; r < 16; r++) mloc = fmaxf(mloc, sacc[r]);
    mloc = fmaxf(mloc, xor32_f(mloc)) * sl2;  // scale > 0 keeps the order
    if (__any(mloc > m + kRescale)) {
      const float mnew = fmaxf(m, mloc);
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      if constexpr (RSUM) {
        o2[0] *= alpha;  // the only nonzero element: row 0 of the sum tile
      } else {
        lsum *= alpha;
      }
#pragma unroll
      for (int r = 0; r < 16; r++) { o0[r] *= alpha; o1[r] *= alpha; }
      m = mnew;
    }
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], sl2, -m));
      sacc[r] = p;
      if constexpr (!RSUM) ps += p;
    }
    if constexpr (!RSUM) lsum += ps;
#pragma unroll
    for (int jh = 0; jh < 2; jh++) {
      half8 pf;
#pragma unroll
      for (int u = 0; u < 8; u++) pf[u] = (half_t)sacc[8 * jh + u];
      o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v0[jh], pf, o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v1[jh], pf, o1, 0, 0, 0);
      if constexpr (RSUM) o2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones_row, pf, o2, 0, 0, 0);
    }
  };
  load_k(0);
  for (int kb = 0; kb < qb; kb++) block(std::false_type{}, kb);
  block(std::true_type{}, qb);
  if constexpr (RSUM) {
    // row 0 of the sum tile sits in o2[0] of lanes 0..31 (the query's lane of the lower half)
    const float other = xor32_f(o2[0]);
    lsum = g == 0 ? o2[0] : other;
  } else {
    lsum += xor32_f(lsum);
  }
  const float inv = 1.0f / lsum;
  half_t* orow = a.out + (tok0 + q) * D + h * HD;
#pragma unroll
  for (int rr = 0; rr < 4; rr++) {
    half4 w0, w1;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      w0[u] = (half_t)(o0[4 * rr + u] * inv);
      w1[u] = (half_t)(o1[4 * rr + u] * inv);
    }
    *reinterpret_cast<half4*>(orow + 8 * rr + 4 * g) = w0;
    *reinterpret_cast<half4*>(orow + 32 + 8 * rr + 4 * g) = w1;
  }
  if (a.lse && g == 0) a.lse[(tok0 + q) * NH + h] = (m + log2f(lsum)) / l2e;
}

// HILO: scores from split operands q = q_hi + q_lo, k = k_hi + k_lo (each
// fp16), s = q_hi.k_hi + q_lo.k_hi + q_hi.k_lo, i.e. ~fp32 accuracy.  Used
// where the scores are large enough for fp16 rounding of q and k to matter
// (the reference's scale-1 recompute, ane/train_full.go:268-269).
// PERQ: one q block per wave (blocks of 2 x pairs waves: wave w takes the
// first block of pair slot w % slots if w < slots, else the second), so a
// pair's two q blocks run on two waves side by side instead of one after
// the other on one wave; 128 VGPRs, so that two 8-wave blocks share a CU.
template <int SMAX, bool HILO, bool PERQ>
__device__ __forceinline__ void attn_fwd_body(const AttnArgs& a) {
  __shared__ __attribute__((aligned(16))) half_t Ks[SMAX * HD];
  __shared__ __attribute__((aligned(16))) half_t Ks_lo[HILO ? SMAX * HD : 8];
  constexpr int VST = SMAX + 4;  // V^T row stride (halves): 2-way-free b64 reads
  __shared__ __attribute__((aligned(16))) half_t Vt[HD * VST];

  const int S = a.S, NH = a.NH, D = NH * HD, D3 = 3 * D;
  const size_t pf_part = ((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  const size_t pf_parts = (size_t)gridDim.x * gridDim.y * gridDim.z;
  const int nthr = blockDim.x, tid = threadIdx.x;
  const int slots = PERQ ? nthr >> 7 : nthr >> 6;  // q-block pairs a block's waves cover
  // Block -> (sequence b, head h, q-block pairs [p0, p0 + np)).  Grid
  // (pair groups, NH, nseq), or with split_from > 0 a 1-D grid: heads below
  // split_from whole, the rest as two half blocks each.
  int hl, p0, np;
  if (a.split_from > 0) {
    const int u = blockIdx.x, half = (S / 64) / 2;
    if (u < a.split_from) {
      hl = u; p0 = 0; np = 2 * half;
    } else {
      hl = a.split_from + (u - a.split_from) / 2; p0 = ((u - a.split_from) & 1) * half; np = half;
    }
  } else {
    hl = blockIdx.z * NH + blockIdx.y; p0 = blockIdx.x * slots; np = slots;
  }
  const int h = hl % NH, b = hl / NH;
  const bool first = p0 == 0;  // the block that writes qkvt of its head
  const size_t tok0 = (size_t)b * S;
  const half_t* base = a.qkv + tok0 * D3;

  // The thread's first V block (8 keys x 8 dims) is loaded ahead, in flight
  // with the first K batch; the prefetch of the next GEMM's weights is
  // issued after both and consumed once the staging is done.
  const int nkc = S / 8;
  half8 vpre[8];
  if (!PERQ && tid < S) {  // PERQ: register budget of 128; V is loaded where it is staged
    const int kc = tid % nkc, dc = tid / nkc;
#pragma unroll
    for (int jj = 0; jj < 8; jj++) vpre[jj] = ld_h8(base + (size_t)(kc * 8 + jj) * D3 + 2 * D + h * HD + dc * 8);
  }

  // ---- stage K: RoPE (+ QK-norm), swizzled rows of 64 halves ----------------
  // Batches of KB chunks per thread: every global load of a batch (the K
  // chunk and its cos / sin as float4) is issued before the first use, so
  // the batch pays one memory latency instead of one per chunk.
  constexpr int KB = PERQ ? 4 : 8;  // PERQ: 512 threads cover S = 256 in one batch of 4
  Prefetch pf{};
  for (int c0 = tid; c0 < S * 8; c0 += KB * nthr) {
    half8 raw[KB];
    float4 cs4[KB], sn4[KB];
#pragma unroll
    for (int u = 0; u < KB; u++) {
      const int c = c0 + u * nthr;
      if (c < S * 8) {
        const int j = c >> 3, ch = c & 7;
        raw[u] = ld_h8(base + (size_t)j * D3 + D + h * HD + ch * 8);
        cs4[u] = *reinterpret_cast<const float4*>(a.rope_cos + j * 32 + ch * 4);
        sn4[u] = *reinterpret_cast<const float4*>(a.rope_sin + j * 32 + ch * 4);
      }
    }
    if (!PERQ && c0 == tid) pf = prefetch_begin(a.pf, a.pf_bytes, pf_part, pf_parts);
#pragma unroll
    for (int u = 0; u < KB; u++) {
      const int c = c0 + u * nthr;
      if (c >= S * 8) break;
      const int j = c >> 3, ch = c & 7;
      k_chunk_store<HILO>(a, raw[u], cs4[u], sn4[u], j, ch, Ks, Ks_lo, tok0, h, first);
    }
  }

  // ---- stage V^T (8 keys x 8 dims per thread), value embeddings added --------
  // (PERQ: threads past S, which stage no V block, stream the block's slice
  // of the next GEMM's weights meanwhile)
  if (PERQ && tid >= S && a.pf && a.pf_bytes >= 16) {
    const uint4* q = reinterpret_cast<const uint4*>(a.pf);
    const size_t n16 = a.pf_bytes / 16, per = (n16 + pf_parts - 1) / pf_parts;
    const size_t i1 = min(n16, (pf_part + 1) * per);
    uint32_t x = 0;
    for (size_t i = pf_part * per + (tid - S); i < i1; i += nthr - S) {
      const uint4 v = q[i];
      x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    asm volatile("" ::"v"(x));
  }
  for (int blk = tid; blk < S; blk += nthr) {
    const int kc = blk % nkc, dc = blk / nkc;
    half8 raw[8];
#pragma unroll
    for (int jj = 0; jj < 8; jj++)
      raw[jj] = !PERQ && blk == tid ? vpre[jj] : ld_h8(base + (size_t)(kc * 8 + jj) * D3 + 2 * D + h * HD + dc * 8);
    v_block_store(a, raw, kc, dc, h, tok0, Vt, VST, first);
  }
  __syncthreads();
  if (!PERQ) prefetch_end(pf, a.pf, a.pf_bytes, pf_part, pf_parts);

  // ---- per wave: q-block pair ------------------------------------------------
  const int wave = tid >> 6;
  const int nqb = S / 32, npairs = nqb / 2;
  const int slot = PERQ ? wave % slots : wave;
  const int pair = p0 + slot;
  if (slot >= np || pair >= npairs) return;
  const int which0 = PERQ ? wave / slots : 0, which1 = PERQ ? which0 + 1 : 2;
  for (int which = which0; which < which1; which++)
    q_block<SMAX, HILO>(a, base, tok0, h, which == 0 ? pair : nqb - 1 - pair, Ks, Ks_lo, Vt);
}

template <int SMAX, bool HILO, bool PERQ>
__global__ __launch_bounds__(PERQ ? 512 : 256) __attribute__((amdgpu_waves_per_eu(PERQ ? 4 : 1)))
void attn_fwd_kernel(AttnArgs a) {
  attn_fwd_body<SMAX, HILO, PERQ>(a);
}

// 1.5 heads per block, one 12-wave block per CU, for 256 < heads <= 384 at
// S = 256 without split operands (the B32 forward: 384 heads).  Block c
// stages head c whole and, for c < 2 (heads - 256), half c % 2 of head
// 256 + c / 2 (its q-block pairs 0-1 or 2-3, which need keys up to q block
// 7 or 5), with all of its K, V and angle loads in one batch; then each wave
// runs one q block.  A q block qb costs qb + 1 key blocks: a whole-head block
// beside a half-head block (two blocks per CU) leaves 18 of them on two
// SIMDs and 9 on the other two, while this table gives each SIMD 12-14 (a
// block's waves are dealt to the CU's four SIMDs in turn, so waves w, w + 4
// and w + 8 share one; measured with the hardware wave ids).  Entry = head *
// 8 + q block (head 0 = the whole one), -1 = none.
__device__ constexpr int8_t kTask15[3][12] = {
    {7, 6, 5, 4, 0, 1, 2, 3, -1, -1, -1, -1},   // no half head
    {7, 15, 6, 14, 4, 3, 5, 2, 0, 1, 8, 9},     // half with q-block pairs 0, 1
    {7, 6, 13, 5, 11, 12, 4, 10, 0, 1, 2, 3}};  // half with q-block pairs 2, 3
constexpr int kWaves15 = 12;

__device__ __forceinline__ void attn_fwd15_body(const AttnArgs& a) {
  constexpr int SMAX = 256, VST = SMAX + 4, NT = 64 * kWaves15;
  __shared__ __attribute__((aligned(16))) half_t Ks[2][SMAX * HD];
  __shared__ __attribute__((aligned(16))) half_t Vt[2][HD * VST];
  const int S = SMAX, NH = a.NH, D = NH * HD, D3 = 3 * D;
  const int tid = threadIdx.x, c = blockIdx.x;
  const int heads = a.nseq * NH;
  const bool has_b = c < 2 * (heads - 256);
  const int p0b = (c & 1) * 2;
  const int rows_b = has_b ? (p0b == 0 ? S : S - 64) : 0;
  int hh[2];
  size_t tok[2];
  const half_t* base[2];
  const int hl[2] = {c, 256 + (c >> 1)};
#pragma unroll
  for (int i = 0; i < 2; i++) {
    hh[i] = hl[i] % NH;
    tok[i] = (size_t)(hl[i] / NH) * S;
    base[i] = a.qkv + tok[i] * D3;
  }
  const bool wt[2] = {true, p0b == 0};  // the blocks that write each head's training copies

  // ---- one batch: K chunks (with angles), one V block per thread -------------
  const int nk = (S + rows_b) * 8, nv = S + rows_b;
  constexpr int KB = (2 * SMAX * 8 + NT - 1) / NT;
  half8 raw[KB];
  float4 cs4[KB], sn4[KB];
#pragma unroll
  for (int u = 0; u < KB; u++) {
    const int k = tid + u * NT;
    if (k < nk) {
      const int hd = k >= S * 8, j = (k - hd * S * 8) >> 3, ch = k & 7;
      raw[u] = ld_h8(base[hd] + (size_t)j * D3 + D + hh[hd] * HD + ch * 8);
      cs4[u] = *reinterpret_cast<const float4*>(a.rope_cos + j * 32 + ch * 4);
      sn4[u] = *reinterpret_cast<const float4*>(a.rope_sin + j * 32 + ch * 4);
    }
  }
  half8 vraw[8];
  int vh = 0, vkc = 0, vdc = 0;
  if (tid < nv) {
    vh = tid >= S;
    const int local = tid - vh * S, nkc = (vh ? rows_b : S) / 8;
    vkc = local % nkc;
    vdc = local / nkc;
#pragma unroll
    for (int jj = 0; jj < 8; jj++)
      vraw[jj] = ld_h8(base[vh] + (size_t)(vkc * 8 + jj) * D3 + 2 * D + hh[vh] * HD + vdc * 8);
  } else if (a.pf && a.pf_bytes >= 16) {
    // threads without a V block stream the block's slice of the next GEMM's weights
    const uint4* q = reinterpret_cast<const uint4*>(a.pf);
    const size_t n16 = a.pf_bytes / 16, per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t i1 = min(n16, (c + 1) * per);
    uint32_t x = 0;
    for (size_t i = c * per + (tid - nv); i < i1; i += NT - nv) {
      const uint4 v = q[i];
      x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    asm volatile("" ::"v"(x));
  }
#pragma unroll
  for (int u = 0; u < KB; u++) {
    const int k = tid + u * NT;
    if (k >= nk) break;
    const int hd = k >= S * 8, j = (k - hd * S * 8) >> 3, ch = k & 7;
    k_chunk_store<false>(a, raw[u], cs4[u], sn4[u], j, ch, Ks[hd], nullptr, tok[hd], hh[hd], wt[hd]);
  }
  if (tid < nv) v_block_store(a, vraw, vkc, vdc, hh[vh], tok[vh], Vt[vh], VST, wt[vh]);
  __syncthreads();

  const int t = kTask15[has_b ? 1 + (p0b != 0) : 0][tid >> 6];
  if (t < 0) return;
  const int hd = t >> 3;
  q_block<SMAX, false, true>(a, base[hd], tok[hd], hh[hd], t & 7, Ks[hd], nullptr, Vt[hd]);
}

}  // namespace

// The per-q-block kernel (S <= 256, no split operands) under a C name for
// a host that loads the code object itself (ane_kernels.h): 512 threads.
extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void ane_k_attn_fwd(AttnArgs a) {
  attn_fwd_body<256, false, true>(a);
}

// 1.5 heads per block (above): 768 threads, grid 256; the library launches it
// under this name too.
extern "C" __global__ __launch_bounds__(64 * kWaves15) __attribute__((amdgpu_waves_per_eu(3)))
void ane_k_attn_fwd15(AttnArgs a) {
  attn_fwd15_body(a);
}

hipError_t attention_fwd(const AttnArgs& a, hipStream_t stream) {
  if (a.S <= 0 || a.S % 64 != 0 || a.S > 512 || a.NH <= 0 || a.nseq <= 0) return hipErrorInvalidValue;
  const int npairs = a.S / 64;
  const int nw = npairs < 4 ? npairs : 4;  // q-block pairs per block
  dim3 grid((npairs + nw - 1) / nw, a.NH, a.nseq);
  // ANE_ATT_PERQ=0: one wave per pair of q blocks (4-wave blocks)
  static const bool perq = [] {
    const char* f = getenv("ANE_ATT_PERQ");
    return !f || atoi(f) != 0;
  }();
  // One block of 4 pairs per head leaves 256 < heads < 512 unevenly spread
  // over the 256 CUs (two blocks on some, one on the rest): the heads past
  // 256 run as two half blocks, one beside each whole block.
  AttnArgs k = a;
  k.split_from = 0;
  const int heads = a.nseq * a.NH;
  if (npairs == 4 && heads > 256 && heads < 512) {
    k.split_from = 256;
    grid = dim3(256 + 2 * (heads - 256), 1, 1);
  }
  if (a.hilo && a.S > 256) return hipErrorInvalidValue;
  // ANE_ATT_15=0: the whole-head and half-head blocks above instead of 1.5 heads per block
  static const bool by15 = [] {
    const char* f = getenv("ANE_ATT_15");
    return !f || atoi(f) != 0;
  }();
  if (!a.hilo && perq && by15 && a.S == 256 && heads > 256 && heads <= 384) {
    k.split_from = 0;
    hipLaunchKernelGGL(ane_k_attn_fwd15, dim3(256), dim3(64 * kWaves15), 0, stream, k);
    return hipGetLastError();
  }
  if (a.hilo)
    hipLaunchKernelGGL((attn_fwd_kernel<256, true, false>), grid, dim3(64 * nw), 0, stream, k);
  else if (a.S <= 256 && perq)
    hipLaunchKernelGGL((attn_fwd_kernel<256, false, true>), grid, dim3(128 * nw), 0, stream, k);
  else if (a.S <= 256)
    hipLaunchKernelGGL((attn_fwd_kernel<256, false, false>), grid, dim3(64 * nw), 0, stream, k);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<512, false, false>), grid, dim3(64 * nw), 0, stream, k);
  return hipGetLastError();
}

}  // namespace ane
