// Decode kernels (see decode.h).  Decode steps are HBM- and latency-bound:
// the weights stream once per step through 64-row MFMA "skinny" GEMMs
// split over K, and the attention reads each sequence's K/V cache once,
// shared by the query heads of a key/value group.
#include <math.h>

#include <algorithm>

#include "decode.h"
#include "decode_dev.h"

namespace ane {

namespace {

// ---- classifier GEMM with the argmax epilogue ---------------------------------
// Block = one column group of 32 vocabulary rows x NWK waves splitting K,
// each wave holding at most two 64-wide k-windows, all loaded in one batch.
// MFMA 32x32x16 with rows = tokens (two tiles: tokens 0-31, 32-63) and
// columns = weight rows; both operands are stored fragment-major
// (decode.h), so each operand load is one contiguous 1 KB per wave.  The K
// partial sums meet in LDS and are added in wave order (deterministic);
// wave 0 then transposes the 64 x 32 logits through LDS and each lane scans
// the 32 columns of its token: (max, first index) per token and group.
template <int NWK>
__global__ __launch_bounds__(64 * NWK) void classifier_argmax_kernel(SkinnyArgs a) {
  // LDS: the partial sums of waves 1..NWK-1 (2048 floats each), then --
  // reusing the same array -- the 64 x 33 transpose tile, which is larger
  // than one wave's partials
  constexpr int NRED = NWK > 1 ? NWK - 1 : 1;
  constexpr int kTile = 64 * 33;
  __shared__ float lds[NRED * 2048 > kTile ? NRED * 2048 : kTile];
  const int tid = threadIdx.x, lane = tid & 63, kw = tid >> 6;
  const int cg = blockIdx.x;
  const int nwin = a.K / 64;
  const int w0 = (kw * nwin) / NWK, w1 = ((kw + 1) * nwin) / NWK;  // this wave's windows [w0, w1), <= 2
  const int row = lane & 31, h = lane >> 5;
  const int col = cg * 32 + row;
  // fragment (w, s): weights at ((cg * nwin + w) * 4 + s) KB, activations at
  // ((w * 4 + s) * 2 + tile) KB; lane l's 16 B at l * 16
  const half_t* wp = a.W + (size_t)cg * nwin * 2048 + lane * 8;
  const half_t* xp0 = a.X + lane * 8;
  // unconditional loads (window index clamped, the surplus copy zeroed)
  half8 w[8], p[8], q[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    const int f = min(w0 + (s >> 2), w1 - 1) * 4 + (s & 3);
    w[s] = ld_h8(wp + (size_t)f * 512);
    p[s] = ld_h8(xp0 + (size_t)f * 1024);
    q[s] = ld_h8(xp0 + (size_t)f * 1024 + 512);
  }
  if (w1 - w0 < 2) {  // one window: the second copy contributes zero
#pragma unroll
    for (int s = 4; s < 8; s++)
#pragma unroll
      for (int j = 0; j < 8; j++) w[s][j] = (half_t)0.f;
  }
  floatx16 c0, c1;
#pragma unroll
  for (int r = 0; r < 16; r++) { c0[r] = 0.f; c1[r] = 0.f; }
#pragma unroll
  for (int s = 0; s < 8; s++) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(p[s], w[s], c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(q[s], w[s], c1, 0, 0, 0);
  }
  if constexpr (NWK > 1) {
    if (kw > 0) {
      float* dst = lds + (kw - 1) * 2048;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        dst[r * 64 + lane] = c0[r];
        dst[(16 + r) * 64 + lane] = c1[r];
      }
    }
    __syncthreads();
  }
  if (kw != 0) return;
  if constexpr (NWK > 1) {
#pragma unroll 1
    for (int o = 1; o < NWK; o++) {
      const float* src = lds + (o - 1) * 2048;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        c0[r] += src[r * 64 + lane];
        c1[r] += src[(16 + r) * 64 + lane];
      }
    }
  }
  // c[r]: token 8*(r/4) + 4*h + r%4 (+32 for c1), column col.  Transpose
  // into tile[t][c] (row stride 33: conflict-free both ways), then lane t
  // scans its row.  Wave 0 is the only one left, and its reads of the other
  // waves' partials above are done.
  float* tile = lds;
  const bool valid = col < a.nvalid;
  // logits of inputs fp16(x * gain) carry the norm's per-token 1 / rms as a
  // factor; it is positive, so the argmax below is taken on the unscaled sums
  const float rr_lane = a.rr ? a.rr[lane] : 1.f;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int t = 8 * (r >> 2) + 4 * h + (r & 3);
    tile[t * 33 + row] = valid ? c0[r] : -INFINITY;
    tile[(t + 32) * 33 + row] = valid ? c1[r] : -INFINITY;
    if (a.logits) {  // uniform: the shuffles run on every lane
      const float s0 = __shfl(rr_lane, t, 64), s1 = __shfl(rr_lane, t + 32, 64);
      if (valid) {
        a.logits[(size_t)t * a.N + col] = c0[r] * s0;
        a.logits[(size_t)(t + 32) * a.N + col] = c1[r] * s1;
      }
    }
  }
  float v = tile[lane * 33];
  int idx = 0;
#pragma unroll
  for (int c = 1; c < 32; c++) {
    const float x = tile[lane * 33 + c];
    if (x > v) { v = x; idx = c; }  // strict: the first index wins ties
  }
  a.amax[(size_t)cg * kDecRows + lane] = make_float2(v, __int_as_float(cg * 32 + idx));
}

__global__ __launch_bounds__(256) void argmax_kernel(uint16_t* tok_out, uint16_t* hist, const int* step,
                                                     const float2* amax, int ngroups, int nb) {
  const int b = blockIdx.x, tid = threadIdx.x;
  float v = -INFINITY;
  int idx = 0x7fffffff;
  for (int g = tid; g < ngroups; g += 256) {
    const float2 p = amax[(size_t)g * kDecRows + b];
    const int pi = __float_as_int(p.y);
    if (p.x > v || (p.x == v && pi < idx)) { v = p.x; idx = pi; }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (ov > v || (ov == v && oi < idx)) { v = ov; idx = oi; }
  }
  __shared__ float sv[4];
  __shared__ int si[4];
  if ((tid & 63) == 0) { sv[tid >> 6] = v; si[tid >> 6] = idx; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; w++)
      if (sv[w] > v || (sv[w] == v && si[w] < idx)) { v = sv[w]; idx = si[w]; }
    tok_out[b] = (uint16_t)idx;
    if (hist) hist[(size_t)(*step) * nb + b] = (uint16_t)idx;
  }
}

__global__ void advance_kernel(int* ctr) {
  if (threadIdx.x == 0) {
    ctr[0] += 1;
    ctr[1] += 1;
    ctr[2] += 1;
  }
}

__global__ void set_ctr_kernel(int* ctr, int pos, int step) {
  if (threadIdx.x == 0) {
    ctr[0] = pos;
    ctr[1] = step;
  }
}

__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  const int tid = threadIdx.x;
  __syncthreads();  // red may still be read by a previous call
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// one block of 256 per row, D <= 1024
__global__ __launch_bounds__(256) void embed_norm_kernel(float* x, half_t* xn, const float* embed,
                                                         const uint16_t* tok, const float* g, int D, int V) {
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int tk = tok[b];
  float v[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    v[i] = (c < D && tk < V) ? embed[(size_t)tk * D + c] : 0.f;
    ss += v[i] * v[i];
  }
  ss = block_sum_256(ss, red);
  const float rr = 1.0f / sqrtf(ss / (float)D + 1e-5f);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    if (c < D) {
      x[(size_t)b * D + c] = v[i];
      xn[act_frag_off(b, c)] = (half_t)(v[i] * rr * g[c]);
    }
  }
}

__global__ __launch_bounds__(256) void norm_kernel(const float* x, half_t* xn, const float* g, int D) {
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  float v[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    v[i] = c < D ? x[(size_t)b * D + c] : 0.f;
    ss += v[i] * v[i];
  }
  ss = block_sum_256(ss, red);
  const float rr = 1.0f / sqrtf(ss / (float)D + 1e-5f);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    if (c < D) xn[act_frag_off(b, c)] = (half_t)(v[i] * rr * g[c]);
  }
}

// ---- split-K skinny GEMM -------------------------------------------------------
// One wave per block: column group cg (32 weight rows) x WPW consecutive
// 64-wide k-windows.  Every operand load is issued before the first MFMA;
// the 64 x 32 fp32 partial goes to part[kc][t][n].  The finish kernels
// below sum the K splits of a row in split order (deterministic) and apply
// the epilogue, so a decode-step GEMM spreads over hundreds of CUs instead
// of one block per column group.
template <int WPW>
__global__ __launch_bounds__(64) void skinny_part_kernel(const half_t* X, const half_t* W, float* part, int N,
                                                         int K) {
  const int cg = blockIdx.x, kc = blockIdx.y, lane = threadIdx.x;
  const int nwin = K / 64;
  const half_t* wp = W + (size_t)cg * nwin * 2048 + lane * 8;
  const half_t* xp = X + lane * 8;
  const int f0 = kc * WPW * 4;
  half8 w[4 * WPW], p[4 * WPW], q[4 * WPW];
#pragma unroll
  for (int s = 0; s < 4 * WPW; s++) {
    w[s] = ld_h8(wp + (size_t)(f0 + s) * 512);
    p[s] = ld_h8(xp + (size_t)(f0 + s) * 1024);
    q[s] = ld_h8(xp + (size_t)(f0 + s) * 1024 + 512);
  }
  floatx16 c0, c1;
#pragma unroll
  for (int r = 0; r < 16; r++) { c0[r] = 0.f; c1[r] = 0.f; }
#pragma unroll
  for (int s = 0; s < 4 * WPW; s++) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(p[s], w[s], c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(q[s], w[s], c1, 0, 0, 0);
  }
  // c[r]: token 8*(r/4) + 4*h + r%4 (+32 for c1), column cg*32 + lane%32
  float* dst = part + (size_t)kc * kDecRows * N + cg * 32 + (lane & 31);
  const int h = lane >> 5;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int t = 8 * (r >> 2) + 4 * h + (r & 3);
    dst[(size_t)t * N] = c0[r];
    dst[(size_t)(t + 32) * N] = c1[r];
  }
}

// sum over the ks <= kMaxSplits splits of part[.][t][c], in split order;
// every load is issued before the first add (unconditional: the index is
// clamped and the surplus values are dropped), so the row pays one memory
// latency, not one per split
constexpr int kMaxSplits = 16;
__device__ __forceinline__ float split_sum(const float* part, int ks, int N, int t, int c) {
  float v[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++) v[s] = part[((size_t)min(s, ks - 1) * kDecRows + t) * N + c];
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++) acc += s < ks ? v[s] : 0.f;
  return acc;
}

// Wo / W2 finish: x[t] += sum of the splits (residual), then
// xn[t] = fp16(rmsnorm(x[t]) * g) in the fragment layout (the next GEMM's
// input: the FFN norm after Wo, the next layer's attention norm -- or the
// final norm -- after W2).  One block of 256 per row, D <= 1024.
__global__ __launch_bounds__(256) void finish_resid_norm_kernel(const float* part, int ks, float* x, half_t* xn,
                                                                const float* g, int D) {
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  float v[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    v[i] = 0.f;
    if (c < D) {
      v[i] = x[(size_t)b * D + c] + split_sum(part, ks, D, b, c);
      x[(size_t)b * D + c] = v[i];
    }
    ss += v[i] * v[i];
  }
  ss = block_sum_256(ss, red);
  const float rr = 1.0f / sqrtf(ss / (float)D + 1e-5f);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    if (c < D) xn[act_frag_off(b, c)] = (half_t)(v[i] * rr * g[c]);
  }
}

// W1|W3 finish: gate[t][j] = silu(h1) * h3 with W1 / W3 rows interleaved by
// 32 (h1 at column (j/32)*64 + j%32, h3 at +32), fragment layout.
__global__ __launch_bounds__(256) void finish_swiglu_kernel(const float* part, int ks, half_t* gate, int H) {
  const int t = blockIdx.x;  // blockIdx.y: a 256-column slice of the row
  for (int j = blockIdx.y * 256 + threadIdx.x; j < min(H, (int)(blockIdx.y + 1) * 256); j += blockDim.x) {
    const int c1 = (j >> 5) * 64 + (j & 31);
    const float h1 = split_sum(part, ks, 2 * H, t, c1), h3 = split_sum(part, ks, 2 * H, t, c1 + 32);
    gate[act_frag_off(t, j)] = (half_t)(h1 / (1.0f + __expf(-h1)) * h3);
  }
}

// ---- decode attention ---------------------------------------------------------
// Block (b, kv head, chunk) for a group of G query heads: 8 lanes per key
// (16 B each), 32 keys per pass, all K/V loads of the chunk in flight
// before the first use.  q.k by v_dot2_f32_f16 summed over the key's 8
// lanes with DPP row operations (no LDS traffic); scores of the G heads in
// LDS; per-head max / sum by one wave each; P.V by v_dot2 over key pairs,
// each thread's sums reduced across the 32 key lanes through LDS.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// sum over the aligned 8-lane group: quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror
__device__ __forceinline__ float sum8_dpp(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  return v;
}

// Over the 8 key groups of a wave (lanes l, l ^ 8, l ^ 16, l ^ 32 ...): each
// 8-lane group holds one value in all its lanes; every lane gets the result.
__device__ __forceinline__ float grp_max8(float v) {
  v = fmaxf(v, dpp_f<0x128>(v));  // row_ror:8 -- the other group of the 16-lane row
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, xor32_f(v));
}
__device__ __forceinline__ float grp_sum8(float v) {
  v += dpp_f<0x128>(v);
  v += __shfl_xor(v, 16, 64);
  return v + xor32_f(v);
}

// One block of NT threads per (sequence, kv head, key split): KP = NT / 8
// keys per pass, NIT passes, so a split holds at most KP * NIT keys.  With
// DIRECT (one split covers the context) the block normalises and writes att
// itself; otherwise it leaves (o, m, l) partials for dec_combine_kernel.
template <int G, int QS, int NT, int NIT, bool DIRECT>
__device__ __forceinline__ void dec_attn_body(const DecAttnArgs& a) {
  constexpr int KP = NT / 8;
  // pv reduction: NR groups of threads each sum KP / NR key lanes per output
  constexpr int NR = NT / (G * 64) < 8 ? NT / (G * 64) : 8;
  const int b = blockIdx.x, kvh = blockIdx.y, sp = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ctx = a.ctr[0] + 1;
  const int chunk = dec_chunk(ctx, a.nsplit);
  const int c0 = sp * chunk;
  if (c0 >= ctx) return;  // uniform over the block, before any barrier
  const int n = min(chunk, ctx - c0);
  __shared__ half_t qs[G][64];
  constexpr int NW = NT / 64;
  __shared__ __attribute__((aligned(16))) float pv[G][KP][64];
  __shared__ float red[NR][G * 64];
  __shared__ float wred[G][NW];  // per-wave maxima, then per-wave sums
  __shared__ __attribute__((aligned(16))) half_t knew[64], vnew[64];
  const float sl2 = a.scale * kL2E;
  const size_t cache0 = ((size_t)b * a.NKV + kvh) * a.max_ctx;
  half_t* Kb = a.kc + (cache0 + c0) * 64;
  half_t* Vb = a.vc + (cache0 + c0) * 64;
  const int kl = tid >> 3, d8 = tid & 7;
  // Projections of this step from the QKV partials, one column pair per
  // thread: q of the G heads (threads < 32 G) and, in the block whose split
  // holds position pos, the new k (next 32) and v (next 32).  Sum in split
  // order as the finish kernels do, RoPE on q and k.
  const int pos = ctx - 1;
  const bool own = pos - c0 < n;
  // Load order: the partials and RoPE factors first (the staging barrier
  // waits for them alone), then every K row, then every V row, so the
  // scores can be formed while the values are still arriving.  Unconditional
  // loads (indices clamped; keys past n unused); sched_barrier fences keep
  // the scheduler from reordering the groups.
  QkvProj<G, QS> qp;
  qp.issue(a, b, kvh, tid, pos, own);
  __builtin_amdgcn_sched_barrier(0);
  half8 kk[NIT], kv[NIT];
#pragma unroll
  for (int it = 0; it < NIT; it++) kk[it] = ld_h8(Kb + (size_t)min(kl + KP * it, n - 1) * 64 + d8 * 8);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int it = 0; it < NIT; it++) kv[it] = ld_h8(Vb + (size_t)min(kl + KP * it, n - 1) * 64 + d8 * 8);
  __builtin_amdgcn_sched_barrier(0);
  qp.finish(a, tid, qs, knew, vnew, Kb, Vb, pos - c0);
  __syncthreads();
  // Row pos is the last row of its split (pos - c0 = n - 1), and every
  // lane whose key index is >= n read it too (clamped): all of them take the
  // new k / v, because the row they read is stale -- in a fresh cache it may
  // hold any bit pattern, and a NaN there would survive the zero
  // probability those lanes carry into P.V.  The substitution is a select
  // at each use: writing into kk / kv here would first wait for every load
  // still in flight into those registers.
  const int jrep = own ? pos - c0 : 1 << 30;
  half8 kn = {}, vn = {};
  if (own) {
    kn = ld_h8(knew + d8 * 8);
    vn = ld_h8(vnew + d8 * 8);
  }
  // this lane's 8 dims of each head as fp16 pairs (fp16 products exact in fp32)
  half2v qr[G][4];
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      qr[h][i][0] = qs[h][d8 * 8 + 2 * i];
      qr[h][i][1] = qs[h][d8 * 8 + 2 * i + 1];
    }
  // Scores stay in registers (every lane of a key's 8-lane group holds the
  // key's score); keys past n score -inf.  The block maximum per head comes
  // from a cross-group wave max and one LDS pass over the waves.
  float sreg[NIT][G], mx[G];
#pragma unroll
  for (int h = 0; h < G; h++) mx[h] = -INFINITY;
#pragma unroll
  for (int it = 0; it < NIT; it++) {
    const int j = kl + KP * it;
    const half8 kx = j >= jrep ? kn : kk[it];
#pragma unroll
    for (int h = 0; h < G; h++) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        half2v kp;
        kp[0] = kx[2 * i];
        kp[1] = kx[2 * i + 1];
        s = __builtin_amdgcn_fdot2(qr[h][i], kp, s, false);
      }
      s = sum8_dpp(s);
      sreg[it][h] = j < n ? s * sl2 : -INFINITY;
      mx[h] = fmaxf(mx[h], sreg[it][h]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
    mx[h] = grp_max8(mx[h]);
    if (lane == 0) wred[h][wave] = mx[h];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; h++) {
    float m = wred[h][0];
#pragma unroll
    for (int w = 1; w < NW; w++) m = fmaxf(m, wred[h][w]);
    mx[h] = m;
  }
  // P.V over this thread's key pairs (it, it + 1): v_dot2 of (p_it, p_it+1)
  // with (v_it[i], v_it+1[i]).  Probabilities are rounded to fp16 (they feed
  // fp16 dot products); the normaliser sums the same rounded values.  Keys
  // past n (and a missing last pass) have p = 0.
  float acc[G][8], ls[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    ls[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) acc[h][i] = 0.f;
  }
#pragma unroll
  for (int it = 0; it < NIT; it += 2) {
    const bool pair = it + 1 < NIT;
    const int j0 = kl + KP * it, j1 = j0 + KP;
    const half8 v0 = j0 >= jrep ? vn : kv[it];
    const half8 v1 = pair ? (j1 >= jrep ? vn : kv[pair ? it + 1 : it]) : half8{};
    half2v vp[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      vp[i][0] = v0[i];
      vp[i][1] = v1[i];
    }
#pragma unroll
    for (int h = 0; h < G; h++) {
      half2v pp;
      pp[0] = (half_t)__builtin_amdgcn_exp2f(sreg[it][h] - mx[h]);
      pp[1] = pair ? (half_t)__builtin_amdgcn_exp2f(sreg[pair ? it + 1 : it][h] - mx[h]) : (half_t)0.f;
      ls[h] += (float)pp[0] + (float)pp[1];
#pragma unroll
      for (int i = 0; i < 8; i++) acc[h][i] = __builtin_amdgcn_fdot2(pp, vp[i], acc[h][i], false);
    }
  }
  // sums over the KP key lanes kl, through LDS: NR groups of G*64 threads
  // each add KP / NR lanes, then the groups' sums are added in order; the
  // normaliser by a cross-group wave sum and the per-wave sums
#pragma unroll
  for (int h = 0; h < G; h++) {
    float4* dst = reinterpret_cast<float4*>(&pv[h][kl][d8 * 8]);
    dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    ls[h] = grp_sum8(ls[h]);
  }
  __syncthreads();  // wred (the maxima) fully read above: reuse it for the sums
#pragma unroll
  for (int h = 0; h < G; h++)
    if (lane == 0) wred[h][wave] = ls[h];
  constexpr int KPR = (KP + NR - 1) / NR;
  if (tid < NR * G * 64) {
    const int r = tid / (G * 64), hd = tid % (G * 64), h = hd >> 6, d = hd & 63;
    float o = 0.f;
#pragma unroll 8
    for (int k = r * KPR; k < min(KP, (r + 1) * KPR); k++) o += pv[h][k][d];
    red[r][hd] = o;
  }
  __syncthreads();
  if (tid < G * 64) {
    const int h = tid >> 6, d = tid & 63;
    float o = 0.f, l = 0.f;
#pragma unroll
    for (int r = 0; r < NR; r++) o += red[r][tid];
#pragma unroll
    for (int w = 0; w < NW; w++) l += wred[h][w];
    if constexpr (DIRECT) {
      a.att[act_frag_off(b, (kvh * G + h) * 64 + d)] = (half_t)(o / l);
    } else {
      float* out = a.part + (((size_t)b * a.NH + kvh * G + h) * a.nsplit + sp) * 66;
      out[d] = o;
      if (d == 0) { out[64] = mx[h]; out[65] = l; }
    }
  }
}

// Narrow form (batches too small for the wide one): 256 threads, 8 passes
// of 32 keys = kDecChunk keys per split, QS = 8 or kMaxSplits.
template <int G>
__global__ __launch_bounds__(256) void dec_attn_kernel8(DecAttnArgs a) {
  dec_attn_body<G, 8, 256, kDecChunk / 32, false>(a);
}
template <int G>
__global__ __launch_bounds__(256) void dec_attn_kernel16(DecAttnArgs a) {
  dec_attn_body<G, kMaxSplits, 256, kDecChunk / 32, false>(a);
}
// Wide form: one 1024-thread block (one per CU) per (sequence, kv head)
// holds up to kDecWideChunk keys with every K / V load in flight at once;
// used when the batch alone gives enough blocks to fill the chip.
template <int G, bool DIRECT>
__global__ __launch_bounds__(1024) void dec_attn_wide_kernel(DecAttnArgs a) {
  __shared__ WideLds lds;
  dec_attn_wide_body<G, DIRECT, false>(a, blockIdx.x, blockIdx.y, blockIdx.z, lds);
}

__global__ __launch_bounds__(64) void dec_combine_kernel(DecAttnArgs a) {
  const int b = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int ctx = a.ctr[0] + 1;
  const int chunk = dec_chunk(ctx, a.nsplit);
  const int ns = (ctx + chunk - 1) / chunk;
  const float* p = a.part + ((size_t)b * a.NH + h) * a.nsplit * 66;
  float M = -INFINITY;
  for (int s = 0; s < ns; s++) M = fmaxf(M, p[s * 66 + 64]);
  float num = 0.f, den = 0.f;
  for (int s = 0; s < ns; s++) {
    const float w = exp2f(p[s * 66 + 64] - M);
    num += w * p[s * 66 + d];
    den += w * p[s * 66 + 65];
  }
  a.att[act_frag_off(b, h * 64 + d)] = (half_t)(num / den);
}

// ---- prefill ------------------------------------------------------------------
__global__ __launch_bounds__(128) void kv_write_kernel(half_t* qkv, half_t* kc, half_t* vc, const float* rc,
                                                       const float* rs, int seq0, int S, int NH, int NKV,
                                                       int max_ctx) {
  const int t = blockIdx.x;  // token row of the chunk
  const int sl = t / S, pos = t % S, b = seq0 + sl;
  const int D = NH * 64, KVD = NKV * 64, N1 = D + 2 * KVD;
  half_t* row = qkv + (size_t)t * N1;
  for (int c2 = threadIdx.x; c2 < N1 / 2; c2 += blockDim.x) {
    const int col = 2 * c2;
    half2v w = *reinterpret_cast<const half2v*>(row + col);
    if (col < D + KVD) {
      const int i = (col & 63) >> 1;
      const float cs = rc[pos * 32 + i], sn = rs[pos * 32 + i];
      const float e = (float)w[0], o = (float)w[1];
      w[0] = (half_t)(e * cs - o * sn);
      w[1] = (half_t)(o * cs + e * sn);
    }
    if (col < D) {
      *reinterpret_cast<half2v*>(row + col) = w;
    } else {
      const bool isk = col < D + KVD;
      const int c = col - (isk ? D : D + KVD);
      const int kvh = c >> 6, d = c & 63;
      half_t* dst = (isk ? kc : vc) + (((size_t)b * NKV + kvh) * max_ctx + pos) * 64 + d;
      *reinterpret_cast<half2v*>(dst) = w;
    }
  }
}

// Block = 4 waves x 32 queries of one (sequence, query head); keys and V^T
// staged through LDS in chunks of KC; scores transposed (S^T = K Q^T) so
// each lane keeps 16 keys of one query and P feeds O^T = V^T P^T from
// registers (the layout of the training forward kernel).
constexpr int KC = 128;
constexpr int VSTP = KC + 4;
__global__ __launch_bounds__(256) void prefill_attn_kernel(PrefillAttnArgs a) {
  __shared__ __attribute__((aligned(16))) half_t Ks[KC * 64];
  __shared__ __attribute__((aligned(16))) half_t Vt[64 * VSTP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qt = blockIdx.x, h = blockIdx.y, sl = blockIdx.z;
  const int S = a.S, G = a.NH / a.NKV, kvh = h / G, b = a.seq0 + sl;
  const int qb = qt * 4 + wave;
  const bool active = qb * 32 < S;
  const int kend = min(S, (qt + 1) * 128);
  const int g = lane >> 5, ql = lane & 31;
  const int q = qb * 32 + ql;
  const size_t cache0 = ((size_t)b * a.NKV + kvh) * a.max_ctx;

  half8 qfrag[4];
  if (active) {
    const half_t* qrow = a.qkv + ((size_t)sl * S + q) * a.ldq + h * 64;
#pragma unroll
    for (int s = 0; s < 4; s++) qfrag[s] = ld_h8(qrow + s * 16 + g * 8);
  }
  floatx16 o0, o1;
#pragma unroll
  for (int r = 0; r < 16; r++) { o0[r] = 0.f; o1[r] = 0.f; }
  float m = -INFINITY, lsum = 0.f;
  const float sl2 = a.scale * kL2E;

  for (int c0 = 0; c0 < kend; c0 += KC) {
    __syncthreads();  // previous chunk fully consumed
    for (int c = tid; c < KC * 8; c += 256) {
      const int j = c >> 3, ch = c & 7;
      half8 v;
      if (c0 + j < S) v = ld_h8(a.kc + (cache0 + c0 + j) * 64 + ch * 8);
      else
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (half_t)0.f;
      st_h8(Ks + j * 64 + swz(j, ch) * 8, v);
    }
    if (tid < KC) {  // 8 keys x 8 dims per thread
      const int kc8 = tid % (KC / 8), dc = tid / (KC / 8);
      half8 v[8];
#pragma unroll
      for (int jj = 0; jj < 8; jj++) {
        const int j = c0 + kc8 * 8 + jj;
        if (j < S) v[jj] = ld_h8(a.vc + (cache0 + j) * 64 + dc * 8);
        else
#pragma unroll
          for (int i = 0; i < 8; i++) v[jj][i] = (half_t)0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; i++) {
        half4 lo, hi;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          lo[jj] = v[jj][i];
          hi[jj] = v[jj + 4][i];
        }
        half_t* dst = Vt + (dc * 8 + i) * VSTP + kc8 * 8;
        *reinterpret_cast<half4*>(dst) = lo;
        *reinterpret_cast<half4*>(dst + 4) = hi;
      }
    }
    __syncthreads();
    if (!active) continue;
    for (int kbl = 0; kbl < KC / 32; kbl++) {
      const int kb = c0 / 32 + kbl;
      if (kb > qb) break;
      floatx16 sacc;
#pragma unroll
      for (int r = 0; r < 16; r++) sacc[r] = 0.f;
      const int krow = kbl * 32 + ql;
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const half8 kf = ld_h8(Ks + krow * 64 + swz(krow, s * 2 + g) * 8);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qfrag[s], sacc, 0, 0, 0);
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        float sv = sacc[r] * sl2;
        if (kb == qb && (8 * (r >> 2) + 4 * g + (r & 3)) > ql) sv = -INFINITY;
        sacc[r] = sv;
        mloc = fmaxf(mloc, sv);
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
      const float mnew = fmaxf(m, mloc);
      const float alpha = exp2f(m - mnew);
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float p = exp2f(sacc[r] - mnew);
        sacc[r] = p;
        ps += p;
      }
      lsum = lsum * alpha + ps;
#pragma unroll
      for (int r = 0; r < 16; r++) { o0[r] *= alpha; o1[r] *= alpha; }
      m = mnew;
#pragma unroll
      for (int jh = 0; jh < 2; jh++) {
        half8 pf;
#pragma unroll
        for (int u = 0; u < 8; u++) pf[u] = (half_t)sacc[8 * jh + u];
        const int k0 = kbl * 32 + 16 * jh + 4 * g;
        const half_t* r0 = Vt + ql * VSTP + k0;
        const half_t* r1 = Vt + (32 + ql) * VSTP + k0;
        const half4 a0 = *reinterpret_cast<const half4*>(r0), a1 = *reinterpret_cast<const half4*>(r0 + 8);
        const half4 b0 = *reinterpret_cast<const half4*>(r1), b1 = *reinterpret_cast<const half4*>(r1 + 8);
        half8 v0, v1;
#pragma unroll
        for (int u = 0; u < 4; u++) {
          v0[u] = a0[u]; v0[u + 4] = a1[u];
          v1[u] = b0[u]; v1[u + 4] = b1[u];
        }
        o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v0, pf, o0, 0, 0, 0);
        o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v1, pf, o1, 0, 0, 0);
      }
    }
  }
  if (!active) return;
  lsum += __shfl_xor(lsum, 32, 64);
  const float inv = 1.0f / lsum;
  half_t* orow = a.out + ((size_t)sl * S + q) * (a.NH * 64) + h * 64;
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
}

__global__ __launch_bounds__(256) void weight_frag_kernel(half_t* dst, const half_t* src, int K, size_t nchunks) {
  const int nf = (K / 64) * 4;  // fragments per 32-row group
  for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < nchunks; c += (size_t)gridDim.x * 256) {
    const int lane = (int)(c & 63);
    const size_t fg = c >> 6;
    const int f = (int)(fg % nf);
    const size_t g = fg / nf;
    const size_t row = g * 32 + (lane & 31);
    const int k = (f >> 2) * 64 + 32 * (lane >> 5) + 8 * (f & 3);
    st_h8(dst + c * 8, ld_h8(src + row * K + k));
  }
}

__global__ __launch_bounds__(256) void gather_last_kernel(float* dst, const float* src, int S, int D) {
  const int i = blockIdx.x;
  const float* s = src + ((size_t)i * S + S - 1) * D;
  for (int c = threadIdx.x; c < D; c += 256) dst[(size_t)i * D + c] = s[c];
}

}  // namespace

// Waves per block splitting K (K <= 1024, the decoder's dim limit: at most
// 16 windows): exactly two k-windows each when the window count allows one
// of the built sizes (no zeroed surplus window, whose weights and
// activations would still be read), else the smallest power of two that
// leaves at most two.  Results: 1, 2, 3, 4, 6 or 8.
int classifier_kwaves(int K) {
  const int nwin = K / 64;
  if (nwin == 2 || nwin == 6 || nwin == 12) return nwin / 2;
  int w = 1;
  while (w < 8 && (nwin + w - 1) / w > 2) w <<= 1;
  return w;
}

hipError_t classifier_argmax(const SkinnyArgs& a, hipStream_t s) {
  if (a.N <= 0 || a.N % 32 || a.K <= 0 || a.K % 64 || a.K > 1024 || a.nb < 1 || a.nb > kDecRows)
    return hipErrorInvalidValue;
  const int nwk = classifier_kwaves(a.K);
  if ((a.K / 64 + nwk - 1) / nwk > 2) return hipErrorInvalidValue;  // K too long for one block
  const dim3 grid(a.N / 32);
  switch (nwk) {
    case 1: hipLaunchKernelGGL(classifier_argmax_kernel<1>, grid, dim3(64), 0, s, a); break;
    case 2: hipLaunchKernelGGL(classifier_argmax_kernel<2>, grid, dim3(128), 0, s, a); break;
    case 4: hipLaunchKernelGGL(classifier_argmax_kernel<4>, grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL(classifier_argmax_kernel<3>, grid, dim3(192), 0, s, a); break;
    case 6: hipLaunchKernelGGL(classifier_argmax_kernel<6>, grid, dim3(384), 0, s, a); break;
    case 8: hipLaunchKernelGGL(classifier_argmax_kernel<8>, grid, dim3(512), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Most windows per wave (fewest splits for the finish kernels to sum) that
// still gives >= 128 one-wave blocks; measured at the decode bench shapes
// against a 256-block floor: 0.698 -> 0.689 ms per step.
int skinny_splits(int N, int K) {
  const int nwin = K / 64, ng = N / 32;
  for (int wpw : {4, 2, 1})
    if (nwin % wpw == 0 && nwin / wpw <= kMaxSplits && (long)ng * (nwin / wpw) >= 128) return nwin / wpw;
  for (int wpw : {1, 2, 4})  // fewest windows per wave within kMaxSplits splits
    if (nwin % wpw == 0 && nwin / wpw <= kMaxSplits) return nwin / wpw;
  return -1;  // skinny_partials refuses
}

hipError_t skinny_partials(const half_t* X, const half_t* W, float* part, size_t part_cap, int N, int K,
                           hipStream_t s) {
  if (N <= 0 || N % 32 || K <= 0 || K % 64) return hipErrorInvalidValue;
  const int ks = skinny_splits(N, K);
  if (ks <= 0 || (size_t)ks * kDecRows * N > part_cap) return hipErrorInvalidValue;
  const int wpw = (K / 64) / ks;
  const dim3 grid(N / 32, ks);
  switch (wpw) {
    case 1: hipLaunchKernelGGL((skinny_part_kernel<1>), grid, dim3(64), 0, s, X, W, part, N, K); break;
    case 2: hipLaunchKernelGGL((skinny_part_kernel<2>), grid, dim3(64), 0, s, X, W, part, N, K); break;
    case 4: hipLaunchKernelGGL((skinny_part_kernel<4>), grid, dim3(64), 0, s, X, W, part, N, K); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t skinny_finish_resid_norm(const float* part, int N, int K, float* x, half_t* xn, const float* g, int nb,
                                    hipStream_t s) {
  if (N > 1024 || nb < 1 || nb > kDecRows) return hipErrorInvalidValue;
  hipLaunchKernelGGL(finish_resid_norm_kernel, dim3(nb), dim3(256), 0, s, part, skinny_splits(N, K), x, xn, g, N);
  return hipGetLastError();
}

hipError_t skinny_finish_swiglu(const float* part, int N, int K, half_t* gate, int nb, hipStream_t s) {
  if (N % 64 || nb < 1 || nb > kDecRows) return hipErrorInvalidValue;
  hipLaunchKernelGGL(finish_swiglu_kernel, dim3(nb, (N / 2 + 255) / 256), dim3(256), 0, s, part, skinny_splits(N, K),
                     gate, N / 2);
  return hipGetLastError();
}

hipError_t argmax_reduce(uint16_t* tok_out, uint16_t* hist, const int* step, const float2* amax, int ngroups,
                         int nb, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(nb), dim3(256), 0, s, tok_out, hist, step, amax, ngroups, nb);
  return hipGetLastError();
}

hipError_t dec_advance(int* ctr, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, s, ctr);
  return hipGetLastError();
}

hipError_t dec_set_ctr(int* ctr, int pos, int step, hipStream_t s) {
  hipLaunchKernelGGL(set_ctr_kernel, dim3(1), dim3(64), 0, s, ctr, pos, step);
  return hipGetLastError();
}

hipError_t dec_embed_norm(float* x, half_t* xn, const float* embed, const uint16_t* tok, const float* g, int nb,
                          int D, int V, hipStream_t s) {
  if (D > 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(embed_norm_kernel, dim3(nb), dim3(256), 0, s, x, xn, embed, tok, g, D, V);
  return hipGetLastError();
}

hipError_t dec_norm(const float* x, half_t* xn, const float* g, int nb, int D, hipStream_t s) {
  if (D > 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(norm_kernel, dim3(nb), dim3(256), 0, s, x, xn, g, D);
  return hipGetLastError();
}

bool dec_attention_fusable(const DecAttnArgs& a) {
  if (a.NKV <= 0 || a.NH % a.NKV || a.NH / a.NKV > kGMax) return false;
  const int wsplit = (a.max_ctx + kDecWideChunk - 1) / kDecWideChunk;
  return wsplit == 1 && wsplit <= a.nsplit && (a.form == 1 || (a.form == 0 && a.nb * a.NKV >= kDecWideMinBlocks));
}

hipError_t dec_attention(const DecAttnArgs& a, hipStream_t s) {
  const int G = a.NH / a.NKV;
  if (a.NH % a.NKV || G > kGMax) return hipErrorInvalidValue;
  if (a.qkv_ks < 1 || a.qkv_ks > kMaxSplits) return hipErrorInvalidValue;
  const bool qs8 = a.qkv_ks <= 8;
  // wide form: enough (sequence, kv head) blocks to fill the chip, or forced
  const int wsplit = (a.max_ctx + kDecWideChunk - 1) / kDecWideChunk;
  const bool wide = qs8 && wsplit <= a.nsplit &&
                    (a.form == 1 || (a.form == 0 && a.nb * a.NKV >= kDecWideMinBlocks));
  if (wide) {
    DecAttnArgs w = a;
    w.nsplit = wsplit;
    const dim3 gw(a.nb, a.NKV, wsplit);
#define DEC_WIDE(G_)                                                                        \
  if (wsplit == 1) hipLaunchKernelGGL((dec_attn_wide_kernel<G_, true>), gw, dim3(1024), 0, s, w); \
  else hipLaunchKernelGGL((dec_attn_wide_kernel<G_, false>), gw, dim3(1024), 0, s, w);
    switch (G) {
      case 1: DEC_WIDE(1); break;
      case 2: DEC_WIDE(2); break;
      case 3: DEC_WIDE(3); break;
      default: DEC_WIDE(4); break;
    }
#undef DEC_WIDE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || wsplit == 1) return e;
    hipLaunchKernelGGL(dec_combine_kernel, dim3(a.nb, a.NH), dim3(64), 0, s, w);
    return hipGetLastError();
  }
  const dim3 grid(a.nb, a.NKV, a.nsplit);
#define DEC_ATTN(G_)                                                                   \
  if (qs8) hipLaunchKernelGGL((dec_attn_kernel8<G_>), grid, dim3(256), 0, s, a);        \
  else hipLaunchKernelGGL((dec_attn_kernel16<G_>), grid, dim3(256), 0, s, a);
  switch (G) {
    case 1: DEC_ATTN(1); break;
    case 2: DEC_ATTN(2); break;
    case 3: DEC_ATTN(3); break;
    default: DEC_ATTN(4); break;
  }
#undef DEC_ATTN
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(dec_combine_kernel, dim3(a.nb, a.NH), dim3(64), 0, s, a);
  return hipGetLastError();
}

hipError_t prefill_kv_write(half_t* qkv, half_t* kc, half_t* vc, const float* rope_cos, const float* rope_sin,
                            int seq0, int nseq, int S, int NH, int NKV, int max_ctx, hipStream_t s) {
  hipLaunchKernelGGL(kv_write_kernel, dim3(nseq * S), dim3(128), 0, s, qkv, kc, vc, rope_cos, rope_sin, seq0, S,
                     NH, NKV, max_ctx);
  return hipGetLastError();
}

hipError_t prefill_attention(const PrefillAttnArgs& a, hipStream_t s) {
  if (a.S <= 0 || a.S % 32 || a.S > a.max_ctx || a.NH % a.NKV) return hipErrorInvalidValue;
  dim3 grid((a.S + 127) / 128, a.NH, a.nseq);
  hipLaunchKernelGGL(prefill_attn_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t weight_to_frag(half_t* dst, const half_t* src, int N, int K, hipStream_t s) {
  if (N <= 0 || N % 32 || K <= 0 || K % 64) return hipErrorInvalidValue;
  const size_t nchunks = (size_t)N * K / 8;
  const int blocks = (int)std::min<size_t>((nchunks + 255) / 256, 4096);
  hipLaunchKernelGGL(weight_frag_kernel, dim3(blocks), dim3(256), 0, s, dst, src, K, nchunks);
  return hipGetLastError();
}

hipError_t gather_last_rows(float* dst, const float* src, int nseq, int S, int D, hipStream_t s) {
  hipLaunchKernelGGL(gather_last_kernel, dim3(nseq), dim3(256), 0, s, dst, src, S, D);
  return hipGetLastError();
}

}  // namespace ane
