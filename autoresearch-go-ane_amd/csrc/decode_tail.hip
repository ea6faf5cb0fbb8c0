// The decode step's per-layer GEMM chain in one launch: Wo (+ residual),
// W1|W3 (+ SwiGLU), W2 (+ residual) and the next layer's QKV projection.
//
// A grid-wide barrier costs ~11 us on MI355X (one device-scope atomic per
// block, serialised) against ~1.7 us for a kernel boundary in a replayed
// graph, so the phases are not separated by barriers.  Instead every block
// (16 waves) owns one 32-column group of a GEMM over the whole K -- the waves
// split K and meet in LDS, in wave order -- applies the epilogue itself and
// counts itself done; a consumer block waits only on the done counter of the
// phase it reads:
//   * blocks are laid out phase by phase (Wo, W13, W2, QKV, then one block
//     that forms the next 1/rms), one per CU and all resident at once (the
//     host checks the occupancy), so a wait never blocks its own producer;
//   * every load a block needs after its wait is issued together (the
//     activations, the residual slice, the norm sums): one device-coherent
//     round trip per phase;
//   * each block loads its weight fragments before it waits: the layer's
//     weights stream from HBM while the first phase computes;
//   * counters only grow: a use is identified by the epoch
//     E = global step * layers + layer + 1, so nothing is cleared between uses.
// (Splitting K over blocks with a last-arriver fix-up per group kept more
// blocks busy but cost two more device-coherent round trips per GEMM:
// measured 31 us per layer against 25 for one launch per GEMM.)
// RMSNorm is applied after the GEMMs it feeds: a block's activations are
// fp16(x * gain), and the per-token 1 / rms -- which needs every column group
// of the residual -- scales the (linear) GEMM output instead: in the SwiGLU
// epilogue (W1|W3) and in the attention's QKV finish (via rr_next).
// Every wait is bounded; a timeout sets *err, and later launches exit at once.
//
// Two forms of the waits (TailArgs::poll).  With done counters, a producer
// drains its stores and counts itself done, and a consumer polls the
// counter, then loads.  In the data-polling form (the default) the data a
// phase hands on goes through one of two buffer sets whose dwords start as
// kTailStale, a pattern no store writes; a consumer wave re-reads its inputs
// until none is stale, and every launch resets the set the previous one
// used.  That form can also run the next layer's decode attention in the
// same launch (TailArgs::b_att): those blocks come after the chain's, issue
// their K / V loads at once and poll q.
//
// Memory: the data blocks exchange inside the launch (the residual, the norm
// sums, the fp16 activation fragments) is stored and loaded device-coherent
// (cache policy sc1: written through to, and read from, the level shared by
// all XCDs), and a block drains its own stores (s_waitcnt vmcnt(0)) before it
// counts an arrival.  The agent-scope release / acquire fences would instead
// write back / invalidate the whole XCD L2 at every arrival: measured 1.7 ms
// per decode step against 0.62 for one launch per GEMM.
#include <math.h>

#include "decode.h"
#include "decode_dev.h"

namespace ane {

namespace {

__device__ __forceinline__ unsigned ld_relaxed(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls *c until it reaches `target` (wave 0; at most `limit` polls of ~100
// cycles); the block reads the producers' data afterwards with
// device-coherent loads.  Returns false (block-uniform) after a timeout or
// when another block has failed; limit 0 fails at once (the host's way to
// exercise the error path).
__device__ bool wait_count(const unsigned* c, unsigned target, unsigned limit, int* err, int* sh) {
  if (threadIdx.x < 64) {
    int ok = limit != 0;
    unsigned spins = 0;
    // wrap-safe: the counters grow by the same amounts as the epoch targets,
    // modulo 2^32, and a counter trails its target by far less than 2^31
    while (ok && (int)(ld_relaxed(c) - target) < 0) {
      if (++spins > limit || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (threadIdx.x == 0) {
      if (!ok) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *sh = ok;
    }
  }
  __syncthreads();
  const bool ok = *sh != 0;
  asm volatile("" ::: "memory");
  return ok;
}

// After the block's epilogue stores: drain them, then count the block done.
__device__ void publish(unsigned* done) {
  drain_stores();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This wave's outcome into its flag (read after the next barrier by
// any_failed); a wave whose inputs never arrived also sets the launch's error.
__device__ __forceinline__ void wave_outcome(bool ok, int* err, int* wfail) {
  if (__lane_id() == 0) {
    wfail[threadIdx.x >> 6] = ok ? 0 : 1;
    if (!ok) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
__device__ __forceinline__ bool any_failed(const int* wfail) {
  int f = 0;
#pragma unroll
  for (int w = 0; w < 16; w++) f |= wfail[w];
  return f != 0;
}

// Windows [w0, w0 + nw) of wave `wave` when nwin windows are split over
// nwave waves (nw <= MAXW).
struct Span {
  int w0, nw;
};
template <int MAXW>
__device__ __forceinline__ Span wave_span(int nwin, int nwave, int wave) {
  const int a = wave * nwin / nwave, b = (wave + 1) * nwin / nwave;
  return Span{a, min(b - a, MAXW)};
}

// One wave's 64 x 32 partial over its windows: weights of column group cg
// (fragment-major, nwin windows per group) preloaded by load_w, activations
// X (activation fragments) loaded after the dependency wait by mma.
template <int MAXW>
struct WaveGemm {
  half8 w[4 * MAXW];
  floatx16 c0, c1;
  __device__ __forceinline__ void load_w(const half_t* W, int cg, int nwin, Span sp) {
    const half_t* wp = W + (size_t)cg * nwin * 2048 + threadIdx.x % 64 * 8;
#pragma unroll
    for (int s = 0; s < 4 * MAXW; s++) {
      const int f = (sp.w0 + min(s >> 2, max(sp.nw - 1, 0))) * 4 + (s & 3);
      w[s] = ld_h8(wp + (size_t)f * 512);
    }
  }
  // coherent: X was written inside this launch (device-coherent loads)
  __device__ __forceinline__ void mma(const half_t* X, Span sp, bool coherent) {
    const int lane8 = threadIdx.x % 64 * 8;
    half8 p[4 * MAXW], q[4 * MAXW];
#pragma unroll
    for (int s = 0; s < 4 * MAXW; s++) {
      const int f = (sp.w0 + min(s >> 2, max(sp.nw - 1, 0))) * 4 + (s & 3);
      if (coherent) {
        p[s] = ld_ch8(X, (uint32_t)(f * 1024 + lane8));
        q[s] = ld_ch8(X, (uint32_t)(f * 1024 + 512 + lane8));
      } else {
        p[s] = ld_h8(X + (size_t)f * 1024 + lane8);
        q[s] = ld_h8(X + (size_t)f * 1024 + 512 + lane8);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; r++) { c0[r] = 0.f; c1[r] = 0.f; }
#pragma unroll
    for (int s = 0; s < 4 * MAXW; s++) {
      if ((s >> 2) < sp.nw) {  // wave-uniform: surplus windows contribute nothing
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(p[s], w[s], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(q[s], w[s], c1, 0, 0, 0);
      }
    }
  }
  // Data-polling form: the activation fragments into px / qx (device-coherent
  // loads); true when no dword of this lane's is stale.  compute() then
  // runs the MFMAs on them.
  half8 px[4 * MAXW], qx[4 * MAXW];
  __device__ __forceinline__ bool load_x(const half_t* X, Span sp) {
    // recomputed each round (opaque to loop-invariant hoisting): the load
    // offsets then hold no register while the round's data is in flight
    int lane8 = threadIdx.x % 64 * 8;
    asm volatile("" : "+v"(lane8));
#pragma unroll
    for (int s = 0; s < 4 * MAXW; s++) {
      const int f = (sp.w0 + min(s >> 2, max(sp.nw - 1, 0))) * 4 + (s & 3);
      px[s] = ld_ch8(X, (uint32_t)(f * 1024 + lane8));
      qx[s] = ld_ch8(X, (uint32_t)(f * 1024 + 512 + lane8));
    }
    bool ok = true;
#pragma unroll
    for (int s = 0; s < 4 * MAXW; s++) {
      ok &= fresh8(px[s]);
      ok &= fresh8(qx[s]);
    }
    return ok;
  }
  __device__ __forceinline__ void compute(Span sp) {
#pragma unroll
    for (int r = 0; r < 16; r++) { c0[r] = 0.f; c1[r] = 0.f; }
#pragma unroll
    for (int s = 0; s < 4 * MAXW; s++) {
      if ((s >> 2) < sp.nw) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(px[s], w[s], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(qx[s], w[s], c1, 0, 0, 0);
      }
    }
  }
  // this wave's partial into red[wave] ([64 rows][32 columns])
  __device__ __forceinline__ void to_lds(float (*red)[64][32]) const {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, col = lane & 31;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int t = 8 * (r >> 2) + 4 * h + (r & 3);
      red[wave][t][col] = c0[r];
      red[wave][t + 32][col] = c1[r];
    }
  }
};

// element pair i (of 1024) of a 64 x 32 tile: row i / 16, columns 2 (i % 16), +1
__device__ __forceinline__ float2 sum_waves(float (*red)[64][32], int w0, int w1) {
  const int row = threadIdx.x >> 4, col = (threadIdx.x & 15) * 2;
  float2 v = make_float2(red[w0][row][col], red[w0][row][col + 1]);
  for (int w = w0 + 1; w < w1; w++) {
    v.x += red[w][row][col];
    v.y += red[w][row][col + 1];
  }
  return v;
}

__device__ __forceinline__ void st_frag2(half_t* X, int t, int k, float a, float b) {
  half2v h;
  h[0] = (half_t)a;
  h[1] = (half_t)b;
  __builtin_amdgcn_raw_buffer_store_b32(not_stale(__builtin_bit_cast(uint32_t, h), 0x7E007E00u), rsrc(X),
                                        (uint32_t)act_frag_off(t, k) * 2u, 0, kSc1);
}

// This thread's element pair of a 64 x 32 tile of column group cg: row
// tid / 16, columns 32 cg + 2 (tid % 16), +1; its index in x [64][D].
__device__ __forceinline__ int x_index(int cg, int D) {
  return (threadIdx.x >> 4) * D + cg * 32 + (threadIdx.x & 15) * 2;
}

// Residual epilogue of column group cg (Wo, W2): xv (this thread's element
// pair of x[:, cg], loaded before the GEMM) += acc and is stored; ssq[cg][t] = sum
// over the group's 32 columns of the new x^2; xg = fp16(x * gain) fragments
// for the consumer.
__device__ void resid_epilogue(float2 acc, float2 xv, int cg, float* x, int D, float* ssq, half_t* xg,
                               const float* gain) {
  const int row = threadIdx.x >> 4, c = cg * 32 + (threadIdx.x & 15) * 2;
  const uint32_t xi = (uint32_t)x_index(cg, D);
  const __amdgpu_buffer_rsrc_t rx = rsrc(x);
  xv.x += acc.x;
  xv.y += acc.y;
  __builtin_amdgcn_raw_buffer_store_b32(not_stale(__float_as_uint(xv.x), 0x7FC00000u), rx, xi * 4u, 0, kSc1);
  __builtin_amdgcn_raw_buffer_store_b32(not_stale(__float_as_uint(xv.y), 0x7FC00000u), rx, xi * 4u + 4u, 0, kSc1);
  float ss = xv.x * xv.x + xv.y * xv.y;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o, 64);  // the row's 16 threads
  if ((threadIdx.x & 15) == 0) st_c1(ssq, (uint32_t)(cg * 64 + row), ss);
  st_frag2(xg, row, c, xv.x * gain[c], xv.y * gain[c + 1]);
}

// 1 / rms of row `row` from the ncg <= 32 column-group sums of squares: all
// loads in flight together, added in group order
__device__ __forceinline__ float rr_of(const float* ssq, int ncg, int row, int D) {
  float v[32];
#pragma unroll
  for (int g = 0; g < 32; g++) v[g] = ld_c1(ssq, (uint32_t)(min(g, ncg - 1) * 64 + row));
  float s = 0.f;
#pragma unroll
  for (int g = 0; g < 32; g++) s += g < ncg ? v[g] : 0.f;
  return 1.0f / sqrtf(s / (float)D + 1e-5f);
}

constexpr int kTailWaves = 16;

// Device-coherent loads of two floats per thread, base[e0] and base[e1],
// straight into LDS (buffer_load ... lds), so that no register is held while
// the GEMM's loads are in flight: lane l of wave w lands at dst[0][64 w + l]
// and dst[1][64 w + l].  They are not in the compiler's wait counts: the
// caller issues them before any compiler-tracked load it waits on, and waits
// (vmcnt(0)) before reading dst.
__device__ __forceinline__ unsigned lds_rows(float (*dst)[64 * kTailWaves], int j) {
  return __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_ptr_t)&dst[j][(threadIdx.x >> 6) * 64]);
}
__device__ __forceinline__ void two_to_lds(const float* base, uint32_t e0, uint32_t e1, unsigned lds0,
                                           unsigned lds1) {
  const __amdgpu_buffer_rsrc_t rs = rsrc(base);
  asm volatile("" : "+v"(e0), "+v"(e1));  // formed where used (see load_x)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen sc1 lds" ::"s"(lds0), "v"(e0 * 4u),
               "s"(rs)
               : "memory", "m0");
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen sc1 lds" ::"s"(lds1), "v"(e1 * 4u),
               "s"(rs)
               : "memory", "m0");
#pragma clang diagnostic pop
}
// This thread's x element pair of column group cg (x_index) -> xs[0][tid],
// xs[1][tid].
__device__ __forceinline__ void x_to_lds(const float* x, int cg, int D, float (*xs)[64 * kTailWaves]) {
  const uint32_t e = (uint32_t)x_index(cg, D);
  two_to_lds(x, e, e + 1, lds_rows(xs, 0), lds_rows(xs, 1));
}

// POLL: the data-polling form (TailArgs::poll): no done counters; each
// consumer wave re-reads its inputs until none is stale, so a phase costs the
// producers' stores reaching the shared level and one read round, instead of
// a store drain, a counter update, a counter read and then the data read.
constexpr int kTailLateAtt = 48;  // attention blocks of the fused launch that start after chain blocks exit

// The chain's LDS, or (for an attention block of the fused launch) the wide
// attention's.
struct ChainLds {
  float red[kTailWaves][64][32];
  float ssq_s[32][kDecRows];
  float xs[2][64 * kTailWaves];
  int sh, wfail[kTailWaves];
};
union TailLds {
  ChainLds c;
  WideLds w;
};

// GA > 0 (data-polling form only): the launch also holds the next layer's
// attention for G = GA query heads per kv head (TailArgs::b_att).
template <bool POLL, int GA>
__global__ __launch_bounds__(64 * kTailWaves) void tail_kernel(TailArgs a) {
  __shared__ TailLds lds;
  auto& red = lds.c.red;
  auto& ssq_s = lds.c.ssq_s;
  auto& xs = lds.c.xs;
  auto& sh = lds.c.sh;
  auto& wfail = lds.c.wfail;
  if (__hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;  // an earlier wait failed
  const int D = a.D, H = a.H, N1 = a.N1, ncg = D / 32, npair = H / 32;
  const int nwd = D / 64, nwh = H / 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: window offsets in SGPRs
  const unsigned E = (unsigned)(*a.gstep) * (unsigned)a.L + (unsigned)a.layer + 1u;
  unsigned* done_wo = a.sync;
  unsigned* done_13 = a.sync + 1;
  unsigned* done_w2 = a.sync + 2;
  TailSet S{};
  if constexpr (POLL) {
    S = tail_set(a.sets[E & 1], D, H, N1);
    // the other set back to stale for the next use: its readers belong to
    // the previous launch, which has finished
    const __amdgpu_buffer_rsrc_t ro = rsrc(a.sets[(E & 1) ^ 1]);
    const u32x4v st = {kTailStale, kTailStale, kTailStale, kTailStale};
    const uint32_t n16 = (uint32_t)(tail_set_bytes(D, H, N1) / 16);
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < n16; k += gridDim.x * blockDim.x)
      __builtin_amdgcn_raw_buffer_store_b128(st, ro, k * 16u, 0, kSc1);
  }
  int b = blockIdx.x;

  if (b < a.b_wo) {  // ---- Wo: x += Wo att --------------------------------------
    const int cg = b;
    // x was last written before this launch (by the previous layer's W2 or the
    // embedding): a plain load, issued with the weights
    float2 xv = *reinterpret_cast<const float2*>(a.x + x_index(cg, D));
    const Span sp = wave_span<1>(nwd, kTailWaves, wave);
    WaveGemm<1> g;
    g.load_w(a.wo, cg, nwd, sp);
    g.mma(a.att, sp, false);  // the attention kernel finished before this launch
    g.to_lds(red);
    __syncthreads();
    if constexpr (POLL) {  // x after Wo goes to x_mid, for this group's W2 block
      resid_epilogue(sum_waves(red, 0, kTailWaves), xv, cg, S.x_mid, D, S.ssq_wo, S.xg_ffn, a.g_ffn);
    } else {
      resid_epilogue(sum_waves(red, 0, kTailWaves), xv, cg, a.x, D, a.ssq_wo, a.xg_ffn, a.g_ffn);
      publish(done_wo);
    }
    return;
  }
  b -= a.b_wo;
  if (b < a.b_13) {  // ---- W1|W3 pair: SwiGLU ------------------------------------
    // pair p: W1 rows of hidden units 32 p.. (group 2 p) on waves 0-7, W3 (2 p + 1) on 8-15
    const int pr = b, half = wave >> 3;
    const Span sp = wave_span<2>(nwd, kTailWaves / 2, wave & 7);
    WaveGemm<2> g;
    g.load_w(a.w13, 2 * pr + half, nwd, sp);
    // the residual's column-group sums of squares (ncg * 64 <= 2 per thread),
    // in flight with the activations
    const int t0 = threadIdx.x, t1 = threadIdx.x + 64 * kTailWaves, nss = ncg * kDecRows;
    if constexpr (POLL) {
      // the sums of squares go straight to ssq_s (flat [2][1024]: thread t's
      // pair at t and t + 1024), then are checked from there
      float (*ssq_f)[64 * kTailWaves] = reinterpret_cast<float (*)[64 * kTailWaves]>(&ssq_s[0][0]);
      const unsigned l0 = lds_rows(ssq_f, 0), l1 = lds_rows(ssq_f, 1);
      bool ok = false;
      for (unsigned r = 0; a.spin_limit != 0; r++) {
        asm volatile("" ::: "memory");
        two_to_lds(S.ssq_wo, (uint32_t)min(t0, nss - 1), (uint32_t)min(t1, nss - 1), l0, l1);
        bool f = g.load_x(S.xg_ffn, sp);
        drain_stores();  // the LDS loads above
        f &= fresh(ssq_f[0][threadIdx.x]);
        f &= fresh(ssq_f[1][threadIdx.x]);
        if (__all(f)) { ok = true; break; }
        if (give_up(r, a.spin_limit, a.err)) break;
      }
      wave_outcome(ok, a.err, wfail);
      g.compute(sp);
      g.to_lds(red);
      __syncthreads();
      if (any_failed(wfail)) return;
    } else {
      if (!wait_count(done_wo, (unsigned)ncg * E, a.spin_limit, a.err, &sh)) return;  // x, its sums of squares, xg_ffn
      const float s0 = t0 < nss ? ld_c1(a.ssq_wo, (uint32_t)t0) : 0.f;
      const float s1 = t1 < nss ? ld_c1(a.ssq_wo, (uint32_t)t1) : 0.f;
      g.mma(a.xg_ffn, sp, true);
      g.to_lds(red);
      if (t0 < nss) ssq_s[t0 / kDecRows][t0 % kDecRows] = s0;
      if (t1 < nss) ssq_s[t1 / kDecRows][t1 % kDecRows] = s1;
      __syncthreads();
    }
    const float2 h1 = sum_waves(red, 0, kTailWaves / 2), h3 = sum_waves(red, kTailWaves / 2, kTailWaves);
    const int row = threadIdx.x >> 4, c = (threadIdx.x & 15) * 2;
    float ss = 0.f;
    for (int q = 0; q < ncg; q++) ss += ssq_s[q][row];
    const float rr = 1.0f / sqrtf(ss / (float)D + 1e-5f);
    const float u0 = h1.x * rr, u1 = h1.y * rr;
    st_frag2(POLL ? S.gate : a.gate, row, 32 * pr + c, u0 / (1.0f + __expf(-u0)) * (h3.x * rr),
             u1 / (1.0f + __expf(-u1)) * (h3.y * rr));
    if constexpr (!POLL) publish(done_13);
    return;
  }
  b -= a.b_13;
  if (b < a.b_w2) {  // ---- W2: x += W2 gate -----------------------------------
    const int cg = b;
    const Span sp = wave_span<2>(nwh, kTailWaves, wave);
    WaveGemm<2> g;
    g.load_w(a.w2, cg, nwh, sp);
    if constexpr (POLL) {
      // x after Wo (x_mid, from this group's Wo block) in the same rounds as
      // the activations, straight into LDS
      const uint32_t xm = (uint32_t)x_index(cg, D);
      const unsigned l0 = lds_rows(xs, 0), l1 = lds_rows(xs, 1);
      bool ok = false;
      for (unsigned r = 0; a.spin_limit != 0; r++) {
        asm volatile("" ::: "memory");
        two_to_lds(S.x_mid, xm, xm + 1, l0, l1);
        bool f = g.load_x(S.gate, sp);
        drain_stores();  // the LDS loads above
        f &= fresh(xs[0][threadIdx.x]);
        f &= fresh(xs[1][threadIdx.x]);
        if (__all(f)) { ok = true; break; }
        if (give_up(r, a.spin_limit, a.err)) break;
      }
      wave_outcome(ok, a.err, wfail);
      g.compute(sp);
      g.to_lds(red);
      __syncthreads();
      if (any_failed(wfail)) return;
    } else {
      // done_13 implies done_wo: x (written by the Wo block of this group) is
      // read device-coherent, in flight with the activations
      if (!wait_count(done_13, (unsigned)npair * E, a.spin_limit, a.err, &sh)) return;
      x_to_lds(a.x, cg, D, xs);
      g.mma(a.gate, sp, true);
      g.to_lds(red);
      drain_stores();  // (also the loads: x_to_lds is not in the compiler's count)
      __syncthreads();
    }
    const float2 xv = make_float2(xs[0][threadIdx.x], xs[1][threadIdx.x]);
    if constexpr (POLL) {  // the last layer's output is for the classifier (after this launch)
      resid_epilogue(sum_waves(red, 0, kTailWaves), xv, cg, a.x, D, S.ssq_w2, a.b_q ? S.xg_next : a.xg_next,
                     a.g_next);
    } else {
      resid_epilogue(sum_waves(red, 0, kTailWaves), xv, cg, a.x, D, a.ssq_w2, a.xg_next, a.g_next);
      publish(done_w2);
    }
    return;
  }
  b -= a.b_w2;
  if (b < a.b_q) {  // ---- next layer's QKV (finished by the attention) ----------------
    const int cg = b;
    const Span sp = wave_span<1>(nwd, kTailWaves, wave);
    WaveGemm<1> g;
    g.load_w(a.wqkv_next, cg, nwd, sp);
    if constexpr (POLL) {
      bool ok = false;
      for (unsigned r = 0; a.spin_limit != 0; r++) {
        asm volatile("" ::: "memory");
        if (__all(g.load_x(S.xg_next, sp))) { ok = true; break; }
        if (give_up(r, a.spin_limit, a.err)) break;
      }
      wave_outcome(ok, a.err, wfail);
      g.compute(sp);
      g.to_lds(red);
      __syncthreads();
      if (any_failed(wfail)) return;
    } else {
      if (!wait_count(done_w2, (unsigned)ncg * E, a.spin_limit, a.err, &sh)) return;
      g.mma(a.xg_next, sp, true);
      g.to_lds(red);
      __syncthreads();
    }
    const float2 v = sum_waves(red, 0, kTailWaves);
    const int row = threadIdx.x >> 4, c = cg * 32 + (threadIdx.x & 15) * 2;
    if (POLL && a.b_att) {  // for the attention blocks of this launch
      st_c1(S.p_q, (uint32_t)(row * N1 + c), v.x);
      st_c1(S.p_q, (uint32_t)(row * N1 + c + 1), v.y);
    } else {
      *reinterpret_cast<float2*>(a.p_q + (size_t)row * N1 + c) = v;
    }
    return;
  }
  b -= a.b_q;
  if constexpr (POLL && GA > 0) {  // ---- the next layer's attention -------------------
    if (b > 0) {
      const int i = b - 1;
      DecAttnArgs aa = a.att_next;
      aa.qkv_part = S.p_q;
      aa.qkv_ks = 1;
      aa.rr = S.rr;
      // The last kTailLateAtt blocks start only as chain blocks exit; the
      // first kTailLateAtt (resident from the start, idle until q) stream
      // their K / V through L2 beforehand: block i for block i + b_att -
      // kTailLateAtt, on the same XCD (block indices 8 apart share one).
      const half_t *pk = nullptr, *pv = nullptr;
      int rows = 0;
      if (a.b_att >= 4 * kTailLateAtt && (a.b_att - kTailLateAtt) % 8 == 0 && i < kTailLateAtt) {
        const int t = i + a.b_att - kTailLateAtt, tb = t % aa.nb, tk = t / aa.nb;
        const size_t c0 = ((size_t)tb * aa.NKV + tk) * aa.max_ctx;
        pk = aa.kc + c0 * 64;
        pv = aa.vc + c0 * 64;
        rows = min(aa.ctr[0] + 1, aa.max_ctx);
      }
      dec_attn_wide_body<GA, true, true>(aa, i % aa.nb, i / aa.nb, 0, lds.w, a.spin_limit, a.err, pk, pv, rows);
      return;
    }
  }
  // ---- 1 / rms of the new residual, for the next consumer ------------------------
  if constexpr (POLL) {
    if (threadIdx.x >= kDecRows) return;  // one wave: a row per lane
    const int row = threadIdx.x;
    float v[32];
    bool ok = false;
    for (unsigned r = 0; a.spin_limit != 0; r++) {
      asm volatile("" ::: "memory");
      bool f = true;
#pragma unroll
      for (int q = 0; q < 32; q++) {
        v[q] = ld_c1(S.ssq_w2, (uint32_t)(min(q, ncg - 1) * 64 + row));
        f &= fresh(v[q]);
      }
      if (__all(f)) { ok = true; break; }
      if (give_up(r, a.spin_limit, a.err)) break;
    }
    if (!ok) {
      if (row == 0) __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < 32; q++) ss += q < ncg ? v[q] : 0.f;
    const float r = 1.0f / sqrtf(ss / (float)D + 1e-5f);
    if (a.b_att) st_c1(S.rr, (uint32_t)row, r);
    else a.rr_next[row] = r;
  } else {
    if (!wait_count(done_w2, (unsigned)ncg * E, a.spin_limit, a.err, &sh)) return;
    if (threadIdx.x < kDecRows) a.rr_next[threadIdx.x] = rr_of(a.ssq_w2, ncg, threadIdx.x, D);
  }
}

// x [64][D] -> xg = fp16(x * g) fragments and rr = 1 / rms(x); with tok, x is
// first the embedding row (zero for tok >= V).  One block of 256 per row.
__global__ __launch_bounds__(256) void row_xg_kernel(float* x, half_t* xg, float* rr, const float* embed,
                                                     const uint16_t* tok, const float* g, int D, int V) {
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int tk = tok ? tok[b] : 0;
  float v[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    v[i] = 0.f;
    if (c < D) {
      if (tok) v[i] = tk < V ? embed[(size_t)tk * D + c] : 0.f;
      else v[i] = x[(size_t)b * D + c];
    }
    ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = red[0] + red[1] + red[2] + red[3];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int c = tid + 256 * i;
    if (c < D) {
      if (tok) x[(size_t)b * D + c] = v[i];
      xg[act_frag_off(b, c)] = (half_t)(v[i] * g[c]);
    }
  }
  if (tid == 0) rr[b] = 1.0f / sqrtf(ss / (float)D + 1e-5f);
}

}  // namespace

hipError_t dec_tail(const TailArgs& a, hipStream_t s) {
  // one window per wave for K = D (<= 16 windows), two for K = H (<= 32)
  if (a.D % 64 || a.D > 1024 || a.H % 64 || a.H > 2048 || a.N1 % 32) return hipErrorInvalidValue;
  if (a.b_wo != a.D / 32 || a.b_13 != a.H / 32 || a.b_w2 != a.D / 32 || (a.b_q && a.b_q != a.N1 / 32))
    return hipErrorInvalidValue;
  if (a.poll && (!a.sets[0] || !a.sets[1])) return hipErrorInvalidValue;
  int ga = 0;
  if (a.b_att) {
    const DecAttnArgs& n = a.att_next;
    if (!a.poll || !a.b_q || !dec_attention_fusable(n) || a.b_att != n.nb * n.NKV || n.nsplit != 1)
      return hipErrorInvalidValue;
    ga = n.NH / n.NKV;
  }
  const int blocks = a.b_wo + a.b_13 + a.b_w2 + a.b_q + 1 + a.b_att;
  const dim3 g(blocks), t(64 * kTailWaves);
  switch (a.poll ? ga + 1 : 0) {
    case 0: hipLaunchKernelGGL((tail_kernel<false, 0>), g, t, 0, s, a); break;
    case 1: hipLaunchKernelGGL((tail_kernel<true, 0>), g, t, 0, s, a); break;
    case 2: hipLaunchKernelGGL((tail_kernel<true, 1>), g, t, 0, s, a); break;
    case 3: hipLaunchKernelGGL((tail_kernel<true, 2>), g, t, 0, s, a); break;
    case 4: hipLaunchKernelGGL((tail_kernel<true, 3>), g, t, 0, s, a); break;
    default: hipLaunchKernelGGL((tail_kernel<true, 4>), g, t, 0, s, a); break;
  }
  return hipGetLastError();
}

// blocks of the chain kernel resident per CU (every form)
int dec_tail_blocks_per_cu() {
  int m = 1 << 30;
  auto occ = [&](const void* k) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, 64 * kTailWaves, 0) != hipSuccess) n = 0;
    m = n < m ? n : m;
  };
  occ((const void*)tail_kernel<false, 0>);
  occ((const void*)tail_kernel<true, 0>);
  occ((const void*)tail_kernel<true, 1>);
  occ((const void*)tail_kernel<true, 2>);
  occ((const void*)tail_kernel<true, 3>);
  occ((const void*)tail_kernel<true, 4>);
  return m;
}

hipError_t dec_row_xg(float* x, half_t* xg, float* rr, const float* embed, const uint16_t* tok, const float* g,
                      int nb, int D, int V, hipStream_t s) {
  if (D > 1024 || nb < 1 || nb > kDecRows) return hipErrorInvalidValue;
  hipLaunchKernelGGL(row_xg_kernel, dim3(nb), dim3(256), 0, s, x, xg, rr, embed, tok, g, D, V);
  return hipGetLastError();
}

}  // namespace ane
