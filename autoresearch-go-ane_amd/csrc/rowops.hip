// Row-wise and elementwise kernels (HBM-bound).  One wave per token row:
// lanes stride the channel dimension, so every load and store is
// coalesced across the wave.
#include <algorithm>

#include "rowops.h"

namespace ane {

namespace {

constexpr int ROWS_PER_BLOCK = 4;  // 4 waves

__global__ __launch_bounds__(256) void embed_kernel(float* x, const float* E, const uint16_t* tok, int T, int D,
                                                    int V) {
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const int tk = tok[t];
  float* xr = x + (size_t)t * D;
  const float* er = E + (size_t)tk * D;
  for (int i = lane; i < D; i += 64) xr[i] = tk < V ? er[i] : 0.f;
}

// Each thread keeps four 16-byte loads in flight per region pass.
__global__ __launch_bounds__(256) void prefetch_list_kernel(PrefetchList l) {
  uint32_t x = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (int r = 0; r < l.n; r++) {
    const uint4* q = reinterpret_cast<const uint4*>(l.p[r]);
    const size_t n = l.bytes[r] / 16;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
      const uint4 a = q[i], b = q[i + stride], c = q[i + 2 * stride], d = q[i + 3 * stride];
      x ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
    }
    for (; i < n; i += stride) {
      const uint4 a = q[i];
      x ^= a.x ^ a.y ^ a.z ^ a.w;
    }
  }
  asm volatile("" ::"v"(x));
}

__global__ __launch_bounds__(256) void embed_norm_kernel(float* xpre, float* x0, half_t* xh, const float* E,
                                                         const uint16_t* tok, int T, int D, int V) {
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const int tk = tok[t];
  const float* er = E + (size_t)tk * D;
  float ss = 0.f;
  for (int i = lane; i < D; i += 64) {
    float v = tk < V ? er[i] : 0.f;
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float sc = 1.0f / sqrtf(ss / (float)D + 1e-5f);
  for (int i = lane; i < D; i += 64) {
    float v = tk < V ? er[i] : 0.f;
    size_t idx = (size_t)t * D + i;
    xpre[idx] = v;
    float y = v * sc;
    x0[idx] = y;
    xh[idx] = (half_t)y;
  }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(half_t* out, const float* x, const float* xsub,
                                                      const float* lamp, const float* gain, int T, int D,
                                                      const void* pf, size_t pf_bytes) {
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  // D is a multiple of 64: each lane owns float4 groups i = 4*lane + 256*k,
  // held in registers between the reduction and the store (D <= 1024).
  // The row, its subtrahend and the gains are requested first, then this
  // block's share of the next GEMM's weights (consumed after the stores).
  const int nv = D / 4;
  const bool row_ok = t < T;
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)(row_ok ? t : 0) * D);
  const float4* sr = xsub ? reinterpret_cast<const float4*>(xsub + (size_t)(row_ok ? t : 0) * D) : nullptr;
  const float4* g4 = reinterpret_cast<const float4*>(gain);
  float4 v[4], sb[4], gg[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int i = lane + 64 * k;
    if (i < nv) {
      v[k] = xr[i];
      if (sr) sb[k] = sr[i];
      gg[k] = gain ? g4[i] : make_float4(1.f, 1.f, 1.f, 1.f);
    }
  }
  const Prefetch pfd = prefetch_begin(pf, pf_bytes, blockIdx.x, gridDim.x);
  const float lam = xsub ? *lamp : 0.f;
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int i = lane + 64 * k;
    if (i < nv) {
      float4 a = v[k];
      if (sr) {
        a.x -= lam * sb[k].x; a.y -= lam * sb[k].y; a.z -= lam * sb[k].z; a.w -= lam * sb[k].w;
      }
      v[k] = a;
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
  }
  ss = wave_sum_dpp(ss);
  const float sc = 1.0f / sqrtf(ss / (float)D + 1e-5f);
  if (row_ok) {
    half4* orow = reinterpret_cast<half4*>(out + (size_t)t * D);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = lane + 64 * k;
      if (i < nv) {
        const float4 a = v[k], g = gg[k];
        half4 h;
        h[0] = (half_t)(a.x * sc * g.x);
        h[1] = (half_t)(a.y * sc * g.y);
        h[2] = (half_t)(a.z * sc * g.z);
        h[3] = (half_t)(a.w * sc * g.w);
        orow[i] = h;
      }
    }
  }
  prefetch_end(pfd, pf, pf_bytes, blockIdx.x, gridDim.x);
}

__global__ void gather_kernel(uint16_t* tok, uint16_t* tgt, const uint16_t* data, const uint64_t* pos, int nseq,
                              int S) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nseq * S) return;
  const int b = i / S, t = i % S;
  const uint64_t p = pos[b] + (uint64_t)t;
  tok[i] = data[p];
  tgt[i] = data[p + 1];
}

// The same with the window starts passed by value (no host-to-device copy
// before the launch).
__global__ void gather_arg_kernel(uint16_t* tok, uint16_t* tgt, const uint16_t* data, WindowStarts pos, int nseq,
                                  int S) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nseq * S) return;
  const int b = i / S, t = i % S;
  const uint64_t p = pos.p[b] + (uint64_t)t;
  tok[i] = data[p];
  tgt[i] = data[p + 1];
}

__global__ void f32_to_f16_kernel(half_t* dst, const float* src, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = (half_t)src[i];
}

__global__ void interleave_w13_kernel(half_t* dst, const float* w1, const float* w3, int H, int D) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t n = (size_t)2 * H * D, stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const int f = (int)(i / D), c = (int)(i % D);
    const int blk = f >> 5;
    const int row = (blk >> 1) * 32 + (f & 31);
    const float* src = (blk & 1) ? w3 : w1;
    dst[i] = (half_t)src[(size_t)row * D + c];
  }
}

inline int rows_grid(int T) { return (T + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK; }
inline int flat_grid(size_t n) {
  size_t g = (n + 255) / 256;
  return (int)(g > 65536 ? 65536 : (g == 0 ? 1 : g));
}

}  // namespace

// Kernels a host loads from the code object itself (ane_kernels.h): C
// names, launched below by the library as well.
extern "C" __global__ __launch_bounds__(256) void ane_k_prefetch(const void* pf, size_t pf_bytes) {
  prefetch_slice(pf, pf_bytes, blockIdx.x, gridDim.x);
}

// x = E[tok] (0 for tok >= V), xg = fp16(x * gain), ssq[t] = sum of x^2 (the
// deferred norm's one partial per row); the next GEMM's weights streamed
// through the caches alongside.
// D <= 1024 (the engine's widths): each lane's float4 groups i = lane + 64 k
// of the row and of the gains are requested before anything is stored (the
// stores could alias later loads, so a load / store loop waits one memory
// round trip per element group); then this block's share of the next
// GEMM's weights, consumed after the stores.  Wider rows take the loop.
extern "C" __global__ __launch_bounds__(256) void ane_k_embed_xg(float* x, half_t* xg, float* ssq, const float* E,
                                                            const uint16_t* tok, const float* gain, int T, int D, int V,
                                                       const void* pf, size_t pf_bytes) {
  const int t = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (D > 1024) {
    prefetch_slice(pf, pf_bytes, blockIdx.x, gridDim.x);
    if (t >= T) return;
    const int tk = tok[t];
    const float* er = E + (size_t)tk * D;
    float ss = 0.f;
    for (int i = lane; i < D; i += 64) {
      const float v = tk < V ? er[i] : 0.f;
      const size_t idx = (size_t)t * D + i;
      x[idx] = v;
      xg[idx] = (half_t)(v * gain[i]);
      ss += v * v;
    }
    ss = wave_sum(ss);
    if (lane == 0) ssq[t] = ss;
    return;
  }
  const int nv = D / 4;
  const bool row_ok = t < T;
  const int tk = row_ok ? tok[t] : V;
  const bool hit = tk < V;
  const float4* er = reinterpret_cast<const float4*>(E + (size_t)(hit ? tk : 0) * D);
  const float4* g4 = reinterpret_cast<const float4*>(gain);
  float4 v[4], gg[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int i = lane + 64 * k;
    if (i < nv) {
      v[k] = hit ? er[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      gg[k] = g4[i];
    }
  }
  const Prefetch pfd = prefetch_begin(pf, pf_bytes, blockIdx.x, gridDim.x);
  float ss = 0.f;
  if (row_ok) {
    float4* xr = reinterpret_cast<float4*>(x + (size_t)t * D);
    half4* hr = reinterpret_cast<half4*>(xg + (size_t)t * D);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = lane + 64 * k;
      if (i < nv) {
        const float4 a = v[k], g = gg[k];
        xr[i] = a;
        half4 h;
        h[0] = (half_t)(a.x * g.x);
        h[1] = (half_t)(a.y * g.y);
        h[2] = (half_t)(a.z * g.z);
        h[3] = (half_t)(a.w * g.w);
        hr[i] = h;
        ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      }
    }
  }
  ss = wave_sum_dpp(ss);
  if (row_ok && lane == 0) ssq[t] = ss;
  prefetch_end(pfd, pf, pf_bytes, blockIdx.x, gridDim.x);
}

// Per token: merge the partials with a running (max, sum) pair; kCeLanes
// lanes split the partials of one token (lane q takes q, q + kCeLanes, ...)
// and combine with xor-shuffles.
constexpr int kCeLanes = 8;
extern "C" __global__ __launch_bounds__(256) void ane_k_ce_token(float* lse_out, float* tok_loss, const float2* partial,
                                                       int np, const float* tgt_logit, const uint16_t* tgt, int V,
                                                       int T) {
  const int n = blockIdx.x * (256 / kCeLanes) + threadIdx.x / kCeLanes, q = threadIdx.x % kCeLanes;
  float mx = -INFINITY, sum = 0.f;
  auto merge = [&](float2 v) {
    const float m2 = fmaxf(mx, v.x);
    sum = sum * __expf(mx - m2) + v.y * __expf(v.x - m2);
    mx = m2;
  };
  if (n < T) {
    // four of the thread's partials requested at a time, merged in order
    int p = q;
    for (; p + 3 * kCeLanes < np; p += 4 * kCeLanes) {
      float2 v[4];
#pragma unroll
      for (int u = 0; u < 4; u++) v[u] = partial[(size_t)(p + kCeLanes * u) * T + n];
#pragma unroll
      for (int u = 0; u < 4; u++) merge(v[u]);
    }
    for (; p < np; p += kCeLanes) merge(partial[(size_t)p * T + n]);
  }
#pragma unroll
  for (int o = 1; o < kCeLanes; o <<= 1) {
    const float om = __shfl_xor(mx, o, 64), os = __shfl_xor(sum, o, 64);
    const float m2 = fmaxf(mx, om);
    sum = (mx == -INFINITY ? 0.f : sum * __expf(mx - m2)) + (om == -INFINITY ? 0.f : os * __expf(om - m2));
    mx = m2;
  }
  if (n < T && q == 0) {
    const float lse = mx + __logf(sum);
    lse_out[n] = lse;
    float l = 0.f;
    if (tgt[n] < V) {
      const float logp = tgt_logit[n] - lse;
      const float floor_ = -23.025850929940457f;  // log(1e-10): p clamped at 1e-10
      l = -(logp > floor_ ? logp : floor_);
    }
    tok_loss[n] = l;
  }
}

extern "C" __global__ __launch_bounds__(256) void ane_k_ce_reduce(float* loss_seq, float* colscale, float dscale,
                                                        const float* tok_loss, const uint16_t* tgt, int V, int S) {
  const int b = blockIdx.x;
  __shared__ float red_l[256];
  __shared__ int red_v[256];
  float lsum = 0.f;
  int nvalid = 0;
  for (int t = threadIdx.x; t < S; t += blockDim.x) {
    const int n = b * S + t;
    if (tgt[n] < V) {
      lsum += tok_loss[n];
      nvalid++;
    }
  }
  red_l[threadIdx.x] = lsum;
  red_v[threadIdx.x] = nvalid;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      red_l[threadIdx.x] += red_l[threadIdx.x + o];
      red_v[threadIdx.x] += red_v[threadIdx.x + o];
    }
    __syncthreads();
  }
  const int valid = red_v[0];
  if (threadIdx.x == 0) loss_seq[b] = valid > 0 ? red_l[0] / (float)valid : 0.f;
  if (colscale) {
    const float cs = valid > 0 ? dscale / (float)valid : 0.f;
    for (int t = threadIdx.x; t < S; t += blockDim.x) {
      const int n = b * S + t;
      colscale[n] = tgt[n] < V ? cs : 0.f;
    }
  }
}


hipError_t embed_lookup(float* x, const float* E, const uint16_t* tok, int T, int D, int V, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(rows_grid(T)), dim3(256), 0, s, x, E, tok, T, D, V);
  return hipGetLastError();
}

hipError_t prefetch_weights(const void* p, size_t bytes, hipStream_t s) {
  if (!p || bytes < 16) return hipSuccess;
  const size_t n16 = bytes / 16;
  const unsigned blocks = (unsigned)std::min<size_t>(1024, (n16 + 255) / 256);
  hipLaunchKernelGGL(ane_k_prefetch, dim3(blocks), dim3(256), 0, s, p, bytes);
  return hipGetLastError();
}

hipError_t prefetch_list(const PrefetchList& l, hipStream_t s) {
  size_t tot = 0;
  for (int r = 0; r < l.n; r++) tot += l.bytes[r];
  if (tot < 16) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<size_t>(512, (tot / 16 / 4 + 255) / 256);
  hipLaunchKernelGGL(prefetch_list_kernel, dim3(blocks), dim3(256), 0, s, l);
  return hipGetLastError();
}

hipError_t embed_xg(float* x, half_t* xg, float* ssq, const float* E, const uint16_t* tok, const float* gain, int T,
                    int D, int V, hipStream_t s, const void* pf, size_t pf_bytes) {
  hipLaunchKernelGGL(ane_k_embed_xg, dim3(rows_grid(T)), dim3(256), 0, s, x, xg, ssq, E, tok, gain, T, D, V, pf,
                     pf_bytes);
  return hipGetLastError();
}

hipError_t embed_norm(float* xpre, float* x0, half_t* xh, const float* E, const uint16_t* tok, int T, int D,
                      int V, hipStream_t s) {
  hipLaunchKernelGGL(embed_norm_kernel, dim3(rows_grid(T)), dim3(256), 0, s, xpre, x0, xh, E, tok, T, D, V);
  return hipGetLastError();
}

hipError_t rmsnorm_f16(half_t* out, const float* x, const float* xsub, const float* lam, const float* gain, int T,
                       int D, hipStream_t s, const void* pf, size_t pf_bytes) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows_grid(T)), dim3(256), 0, s, out, x, xsub, lam, gain, T, D, pf,
                     pf_bytes);
  return hipGetLastError();
}

hipError_t gather_windows(uint16_t* tok, uint16_t* tgt, const uint16_t* data, const uint64_t* pos, int nseq, int S,
                          hipStream_t s) {
  const int n = nseq * S;
  hipLaunchKernelGGL(gather_kernel, dim3((n + 255) / 256), dim3(256), 0, s, tok, tgt, data, pos, nseq, S);
  return hipGetLastError();
}

hipError_t gather_windows_args(uint16_t* tok, uint16_t* tgt, const uint16_t* data, const uint64_t* pos_host, int nseq,
                               int S, hipStream_t s) {
  if (nseq <= 0 || nseq > kArgWindows) return hipErrorInvalidValue;
  WindowStarts w;
  for (int b = 0; b < nseq; b++) w.p[b] = pos_host[b];
  const int n = nseq * S;
  hipLaunchKernelGGL(gather_arg_kernel, dim3((n + 255) / 256), dim3(256), 0, s, tok, tgt, data, w, nseq, S);
  return hipGetLastError();
}

hipError_t ce_reduce(float* loss_seq, float* lse, float* tok_loss, float* colscale, float dscale,
                     const float2* partial, int np, const float* tgt_logit, const uint16_t* tgt, int V, int nseq, int S,
                     hipStream_t s) {
  const int T = nseq * S;
  hipLaunchKernelGGL(ane_k_ce_token, dim3((T + 256 / kCeLanes - 1) / (256 / kCeLanes)), dim3(256), 0, s, lse, tok_loss,
                     partial, np, tgt_logit, tgt, V, T);
  hipLaunchKernelGGL(ane_k_ce_reduce, dim3(nseq), dim3(256), 0, s, loss_seq, colscale, dscale, tok_loss, tgt, V, S);
  return hipGetLastError();
}

hipError_t f32_to_f16(half_t* dst, const float* src, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3(flat_grid(n)), dim3(256), 0, s, dst, src, n);
  return hipGetLastError();
}

hipError_t interleave_w13(half_t* dst, const float* w1, const float* w3, int H, int D, hipStream_t s) {
  hipLaunchKernelGGL(interleave_w13_kernel, dim3(flat_grid((size_t)2 * H * D)), dim3(256), 0, s, dst, w1, w3, H,
                     D);
  return hipGetLastError();
}

}  // namespace ane
