// Backward-pass row kernels and the on-device optimizer (HBM-bound).
// Rows are token-major [T, D]; one wave per row, float4 per lane.
#include "train_ops.h"

#include <cstdlib>

namespace ane {

namespace {

constexpr int kMaxVec = 4;  // D <= 1024: float4 groups per lane

__global__ __launch_bounds__(256) void norm_bwd_kernel(NormBwdArgs a) {
  __shared__ float gsh[4][1024];
  __shared__ double lsh[4][2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int D = a.D, nv = D / 4;
  const float alpha = a.alpha_p ? *a.alpha_p : a.alpha;
  const float xl = a.xl_p ? *a.xl_p : 0.f;
  float4 dg[kMaxVec];
#pragma unroll
  for (int k = 0; k < kMaxVec; k++) dg[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  double la = 0.0, lb = 0.0;
  for (int rr = 0; rr < kNormBwdRows / 4; rr++) {
    const int t = blockIdx.x * kNormBwdRows + wave * (kNormBwdRows / 4) + rr;
    if (t >= a.T) break;
    const size_t ro = (size_t)t * D;
    float4 dy[kMaxVec], xv[kMaxVec], gv[kMaxVec];
    float ss = 0.f, dot = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxVec; k++) {
      const int i = lane + 64 * k;
      if (i < nv) {
        dy[k] = reinterpret_cast<const float4*>(a.dy + ro)[i];
        xv[k] = reinterpret_cast<const float4*>(a.x + ro)[i];
        gv[k] = a.gain ? reinterpret_cast<const float4*>(a.gain)[i] : make_float4(1.f, 1.f, 1.f, 1.f);
        ss += xv[k].x * xv[k].x + xv[k].y * xv[k].y + xv[k].z * xv[k].z + xv[k].w * xv[k].w;
        dot += dy[k].x * xv[k].x * gv[k].x + dy[k].y * xv[k].y * gv[k].y + dy[k].z * xv[k].z * gv[k].z +
               dy[k].w * xv[k].w * gv[k].w;
      }
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    const float rrms = 1.0f / sqrtf(ss / (float)D + 1e-5f);
    const float c = dot * rrms * rrms / (float)D;  // both forms: dx = (dy - x*c) * rrms * gain
    float pa = 0.f, pb = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxVec; k++) {
      const int i = lane + 64 * k;
      if (i >= nv) continue;
      float o[4] = {(dy[k].x - xv[k].x * c) * rrms * gv[k].x, (dy[k].y - xv[k].y * c) * rrms * gv[k].y,
                    (dy[k].z - xv[k].z * c) * rrms * gv[k].z, (dy[k].w - xv[k].w * c) * rrms * gv[k].w};
      if (a.dgain_part) {
        dg[k].x += dy[k].x * xv[k].x * rrms;
        dg[k].y += dy[k].y * xv[k].y * rrms;
        dg[k].z += dy[k].z * xv[k].z * rrms;
        dg[k].w += dy[k].w * xv[k].w * rrms;
      }
      if (a.addend) {
        const float4 ad = reinterpret_cast<const float4*>(a.addend + ro)[i];
        const float av[4] = {ad.x, ad.y, ad.z, ad.w};
#pragma unroll
        for (int u = 0; u < 4; u++) o[u] += alpha * av[u];
        if (a.lam_x) {
          const float4 lx = reinterpret_cast<const float4*>(a.lam_x + ro)[i];
          pa += av[0] * lx.x + av[1] * lx.y + av[2] * lx.z + av[3] * lx.w;
        }
        if (a.lam_x0) {
          const float4 lx = reinterpret_cast<const float4*>(a.lam_x0 + ro)[i];
          pb += av[0] * lx.x + av[1] * lx.y + av[2] * lx.z + av[3] * lx.w;
        }
        if (a.gx0) {
          float4* gp = reinterpret_cast<float4*>(a.gx0 + ro) + i;
          float4 gg = *gp;
          gg.x += xl * av[0]; gg.y += xl * av[1]; gg.z += xl * av[2]; gg.w += xl * av[3];
          *gp = gg;
        }
      }
      if (a.addend2) {
        const float4 ad = reinterpret_cast<const float4*>(a.addend2 + ro)[i];
        o[0] += ad.x; o[1] += ad.y; o[2] += ad.z; o[3] += ad.w;
      }
      if (a.ve_dx && i < 3) {  // channels 0..11 = float4 groups 0..2
#pragma unroll
        for (int u = 0; u < 4; u++) o[u] += a.ve_dx[(size_t)t * 12 + 4 * i + u];
      }
      reinterpret_cast<float4*>(a.out + ro)[i] = make_float4(o[0], o[1], o[2], o[3]);
      if (a.out_h) {
        half4 hv;
#pragma unroll
        for (int u = 0; u < 4; u++) hv[u] = (half_t)o[u];
        reinterpret_cast<half4*>(a.out_h + ro)[i] = hv;
      }
    }
    la += (double)pa;
    lb += (double)pb;
  }
  if (a.dgain_part) {
#pragma unroll
    for (int k = 0; k < kMaxVec; k++) {
      const int i = lane + 64 * k;
      if (i < nv) {
        gsh[wave][4 * i] = dg[k].x; gsh[wave][4 * i + 1] = dg[k].y;
        gsh[wave][4 * i + 2] = dg[k].z; gsh[wave][4 * i + 3] = dg[k].w;
      }
    }
  }
  if (a.lam_part) {
    la = wave_sum_d(la);
    lb = wave_sum_d(lb);
    if (lane == 0) { lsh[wave][0] = la; lsh[wave][1] = lb; }
  }
  __syncthreads();
  if (a.dgain_part)
    for (int i = threadIdx.x; i < D; i += 256)
      a.dgain_part[(size_t)blockIdx.x * D + i] = gsh[0][i] + gsh[1][i] + gsh[2][i] + gsh[3][i];
  if (a.lam_part && threadIdx.x < 2)
    a.lam_part[blockIdx.x * 2 + threadIdx.x] =
        lsh[0][threadIdx.x] + lsh[1][threadIdx.x] + lsh[2][threadIdx.x] + lsh[3][threadIdx.x];
}

// The gain form without the lambda, value-embedding and second-addend terms
// (llama2: the final norm, and each layer's two norms with addend = the
// residual gradient): one wave per row, kNormBwdRows waves per block, and
// every load of the row -- dy, x, the gain and the addend -- issued before
// its two reductions, so a row costs one memory round trip (the general
// kernel above loads the addend after them, two rows per wave in turn).
// The block's dgain partial sums its rows in row order.
template <bool ADD>
__global__ __launch_bounds__(64 * kNormBwdRows) void norm_bwd_gain_kernel(NormBwdArgs a) {
  __shared__ float gsh[kNormBwdRows][1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int D = a.D, nv = D / 4;
  const int t = blockIdx.x * kNormBwdRows + wave;
  const size_t ro = (size_t)min(t, a.T - 1) * D;  // a row past T (last block) reads row T - 1, stores nothing
  float4 dy[kMaxVec], xv[kMaxVec], gv[kMaxVec], ad[kMaxVec];
#pragma unroll
  for (int k = 0; k < kMaxVec; k++) {
    if (64 * k < nv) {  // uniform; lanes past nv read a valid group, their values unused
      const int i = min(lane + 64 * k, nv - 1);
      dy[k] = reinterpret_cast<const float4*>(a.dy + ro)[i];
      xv[k] = reinterpret_cast<const float4*>(a.x + ro)[i];
      gv[k] = reinterpret_cast<const float4*>(a.gain)[i];
      if constexpr (ADD) ad[k] = reinterpret_cast<const float4*>(a.addend + ro)[i];
    }
  }
  const float alpha = ADD ? (a.alpha_p ? *a.alpha_p : a.alpha) : 0.f;
  float ss = 0.f, dot = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxVec; k++) {
    if (64 * k < nv && lane + 64 * k < nv) {
      ss += xv[k].x * xv[k].x + xv[k].y * xv[k].y + xv[k].z * xv[k].z + xv[k].w * xv[k].w;
      dot += dy[k].x * xv[k].x * gv[k].x + dy[k].y * xv[k].y * gv[k].y + dy[k].z * xv[k].z * gv[k].z +
             dy[k].w * xv[k].w * gv[k].w;
    }
  }
  ss = wave_sum_dpp(ss);
  dot = wave_sum_dpp(dot);
  const float rrms = 1.0f / sqrtf(ss / (float)D + 1e-5f);
  const float c = dot * rrms * rrms / (float)D;
  const bool row_ok = t < a.T;
#pragma unroll
  for (int k = 0; k < kMaxVec; k++) {
    const int i = lane + 64 * k;
    if (64 * k >= nv) continue;
    float o[4] = {(dy[k].x - xv[k].x * c) * rrms * gv[k].x, (dy[k].y - xv[k].y * c) * rrms * gv[k].y,
                  (dy[k].z - xv[k].z * c) * rrms * gv[k].z, (dy[k].w - xv[k].w * c) * rrms * gv[k].w};
    if constexpr (ADD) {
      o[0] += alpha * ad[k].x; o[1] += alpha * ad[k].y; o[2] += alpha * ad[k].z; o[3] += alpha * ad[k].w;
    }
    if (i < nv) {
      const bool live = row_ok;
      gsh[wave][4 * i] = live ? dy[k].x * xv[k].x * rrms : 0.f;
      gsh[wave][4 * i + 1] = live ? dy[k].y * xv[k].y * rrms : 0.f;
      gsh[wave][4 * i + 2] = live ? dy[k].z * xv[k].z * rrms : 0.f;
      gsh[wave][4 * i + 3] = live ? dy[k].w * xv[k].w * rrms : 0.f;
      if (row_ok) {
        reinterpret_cast<float4*>(a.out + ro)[i] = make_float4(o[0], o[1], o[2], o[3]);
        if (a.out_h) {
          half4 hv;
#pragma unroll
          for (int u = 0; u < 4; u++) hv[u] = (half_t)o[u];
          reinterpret_cast<half4*>(a.out_h + ro)[i] = hv;
        }
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < D; i += 64 * kNormBwdRows) {
    float g = gsh[0][i];
#pragma unroll
    for (int w = 1; w < kNormBwdRows; w++) g += gsh[w][i];
    a.dgain_part[(size_t)blockIdx.x * D + i] = g;
  }
}

// One block per 64 columns: 16 waves each sum every 16th partial row of
// the block's columns (independent loads, four in flight per lane), then
// the 16 wave sums are added in a fixed order.
__global__ __launch_bounds__(1024) void reduce_partials_kernel(float* dst, const float* part, int nblocks, int n,
                                                              int overwrite) {
  __shared__ float sh[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = blockIdx.x * 64 + lane;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (i < n) {
    int b = wave;
    for (; b + 48 < nblocks; b += 64) {
      s0 += part[(size_t)b * n + i];
      s1 += part[(size_t)(b + 16) * n + i];
      s2 += part[(size_t)(b + 32) * n + i];
      s3 += part[(size_t)(b + 48) * n + i];
    }
    for (; b < nblocks; b += 16) s0 += part[(size_t)b * n + i];
  }
  sh[wave][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (wave == 0 && i < n) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < 16; w++) s += sh[w][lane];
    dst[i] = overwrite ? s : dst[i] + s;
  }
}

__global__ __launch_bounds__(256) void reduce_dots_kernel(float* d0, float* d1, const double* part, int nblocks,
                                                          float sign) {
  __shared__ double sh[2][256];
  double s0 = 0.0, s1 = 0.0;
  for (int b = threadIdx.x; b < nblocks; b += 256) {
    s0 += part[2 * b];
    s1 += part[2 * b + 1];
  }
  sh[0][threadIdx.x] = s0;
  sh[1][threadIdx.x] = s1;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      sh[0][threadIdx.x] += sh[0][threadIdx.x + o];
      sh[1][threadIdx.x] += sh[1][threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (d0) *d0 += (float)(sign * sh[0][0]);
    if (d1) *d1 += (float)(sign * sh[1][0]);
  }
}

__global__ __launch_bounds__(256) void backout_bwd_kernel(float* ginj, double* part, const float* d, const float* xm,
                                                          const float* lam_p, size_t n) {
  __shared__ double sh[256];
  const float lam = *lam_p;
  double acc = 0.0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    acc += (double)(d[i] * xm[i]);
    ginj[i] = -lam * d[i];
  }
  sh[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) sh[threadIdx.x] += sh[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) { part[2 * blockIdx.x] = sh[0]; part[2 * blockIdx.x + 1] = 0.0; }
}

__global__ void backout_fwd_kernel(float* out, const float* x, const float* xm, const float* lam_p, size_t n) {
  const float lam = *lam_p;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = x[i] - lam * xm[i];
}

__global__ void axpy_kernel(float* y, const float* x, half_t* yh, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float v = y[i] + x[i];
    y[i] = v;
    if (yh) yh[i] = (half_t)v;
  }
}

__global__ __launch_bounds__(256) void smear_bwd_kernel(half_t* dgp, float* dout2, double* part, const float* dy,
                                                        const float* gact, const float* x0, const float* lam_p, int T,
                                                        int D, int seq) {
  __shared__ double sh[256];
  const float lam = *lam_p;
  const size_t n = (size_t)T * D;
  double acc = 0.0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const int t = (int)(i / D);
    const bool first = (t % seq) == 0, last = (t % seq) == seq - 1;
    const float g = gact[i], y = dy[i];
    const float s = first ? 0.f : x0[i - D];
    acc += (double)(y * g * s);
    dgp[i] = (half_t)(y * lam * s * g * (1.f - g));
    float o = y;
    if (!last) o += dy[i + D] * lam * gact[i + D];
    dout2[i] = o;
  }
  sh[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) sh[threadIdx.x] += sh[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) { part[2 * blockIdx.x] = sh[0]; part[2 * blockIdx.x + 1] = 0.0; }
}

__global__ __launch_bounds__(256) void embed_bwd_kernel(float* G, const float* dx, const uint16_t* tok, int T, int D,
                                                        int V) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const int tk = tok[t];
  if (tk >= V) return;
  float* gr = G + (size_t)tk * D;
  const float* xr = dx + (size_t)t * D;
  for (int i = lane; i < D; i += 64) atomicAdd(gr + i, xr[i]);
}

// one wave per token; lane = dim within a head, loop over heads
__global__ __launch_bounds__(256) void ve_bwd_kernel(float* gemb, float* ggate, float* ve_dx, const half_t* dv,
                                                     int ldv, const float* x, const float* emb, const float* vg,
                                                     const uint16_t* tok, int T, int D, int NH, int V) {
  __shared__ float gsh[4][16 * 12];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  for (int i = lane; i < NH * 12; i += 64) gsh[wave][i] = 0.f;
  if (t < T) {
    const int tk = tok[t];
    const float* xr = x + (size_t)t * D;
    float xc[12];
#pragma unroll
    for (int c = 0; c < 12; c++) xc[c] = xr[c];
    float dxc[12];
#pragma unroll
    for (int c = 0; c < 12; c++) dxc[c] = 0.f;
    for (int h = 0; h < NH; h++) {
      float gp = 0.f;
#pragma unroll
      for (int c = 0; c < 12; c++) gp += vg[h * 12 + c] * xc[c];
      const float act = (float)(1.0 / (1.0 + exp(-(double)gp)));
      const float gate = 3.0f * act;
      const float dvd = (float)dv[(size_t)t * ldv + h * 64 + lane];
      const float ev = tk < V ? emb[(size_t)tk * D + h * 64 + lane] : 0.f;
      if (tk < V) atomicAdd(gemb + (size_t)tk * D + h * 64 + lane, dvd * gate);
      const float dg = wave_sum(dvd * ev);
      const float dgp = dg * 3.0f * act * (1.f - act);
      if (lane < 12) gsh[wave][h * 12 + lane] = dgp * xc[lane];
#pragma unroll
      for (int c = 0; c < 12; c++) dxc[c] += dgp * vg[h * 12 + c];
    }
    if (lane < 12) ve_dx[(size_t)t * 12 + lane] = dxc[lane];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NH * 12; i += 256)
    atomicAdd(ggate + i, gsh[0][i] + gsh[1][i] + gsh[2][i] + gsh[3][i]);
}

__global__ void fill_kernel(float* p, size_t n, float v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// float4 loads, two in flight per lane; the n % 4 tail is summed by block 0
__global__ __launch_bounds__(256) void sumsq_kernel(double* part, const float* g, size_t n) {
  __shared__ double sh[256];
  double acc = 0.0, acc2 = 0.0;
  const size_t n4 = n / 4, stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + stride < n4; i += 2 * stride) {
    const float4 a = ld_nt_f4(g + 4 * i), b = ld_nt_f4(g + 4 * (i + stride));
    acc += (double)a.x * a.x + (double)a.y * a.y + (double)a.z * a.z + (double)a.w * a.w;
    acc2 += (double)b.x * b.x + (double)b.y * b.y + (double)b.z * b.z + (double)b.w * b.w;
  }
  if (i < n4) {
    const float4 a = ld_nt_f4(g + 4 * i);
    acc += (double)a.x * a.x + (double)a.y * a.y + (double)a.z * a.z + (double)a.w * a.w;
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
    const double f = g[4 * n4 + threadIdx.x];
    acc += f * f;
  }
  acc += acc2;
  sh[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) sh[threadIdx.x] += sh[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = sh[0];
}

__global__ __launch_bounds__(256) void sumsq_final_kernel(double* out, const double* part, int n) {
  __shared__ double sh[256];
  double acc = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) acc += part[i];
  sh[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) sh[threadIdx.x] += sh[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = sh[0];
}

__global__ __launch_bounds__(256) void adam_kernel(AdamArgs a) {
  const AdamSeg& sg = a.seg[blockIdx.y];
  float cf = 1.f;
  if (sg.clip && a.clip > 0.f) {
    const double n2 = *a.sumsq * (double)a.gscale * (double)a.gscale;
    if (n2 > 0.0) {
      const float norm = (float)sqrt(n2);
      if (norm > a.clip) cf = a.clip / norm;
    }
  }
  const float gs = a.gscale;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < sg.len; i += (int64_t)gridDim.x * 256) {
    const int64_t k = sg.off + i;
    float g = a.g[k] * gs;
    g *= cf;
    const float m = sg.b1 * a.m[k] + (1.f - sg.b1) * g;
    const float v = sg.b2 * a.v[k] + (1.f - sg.b2) * g * g;
    a.m[k] = m;
    a.v[k] = v;
    const float mh = m * sg.i1, vh = v * sg.i2;
    float upd = mh / (sqrtf(vh) + a.eps);
    if (sg.wd != 0.f) upd += sg.wd * a.w[k];
    a.w[k] -= sg.lr * upd;
  }
}

// One block per kUpdateChunk elements of one job (binary search over blk0);
// block blockIdx.x is block blk_base + blockIdx.x of the table.
__global__ __launch_bounds__(256) void adam_fused_kernel(AdamArgs a, const UpdateJob* jobs, int njobs, int blk_base) {
  const int blk = blk_base + (int)blockIdx.x;
  int lo = 0, hi = njobs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (jobs[mid].blk0 <= blk) lo = mid;
    else hi = mid - 1;
  }
  const UpdateJob jb = jobs[lo];
  const AdamSeg& sg = a.seg[jb.seg];
  float cf = 1.f;
  if (sg.clip && a.clip > 0.f) {
    const double n2 = *a.sumsq * (double)a.gscale * (double)a.gscale;
    if (n2 > 0.0) {
      const float norm = (float)sqrt(n2);
      if (norm > a.clip) cf = a.clip / norm;
    }
  }
  const float gs = a.gscale;
  // the per-element update of adam_kernel
  auto upd = [&](float g, float& m, float& v, float& w) {
    g = g * gs;
    g *= cf;
    m = sg.b1 * m + (1.f - sg.b1) * g;
    v = sg.b2 * v + (1.f - sg.b2) * g * g;
    const float mh = m * sg.i1, vh = v * sg.i2;
    float u = mh / (sqrtf(vh) + a.eps);
    if (sg.wd != 0.f) u += sg.wd * w;
    w -= sg.lr * u;
  };
  const int64_t base = (int64_t)(blk - jb.blk0) * kUpdateChunk;
  if (jb.vec) {
#pragma unroll
    for (int u = 0; u < kUpdateChunk / 1024; u++) {
      const int64_t i = base + (int64_t)(u * 256 + (int)threadIdx.x) * 4;
      if (i >= jb.len) break;
      const int64_t k = jb.off + i;
      const float4 g4 = ld_nt_f4(a.g + k);
      float4 m4 = ld_nt_f4(a.m + k), v4 = ld_nt_f4(a.v + k), w4 = ld_nt_f4(a.w + k);
      upd(g4.x, m4.x, v4.x, w4.x);
      upd(g4.y, m4.y, v4.y, w4.y);
      upd(g4.z, m4.z, v4.z, w4.z);
      upd(g4.w, m4.w, v4.w, w4.w);
      st_nt_f4(a.m + k, m4);
      st_nt_f4(a.v + k, v4);
      st_nt_f4(a.w + k, w4);
      if (a.zero_g) st_nt_f4(a.g + k, make_float4(0.f, 0.f, 0.f, 0.f));
      if (jb.sh) {
        const int64_t r = i / jb.C;
        const int c = (int)(i - r * jb.C);
        const int64_t sr = (r >> 5) * jb.blk_stride + jb.blk_off + (r & 31);
        half4 h;
        h[0] = (half_t)w4.x; h[1] = (half_t)w4.y; h[2] = (half_t)w4.z; h[3] = (half_t)w4.w;
        *reinterpret_cast<half4*>(jb.sh + sr * jb.C + c) = h;
      }
    }
  } else {
    const int64_t end = base + kUpdateChunk < jb.len ? base + kUpdateChunk : jb.len;
    for (int64_t i = base + threadIdx.x; i < end; i += 256) {
      const int64_t k = jb.off + i;
      float m = a.m[k], v = a.v[k], w = a.w[k];
      upd(a.g[k], m, v, w);
      a.m[k] = m;
      a.v[k] = v;
      a.w[k] = w;
      if (a.zero_g) a.g[k] = 0.f;
    }
  }
}

inline int flat_grid(size_t n, int cap = 4096) {
  size_t g = (n + 255) / 256;
  return (int)(g > (size_t)cap ? cap : (g == 0 ? 1 : g));
}

// LDS tile rows of the shadow kernel: 72 halves (144 B, 16-byte aligned).
constexpr int kTp = 72;
// Transposes by 8x8 register blocks, one wave per 64x64 tile: lane (rb, cb)
// reads rows 8 rb + [0, 8) at columns 8 cb + [0, 8) of the tile (every load
// instruction covers 8 rows x 128 contiguous bytes), swaps the block in
// registers and writes rows 8 cb + [0, 8) of the output at columns
// 8 rb + [0, 8) (every store: 8 rows x 128 bytes).  No LDS and no barrier;
// a launch carries two independent jobs (the two operands of one GEMM).
struct TransposeJob {
  half_t* out;
  const half_t* in;
  int C, ldi, ldo, ntiles;
};
__global__ __launch_bounds__(256) void transpose2_kernel(TransposeJob ja, TransposeJob jb) {
  int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  const bool second = t >= ja.ntiles;
  const TransposeJob& j = second ? jb : ja;
  if (second) t -= ja.ntiles;
  if (t >= j.ntiles) return;  // whole wave
  const int lane = threadIdx.x & 63, rb = lane >> 3, cb = lane & 7;
  const int tiles_c = j.C >> 6;
  const int r0 = (t / tiles_c) * 64 + rb * 8, c0 = (t % tiles_c) * 64 + cb * 8;
  half8 v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = ld_h8(j.in + (size_t)(r0 + i) * j.ldi + c0);
#pragma unroll
  for (int k = 0; k < 8; k++) {
    half8 w;
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = v[i][k];
    st_h8(j.out + (size_t)(c0 + k) * j.ldo + r0, w);
  }
}

__device__ __forceinline__ int shadow_row(const ShadowJob& jb, int r) {
  return (r >> 5) * jb.blk_stride + jb.blk_off + (r & 31);
}

// One 64x64 tile of one job per block; jobs are sorted by tile0.  FROM_PLAIN:
// only the transposed shadow, from the plain fp16 shadow rows.
template <bool FROM_PLAIN>
__global__ __launch_bounds__(256) void shadow_kernel(const ShadowJob* jobs, int njobs) {
  __shared__ __attribute__((aligned(16))) half_t tile[64 * kTp];
  int j = 0, hi = njobs - 1;  // the last job with tile0 <= blockIdx.x
  while (j < hi) {
    const int mid = (j + hi + 1) >> 1;
    if (jobs[mid].tile0 <= (int)blockIdx.x) j = mid;
    else hi = mid - 1;
  }
  const ShadowJob jb = jobs[j];
  const int t = (int)blockIdx.x - jb.tile0;
  const int tiles_c = jb.C >> 6;
  const int r0 = (t / tiles_c) * 64, c0 = (t % tiles_c) * 64;
  const int tid = threadIdx.x;
  if constexpr (FROM_PLAIN) {
    if (!jb.dst_t) return;  // block-uniform
#pragma unroll
    for (int p = 0; p < 2; p++) {  // 16-byte loads: 8 per 64-half row
      const int idx = tid + 256 * p, row = idx >> 3, ch = idx & 7;
      const half8 h = ld_h8(jb.dst + (size_t)shadow_row(jb, r0 + row) * jb.C + c0 + ch * 8);
      *reinterpret_cast<half8*>(tile + row * kTp + ch * 8) = h;
    }
  } else {
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int idx = tid + 256 * p, row = idx >> 4, ch = idx & 15;
      const float4 v = *reinterpret_cast<const float4*>(jb.src + (size_t)(r0 + row) * jb.C + c0 + ch * 4);
      half4 h;
      h[0] = (half_t)v.x; h[1] = (half_t)v.y; h[2] = (half_t)v.z; h[3] = (half_t)v.w;
      *reinterpret_cast<half4*>(jb.dst + (size_t)shadow_row(jb, r0 + row) * jb.C + c0 + ch * 4) = h;
      *reinterpret_cast<half4*>(tile + row * kTp + ch * 4) = h;
    }
  }
  if (!jb.dst_t) return;  // block-uniform
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int idx = tid + 256 * p, c = idx >> 3, rch = idx & 7;
    half8 w;
#pragma unroll
    for (int q = 0; q < 8; q++) w[q] = tile[(rch * 8 + q) * kTp + c];
    // 8 consecutive source rows never straddle a 32-row block
    st_h8(jb.dst_t + (size_t)(c0 + c) * jb.ldt + shadow_row(jb, r0 + rch * 8), w);
  }
}

}  // namespace

// ANE_NORM_BWD_FAST=0: every RMSNorm backward through the general kernel
// (read once per process)
static bool norm_bwd_fast() {
  static const bool on = [] {
    const char* f = getenv("ANE_NORM_BWD_FAST");
    return !f || atoi(f) != 0;
  }();
  return on;
}

hipError_t norm_bwd(const NormBwdArgs& a, hipStream_t s) {
  if (a.D % 64 || a.D > 1024 || a.T <= 0) return hipErrorInvalidValue;
  const dim3 g(norm_bwd_blocks(a.T));
  const bool gain_only = a.gain && a.dgain_part && !a.addend2 && !a.ve_dx && !a.lam_x && !a.lam_x0 && !a.lam_part &&
                         !a.gx0 && !a.general && norm_bwd_fast();
  if (gain_only && a.addend) hipLaunchKernelGGL(norm_bwd_gain_kernel<true>, g, dim3(64 * kNormBwdRows), 0, s, a);
  else if (gain_only) hipLaunchKernelGGL(norm_bwd_gain_kernel<false>, g, dim3(64 * kNormBwdRows), 0, s, a);
  else hipLaunchKernelGGL(norm_bwd_kernel, g, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t reduce_partials_add(float* dst, const float* part, int nblocks, int n, hipStream_t s, bool overwrite) {
  hipLaunchKernelGGL(reduce_partials_kernel, dim3((n + 63) / 64), dim3(1024), 0, s, dst, part, nblocks, n,
                     overwrite ? 1 : 0);
  return hipGetLastError();
}

hipError_t reduce_dots_add(float* d0, float* d1, const double* part, int nblocks, float sign, hipStream_t s) {
  hipLaunchKernelGGL(reduce_dots_kernel, dim3(1), dim3(256), 0, s, d0, d1, part, nblocks, sign);
  return hipGetLastError();
}

hipError_t backout_bwd(float* ginj, double* part, const float* d, const float* xmid, const float* lam_p, int T, int D,
                       hipStream_t s) {
  hipLaunchKernelGGL(backout_bwd_kernel, dim3(256), dim3(256), 0, s, ginj, part, d, xmid, lam_p, (size_t)T * D);
  return hipGetLastError();
}

hipError_t backout_fwd(float* out, const float* x, const float* xm, const float* lam_p, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(backout_fwd_kernel, dim3(flat_grid(n)), dim3(256), 0, s, out, x, xm, lam_p, n);
  return hipGetLastError();
}

hipError_t axpy_inplace(float* y, const float* x, half_t* yh, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(axpy_kernel, dim3(flat_grid(n)), dim3(256), 0, s, y, x, yh, n);
  return hipGetLastError();
}

hipError_t smear_bwd_prep(half_t* dgp, float* dout2, double* part, const float* dy, const float* gact,
                          const float* x0, const float* lam_p, int T, int D, int seq, hipStream_t s) {
  hipLaunchKernelGGL(smear_bwd_kernel, dim3(256), dim3(256), 0, s, dgp, dout2, part, dy, gact, x0, lam_p, T, D, seq);
  return hipGetLastError();
}

hipError_t embed_bwd(float* G, const float* dx, const uint16_t* tok, int T, int D, int V, hipStream_t s) {
  hipLaunchKernelGGL(embed_bwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, G, dx, tok, T, D, V);
  return hipGetLastError();
}

hipError_t ve_bwd(float* gemb, float* ggate, float* ve_dx, const half_t* dv, int ldv, const float* x, const float* emb,
                  const float* vg, const uint16_t* tok, int T, int D, int NH, int V, hipStream_t s) {
  if (NH > 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ve_bwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, gemb, ggate, ve_dx, dv, ldv, x, emb, vg, tok,
                     T, D, NH, V);
  return hipGetLastError();
}

static bool transpose_ok(int R, int C, int ldi, int ldo) {
  return R > 0 && C > 0 && R % 64 == 0 && C % 64 == 0 && ldi >= C && ldo >= R && ldi % 8 == 0 && ldo % 8 == 0;
}

hipError_t transpose2_h(half_t* out_a, const half_t* in_a, int Ra, int Ca, int ldi_a, int ldo_a, half_t* out_b,
                        const half_t* in_b, int Rb, int Cb, int ldi_b, int ldo_b, hipStream_t s) {
  if (!transpose_ok(Ra, Ca, ldi_a, ldo_a)) return hipErrorInvalidValue;
  TransposeJob ja{out_a, in_a, Ca, ldi_a, ldo_a, (Ra / 64) * (Ca / 64)};
  TransposeJob jb{nullptr, nullptr, 64, 64, 64, 0};
  if (out_b) {
    if (!transpose_ok(Rb, Cb, ldi_b, ldo_b)) return hipErrorInvalidValue;
    jb = TransposeJob{out_b, in_b, Cb, ldi_b, ldo_b, (Rb / 64) * (Cb / 64)};
  }
  const int tiles = ja.ntiles + jb.ntiles;
  hipLaunchKernelGGL(transpose2_kernel, dim3((tiles + 3) / 4), dim3(256), 0, s, ja, jb);
  return hipGetLastError();
}

hipError_t transpose_h(half_t* out, const half_t* in, int R, int C, int ldi, int ldo, hipStream_t s) {
  return transpose2_h(out, in, R, C, ldi, ldo, nullptr, nullptr, 0, 0, 0, 0, s);
}

hipError_t shadow_refresh(const ShadowJob* jobs_dev, int njobs, int ntiles, hipStream_t s) {
  if (njobs <= 0 || ntiles <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(shadow_kernel<false>, dim3(ntiles), dim3(256), 0, s, jobs_dev, njobs);
  return hipGetLastError();
}

hipError_t shadow_transpose(const ShadowJob* jobs_dev, int njobs, int ntiles, hipStream_t s) {
  if (njobs <= 0 || ntiles <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(shadow_kernel<true>, dim3(ntiles), dim3(256), 0, s, jobs_dev, njobs);
  return hipGetLastError();
}

hipError_t adam_fused_update(const AdamArgs& a, const UpdateJob* jobs_dev, int njobs, int nblocks, int blk_base,
                             hipStream_t s) {
  if (a.nseg <= 0 || a.nseg > kMaxAdamSegs || njobs <= 0 || nblocks <= 0 || blk_base < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(adam_fused_kernel, dim3(nblocks), dim3(256), 0, s, a, jobs_dev, njobs, blk_base);
  return hipGetLastError();
}

hipError_t fill_f32(float* p, size_t n, float v, hipStream_t s) {
  hipLaunchKernelGGL(fill_kernel, dim3(flat_grid(n)), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

hipError_t sumsq(double* out, double* part, const float* g, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(sumsq_kernel, dim3(kSumsqBlocks), dim3(256), 0, s, part, g, n);
  hipLaunchKernelGGL(sumsq_final_kernel, dim3(1), dim3(256), 0, s, out, part, kSumsqBlocks);
  return hipGetLastError();
}

hipError_t adam_update(const AdamArgs& a, hipStream_t s) {
  if (a.nseg <= 0 || a.nseg > kMaxAdamSegs) return hipErrorInvalidValue;
  int64_t mx = 1;
  for (int i = 0; i < a.nseg; i++) mx = a.seg[i].len > mx ? a.seg[i].len : mx;
  hipLaunchKernelGGL(adam_kernel, dim3(flat_grid((size_t)mx, 2048), a.nseg), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace ane
