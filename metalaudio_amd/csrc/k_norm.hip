// GroupNorm and LayerNorm kernels.
//
// GroupNorm (Normalization.swift:32-725) launches one 256-thread workgroup per (batch, group) in
// the reference, which serialises a GroupNorm(1 group) over millions of elements on one CU. Here
// the statistics are a grid-wide reduction in three steps: per-chunk partials (count, mean, M2)
// from many workgroups, a fixed-order Chan merge in fp64 (deterministic), and the apply step
// y = act(x*scale + shift) with per-channel coefficients. The partials can also come from the
// epilogue of the producing convolution, and the apply step can be folded into the consumer
// GEMM's operand load, so the normalised tensor never has to be written to HBM.
//
// LayerNorm (Normalization.swift:804-879): one wave per row, the row held in registers, so the
// row is read from HBM once (the reference reads it three times). Two-pass statistics
// (mean, then E[(x-mean)^2]), biased variance, eps inside the square root.
#include "device_utils.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"  // wait_vmcnt

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 4096;  // elements per GroupNorm statistics partial

// One partial per chunk of kChunk consecutive elements of a group (a group's channels are
// contiguous in [B][C][L]): every thread loads its kChunk / kThreads elements up front (16-byte
// vectors when the rows allow), takes their mean and M2 in two passes over its registers, and the
// workgroup merges the threads' (count, mean, M2) in a fixed order.
constexpr int kStatPer = kChunk / kThreads;  // elements per thread
static_assert(kStatPer % 4 == 0, "whole float4 vectors per thread");
__global__ __launch_bounds__(kThreads) void gn_stats_partial_kernel(const float* __restrict__ x,
                                                                    int C, int64_t L, int G,
                                                                    float* __restrict__ partials,
                                                                    int nchunk, int vec) {
  __shared__ float red[3 * (kThreads / 64)];
  const int bg = blockIdx.y;
  const int b = bg / G, g = bg % G;
  const int cpg = C / G;
  const int64_t total = (int64_t)cpg * L;
  const float* base = x + ((int64_t)b * C + (int64_t)g * cpg) * L;
  const int64_t start = (int64_t)blockIdx.x * kChunk;
  float v[kStatPer];
  bool ok[kStatPer];
  if (vec) {
    // thread t covers vectors start/4 + t + kThreads * k: coalesced 16-byte loads
    const float4* b4 = reinterpret_cast<const float4*>(base + start);
    const int64_t n4 = (min(start + (int64_t)kChunk, total) - start) >> 2;
#pragma unroll
    for (int k = 0; k < kStatPer / 4; ++k) {
      const int64_t i = threadIdx.x + (int64_t)kThreads * k;
      const float4 q = b4[min(i, max(n4 - 1, (int64_t)0))];
      v[4 * k + 0] = q.x;
      v[4 * k + 1] = q.y;
      v[4 * k + 2] = q.z;
      v[4 * k + 3] = q.w;
#pragma unroll
      for (int e = 0; e < 4; ++e) ok[4 * k + e] = i < n4;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kStatPer; ++k) {
      const int64_t i = start + threadIdx.x + (int64_t)kThreads * k;
      ok[k] = i < total;
      v[k] = base[min(i, total - 1)];
    }
  }
  float n = 0.f, s = 0.f;
#pragma unroll
  for (int k = 0; k < kStatPer; ++k) {
    n += ok[k] ? 1.f : 0.f;
    s += ok[k] ? v[k] : 0.f;
  }
  const float mean0 = n > 0.f ? s / n : 0.f;
  float m2 = 0.f;
#pragma unroll
  for (int k = 0; k < kStatPer; ++k) {
    const float d = v[k] - mean0;
    m2 = ok[k] ? fmaf(d, d, m2) : m2;
  }
  float mean = mean0;
  block_welford(n, mean, m2, red);
  if (threadIdx.x == 0) {
    float* p = partials + ((int64_t)bg * nchunk + blockIdx.x) * 3;
    p[0] = n;
    p[1] = mean;
    p[2] = m2;
  }
}

__global__ __launch_bounds__(kThreads) void gn_finalize_kernel(const float* __restrict__ partials,
                                                               int C, int G, int nchunk, float eps,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ beta,
                                                               float* __restrict__ coef) {
  __shared__ double sn[kThreads], smean[kThreads], sm2[kThreads];
  __shared__ float s_mean, s_rstd;
  const int bg = blockIdx.x;
  const int b = bg / G, g = bg % G;
  const float* p = partials + (int64_t)bg * nchunk * 3;
  // each thread merges a strided subset in increasing order
  double n = 0.0, mean = 0.0, m2 = 0.0;
  for (int j = threadIdx.x; j < nchunk; j += kThreads) {
    double n2 = p[j * 3 + 0], mean2 = p[j * 3 + 1], m22 = p[j * 3 + 2];
    double nt = n + n2;
    if (nt > 0.0) {
      double d = mean2 - mean;
      double w = n2 / nt;
      mean += d * w;
      m2 += m22 + d * d * n * w;
    }
    n = nt;
  }
  sn[threadIdx.x] = n;
  smean[threadIdx.x] = mean;
  sm2[threadIdx.x] = m2;
  __syncthreads();
  for (int off = kThreads / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) {
      double na = sn[threadIdx.x], ma = smean[threadIdx.x], qa = sm2[threadIdx.x];
      double nb = sn[threadIdx.x + off], mb = smean[threadIdx.x + off], qb = sm2[threadIdx.x + off];
      double nt = na + nb;
      if (nt > 0.0) {
        double d = mb - ma;
        double w = nb / nt;
        smean[threadIdx.x] = ma + d * w;
        sm2[threadIdx.x] = qa + qb + d * d * na * w;
      }
      sn[threadIdx.x] = nt;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    double cnt = sn[0];
    double var = cnt > 0.0 ? sm2[0] / cnt : 0.0;  // biased (population) variance
    float rstd = (float)(1.0 / sqrt(var + (double)eps));
    if (!isfinite(rstd)) rstd = 0.f;  // reference CPU path guard (Normalization.swift:695-699)
    s_mean = (float)smean[0];
    s_rstd = rstd;
  }
  __syncthreads();
  const int cpg = C / G;
  for (int cc = threadIdx.x; cc < cpg; cc += kThreads) {
    const int ch = g * cpg + cc;
    const float gm = gamma ? gamma[ch] : 1.f;
    const float bt = beta ? beta[ch] : 0.f;
    const float scale = gm * s_rstd;
    float* o = coef + ((int64_t)b * C + ch) * 2;
    o[0] = scale;
    o[1] = bt - s_mean * scale;
  }
}

__global__ __launch_bounds__(kThreads) void gn_apply_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t L,
                                                            const float* __restrict__ coef,
                                                            int act, int vec) {
  const int64_t row = blockIdx.y;  // b*C + c
  const float sc = coef[row * 2 + 0], sh = coef[row * 2 + 1];
  const float* xr = x + row * L;
  float* yr = y + row * L;
  if (vec) {
    const int64_t L4 = L >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    float4* y4 = reinterpret_cast<float4*>(yr);
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < L4;
         i += (int64_t)gridDim.x * kThreads) {
      float4 v = x4[i];
      v.x = apply_act(fmaf(v.x, sc, sh), act);
      v.y = apply_act(fmaf(v.y, sc, sh), act);
      v.z = apply_act(fmaf(v.z, sc, sh), act);
      v.w = apply_act(fmaf(v.w, sc, sh), act);
      y4[i] = v;
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < L;
         i += (int64_t)gridDim.x * kThreads)
      yr[i] = apply_act(fmaf(xr[i], sc, sh), act);
  }
}

// GroupNorm apply with the statistics merged in the workgroup: x, y [B][C][L]; group (b, g) covers
// the contiguous cpg * L elements of channels [g * cpg, (g + 1) * cpg); its nparts partials sit
// at parts[((b * G + g) * nparts + j) * 3]. y = act((x - mean) * rstd * gamma_c + beta_c), biased
// variance, rsqrt(var + eps) as gn_finalize. Each workgroup handles kApplyItems float4 (vec) or
// floats of one group; its loads are issued before the merge so the two overlap.
constexpr int kApplyPer = 4;  // items per thread
__global__ __launch_bounds__(kThreads) void gn_apply_parts_kernel(
    const float* __restrict__ x, float* __restrict__ y, int C, int64_t L, int G,
    const float* __restrict__ parts, int nparts, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, int act, int vec) {
  const int bg = blockIdx.y;
  const int cpg = C / G;
  const int64_t total = (int64_t)cpg * L;
  const int64_t gbase = (int64_t)bg * total;  // (b * G + g) * cpg * L
  const int c0 = (bg % G) * cpg;
  // Every load is issued before the merge: the items, their channels' gamma / beta (through an
  // always-valid address: a missing vector reads x and is replaced by its fill), the partials.
  // Indices are 32-bit (the host checks cpg * L < 2^31).
  const int tot = (int)total, Li = (int)L;
  const int j0 = (int)blockIdx.x * kApplyPer * kThreads + (int)threadIdx.x;
  float gk[kApplyPer], bk[kApplyPer];
  auto chan_consts = [&](int k, int ch) {
    const float gv = *(gamma ? gamma + ch : x);
    const float bv = *(beta ? beta + ch : x);
    gk[k] = gamma ? gv : 1.f;
    bk[k] = beta ? bv : 0.f;
  };
  if (vec) {
    const int total4 = tot >> 2, L4 = Li >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(x + gbase);
    float4* y4 = reinterpret_cast<float4*>(y + gbase);
    float4 v[kApplyPer];
#pragma unroll
    for (int k = 0; k < kApplyPer; ++k) {
      const int i = min(j0 + k * kThreads, total4 - 1);
      v[k] = x4[i];
      chan_consts(k, c0 + i / L4);
    }
    PartsBatch<8> pb;
    pb.load(parts + (int64_t)bg * nparts * 3, nparts);
    double n, mean, m2;
    pb.merge(parts + (int64_t)bg * nparts * 3, nparts, n, mean, m2);
    const double var = n > 0.0 ? m2 / n : 0.0;
    float rstd = (float)(1.0 / sqrt(var + (double)eps));
    if (!isfinite(rstd)) rstd = 0.f;
    const float mf = (float)mean;
#pragma unroll
    for (int k = 0; k < kApplyPer; ++k) {
      const int i = j0 + k * kThreads;
      if (i < total4) {
        const float sc = gk[k] * rstd;
        const float sh = bk[k] - mf * sc;
        float4 o;
        o.x = apply_act(fmaf(v[k].x, sc, sh), act);
        o.y = apply_act(fmaf(v[k].y, sc, sh), act);
        o.z = apply_act(fmaf(v[k].z, sc, sh), act);
        o.w = apply_act(fmaf(v[k].w, sc, sh), act);
        y4[i] = o;
      }
    }
  } else {
    float v[kApplyPer];
#pragma unroll
    for (int k = 0; k < kApplyPer; ++k) {
      const int i = min(j0 + k * kThreads, tot - 1);
      v[k] = x[gbase + i];
      chan_consts(k, c0 + i / Li);
    }
    PartsBatch<8> pb;
    pb.load(parts + (int64_t)bg * nparts * 3, nparts);
    double n, mean, m2;
    pb.merge(parts + (int64_t)bg * nparts * 3, nparts, n, mean, m2);
    const double var = n > 0.0 ? m2 / n : 0.0;
    float rstd = (float)(1.0 / sqrt(var + (double)eps));
    if (!isfinite(rstd)) rstd = 0.f;
    const float mf = (float)mean;
#pragma unroll
    for (int k = 0; k < kApplyPer; ++k) {
      const int i = j0 + k * kThreads;
      if (i < tot) {
        const float sc = gk[k] * rstd;
        const float sh = bk[k] - mf * sc;
        y[gbase + i] = apply_act(fmaf(v[k], sc, sh), act);
      }
    }
  }
}

// LayerNorm, row in registers: NV float4 per lane, F % 4 == 0, F <= 256 * NV.
template <int NV>
__global__ __launch_bounds__(kThreads) void layernorm_reg_kernel(const float* __restrict__ x,
                                                                 float* __restrict__ y,
                                                                 int64_t rows, int F,
                                                                 const float* __restrict__ gamma,
                                                                 const float* __restrict__ beta,
                                                                 float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int F4 = F >> 2;
  const float4* xr = reinterpret_cast<const float4*>(x + row * F);
  const float4* g4 = reinterpret_cast<const float4*>(gamma);
  const float4* b4 = reinterpret_cast<const float4*>(beta);
  // gamma and beta are loaded with the row: a load between the stores below would make each
  // store wait for the earlier ones
  float4 v[NV], gv[NV], bv[NV];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < F4) {
      v[i] = xr[idx];
      gv[i] = g4[idx];
      bv[i] = b4[idx];
      s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    } else {
      v[i] = gv[i] = bv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const float mean = wave_sum_dpp(s) / (float)F;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < F4) {
      float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
      q += (a * a + b * b) + (c * c + d * d);
    }
  }
  const float var = wave_sum_dpp(q) / (float)F;
  const float rstd = 1.f / sqrtf(var + eps);
  float4* yr = reinterpret_cast<float4*>(y + row * F);
  wait_vmcnt<0>();  // every load has landed: the stores below need no waits between them
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = lane + 64 * i;
    if (idx < F4) {
      const float4 g = gv[i], bb = bv[i];
      float4 o;
      o.x = g.x * ((v[i].x - mean) * rstd) + bb.x;
      o.y = g.y * ((v[i].y - mean) * rstd) + bb.y;
      o.z = g.z * ((v[i].z - mean) * rstd) + bb.z;
      o.w = g.w * ((v[i].w - mean) * rstd) + bb.w;
      yr[idx] = o;
    }
  }
}

// Rows of exactly 256 * NV features, RPW rows per wave (rows w, w + W, ... for W waves in all),
// software-pipelined: the next row's loads are issued before the current row is reduced and
// stored, so its reads overlap this row's writes (with one row per wave, every wave loads at
// once and then stores at once). Every load is unconditional (the row index is clamped), so the
// compiler's waits count exactly the loads a use needs: the previous row's stores and the next
// row's loads stay in flight. x, gamma and beta are plain pointers and a scheduling barrier
// follows the loads: loads through restrict pointers count as invariant and were sunk past the
// reduction. gamma / beta stay in registers for every row.
template <int NV, int RPW>
__global__ __launch_bounds__(kThreads) void layernorm_pipe_kernel(
    const float* x, float* __restrict__ y, int64_t rows, const float* gamma, const float* beta,
    float eps) {
  constexpr int F = 256 * NV;
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t W = (int64_t)gridDim.x * (kThreads / 64);
  const float4* g4 = reinterpret_cast<const float4*>(gamma);
  const float4* b4 = reinterpret_cast<const float4*>(beta);
  float4 gv[NV], bv[NV], v[2][NV];
  auto load_row = [&](int64_t row, float4 (&d)[NV]) {
    const float4* xr = reinterpret_cast<const float4*>(x + min(row, rows - 1) * F);
#pragma unroll
    for (int i = 0; i < NV; ++i) d[i] = xr[lane + 64 * i];
  };
  load_row(w0, v[0]);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    gv[i] = g4[lane + 64 * i];
    bv[i] = b4[lane + 64 * i];
  }
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int64_t row = w0 + k * W;
    float4(&cur)[NV] = v[k & 1];
    if (k + 1 < RPW) load_row(row + W, v[(k + 1) & 1]);
    __builtin_amdgcn_sched_barrier(0);  // the loads above stay ahead of this row's work
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) s += (cur[i].x + cur[i].y) + (cur[i].z + cur[i].w);
    const float mean = wave_sum_dpp(s) / (float)F;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const float a = cur[i].x - mean, b = cur[i].y - mean, c = cur[i].z - mean,
                  d = cur[i].w - mean;
      q += (a * a + b * b) + (c * c + d * d);
    }
    const float rstd = 1.f / sqrtf(wave_sum_dpp(q) / (float)F + eps);
    // unconditional stores: a row past the last one was computed from the last row and writes
    // the same bytes there (under a branch, the compiler's waits after it would also wait for
    // these stores)
    float4* yr = reinterpret_cast<float4*>(y + min(row, rows - 1) * F);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float4 o;
      o.x = gv[i].x * ((cur[i].x - mean) * rstd) + bv[i].x;
      o.y = gv[i].y * ((cur[i].y - mean) * rstd) + bv[i].y;
      o.z = gv[i].z * ((cur[i].z - mean) * rstd) + bv[i].z;
      o.w = gv[i].w * ((cur[i].w - mean) * rstd) + bv[i].w;
      yr[lane + 64 * i] = o;
    }
  }
}

// gamma / beta are deliberately not __restrict__: loads through restrict pointers to constant
// data count as invariant, and the compiler then moves them freely past the wait below.
// DUAL: a second LayerNorm of the same rows (its own gamma2 / beta2 / eps2) into y2, so two
// normalisations of one input read it once.
template <int NV, bool DUAL>
__global__ __launch_bounds__(kThreads) void layernorm_row16_kernel(
    const float* __restrict__ x, float* __restrict__ y, int64_t rows, const float* gamma,
    const float* beta, float eps, float* __restrict__ y2, const float* gamma2, const float* beta2,
    float eps2) {
  constexpr int F = 64 * NV;
  const int lane = threadIdx.x & 63, sub = lane & 15;
  const int64_t row = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * 4 + lane / 16;
  const bool live = row < rows;
  const int64_t r = live ? row : rows - 1;  // dead rows compute on a valid row, store nothing
  const float4* xr = reinterpret_cast<const float4*>(x + r * F);
  float4 v[NV], gv[NV], bv[NV], gv2[DUAL ? NV : 1], bv2[DUAL ? NV : 1];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = xr[sub + 16 * i];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    gv[i] = reinterpret_cast<const float4*>(gamma)[sub + 16 * i];
    bv[i] = reinterpret_cast<const float4*>(beta)[sub + 16 * i];
    if constexpr (DUAL) {
      gv2[i] = reinterpret_cast<const float4*>(gamma2)[sub + 16 * i];
      bv2[i] = reinterpret_cast<const float4*>(beta2)[sub + 16 * i];
    }
  }
  // one wait for every load above; the scheduling barriers and the memory clobber keep the
  // compiler from moving the gamma / beta loads behind the reductions (next to their use: a
  // second memory round trip)
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
  const float mean = row16_sum(s) * (1.f / F);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i].x -= mean;
    v[i].y -= mean;
    v[i].z -= mean;
    v[i].w -= mean;
    q += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
  }
  const float var = row16_sum(q) * (1.f / F);
  const float rstd = 1.f / sqrtf(var + eps);
  const float rstd2 = DUAL ? 1.f / sqrtf(var + eps2) : 0.f;
  // outputs computed before the store branch (the loads stay in the block of the wait above)
  float4 o[NV], o2[DUAL ? NV : 1];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    o[i].x = gv[i].x * (v[i].x * rstd) + bv[i].x;
    o[i].y = gv[i].y * (v[i].y * rstd) + bv[i].y;
    o[i].z = gv[i].z * (v[i].z * rstd) + bv[i].z;
    o[i].w = gv[i].w * (v[i].w * rstd) + bv[i].w;
    if constexpr (DUAL) {
      o2[i].x = gv2[i].x * (v[i].x * rstd2) + bv2[i].x;
      o2[i].y = gv2[i].y * (v[i].y * rstd2) + bv2[i].y;
      o2[i].z = gv2[i].z * (v[i].z * rstd2) + bv2[i].z;
      o2[i].w = gv2[i].w * (v[i].w * rstd2) + bv2[i].w;
    }
  }
  if (!live) return;
  float4* yr = reinterpret_cast<float4*>(y + r * F);
#pragma unroll
  for (int i = 0; i < NV; ++i) yr[sub + 16 * i] = o[i];
  if constexpr (DUAL) {
    float4* yr2 = reinterpret_cast<float4*>(y2 + r * F);
#pragma unroll
    for (int i = 0; i < NV; ++i) yr2[sub + 16 * i] = o2[i];
  }
}

// LayerNorm, any F: three passes over the row from memory, one wave per row.
__global__ __launch_bounds__(kThreads) void layernorm_generic_kernel(
    const float* __restrict__ x, float* __restrict__ y, int64_t rows, int F,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * F;
  float s = 0.f;
  for (int i = lane; i < F; i += 64) s += xr[i];
  const float mean = wave_sum_dpp(s) / (float)F;
  float q = 0.f;
  for (int i = lane; i < F; i += 64) {
    float d = xr[i] - mean;
    q += d * d;
  }
  const float var = wave_sum_dpp(q) / (float)F;
  const float rstd = 1.f / sqrtf(var + eps);
  float* yr = y + row * F;
  for (int i = lane; i < F; i += 64) yr[i] = gamma[i] * ((xr[i] - mean) * rstd) + beta[i];
}

// (mean, M2) of each 64 consecutive features of every row (F % 64 == 0): a 16-lane group per
// 64 features, one float4 per lane, DPP reductions within the group. Optionally copies x to y on
// the way (the same float4s).
__global__ __launch_bounds__(kThreads) void ln_row_parts_kernel(const float* __restrict__ x,
                                                                float* __restrict__ y,
                                                                float* __restrict__ parts,
                                                                int64_t n4) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const bool live = i < n4;
  const float4 v = reinterpret_cast<const float4*>(x)[live ? i : n4 - 1];
  if (y && live) reinterpret_cast<float4*>(y)[i] = v;
  const float mean = row16_sum((v.x + v.y) + (v.z + v.w)) * (1.f / 64.f);
  const float dx = v.x - mean, dy = v.y - mean, dz = v.z - mean, dw = v.w - mean;
  const float m2 = row16_sum((dx * dx + dy * dy) + (dz * dz + dw * dw));
  if (live && (i & 15) == 0) reinterpret_cast<float2*>(parts)[i >> 4] = make_float2(mean, m2);
}

// LayerNorm folded into the following linear map y = LN(x) W^T + b: Wf[n][k] = W[n][k] * gamma[k],
// c[n] = sum_k Wf[n][k], bf[n] = b[n] + sum_k W[n][k] * beta[k] (sums in fp64). One wave per n.
__global__ __launch_bounds__(kThreads) void ln_fold_kernel(const float* __restrict__ W,
                                                           const float* __restrict__ b,
                                                           const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, int N,
                                                           int K, float* __restrict__ Wf,
                                                           float* __restrict__ c,
                                                           float* __restrict__ bf) {
  const int n = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;  // whole wave
  double cs = 0.0, bs = 0.0;
  for (int k = lane; k < K; k += 64) {
    const float w = W[(int64_t)n * K + k];
    const float wf = w * gamma[k];
    Wf[(int64_t)n * K + k] = wf;
    cs += (double)wf;
    bs += (double)w * (double)beta[k];
  }
  cs = wave_sum_dpp_d(cs);
  bs = wave_sum_dpp_d(bs);
  if (lane == 0) {
    c[n] = (float)cs;
    bf[n] = (float)((b ? (double)b[n] : 0.0) + bs);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void ln_row_parts(const LaunchCtx& c, const float* x, float* y, int64_t rows, int F,
                  float* parts) {
  MNN_REQUIRE(F % 64 == 0 && aligned16(x) && (!y || aligned16(y)) &&
                  (reinterpret_cast<uintptr_t>(parts) & 7) == 0,
              MNN_ERR_INVALID_ARGUMENT,
              "ln_row_parts: F % 64 == 0 and 16-byte aligned rows required");
  if (rows <= 0) return;
  const int64_t n4 = rows * F / 4;
  launch(c, "ln_row_parts_f32", ln_row_parts_kernel, dim3((unsigned)cdiv(n4, kThreads)),
         dim3(kThreads), 0, x, y, parts, n4);
}

void ln_fold(const LaunchCtx& c, const float* W, const float* b, const float* gamma,
             const float* beta, int N, int K, float* Wf, float* cvec, float* bf) {
  if (N <= 0) return;
  launch(c, "ln_fold_f32", ln_fold_kernel, dim3((unsigned)cdiv(N, kThreads / 64)), dim3(kThreads),
         0, W, b, gamma, beta, N, K, Wf, cvec, bf);
}

// Statistics partials of the allocation-free GroupNorm entry point. One copy per GPU, held until
// the process ends; every allocation-free call on a GPU uses that GPU's copy.
static __device__ __align__(256) float scratch[kGnScratchFloats];

float* gn_scratch(int device) {
  // hipGetSymbolAddress once per device, with that device current (the caller made it current);
  // host code uses the returned address, never the symbol itself
  static std::mutex mu;
  static std::map<int, float*> ptrs;
  std::lock_guard<std::mutex> lk(mu);
  auto it = ptrs.find(device);
  if (it != ptrs.end()) return it->second;
  int cur = -1;
  HIP_CHECK(hipGetDevice(&cur));
  MNN_REQUIRE(cur == device, MNN_ERR_INVALID_ARGUMENT,
              "gn_scratch: device " << device << " is not the current device");
  float* p = nullptr;
  HIP_CHECK(hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(scratch)));
  MNN_REQUIRE(p, MNN_ERR_GPU_EXECUTION, "no device address for the GroupNorm scratch");
  ptrs.emplace(device, p);
  return p;
}

int gn_num_chunks(int C, int G, int64_t L) {
  const int64_t total = (int64_t)(C / G) * L;
  return (int)std::max<int64_t>(1, (total + kChunk - 1) / kChunk);
}

void gn_stats_partial(const LaunchCtx& c, const float* x, int B, int C, int64_t L, int G,
                      float* partials, int nchunk) {
  // 16-byte loads when every group and chunk start is 16-byte aligned (chunks are 4096 floats)
  const int vec = (L % 4 == 0) && ((int64_t)(C / G) * L) % 4 == 0 && aligned16(x);
  launch(c, "gn_stats_partial", gn_stats_partial_kernel, dim3(nchunk, B * G), dim3(kThreads), 0,
         x, C, L, G, partials, nchunk, vec);
}

void gn_finalize(const LaunchCtx& c, const float* partials, int B, int C, int G, int nchunk,
                 float eps, const float* gamma, const float* beta, float* coef) {
  launch(c, "gn_finalize", gn_finalize_kernel, dim3(B * G), dim3(kThreads), 0, partials, C, G,
         nchunk, eps, gamma, beta, coef);
}

void gn_apply(const LaunchCtx& c, const float* x, float* y, int B, int C, int64_t L,
              const float* coef, int act) {
  const int vec = (L % 4 == 0) && aligned16(x) && aligned16(y);
  const int64_t items = vec ? L / 4 : L;
  unsigned gx = (unsigned)std::min<int64_t>((items + kThreads - 1) / kThreads, 4096);
  launch(c, "gn_apply", gn_apply_kernel, dim3(gx, (unsigned)(B * C)), dim3(kThreads), 0, x, y, L,
         coef, act, vec);
}

void gn_apply_parts(const LaunchCtx& c, const float* x, float* y, int B, int C, int64_t L, int G,
                    const float* parts, int nparts, const float* gamma, const float* beta,
                    float eps, int act) {
  MNN_REQUIRE((int64_t)(C / G) * L < ((int64_t)1 << 31) && nparts > 0, MNN_ERR_INVALID_ARGUMENT,
              "gn_apply_parts: a group holds 2^31 elements or more");
  const int vec = (L % 4 == 0) && aligned16(x) && aligned16(y);
  const int64_t total = (int64_t)(C / G) * L;
  const int64_t items = vec ? total / 4 : total;
  const int64_t per_wg = (int64_t)kApplyPer * kThreads;
  const unsigned gx = (unsigned)std::max<int64_t>(1, (items + per_wg - 1) / per_wg);
  launch(c, "gn_apply_parts", gn_apply_parts_kernel, dim3(gx, (unsigned)(B * G)), dim3(kThreads),
         0, x, y, C, L, G, parts, nparts, gamma, beta, eps, act, vec);
}

namespace {
void layernorm_row16(const LaunchCtx& c, const float* x, int64_t rows, int F, float* y,
                     const float* g, const float* b, float eps, float* y2, const float* g2,
                     const float* b2, float eps2) {
  const dim3 grid(cdiv(rows, 4 * (kThreads / 64))), block(kThreads);
#define MNN_LN16(NV)                                                                           \
  return y2 ? launch(c, "layernorm_f32", layernorm_row16_kernel<NV, true>, grid, block, 0, x, y, \
                     rows, g, b, eps, y2, g2, b2, eps2)                                         \
            : launch(c, "layernorm_f32", layernorm_row16_kernel<NV, false>, grid, block, 0, x, \
                     y, rows, g, b, eps, y2, g2, b2, eps2)
  switch (F / 64) {
    case 1: MNN_LN16(1);
    case 2: MNN_LN16(2);
    case 3: MNN_LN16(3);
    case 4: MNN_LN16(4);
    case 5: MNN_LN16(5);
    case 6: MNN_LN16(6);
    case 7: MNN_LN16(7);
    default: MNN_LN16(8);
  }
#undef MNN_LN16
}
}  // namespace

void layernorm2(const LaunchCtx& c, const float* x, int64_t rows, int F, float* y,
                const float* gamma, const float* beta, float eps, float* y2,
                const float* gamma2, const float* beta2, float eps2) {
  if (rows <= 0) return;
  const bool vec = (F % 4 == 0) && aligned16(x) && aligned16(y) && aligned16(y2) &&
                   aligned16(gamma) && aligned16(beta) && aligned16(gamma2) && aligned16(beta2);
  if (vec && F % 64 == 0 && F <= 512)
    return layernorm_row16(c, x, rows, F, y, gamma, beta, eps, y2, gamma2, beta2, eps2);
  layernorm(c, x, y, rows, F, gamma, beta, eps);
  layernorm(c, x, y2, rows, F, gamma2, beta2, eps2);
}

void layernorm(const LaunchCtx& c, const float* x, float* y, int64_t rows, int F,
               const float* gamma, const float* beta, float eps) {
  if (rows <= 0) return;
  dim3 grid(cdiv(rows, kThreads / 64)), block(kThreads);
  const bool vec = (F % 4 == 0) && aligned16(x) && aligned16(y) && aligned16(gamma) &&
                   aligned16(beta);
  const int nv = (F + 255) / 256;
  // rows of 64 * NV floats: 16 lanes per row, DPP reductions
  if (vec && F % 64 == 0 && F <= 512)
    return layernorm_row16(c, x, rows, F, y, gamma, beta, eps, nullptr, nullptr, nullptr, 0.f);
  if (vec && F == 2048 && rows >= 2 * 256 * (kThreads / 64)) {
    // two rows per wave, pipelined (at least a full device of waves)
    const dim3 pgrid((unsigned)cdiv(cdiv(rows, 2), kThreads / 64));
    return launch(c, "layernorm_f32", layernorm_pipe_kernel<8, 2>, pgrid, block, 0, x, y, rows,
                  gamma, beta, eps);
  }
  if (vec && nv <= 8) {
    switch (nv) {
      case 1: return launch(c, "layernorm_f32", layernorm_reg_kernel<1>, grid, block, 0, x, y, rows, F, gamma, beta, eps);
      case 2: return launch(c, "layernorm_f32", layernorm_reg_kernel<2>, grid, block, 0, x, y, rows, F, gamma, beta, eps);
      case 3: return launch(c, "layernorm_f32", layernorm_reg_kernel<3>, grid, block, 0, x, y, rows, F, gamma, beta, eps);
      case 4: return launch(c, "layernorm_f32", layernorm_reg_kernel<4>, grid, block, 0, x, y, rows, F, gamma, beta, eps);
      default: return launch(c, "layernorm_f32", layernorm_reg_kernel<8>, grid, block, 0, x, y, rows, F, gamma, beta, eps);
    }
  }
  launch(c, "layernorm_f32", layernorm_generic_kernel, grid, block, 0, x, y, rows, F, gamma, beta,
         eps);
}

}  // namespace k
}  // namespace mnn
