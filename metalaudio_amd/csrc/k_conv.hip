// Direct 1-D convolution for small contractions (Cin/groups * K small, e.g. the 2-channel
// first encoder level where Cin*K = 16 and the layer is HBM-bound). Dense contractions go to the
// implicit-GEMM MFMA path in k_gemm.hip instead.
//
// Semantics follow dynamic_conv1d_forward / conv1d_forward (DynamicConv1D.swift:358-401,
// Conv1D.swift:310-512): y[b][co][t] = bias[co] + sum_ci sum_k x[b][ci][t*s - p + k*d] * W[co][ci][k]
// with the reflect padding of DynamicConv1D.swift:288-324 applied by index arithmetic
// (x[-i] = x[i], x[L-1+i] = x[L-1-i]) instead of a host-side padded copy.
//
// One thread per output position; each thread produces a block of COB output channels so the
// input window is loaded once per block and every output is written once, coalesced along t.
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int kThreads = 256;

template <int COB>
__global__ __launch_bounds__(kThreads) void conv1d_direct_kernel(ConvParams p,
                                                                 const float* __restrict__ x,
                                                                 const float* __restrict__ w,
                                                                 const float* __restrict__ bias,
                                                                 float* __restrict__ y, int act,
                                                                 float* __restrict__ partials) {
  __shared__ float red[3 * (kThreads / 64)];
  const int b = blockIdx.z;
  const int co0 = blockIdx.y * COB;
  const int t = blockIdx.x * kThreads + threadIdx.x;
  const int cinpg = p.Cin / p.groups, coutpg = p.Cout / p.groups;
  const int grp = co0 / coutpg;  // COB divides coutpg, so the block is inside one group
  const float* xb = x + ((int64_t)b * p.Cin + (int64_t)grp * cinpg) * p.Lin;
  float acc[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = 0.f;
  const bool valid = t < p.Lout;
  if (valid) {
    const int base = t * p.stride - p.pad;
    for (int ci = 0; ci < cinpg; ++ci) {
      const float* xr = xb + (int64_t)ci * p.Lin;
      for (int kk = 0; kk < p.K; ++kk) {
        int pos = base + kk * p.dilation;
        float xv;
        if (p.reflect) {
          pos = pos < 0 ? -pos : pos;
          pos = pos >= p.Lin ? 2 * (p.Lin - 1) - pos : pos;
          xv = xr[pos];
        } else {
          xv = (pos >= 0 && pos < p.Lin) ? xr[pos] : 0.f;
        }
        const float* wp = w + ((int64_t)co0 * cinpg + ci) * p.K + kk;
#pragma unroll
        for (int j = 0; j < COB; ++j) acc[j] = fmaf(xv, wp[(int64_t)j * cinpg * p.K], acc[j]);
      }
    }
  }
  float n = 0.f, mean = 0.f, m2 = 0.f;
#pragma unroll
  for (int j = 0; j < COB; ++j) {
    const int co = co0 + j;
    if (valid && co < p.Cout) {
      float v = acc[j] + (bias ? bias[co] : 0.f);
      if (partials) {
        n += 1.f;
        float d = v - mean;
        mean += d / n;
        m2 += d * (v - mean);
      }
      y[((int64_t)b * p.Cout + co) * p.Lout + t] = apply_act(v, act);
    }
  }
  if (partials) {
    block_welford(n, mean, m2, red);
    if (threadIdx.x == 0) {
      const int nchunk = gridDim.x * gridDim.y;
      float* o = partials + ((int64_t)b * nchunk + blockIdx.y * gridDim.x + blockIdx.x) * 3;
      o[0] = n;
      o[1] = mean;
      o[2] = m2;
    }
  }
}

int co_block(const ConvParams& p) {
  const int coutpg = p.Cout / p.groups;
  return (coutpg % 16 == 0) ? 16 : 1;
}

}  // namespace

int conv1d_direct_num_chunks(const ConvParams& p) {
  return (int)cdiv(p.Lout, kThreads) * (p.Cout / co_block(p));
}

void conv1d_direct(const LaunchCtx& c, const ConvParams& p, const float* x, const float* w,
                   const float* bias, float* y, int act, float* partials, int* nchunk) {
  const int cob = co_block(p);
  dim3 grid(cdiv(p.Lout, kThreads), p.Cout / cob, p.B);
  if (nchunk) *nchunk = (int)(grid.x * grid.y);
  if (cob == 16)
    launch(c, "conv1d_direct_f32", conv1d_direct_kernel<16>, grid, dim3(kThreads), 0, p, x, w,
           bias, y, act, partials);
  else
    launch(c, "conv1d_direct_f32", conv1d_direct_kernel<1>, grid, dim3(kThreads), 0, p, x, w,
           bias, y, act, partials);
}

}  // namespace k
}  // namespace mnn
