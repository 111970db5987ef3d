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
constexpr int kMaxRegCout = 128;

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
  ShiftedStats st;
#pragma unroll
  for (int j = 0; j < COB; ++j) {
    const int co = co0 + j;
    if (valid && co < p.Cout) {
      float v = acc[j] + (bias ? bias[co] : 0.f);
      if (partials) st.add(v);
      v = apply_act(v, act, p.alpha);
      if (p.res) v += p.res[((int64_t)b * p.Cout + co) * p.ldr + t];
      if (y) y[((int64_t)b * p.Cout + co) * p.ldy + t] = v;
    }
  }
  if (partials) {
    float n, mean, m2;
    st.finish(n, mean, m2);
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

// Small contractions (groups = 1, Cin*K = CK <= 32): each thread loads its whole input window
// (CK samples) into registers with all loads in flight together, then produces the COB output
// channels of its workgroup (grid.y spreads the channels, so there are enough waves per SIMD to
// hide memory latency). Weights are staged in LDS and read as broadcasts.
template <int CK, int COB, bool REFLECT>
__global__ __launch_bounds__(kThreads) void conv1d_direct_reg_kernel(ConvParams p,
                                                                     const float* __restrict__ x,
                                                                     const float* __restrict__ w,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ y, int act,
                                                                     float* __restrict__ partials) {
  __shared__ float red[3 * (kThreads / 64)];
  // this workgroup's COB output channels, weights transposed to [e][co] so one 16-byte LDS
  // read serves four output channels
  __shared__ __attribute__((aligned(16))) float wt[CK * COB];
  const int b = blockIdx.z;
  const int cob0 = blockIdx.y * COB;
  const int t = blockIdx.x * kThreads + threadIdx.x;
  const bool valid = t < p.Lout;
  for (int i = threadIdx.x; i < CK * COB; i += kThreads) {
    const int co = i / CK, e = i - co * CK;
    wt[e * COB + co] = w[(int64_t)(cob0 + co) * CK + e];
  }
  __syncthreads();
  const float* xb = x + (int64_t)b * p.Cin * p.Lin;
  float xv[CK];
  // every window load is issued before any is used: addresses are clamped (zero padding) or
  // mirrored (reflect) instead of branched around (a load under a branch makes the compiler wait
  // for it, and for all earlier loads, before the next one); out-of-range taps are zeroed after
  const int base = min(t, p.Lout - 1) * p.stride - p.pad;
#pragma unroll
  for (int e = 0; e < CK; ++e) {
    const int ci = e / p.K, kk = e - ci * p.K;
    int pos = base + kk * p.dilation;
    float keep = valid ? 1.f : 0.f;
    if constexpr (REFLECT) {
      pos = abs(pos);
      pos = min(pos, 2 * (p.Lin - 1) - pos);
    } else {
      keep = (pos >= 0 && pos < p.Lin) ? keep : 0.f;
      pos = min(max(pos, 0), p.Lin - 1);
    }
    xv[e] = xb[(int64_t)ci * p.Lin + pos] * keep;  // x is finite: 0 * x = 0
  }
  ShiftedStats st;
  {
    const int co0 = cob0;
    float acc[COB];
#pragma unroll
    for (int j = 0; j < COB; ++j) acc[j] = bias ? bias[co0 + j] : 0.f;
#pragma unroll
    for (int e = 0; e < CK; ++e)
#pragma unroll
      for (int j4 = 0; j4 < COB; j4 += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(wt + e * COB + j4);
        acc[j4 + 0] = fmaf(xv[e], w4.x, acc[j4 + 0]);
        acc[j4 + 1] = fmaf(xv[e], w4.y, acc[j4 + 1]);
        acc[j4 + 2] = fmaf(xv[e], w4.z, acc[j4 + 2]);
        acc[j4 + 3] = fmaf(xv[e], w4.w, acc[j4 + 3]);
      }
    if (valid) {
#pragma unroll
      for (int j = 0; j < COB; ++j) {
        if (partials) st.add(acc[j]);
        float v = apply_act(acc[j], act, p.alpha);
        if (p.res) v += p.res[((int64_t)b * p.Cout + co0 + j) * p.ldr + t];
        if (y) y[((int64_t)b * p.Cout + co0 + j) * p.ldy + t] = v;
      }
    }
  }
  if (partials) {
    float n, mean, m2;
    st.finish(n, mean, m2);
    block_welford(n, mean, m2, red);
    float* pb = partials + (int64_t)b * gridDim.x * gridDim.y * 3;
    if (threadIdx.x == 0) {
      float* o = pb + (int64_t)(blockIdx.y * gridDim.x + blockIdx.x) * 3;
      o[0] = n;
      o[1] = mean;
      o[2] = m2;
    }
  }
}

// Register-window variant applies when groups = 1, Cin*K is 8, 16, 24 or 32, Cout % 16 == 0
// and Cout <= kMaxRegCout.
int reg_ck(const ConvParams& p) {
  const int ck = p.Cin * p.K;
  if (p.groups != 1 || p.Cout % 16 != 0 || p.Cout > kMaxRegCout) return 0;
  return (ck == 8 || ck == 16 || ck == 24 || ck == 32) ? ck : 0;
}

int co_block(const ConvParams& p) {
  const int coutpg = p.Cout / p.groups;
  return (coutpg % 16 == 0) ? 16 : 1;
}

}  // namespace

int conv1d_direct_num_chunks(const ConvParams& p) {
  if (reg_ck(p)) return (int)cdiv(p.Lout, kThreads) * (p.Cout / 16);
  return (int)cdiv(p.Lout, kThreads) * (p.Cout / co_block(p));
}

void conv1d_direct(const LaunchCtx& c, const ConvParams& p0, const float* x, const float* w,
                   const float* bias, float* y, int act, float* partials, int* nchunk) {
  ConvParams p = p0;
  if (p.ldy == 0) p.ldy = p.Lout;
  if (p.ldr == 0) p.ldr = p.ldy;
  if (const int ck = reg_ck(p)) {
    dim3 grid(cdiv(p.Lout, kThreads), p.Cout / 16, p.B);
    if (nchunk) *nchunk = (int)(grid.x * grid.y);
#define MNN_REG(CKV, R) launch(c, "conv1d_direct_f32", conv1d_direct_reg_kernel<CKV, 16, R>, grid, dim3(kThreads), 0, p, x, w, bias, y, act, partials)
    switch (ck * 2 + (p.reflect ? 1 : 0)) {
      case 16: return MNN_REG(8, false);
      case 17: return MNN_REG(8, true);
      case 32: return MNN_REG(16, false);
      case 33: return MNN_REG(16, true);
      case 48: return MNN_REG(24, false);
      case 49: return MNN_REG(24, true);
      case 64: return MNN_REG(32, false);
      default: return MNN_REG(32, true);
    }
#undef MNN_REG
  }
  MNN_REQUIRE(y, MNN_ERR_INVALID_ARGUMENT, "conv1d_direct: output required");
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

bool conv1d_direct_fusable(const ConvParams& p) { return reg_ck(p) != 0; }

}  // namespace k
}  // namespace mnn
