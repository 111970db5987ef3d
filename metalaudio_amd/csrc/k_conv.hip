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
#include <algorithm>
#include <type_traits>

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

// ---- Conv1D -> GroupNorm(1) [-> activation] in two passes (Sequential's fused chain) ----------
// The convolution's contraction is tiny (Cin * K <= 32), so the second pass recomputes it from the
// input (a few hundred KB, resident in L2) instead of reading back a stored pre-norm output: the
// only HBM stream is the output, written once. Each thread owns one output position and COB
// channels; weights are staged in LDS transposed to [e][co] and read as 16-byte broadcasts.

template <int CK, bool REFLECT>
__device__ __forceinline__ void load_window(const ConvParams& p, const float* __restrict__ xb, int t,
                                            bool valid, float (&xv)[CK]) {
  // branch-free addresses (clamped or mirrored) so that every load is in flight together
  const int base = min(t, p.Lout - 1) * p.stride - p.pad;
  int ci = 0, kk = 0;  // tap e = ci * K + kk, stepped without divisions
#pragma unroll
  for (int e = 0; e < CK; ++e) {
    int pos = base + kk * p.dilation;
    float keep = valid ? 1.f : 0.f;
    if constexpr (REFLECT) {
      pos = abs(pos);
      pos = min(pos, 2 * (p.Lin - 1) - pos);
    } else {
      keep = (pos >= 0 && pos < p.Lin) ? keep : 0.f;
      pos = min(max(pos, 0), p.Lin - 1);
    }
    xv[e] = xb[(int64_t)ci * p.Lin + pos] * keep;
    if (++kk == p.K) {
      kk = 0;
      ++ci;
    }
  }
}

// A workgroup's constants, staged in LDS: weights transposed to [e][co], then NX vectors of COB
// per-channel values (bias, GroupNorm gamma / beta; a null vector reads as its fill value). The
// loads are issued into registers first (fetch) and written to LDS later (put), so that the
// caller can put its own loads in flight between the two and wait once for all of them. Every
// load reads a valid global address (a null vector reads the weights instead and its value is
// replaced by the fill), so no load sits under a branch or behind a pointer select.
template <int CK, int COB, int NX, int NT = kThreads>
struct ConstStage {
  static_assert(NX >= 1 && NX <= 3, "one to three per-channel vectors");
  static constexpr int N = CK * COB + NX * COB;
  static constexpr int PER = (N + NT - 1) / NT;
  float v[PER];
  __device__ __forceinline__ void fetch(const float* __restrict__ w, int cob0, const float* e0,
                                        const float* e1, const float* e2, float f0, float f1,
                                        float f2) {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int i = threadIdx.x + r * NT;
      const int iw = min(i, CK * COB - 1);
      const int co = iw / CK, e = iw - co * CK;
      const int q = min(max(i - CK * COB, 0) / COB, NX - 1);
      const int j = min(max(i - CK * COB, 0) - q * COB, COB - 1);
      const float* src = q == 0 ? e0 : (q == 1 ? e1 : e2);
      const float fill = q == 0 ? f0 : (q == 1 ? f1 : f2);
      const bool wgt = i < CK * COB, have = src != nullptr;
      const float* addr = wgt || !have ? w + (int64_t)(cob0 + co) * CK + e : src + cob0 + j;
      const float val = *addr;
      v[r] = (wgt || have) ? val : fill;
    }
  }
  // LDS image: wt[e * COB + co] for the weights, then the extra vectors in order
  __device__ __forceinline__ void put(float* lds) const {
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int i = threadIdx.x + r * NT;
      if (i < CK * COB) {
        const int co = i / CK, e = i - co * CK;
        lds[e * COB + co] = v[r];
      } else if (i < N) {
        lds[i] = v[r];
      }
    }
  }
};

template <int CK, int COB>
__device__ __forceinline__ void window_dot(const float (&xv)[CK], const float* wt,
                                           float (&acc)[COB]) {
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
}

// Small contractions (groups = 1, Cin*K = CK <= 32): each thread loads its whole input window
// (CK samples) into registers, then produces the COB output channels of its workgroup (grid.y
// spreads the channels, so there are enough waves per SIMD to hide memory latency). Weights and
// bias are staged in LDS, their loads issued before the window's so that one wait covers both.
template <int CK, int COB, bool REFLECT>
__global__ __launch_bounds__(kThreads) void conv1d_direct_reg_kernel(ConvParams p,
                                                                     const float* __restrict__ x,
                                                                     const float* __restrict__ w,
                                                                     const float* __restrict__ bias,
                                                                     float* __restrict__ y, int act,
                                                                     float* __restrict__ partials) {
  __shared__ float red[3 * (kThreads / 64)];
  using Stage = ConstStage<CK, COB, 1>;
  __shared__ __attribute__((aligned(16))) float wt[Stage::N];  // weights, bias
  const int b = blockIdx.z;
  const int co0 = blockIdx.y * COB;
  const int t = blockIdx.x * kThreads + threadIdx.x;
  const bool valid = t < p.Lout;
  Stage stg;
  stg.fetch(w, co0, bias, nullptr, nullptr, 0.f, 0.f, 0.f);
  float xv[CK];
  load_window<CK, REFLECT>(p, x + (int64_t)b * p.Cin * p.Lin, t, valid, xv);
  stg.put(wt);
  __syncthreads();
  ShiftedStats st;
  float acc[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = wt[CK * COB + j];
  window_dot<CK, COB>(xv, wt, acc);
  if (valid) {
    if (partials) {
#pragma unroll
      for (int j = 0; j < COB; ++j) st.add(acc[j]);
    }
    if (y) {
      // one unrolled store loop per activation code, so no loop carries every code's registers
      const float* rb = p.res ? p.res + ((int64_t)b * p.Cout + co0) * p.ldr + t : nullptr;
      float* yb = y + ((int64_t)b * p.Cout + co0) * p.ldy + t;
      auto store = [&](auto code) {
        float rv[COB];
#pragma unroll
        for (int j = 0; j < COB; ++j) rv[j] = rb ? rb[(int64_t)j * p.ldr] : 0.f;
#pragma unroll
        for (int j = 0; j < COB; ++j)
          yb[(int64_t)j * p.ldy] = apply_act(acc[j], code.value, p.alpha) + rv[j];
      };
      switch (act) {
        case 1: store(std::integral_constant<int, 1>{}); break;
        case 2: store(std::integral_constant<int, 2>{}); break;
        case 3: store(std::integral_constant<int, 3>{}); break;
        case 4: store(std::integral_constant<int, 4>{}); break;
        case 5: store(std::integral_constant<int, 5>{}); break;
        case 6: store(std::integral_constant<int, 6>{}); break;
        default: store(std::integral_constant<int, 0>{}); break;
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

// (count, mean, M2) of one thread's COB values, two passes in registers; zero when the thread's
// position is past the output
template <int COB>
__device__ __forceinline__ void thread_stats(const float (&acc)[COB], bool valid, float& n,
                                             float& mean, float& m2) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < COB; ++j) s += acc[j];
  mean = s * (1.f / COB);
  m2 = 0.f;
#pragma unroll
  for (int j = 0; j < COB; ++j) m2 = fmaf(acc[j] - mean, acc[j] - mean, m2);
  n = valid ? (float)COB : 0.f;
  if (!valid) mean = m2 = 0.f;
}

// Pass 1: GroupNorm(1) statistics of conv(x) + bias, one (count, mean, M2) partial per workgroup
// at parts[(b * nparts + blockIdx.y * gridDim.x + blockIdx.x) * 3]; nothing else is written.
template <int CK, int COB, bool REFLECT>
__global__ __launch_bounds__(kThreads) void conv_gn_stats_kernel(ConvParams p,
                                                                 const float* __restrict__ x,
                                                                 const float* __restrict__ w,
                                                                 const float* __restrict__ bias,
                                                                 float* __restrict__ parts) {
  __shared__ float red[3 * (kThreads / 64)];
  using Stage = ConstStage<CK, COB, 1>;
  __shared__ __attribute__((aligned(16))) float wt[Stage::N];  // weights, bias
  const int b = blockIdx.z, cob0 = blockIdx.y * COB;
  const int t = blockIdx.x * kThreads + threadIdx.x;
  const bool valid = t < p.Lout;
  Stage st;
  st.fetch(w, cob0, bias, nullptr, nullptr, 0.f, 0.f, 0.f);
  float xv[CK];
  load_window<CK, REFLECT>(p, x + (int64_t)b * p.Cin * p.Lin, t, valid, xv);
  st.put(wt);
  __syncthreads();
  float acc[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = wt[CK * COB + j];
  window_dot<CK, COB>(xv, wt, acc);
  float n, mean, m2;
  thread_stats<COB>(acc, valid, n, mean, m2);
  block_welford(n, mean, m2, red);
  if (threadIdx.x == 0) {
    float* o = parts + ((int64_t)b * gridDim.x * gridDim.y + blockIdx.y * gridDim.x + blockIdx.x) * 3;
    o[0] = n;
    o[1] = mean;
    o[2] = m2;
  }
}

// Pass 2: y = act(gamma_c * (conv(x)_c + bias_c - mean) * rstd + beta_c). The window loads are
// issued first; every workgroup merges the nparts partials of its batch (fp64, the same order in
// every workgroup) while they are in flight. ACT >= 0 is a fixed activation code, -1 reads `act`.
template <int CK, int COB, bool REFLECT, int ACT>
__global__ __launch_bounds__(kThreads) void conv_gn_apply_kernel(
    ConvParams p, const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ bias, const float* __restrict__ parts, int nparts,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps, int act,
    float* __restrict__ y) {
  using Stage = ConstStage<CK, COB, 3>;
  __shared__ __attribute__((aligned(16))) float wt[Stage::N];  // weights, bias, gamma, beta
  const int b = blockIdx.z, cob0 = blockIdx.y * COB;
  const int t = blockIdx.x * kThreads + threadIdx.x;
  const bool valid = t < p.Lout;
  __shared__ double s_sums[4 * (kThreads / 64)];
  const float* pb = parts + (int64_t)b * nparts * 3;
  // every load is issued before any is waited for: the partials (each read once per workgroup),
  // the workgroup's constants, the input window
  BlockParts<2> pts;
  pts.load(pb, nparts);
  Stage st;
  st.fetch(w, cob0, bias, gamma, beta, 0.f, 1.f, 0.f);
  float xv[CK];
  load_window<CK, REFLECT>(p, x + (int64_t)b * p.Cin * p.Lin, t, valid, xv);
  st.put(wt);
  pts.reduce_waves(pb, nparts, s_sums);
  __syncthreads();
  double n, mean, m2;
  BlockParts<2>::finish(s_sums, n, mean, m2);
  const double var = n > 0.0 ? m2 / n : 0.0;
  float rstd = (float)(1.0 / sqrt(var + (double)eps));
  if (!isfinite(rstd)) rstd = 0.f;
  const float mf = (float)mean;
  float acc[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = 0.f;
  window_dot<CK, COB>(xv, wt, acc);
  if (!valid) return;
  float* yb = y + ((int64_t)b * p.Cout + cob0) * p.ldy + t;
  const float* cb = wt + CK * COB;  // bias, gamma, beta of this workgroup's channels
  auto store = [&](auto code) {
#pragma unroll
    for (int j = 0; j < COB; ++j) {
      const float sc = cb[COB + j] * rstd;  // scale and shift with the bias folded in
      const float sh = cb[2 * COB + j] + (cb[j] - mf) * sc;
      yb[(int64_t)j * p.ldy] = apply_act(fmaf(acc[j], sc, sh), code.value, p.alpha);
    }
  };
  if constexpr (ACT >= 0) {
    store(std::integral_constant<int, ACT>{});
  } else {  // one unrolled store loop per code, so no loop carries every activation's registers
    switch (act) {
      case 1: store(std::integral_constant<int, 1>{}); break;
      case 2: store(std::integral_constant<int, 2>{}); break;
      case 3: store(std::integral_constant<int, 3>{}); break;
      case 4: store(std::integral_constant<int, 4>{}); break;
      case 5: store(std::integral_constant<int, 5>{}); break;
      case 6: store(std::integral_constant<int, 6>{}); break;
      default: store(std::integral_constant<int, 0>{}); break;
    }
  }
}

// Both passes in one launch. Each workgroup computes a tile of COB channels x 256 positions of
// the convolution into registers (SPLIT x 256 threads, COB / SPLIT channels each) and publishes
// the tile's statistics partial; it then collects every partial of its batch (each workgroup
// polls them all: at this grid size that is fewer round trips than waiting for one merger),
// merges them and writes the normalised output from the registers it kept. The words carry the
// batch's epoch tag (device_utils.hpp, exchange with one merger), so nothing is cleared and no
// workgroup counts out (one read-modify-write per workgroup on one word serialised at the end of
// the kernel); workgroup 0 of the batch waits without bound and, having seen every partial,
// advances the epoch. The others' waits are bounded: a workgroup whose wait runs out computes
// every partial of its batch itself (the same code on the same inputs as their owners, so the
// same bits), so each workgroup ends with the same result whatever the scheduling.
constexpr int kOneMaxParts = 1024;  // partials per batch (LDS: 8 bytes each)
constexpr int kOneMaxSlots = 4096;  // partials over all batches

// (mean, M2) of one tile of n values spread over NW waves, two passes over the registers: the
// mean from a block sum, then M2 about it. Every thread returns the same bits. red: 2 * NW floats
// of LDS; calls in a loop need no barrier between them (each reads its first half before its
// second barrier).
template <int CPT, int NW>
__device__ __forceinline__ void tile_stats(const float (&acc)[CPT], bool valid, float n,
                                           float* red, float& mean, float& m2) {
  const int wid = threadIdx.x >> 6;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CPT; ++j) s += acc[j];
  s = wave_sum_dpp(valid ? s : 0.f);
  if ((threadIdx.x & 63) == 0) red[wid] = s;
  lds_barrier();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < NW; ++k) tot += red[k];
  mean = tot / n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < CPT; ++j) q = fmaf(acc[j] - mean, acc[j] - mean, q);
  q = wave_sum_dpp(valid ? q : 0.f);
  if ((threadIdx.x & 63) == 0) red[NW + wid] = q;
  lds_barrier();
  m2 = 0.f;
#pragma unroll
  for (int k = 0; k < NW; ++k) m2 += red[NW + k];
}

template <int CK, int COB, int SPLIT, bool REFLECT, int ACT>
__global__ __launch_bounds__(kThreads * SPLIT) void conv_gn_oneshot_kernel(
    ConvParams p, const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ bias, unsigned long long* xch, int spin_limit,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps, int act,
    float* __restrict__ y) {
  constexpr int NT = kThreads * SPLIT, NW = NT / 64, CPT = COB / SPLIT;
  static_assert(COB % (4 * SPLIT) == 0, "whole float4 weight groups per thread");
  using Stage = ConstStage<CK, COB, 3, NT>;
  __shared__ __attribute__((aligned(16))) float wt[Stage::N];  // weights, bias, gamma, beta
  __shared__ float red[2 * NW];
  __shared__ float2 sp[kOneMaxParts];  // (mean, M2) of every partial of this batch
  __shared__ unsigned s_tag;
  const int b = blockIdx.z, cob0 = blockIdx.y * COB;
  const int pos = threadIdx.x & (kThreads - 1), part = threadIdx.x / kThreads;  // part: per wave
  const int t = blockIdx.x * kThreads + pos;
  const bool valid = t < p.Lout;
  const int nparts = gridDim.x * gridDim.y;
  const float* xb = x + (int64_t)b * p.Cin * p.Lin;
  if (threadIdx.x == 0) s_tag = xm_tag(xch, b);  // read after the barrier below
  Stage st;
  st.fetch(w, cob0, bias, gamma, beta, 0.f, 1.f, 0.f);
  float xv[CK];
  load_window<CK, REFLECT>(p, xb, t, valid, xv);
  st.put(wt);
  lds_barrier();
  float acc[CPT];
  const int c0 = part * CPT;  // this thread's first channel within the tile
#pragma unroll
  for (int j = 0; j < CPT; ++j) acc[j] = wt[CK * COB + c0 + j];
#pragma unroll
  for (int e = 0; e < CK; ++e)
#pragma unroll
    for (int j4 = 0; j4 < CPT; j4 += 4) {
      const float4 w4 = *reinterpret_cast<const float4*>(wt + e * COB + c0 + j4);
      acc[j4 + 0] = fmaf(xv[e], w4.x, acc[j4 + 0]);
      acc[j4 + 1] = fmaf(xv[e], w4.y, acc[j4 + 1]);
      acc[j4 + 2] = fmaf(xv[e], w4.z, acc[j4 + 2]);
      acc[j4 + 3] = fmaf(xv[e], w4.w, acc[j4 + 3]);
    }
  auto tile_count = [&](int vx) { return (float)(COB * min(kThreads, p.Lout - vx * kThreads)); };
  const unsigned tag = s_tag;
  const bool advancer = blockIdx.x == 0 && blockIdx.y == 0;
  {
    float mean, m2;
    tile_stats<CPT, NW>(acc, valid, tile_count(blockIdx.x), red, mean, m2);
    if (threadIdx.x == 0) xm_put(xch, b, nparts, blockIdx.y * gridDim.x + blockIdx.x, tag, mean, m2);
  }
  // collect: every thread polls its share of the partials until all are published
  const bool late = !xm_collect<NT, (kOneMaxParts + NT - 1) / NT>(xch, b, nparts, tag, sp,
                                                                   advancer ? -1 : spin_limit);
  if (advancer && threadIdx.x == 0) xm_advance(xch, b, tag);
  if (late) {
    // compute every partial of this batch here, each as its owner computes it (weights and bias
    // read from global memory hold the values the owner staged in LDS; the fmaf order over the
    // taps is the same)
    for (int v = 0; v < nparts; ++v) {
      const int vx = v % gridDim.x, vy = v / gridDim.x;
      const int tv = vx * kThreads + pos;
      const int cv = vy * COB + c0;
      float xw[CK], av[CPT];
      load_window<CK, REFLECT>(p, xb, tv, tv < p.Lout, xw);
#pragma unroll
      for (int j = 0; j < CPT; ++j) av[j] = bias ? bias[cv + j] : 0.f;
#pragma unroll
      for (int e = 0; e < CK; ++e)
#pragma unroll
        for (int j = 0; j < CPT; ++j) av[j] = fmaf(xw[e], w[(int64_t)(cv + j) * CK + e], av[j]);
      float mean, m2;
      tile_stats<CPT, NW>(av, tv < p.Lout, tile_count(vx), red, mean, m2);
      if (threadIdx.x == 0) sp[v] = make_float2(mean, m2);
    }
    lds_barrier();
  }
  // merge in a fixed order, in every wave; the total count is Cout x Lout
  const float2 mr = xch_merge(sp, nparts, [&](int v) { return tile_count(v % gridDim.x); },
                              (double)p.Cout * p.Lout, eps);
  const float rstd = mr.y, mf = mr.x;
  if (valid) {
    float* yb = y + ((int64_t)b * p.Cout + cob0 + c0) * p.ldy + t;
    const float* cb = wt + CK * COB + c0;  // bias, gamma, beta of this thread's channels
    auto store = [&](auto code) {
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        // acc holds conv + bias, so the shift is beta - mean * scale
        const float sc = cb[COB + j] * rstd;
        const float sh = cb[2 * COB + j] - mf * sc;
        yb[(int64_t)j * p.ldy] = apply_act(fmaf(acc[j], sc, sh), code.value, p.alpha);
      }
    };
    if constexpr (ACT >= 0) {
      store(std::integral_constant<int, ACT>{});
    } else {
      switch (act) {
        case 1: store(std::integral_constant<int, 1>{}); break;
        case 2: store(std::integral_constant<int, 2>{}); break;
        case 3: store(std::integral_constant<int, 3>{}); break;
        case 4: store(std::integral_constant<int, 4>{}); break;
        case 5: store(std::integral_constant<int, 5>{}); break;
        case 6: store(std::integral_constant<int, 6>{}); break;
        default: store(std::integral_constant<int, 0>{}); break;
      }
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

namespace {
// channels per thread of the two-pass Conv1D -> GroupNorm(1) chain: the statistics pass takes
// twice the apply pass's, halving the partials every apply workgroup merges
constexpr int kGnCob = 8, kGnStatsCob = 16;
}

int conv_gn_num_parts(const ConvParams& p) {
  return (int)cdiv(p.Lout, kThreads) * (p.Cout / kGnStatsCob);
}

void conv_gn_stats(const LaunchCtx& c, const ConvParams& p, const float* x, const float* w,
                   const float* bias, float* parts) {
  const int ck = reg_ck(p);
  MNN_REQUIRE(ck, MNN_ERR_INVALID_ARGUMENT, "conv_gn_stats: not a register-window convolution");
  dim3 grid(cdiv(p.Lout, kThreads), p.Cout / kGnStatsCob, p.B);
#define MNN_ST(CKV, R) launch(c, "conv_gn_stats_f32", conv_gn_stats_kernel<CKV, kGnStatsCob, R>, grid, dim3(kThreads), 0, p, x, w, bias, parts)
  switch (ck * 2 + (p.reflect ? 1 : 0)) {
    case 16: return MNN_ST(8, false);
    case 17: return MNN_ST(8, true);
    case 32: return MNN_ST(16, false);
    case 33: return MNN_ST(16, true);
    case 48: return MNN_ST(24, false);
    case 49: return MNN_ST(24, true);
    case 64: return MNN_ST(32, false);
    default: return MNN_ST(32, true);
  }
#undef MNN_ST
}

void conv_gn_apply(const LaunchCtx& c, const ConvParams& p0, const float* x, const float* w,
                   const float* bias, const float* parts, int nparts, const float* gamma,
                   const float* beta, float eps, int act, float* y) {
  ConvParams p = p0;
  if (p.ldy == 0) p.ldy = p.Lout;
  const int ck = reg_ck(p);
  MNN_REQUIRE(ck, MNN_ERR_INVALID_ARGUMENT, "conv_gn_apply: not a register-window convolution");
  dim3 grid(cdiv(p.Lout, kThreads), p.Cout / kGnCob, p.B);
  const int a = (act == 0 || act == 3) ? act : -1;
#define MNN_AP(CKV, R, A) launch(c, "conv_gn_apply_f32", conv_gn_apply_kernel<CKV, kGnCob, R, A>, grid, dim3(kThreads), 0, p, x, w, bias, parts, nparts, gamma, beta, eps, act, y)
#define MNN_AP3(CKV, R) return a == 0 ? MNN_AP(CKV, R, 0) : a == 3 ? MNN_AP(CKV, R, 3) : MNN_AP(CKV, R, -1)
  switch (ck * 2 + (p.reflect ? 1 : 0)) {
    case 16: MNN_AP3(8, false);
    case 17: MNN_AP3(8, true);
    case 32: MNN_AP3(16, false);
    case 33: MNN_AP3(16, true);
    case 48: MNN_AP3(24, false);
    case 49: MNN_AP3(24, true);
    case 64: MNN_AP3(32, false);
    default: MNN_AP3(32, true);
  }
#undef MNN_AP3
#undef MNN_AP
}

namespace {
constexpr int kOneCob = 16;   // channels per tile of the one-launch chain
constexpr int kOneSplit = 2;  // threads per tile position

template <int CK, bool R, int A>
bool oneshot_dispatch(const LaunchCtx& c, const ConvParams& p, bool go, const float* x,
                      const float* w, const float* bias, unsigned long long* xch, int spin_limit,
                      const float* gamma, const float* beta, float eps, int act, float* y) {
  auto* kern = conv_gn_oneshot_kernel<CK, kOneCob, kOneSplit, R, A>;
  // workgroups of this kernel one CU holds at once (the same for every gfx950 device)
  static const int per_cu = [&] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kThreads * kOneSplit, 0) !=
        hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    return n;
  }();
  const dim3 grid(cdiv(p.Lout, kThreads), p.Cout / kOneCob, p.B);
  const int64_t nparts = (int64_t)grid.x * grid.y, blocks = nparts * grid.z;
  if (nparts > kOneMaxParts || blocks > kOneMaxSlots || grid.z > (unsigned)kXmMaxBatch ||
      blocks > (int64_t)per_cu * c.dev->props.multiProcessorCount)
    return false;
  if (go)
    launch(c, "conv_gn_oneshot_f32", kern, grid, dim3(kThreads * kOneSplit), 0, p, x, w, bias, xch,
           spin_limit, gamma, beta, eps, act, y);
  return true;
}

bool oneshot(const LaunchCtx& c, const ConvParams& p0, bool go, const float* x, const float* w,
             const float* bias, unsigned long long* xch, int spin_limit, const float* gamma,
             const float* beta, float eps, int act, float* y) {
  ConvParams p = p0;
  if (p.ldy == 0) p.ldy = p.Lout;
  const int ck = reg_ck(p);
  if (!ck || p.Cout % kOneCob != 0) return false;
  const int a = (act == 0 || act == 3) ? act : -1;
#define MNN_OS(CKV, R, A) oneshot_dispatch<CKV, R, A>(c, p, go, x, w, bias, xch, spin_limit, gamma, beta, eps, act, y)
#define MNN_OS3(CKV, R) return a == 0 ? MNN_OS(CKV, R, 0) : a == 3 ? MNN_OS(CKV, R, 3) : MNN_OS(CKV, R, -1)
  switch (ck * 2 + (p.reflect ? 1 : 0)) {
    case 16: MNN_OS3(8, false);
    case 17: MNN_OS3(8, true);
    case 32: MNN_OS3(16, false);
    case 33: MNN_OS3(16, true);
    case 48: MNN_OS3(24, false);
    case 49: MNN_OS3(24, true);
    case 64: MNN_OS3(32, false);
    default: MNN_OS3(32, true);
  }
#undef MNN_OS3
#undef MNN_OS
}
}  // namespace

size_t conv_gn_oneshot_exchange_bytes() {
  return 8 * (4 * (size_t)kXmMaxBatch + 2 * (size_t)kOneMaxSlots);
}

bool conv_gn_oneshot_fits(const LaunchCtx& c, const ConvParams& p) {
  // tuning override: MNN_CONV_GN_ONESHOT=0 takes the two-pass form wherever it applies
  static const bool off = [] {
    const char* e = std::getenv("MNN_CONV_GN_ONESHOT");
    return e && std::atoi(e) == 0;
  }();
  return !off && oneshot(c, p, false, nullptr, nullptr, nullptr, nullptr, 0, nullptr, nullptr,
                         0.f, 0, nullptr);
}

void conv_gn_oneshot(const LaunchCtx& c, const ConvParams& p, const float* x, const float* w,
                     const float* bias, void* xch, int spin_limit, const float* gamma,
                     const float* beta, float eps, int act, float* y) {
  MNN_REQUIRE(oneshot(c, p, true, x, w, bias, static_cast<unsigned long long*>(xch),
                      std::max(spin_limit, 0), gamma, beta, eps, act, y),
              MNN_ERR_INVALID_ARGUMENT,
              "conv_gn_oneshot: not a register-window convolution, or the grid does not fit the "
              "device at once");
}

}  // namespace k
}  // namespace mnn
