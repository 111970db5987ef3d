// Transposed 1-D convolution (DynamicConvTranspose1D, DynamicConv1D.swift:411-645) and the channel
// concat of UNetDecoderBlock (UNet.swift:262-280, concatenateChannels :303-331).
//
// Reference semantics (dynamic_conv_transpose1d_forward, DynamicConv1D.swift:588-640):
//   y[oc][o] = bias[oc] + sum_ic sum_k x[ic][i] * W[ic][oc_g][k],  i = (o + pad - k*dil) / stride
// over the (ic, k) for which the division is exact and 0 <= i < L; W is [Cin][Cout/groups][K].
//
// Matrix-core form (groups 1, dilation 1, K = T * stride): with o + pad = stride*q + r
// (0 <= r < stride) the taps that reach o are k = r + stride*t at input i = q - t, t < T, so
//   y[oc][stride*q + r - pad] = bias[oc] + sum_t sum_ic x[ic][q - t] * W[ic][oc][r + stride*t].
// That is a GEMM over K' = T * Cp (Cp = Cin rounded up to 32, padded channels zero):
//   rows m = stride*oc + r, A[m][(t, ic)] = W[ic][oc][r + stride*t]   (weights, packed at load)
//   columns q, B[q][(t, ic)] = x[ic][q - t] (zero outside [0, L))      (convt_pack_kernel)
// on the LDS-DMA GEMM with its transposed-conv epilogue, which scatters row m, column q to
// y[oc][stride*q + r - pad] (+bias). The pack kernel reads the input rows once and writes their
// unfolded transpose (T times the input), concatenating the decoder's skip on the way.
#include <algorithm>

#include "device_utils.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

// output rows q per pack tile: on the time decoder's levels (264-1011 tiles of 64 rows) 32 rows
// took 24 us against 34 (64) and 26 (16): more, shorter workgroups keep more loads in flight
constexpr int kPQ = 32;
constexpr int kPC = 64;   // channels per pack tile

// One tile: channels [c0, c0 + 64) x rows q in [q0, q0 + kPQ). The input window of a channel is
// positions q0 - (T - 1) .. q0 + kPQ - 1, staged in LDS: every thread issues all its window loads
// (clamped addresses, out-of-range values zeroed by a select, no load under a branch) before its
// first LDS store. The unfolded rows are written 16 bytes per thread along the channel dimension.
// The LDS tile is position-major with an odd pitch (65 channels): the stores (consecutive
// positions of a channel) and the reads (4 channels of a position, consecutive lanes 4 channels
// apart, the next position every 16 lanes) fall on distinct banks (a channel-major tile gave 6.4
// conflict cycles per LDS instruction).
template <int T>
__global__ __launch_bounds__(256) void convt_pack_kernel(ConvTPackArgs a) {
  constexpr int W = kPQ + T - 1;  // window positions per channel
  constexpr int CPITCH = kPC + 1;
  constexpr int NE = (kPC * W + 255) / 256;  // window elements per thread
  __shared__ float tile[W * CPITCH];
  const int b = blockIdx.z;
  const int64_t q0 = (int64_t)blockIdx.x * kPQ;
  const int c0 = blockIdx.y * kPC;
  const int tid = threadIdx.x;
  const int Cin = a.C1 + a.C2;
  const int64_t L = a.L;
  const float* x1 = a.x1 + (int64_t)b * a.C1 * L;
  const float* x2 = a.x2 ? a.x2 + (int64_t)b * a.C2 * L : x1;
  float v[NE];
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int e = tid + 256 * k, i = e / W, jj = e % W;
    const int c = c0 + i;
    const int64_t p = q0 - (T - 1) + jj;
    const bool ok = e < kPC * W && c < Cin && p >= 0 && p < L;
    const int cc = min(c, Cin - 1);
    const int64_t pp = min(max(p, (int64_t)0), L - 1);
    const float* src = cc < a.C1 ? x1 + (int64_t)cc * L : x2 + (int64_t)(cc - a.C1) * L;
    const float val = src[pp];
    v[k] = ok ? val : 0.f;
  }
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int e = tid + 256 * k;
    if (e < kPC * W) tile[(e % W) * CPITCH + e / W] = v[k];
  }
  __syncthreads();
  const int kp = T * a.Cp;
  float* __restrict__ ub = a.u + (int64_t)b * a.Lq * kp;
  for (int e = tid; e < T * kPQ * (kPC / 4); e += 256) {
    const int c4 = e % (kPC / 4), qq = (e / (kPC / 4)) % kPQ, t = e / ((kPC / 4) * kPQ);
    const int64_t q = q0 + qq;
    const int c = c0 + 4 * c4;
    if (q >= a.Lq || c >= a.Cp) continue;
    const int col = qq + (T - 1) - t;
    const float* tr = tile + col * CPITCH + 4 * c4;
    const float4 v = make_float4(tr[0], tr[1], tr[2], tr[3]);
    *reinterpret_cast<float4*>(ub + q * kp + t * a.Cp + c) = v;
  }
}

// Direct form for every other configuration (groups, dilation, K not a multiple of the stride):
// one thread per output, the reference's gather loop (ic, then k; bias last).
__global__ __launch_bounds__(256) void convt_direct_kernel(ConvTArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_b = (int64_t)a.Cout * a.Lout;
  if (idx >= per_b * a.B) return;
  const int b = (int)(idx / per_b);
  const int oc = (int)((idx % per_b) / a.Lout);
  const int64_t o = idx % a.Lout;
  const int Cin = a.C1 + a.C2;
  const int coutpg = a.Cout / a.groups, cinpg = Cin / a.groups;
  const int g = oc / coutpg, ocg = oc % coutpg;
  float sum = 0.f;
  for (int icg = 0; icg < cinpg; ++icg) {
    const int ic = g * cinpg + icg;
    const float* xr = ic < a.C1 ? a.x1 + ((int64_t)b * a.C1 + ic) * a.L
                                : a.x2 + ((int64_t)b * a.C2 + (ic - a.C1)) * a.L;
    for (int k = 0; k < a.K; ++k) {
      const int64_t num = o + a.pad - (int64_t)k * a.dil;
      if (num >= 0 && num % a.stride == 0) {
        const int64_t i = num / a.stride;
        if (i < a.L) sum = fmaf(xr[i], a.w[((int64_t)ic * coutpg + ocg) * a.K + k], sum);
      }
    }
  }
  if (a.bias) sum += a.bias[oc];
  a.y[idx] = sum;
}

// Few output channels (stride * Cout < 32, e.g. the decoder's last, 2-channel level): a 64-row
// matrix-core tile would be mostly padding, so each lane computes all Cout * S outputs of one
// column q in registers, reading its T input samples x[c][q - t] straight from global memory
// (consecutive lanes read consecutive samples; no unfold). A workgroup covers 64 columns; its
// four waves split the input channels and add their accumulators through LDS in wave order at
// the end (more waves in flight than one wave per 64 columns would give). The channel row is the
// same for every lane, and all the weights are staged in LDS once and read at wave-uniform
// addresses (broadcasts). A wave's channels go in batches of CB, the next batch's loads issued
// before the current batch is used.
constexpr int kSmallWaves = 4, kSmallWMax = 12288;  // at most 48 KB of weights staged in LDS
template <int COUT, int S, int T>
__global__ __launch_bounds__(64 * kSmallWaves) void convt_small_kernel(ConvTArgs a) {
  constexpr int CB = 4;              // channels per load batch (13.2 us at 4, 14.1 at 8)
  constexpr int CST = COUT * S * T;  // weights per input channel, W[c][oc][r + S*t]
  extern __shared__ __attribute__((aligned(16))) float wl[];  // Cin * CST floats (dynamic)
  __shared__ float part[kSmallWaves - 1][COUT * S][64];
  // XCD-aware numbering: consecutive column blocks (which share a one-sample halo) on one XCD
  const int unit = xcd_logical_tile(blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
  const int bx = unit % gridDim.x, b = unit / gridDim.x, lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int64_t q = (int64_t)bx * 64 + lane;
  const int Cin = a.C1 + a.C2;
  const int64_t L = a.L;
  const float* x1 = a.x1 + (int64_t)b * a.C1 * L;
  const float* x2 = a.x2 ? a.x2 + (int64_t)b * a.C2 * L : x1;
  // this wave's channels: [cb, ce), whole batches except at the end of the range
  const int per = (Cin + kSmallWaves * CB - 1) / (kSmallWaves * CB) * CB;
  const int cb = min(wave * per, Cin), ce = min(cb + per, Cin);
  // tap t of column q is sample q - t (zero outside the signal): clamped address, zeroed value
  int64_t pos[T];
  float keep[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int64_t p = q - t;
    keep[t] = (p >= 0 && p < L) ? 1.f : 0.f;
    pos[t] = min(max(p, (int64_t)0), L - 1);
  }
  auto load_batch = [&](int c0, float (&xv)[CB][T]) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int c = min(c0 + j, Cin - 1);
      const float* row = c < a.C1 ? x1 + (int64_t)c * L : x2 + (int64_t)(c - a.C1) * L;
#pragma unroll
      for (int t = 0; t < T; ++t) xv[j][t] = row[pos[t]];
    }
  };
  float xv[CB][T];
  load_batch(cb, xv);
  for (int e = threadIdx.x; e < Cin * CST; e += 64 * kSmallWaves) wl[e] = a.w[e];
  __syncthreads();
  float acc[COUT][S];
#pragma unroll
  for (int oc = 0; oc < COUT; ++oc)
#pragma unroll
    for (int r = 0; r < S; ++r) acc[oc][r] = 0.f;
  for (int c0 = cb; c0 < ce; c0 += CB) {
    float xn[CB][T];
    load_batch(min(c0 + CB, ce - 1), xn);  // after the last batch: reloaded, unused
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      if (c0 + j < ce) {  // uniform
        const float* wc = wl + (c0 + j) * CST;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const float xt = xv[j][t] * keep[t];
#pragma unroll
          for (int oc = 0; oc < COUT; ++oc)
#pragma unroll
            for (int r = 0; r < S; ++r)
              acc[oc][r] = fmaf(xt, wc[oc * (S * T) + r + S * t], acc[oc][r]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int t = 0; t < T; ++t) xv[j][t] = xn[j][t];
  }
  if (wave > 0) {
#pragma unroll
    for (int oc = 0; oc < COUT; ++oc)
#pragma unroll
      for (int r = 0; r < S; ++r) part[wave - 1][oc * S + r][lane] = acc[oc][r];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kSmallWaves - 1; ++w)
#pragma unroll
    for (int oc = 0; oc < COUT; ++oc)
#pragma unroll
      for (int r = 0; r < S; ++r) acc[oc][r] += part[w][oc * S + r][lane];
  float* yb = a.y + (int64_t)b * a.Cout * a.Lout;
#pragma unroll
  for (int oc = 0; oc < COUT; ++oc) {
    const float bv = a.bias ? a.bias[oc] : 0.f;
#pragma unroll
    for (int r = 0; r < S; ++r) {
      const int64_t o = S * q + r - a.pad;
      if (o >= 0 && o < a.Lout) yb[(int64_t)oc * a.Lout + o] = acc[oc][r] + bv;
    }
  }
}

// Sum of the K parts of the GEMM form, then the scatter of convt's epilogue:
// y[b][oc][s*q + r - pad] = bias[oc] + sum_p ws[b][p][s*oc + r][q]. One thread per column q of one
// output channel: it reads the s phase rows (coalesced over q) and writes s consecutive samples.
// With stats, each workgroup writes the GroupNorm partial (count, mean, M2) of the samples it
// stored for the group of its channel (G groups of Cout / G channels): at
// stats[((b * G + g) * parts + j) * 3], parts = (Cout / G) * gridDim.x, j = (oc mod (Cout / G)) *
// gridDim.x + blockIdx.x.
__global__ __launch_bounds__(256) void convt_reduce_kernel(const float* __restrict__ ws, int ksplit,
                                                           int M, int64_t N, int stride, int pad,
                                                           const float* __restrict__ bias,
                                                           float* __restrict__ y, int64_t Lout,
                                                           int Cout, float* __restrict__ stats,
                                                           int G) {
  __shared__ float red[3 * 4];
  const int oc = blockIdx.y, b = blockIdx.z;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  ShiftedStats st;
  if (q < N) {
    const float* wb = ws + (int64_t)b * ksplit * M * N + (int64_t)stride * oc * N + q;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < ksplit; ++p)
      for (int r = 0; r < stride && r < 4; ++r) v[r] += wb[(int64_t)p * M * N + (int64_t)r * N];
    const float bv = bias ? bias[oc] : 0.f;
    float* yr = y + ((int64_t)b * Cout + oc) * Lout;
    for (int r = 0; r < stride && r < 4; ++r) {
      const int64_t o = stride * q + r - pad;
      if (o >= 0 && o < Lout) {
        yr[o] = v[r] + bv;
        st.add(v[r] + bv);
      }
    }
  }
  if (stats) {  // uniform over the grid
    float sn, smean, sm2;
    st.finish(sn, smean, sm2);
    block_welford(sn, smean, sm2, red);
    if (threadIdx.x == 0) {
      const int cpg = Cout / G, gi = oc / cpg;
      const int64_t parts = (int64_t)cpg * gridDim.x, j = (int64_t)(oc - gi * cpg) * gridDim.x + blockIdx.x;
      float* o = stats + (((int64_t)b * G + gi) * parts + j) * 3;
      o[0] = sn;
      o[1] = smean;
      o[2] = sm2;
    }
  }
}

// K split of the GEMM form, for grids of at most ~1.5 64 x 64 tiles per CU: the most parts
// (dividing the stage count, at least 6 stages each) that keep the grid within about four tiles
// per CU. The deepest decoder level has few output columns and a long contraction; without a
// split a CU runs one long tile alone. Larger grids lose more to the reduce pass than they gain
// (measured on the decoder levels).
int convt_ksplit(int B, int Cin, int Cout, int K, int stride, int pad, int64_t Lout) {
  if (stride > 4) return 1;
  const int64_t M = (int64_t)stride * Cout, N = convt_rows(Lout, stride, pad);
  const int nk = (K / stride) * convt_padded_cin(Cin) / 32;
  const int64_t tiles = cdiv(M, 64) * (int64_t)cdiv(N, 64) * B;
  int best = 1;
  if (tiles > 384) return best;
  for (int p : {2, 3, 4, 6, 8})
    if (nk % p == 0 && nk / p >= 6 && tiles * p <= 1024) best = p;
  return best;
}

}  // namespace

int64_t convt_split_ws_floats(int B, int Cin, int Cout, int K, int stride, int pad, int64_t Lout) {
  const int p = convt_ksplit(B, Cin, Cout, K, stride, pad, Lout);
  return p > 1 ? (int64_t)B * p * stride * Cout * convt_rows(Lout, stride, pad) : 0;
}

bool convt_small_supported(int Cin, int Cout, int K, int stride, int dil, int groups) {
  return groups == 1 && dil == 1 && stride == 4 && K == 8 && Cin > 0 &&
         (Cout == 1 || Cout == 2 || Cout == 4) && (int64_t)Cin * Cout * K <= kSmallWMax;
}

void convt_small(const LaunchCtx& c, const ConvTArgs& a) {
  MNN_REQUIRE(convt_small_supported(a.C1 + a.C2, a.Cout, a.K, a.stride, a.dil, a.groups) &&
                  a.x1 && (a.C2 == 0 || a.x2) && a.w && a.y && a.L > 0 && a.Lout > 0 &&
                  // the workgroup numbering (column blocks x batch) is a 32-bit int
                  cdiv(convt_rows(a.Lout, a.stride, a.pad), 64) * a.B < ((int64_t)1 << 31),
              MNN_ERR_INVALID_ARGUMENT, "convt_small: configuration outside the kernel's form");
  const dim3 grid((unsigned)cdiv(convt_rows(a.Lout, a.stride, a.pad), 64), (unsigned)a.B),
      block(64 * kSmallWaves);
  const size_t lds = sizeof(float) * (size_t)(a.C1 + a.C2) * a.Cout * a.K;  // the staged weights
  switch (a.Cout) {
    case 1: return launch(c, "convt_small_f32", convt_small_kernel<1, 4, 2>, grid, block, lds, a);
    case 2: return launch(c, "convt_small_f32", convt_small_kernel<2, 4, 2>, grid, block, lds, a);
    default: return launch(c, "convt_small_f32", convt_small_kernel<4, 4, 2>, grid, block, lds, a);
  }
}

bool convt_gemm_supported(int Cin, int Cout, int K, int stride, int dil, int groups) {
  return groups == 1 && dil == 1 && stride >= 1 && K % stride == 0 && (K / stride == 1 ||
         K / stride == 2 || K / stride == 4) && Cin > 0 && Cout > 0;
}

int convt_padded_cin(int Cin) { return (Cin + 31) / 32 * 32; }

int64_t convt_rows(int64_t Lout, int stride, int pad) { return (Lout - 1 + pad) / stride + 1; }

void convt_pack_weights(const float* w, int Cin, int Cout, int K, int stride, float* out) {
  const int T = K / stride, Cp = convt_padded_cin(Cin), kp = T * Cp;
  for (int64_t i = 0; i < (int64_t)stride * Cout * kp; ++i) out[i] = 0.f;
  for (int oc = 0; oc < Cout; ++oc)
    for (int r = 0; r < stride; ++r)
      for (int t = 0; t < T; ++t)
        for (int ic = 0; ic < Cin; ++ic)
          out[((int64_t)stride * oc + r) * kp + t * Cp + ic] =
              w[((int64_t)ic * Cout + oc) * K + r + stride * t];
}

namespace {
// The GEMM of the transposed conv: rows (oc, phase), columns q, K = T * Cp over the unfolded input.
GemmArgs convt_gemm_args(const ConvTArgs& a, const float* wpack, const float* unfold,
                         float* split_ws) {
  const int Cin = a.C1 + a.C2;
  const int T = a.K / a.stride, Cp = convt_padded_cin(Cin);
  const int64_t Lq = convt_rows(a.Lout, a.stride, a.pad);
  GemmArgs g;
  g.M = a.stride * a.Cout;
  g.N = (int)Lq;
  g.K = T * Cp;
  g.batch = a.B;
  g.A = wpack;
  g.lda = g.K;
  g.sA = 0;
  g.B = unfold;
  g.ldb = g.K;
  g.sB = Lq * g.K;
  g.blayout = B_NK;
  g.C = a.y;
  g.ldc = a.Lout;
  g.sC = (int64_t)a.Cout * a.Lout;
  g.bias = a.bias;
  g.bias_mode = a.bias ? BIAS_M : BIAS_NONE;
  g.ct_stride = a.stride;
  g.ct_pad = a.pad;
  g.ct_len = a.Lout;
  g.stats = a.stats;
  g.name = "convt_f32_mfma";
  const int parts = convt_ksplit(a.B, Cin, a.Cout, a.K, a.stride, a.pad, a.Lout);
  if (parts > 1) {
    g.ksplit = parts;
    g.ws = split_ws;
    g.ct_stride = 0;  // partial products only; the reduce applies bias and scatter
    g.bias = nullptr;
    g.bias_mode = BIAS_NONE;
    g.stats = nullptr;  // the reduce writes the statistics
  }
  return g;
}
}  // namespace

int convt_stats_parts(const ConvTArgs& a) {
  const int Cin = a.C1 + a.C2, G = std::max(a.stat_groups, 1);
  if (a.Cout % G != 0 || convt_small_supported(Cin, a.Cout, a.K, a.stride, a.dil, a.groups) ||
      !convt_gemm_supported(Cin, a.Cout, a.K, a.stride, a.dil, a.groups))
    return 0;
  const int64_t Lq = convt_rows(a.Lout, a.stride, a.pad);
  const int parts = convt_ksplit(a.B, Cin, a.Cout, a.K, a.stride, a.pad, a.Lout);
  if (parts > 1) return a.Cout / G * (int)cdiv(Lq, 256);
  if (G > 1) return 0;
  return (int)gemm_nk_lds_tiles(convt_gemm_args(a, nullptr, nullptr, nullptr));
}

void convt_gemm(const LaunchCtx& c, const ConvTArgs& a, const float* wpack, float* unfold,
                float* split_ws) {
  const int Cin = a.C1 + a.C2;
  MNN_REQUIRE(convt_gemm_supported(Cin, a.Cout, a.K, a.stride, a.dil, a.groups) && wpack &&
                  unfold && a.x1 && (a.C2 == 0 || a.x2) && a.y && a.L > 0 && a.Lout > 0,
              MNN_ERR_INVALID_ARGUMENT, "convt_gemm: configuration outside the GEMM form");
  const int T = a.K / a.stride, Cp = convt_padded_cin(Cin);
  ConvTPackArgs p;
  p.x1 = a.x1;
  p.x2 = a.C2 ? a.x2 : nullptr;
  p.C1 = a.C1;
  p.C2 = a.C2;
  p.L = a.L;
  p.Cp = Cp;
  p.Lq = convt_rows(a.Lout, a.stride, a.pad);
  p.u = unfold;
  const dim3 grid((unsigned)cdiv(p.Lq, kPQ), (unsigned)cdiv(Cp, kPC), (unsigned)a.B);
  switch (T) {
    case 1: launch(c, "convt_pack_f32", convt_pack_kernel<1>, grid, dim3(256), 0, p); break;
    case 2: launch(c, "convt_pack_f32", convt_pack_kernel<2>, grid, dim3(256), 0, p); break;
    default: launch(c, "convt_pack_f32", convt_pack_kernel<4>, grid, dim3(256), 0, p); break;
  }
  const GemmArgs g = convt_gemm_args(a, wpack, unfold, split_ws);
  const int parts = g.ksplit;
  MNN_REQUIRE(parts == 1 || split_ws, MNN_ERR_INVALID_ARGUMENT,
              "convt_gemm: the K split needs a workspace");
  MNN_REQUIRE(gemm_nk_lds_supported(g), MNN_ERR_INVALID_ARGUMENT,
              "convt_gemm: operands outside the LDS GEMM contract");
  gemm_nk_lds(c, g);
  if (parts > 1)
    launch(c, "convt_reduce_f32", convt_reduce_kernel,
           dim3((unsigned)cdiv(p.Lq, 256), (unsigned)a.Cout, (unsigned)a.B), dim3(256), 0,
           (const float*)split_ws, parts, g.M, (int64_t)g.N, a.stride, a.pad, a.bias, a.y,
           a.Lout, a.Cout, a.stats, std::max(a.stat_groups, 1));
}

void convt_pack_t1(const LaunchCtx& c, const ConvTPackArgs& p, int B) {
  MNN_REQUIRE(p.x1 && (p.C2 == 0 || p.x2) && p.u && p.Cp % 4 == 0 && p.Cp >= p.C1 + p.C2 &&
                  p.Lq == p.L && p.L > 0 && B > 0 && B <= 65535,
              MNN_ERR_INVALID_ARGUMENT, "convt_pack_t1: invalid arguments");
  const dim3 grid((unsigned)cdiv(p.Lq, kPQ), (unsigned)cdiv(p.Cp, kPC), (unsigned)B);
  launch(c, "convt_pack_f32", convt_pack_kernel<1>, grid, dim3(256), 0, p);
}

int64_t convt_unfold_floats(int B, int Cin, int K, int stride, int pad, int64_t Lout) {
  return (int64_t)B * convt_rows(Lout, stride, pad) * (K / stride) * convt_padded_cin(Cin);
}

void convt_direct(const LaunchCtx& c, const ConvTArgs& a) {
  const int Cin = a.C1 + a.C2;
  MNN_REQUIRE(a.groups > 0 && Cin % a.groups == 0 && a.Cout % a.groups == 0 && a.stride > 0 &&
                  a.dil > 0 && a.K > 0 && a.x1 && (a.C2 == 0 || a.x2) && a.w && a.y,
              MNN_ERR_INVALID_ARGUMENT, "convt_direct: invalid configuration");
  const int64_t n = (int64_t)a.B * a.Cout * a.Lout;
  if (n == 0) return;
  launch(c, "convt_direct_f32", convt_direct_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
         a);
}

}  // namespace k
}  // namespace mnn
