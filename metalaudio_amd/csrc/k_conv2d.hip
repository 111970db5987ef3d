// 2-D convolution and transposed convolution of the frequency branch (DynamicConv2D and
// DynamicConvTranspose2D, DynamicConv2D.swift:37-959). Layout [B][C][H][W], fp32.
//
// Conv2D (dynamic_conv2d_forward, DynamicConv2D.swift:525-590):
//   y[oc][oh][ow] = bias[oc] + sum_{icg, kh, kw} x[ic][ih][iw] * w[oc][icg][kh][kw],
//   ih = oh*sh - ph + kh*dh, iw = ow*sw - pw + kw*dw, ic = group(oc)*Cin/G + icg,
// zero outside the input; with reflect padding the input is first padded by (ph, pw) with
// mirrored samples (applyReflectPadding2D, :424-475: i < 0 -> -i, i >= n -> 2n - i - 2, then
// clamped to [0, n)) and the conv runs unpadded on the padded input.
// Matrix-core form (groups 1): per batch a GEMM Y[oc][(oh, ow)] = W[oc][k] * U[(oh, ow)][k] over
// k = (icg, kh, kw) (rounded up to 32 with zero columns): conv2d_unfold_kernel writes U (the
// padding resolved there) and the LDS-DMA GEMM adds the bias per row. 1x1 stride-1 unpadded
// convs skip the unfold: the input [C][H*W] is the GEMM's [K][N] operand as it is.
//
// ConvTranspose2D (dynamic_conv_transpose2d_forward, :890-955): W is [Cin][Cout/G][KH][KW],
//   y[oc][oh][ow] = bias[oc] + sum x[ic][ih][iw] * W[ic][ocg][kh][kw] over the (ic, kh, kw) with
//   oh + ph - kh*dh = ih*sh and ow + pw - kw*dw = iw*sw exactly, 0 <= ih < H, 0 <= iw < W.
// Matrix-core form (groups 1): Z[(oc, kh, kw)][(ih, iw)] = sum_ic W[ic][oc][kh][kw] x[ic][ih][iw]
// is a GEMM on the LDS-DMA path: the input (with the decoder's skip, the concat folded in) is
// packed transposed to [H*W][Cp] by the 1-D transposed conv's pack kernel, then
// convt2d_gather_kernel sums the taps that land on each output
// (KH*KW / (sh*sw) of them on average) and adds the bias. No atomics; fixed summation order.
#include <cstdlib>

#include "device_utils.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

__device__ __forceinline__ int reflect_index(int i, int n) {
  if (i < 0) i = -i;
  if (i >= n) i = 2 * n - i - 2;
  return min(max(i, 0), n - 1);
}

// Input sample for padded-frame coordinates (r, s) relative to the unpadded origin: zero padding
// reads zero outside, reflect padding mirrors (r, s already shifted by -pad).
__device__ __forceinline__ float conv2d_sample(const float* xc, int r, int s, int H, int W,
                                               bool reflect) {
  if (reflect) return xc[(int64_t)reflect_index(r, H) * W + reflect_index(s, W)];
  if (r < 0 || r >= H || s < 0 || s >= W) return 0.f;
  return xc[(int64_t)r * W + s];
}

// U[b][n][k] for n = oh*Wo + ow, k = (ic, kh, kw) < K, zero for K <= k < Kp; four k per thread
// (one 16-byte store).
// Index math is 32-bit (the host checks N * Kp / 4 < 2^31). KH_/KW_ > 0 fix the kernel size at
// compile time (the divisions by it become multiplications); 0 reads it from the arguments.
template <int KH_, int KW_>
__global__ __launch_bounds__(256) void conv2d_unfold_kernel(Conv2DArgs a) {
  const unsigned N = (unsigned)a.Ho * (unsigned)a.Wo;
  const unsigned kq = (unsigned)a.Kp / 4;
  const unsigned e = blockIdx.x * 256u + threadIdx.x;
  if (e >= N * kq) return;
  const int b = blockIdx.y;
  const unsigned n = e / kq;
  const int k0 = (int)(e - n * kq) * 4;
  const int oh = (int)(n / (unsigned)a.Wo), ow = (int)(n - (unsigned)oh * a.Wo);
  const int KW = KW_ > 0 ? KW_ : a.KW;
  const int ks = KH_ > 0 ? KH_ * KW_ : a.KH * a.KW, K = a.Cin * ks;
  const float* xb = a.x + (int64_t)b * a.Cin * a.H * a.W;
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int k = k0 + j;
    v[j] = 0.f;
    if (k < K) {
      const int ic = k / ks, kh = (k % ks) / KW, kw = k % KW;
      v[j] = conv2d_sample(xb + (int64_t)ic * a.H * a.W, oh * a.sh - a.ph + kh * a.dh,
                           ow * a.sw - a.pw + kw * a.dw, a.H, a.W, a.reflect);
    }
  }
  *reinterpret_cast<float4*>(a.u + ((int64_t)b * N + n) * a.Kp + k0) =
      make_float4(v[0], v[1], v[2], v[3]);
}

// Tiled unfold: a workgroup takes 64 consecutive rows n = oh * Wo + ow of U (contiguous in
// memory, across output rows when Wo is small) x 32 k. Lane c takes row n0 + c; each k = (ic,
// kh, kw) is then a gather at input (oh * sh - ph + kh * dh, ow * sw - pw + kw * dw), its
// padding resolved by clamped or mirrored indices and a select, so no load sits under a branch
// and all eight of a thread's loads are in flight together. The tile is transposed through LDS
// (row pitch 33: the column-major writes of a wave hit distinct banks) and written as 64 row
// segments of U of 128 contiguous bytes. Grid (ceil(Ho * Wo / 64), Kp / 32, B). (Numbering the
// workgroups so that consecutive position blocks run on one XCD measured 13 % slower.)
constexpr int kUfRows = 64, kUfK = 32, kUfPitch = kUfK + 1;
__global__ __launch_bounds__(256) void conv2d_unfold_tiled_kernel(Conv2DArgs a) {
  __shared__ float t[kUfRows * kUfPitch];
  const int b = blockIdx.z;
  const int k0 = blockIdx.y * kUfK;
  const int N = a.Ho * a.Wo;
  const int n0 = blockIdx.x * kUfRows;
  const int ks = a.KH * a.KW, K = a.Cin * ks;
  const float* xb = a.x + (int64_t)b * a.Cin * a.H * a.W;
  const int tid = threadIdx.x, c = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: the k math below is too
  const int n = min(n0 + c, N - 1);
  const int oh = n / a.Wo, ow = n - oh * a.Wo;
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = wave + 4 * j;  // wave-uniform k row
    const int k = min(k0 + r, K - 1);
    const int ic = k / ks, rem = k - ic * ks, kh = rem / a.KW, kw = rem - kh * a.KW;
    int ih = oh * a.sh - a.ph + kh * a.dh, iw = ow * a.sw - a.pw + kw * a.dw;
    bool zero = k0 + r >= K;
    if (a.reflect) {
      ih = reflect_index(ih, a.H);
      iw = reflect_index(iw, a.W);
    } else {
      zero = zero || ih < 0 || ih >= a.H || iw < 0 || iw >= a.W;
    }
    ih = min(max(ih, 0), a.H - 1);
    iw = min(max(iw, 0), a.W - 1);
    const float q = xb[((int64_t)ic * a.H + ih) * a.W + iw];
    v[j] = zero ? 0.f : q;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) t[c * kUfPitch + wave + 4 * j] = v[j];
  __syncthreads();
  // stores: 64 rows x 8 float4 of k, two per thread (row tid / 8 + 32 i, quad tid % 8)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rl = (tid >> 3) + 32 * i, kq = 4 * (tid & 7);
    if (n0 + rl < N) {
      const float* src = t + rl * kUfPitch + kq;
      *reinterpret_cast<float4*>(a.u + ((int64_t)b * N + n0 + rl) * a.Kp + k0 + kq) =
          make_float4(src[0], src[1], src[2], src[3]);
    }
  }
}

// Few input channels (CIN * 3 * 3 taps: the frequency encoder's first level, 2 channels): the
// contraction is too short for the matrix cores, so one thread per output position loads its
// whole input window (CIN x 3 x 3 samples, branch-free: mirrored or clamped indices, padding
// zeroed by a select) into registers and produces COB output channels from weights staged in
// LDS ([tap][channel], 16-byte broadcasts). With stats, each workgroup also writes the GroupNorm
// partial (count, mean, M2) of its outputs (two passes over a thread's registers, then the
// workgroup merge) for the group its COB channels belong to (the host checks that COB divides the
// group's channel count): parts[((b * G + g) * nparts + j) * 3], j = (channel block within the
// group) * gridDim.x + position block, nparts = (C / G / COB) * gridDim.x. Large workgroups (NT
// threads, 512 or 1024) keep the partial count (which every apply workgroup merges) low.
template <int CIN, int COB, bool REFLECT, int NT>
__global__ __launch_bounds__(NT) void conv2d_small_kernel(Conv2DArgs a, float* stats, int G) {
  constexpr int CK = CIN * 9;
  __shared__ __attribute__((aligned(16))) float wt[CK * COB + COB];  // [tap][co], then bias
  __shared__ float red[3 * (NT / 64)];
  // (numbering the workgroups that read one input window, one per block of COB output channels,
  // onto one XCD measured 11 % slower)
  const int nx = gridDim.x, bx = blockIdx.x, b = blockIdx.z, co0 = blockIdx.y * COB;
  const unsigned hw = (unsigned)a.Ho * (unsigned)a.Wo;
  const unsigned n = bx * (unsigned)NT + threadIdx.x;
  const bool valid = n < hw;
  const unsigned nc = valid ? n : hw - 1;
  const int oh = (int)(nc / (unsigned)a.Wo), ow = (int)(nc - (unsigned)oh * a.Wo);
  // weights and bias of this workgroup's channels (issued first)
  constexpr int NW = CK * COB + COB, PER = (NW + NT - 1) / NT;
  float wv[PER];
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int i = threadIdx.x + NT * r;
    const int iw = min(i, CK * COB - 1), co = iw / CK, e = iw - co * CK;
    const float* src = i < CK * COB ? a.w + (int64_t)(co0 + co) * CK + e
                                    : (a.bias ? a.bias + co0 + min(i - CK * COB, COB - 1)
                                              : a.w);
    const float v = *src;
    wv[r] = (i < CK * COB || a.bias) ? v : 0.f;
  }
  // the input window
  const float* xb = a.x + (int64_t)b * CIN * a.H * a.W;
  float xv[CK];
#pragma unroll
  for (int ic = 0; ic < CIN; ++ic)
#pragma unroll
    for (int kh = 0; kh < 3; ++kh)
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) {
        int r = oh * a.sh - a.ph + kh, c = ow * a.sw - a.pw + kw;
        float keep = 1.f;
        if constexpr (REFLECT) {
          r = reflect_index(r, a.H);
          c = reflect_index(c, a.W);
        } else {
          keep = (r >= 0 && r < a.H && c >= 0 && c < a.W) ? 1.f : 0.f;
          r = min(max(r, 0), a.H - 1);
          c = min(max(c, 0), a.W - 1);
        }
        xv[(ic * 3 + kh) * 3 + kw] = xb[((int64_t)ic * a.H + r) * a.W + c] * keep;
      }
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int i = threadIdx.x + NT * r;
    if (i < CK * COB) {
      const int co = i / CK, e = i - co * CK;
      wt[e * COB + co] = wv[r];
    } else if (i < NW) {
      wt[i] = wv[r];
    }
  }
  __syncthreads();
  float acc[COB];
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = wt[CK * COB + j];
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
    float* yb = a.y + ((int64_t)b * a.Cout + co0) * hw + n;
#pragma unroll
    for (int j = 0; j < COB; ++j) yb[(int64_t)j * hw] = acc[j];
  }
  if (stats) {  // uniform
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < COB; ++j) s += acc[j];
    float mean = s * (1.f / COB), m2 = 0.f;
#pragma unroll
    for (int j = 0; j < COB; ++j) m2 = fmaf(acc[j] - mean, acc[j] - mean, m2);
    float cnt = valid ? (float)COB : 0.f;
    if (!valid) mean = m2 = 0.f;
    block_welford(cnt, mean, m2, red);
    if (threadIdx.x == 0) {
      const int cpg = a.Cout / G, g = co0 / cpg, nblk = cpg / COB;
      const int nparts = nblk * nx, j = (co0 % cpg) / COB * nx + bx;
      float* o = stats + (((int64_t)b * G + g) * nparts + j) * 3;
      o[0] = cnt;
      o[1] = mean;
      o[2] = m2;
    }
  }
}

// Grid (output plane / 256, Cout, B); 32-bit plane index (host-checked).
__global__ __launch_bounds__(256) void conv2d_direct_kernel(Conv2DArgs a) {
  const unsigned hw = (unsigned)a.Ho * (unsigned)a.Wo;
  const unsigned n = blockIdx.x * 256u + threadIdx.x;
  if (n >= hw) return;
  const int oc = blockIdx.y, b = blockIdx.z;
  const int oh = (int)(n / (unsigned)a.Wo), ow = (int)(n - (unsigned)oh * a.Wo);
  const int64_t idx = ((int64_t)b * a.Cout + oc) * hw + n;
  const int cinpg = a.Cin / a.groups, coutpg = a.Cout / a.groups, g = oc / coutpg;
  const float* xb = a.x + (int64_t)b * a.Cin * a.H * a.W;
  float sum = 0.f;
  for (int icg = 0; icg < cinpg; ++icg) {
    const float* xc = xb + (int64_t)(g * cinpg + icg) * a.H * a.W;
    const float* wr = a.w + ((int64_t)oc * cinpg + icg) * a.KH * a.KW;
    for (int kh = 0; kh < a.KH; ++kh)
      for (int kw = 0; kw < a.KW; ++kw)
        sum = fmaf(conv2d_sample(xc, oh * a.sh - a.ph + kh * a.dh, ow * a.sw - a.pw + kw * a.dw,
                                 a.H, a.W, a.reflect),
                   wr[kh * a.KW + kw], sum);
  }
  if (a.bias) sum += a.bias[oc];
  a.y[idx] = sum;
}

// y[b][oc][oh][ow] = bias[oc] + the taps of Z[b][(oc*KH + kh)*KW + kw][ih*W + iw] that reach it,
// summed in (kh, kw) order.
__global__ __launch_bounds__(256) void convt2d_gather_kernel(ConvT2DArgs a) {
  const unsigned hw = (unsigned)a.Ho * (unsigned)a.Wo;
  const unsigned n = blockIdx.x * 256u + threadIdx.x;
  if (n >= hw) return;
  const int oc = blockIdx.y, b = blockIdx.z;
  const int oh = (int)(n / (unsigned)a.Wo), ow = (int)(n - (unsigned)oh * a.Wo);
  const int64_t idx = ((int64_t)b * a.Cout + oc) * hw + n;
  const int64_t n_in = (int64_t)a.H * a.W;
  const float* zb = a.z + ((int64_t)b * a.Cout + oc) * a.KH * a.KW * n_in;
  float sum = 0.f;
  for (int kh = 0; kh < a.KH; ++kh) {
    const int nh = oh + a.ph - kh * a.dh;
    if (nh < 0 || nh % a.sh) continue;
    const int ih = nh / a.sh;
    if (ih >= a.H) continue;
    for (int kw = 0; kw < a.KW; ++kw) {
      const int nw = ow + a.pw - kw * a.dw;
      if (nw < 0 || nw % a.sw) continue;
      const int iw = nw / a.sw;
      if (iw >= a.W) continue;
      sum += zb[(int64_t)(kh * a.KW + kw) * n_in + (int64_t)ih * a.W + iw];
    }
  }
  if (a.bias) sum += a.bias[oc];
  a.y[idx] = sum;
}

// Dilation 1, stride_w <= 8: one thread per (oh, q) computes the sw outputs ow = sw*q + r. For
// each r the taps kw = (r + pw) mod sw, + sw, ... are the same for every lane, and lanes with
// consecutive q read consecutive iw = (ow + pw - kw) / sw, so the reads coalesce and no lane
// diverges on the column taps. Per output the taps are summed kh-major, kw ascending, as in
// convt2d_gather_kernel.
__global__ __launch_bounds__(256) void convt2d_gather_phase_kernel(ConvT2DArgs a) {
  constexpr int kMaxSW = 8;
  const unsigned nq = ((unsigned)a.Wo + a.sw - 1) / a.sw;
  const unsigned e = blockIdx.x * 256u + threadIdx.x;
  if (e >= (unsigned)a.Ho * nq) return;
  const int oc = blockIdx.y, b = blockIdx.z;
  const int oh = (int)(e / nq), q = (int)(e - (unsigned)oh * nq);
  const int64_t n_in = (int64_t)a.H * a.W;
  const float* zb = a.z + ((int64_t)b * a.Cout + oc) * a.KH * a.KW * n_in;
  float acc[kMaxSW];
#pragma unroll
  for (int r = 0; r < kMaxSW; ++r) acc[r] = 0.f;
  const int th = oh + a.ph;
  for (int kh = th % a.sh; kh < a.KH && kh <= th; kh += a.sh) {
    const int ih = (th - kh) / a.sh;
    if (ih >= a.H) continue;
    const float* zr = zb + (int64_t)kh * a.KW * n_in + (int64_t)ih * a.W;
#pragma unroll
    for (int r = 0; r < kMaxSW; ++r) {
      if (r >= a.sw) break;
      const int tw = a.sw * q + r + a.pw;
      for (int kw = tw % a.sw; kw < a.KW && kw <= tw; kw += a.sw) {
        const int iw = (tw - kw) / a.sw;
        if (iw < a.W) acc[r] += zr[(int64_t)kw * n_in + iw];
      }
    }
  }
  float* yr = a.y + (((int64_t)b * a.Cout + oc) * a.Ho + oh) * a.Wo;
  const float bias = a.bias ? a.bias[oc] : 0.f;
#pragma unroll
  for (int r = 0; r < kMaxSW; ++r) {
    const int ow = a.sw * q + r;
    if (r < a.sw && ow < a.Wo) yr[ow] = acc[r] + bias;
  }
}

// The phase form for a fixed kernel and stride (dilation 1): the taps of output (oh, SW*q + r) are
// kh = (oh + ph) mod SH + SH*jh and kw = (SW*q + r + pw) mod SW + SW*jw, so each thread loads
// ceil(KH/SH) x SW x ceil(KW/SW) values at clamped addresses (taps outside the kernel or the input
// zeroed by a select), every load in flight at once, and sums them in the same order as the
// general kernels (kh ascending, then kw ascending).
//
// STATS: each thread computes CPT cells (cells e + 256 k of its workgroup's block of 256 * CPT,
// every load issued before any sum), so a workgroup covers CPT times the cells and writes a
// GroupNorm partial (count, mean, M2) of its outputs for CPT times fewer partials (every apply
// workgroup merges all of its group's partials): stats[((b * G + g) * nparts + j) * 3],
// j = (channel within the group) * gridDim.x + blockIdx.x, nparts = Cout / G * gridDim.x
// (gn_apply_parts' layout), so no statistics pass reads y. The partial comes from sums of the
// outputs less the channel's bias (the tap sums) and of their squares, reduced by DPP row sums
// and one LDS exchange between the waves: a Welford merge over lanes (a division and a chain of
// LDS permutes per step) left every wave waiting ~1 us at its end, which made the gather a third
// slower.
template <int KH, int KW, int SH, int SW, bool STATS, int CPT = 1>
__global__ __launch_bounds__(256) void convt2d_gather_fixed_kernel(ConvT2DArgs a) {
  constexpr int NJH = (KH + SH - 1) / SH, NJW = (KW + SW - 1) / SW;
  static_assert(STATS || CPT == 1, "several cells per thread only with the partials");
  __shared__ float red[STATS ? 3 * (256 / 64) : 1];
  const unsigned nq = ((unsigned)a.Wo + SW - 1) / SW, cells = (unsigned)a.Ho * nq;
  const int oc = blockIdx.y, b = blockIdx.z;
  const int64_t n_in = (int64_t)a.H * a.W;
  const float* zb = a.z + ((int64_t)b * a.Cout + oc) * KH * KW * n_in;
  float v[CPT][NJH][SW][NJW];
  bool ok[CPT][NJH][SW][NJW];
  int ohs[CPT], qs[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const unsigned e = (blockIdx.x * CPT + c) * 256u + threadIdx.x;
    const unsigned ec = min(e, cells - 1);
    const int oh = (int)(ec / nq), q = (int)(ec - (unsigned)oh * nq);
    ohs[c] = oh;
    qs[c] = e < cells ? q : -1;  // -1: past the plane
    const int th = oh + a.ph;
#pragma unroll
    for (int jh = 0; jh < NJH; ++jh) {
      const int kh = th % SH + SH * jh, ih = (th - kh) / SH;
      const bool okh = kh < KH && th - kh >= 0 && ih < a.H;
      const int khc = min(kh, KH - 1), ihc = min(max(ih, 0), a.H - 1);
#pragma unroll
      for (int r = 0; r < SW; ++r) {
        const int tw = SW * q + r + a.pw;
#pragma unroll
        for (int jw = 0; jw < NJW; ++jw) {
          const int kw = tw % SW + SW * jw, iw = (tw - kw) / SW;
          const bool okw = kw < KW && tw - kw >= 0 && iw < a.W;
          const int kwc = min(kw, KW - 1), iwc = min(max(iw, 0), a.W - 1);
          v[c][jh][r][jw] = zb[(int64_t)(khc * KW + kwc) * n_in + (int64_t)ihc * a.W + iwc];
          ok[c][jh][r][jw] = okh && okw;
        }
      }
    }
  }
  const float bias = a.bias ? a.bias[oc] : 0.f;
  float sn = 0.f, s1 = 0.f, s2 = 0.f;  // count, sum and sum of squares of acc = y - bias
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    float acc[SW];
#pragma unroll
    for (int r = 0; r < SW; ++r) acc[r] = 0.f;
#pragma unroll
    for (int jh = 0; jh < NJH; ++jh)
#pragma unroll
      for (int r = 0; r < SW; ++r)
#pragma unroll
        for (int jw = 0; jw < NJW; ++jw)
          if (ok[c][jh][r][jw]) acc[r] += v[c][jh][r][jw];
    if (qs[c] < 0) continue;
    float* yr = a.y + (((int64_t)b * a.Cout + oc) * a.Ho + ohs[c]) * a.Wo;
#pragma unroll
    for (int r = 0; r < SW; ++r) {
      const int ow = SW * qs[c] + r;
      if (ow < a.Wo) {
        yr[ow] = acc[r] + bias;
        if (STATS) {
          sn += 1.f;
          s1 += acc[r];
          s2 = fmaf(acc[r], acc[r], s2);
        }
      }
    }
  }
  if (STATS) {
    sn = wave_sum_dpp(sn);
    s1 = wave_sum_dpp(s1);
    s2 = wave_sum_dpp(s2);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) {
      red[3 * wid + 0] = sn;
      red[3 * wid + 1] = s1;
      red[3 * wid + 2] = s2;
    }
    lds_barrier();
    if (threadIdx.x == 0) {
      float n = 0.f, t1 = 0.f, t2 = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        n += red[3 * w + 0];
        t1 += red[3 * w + 1];
        t2 += red[3 * w + 2];
      }
      const float md = n > 0.f ? t1 / n : 0.f;
      const int cpg = a.Cout / a.stat_groups, g = oc / cpg;
      const int nparts = cpg * (int)gridDim.x, j = (oc % cpg) * gridDim.x + blockIdx.x;
      float* o = a.stats + (((int64_t)b * a.stat_groups + g) * nparts + j) * 3;
      o[0] = n;
      o[1] = bias + md;
      o[2] = fmaxf(t2 - t1 * md, 0.f);
    }
  }
}

// Few output channels, 3x3 kernel, stride 2, padding 1, dilation 1 (the frequency decoder's last
// level, 2 channels): a matrix-core tile over Cout * 9 tap rows would be mostly padding. Output
// o = 2i + k - 1, so the outputs 2m and 2m + 1 of a dimension take the taps (k 1 at i = m) and
// (k 0 at i = m + 1, k 2 at i = m). A lane owns four consecutive input cells of one row,
// (mh, 4g .. 4g + 3), and computes their 2 x 8 outputs of every output channel from input rows mh
// and mh + 1, columns 4g .. 4g + 4 (zero past the input): per channel and row one 16-byte load
// (VEC: rows 16-byte aligned) and one scalar. The 64 lanes of a wave take 64 consecutive column
// groups of the row-major sequence of groups (ceil(W / 4) per row), so no lane idles on a row's
// end (with 64-column blocks, W = 168 left 1/8 of the lanes idle and needed 774 workgroups for
// 768 slots, one almost empty second round); the four waves of a workgroup split the input
// channels (batches of CB, the next batch's loads in flight) and add their accumulators through
// LDS in wave order; the weights are staged in LDS once and read as broadcasts. With a.stats, the
// first wave (which stores the workgroup's outputs) also writes each channel's GroupNorm partial
// (count, mean, M2) over them: a.stats[((b * G + g) * nparts + j) * 3], j = (channel within the
// group) * gridDim.x + block, nparts = (Cout / G) * gridDim.x (gn_apply_parts' layout).
constexpr int kT2Waves = 4, kT2WMax = 12288;  // at most 48 KB of weights staged in LDS
template <int COUT, bool VEC>
__global__ __launch_bounds__(64 * kT2Waves) void convt2d_small_kernel(ConvT2DArgs a) {
  // channels per load batch (the frequency decoder's last level: 26.3 us at 2, 27.9 at 3, 28.1 at 4)
  constexpr int CB = 2;
  constexpr int CST = COUT * 9;  // weights per input channel, w[c][oc][kh][kw]
  extern __shared__ __attribute__((aligned(16))) float wl[];  // Cin * CST floats (dynamic)
  __shared__ float part[kT2Waves - 1][COUT * 16][64];
  // XCD-aware numbering: consecutive blocks of column groups (the next input row is the row below
  // of the previous blocks) run on one XCD and share its L2
  const int unit = xcd_logical_tile(blockIdx.x + gridDim.x * blockIdx.z, gridDim.x * gridDim.z);
  const int bx = unit % gridDim.x, b = unit / gridDim.x, lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int gw = (a.W + 3) / 4;  // column groups per row
  const int64_t ng = (int64_t)a.H * gw, gi = (int64_t)bx * 64 + lane;
  const bool live = gi < ng;
  const int64_t gc = live ? gi : ng - 1;  // lanes past the last group load the last one
  const int mh = (int)(gc / gw), mw0 = 4 * (int)(gc % gw);
  const int Cin = a.C1 + a.C2;
  const int64_t hw = (int64_t)a.H * a.W;
  const float* x1 = a.x1 + (int64_t)b * a.C1 * hw;
  const float* x2 = a.x2 ? a.x2 + (int64_t)b * a.C2 * hw : x1;
  const int per = (Cin + kT2Waves * CB - 1) / (kT2Waves * CB) * CB;
  const int cb = min(wave * per, Cin), ce = min(cb + per, Cin);
  // input rows mh, mh + 1 (clamped; a row past the input reads as zero), columns mw0 .. mw0 + 4
  const int r0 = min(mh, a.H - 1), r1 = min(mh + 1, a.H - 1);
  const float rk1 = mh + 1 < a.H ? 1.f : 0.f;
  float ck[5];
  int col[5];
#pragma unroll
  for (int e = 0; e < 5; ++e) {
    ck[e] = mw0 + e < a.W ? 1.f : 0.f;
    col[e] = min(mw0 + e, a.W - 1);
  }
  // xv[j][row][e]: channel c0 + j, input row mh + row, column mw0 + e
  auto load_batch = [&](int c0, float (&xv)[CB][2][5]) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int c = min(c0 + j, Cin - 1);
      const float* pl = c < a.C1 ? x1 + (int64_t)c * hw : x2 + (int64_t)(c - a.C1) * hw;
#pragma unroll
      for (int row = 0; row < 2; ++row) {
        const float* pr = pl + (int64_t)(row ? r1 : r0) * a.W;
        if constexpr (VEC) {
          const float4 v4 = *reinterpret_cast<const float4*>(pr + min(mw0, a.W - 4));
          xv[j][row][0] = v4.x;
          xv[j][row][1] = v4.y;
          xv[j][row][2] = v4.z;
          xv[j][row][3] = v4.w;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) xv[j][row][e] = pr[col[e]];
        }
        xv[j][row][4] = pr[col[4]];
      }
    }
  };
  float xv[CB][2][5];
  load_batch(cb, xv);
  for (int e = threadIdx.x; e < Cin * CST; e += 64 * kT2Waves) wl[e] = a.w[e];
  __syncthreads();
  // acc[oc][rh][ocol]: output row 2 mh + rh, output column 2 mw0 + ocol
  float acc[COUT][2][8];
#pragma unroll
  for (int oc = 0; oc < COUT; ++oc)
#pragma unroll
    for (int rh = 0; rh < 2; ++rh)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[oc][rh][e] = 0.f;
  for (int c0 = cb; c0 < ce; c0 += CB) {
    float xn[CB][2][5];
    load_batch(min(c0 + CB, ce - 1), xn);  // after the last batch: reloaded, unused
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      if (c0 + j < ce) {  // uniform
        float x0[5], x1v[5];
#pragma unroll
        for (int e = 0; e < 5; ++e) {
          x0[e] = xv[j][0][e] * ck[e];
          x1v[e] = xv[j][1][e] * ck[e] * rk1;
        }
#pragma unroll
        for (int oc = 0; oc < COUT; ++oc) {
          const float* k = wl + (c0 + j) * CST + oc * 9;  // k[3 * kh + kw]
          const float k0 = k[0], k1 = k[1], k2 = k[2], k3 = k[3], k4 = k[4], k5 = k[5],
                      k6 = k[6], k7 = k[7], k8 = k[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // cell column e: x0[e] = x(mh, m), x0[e + 1] = x(mh, m + 1), x1v the row below
            acc[oc][0][2 * e] = fmaf(x0[e], k4, acc[oc][0][2 * e]);
            acc[oc][0][2 * e + 1] = fmaf(x0[e], k5, fmaf(x0[e + 1], k3, acc[oc][0][2 * e + 1]));
            acc[oc][1][2 * e] = fmaf(x0[e], k7, fmaf(x1v[e], k1, acc[oc][1][2 * e]));
            acc[oc][1][2 * e + 1] =
                fmaf(x0[e], k8, fmaf(x0[e + 1], k6, fmaf(x1v[e], k2, fmaf(x1v[e + 1], k0,
                                                                            acc[oc][1][2 * e + 1]))));
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int row = 0; row < 2; ++row)
#pragma unroll
        for (int e = 0; e < 5; ++e) xv[j][row][e] = xn[j][row][e];
  }
  if (wave > 0) {
#pragma unroll
    for (int oc = 0; oc < COUT; ++oc)
#pragma unroll
      for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int e = 0; e < 8; ++e) part[wave - 1][(oc * 2 + rh) * 8 + e][lane] = acc[oc][rh][e];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kT2Waves - 1; ++w)
#pragma unroll
    for (int oc = 0; oc < COUT; ++oc)
#pragma unroll
      for (int rh = 0; rh < 2; ++rh)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[oc][rh][e] += part[w][(oc * 2 + rh) * 8 + e][lane];
#pragma unroll
  for (int oc = 0; oc < COUT; ++oc) {
    const float bv = a.bias ? a.bias[oc] : 0.f;
    float sn = 0.f, s1 = 0.f, s2 = 0.f;  // count, sum and sum of squares of acc = y - bias
#pragma unroll
    for (int rh = 0; rh < 2; ++rh) {
      const int oh = 2 * mh + rh;
      if (!live || oh >= a.Ho) continue;
      float* yr = a.y + (((int64_t)b * a.Cout + oc) * a.Ho + oh) * a.Wo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int ow = 2 * mw0 + e;
        if (ow < a.Wo) {
          yr[ow] = acc[oc][rh][e] + bv;
          sn += 1.f;
          s1 += acc[oc][rh][e];
          s2 = fmaf(acc[oc][rh][e], acc[oc][rh][e], s2);
        }
      }
    }
    if (a.stats) {  // uniform: the channel's GroupNorm partial over this workgroup's outputs
      sn = wave_sum_dpp(sn);
      s1 = wave_sum_dpp(s1);
      s2 = wave_sum_dpp(s2);
      if (lane == 0) {
        const float md = sn > 0.f ? s1 / sn : 0.f;
        const int cpg = a.Cout / a.stat_groups, g = oc / cpg;
        const int nparts = cpg * (int)gridDim.x, j = (oc % cpg) * (int)gridDim.x + bx;
        float* o = a.stats + (((int64_t)b * a.stat_groups + g) * nparts + j) * 3;
        o[0] = sn;
        o[1] = bv + md;
        o[2] = fmaxf(s2 - s1 * md, 0.f);
      }
    }
  }
}

__global__ __launch_bounds__(256) void convt2d_direct_kernel(ConvT2DArgs a) {
  const unsigned hw = (unsigned)a.Ho * (unsigned)a.Wo;
  const unsigned n = blockIdx.x * 256u + threadIdx.x;
  if (n >= hw) return;
  const int oc = blockIdx.y, b = blockIdx.z;
  const int oh = (int)(n / (unsigned)a.Wo), ow = (int)(n - (unsigned)oh * a.Wo);
  const int64_t idx = ((int64_t)b * a.Cout + oc) * hw + n;
  const int Cin = a.C1 + a.C2;
  const int coutpg = a.Cout / a.groups, cinpg = Cin / a.groups;
  const int g = oc / coutpg, ocg = oc % coutpg;
  const int64_t n_in = (int64_t)a.H * a.W;
  float sum = 0.f;
  for (int icg = 0; icg < cinpg; ++icg) {
    const int ic = g * cinpg + icg;
    const float* xc = ic < a.C1 ? a.x1 + ((int64_t)b * a.C1 + ic) * n_in
                                : a.x2 + ((int64_t)b * a.C2 + (ic - a.C1)) * n_in;
    const float* wr = a.w + ((int64_t)ic * coutpg + ocg) * a.KH * a.KW;
    for (int kh = 0; kh < a.KH; ++kh) {
      const int nh = oh + a.ph - kh * a.dh;
      if (nh < 0 || nh % a.sh) continue;
      const int ih = nh / a.sh;
      if (ih >= a.H) continue;
      for (int kw = 0; kw < a.KW; ++kw) {
        const int nw = ow + a.pw - kw * a.dw;
        if (nw < 0 || nw % a.sw) continue;
        const int iw = nw / a.sw;
        if (iw >= a.W) continue;
        sum = fmaf(xc[(int64_t)ih * a.W + iw], wr[kh * a.KW + kw], sum);
      }
    }
  }
  if (a.bias) sum += a.bias[oc];
  a.y[idx] = sum;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

dim3 plane_grid(int64_t hw, int C, int B) {
  MNN_REQUIRE(hw > 0 && hw < (1LL << 31) && C > 0 && C <= 65535 && B > 0 && B <= 65535,
              MNN_ERR_INVALID_ARGUMENT, "2-D conv: output plane / channel / batch count too large");
  return dim3((unsigned)cdiv(hw, 256), (unsigned)C, (unsigned)B);
}

// y[b][m][n] = bias[m] + sum over the K parts q (ascending) of ws[b][q][m][n].
__global__ __launch_bounds__(256) void conv2d_split_reduce_kernel(const float* __restrict__ ws,
                                                                  const float* __restrict__ bias,
                                                                  float* __restrict__ y, int M,
                                                                  unsigned N, int parts) {
  const int b = blockIdx.y;
  const unsigned e = blockIdx.x * 256u + threadIdx.x;
  if (e >= (unsigned)M * N) return;
  const int m = (int)(e / N);
  const int64_t mn = (int64_t)M * N;
  const float* w = ws + (int64_t)b * parts * mn + e;
  float acc = 0.f;
  for (int q = 0; q < parts; ++q) acc += w[q * mn];
  y[(int64_t)b * mn + e] = acc + (bias ? bias[m] : 0.f);
}

// The same sum for one output channel per workgroup row (grid (ceil(N / 1024), M, B), four
// positions per thread), which also writes the GroupNorm partial (count, mean, M2) of its outputs
// for the group of its channel (G groups of M / G channels): stats[((b * G + g) * nparts + j) * 3],
// j = (m mod (M / G)) * gridDim.x + blockIdx.x, nparts = (M / G) * gridDim.x (gn_apply_parts'
// layout), so no statistics pass reads y. The partial comes from sums of the K-part sums (the
// outputs less the bias) and of their squares, reduced by DPP row sums and one LDS exchange.
constexpr int kRedGnPer = 4;  // positions per thread
__global__ __launch_bounds__(256) void conv2d_split_reduce_gn_kernel(
    const float* __restrict__ ws, const float* __restrict__ bias, float* __restrict__ y, int M,
    int N, int parts, float* __restrict__ stats, int G) {
  __shared__ float red[3 * 4];
  const int m = blockIdx.y, b = blockIdx.z;
  const int64_t mn = (int64_t)M * N;
  const float* w = ws + (int64_t)b * parts * mn + (int64_t)m * N;
  float* yr = y + (int64_t)b * mn + (int64_t)m * N;
  const float bv = bias ? bias[m] : 0.f;
  float acc[kRedGnPer];
#pragma unroll
  for (int j = 0; j < kRedGnPer; ++j) acc[j] = 0.f;
  const int n0 = blockIdx.x * 256 * kRedGnPer + threadIdx.x;
  for (int q = 0; q < parts; ++q)  // every load of a part in flight together
#pragma unroll
    for (int j = 0; j < kRedGnPer; ++j) acc[j] += w[q * mn + min(n0 + 256 * j, N - 1)];
  float sn = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int j = 0; j < kRedGnPer; ++j) {
    if (n0 + 256 * j < N) {
      yr[n0 + 256 * j] = acc[j] + bv;
      sn += 1.f;
      s1 += acc[j];
      s2 = fmaf(acc[j], acc[j], s2);
    }
  }
  sn = wave_sum_dpp(sn);
  s1 = wave_sum_dpp(s1);
  s2 = wave_sum_dpp(s2);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    red[3 * wid + 0] = sn;
    red[3 * wid + 1] = s1;
    red[3 * wid + 2] = s2;
  }
  lds_barrier();
  if (threadIdx.x == 0) {
    float n = 0.f, t1 = 0.f, t2 = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      n += red[3 * v + 0];
      t1 += red[3 * v + 1];
      t2 += red[3 * v + 2];
    }
    const float md = n > 0.f ? t1 / n : 0.f;
    const int cpg = M / G, g = m / cpg;
    const int nparts = cpg * (int)gridDim.x, j = (m % cpg) * gridDim.x + blockIdx.x;
    float* o = stats + (((int64_t)b * G + g) * nparts + j) * 3;
    o[0] = n;
    o[1] = bv + md;
    o[2] = fmaxf(t2 - t1 * md, 0.f);
  }
}

// ---------------------------------------------------------------- implicit-GEMM 3x3 conv
// 3x3 kernel, padding 1 (reflect or zero), dilation 1, stride sh, sw in {1, 2}, groups 1, without
// an unfolded operand: y[b][co][n] = bias[co] + sum over (ci, kh, kw) of
// w[co][ci][kh][kw] * x[b][ci][sh*oh - 1 + kh][sw*ow - 1 + kw], n = oh * Wo + ow.
//
// A workgroup (four waves) computes 96 output channels x 128 consecutive positions n (which span
// at most a few output rows), wave w the positions 32 w .. 32 w + 31 of all 96 channels as three
// 32x32 blocks on v_mfma_f32_32x32x2_f32. The contraction runs over stages of 4 input channels
// (36 k). A stage stages in LDS the input window its positions read (input rows
// sh*oh_first - 1 .. sh*oh_last + 1, full width plus a padding column each side, reflected or
// zero at load time, so the operand reads need no bounds logic) and the 96 x 36 weight slice.
// MFMA step t (0..17) gives k slot g the channel 2 (t / 9) + g and tap t % 9, so the two halves
// of a wave read windows one channel apart; the channel pitch in LDS is odd, so at stride 2 (the
// 32 positions of a half on even banks) the other half reads the odd banks.
//
// Every address is fixed per workgroup: a thread's window and weight elements of a stage are
// LDS-DMA buffer loads (buffer_load_dword ... lds) at per-thread offsets from the stage's resource
// (zero padding is an offset past the end, which reads 0) into LDS word tid + 256 i; the 18 B
// operand addresses of a lane are precomputed and the weight slice is laid out per lane
// ([lane row][block][k]), so its reads take immediate offsets. No VALU address work remains in
// the loop (VALU issue does not overlap the fp32 MFMAs of a SIMD), and no registers or LDS stores
// stage the operands: the next stage's copies go to the other LDS buffer while this stage's
// MFMAs run; one wait and one barrier per stage. With ksplit > 1
// the stages are split over blockIdx.z and the raw sums go to
// ws[((b * ksplit + p) * Cout + co) * N + n] for conv2d_split_reduce_kernel.
constexpr int kIgBM = 96, kIgBN = 128, kIgCc = 4, kIgKS = kIgCc * 9;
constexpr int kIgWinMax = 1200;  // window words per channel, R * (W + 2) (host-checked)
constexpr int kIgWinPer = (kIgCc * (kIgWinMax + 1) + 255) / 256;  // window loads per thread
constexpr int kIgARow = 3 * 37;  // a lane row's three blocks of 36 k (+1 pad each)
constexpr int kIgAPer = (32 * kIgARow + 255) / 256;               // weight loads per thread
constexpr unsigned kIgZero = 0x80000000u;  // buffer offset past any stage: reads 0
constexpr int kIgBufDw = 0x00020000;       // buffer resource word 3 (gfx9 raw 32-bit loads)

__global__ __launch_bounds__(256, 2) void conv2d_igemm_kernel(Conv2DArgs a, float* ws,
                                                              int ksplit) {
  __shared__ float win[2][256 * kIgWinPer];
  __shared__ float as[2][256 * kIgAPer];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.Ho * a.Wo, K = a.Cin * 9;
  const int n0 = blockIdx.x * kIgBN, m0 = blockIdx.y * kIgBM;
  const int b = blockIdx.z / ksplit, part = blockIdx.z % ksplit;
  const int nst = a.Cin / kIgCc / ksplit, st0 = part * nst;
  const int WP = a.W + 2;
  const int oh_first = n0 / a.Wo, oh_last = min(n0 + kIgBN - 1, N - 1) / a.Wo;
  const int R = a.sh * (oh_last - oh_first) + 3, RWP = R * WP;
  const int CP = RWP | 1;  // odd channel pitch of the LDS window
  const int plane = a.H * a.W;
  const float* xb = a.x + (int64_t)b * a.Cin * plane;
  const float* wb = a.w + (int64_t)m0 * K;

  // window element e = tid + 256 i: (channel c, row r, column j), its byte offset from the
  // stage's first channel (kIgZero: zero padding or a pad slot)
  // (quotients by the run-time pitches through a float reciprocal, corrected by one: exact for
  // these magnitudes and a fraction of an integer division's instructions)
  auto qdiv = [](int v, int d, float rd) {
    int q = (int)((float)v * rd);
    q -= q * d > v;
    q += (q + 1) * d <= v;
    return q;
  };
  const float rCP = 1.f / (float)CP, rWP = 1.f / (float)WP;
  unsigned woff[kIgWinPer];
#pragma unroll
  for (int i = 0; i < kIgWinPer; ++i) {
    const int e = tid + 256 * i;
    const int c = min(qdiv(e, CP, rCP), kIgCc - 1), rem = e - c * CP, r = qdiv(rem, WP, rWP),
              j = rem - r * WP;
    int ih = a.sh * oh_first - 1 + r, iw = j - 1;
    bool zero = e >= kIgCc * CP || rem >= RWP;
    if (a.reflect) {
      ih = reflect_index(ih, a.H);
      iw = reflect_index(iw, a.W);
    } else {
      zero = zero || ih < 0 || ih >= a.H || iw < 0 || iw >= a.W;
    }
    ih = min(max(ih, 0), a.H - 1);
    iw = min(max(iw, 0), a.W - 1);
    woff[i] = zero ? kIgZero : 4u * (unsigned)(c * plane + ih * a.W + iw);
  }
  // weight element p = tid + 256 i at LDS word p of the [lane row][block][37] layout: row
  // 32 block + lane row, k (the pad word reads k 0)
  unsigned aoff[kIgAPer];
#pragma unroll
  for (int i = 0; i < kIgAPer; ++i) {
    const int p = min(tid + 256 * i, 32 * kIgARow - 1);
    const int lr = p / kIgARow, rem = p - lr * kIgARow, blk = rem / 37, kk = min(rem - blk * 37, 35);
    aoff[i] = 4u * (unsigned)((32 * blk + lr) * K + kk);
  }
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)wb, (short)0, kIgBM * K * 4, kIgBufDw);
  // stage st's window and weights into LDS buffer buf by LDS-DMA: element tid + 256 i lands at
  // word tid + 256 i, i.e. wave w's 64 lanes at words 64 w + 256 i onwards
  const unsigned win_lds = lds_address(&win[0][0]), as_lds = lds_address(&as[0][0]);
  auto issue = [&](int st, int buf) {
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(xb + (int64_t)(st0 + st) * kIgCc * plane), (short)0, kIgCc * plane * 4, kIgBufDw);
    const unsigned wl = win_lds + 4u * (unsigned)(buf * 256 * kIgWinPer + 64 * wave);
#pragma unroll
    for (int i = 0; i < kIgWinPer; ++i) lds_dma4_buf(xrs, woff[i], 0u, wl + 1024u * i);
    const unsigned so = (unsigned)(st0 + st) * kIgKS * 4u;
    const unsigned al = as_lds + 4u * (unsigned)(buf * 256 * kIgAPer + 64 * wave);
#pragma unroll
    for (int i = 0; i < kIgAPer; ++i) lds_dma4_buf(wrs, aoff[i], so, al + 1024u * i);
  };

  // this lane's operand addresses: B at position n (clamped) for the 18 steps, A lane row base
  const int g = lane >> 5, l32 = lane & 31;
  const int n = min(n0 + 32 * wave + l32, N - 1);
  const int oh = n / a.Wo, ow = n - oh * a.Wo;
  const int bbase = a.sh * (oh - oh_first) * WP + a.sw * ow + g * CP;
  int bptr[18];
#pragma unroll
  for (int t = 0; t < 18; ++t) {
    const int tap = t % 9;
    bptr[t] = bbase + 2 * (t / 9) * CP + (tap / 3) * WP + tap % 3;
  }
  const int abase = l32 * kIgARow + 9 * g;

  floatx16 acc[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;

  // one stage on LDS buffer st % 2; the next stage's loads in flight meanwhile
  auto stage = [&](int st, const float* wn, const float* an) {
    if (st + 1 < nst) issue(st + 1, (st + 1) & 1);
    // operands of 6 steps at a time, the next 6 read while these 6 steps' MFMAs run
    float fa[2][6][3], fb[2][6];
    auto read6 = [&](int c, float (&xa)[6][3], float (&xb)[6]) {
#pragma unroll
      for (int u = 0; u < 6; ++u) {
        const int t = 6 * c + u;
        xb[u] = wn[bptr[t]];
#pragma unroll
        for (int i = 0; i < 3; ++i) xa[u][i] = an[abase + 37 * i + 18 * (t / 9) + t % 9];
      }
    };
    read6(0, fa[0], fb[0]);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      __builtin_amdgcn_sched_barrier(0);
      if (c + 1 < 3) read6(c + 1, fa[(c + 1) & 1], fb[(c + 1) & 1]);
#pragma unroll
      for (int u = 0; u < 6; ++u)
#pragma unroll
        for (int i = 0; i < 3; ++i)
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[c & 1][u][i], fb[c & 1][u], acc[i], 0,
                                                        0, 0);
      // the next chunk's LDS reads spread between this chunk's MFMAs
      if (c + 1 < 3) {
#pragma unroll
        for (int r = 0; r < 18; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS reads
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<0>();  // this wave's copies of the next stage have landed ...
    __syncthreads();  // ... and every wave's; every wave is done with this stage's buffer
  };

  issue(0, 0);
  wait_vmcnt<0>();
  __syncthreads();
  for (int st = 0; st < nst; st += 2) {
    stage(st, win[0], as[0]);
    if (st + 1 < nst) stage(st + 1, win[1], as[1]);
  }

  // lane l, register v of block i: channel m0 + 32 i + 8 (v / 4) + 4 g + v % 4, position n
  const int nn = n0 + 32 * wave + l32;
  if (nn >= N) return;
  if (ksplit > 1) {
    float* o = ws + ((int64_t)(b * ksplit + part) * a.Cout + m0) * N + nn;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[(int64_t)(32 * i + 8 * (v / 4) + 4 * g + v % 4) * N] = acc[i][v];
    return;
  }
  float* o = a.y + ((int64_t)b * a.Cout + m0) * N + nn;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = 32 * i + 8 * (v / 4) + 4 * g + v % 4;
      o[(int64_t)m * N] = acc[i][v] + (a.bias ? a.bias[m0 + m] : 0.f);
    }
}

// K split of the unfold GEMM for grids too small to fill the chip (few output tiles, long K):
// parts p with (Kp/32) % p == 0, at least 6 K steps each, at most 1024 tiles in all.
int conv2d_ksplit(const Conv2DArgs& a) {
  if (conv2d_pointwise(a)) return 1;
  const int64_t N = (int64_t)a.Ho * a.Wo;
  const int nk = conv2d_padded_k(a.Cin, a.KH, a.KW) / 32;
  const int64_t tiles = cdiv(a.Cout, 64) * cdiv(N, 64) * a.B;
  int best = 1;
  if (tiles > 384) return best;
  for (int p : {2, 3, 4, 6, 8})
    if (nk % p == 0 && nk / p >= 6 && tiles * p <= 1024) best = p;
  return best;
}

void check_conv2d(const Conv2DArgs& a) {
  MNN_REQUIRE(a.B > 0 && a.Cin > 0 && a.Cout > 0 && a.groups > 0 && a.Cin % a.groups == 0 &&
                  a.Cout % a.groups == 0 && a.KH > 0 && a.KW > 0 && a.sh > 0 && a.sw > 0 &&
                  a.dh > 0 && a.dw > 0 && a.ph >= 0 && a.pw >= 0 && a.H > 0 && a.W > 0 &&
                  a.Ho > 0 && a.Wo > 0 && a.x && a.w && a.y,
              MNN_ERR_INVALID_ARGUMENT, "conv2d: invalid configuration");
  // every tap of every output lies in the (padded) input
  MNN_REQUIRE((int64_t)(a.Ho - 1) * a.sh + (int64_t)(a.KH - 1) * a.dh < (int64_t)a.H + 2 * a.ph &&
                  (int64_t)(a.Wo - 1) * a.sw + (int64_t)(a.KW - 1) * a.dw <
                      (int64_t)a.W + 2 * a.pw,
              MNN_ERR_INVALID_ARGUMENT, "conv2d: output size exceeds the padded input");
}

void check_convt2d(const ConvT2DArgs& a) {
  const int Cin = a.C1 + a.C2;
  MNN_REQUIRE(a.B > 0 && Cin > 0 && a.Cout > 0 && a.groups > 0 && Cin % a.groups == 0 &&
                  a.Cout % a.groups == 0 && a.KH > 0 && a.KW > 0 && a.sh > 0 && a.sw > 0 &&
                  a.dh > 0 && a.dw > 0 && a.ph >= 0 && a.pw >= 0 && a.H > 0 && a.W > 0 &&
                  a.Ho > 0 && a.Wo > 0 && a.x1 && (a.C2 == 0 || a.x2) && a.y,
              MNN_ERR_INVALID_ARGUMENT, "conv_transpose2d: invalid configuration");
}

}  // namespace

int conv2d_padded_k(int Cin, int KH, int KW) { return (Cin * KH * KW + 31) / 32 * 32; }

bool conv2d_gemm_supported(const Conv2DArgs& a) { return a.groups == 1; }

bool conv2d_pointwise(const Conv2DArgs& a) {
  return a.groups == 1 && a.KH == 1 && a.KW == 1 && a.sh == 1 && a.sw == 1 && a.ph == 0 &&
         a.pw == 0 && a.Ho == a.H && a.Wo == a.W;
}

bool conv2d_igemm_supported(const Conv2DArgs& a) {
  static const bool off = [] {  // tuning override: MNN_CONV2D_IGEMM=0 keeps unfold + GEMM
    const char* e = std::getenv("MNN_CONV2D_IGEMM");
    return e && std::atoi(e) == 0;
  }();
  if (off || a.groups != 1 || a.KH != 3 || a.KW != 3 || a.dh != 1 || a.dw != 1 || a.ph != 1 ||
      a.pw != 1 || a.sh < 1 || a.sh > 2 || a.sw < 1 || a.sw > 2 || a.Cin % kIgCc != 0 ||
      a.Cout % kIgBM != 0 || a.H < 2 || a.W < 2 || a.B > 8191)
    return false;
  const int64_t N = (int64_t)a.Ho * a.Wo;
  // rows of output spanned by 128 consecutive positions, and the window that covers them
  const int64_t rows = (a.Wo - 1 + kIgBN - 1) / a.Wo + 1;
  const int64_t R = a.sh * (std::min<int64_t>(rows, a.Ho) - 1) + 3;
  // buffer resources: a stage's 4 channels and the 96-row weight slice in 32-bit byte ranges
  return R * (a.W + 2) <= kIgWinMax && (int64_t)a.Cin * a.H * a.W * 4 < (1LL << 31) &&
         (int64_t)a.Cout * a.Cin * 9 * 4 < (1LL << 31) && N * a.Cout < (1LL << 31) &&
         cdiv(N, kIgBN) < 65536 * 32;
}

namespace {
// K split of the implicit GEMM: the most parts (dividing the stage count, at least 6 stages each)
// that keep the grid within two workgroups per CU. (Splitting further where GroupNorm partials
// are wanted, so that the reduce pass replaces a statistics pass, measured slower: the frequency
// encoder's second level in two parts and the deeper ones in more lost 24 us over the row.)
int conv2d_igemm_ksplit(const Conv2DArgs& a) {
  const int64_t tiles = cdiv((int64_t)a.Ho * a.Wo, kIgBN) * (a.Cout / kIgBM) * a.B;
  const int nst = a.Cin / kIgCc;
  int best = 1;
  for (int p : {2, 3, 4, 6, 8})
    if (nst % p == 0 && nst / p >= 6 && tiles * p <= 512) best = p;
  return best;
}
}  // namespace

int conv2d_gemm_stats_parts(const Conv2DArgs& a) {
  const int G = a.stat_groups;
  if (G <= 0 || a.Cout % G != 0 || !conv2d_igemm_supported(a) || conv2d_igemm_ksplit(a) < 2)
    return 0;
  return a.Cout / G * (int)cdiv((int64_t)a.Ho * a.Wo, 256 * kRedGnPer);
}

int64_t conv2d_split_ws_floats(const Conv2DArgs& a) {
  if (conv2d_igemm_supported(a)) {
    const int p = conv2d_igemm_ksplit(a);
    return p > 1 ? (int64_t)a.B * p * a.Cout * a.Ho * a.Wo : 0;
  }
  const int p = conv2d_ksplit(a);
  return p > 1 ? (int64_t)a.B * p * a.Cout * a.Ho * a.Wo : 0;
}

int64_t conv2d_unfold_floats(const Conv2DArgs& a) {
  return conv2d_pointwise(a) || conv2d_igemm_supported(a) ? 0 : (int64_t)a.B * a.Ho * a.Wo * conv2d_padded_k(a.Cin, a.KH, a.KW);
}

void conv2d_pack_weights(const float* w, int Cout, int Cin, int KH, int KW, float* out) {
  const int K = Cin * KH * KW, Kp = conv2d_padded_k(Cin, KH, KW);
  for (int oc = 0; oc < Cout; ++oc)
    for (int k = 0; k < Kp; ++k) out[(int64_t)oc * Kp + k] = k < K ? w[(int64_t)oc * K + k] : 0.f;
}

void conv2d_gemm(const LaunchCtx& c, const Conv2DArgs& a_in, const float* wpack, float* unfold,
                 float* split_ws) {
  Conv2DArgs a = a_in;
  check_conv2d(a);
  MNN_REQUIRE(conv2d_gemm_supported(a) && wpack, MNN_ERR_INVALID_ARGUMENT,
              "conv2d_gemm: configuration outside the GEMM form");
  const int64_t N = (int64_t)a.Ho * a.Wo;
  MNN_REQUIRE(N < (1LL << 31), MNN_ERR_INVALID_ARGUMENT, "conv2d_gemm: output plane too large");
  GemmArgs g;
  g.M = a.Cout;
  g.N = (int)N;
  g.batch = a.B;
  g.A = wpack;
  g.C = a.y;
  g.ldc = N;
  g.sC = (int64_t)a.Cout * N;
  g.bias = a.bias;
  g.bias_mode = a.bias ? BIAS_M : BIAS_NONE;
  g.name = "conv2d_f32_mfma";
  if (conv2d_pointwise(a)) {
    g.K = a.Cin;
    g.lda = conv2d_padded_k(a.Cin, 1, 1);
    g.B = a.x;
    g.blayout = B_KN;
    g.ldb = N;
    g.sB = (int64_t)a.Cin * N;
    return gemm(c, g);
  }
  if (conv2d_igemm_supported(a)) {
    MNN_REQUIRE(!a.stats || conv2d_gemm_stats_parts(a) > 0, MNN_ERR_INVALID_ARGUMENT,
                "conv2d_gemm: GroupNorm partials outside the implicit GEMM's split form");
    const int parts = conv2d_igemm_ksplit(a);
    MNN_REQUIRE(parts == 1 || split_ws, MNN_ERR_INVALID_ARGUMENT,
                "conv2d_gemm: the K split needs a workspace");
    const dim3 grid((unsigned)cdiv(N, kIgBN), (unsigned)(a.Cout / kIgBM),
                    (unsigned)(a.B * parts));
    launch(c, "conv2d_igemm_f32", conv2d_igemm_kernel, grid, dim3(256), 0, a, split_ws, parts);
    if (a.stats)
      launch(c, "conv2d_split_reduce_f32", conv2d_split_reduce_gn_kernel,
             dim3((unsigned)cdiv(N, 256 * kRedGnPer), (unsigned)a.Cout, (unsigned)a.B), dim3(256),
             0, split_ws, a.bias, a.y, a.Cout, (int)N, parts, a.stats, a.stat_groups);
    else if (parts > 1)
      launch(c, "conv2d_split_reduce_f32", conv2d_split_reduce_kernel,
             dim3((unsigned)cdiv(N * a.Cout, 256), (unsigned)a.B), dim3(256), 0, split_ws,
             a.bias, a.y, a.Cout, (unsigned)N, parts);
    return;
  }
  MNN_REQUIRE(unfold, MNN_ERR_INVALID_ARGUMENT, "conv2d_gemm: unfold buffer required");
  a.Kp = conv2d_padded_k(a.Cin, a.KH, a.KW);
  a.u = unfold;
  MNN_REQUIRE(N * (a.Kp / 4) < (1LL << 31) && a.B <= 65535, MNN_ERR_INVALID_ARGUMENT,
              "conv2d_gemm: unfold too large");
  const dim3 ug((unsigned)cdiv(N * (a.Kp / 4), 256), (unsigned)a.B);
  if (a.Kp % kUfK == 0 && a.Kp / kUfK < 65536)
    launch(c, "conv2d_unfold_f32", conv2d_unfold_tiled_kernel,
           dim3(cdiv(N, kUfRows), (unsigned)(a.Kp / kUfK), (unsigned)a.B), dim3(256), 0, a);
  else if (a.KH == 3 && a.KW == 3)
    launch(c, "conv2d_unfold_f32", conv2d_unfold_kernel<3, 3>, ug, dim3(256), 0, a);
  else if (a.KH == 8 && a.KW == 1)
    launch(c, "conv2d_unfold_f32", conv2d_unfold_kernel<8, 1>, ug, dim3(256), 0, a);
  else
    launch(c, "conv2d_unfold_f32", conv2d_unfold_kernel<0, 0>, ug, dim3(256), 0, a);
  g.K = a.Kp;
  g.lda = a.Kp;
  g.B = unfold;
  g.blayout = B_NK;
  g.ldb = a.Kp;
  g.sB = N * a.Kp;
  const int parts = conv2d_ksplit(a);
  if (parts > 1 && split_ws) {
    g.ksplit = parts;
    g.ws = split_ws;
    g.bias = nullptr;
    g.bias_mode = BIAS_NONE;
    if (gemm_nk_lds_supported(g)) {
      gemm_nk_lds(c, g);
      launch(c, "conv2d_split_reduce_f32", conv2d_split_reduce_kernel,
             dim3((unsigned)cdiv(N * a.Cout, 256), (unsigned)a.B), dim3(256), 0, split_ws,
             a.bias, a.y, a.Cout, (unsigned)N, parts);
      return;
    }
    g.ksplit = 1;
    g.ws = nullptr;
    g.bias = a.bias;
    g.bias_mode = a.bias ? BIAS_M : BIAS_NONE;
  }
  gemm(c, g);
}

void conv2d_direct(const LaunchCtx& c, const Conv2DArgs& a) {
  check_conv2d(a);
  launch(c, "conv2d_direct_f32", conv2d_direct_kernel,
         plane_grid((int64_t)a.Ho * a.Wo, a.Cout, a.B), dim3(256), 0, a);
}

int convt2d_padded_cin(int Cin) { return (Cin + 31) / 32 * 32; }

namespace {
// The fixed-kernel gather's form (3x3, stride 2, dilation 1) and its cells (two outputs each).
bool convt2d_gather_fixed(const ConvT2DArgs& a) {
  return a.dh == 1 && a.dw == 1 && a.KH == 3 && a.KW == 3 && a.sh == 2 && a.sw == 2;
}
int64_t convt2d_gather_cells(const ConvT2DArgs& a) { return (int64_t)a.Ho * ((a.Wo + 1) / 2); }
#ifndef MNN_GATHER_CPT
#define MNN_GATHER_CPT 4
#endif
constexpr int kGatherStatsCells = MNN_GATHER_CPT;  // cells per thread of the gather with partials
}  // namespace

int convt2d_stats_parts(const ConvT2DArgs& a) {
  const int G = a.stat_groups;
  if (G <= 0 || a.Cout % G != 0 || a.Ho <= 0 || a.Wo <= 0) return 0;
  if (convt2d_small_supported(a))  // one partial per channel of each workgroup
    return a.Cout / G * (int)cdiv((int64_t)a.H * ((a.W + 3) / 4), 64);
  if (!convt2d_gemm_supported(a) || !convt2d_gather_fixed(a)) return 0;
  return a.Cout / G * (int)cdiv(convt2d_gather_cells(a), 256 * kGatherStatsCells);
}

bool convt2d_gemm_supported(const ConvT2DArgs& a) { return a.groups == 1; }

int64_t convt2d_z_floats(const ConvT2DArgs& a) {
  return (int64_t)a.B * a.Cout * a.KH * a.KW * a.H * a.W;
}

void convt2d_pack_weights(const float* w, int Cin, int Cout, int KH, int KW, float* out) {
  const int ks = KH * KW, Cp = convt2d_padded_cin(Cin);
  for (int m = 0; m < Cout * ks; ++m)
    for (int ic = 0; ic < Cp; ++ic)
      out[(int64_t)m * Cp + ic] = ic < Cin ? w[((int64_t)ic * Cout + m / ks) * ks + m % ks] : 0.f;
}

void convt2d_gemm(const LaunchCtx& c, const ConvT2DArgs& a, const float* wpack, float* z,
                  float* unfold) {
  check_convt2d(a);
  MNN_REQUIRE(convt2d_gemm_supported(a) && wpack && z && unfold, MNN_ERR_INVALID_ARGUMENT,
              "convt2d_gemm: configuration outside the GEMM form");
  const int64_t n_in = (int64_t)a.H * a.W;
  const int Cin = a.C1 + a.C2, Cp = convt2d_padded_cin(Cin);
  MNN_REQUIRE(n_in * Cp < (1LL << 31) && a.B <= 65535, MNN_ERR_INVALID_ARGUMENT,
              "convt2d_gemm: input too large");
  const int ks = a.KH * a.KW;
  GemmArgs g;
  g.M = a.Cout * ks;
  g.N = (int)n_in;
  g.K = Cp;
  g.batch = a.B;
  g.A = wpack;
  g.lda = Cp;
  g.C = z;
  g.ldc = n_in;
  g.sC = (int64_t)g.M * n_in;
  g.name = "convt2d_f32_mfma";
  // B = the input and the decoder's skip read in place as k-major rows [channel][H*W] (their
  // concat and the channel padding resolved by the GEMM's loader, whose zero weight columns
  // cancel the padding rows), where the LDS-DMA path takes them
  g.blayout = B_KN;
  g.bkn_lds = true;
  g.B = a.x1;
  g.sB = (int64_t)a.C1 * n_in;
  g.B2 = a.C2 ? a.x2 : nullptr;
  g.sB2 = (int64_t)a.C2 * n_in;
  g.kc1 = a.C1;
  g.kvalid = Cin;
  g.ldb = n_in;
  if (!gemm_nk_lds_supported(g)) {
    // operand [H*W][Cp]: the input (and the decoder's skip) transposed, channels zero-padded
    ConvTPackArgs p;
    p.x1 = a.x1;
    p.x2 = a.C2 ? a.x2 : nullptr;
    p.C1 = a.C1;
    p.C2 = a.C2;
    p.Cp = Cp;
    p.L = n_in;
    p.Lq = n_in;
    p.u = unfold;
    convt_pack_t1(c, p, a.B);
    g.blayout = B_NK;
    g.bkn_lds = false;
    g.B = unfold;
    g.B2 = nullptr;
    g.sB2 = 0;
    g.ldb = Cp;
    g.sB = n_in * Cp;
  }
  gemm(c, g);
  ConvT2DArgs t = a;
  t.z = z;
  if (a.stats) {
    MNN_REQUIRE(convt2d_stats_parts(a) > 0, MNN_ERR_INVALID_ARGUMENT,
                "convt2d_gemm: GroupNorm partials outside the fixed-kernel gather");
    dim3 grid = plane_grid(convt2d_gather_cells(a), a.Cout, a.B);
    grid.x = (unsigned)cdiv(convt2d_gather_cells(a), 256 * kGatherStatsCells);
    launch(c, "convt2d_gather_f32",
           convt2d_gather_fixed_kernel<3, 3, 2, 2, true, kGatherStatsCells>, grid, dim3(256), 0,
           t);
  } else if (convt2d_gather_fixed(a)) {
    launch(c, "convt2d_gather_f32", convt2d_gather_fixed_kernel<3, 3, 2, 2, false>,
           plane_grid(convt2d_gather_cells(a), a.Cout, a.B), dim3(256), 0, t);
  } else if (a.dh == 1 && a.dw == 1 && a.sw <= 8) {
    const int64_t cells = (int64_t)a.Ho * ((a.Wo + a.sw - 1) / a.sw);
    launch(c, "convt2d_gather_f32", convt2d_gather_phase_kernel, plane_grid(cells, a.Cout, a.B),
           dim3(256), 0, t);
  } else {
    launch(c, "convt2d_gather_f32", convt2d_gather_kernel,
           plane_grid((int64_t)a.Ho * a.Wo, a.Cout, a.B), dim3(256), 0, t);
  }
}

int64_t convt2d_unfold_floats(const ConvT2DArgs& a) {
  return (int64_t)a.B * a.H * a.W * convt2d_padded_cin(a.C1 + a.C2);
}

namespace {
constexpr int kC2Cob = 8;  // output channels per thread of conv2d_small_kernel (the smaller form)
// (output channels per thread, threads per workgroup): 24 x 512 where the channels (and the
// GroupNorm's groups) split into blocks of 24, else 8 x 1024. On the frequency encoder's first
// level (48 channels, 2 groups) 24 x 512 took 16.0 + 15.7 us (conv + apply) against 19.0 + 15.7:
// a thread's window loads and index work serve three times as many outputs, and 512-thread
// workgroups keep the partials the apply merges at 339 per group (256 threads: 678, apply 17.2).
struct C2Shape { int cob, nt; };
C2Shape small_shape(const Conv2DArgs& a, int G) {
  const bool by24 = a.Cout % 24 == 0 && (G <= 0 || (a.Cout % G == 0 && (a.Cout / G) % 24 == 0));
  return by24 ? C2Shape{24, 512} : C2Shape{kC2Cob, 1024};
}
}

bool conv2d_small_supported(const Conv2DArgs& a) {
  return a.groups == 1 && (a.Cin == 1 || a.Cin == 2) && a.KH == 3 && a.KW == 3 && a.dh == 1 &&
         a.dw == 1 && a.Cout % kC2Cob == 0 && (int64_t)a.Ho * a.Wo < ((int64_t)1 << 31) &&
         a.Cout / kC2Cob <= 65535 && a.B <= 65535;
}

int conv2d_small_parts(const Conv2DArgs& a, int G) {
  if (!conv2d_small_supported(a) || G <= 0 || a.Cout % G != 0 || (a.Cout / G) % kC2Cob != 0)
    return 0;
  const C2Shape sh = small_shape(a, G);
  return (a.Cout / G / sh.cob) * (int)cdiv((int64_t)a.Ho * a.Wo, sh.nt);
}

void conv2d_small(const LaunchCtx& c, const Conv2DArgs& a, float* stats, int G) {
  check_conv2d(a);
  MNN_REQUIRE(conv2d_small_supported(a) && a.w && (!stats || conv2d_small_parts(a, G) > 0),
              MNN_ERR_INVALID_ARGUMENT, "conv2d_small: configuration outside the kernel's form");
  const C2Shape sh = small_shape(a, G);
  const dim3 grid((unsigned)cdiv((int64_t)a.Ho * a.Wo, sh.nt), (unsigned)(a.Cout / sh.cob),
                  (unsigned)a.B);
#define MNN_C2S(CI, R, COB, NT) \
  return launch(c, "conv2d_small_f32", conv2d_small_kernel<CI, COB, R, NT>, grid, dim3(NT), 0, a, \
                stats, G)
#define MNN_C2S_CI(CI, R) \
  if (sh.cob == 24) MNN_C2S(CI, R, 24, 512); \
  MNN_C2S(CI, R, 8, 1024)
  if (a.Cin == 1) {
    if (a.reflect) { MNN_C2S_CI(1, true); }
    MNN_C2S_CI(1, false);
  }
  if (a.reflect) { MNN_C2S_CI(2, true); }
  MNN_C2S_CI(2, false);
#undef MNN_C2S_CI
#undef MNN_C2S
}

bool convt2d_small_supported(const ConvT2DArgs& a) {
  return a.groups == 1 && a.KH == 3 && a.KW == 3 && a.sh == 2 && a.sw == 2 && a.ph == 1 &&
         a.pw == 1 && a.dh == 1 && a.dw == 1 && (a.Cout == 1 || a.Cout == 2 || a.Cout == 4) &&
         (int64_t)(a.C1 + a.C2) * a.Cout * 9 <= kT2WMax && a.Ho <= 2 * a.H && a.Wo <= 2 * a.W &&
         a.W >= 4 && a.B <= 65535 &&
         // the workgroup numbering (column-group blocks x batch) is a 32-bit int
         cdiv((int64_t)a.H * ((a.W + 3) / 4), 64) * a.B < ((int64_t)1 << 31);
}

void convt2d_small(const LaunchCtx& c, const ConvT2DArgs& a) {
  check_convt2d(a);
  MNN_REQUIRE(a.w && convt2d_small_supported(a), MNN_ERR_INVALID_ARGUMENT,
              "convt2d_small: configuration outside the kernel's form");
  const dim3 grid((unsigned)cdiv((int64_t)a.H * ((a.W + 3) / 4), 64), 1, (unsigned)a.B),
      block(64 * kT2Waves);
  const size_t lds = sizeof(float) * (size_t)(a.C1 + a.C2) * a.Cout * 9;
  // 16-byte row loads when every row start is 16-byte aligned (a column group past W - 4 loads
  // the last four columns and uses none of them)
  const bool vec = a.W % 4 == 0 && (reinterpret_cast<uintptr_t>(a.x1) & 15) == 0 &&
                   (a.C2 == 0 || (reinterpret_cast<uintptr_t>(a.x2) & 15) == 0);
#define MNN_T2S(CO) \
  return vec ? launch(c, "convt2d_small_f32", convt2d_small_kernel<CO, true>, grid, block, lds, a) \
             : launch(c, "convt2d_small_f32", convt2d_small_kernel<CO, false>, grid, block, lds, a)
  switch (a.Cout) {
    case 1: MNN_T2S(1);
    case 2: MNN_T2S(2);
    default: MNN_T2S(4);
  }
#undef MNN_T2S
}

void convt2d_direct(const LaunchCtx& c, const ConvT2DArgs& a) {
  check_convt2d(a);
  MNN_REQUIRE(a.w, MNN_ERR_INVALID_ARGUMENT, "convt2d_direct: weights required");
  launch(c, "convt2d_direct_f32", convt2d_direct_kernel,
         plane_grid((int64_t)a.Ho * a.Wo, a.Cout, a.B), dim3(256), 0, a);
}

}  // namespace k
}  // namespace mnn
