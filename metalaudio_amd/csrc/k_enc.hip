// Encoder-level kernels (one UNet encoder block = strided conv -> GroupNorm(1) + GELU -> 1x1
// rewrite conv C -> 2C -> GLU):
//
//   enc_conv_kernel       strided Conv1D, kernel 8 / stride 4 / dilation 1 / groups 1, zero or
//                         reflect padding < 4 (DynamicConv1D.swift:288-324,358-401; UNet.swift:52),
//                         as an implicit GEMM on v_mfma_f32_32x32x2_f32:
//                         y[co][t] = bias[co] + sum_{ci,j} W[co][ci*8+j] * x[ci][4t - pad + j],
//                         with per-workgroup GroupNorm(1) statistics partials of y (biased
//                         variance, Normalization.swift:479-597); deep levels split K over
//                         workgroups and finish in enc_conv_reduce_kernel;
//   enc_gn_gelu_t_kernel  z = GELU(GroupNorm(y)) written transposed, z^T[t][k] (k padded to a
//                         multiple of 32 with zeros): the B operand of the rewrite GEMM;
//   rewrite               the fp32 LDS-DMA GEMM of k_gemm_lds.hip over z^T with the GLU epilogue
//                         (NN.metal:1012-1023).
//
// The conv kernel has the structure of the transformer GEMM (k_gemm_lds.hip): 64x64 output blocks
// per wave, operands staged by LDS-DMA in a ring of S stages of 32 k (= 4 input channels), the
// one barrier per stage placed halfway through the stage, and the next stage's fragments read
// while the second half's MFMAs run. A is the padded weight matrix [Cout][Cinp*8] in the swizzled
// [rows][32 floats] layout. B is never materialised: a stage holds, per input channel, the window
// of BN + 1 consecutive 16-byte chunks x[ci][4*n0 - pad + 4c .. +3] (c = 0..BN), and the operand
// of output column t, taps 4h..4h+3 (h = 0, 1), is chunk t - n0 + h: one 16-byte LDS read. Chunks
// that cross a signal end are loaded clamped to x[0..3] / x[L-4..L-1], which holds every sample
// their reflect (or zero) padding needs, and are rewritten in LDS by the lane that loaded them
// (edge tiles only).
//
// GroupNorm + GELU is applied once per element in its own pass (HBM bound) rather than on the
// rewrite GEMM's operand fragments: on CDNA4 the VALU work of a wave does not overlap fp32 MFMAs
// on its SIMD, and the operand transform would be repeated for every M tile.
#include "device_utils.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int BK = 32;

template <int WMW, int WNW, int WM, int WN, int S>
struct ConvCfg {
  static constexpr int BM = WMW * WM * 32, BN = WNW * WN * 32;
  static constexpr int NW = WMW * WNW, NT = NW * 64;
  static constexpr int A_WL = BM / 8;            // A wave loads per stage (8 rows of 32 floats)
  static constexpr int WCH = BN + 1;             // chunks per channel window
  static constexpr int B_CH = 4 * WCH;           // B chunks per stage
  static constexpr int B_WL = (B_CH + 63) / 64;  // B wave loads per stage
  static constexpr int T = A_WL + B_WL;          // wave loads per stage
  static constexpr int L = (T + NW - 1) / NW;    // per wave (waves >= T % NW issue L - 1)
  static constexpr int A_FLOATS = BM * 32;
  static constexpr int STAGE = A_FLOATS + B_WL * 256;
  static_assert((S - 1) * L < 64, "vmcnt range");
};

struct ConvKArgs {
  int M = 0, N = 0, K = 0;  // Cout, Lout, Cinp * 8
  int Cin = 0, L = 0, pad = 0;
  bool reflect = true;
  const float* W = nullptr;  // [M][K]
  const float* x = nullptr;  // [b][Cin][L]
  int64_t x_bs = 0;
  const float* bias = nullptr;
  float* y = nullptr;  // splits == 1: y[b][m][n], row pitch ldy
  int64_t ldy = 0, y_bs = 0;
  float* parts = nullptr;  // splits == 1: statistics partial per workgroup
  float* ws = nullptr;     // splits > 1: ws[((b * splits + s) * M + m) * N + n]
  int splits = 1;
};

// Value of padded-signal position p given the 4 samples of the clamped chunk starting at q0.
__device__ __forceinline__ float padded_sample(const float4& v, int p, int q0, int L,
                                               bool reflect) {
  int q = p;
  if (reflect) {
    q = q < 0 ? -q : q;
    q = q > L - 1 ? 2 * (L - 1) - q : q;
  } else if (p < 0 || p > L - 1) {
    return 0.f;
  }
  const int i = min(max(q - q0, 0), 3);  // outside 0..3 only for chunks no stored column uses
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <int WMW, int WNW, int WM, int WN, int S, bool SPLIT>
__global__ __launch_bounds__(WMW* WNW * 64) void enc_conv_kernel(ConvKArgs a) {
  using Cfg = ConvCfg<WMW, WNW, WM, WN, S>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NW = Cfg::NW, L = Cfg::L, T = Cfg::T;
  constexpr int A_WL = Cfg::A_WL, WCH = Cfg::WCH, STAGE = Cfg::STAGE;
  __shared__ __attribute__((aligned(1024))) float smem[S * STAGE];
  __shared__ float red[3 * NW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNW, wn = wave % WNW;
  const int b = blockIdx.z / a.splits, sp = blockIdx.z % a.splits;
  const int gx = gridDim.x;
  const int tile = xcd_logical_tile(blockIdx.x + gx * blockIdx.y, gx * gridDim.y);
  const int tn = tile % gx, tm = tile / gx;
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = a.M, N = a.N, K = a.K, Ls = a.L;
  const int nk = K / BK / a.splits, kt0 = sp * nk;
  const float* __restrict__ xb = a.x + (int64_t)b * a.x_bs;

  // ---- per-lane load geometry: wave load j = i*NW + wave of a stage is A (j < A_WL) or B
  unsigned off[L];      // byte offset from the stage's scalar base
  int bpos[L], bch[L];  // B: window chunk start position (unclamped), channel within the stage
  bool bvalid[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const int j = i * NW + wave;
    bpos[i] = 0;
    bch[i] = 0;
    bvalid[i] = false;
    if (j < A_WL) {
      const int rr = j * 8 + (lane >> 3);
      off[i] = 4u * (unsigned)(min(m0 + rr, M - 1) * K + 4 * ((lane & 7) ^ chunk_swizzle(rr)));
    } else {
      const int e = (j - A_WL) * 64 + lane;
      bvalid[i] = j < T && e < Cfg::B_CH;
      const int ee = bvalid[i] ? e : 0;  // past the window: a valid address, never read
      bch[i] = ee / WCH;
      bpos[i] = 4 * n0 - a.pad + 4 * (ee % WCH);
      off[i] = 4u * (unsigned)(bch[i] * Ls + min(max(bpos[i], 0), Ls - 4));
    }
  }
  // tiles whose window crosses a signal end rewrite those chunks after they land
  const bool edge = 4 * n0 - a.pad < 0 || 4 * (n0 + BN) - a.pad + 3 > Ls - 1;
  const unsigned lds0 = lds_address(smem);
  auto issue = [&](int kl) {
    const int kt = kt0 + kl;
    const unsigned base = lds0 + 4u * (unsigned)((kl % S) * STAGE);
    const float* asrc = a.W + kt * BK;
    const float* bsrc = xb + (int64_t)(4 * kt) * Ls;
    // padded input channels read the last real one; that stage's offsets are computed in a branch
    // of its own, around its own loads (with only the offset under the branch the compiler
    // if-converted it, and every stage paid the clamp arithmetic)
    if (4 * kt + 4 > a.Cin) {
#pragma unroll
      for (int i = 0; i < L; ++i) {
        const int j = i * NW + wave;
        if (j < A_WL) {
          lds_dma16_s(asrc, off[i], base + 4u * (unsigned)(j * 256));
        } else if (j < T) {
          const unsigned o = 4u * (unsigned)((min(4 * kt + bch[i], a.Cin - 1) - 4 * kt) * Ls +
                                             min(max(bpos[i], 0), Ls - 4));
          lds_dma16_s(bsrc, o, base + 4u * (unsigned)(Cfg::A_FLOATS + (j - A_WL) * 256));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < L; ++i) {
        const int j = i * NW + wave;
        if (j < A_WL)
          lds_dma16_s(asrc, off[i], base + 4u * (unsigned)(j * 256));
        else if (j < T)
          lds_dma16_s(bsrc, off[i], base + 4u * (unsigned)(Cfg::A_FLOATS + (j - A_WL) * 256));
      }
    }
  };
  // rewrites this lane's landed chunks of stage kl that cross a signal end (before the barrier)
  auto fix_edges = [&](int kl) {
    float* stage = smem + (kl % S) * STAGE + Cfg::A_FLOATS;
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const int j = i * NW + wave;
      if (j >= A_WL && j < T && bvalid[i] && (bpos[i] < 0 || bpos[i] + 3 > Ls - 1)) {
        float4* cp = reinterpret_cast<float4*>(stage + 4 * ((j - A_WL) * 64 + lane));
        const float4 v = *cp;
        const int q0 = min(max(bpos[i], 0), Ls - 4);
        float4 r;
        r.x = padded_sample(v, bpos[i] + 0, q0, Ls, a.reflect);
        r.y = padded_sample(v, bpos[i] + 1, q0, Ls, a.reflect);
        r.z = padded_sample(v, bpos[i] + 2, q0, Ls, a.reflect);
        r.w = padded_sample(v, bpos[i] + 3, q0, Ls, a.reflect);
        *cp = r;
      }
    }
    wait_lgkmcnt0();
  };
  // this wave's loads: L per stage, or L - 1 for waves past T % NW
  const bool full = (T % NW == 0) || wave < T % NW;

  floatx16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int g = lane >> 5, l32 = lane & 31;
  int aoff[WM], asw[WM], boff[WN];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int rr = wm * WM * 32 + 32 * i + l32;
    aoff[i] = rr * BK;
    asw[i] = chunk_swizzle(rr);
  }
#pragma unroll
  for (int j = 0; j < WN; ++j) boff[j] = Cfg::A_FLOATS + 4 * (wn * WN * 32 + 32 * j + l32);

  float4 fa[4][WM], fb[4][WN];
  // k = 16g + 4q + s of a stage: A column k; B channel (16g + 4q) / 8 = 2g + q/2, taps
  // 4(q%2)..+3 of output column t = chunk t - n0 + q%2 of that channel's window
  auto read_frags = [&](int kl, float4 (&xa)[4][WM], float4 (&xb)[4][WN]) {
    const float* base = smem + (kl % S) * STAGE;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int c = 4 * g + q4;
#pragma unroll
      for (int i = 0; i < WM; ++i)
        xa[q4][i] = *reinterpret_cast<const float4*>(base + aoff[i] + 4 * (c ^ asw[i]));
      const int chan = 2 * g + (q4 >> 1);
#pragma unroll
      for (int j = 0; j < WN; ++j)
        xb[q4][j] = *reinterpret_cast<const float4*>(base + boff[j] + chan * (4 * WCH) +
                                                     4 * (q4 & 1));
    }
  };
  auto mfma_slice = [&](int q4) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[q4][i][s], fb[q4][j][s], acc[i][j],
                                                           0, 0, 0);
  };

#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < nk) issue(s);
  // stage 0: at most the S-1 newer stages may still be in flight
  if (S - 1 < nk) {
    if (full) wait_vmcnt<(S - 1) * L>();
    else wait_vmcnt<(S - 1) * (L - 1)>();
  } else {
    wait_vmcnt<0>();
  }
  if (edge) fix_edges(0);
  stage_barrier();
  read_frags(0, fa, fb);
  for (int kl = 0; kl + 1 < nk; ++kl) {
    mfma_slice(0);
    mfma_slice(1);
    __builtin_amdgcn_sched_barrier(0);
    if (kl + S - 1 < nk) {
      if (full) wait_vmcnt<(S - 2) * L>();
      else wait_vmcnt<(S - 2) * (L - 1)>();
    } else {
      wait_vmcnt<0>();
    }
    if (edge) fix_edges(kl + 1);
    stage_barrier();  // stage kl+1 complete everywhere; every wave's reads of stage kl are done
    if (kl + S < nk) issue(kl + S);
    float4 na[4][WM], nb[4][WN];
    read_frags(kl + 1, na, nb);
    mfma_slice(2);
    mfma_slice(3);
    constexpr int kReads = 4 * (WM + WN), kMfma = 8 * WM * WN;
#pragma unroll
    for (int r = 0; r < kReads; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
#pragma unroll
      for (int i = 0; i < WM; ++i) fa[q4][i] = na[q4][i];
#pragma unroll
      for (int j = 0; j < WN; ++j) fb[q4][j] = nb[q4][j];
    }
  }
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) mfma_slice(q4);

  // ---- epilogue; accumulator layout of a 32x32 block: lane l, register v -> row
  // 8*(v/4) + 4*(l/32) + v%4, column l%32
  if constexpr (SPLIT) {
    float* __restrict__ wp = a.ws + ((int64_t)blockIdx.z * M) * N;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int mblk = m0 + wm * WM * 32 + i * 32;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int gn = n0 + wn * WN * 32 + j * 32 + l32;
        if (gn >= N) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
          if (gm < M) wp[(int64_t)gm * N + gn] = acc[i][j][v];
        }
      }
    }
  } else {
    // bias rows first (the compiler may not move these loads past the stores to y); four
    // statistics accumulators so the per-element updates are not one dependent chain
    ShiftedStats st[4];
    float* __restrict__ yp = a.y + (int64_t)b * a.y_bs;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int mblk = m0 + wm * WM * 32 + i * 32;
      float bv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) bv[v] = a.bias[min(mblk + 8 * (v / 4) + 4 * g + (v % 4), M - 1)];
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int gn = n0 + wn * WN * 32 + j * 32 + l32;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
          if (gm < M && gn < N) {
            const float val = acc[i][j][v] + bv[v];
            st[v & 3].add(val);
            yp[(int64_t)gm * a.ldy + gn] = val;
          }
        }
      }
    }
    if (a.parts) {
      float sn, smean, sm2;
      st[0].finish(sn, smean, sm2);
#pragma unroll
      for (int q = 1; q < 4; ++q) {
        float n2, mean2, m22;
        st[q].finish(n2, mean2, m22);
        welford_combine(sn, smean, sm2, n2, mean2, m22);
      }
      block_welford(sn, smean, sm2, red);
      if (tid == 0) {
        float* o = a.parts + ((int64_t)b * gx * gridDim.y + tile) * 3;
        o[0] = sn;
        o[1] = smean;
        o[2] = sm2;
      }
    }
  }
}

// Split-K finish: y[b][m][n] = sum_s ws[b][s][m][n] + bias[m] (fixed order). Workgroup (x, m, b)
// covers columns [kRedCols*x, kRedCols*(x+1)) of row m and writes one GroupNorm(1) statistics
// partial at parts[(b * M + m) * gridDim.x + x].
constexpr int kRedThreads = 256, kRedCols = 1024;
__global__ __launch_bounds__(kRedThreads) void enc_conv_reduce_kernel(
    const float* __restrict__ ws, int splits, int M, int N, const float* __restrict__ bias,
    float* __restrict__ y, int64_t ldy, int64_t y_bs, float* __restrict__ parts) {
  __shared__ float red[3 * kRedThreads / 64];
  const int m = blockIdx.y, b = blockIdx.z;
  const int64_t total = (int64_t)M * N;
  const float* __restrict__ wr = ws + (int64_t)b * splits * total + (int64_t)m * N;
  float* __restrict__ yr = y + (int64_t)b * y_bs + (int64_t)m * ldy;
  const float bm = bias[m];
  ShiftedStats st;
  const int c0 = blockIdx.x * kRedCols;
  constexpr int U = kRedCols / kRedThreads;
  // partials summed in split order (as before), four splits' loads in flight at a time; every
  // load precedes the stores
  float v[U];
  int nn[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    v[u] = 0.f;
    nn[u] = min(c0 + u * kRedThreads + (int)threadIdx.x, N - 1);
  }
  // groups of four splits, all loads of a group in flight together (a group's splits past the
  // last are loaded from the last and not added)
  for (int s = 0; s < splits; s += 4) {
    float t[4][U];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int u = 0; u < U; ++u) t[j][u] = wr[(int64_t)min(s + j, splits - 1) * total + nn[u]];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] += s + j < splits ? t[j][u] : 0.f;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = c0 + u * kRedThreads + threadIdx.x;
    if (n < N) {
      v[u] += bm;
      st.add(v[u]);
      yr[n] = v[u];
    }
  }
  float sn, smean, sm2;
  st.finish(sn, smean, sm2);
  block_welford(sn, smean, sm2, red);
  if (threadIdx.x == 0) {
    float* o = parts + (((int64_t)b * M + m) * gridDim.x + blockIdx.x) * 3;
    o[0] = sn;
    o[1] = smean;
    o[2] = sm2;
  }
}

// Split-K finish, GroupNorm(1) and GELU in one launch, for grids resident at once: a workgroup
// sums the K parts of a tile of kGC channels x kGT positions in split order (as
// enc_conv_reduce_kernel) and adds the bias, publishes the tile's (mean, M2) through the
// grid-wide exchange (device_utils.hpp), merges every partial of its batch and writes
// z^T[b][t][c] = GELU(GroupNorm(y))[c][t] through an LDS transpose: the rewrite GEMM's operand,
// with no pre-norm y in HBM and no separate normalisation pass. C % kGC == 0, so z^T rows hold
// exactly C channels (the rewrite's K).
constexpr int kGT = 64, kGC = 32;    // positions x channels per tile (256 threads, 8 values each)
constexpr int kGnMaxParts = 2048;    // tiles per batch (LDS: 8 bytes each)
constexpr int kGnMaxSlots = 4096;    // tiles over all batches

struct EncGnKArgs {
  const float* ws = nullptr;  // ws[((b * splits + s) * C + c) * N + n]
  int splits = 1, C = 0, N = 0;
  const float* bias = nullptr;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  float eps = 1e-5f;
  float* zt = nullptr;  // [b][N][C]
  unsigned long long* xch = nullptr;
  int spin_limit = 0;
};

// Thread (wave w, lane) holds channels tc * kGC + w + 4 i (i < 8) at position tt * kGT + lane
// (clamped to the last position for the tail tile).
__device__ __forceinline__ void gn_tile_values(const EncGnKArgs& a, int b, int tc, int tt,
                                               float (&v)[8]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t total = (int64_t)a.C * a.N;
  const float* __restrict__ wb = a.ws + (int64_t)b * a.splits * total;
  const int n = min(tt * kGT + lane, a.N - 1);
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  // parts added in split order, the loads of up to four parts in flight together
  auto parts = [&](int s, auto nj) {
    constexpr int J = decltype(nj)::value;
    float t[J][8];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        t[j][i] = wb[(int64_t)(s + j) * total + (int64_t)(tc * kGC + w + 4 * i) * a.N + n];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += t[j][i];
  };
  int s = 0;
  for (; s + 4 <= a.splits; s += 4) parts(s, std::integral_constant<int, 4>{});
  if (s + 2 <= a.splits) {
    parts(s, std::integral_constant<int, 2>{});
    s += 2;
  }
  if (s < a.splits) parts(s, std::integral_constant<int, 1>{});
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = acc[i] + a.bias[tc * kGC + w + 4 * i];
}

// (mean, M2) of a tile (two passes over the registers); every thread returns the same bits.
__device__ __forceinline__ void gn_tile_stats(const float (&v)[8], bool valid, float n, float* red,
                                              float& mean, float& m2) {
  const int wid = threadIdx.x >> 6;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += v[i];
  s = wave_sum_dpp(valid ? s : 0.f);
  if ((threadIdx.x & 63) == 0) red[wid] = s;
  lds_barrier();
  mean = ((red[0] + red[1]) + (red[2] + red[3])) / n;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) q = fmaf(v[i] - mean, v[i] - mean, q);
  q = wave_sum_dpp(valid ? q : 0.f);
  if ((threadIdx.x & 63) == 0) red[4 + wid] = q;
  lds_barrier();
  m2 = (red[4] + red[5]) + (red[6] + red[7]);
}

__global__ __launch_bounds__(256, 4) void enc_reduce_gn_t_kernel(EncGnKArgs a) {
  __shared__ float2 sp[kGnMaxParts];
  __shared__ float tileb[kGC][kGT + 1];
  __shared__ float red[8];
  __shared__ float2 s_res;
  __shared__ float s_gb[2 * kGC];  // gamma, beta of the tile's channels
  __shared__ unsigned s_tag;
  const int tt = blockIdx.x, tc = blockIdx.y, b = blockIdx.z;
  const int ntt = gridDim.x, nparts = gridDim.x * gridDim.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (threadIdx.x == 0) s_tag = xm_tag(a.xch, b);  // read after the statistics' barriers
  auto tile_count = [&](int v) { return (float)(kGC * min(kGT, a.N - (v % ntt) * kGT)); };
  if (threadIdx.x < kGC) {
    const int c = tc * kGC + threadIdx.x;
    s_gb[threadIdx.x] = a.gamma ? a.gamma[c] : 1.f;
    s_gb[kGC + threadIdx.x] = a.beta ? a.beta[c] : 0.f;
  }
  float v[8];
  gn_tile_values(a, b, tc, tt, v);
  const bool valid = tt * kGT + lane < a.N;
  float mean, m2;
  gn_tile_stats(v, valid, tile_count(tc * ntt + tt), red, mean, m2);
  // every partial of the batch computed here from the K parts, as their owners compute them
  auto all_parts = [&]() {
    for (int u = 0; u < nparts; ++u) {
      float vu[8];
      gn_tile_values(a, b, u / ntt, u % ntt, vu);
      float mu, m2u;
      gn_tile_stats(vu, (u % ntt) * kGT + lane < a.N, tile_count(u), red, mu, m2u);
      if (threadIdx.x == 0) sp[u] = make_float2(mu, m2u);
    }
    lds_barrier();
  };
  // tile 0 merges and publishes; the others take its result, or compute every partial themselves
  // when their bounded wait runs out
  const unsigned tag = s_tag;
  const int me = tc * ntt + tt;
  if (threadIdx.x == 0) xm_put(a.xch, b, nparts, me, tag, mean, m2);
  const bool merger = me == 0;
  bool self = false;
  if (merger)
    xm_collect<256, 4>(a.xch, b, nparts, tag, sp);
  else
    self = !xm_wait(a.xch, b, tag, a.spin_limit, &s_res);
  if (self) all_parts();
  float2 mr = s_res;
  if (merger || self) mr = xch_merge(sp, nparts, tile_count, (double)a.C * a.N, a.eps);
  if (merger && threadIdx.x == 0) xm_publish(a.xch, b, tag, mr);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float sc = s_gb[w + 4 * i] * mr.y;
    tileb[w + 4 * i][lane] = gelu_tanh(fmaf(v[i], sc, s_gb[kGC + w + 4 * i] - mr.x * sc));
  }
  lds_barrier();
  // stores: thread covers positions tt * kGT + tid / 8 + 32 j, channels 4 (tid % 8) .. + 3
  float* __restrict__ zb = a.zt + (int64_t)b * a.N * a.C;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int pr = (int)threadIdx.x / 8 + 32 * j, c4 = 4 * ((int)threadIdx.x % 8);
    const int t = tt * kGT + pr;
    if (t < a.N) {
      const float4 z = make_float4(tileb[c4][pr], tileb[c4 + 1][pr], tileb[c4 + 2][pr],
                                   tileb[c4 + 3][pr]);
      *reinterpret_cast<float4*>(zb + (int64_t)t * a.C + tc * kGC + c4) = z;
    }
  }
}

// z^T[b][t][k] = GELU(y[b][k][t] * scale_k + shift_k) for k < C, 0 for C <= k < kp. GroupNorm(1)
// comes from the producer's statistics partials (merged in fp64 in a fixed order, once per
// workgroup) with gamma / beta, or from per-row coefficients coef[b][k] = (scale, shift).
// Workgroups walk the 64 x 64 tiles of their batch (grid-stride) and transpose through LDS; each
// thread moves 16-byte vectors (4 t of one row in, 4 k of one row out), and the next tile's loads
// are issued before the current tile is transformed (the first tile's before the merge).
constexpr int kTT = 64;
__global__ __launch_bounds__(256) void enc_gn_gelu_t_kernel(EncRewriteArgs a) {
  __shared__ float tileb[kTT][kTT + 4];
  __shared__ float2 cf[kTT];
  __shared__ double redd[3 * 4];
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int ntt = (int)((a.Lout + kTT - 1) / kTT), nkt = (a.kp + kTT - 1) / kTT;
  const float* __restrict__ yb = a.y + (int64_t)b * a.C * a.ldy;
  float* __restrict__ zb = a.zt + (int64_t)b * a.Lout * a.kp;
  // loads: thread covers rows r = tid/16 + 16i (i < 4), columns 4*(tid%16) .. +3
  const int lr = tid >> 4, lc = 4 * (tid & 15);
  const bool vec = (a.ldy & 3) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
  auto load_tile = [&](int tile, float4 (&v)[4]) {
    const int t0 = (tile % ntt) * kTT, k0 = (tile / ntt) * kTT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = k0 + lr + 16 * i, t = t0 + lc;
      v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (k < a.C) {
        const float* row = yb + (int64_t)k * a.ldy;
        if (vec && t + 3 < a.Lout) {
          v[i] = *reinterpret_cast<const float4*>(row + t);
        } else {
          if (t + 0 < a.Lout) v[i].x = row[t + 0];
          if (t + 1 < a.Lout) v[i].y = row[t + 1];
          if (t + 2 < a.Lout) v[i].z = row[t + 2];
          if (t + 3 < a.Lout) v[i].w = row[t + 3];
        }
      }
    }
  };
  const int ntiles = ntt * nkt;
  int tile = blockIdx.x;
  float4 cur[4];
  if (tile < ntiles) load_tile(tile, cur);
  float mean = 0.f, rstd = 0.f;
  if (!a.coef) {
    const float2 ms =
        gn1_merge_one_round(a.parts + (int64_t)b * a.nparts * 3, a.nparts, a.eps, redd);
    mean = ms.x;
    rstd = ms.y;
  }
  for (; tile < ntiles; tile += gridDim.x) {
    const int t0 = (tile % ntt) * kTT, k0 = (tile / ntt) * kTT;
    float4 nxt[4];
    if (tile + (int)gridDim.x < ntiles) load_tile(tile + gridDim.x, nxt);
    __syncthreads();  // the previous tile's reads of tileb / cf are done
    if (tid < kTT) {
      const int k = k0 + tid;
      float2 c = make_float2(0.f, 0.f);
      if (k < a.C) {
        if (a.coef) {
          c = *reinterpret_cast<const float2*>(a.coef + ((int64_t)b * a.C + k) * 2);
        } else {
          const float sc = (a.gamma ? a.gamma[k] : 1.f) * rstd;
          c = make_float2(sc, (a.beta ? a.beta[k] : 0.f) - mean * sc);
        }
      }
      cf[tid] = c;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = lr + 16 * i;
      const float2 c = cf[r];
      const bool live = k0 + r < a.C;  // padded rows stay zero
      float4 z;
      z.x = live ? gelu_tanh(fmaf(cur[i].x, c.x, c.y)) : 0.f;
      z.y = live ? gelu_tanh(fmaf(cur[i].y, c.x, c.y)) : 0.f;
      z.z = live ? gelu_tanh(fmaf(cur[i].z, c.x, c.y)) : 0.f;
      z.w = live ? gelu_tanh(fmaf(cur[i].w, c.x, c.y)) : 0.f;
      tileb[r][lc + 0] = z.x;
      tileb[r][lc + 1] = z.y;
      tileb[r][lc + 2] = z.z;
      tileb[r][lc + 3] = z.w;
    }
    __syncthreads();
    // stores: thread covers rows t = t0 + tid/16 + 16i, columns k = k0 + 4*(tid%16) .. +3
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tr = lr + 16 * i, t = t0 + tr, k = k0 + lc;
      if (t < a.Lout && k < a.kp) {
        const float4 z = make_float4(tileb[lc + 0][tr], tileb[lc + 1][tr], tileb[lc + 2][tr],
                                     tileb[lc + 3][tr]);
        *reinterpret_cast<float4*>(zb + (int64_t)t * a.kp + k) = z;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
  }
}

// ---------------------------------------------------------------- first level, fused
// A level whose conv has few input channels (Cin * 8 = K1 <= 32) and C = 48 output channels
// (HTDemucs' first time-encoder level): conv -> GroupNorm(1) -> GELU -> rewrite 48 -> 96 -> GLU
// in one pass per 32 output columns, nothing but the block output written to HBM. The GroupNorm
// statistics come from a statistics-only pass of the direct conv (k_conv.hip) and are folded into
// the conv: GN(W1 x + b1) = (sc . W1) x + (sc b1 + sh), sc = gamma * rstd, sh = beta - mean * sc.
//
// Per wave and 32 columns t:
//   conv     two 32x32 blocks of channels (48 real) on v_mfma_f32_32x32x2_f32, K1 = Cin * 8 taps:
//            lane l feeds A = W1'[32 cb + l%32][2s + l/32] and B = x[e / 8][4t - pad + e % 8],
//            e = 2s + l/32, straight from global memory (reflect / zero padding by index);
//   GELU     on the accumulators: lane l, register v of block cb holds channel
//            ch(cb, v, g) = 32 cb + 8 (v/4) + 4 g + v%4 (g = l/32) at column l%32;
//   rewrite  three 32-row blocks of the regrouped weight [a0..a15 | b0..b15] times z, K = 48: the
//            MFMA's k slot g of k pair p = 16 cb + v is channel ch(cb, v, g), which is exactly the
//            value lane l already holds, so the GELU output feeds the B operand in place; the A
//            operand (rewrite weight columns in that order) is packed on the host as
//            a_rw[(mb * 24 + p) * 64 + lane] and held in registers for the whole kernel;
//   GLU      registers v and v + 8 of a block are partners (rows rr and rr + 16).
constexpr int kL1C = 48, kL1MB = 3, kL1KP = 24;
struct EncL1KArgs {
  int C = 0, Cin = 0, pad = 0, nparts = 0;
  int64_t L = 0, Lout = 0, ldo = 0;
  float eps = 1e-5f;
  const float* x = nullptr;
  const float* w1 = nullptr;  // [C][Cin * 8]
  const float* b1 = nullptr;
  const float* gamma = nullptr;
  const float* beta = nullptr;
  float* parts = nullptr;       // [B][nparts] GroupNorm(1) partials (written by the stats pass)
  const float* a_rw = nullptr;  // [3][24][64] packed rewrite A operand
  const float* rb = nullptr;    // [96] regrouped rewrite bias
  float* out = nullptr;
};

// The conv operand of one 32-column task: lane l supplies, for MFMA k step s, the tap
// e = 2s + l/32 of column t = 32 task + l%32, i.e. x[e / 8][4t - pad + e % 8]. Addresses are
// mirrored (reflect) or clamped (zero padding, the value then zeroed) rather than branched around,
// so every load of the task is in flight at once.
template <int CIN, bool REFLECT>
__device__ __forceinline__ void l1_load_x(const float* __restrict__ xb, int Ls, int Lout, int pad,
                                          int task, int lane, float (&xv)[4 * CIN]) {
  const int g = lane >> 5, l32 = lane & 31;
  const int t = min(task * 32 + l32, Lout - 1);
#pragma unroll
  for (int s = 0; s < 4 * CIN; ++s) {
    const int e = 2 * s + g, ci = e >> 3, j = e & 7;
    int pos = 4 * t - pad + j;
    float keep = 1.f;
    if constexpr (REFLECT) {
      pos = abs(pos);
      pos = min(pos, 2 * (Ls - 1) - pos);
    } else {
      keep = (pos >= 0 && pos < Ls) ? 1.f : 0.f;
      pos = min(max(pos, 0), Ls - 1);
    }
    xv[s] = xb[(int64_t)ci * Ls + pos] * keep;  // x is finite: 0 * x = 0
  }
}

// Two 32-channel blocks of the conv of one task on v_mfma_f32_32x32x2_f32 (A: lane l holds the
// weight of channel 32 cb + l%32, tap 2s + l/32; the accumulators arrive holding the bias).
template <int CIN>
__device__ __forceinline__ void l1_conv(const float (&acv)[2][4 * CIN],
                                        const float (&xv)[4 * CIN], floatx16 (&ac)[2]) {
#pragma unroll
  for (int s = 0; s < 4 * CIN; ++s)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
      ac[cb] = __builtin_amdgcn_mfma_f32_32x32x2f32(acv[cb][s], xv[s], ac[cb], 0, 0, 0);
}

// Statistics pass of the fused first level: the conv y = W1 x + b1 of every column (as the fused
// pass computes it), reduced to one GroupNorm(1) partial (count, mean, M2) per workgroup at
// parts[b * gridDim.x + blockIdx.x]. Lane sums are shifted by the lane's first value; workgroup
// merge by Chan's formula.
template <int CIN, bool REFLECT>
__global__ __launch_bounds__(256) void enc_l1_stats_kernel(EncL1KArgs a) {
  constexpr int C = kL1C, KS = 4 * CIN, K1 = 8 * CIN;
  __shared__ float red[3 * 4];
  __shared__ float s_b1[64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int b = blockIdx.y;
  if (tid < 64) s_b1[tid] = (tid < C && a.b1) ? a.b1[tid] : 0.f;
  float acv[2][KS];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int c = 32 * cb + l32, cc = min(c, C - 1);
    const float live = c < C ? 1.f : 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) acv[cb][s] = a.w1[cc * K1 + 2 * s + g] * live;
  }
  __syncthreads();
  const float* __restrict__ xb = a.x + (int64_t)b * CIN * a.L;
  const int Ls = (int)a.L, Lo = (int)a.Lout;
  const int tasks = (Lo + 31) / 32;
  const int stride = gridDim.x * 4;
  // sums of (v - shift) and its square with one shift per lane, a bias of the lane's channels
  // (outputs sit near their channel's bias), in two chains; the count is 24 per valid column
  const float shift = s_b1[4 * g];
  float s1[2] = {0.f, 0.f}, s2[2] = {0.f, 0.f}, cnt = 0.f;
  int task = blockIdx.x * 4 + wave;
  float xv[KS];
  if (task < tasks) l1_load_x<CIN, REFLECT>(xb, Ls, Lo, a.pad, task, lane, xv);
  for (; task < tasks; task += stride) {
    float xn[KS];
    if (task + stride < tasks) l1_load_x<CIN, REFLECT>(xb, Ls, Lo, a.pad, task + stride, lane, xn);
    floatx16 ac[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int v = 0; v < 16; ++v) ac[cb][v] = s_b1[32 * cb + 8 * (v / 4) + 4 * g + (v % 4)];
    l1_conv<CIN>(acv, xv, ac);
    if (task * 32 + l32 < Lo) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float d = ac[0][v] - shift;
        s1[v & 1] += d;
        s2[v & 1] = fmaf(d, d, s2[v & 1]);
      }
#pragma unroll
      for (int v = 0; v < 8; ++v) {  // channels 32..47
        const float d = ac[1][v] - shift;
        s1[v & 1] += d;
        s2[v & 1] = fmaf(d, d, s2[v & 1]);
      }
      cnt += 24.f;
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) xv[s] = xn[s];
  }
  float sn = cnt, smean = 0.f, sm2 = 0.f;
  if (cnt > 0.f) {
    const float t1 = s1[0] + s1[1], md = t1 / cnt;
    smean = shift + md;
    sm2 = fmaxf((s2[0] + s2[1]) - t1 * md, 0.f);
  }
  block_welford(sn, smean, sm2, red);
  if (tid == 0) {
    float* o = a.parts + ((int64_t)b * gridDim.x + blockIdx.x) * 3;
    o[0] = sn;
    o[1] = smean;
    o[2] = sm2;
  }
}

// The rewrite's A operand (72 values per lane) stays in registers for the whole kernel: read
// from LDS per MFMA, each MFMA would wait for its read (the register budget of more waves per
// SIMD leaves no room to read ahead), which measured 4x slower.
template <int CIN, bool REFLECT>
__global__ __launch_bounds__(256, 2) void enc_l1_fused_kernel(EncL1KArgs a) {
  constexpr int C = kL1C, KS = 4 * CIN, K1 = 8 * CIN;
  __shared__ double redd[3 * 4];
  __shared__ float s_sc[64], s_bp[64], s_rb[2 * kL1C];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int b = blockIdx.y;
  // loaded while the statistics merge runs
  float arw[kL1MB][kL1KP];
#pragma unroll
  for (int mb = 0; mb < kL1MB; ++mb)
#pragma unroll
    for (int p = 0; p < kL1KP; ++p) arw[mb][p] = a.a_rw[(mb * kL1KP + p) * 64 + lane];
  const float2 ms = gn1_merge_one_round(a.parts + (int64_t)b * a.nparts * 3, a.nparts, a.eps, redd);
  if (tid < 64) {
    float sc = 0.f, bp = 0.f;
    if (tid < C) {
      sc = (a.gamma ? a.gamma[tid] : 1.f) * ms.y;
      bp = fmaf(a.b1 ? a.b1[tid] : 0.f, sc, (a.beta ? a.beta[tid] : 0.f) - ms.x * sc);
    }
    s_sc[tid] = sc;
    s_bp[tid] = bp;
  } else if (tid < 64 + 2 * C) {
    s_rb[tid - 64] = a.rb[tid - 64];
  }
  __syncthreads();
  // conv weights scaled by the GroupNorm scale of their channel (rows 48..63: scale 0); the
  // loads are unconditional (clamped rows) so that they are all in flight together
  float acv[2][KS];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int c = 32 * cb + l32, cc = min(c, C - 1);
    const float sc = s_sc[c];
#pragma unroll
    for (int s = 0; s < KS; ++s) acv[cb][s] = a.w1[cc * K1 + 2 * s + g] * sc;
  }
  const float* __restrict__ xb = a.x + (int64_t)b * CIN * a.L;
  float* __restrict__ ob = a.out + (int64_t)b * C * a.ldo;
  const int Ls = (int)a.L, Lo = (int)a.Lout;
  const int tasks = (Lo + 31) / 32;
  const int stride = gridDim.x * 4;
  int task = blockIdx.x * 4 + wave;
  float xv[KS];
  if (task < tasks) l1_load_x<CIN, REFLECT>(xb, Ls, Lo, a.pad, task, lane, xv);
  for (; task < tasks; task += stride) {
    float xn[KS];
    if (task + stride < tasks) l1_load_x<CIN, REFLECT>(xb, Ls, Lo, a.pad, task + stride, lane, xn);
    floatx16 ac[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int ch = 32 * cb + 8 * (v / 4) + 4 * g + (v % 4);
        ac[cb][v] = s_bp[ch];  // zero for the padding channels 48..63
      }
    l1_conv<CIN>(acv, xv, ac);
    float z[kL1KP];
#pragma unroll
    for (int p = 0; p < kL1KP; ++p) z[p] = gelu_tanh(ac[p / 16][p % 16]);
    floatx16 ar[kL1MB];
#pragma unroll
    for (int mb = 0; mb < kL1MB; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) ar[mb][v] = 0.f;
#pragma unroll
    for (int p = 0; p < kL1KP; ++p)
#pragma unroll
      for (int mb = 0; mb < kL1MB; ++mb)
        ar[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(arw[mb][p], z[p], ar[mb], 0, 0, 0);
    const int tc = task * 32 + l32;
    if (tc < a.Lout) {
#pragma unroll
      for (int mb = 0; mb < kL1MB; ++mb)
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int rr = 8 * (v / 4) + 4 * g + (v % 4);
          const float va = ar[mb][v] + s_rb[32 * mb + rr];
          const float vb = ar[mb][v + 8] + s_rb[32 * mb + 16 + rr];
          ob[(int64_t)(16 * mb + rr) * a.ldo + tc] = va * stable_sigmoid(vb);
        }
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) xv[s] = xn[s];
  }
}

// ---------------------------------------------------------------- first level, one launch
// The same level in one launch when its grid is resident at once: every wave computes the conv of
// its tasks (one or two, with the raw weights and bias), the workgroup publishes the
// GroupNorm(1) partial of its tiles through the grid-wide exchange (device_utils.hpp) and keeps
// the pre-norm tiles in LDS; once it has merged every partial of its batch it applies
// GroupNorm + GELU to the kept tiles and runs the rewrite and GLU as the two-pass form does. No
// statistics pass, and the input is read once.
constexpr int kL1MaxTPW = 2;        // tasks per wave
constexpr int kL1MaxParts = 1024;   // workgroups per batch (LDS: 8 bytes each)
constexpr int kL1MaxSlots = 4096;   // workgroups over all batches

// The conv (plus bias) of the tasks task0 + k * stride (k < TPW) of one wave; tasks past the
// last are computed on the last one's columns and never counted or stored. Split into the input
// loads and the matrix work, so a caller can issue the loads before a barrier.
template <int CIN, bool REFLECT, int TPW>
__device__ __forceinline__ void l1_wave_load(const float* __restrict__ xb, int Ls, int Lo, int pad,
                                             int task0, int stride, int lane,
                                             float (&xv)[TPW][4 * CIN]) {
  const int tasks = (Lo + 31) / 32;
#pragma unroll
  for (int k = 0; k < TPW; ++k)
    l1_load_x<CIN, REFLECT>(xb, Ls, Lo, pad, min(task0 + k * stride, tasks - 1), lane, xv[k]);
}

template <int CIN, int TPW>
__device__ __forceinline__ void l1_wave_mma(const float (&xv)[TPW][4 * CIN], int lane,
                                            const float (&acv)[2][4 * CIN], const float* s_b1,
                                            floatx16 (&ac)[TPW][2]) {
  const int g = lane >> 5;
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int v = 0; v < 16; ++v) ac[k][cb][v] = s_b1[32 * cb + 8 * (v / 4) + 4 * g + (v % 4)];
    l1_conv<CIN>(acv, xv[k], ac[k]);
  }
}

template <int CIN, bool REFLECT, int TPW>
__device__ __forceinline__ void l1_wave_conv(const float* __restrict__ xb, int Ls, int Lo, int pad,
                                             int task0, int stride, int lane,
                                             const float (&acv)[2][4 * CIN], const float* s_b1,
                                             floatx16 (&ac)[TPW][2]) {
  float xv[TPW][4 * CIN];
  l1_wave_load<CIN, REFLECT, TPW>(xb, Ls, Lo, pad, task0, stride, lane, xv);
  l1_wave_mma<CIN, TPW>(xv, lane, acv, s_b1, ac);
}

// Element count of workgroup blk's partial: 48 channels x the valid columns of its waves' tasks.
template <int TPW>
__device__ __forceinline__ float l1_block_count(int blk, int stride, int Lo) {
  const int tasks = (Lo + 31) / 32;
  float n = 0.f;
  for (int w = 0; w < 4; ++w)
    for (int k = 0; k < TPW; ++k) {
      const int t = blk * 4 + w + k * stride;
      if (t < tasks) n += (float)(kL1C * min(32, Lo - 32 * t));
    }
  return n;
}

// (mean, M2) of the 48 real channels of a workgroup's tasks, two passes over the registers (the
// mean from a block sum, then M2 about it); every thread returns the same bits. red: 8 floats.
template <int TPW>
__device__ __forceinline__ void l1_block_stats(const floatx16 (&ac)[TPW][2], int task0,
                                               int stride, int Lo, int lane, float n, float* red,
                                               float& mean, float& m2) {
  const int wid = threadIdx.x >> 6, l32 = lane & 31;
  const int tasks = (Lo + 31) / 32;
  bool valid[TPW];
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    const int t = task0 + k * stride;
    valid[k] = t < tasks && t * 32 + l32 < Lo;
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    float sk = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) sk += ac[k][0][v];
#pragma unroll
    for (int v = 0; v < 8; ++v) sk += ac[k][1][v];  // channels 32..47
    s += valid[k] ? sk : 0.f;
  }
  s = wave_sum_dpp(s);
  if (lane == 0) red[wid] = s;
  lds_barrier();
  mean = ((red[0] + red[1]) + (red[2] + red[3])) / n;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    float qk = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) qk = fmaf(ac[k][0][v] - mean, ac[k][0][v] - mean, qk);
#pragma unroll
    for (int v = 0; v < 8; ++v) qk = fmaf(ac[k][1][v] - mean, ac[k][1][v] - mean, qk);
    q += valid[k] ? qk : 0.f;
  }
  q = wave_sum_dpp(q);
  if (lane == 0) red[4 + wid] = q;
  lds_barrier();
  m2 = (red[4] + red[5]) + (red[6] + red[7]);
}

// TPW tasks per wave: 1 with three workgroups per CU, 2 with two (the pre-norm tiles in LDS:
// 32 or 64 KiB per workgroup).
template <int CIN, bool REFLECT, int TPW>
__global__ __launch_bounds__(256, TPW == 1 ? 3 : 2) void enc_l1_oneshot_kernel(
    EncL1KArgs a, unsigned long long* xch, int spin_limit) {
  constexpr int C = kL1C, KS = 4 * CIN, K1 = 8 * CIN;
  __shared__ float stash[4 * TPW * 32 * 64];  // pre-norm tiles: [wave][task][register][lane]
  __shared__ float2 sp[kL1MaxParts];
  __shared__ float red[8];
  __shared__ float s_b1[64], s_sc[64], s_sh[64], s_rb[2 * kL1C];
  __shared__ float2 s_res;
  __shared__ unsigned s_tag;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int b = blockIdx.y, G = gridDim.x;
  if (tid == 0) s_tag = xm_tag(xch, b);  // read after the barrier below
  if (tid < 64) {
    s_b1[tid] = (tid < C && a.b1) ? a.b1[tid] : 0.f;
  } else if (tid < 64 + 2 * C) {
    s_rb[tid - 64] = a.rb[tid - 64];
  }
  float acv[2][KS];  // raw conv weights (rows 48..63 zero)
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int c = 32 * cb + l32, cc = min(c, C - 1);
    const float live = c < C ? 1.f : 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) acv[cb][s] = a.w1[cc * K1 + 2 * s + g] * live;
  }
  // the input windows and the GroupNorm affine parameters are loaded before the barrier: none
  // depends on it, and each is otherwise a dependent memory round trip on the workgroup's path
  // (the window after the barrier, gamma / beta after the statistics exchange)
  const float* __restrict__ xb = a.x + (int64_t)b * CIN * a.L;
  const int Ls = (int)a.L, Lo = (int)a.Lout;
  const int tasks = (Lo + 31) / 32;
  const int stride = G * 4;
  const int task0 = blockIdx.x * 4 + wave;
  float xv[TPW][KS];
  l1_wave_load<CIN, REFLECT, TPW>(xb, Ls, Lo, a.pad, task0, stride, lane, xv);
  const float gam = (tid < C && a.gamma) ? a.gamma[min(tid, C - 1)] : 1.f;
  const float bet = (tid < C && a.beta) ? a.beta[min(tid, C - 1)] : 0.f;
  lds_barrier();
  const unsigned tag = s_tag;
  float mean, m2;
  {
    floatx16 ac[TPW][2];
    l1_wave_mma<CIN, TPW>(xv, lane, acv, s_b1, ac);
    l1_block_stats(ac, task0, stride, Lo, lane, l1_block_count<TPW>(blockIdx.x, stride, Lo), red, mean,
                   m2);
#pragma unroll
    for (int k = 0; k < TPW; ++k)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          stash[((wave * TPW + k) * 32 + 16 * cb + v) * 64 + lane] = ac[k][cb][v];
  }
  // the rewrite operand, in flight while the partials are collected
  float arw[kL1MB][kL1KP];
#pragma unroll
  for (int mb = 0; mb < kL1MB; ++mb)
#pragma unroll
    for (int p = 0; p < kL1KP; ++p) arw[mb][p] = a.a_rw[(mb * kL1KP + p) * 64 + lane];
  // every partial of the batch computed here as its owner does (wave w of this workgroup takes
  // wave w's tasks)
  auto all_parts = [&]() {
    for (int v = 0; v < G; ++v) {
      floatx16 ac[TPW][2];
      const int t0 = v * 4 + wave;
      l1_wave_conv<CIN, REFLECT, TPW>(xb, Ls, Lo, a.pad, t0, stride, lane, acv, s_b1, ac);
      float mu, m2u;
      l1_block_stats(ac, t0, stride, Lo, lane, l1_block_count<TPW>(v, stride, Lo), red, mu, m2u);
      if (tid == 0) sp[v] = make_float2(mu, m2u);
    }
    lds_barrier();
  };
  auto count = [&](int v) { return l1_block_count<TPW>(v, stride, Lo); };
  // workgroup 0 merges and publishes; the others take its result, or compute every partial
  // themselves when their bounded wait runs out
  if (tid == 0) xm_put(xch, b, G, blockIdx.x, tag, mean, m2);
  const bool merger = blockIdx.x == 0;
  bool self = false;
  if (merger)
    xm_collect<256, 4>(xch, b, G, tag, sp);
  else
    self = !xm_wait(xch, b, tag, spin_limit, &s_res);
  if (self) all_parts();
  float2 mr = s_res;
  if (merger || self) mr = xch_merge(sp, G, count, (double)C * Lo, a.eps);
  if (merger && tid == 0) xm_publish(xch, b, tag, mr);
  if (tid < 64) {
    float sc = 0.f, sh = 0.f;
    if (tid < C) {
      sc = gam * mr.y;
      sh = bet - mr.x * sc;
    }
    s_sc[tid] = sc;
    s_sh[tid] = sh;
  }
  lds_barrier();
  float* __restrict__ ob = a.out + (int64_t)b * C * a.ldo;
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    const int task = task0 + k * stride;
    if (task >= tasks) break;
    float z[kL1KP];
#pragma unroll
    for (int p = 0; p < kL1KP; ++p) {
      const int cb = p / 16, v = p % 16;
      const int ch = 32 * cb + 8 * (v / 4) + 4 * g + (v % 4);
      const float y = stash[((wave * TPW + k) * 32 + p) * 64 + lane];
      z[p] = gelu_tanh(fmaf(y, s_sc[ch], s_sh[ch]));
    }
    floatx16 ar[kL1MB];
#pragma unroll
    for (int mb = 0; mb < kL1MB; ++mb)
#pragma unroll
      for (int v = 0; v < 16; ++v) ar[mb][v] = 0.f;
#pragma unroll
    for (int p = 0; p < kL1KP; ++p)
#pragma unroll
      for (int mb = 0; mb < kL1MB; ++mb)
        ar[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(arw[mb][p], z[p], ar[mb], 0, 0, 0);
    const int tc = task * 32 + l32;
    if (tc < Lo) {
#pragma unroll
      for (int mb = 0; mb < kL1MB; ++mb)
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int rr = 8 * (v / 4) + 4 * g + (v % 4);
          const float va = ar[mb][v] + s_rb[32 * mb + rr];
          const float vb = ar[mb][v + 8] + s_rb[32 * mb + 16 + rr];
          ob[(int64_t)(16 * mb + rr) * a.ldo + tc] = va * stable_sigmoid(vb);
        }
    }
  }
}

// ---------------------------------------------------------------- host-side selection
// Kernel-timing name of an encoder launch tagged with the level's channel count, e.g.
// "enc_conv_f32[c96]" (timing queries match by substring, so the family name still sums them).
std::string level_name(const char* family, int channels) {
  return std::string(family) + "[c" + std::to_string(channels) + "]";
}

struct ConvTile {
  int id, bm, bn;
  int lds_kb;  // LDS per workgroup (KiB, rounded up)
  double eff;  // relative matrix-core efficiency of the shape
};
constexpr ConvTile kConvTiles[] = {
    {0, 128, 128, 76, 1.00},  // <2,2,2,2> S3
    {1, 128, 64, 64, 0.93},   // <2,2,2,1> S3
    {2, 64, 128, 52, 0.93},   // <2,2,1,2> S3
    {3, 64, 64, 53, 0.85},    // <2,2,1,1> S4
    {4, 32, 128, 53, 0.85},   // <1,4,1,1> S4
};
constexpr int kCUs = 256;

int env_int(const char* name) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : -1;
}

struct ConvPlan {
  const ConvTile* t = nullptr;
  int splits = 1;
  int tiles = 0;  // output tiles per batch
};

// Critical path per CU: rounds of concurrent workgroups x per-workgroup time (its stages plus a
// fixed prologue / epilogue share, scaled by tile area / efficiency), slowed when a CU holds few
// workgroups, plus the split-K partial traffic (written and read once) in the same units.
ConvPlan plan_conv(int M, int N, int K, int batch, int min_splits = 1) {
  const int nk = K / BK;
  const int ft = env_int("MNN_ENC_CONV_TILE"), fs = env_int("MNN_ENC_CONV_SPLIT");
  ConvPlan best;
  double best_cost = 1e300;
  for (const ConvTile& t : kConvTiles) {
    if (ft >= 0 && t.id != ft) continue;
    const int tiles = (int)(cdiv(M, t.bm) * cdiv(N, t.bn));
    const int occ = std::max(1, std::min(160 / t.lds_kb, 8));
    for (int s : {1, 2, 3, 4, 6, 8, 12, 16}) {
      // a forced split applies where it divides the stages
      if (nk % s != 0 || s < min_splits || (fs > 0 && nk % fs == 0 && s != fs)) continue;
      const int64_t wgs = (int64_t)tiles * batch * s;
      const double rounds = std::ceil((double)wgs / (kCUs * occ));
      const double fill = std::min(1.0, (double)wgs / (kCUs * occ));
      const double per_wg = ((double)nk / s + 3.0) * t.bm * t.bn / t.eff;
      // unit: one 128x128 x 32-k stage on a CU (~2 us); HBM at ~8 TB/s
      const double split_cost =
          s > 1 ? (8.0 * s * M * N * batch / 8e12 / 2e-6 + 1.0) * 16384.0 : 0.0;
      // rows a tile pads past M are computed and dropped: priced as work (measured on the
      // 96-channel level, where the 32-row tile beats 64-row tiles by ~15 %)
      const double pad = (double)cdiv(M, t.bm) * t.bm / M;
      const double cost = rounds * per_wg * pad / (0.6 + 0.4 * fill) + split_cost;
      if (cost < best_cost * 0.999) {
        best_cost = cost;
        best.t = &t;
        best.splits = s;
        best.tiles = tiles;
      }
    }
  }
  MNN_REQUIRE(best.t, MNN_ERR_INVALID_ARGUMENT, "enc_conv: no tile configuration fits K = " << K);
  return best;
}

int conv_parts(const ConvPlan& p, int M, int N) {
  return p.splits > 1 ? M * (int)cdiv(N, kRedCols) : p.tiles;
}

template <int WMW, int WNW, int WM, int WN, int S>
void launch_conv(const LaunchCtx& c, const ConvKArgs& a, int batch) {
  using Cfg = ConvCfg<WMW, WNW, WM, WN, S>;
  dim3 grid(cdiv(a.N, Cfg::BN), cdiv(a.M, Cfg::BM), batch * a.splits), block(Cfg::NT);
  if (a.splits > 1)
    launch(c, level_name("enc_conv_f32", a.M).c_str(), enc_conv_kernel<WMW, WNW, WM, WN, S, true>,
           grid, block, 0, a);
  else
    launch(c, level_name("enc_conv_f32", a.M).c_str(),
           enc_conv_kernel<WMW, WNW, WM, WN, S, false>, grid, block, 0, a);
}

}  // namespace

bool enc_conv_supported(int Cin, int Cout, int ks, int stride, int dil, int groups, int pad,
                        int64_t L) {
  return Cin > 0 && Cout > 0 && ks == 8 && stride == 4 && dil == 1 && groups == 1 && pad >= 0 &&
         pad < 4 && L >= 8 && (int64_t)enc_conv_padded_cin(Cin) * L < (1LL << 29) &&
         (int64_t)Cout * 8 * enc_conv_padded_cin(Cin) < (1LL << 28);
}

int enc_conv_padded_cin(int Cin) { return (Cin + 3) / 4 * 4; }

void enc_conv_plan_info(int Cin, int Cout, int64_t Lout, int batch, bool gn, int* splits,
                        int* bm, int* bn) {
  const ConvPlan p = plan_conv(Cout, (int)Lout, enc_conv_padded_cin(Cin) * 8, batch, gn ? 2 : 1);
  *splits = p.splits;
  *bm = p.t->bm;
  *bn = p.t->bn;
}

int enc_conv_parts(int Cout, int64_t Lout, int K, int batch) {
  return conv_parts(plan_conv(Cout, (int)Lout, K, batch), Cout, (int)Lout);
}

int64_t enc_conv_ws_floats(int Cout, int64_t Lout, int K, int batch, bool gn) {
  const ConvPlan p = plan_conv(Cout, (int)Lout, K, batch, gn ? 2 : 1);
  return p.splits > 1 ? (int64_t)p.splits * batch * Cout * Lout : 0;
}

size_t enc_exchange_bytes() {
  return 8 * (4 * (size_t)kXmMaxBatch + 2 * (size_t)std::max(kGnMaxSlots, kL1MaxSlots));
}

bool enc_conv_gn_fits(const LaunchCtx& c, int Cin, int Cout, int64_t L, int64_t Lout, int B) {
  // workgroups of the finish one CU holds at once (the same for every gfx950 device)
  static const int per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, enc_reduce_gn_t_kernel, 256, 0) !=
        hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    return n;
  }();
  if (Cout % kGC != 0 || !enc_conv_supported(Cin, Cout, 8, 4, 1, 1, 0, L) || Lout < 1 ||
      Lout >= (1LL << 24))
    return false;
  const int nk = enc_conv_padded_cin(Cin) * 8 / BK;
  if (nk < 2) return false;  // K cannot be split
  const int64_t nparts = cdiv(Lout, kGT) * (Cout / kGC);
  return nparts <= kGnMaxParts && B <= kXmMaxBatch && B * nparts <= kGnMaxSlots &&
         B * nparts <= (int64_t)per_cu * c.dev->props.multiProcessorCount;
}

void enc_conv(const LaunchCtx& c, const EncConvArgs& p) {
  ConvKArgs a;
  a.M = p.Cout;
  a.N = (int)p.Lout;
  a.K = enc_conv_padded_cin(p.Cin) * 8;
  a.Cin = p.Cin;
  a.L = (int)p.L;
  a.pad = p.pad;
  a.reflect = p.reflect;
  a.W = p.w;
  a.x = p.x;
  a.x_bs = (int64_t)p.Cin * p.L;
  a.bias = p.bias;
  a.y = p.y;
  a.ldy = p.ldy;
  a.y_bs = (int64_t)p.Cout * p.ldy;
  const bool gn = p.zt != nullptr;
  MNN_REQUIRE(enc_conv_supported(p.Cin, p.Cout, 8, 4, 1, 1, p.pad, p.L) && p.Lout >= 1 &&
                  p.bias && (gn || (p.ldy >= p.Lout && p.parts)) &&
                  (p.Lout - 1) * 4 + 8 <= p.L + 2 * p.pad,
              MNN_ERR_INVALID_ARGUMENT, "enc_conv: unsupported configuration");
  MNN_REQUIRE(!gn || (p.xch && enc_conv_gn_fits(c, p.Cin, p.Cout, p.L, p.Lout, p.B)),
              MNN_ERR_INVALID_ARGUMENT, "enc_conv: GroupNorm finish outside its contract");
  const ConvPlan plan = plan_conv(a.M, a.N, a.K, p.B, gn ? 2 : 1);
  a.splits = plan.splits;
  if (plan.splits > 1) {
    MNN_REQUIRE(p.ws, MNN_ERR_INVALID_ARGUMENT, "enc_conv: split-K needs a workspace");
    a.ws = p.ws;
  } else {
    a.parts = p.parts;
  }
  switch (plan.t->id) {
    case 0: launch_conv<2, 2, 2, 2, 3>(c, a, p.B); break;
    case 1: launch_conv<2, 2, 2, 1, 3>(c, a, p.B); break;
    case 2: launch_conv<2, 2, 1, 2, 3>(c, a, p.B); break;
    case 4: launch_conv<1, 4, 1, 1, 4>(c, a, p.B); break;
    default: launch_conv<2, 2, 1, 1, 4>(c, a, p.B); break;
  }
  if (gn) {
    EncGnKArgs g;
    g.ws = p.ws;
    g.splits = plan.splits;
    g.C = a.M;
    g.N = a.N;
    g.bias = p.bias;
    g.gamma = p.gamma;
    g.beta = p.beta;
    g.eps = p.eps;
    g.zt = p.zt;
    g.xch = static_cast<unsigned long long*>(p.xch);
    g.spin_limit = std::max(p.spin_limit, 0);
    launch(c, level_name("enc_conv_reduce_gn_f32", a.M).c_str(), enc_reduce_gn_t_kernel,
           dim3(cdiv(a.N, kGT), a.M / kGC, p.B), dim3(256), 0, g);
  } else if (plan.splits > 1)
    launch(c, level_name("enc_conv_reduce_f32", a.M).c_str(), enc_conv_reduce_kernel,
           dim3(cdiv(a.N, kRedCols), a.M, p.B),
           dim3(kRedThreads), 0, (const float*)p.ws, plan.splits, a.M, a.N, p.bias, p.y, p.ldy,
           a.y_bs, p.parts);
}

bool enc_l1_supported(int Cin, int Cout, int ks, int stride, int dil, int groups, int pad,
                      int64_t L) {
  return Cin >= 1 && Cin <= 4 && Cout == kL1C && ks == 8 && stride == 4 && dil == 1 &&
         groups == 1 && pad >= 0 && pad < 4 && L > pad && L >= 8 && Cin * L < (1LL << 31);
}

void enc_l1_pack_rewrite(const float* wperm, float* out) {
  // out[(mb * 24 + p) * 64 + lane] = wperm[32 mb + lane % 32][ch(p / 16, p % 16, lane / 32)],
  // ch(cb, v, g) = 32 cb + 8 (v / 4) + 4 g + v % 4 (the channel lane holds in register v)
  for (int mb = 0; mb < kL1MB; ++mb)
    for (int p = 0; p < kL1KP; ++p)
      for (int lane = 0; lane < 64; ++lane) {
        const int cb = p / 16, v = p % 16, gg = lane / 32;
        const int ch = 32 * cb + 8 * (v / 4) + 4 * gg + (v % 4);
        out[(mb * kL1KP + p) * 64 + lane] = wperm[(32 * mb + lane % 32) * kL1C + ch];
      }
}

int enc_l1_parts(int64_t Lout) {
  const int f = env_int("MNN_ENC_L1_SWGS");  // tuning override: statistics-pass workgroups
  return (int)std::min<int64_t>(cdiv(cdiv(Lout, 32), 4), f > 0 ? f : 2 * kCUs);
}

namespace {
// Workgroups per batch of the one-launch first level with TPW tasks per wave (0: it does not
// apply): as many as the 32-column tasks need at four waves each, within what the device holds at
// once, with at most TPW tasks per wave.
template <int CIN, bool R, int TPW>
int l1_oneshot_grid(const LaunchCtx& c, int64_t tasks, int B) {
  static const int per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, enc_l1_oneshot_kernel<CIN, R, TPW>, 256,
                                                     0) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    return n;
  }();
  const int64_t resident = (int64_t)per_cu * c.dev->props.multiProcessorCount / B;
  const int64_t G = std::min<int64_t>(cdiv(tasks, 4), resident);
  if (G < 1 || G > kL1MaxParts || B > kXmMaxBatch || G * B > kL1MaxSlots ||
      cdiv(tasks, 4 * G) > TPW)
    return 0;
  return (int)G;
}

// One task per wave where the device holds enough waves at once, else two.
template <int CIN, bool R>
bool l1_oneshot(const LaunchCtx& c, const EncL1Args& p, const EncL1KArgs& a) {
  if (!p.xch) return false;
  const int64_t tasks = cdiv(p.Lout, 32);
  auto go = [&](auto kern, int G) {
    launch(c, level_name("enc_l1_oneshot_f32", p.C).c_str(), kern, dim3((unsigned)G, p.B),
           dim3(256), 0, a, static_cast<unsigned long long*>(p.xch), std::max(p.spin_limit, 0));
  };
  if (const int G = l1_oneshot_grid<CIN, R, 1>(c, tasks, p.B)) {
    go(enc_l1_oneshot_kernel<CIN, R, 1>, G);
    return true;
  }
  if (const int G = l1_oneshot_grid<CIN, R, kL1MaxTPW>(c, tasks, p.B)) {
    go(enc_l1_oneshot_kernel<CIN, R, kL1MaxTPW>, G);
    return true;
  }
  return false;
}
}  // namespace

void enc_l1(const LaunchCtx& c, const EncL1Args& p) {
  MNN_REQUIRE(enc_l1_supported(p.Cin, p.C, 8, 4, 1, 1, p.pad, p.L) && (p.parts || p.xch) &&
                  p.a_rw && p.rb && p.w1 && p.out && p.ldo >= p.Lout && p.Lout >= 1 &&
                  (p.Lout - 1) * 4 + 8 <= p.L + 2 * p.pad,
              MNN_ERR_INVALID_ARGUMENT, "enc_l1: unsupported configuration");
  EncL1KArgs a;
  a.C = p.C;
  a.Cin = p.Cin;
  a.pad = p.pad;
  a.L = p.L;
  a.Lout = p.Lout;
  a.ldo = p.ldo;
  a.eps = p.eps;
  a.x = p.x;
  a.w1 = p.w1;
  a.b1 = p.b1;
  a.gamma = p.gamma;
  a.beta = p.beta;
  a.parts = p.parts;
  a.a_rw = p.a_rw;
  a.rb = p.rb;
  a.out = p.out;
  {
    bool done = false;
    switch (p.Cin * 2 + (p.reflect ? 1 : 0)) {
      case 2: done = l1_oneshot<1, false>(c, p, a); break;
      case 3: done = l1_oneshot<1, true>(c, p, a); break;
      case 4: done = l1_oneshot<2, false>(c, p, a); break;
      case 5: done = l1_oneshot<2, true>(c, p, a); break;
      case 6: done = l1_oneshot<3, false>(c, p, a); break;
      case 7: done = l1_oneshot<3, true>(c, p, a); break;
      case 8: done = l1_oneshot<4, false>(c, p, a); break;
      default: done = l1_oneshot<4, true>(c, p, a); break;
    }
    if (done) return;
  }
  MNN_REQUIRE(p.parts, MNN_ERR_INVALID_ARGUMENT, "enc_l1: the two-pass form needs a workspace");
  const int64_t tasks = cdiv(p.Lout, 32);
  {  // statistics pass: one partial per workgroup
    a.nparts = enc_l1_parts(p.Lout);
    dim3 sgrid((unsigned)a.nparts, p.B), block(256);
    const std::string sname = level_name("enc_l1_stats_f32", p.C);
#define MNN_L1S(CIN, R) launch(c, sname.c_str(), enc_l1_stats_kernel<CIN, R>, sgrid, block, 0, a)
    switch (p.Cin * 2 + (p.reflect ? 1 : 0)) {
      case 2: MNN_L1S(1, false); break;
      case 3: MNN_L1S(1, true); break;
      case 4: MNN_L1S(2, false); break;
      case 5: MNN_L1S(2, true); break;
      case 6: MNN_L1S(3, false); break;
      case 7: MNN_L1S(3, true); break;
      case 8: MNN_L1S(4, false); break;
      default: MNN_L1S(4, true); break;
    }
#undef MNN_L1S
  }
  const int fw = env_int("MNN_ENC_L1_WGS");  // tuning override: fused-pass workgroups
  dim3 grid((unsigned)std::min<int64_t>(cdiv(tasks, 4), fw > 0 ? fw : 2 * kCUs), p.B), block(256);
  const std::string fname = level_name("enc_l1_fused_f32", p.C);
#define MNN_L1(CIN, R) launch(c, fname.c_str(), enc_l1_fused_kernel<CIN, R>, grid, block, 0, a)
  switch (p.Cin * 2 + (p.reflect ? 1 : 0)) {
    case 2: return MNN_L1(1, false);
    case 3: return MNN_L1(1, true);
    case 4: return MNN_L1(2, false);
    case 5: return MNN_L1(2, true);
    case 6: return MNN_L1(3, false);
    case 7: return MNN_L1(3, true);
    case 8: return MNN_L1(4, false);
    default: return MNN_L1(4, true);
  }
#undef MNN_L1
}

int enc_rewrite_kp(int C) { return (C + 31) / 32 * 32; }

void enc_rewrite(const LaunchCtx& c, const EncRewriteArgs& p) {
  MNN_REQUIRE(p.C % 16 == 0 && p.C > 0 && p.kp == enc_rewrite_kp(p.C) && p.zt && p.w && p.bias &&
                  p.ldo >= p.Lout &&
                  (p.zt_ready || (p.ldy >= p.Lout && ((p.parts && p.nparts > 0) || p.coef))),
              MNN_ERR_INVALID_ARGUMENT, "enc_rewrite: unsupported configuration");
  if (!p.zt_ready) {
    // about 1024 workgroups in all, each with the same number of tiles
    const int64_t tiles = (int64_t)cdiv(p.Lout, kTT) * cdiv(p.kp, kTT);
    const int64_t per = cdiv(tiles, std::max<int64_t>(1, 1024 / p.B));
    launch(c, level_name("enc_gn_gelu_t_f32", p.C).c_str(), enc_gn_gelu_t_kernel,
           dim3((unsigned)cdiv(tiles, per), 1, p.B), dim3(256), 0, p);
  }
  GemmArgs g;
  g.M = 2 * p.C;
  g.N = (int)p.Lout;
  g.K = p.kp;
  g.batch = p.B;
  g.A = p.w;
  g.lda = p.kp;
  g.B = p.zt;
  g.ldb = p.kp;
  g.sB = (int64_t)p.Lout * p.kp;
  g.blayout = B_NK;
  g.C = p.out;
  g.ldc = p.ldo;
  g.sC = (int64_t)p.C * p.ldo;
  g.bias = p.bias;
  g.bias_mode = BIAS_M;
  g.glu = true;
  const std::string rname = level_name("enc_rewrite_f32", p.C);
  g.name = rname.c_str();
  MNN_REQUIRE(gemm_nk_lds_supported(g), MNN_ERR_INVALID_ARGUMENT,
              "enc_rewrite: operands outside the LDS GEMM's contract");
  gemm_nk_lds(c, g);
}

}  // namespace k
}  // namespace mnn
