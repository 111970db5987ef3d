// GEMM on the CDNA4 matrix cores, fp32 accumulation. fp32 operands use v_mfma_f32_32x32x2_f32;
// with precision BF16 the operands are rounded to bf16 (round to nearest even) as they are read
// from LDS and multiplied with v_mfma_f32_32x32x16_bf16 (HalfLinear's fp16-in/fp32-accumulate
// contract, HalfPrecisionLinear.swift:60-212, with bf16). Modes without a bf16 form run in fp32.
//
// C[b] = epilogue(A[b] * B[b]) with A [M][K] row-major and these operand modes for B:
//   B_NK    : B^T stored [N][K] (Linear / attention projections, PyTorch weight layout;
//             Linear.swift:337-352 computes y = x W^T + b),
//   B_KN(4) : B stored [K][N] (1x1 convolution over [C][L] activations); the "4" form loads
//             16-byte vectors when rows are 16-byte aligned (padded pitch),
//   B_CONV  : implicit im2col of a [Cin][L] signal (strided Conv1D with zero or reflect padding,
//             DynamicConv1D.swift:288-324,358-401), gathered element by element,
//   B_CONVW : the same for kernel 8 / stride 4 / dilation 1 (the HTDemucs encoder conv): the raw
//             signal window of 4 channels is staged in LDS and each lane reads its 8 taps as two
//             16-byte LDS reads, so im2col exists neither in HBM nor in LDS.
// Fusions: per-k affine + activation on B while it is loaded (GroupNorm-apply + GELU of the
// producer), epilogues bias (per N or per M), activation, GLU over row pairs, residual with
// per-column LayerScale, and GroupNorm(1) partial statistics of the output.
//
// Tiling: workgroup = WAVES_M x WAVES_N waves, each wave owns WM x WN blocks of 32x32 outputs.
// K advances in steps of 32 through one LDS buffer; the next step's global loads are issued
// before the matrix cores start on the current step, and several workgroups share a CU.
// Within a K step, lane group g = lane/32 owns k in [16g, 16g+16): the MFMA's two k slots are
// fed k = s and 16 + s in sub-step s. A and B use the same assignment, so the sum over k is
// unchanged, and each lane reads its 16 k values of a row with four 16-byte LDS reads.
// Workgroups are renumbered so that the ones the hardware places on the same XCD (round robin
// over 8 XCDs) work on neighbouring tiles that share an operand panel in that XCD's L2.
// Long-K GEMMs that cannot fill the chip (the encoder's deeper levels) use 128-deep K steps so
// each step's loads are covered by four times as much matrix work.
#include <cstdlib>

#include "device_utils.hpp"
#include "kernels.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int PADK = 4;  // LDS row padding (floats) for [row][k] tiles
constexpr int kXcds = 8;

template <int WAVES_M, int WAVES_N, int WM, int WN, int BMODE, int BK>
struct GemmCfg {
  static constexpr int BM = WAVES_M * WM * 32;
  static constexpr int BN = WAVES_N * WN * 32;
  static constexpr int NT = WAVES_M * WAVES_N * 64;
  static constexpr int LDA = BK + PADK;
  static constexpr bool KN = BMODE == B_KN || BMODE == B_KN4 || BMODE == B_CONVREC;
  static constexpr int LDB = KN ? (BN + 4) : (BK + PADK);
  // conv window: BK/8 channels x (4*(BN-1) + 8) samples, row pitch WP (multiple of 4)
  static constexpr int WCH = BK / 8;
  static constexpr int WIN = 4 * BN + 4;
  static constexpr int WP = WIN + 4;
  // conv recompute: KPT output channels per thread for one column
  static constexpr int KGROUPS = NT / BN;
  static constexpr int KPT = BK / (KGROUPS > 0 ? KGROUPS : 1);
  static constexpr int A_FLOATS = BM * LDA;
  static constexpr int B_FLOATS = BMODE == B_CONVW ? WCH * WP : (KN ? BK * LDB : BN * LDB);
  static constexpr int A_V4 = BM * BK / 4 / NT;  // float4 per thread per stage
  static constexpr int B_V4 = (BMODE == B_NK || BMODE == B_KN4) ? BN * BK / 4 / NT : 0;
  static constexpr int B_SC = BMODE == B_KN || BMODE == B_CONV ? BN * BK / NT
                              : BMODE == B_CONVW              ? (WCH * WIN + NT - 1) / NT
                              : BMODE == B_CONVREC            ? KPT
                                                              : 0;
  // Prefetch depth: number of K steps whose global loads are in flight in registers. Small
  // tiles (little matrix work per step, few waves per SIMD) need several to cover memory latency.
  static constexpr int STAGE_REGS = 4 * A_V4 + 4 * B_V4 + B_SC;
  static constexpr int NPF = (BMODE == B_KN || BK > 32) ? 1
                             : STAGE_REGS <= 16            ? 4
                             : STAGE_REGS <= 28            ? 2
                                                           : 1;
  static_assert(BM * BK / 4 % NT == 0, "A tile must split evenly over threads");
  static_assert(BN * BK / 4 % NT == 0, "B tile must split evenly over threads");
  static_assert(BMODE != B_CONVREC || (NT % BN == 0 && BK % (NT / BN) == 0),
                "conv recompute needs whole columns per thread group");
};

__device__ __forceinline__ int reflect_index(int p, int L) {
  p = p < 0 ? -p : p;
  return p >= L ? 2 * (L - 1) - p : p;
}

template <int WAVES_M, int WAVES_N, int WM, int WN, int BMODE, int BK, bool BF = false>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64, 2) void gemm_f32_mfma_kernel(GemmArgs a,
                                                                                 int m_fastest) {
  using Cfg = GemmCfg<WAVES_M, WAVES_N, WM, WN, BMODE, BK>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT, LDA = Cfg::LDA, LDB = Cfg::LDB;
  __shared__ __attribute__((aligned(16))) float As[Cfg::A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs[Cfg::B_FLOATS];
  __shared__ float red[3 * (NT / 64)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int bz = blockIdx.z;
  // XCD-aware renumbering of the (N tiles x M tiles) grid
  const int gx = gridDim.x, gy = gridDim.y, total = gx * gy;
  const int lin = blockIdx.x + gx * blockIdx.y;
  const int xcd = lin % kXcds, slot = lin / kXcds;
  const int q = total / kXcds, r = total % kXcds;
  const int logical = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
  int tn, tm;
  if (m_fastest) {
    tm = logical % gy;
    tn = logical / gy;
  } else {
    tn = logical % gx;
    tm = logical / gx;
  }
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = a.M, N = a.N, K = a.K;
  const float* __restrict__ A = a.A + (int64_t)bz * a.sA;
  const float* __restrict__ B = a.B + (int64_t)bz * a.sB;
  const float* __restrict__ coef = a.pro_coef ? a.pro_coef + (int64_t)bz * 2 * K : nullptr;
  // GroupNorm(1) of the producer from its statistics partials (merged here, every workgroup
  // the same way); coefficients per k are then gamma_k * rstd and beta_k - mean * gamma_k * rstd
  float2 gstat = make_float2(0.f, 0.f);
  const bool have_pro = coef != nullptr || a.pro_stats != nullptr;
  if (a.pro_stats) {
    gstat = gn1_merge(a.pro_stats + (int64_t)bz * a.pro_nparts * 3, a.pro_nparts, a.pro_eps,
                      reinterpret_cast<double*>(As));
  }
  auto pro_coef = [&](int gk) -> float2 {
    if (coef) return *reinterpret_cast<const float2*>(coef + 2 * gk);
    const float sc = (a.pro_gamma ? a.pro_gamma[gk] : 1.f) * gstat.y;
    return make_float2(sc, (a.pro_beta ? a.pro_beta[gk] : 0.f) - gstat.x * sc);
  };

  constexpr int NPF = Cfg::NPF;
  float4 ra[NPF][Cfg::A_V4];
  float4 rb4[NPF][Cfg::B_V4 > 0 ? Cfg::B_V4 : 1];
  float rbs[NPF][Cfg::B_SC > 0 ? Cfg::B_SC : 1];

  // conv recompute: this thread's column and its 16-sample input window (2 channels x 8 taps
  // or 1 x 16, any Cin * taps = 16), loaded once for the whole K loop
  float xw[BMODE == B_CONVREC ? 16 : 1];
  int rc_k0 = 0;
  __shared__ __attribute__((aligned(16))) float rcw[BMODE == B_CONVREC ? 17 * 96 : 1];
  if constexpr (BMODE == B_CONVREC) {
    // conv weights of this GEMM's K rows (K <= 96), stored [k][16] with a pad word per row
    for (int e = tid; e < K * 16; e += NT) rcw[(e >> 4) * 17 + (e & 15)] = a.rc_w[e];
    __syncthreads();
    const int ncol = tid % BN;
    rc_k0 = __builtin_amdgcn_readfirstlane((tid / BN) * Cfg::KPT);
    const int gn = n0 + ncol;
    const int L = a.conv_L;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int ci = e / a.conv_ks, kk = e - ci * a.conv_ks;
      const int pos = gn * a.conv_stride - a.conv_pad + kk * a.conv_dil;
      float v = 0.f;
      if (gn < N) {
        if (a.conv_reflect)
          v = B[(int64_t)ci * a.ldb + reflect_index(pos, L)];
        else if (pos >= 0 && pos < L)
          v = B[(int64_t)ci * a.ldb + pos];
      }
      xw[e] = v;
    }
  }

  auto load_tiles = [&](int k0, int ps) {
#pragma unroll
    for (int i = 0; i < Cfg::A_V4; ++i) {
      const int idx = tid + i * NT;
      const int row = idx / (BK / 4), kc = idx % (BK / 4);
      const int gm = m0 + row, gk = k0 + kc * 4;
      ra[ps][i] = (gm < M && gk < K) ? *reinterpret_cast<const float4*>(A + (int64_t)gm * a.lda + gk)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if constexpr (BMODE == B_NK) {
#pragma unroll
      for (int i = 0; i < Cfg::B_V4; ++i) {
        const int idx = tid + i * NT;
        const int row = idx / (BK / 4), kc = idx % (BK / 4);
        const int gn = n0 + row, gk = k0 + kc * 4;
        rb4[ps][i] = (gn < N && gk < K)
                     ? *reinterpret_cast<const float4*>(B + (int64_t)gn * a.ldb + gk)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    } else if constexpr (BMODE == B_KN4) {
      constexpr int NC4 = BN / 4, RPP = NT / NC4;  // float4 per row, rows per pass
#pragma unroll
      for (int i = 0; i < Cfg::B_V4; ++i) {
        const int kr = tid / NC4 + i * RPP, c4 = tid % NC4;
        const int gk = k0 + kr, gn = n0 + 4 * c4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gk < K && gn < N) {
          v = *reinterpret_cast<const float4*>(B + (int64_t)gk * a.ldb + gn);
          if (have_pro) {
            const float2 cf = pro_coef(gk);
            v.x = apply_act(fmaf(v.x, cf.x, cf.y), a.pro_act);
            v.y = apply_act(fmaf(v.y, cf.x, cf.y), a.pro_act);
            v.z = apply_act(fmaf(v.z, cf.x, cf.y), a.pro_act);
            v.w = apply_act(fmaf(v.w, cf.x, cf.y), a.pro_act);
          }
          if (gn + 1 >= N) v.y = 0.f;
          if (gn + 2 >= N) v.z = 0.f;
          if (gn + 3 >= N) v.w = 0.f;
        }
        rb4[ps][i] = v;
      }
    } else if constexpr (BMODE == B_KN) {
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int idx = tid + i * NT;
        const int kr = idx / BN, nc = idx % BN;
        const int gk = k0 + kr, gn = n0 + nc;
        float v = 0.f;
        if (gk < K && gn < N) {
          v = B[(int64_t)gk * a.ldb + gn];
          if (have_pro) {
            const float2 cf = pro_coef(gk);
            v = apply_act(fmaf(v, cf.x, cf.y), a.pro_act);
          }
        }
        rbs[ps][i] = v;
      }
    } else if constexpr (BMODE == B_CONV) {
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int idx = tid + i * NT;
        const int kc = idx % BK, nr = idx / BK;
        const int gk = k0 + kc, gn = n0 + nr;
        float v = 0.f;
        if (gk < K && gn < N) {
          const int ci = gk / a.conv_ks, kk = gk - ci * a.conv_ks;
          const int pos = gn * a.conv_stride - a.conv_pad + kk * a.conv_dil;
          if (a.conv_reflect)
            v = B[(int64_t)ci * a.ldb + reflect_index(pos, a.conv_L)];
          else if (pos >= 0 && pos < a.conv_L)
            v = B[(int64_t)ci * a.ldb + pos];
        }
        rbs[ps][i] = v;
      }
    } else if constexpr (BMODE == B_CONVREC) {
      // KPT consecutive output channels of one column; conv weights/bias/coefficients are
      // uniform across the wave (scalar loads)
      const int ncol = tid % BN;
      const bool colok = n0 + ncol < N;
#pragma unroll
      for (int i = 0; i < Cfg::KPT; ++i) {
        const int gk = k0 + rc_k0 + i;
        float v = 0.f;
        if (gk < K) {
          const float* wr = rcw + gk * 17;
          float acc = a.rc_b ? a.rc_b[gk] : 0.f;
#pragma unroll
          for (int e = 0; e < 16; ++e) acc = fmaf(xw[e], wr[e], acc);
          const float2 cf = pro_coef(gk);
          v = colok ? apply_act(fmaf(acc, cf.x, cf.y), a.pro_act) : 0.f;
        }
        rbs[ps][i] = v;
      }
    } else {  // B_CONVW: window of WCH channels starting at channel k0/8
      const int ci0 = k0 >> 3;
      const int pos0 = n0 * 4 - a.conv_pad;
      const int L = a.conv_L;
      const int plim = L - 1 + a.conv_pad;  // no valid output needs a sample beyond this
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int e = tid + i * NT;
        const int c = e / Cfg::WIN, j = e - c * Cfg::WIN;
        float v = 0.f;
        const int p = pos0 + j;
        if (c < Cfg::WCH && ci0 + c < (K >> 3) && p <= plim) {
          if (a.conv_reflect)
            v = B[(int64_t)(ci0 + c) * a.ldb + reflect_index(p, L)];
          else if (p >= 0 && p < L)
            v = B[(int64_t)(ci0 + c) * a.ldb + p];
        }
        rbs[ps][i] = v;
      }
    }
  };

  auto store_tiles = [&](int ps) {
#pragma unroll
    for (int i = 0; i < Cfg::A_V4; ++i) {
      const int idx = tid + i * NT;
      const int row = idx / (BK / 4), kc = idx % (BK / 4);
      *reinterpret_cast<float4*>(As + row * LDA + kc * 4) = ra[ps][i];
    }
    if constexpr (BMODE == B_NK) {
#pragma unroll
      for (int i = 0; i < Cfg::B_V4; ++i) {
        const int idx = tid + i * NT;
        const int row = idx / (BK / 4), kc = idx % (BK / 4);
        *reinterpret_cast<float4*>(Bs + row * LDB + kc * 4) = rb4[ps][i];
      }
    } else if constexpr (BMODE == B_KN4) {
      constexpr int NC4 = BN / 4, RPP = NT / NC4;
#pragma unroll
      for (int i = 0; i < Cfg::B_V4; ++i) {
        const int kr = tid / NC4 + i * RPP, c4 = tid % NC4;
        *reinterpret_cast<float4*>(Bs + kr * LDB + 4 * c4) = rb4[ps][i];
      }
    } else if constexpr (BMODE == B_KN) {
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int idx = tid + i * NT;
        Bs[(idx / BN) * LDB + (idx % BN)] = rbs[ps][i];
      }
    } else if constexpr (BMODE == B_CONV) {
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int idx = tid + i * NT;
        Bs[(idx / BK) * LDB + (idx % BK)] = rbs[ps][i];
      }
    } else if constexpr (BMODE == B_CONVREC) {
      const int ncol = tid % BN;
#pragma unroll
      for (int i = 0; i < Cfg::KPT; ++i) Bs[(rc_k0 + i) * LDB + ncol] = rbs[ps][i];
    } else {
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int e = tid + i * NT;
        const int c = e / Cfg::WIN, j = e - c * Cfg::WIN;
        if (c < Cfg::WCH) Bs[c * Cfg::WP + j] = rbs[ps][i];
      }
    }
  };

  // Independent accumulator chains: with fewer than 3 output blocks per wave, consecutive
  // k sub-steps rotate over NCH copies so back-to-back MFMAs never wait on each other's result.
  constexpr int NCH = WM * WN >= 3 ? 1 : (WM * WN == 2 ? 2 : 4);
  floatx16 acc[NCH][WM][WN];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[c][i][j][v] = 0.f;

  const int g = lane >> 5, l32 = lane & 31;
  const int arow0 = wm * WM * 32 + l32;
  const int bcol0 = wn * WN * 32 + l32;

  const int nk = (K + BK - 1) / BK;
#pragma unroll
  for (int ps = 0; ps < NPF; ++ps)
    if (ps < nk) load_tiles(ps * BK, ps);
  for (int kt0 = 0; kt0 < nk; kt0 += NPF) {
#pragma unroll
    for (int ps = 0; ps < NPF; ++ps) {
    const int kt = kt0 + ps;
    if (kt >= nk) break;
    if (kt > 0) __syncthreads();  // everyone is done reading the previous step
    store_tiles(ps);
    __syncthreads();
    if (kt + NPF < nk) load_tiles((kt + NPF) * BK, ps);  // in flight for NPF steps

#pragma unroll
    for (int kb = 0; kb < BK / 32; ++kb) {
      if constexpr (BF) {
        // bf16 operands (rounded to nearest even from the fp32 tiles), fp32 accumulation:
        // v_mfma_f32_32x32x16_bf16, lane group g supplies k in [kq, kq + 8) of each step
#pragma unroll
        for (int s8 = 0; s8 < 2; ++s8) {
          const int kq = 32 * kb + 16 * g + 8 * s8;
          bf16x8 a8[WM], b8[WN];
#pragma unroll
          for (int i = 0; i < WM; ++i) {
            const float* p = As + (arow0 + i * 32) * LDA + kq;
            const float4 t0 = *reinterpret_cast<const float4*>(p);
            const float4 t1 = *reinterpret_cast<const float4*>(p + 4);
            a8[i] = bf16x8{(__bf16)t0.x, (__bf16)t0.y, (__bf16)t0.z, (__bf16)t0.w,
                           (__bf16)t1.x, (__bf16)t1.y, (__bf16)t1.z, (__bf16)t1.w};
          }
#pragma unroll
          for (int j = 0; j < WN; ++j) {
            float v[8];
            if constexpr (Cfg::KN) {
#pragma unroll
              for (int t = 0; t < 8; ++t) v[t] = Bs[(kq + t) * LDB + bcol0 + j * 32];
            } else {
              const float* p = BMODE == B_CONVW
                                   ? Bs + (kq >> 3) * Cfg::WP + 4 * (bcol0 + j * 32)
                                   : Bs + (bcol0 + j * 32) * LDB + kq;
              const float4 t0 = *reinterpret_cast<const float4*>(p);
              const float4 t1 = *reinterpret_cast<const float4*>(p + 4);
              v[0] = t0.x; v[1] = t0.y; v[2] = t0.z; v[3] = t0.w;
              v[4] = t1.x; v[5] = t1.y; v[6] = t1.z; v[7] = t1.w;
            }
            b8[j] = bf16x8{(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3],
                           (__bf16)v[4], (__bf16)v[5], (__bf16)v[6], (__bf16)v[7]};
          }
#pragma unroll
          for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
              acc[s8 % NCH][i][j] =
                  __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8[i], b8[j], acc[s8 % NCH][i][j], 0, 0, 0);
        }
        continue;
      }
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {  // four groups of four k sub-steps
        const int kq = 32 * kb + 16 * g + 4 * q4;  // first k of this lane's group
        float af[WM][4];
        float bf[WN][4];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
          const float4 t = *reinterpret_cast<const float4*>(As + (arow0 + i * 32) * LDA + kq);
          af[i][0] = t.x; af[i][1] = t.y; af[i][2] = t.z; af[i][3] = t.w;
        }
        if constexpr (Cfg::KN) {
#pragma unroll
          for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s) bf[j][s] = Bs[(kq + s) * LDB + bcol0 + j * 32];
        } else if constexpr (BMODE == B_CONVW) {
          // k = kq + s -> channel kq/8, tap kq%8 + s, window sample 4n + tap
#pragma unroll
          for (int j = 0; j < WN; ++j) {
            const float4 t = *reinterpret_cast<const float4*>(
                Bs + (kq >> 3) * Cfg::WP + 4 * (bcol0 + j * 32) + (kq & 7));
            bf[j][0] = t.x; bf[j][1] = t.y; bf[j][2] = t.z; bf[j][3] = t.w;
          }
        } else {
#pragma unroll
          for (int j = 0; j < WN; ++j) {
            const float4 t = *reinterpret_cast<const float4*>(Bs + (bcol0 + j * 32) * LDB + kq);
            bf[j][0] = t.x; bf[j][1] = t.y; bf[j][2] = t.z; bf[j][3] = t.w;
          }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
              acc[s % NCH][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                  af[i][s], bf[j][s], acc[s % NCH][i][j], 0, 0, 0);
      }
    }
    }
  }

#pragma unroll
  for (int c = 1; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[0][i][j] += acc[c][i][j];

  // ---------------------------------------------------------------- epilogue
  // accumulator layout (32x32 block): lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32
  float* __restrict__ Cp = a.C + (int64_t)bz * a.sC;
  const float* __restrict__ Rp = a.R ? a.R + (int64_t)bz * a.sR : nullptr;
  ShiftedStats st;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int mblk = m0 + wm * WM * 32 + i * 32;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int gn = n0 + wn * WN * 32 + j * 32 + l32;
      if (a.glu) {
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int rr = 8 * (v / 4) + 4 * g + (v % 4);  // < 16
          const int gm = mblk + rr;
          if (gm < M && gn < N) {
            float va = acc[0][i][j][v], vb = acc[0][i][j][v + 8];
            if (a.bias_mode == BIAS_M) {
              va += a.bias[gm];
              vb += a.bias[gm + 16];
            } else if (a.bias_mode == BIAS_N) {
              va += a.bias[gn];
              vb += a.bias[gn];
            }
            const int orow = (mblk / 32) * 16 + rr;
            Cp[(int64_t)orow * a.ldc + gn] = va * stable_sigmoid(vb);
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
          if (gm < M && gn < N) {
            float val = acc[0][i][j][v];
            if (a.bias_mode == BIAS_N) val += a.bias[gn];
            else if (a.bias_mode == BIAS_M) val += a.bias[gm];
            if (a.stats) st.add(val);
            val = apply_act(val, a.act, a.act_alpha);
            if (Rp) {
              const float rs = a.rscale ? a.rscale[gn] : 1.f;
              val = Rp[(int64_t)gm * a.ldr + gn] + rs * val;
            }
            Cp[(int64_t)gm * a.ldc + gn] = val;
          }
        }
      }
    }
  }
  if (a.stats) {
    float sn, smean, sm2;
    st.finish(sn, smean, sm2);
    block_welford(sn, smean, sm2, red);
    if (tid == 0) {
      float* o = a.stats + ((int64_t)bz * total + tm * gx + tn) * 3;
      o[0] = sn;
      o[1] = smean;
      o[2] = sm2;
    }
  }
}

// Fallback for shapes the MFMA path does not take (K or leading dimensions not multiples of 4,
// unaligned pointers): one thread per output, fp32 FMA. Same epilogue semantics except GLU.
__global__ __launch_bounds__(256) void gemm_f32_simple_kernel(GemmArgs a) {
  __shared__ float red[3 * 4];
  const int bz = blockIdx.z;
  const int gn = blockIdx.x * 16 + (threadIdx.x & 15);
  const int gm = blockIdx.y * 16 + (threadIdx.x >> 4);
  const float* A = a.A + (int64_t)bz * a.sA;
  const float* B = a.B + (int64_t)bz * a.sB;
  const float* coef = a.pro_coef ? a.pro_coef + (int64_t)bz * 2 * a.K : nullptr;
  float sn = 0.f, smean = 0.f, sm2 = 0.f;
  if (gm < a.M && gn < a.N) {
    float acc = 0.f;
    for (int kk = 0; kk < a.K; ++kk) {
      float bv;
      if (a.blayout == B_NK) {
        bv = B[(int64_t)gn * a.ldb + kk];
      } else if (a.blayout == B_KN || a.blayout == B_KN4) {
        bv = B[(int64_t)kk * a.ldb + gn];
        if (coef) bv = apply_act(fmaf(bv, coef[2 * kk], coef[2 * kk + 1]), a.pro_act);
      } else {
        const int ci = kk / a.conv_ks, t = kk - ci * a.conv_ks;
        const int pos = gn * a.conv_stride - a.conv_pad + t * a.conv_dil;
        if (a.conv_reflect)
          bv = B[(int64_t)ci * a.ldb + reflect_index(pos, a.conv_L)];
        else
          bv = (pos >= 0 && pos < a.conv_L) ? B[(int64_t)ci * a.ldb + pos] : 0.f;
      }
      acc = fmaf(A[(int64_t)gm * a.lda + kk], bv, acc);
    }
    if (a.bias_mode == BIAS_N) acc += a.bias[gn];
    else if (a.bias_mode == BIAS_M) acc += a.bias[gm];
    if (a.stats) {
      sn = 1.f;
      smean = acc;
    }
    acc = apply_act(acc, a.act, a.act_alpha);
    if (a.R) {
      const float rs = a.rscale ? a.rscale[gn] : 1.f;
      acc = a.R[(int64_t)bz * a.sR + (int64_t)gm * a.ldr + gn] + rs * acc;
    }
    a.C[(int64_t)bz * a.sC + (int64_t)gm * a.ldc + gn] = acc;
  }
  if (a.stats) {
    block_welford(sn, smean, sm2, red);
    if (threadIdx.x == 0) {
      const int tiles = gridDim.x * gridDim.y;
      float* o = a.stats + ((int64_t)bz * tiles + blockIdx.y * gridDim.x + blockIdx.x) * 3;
      o[0] = sn;
      o[1] = smean;
      o[2] = sm2;
    }
  }
}

// ---------------------------------------------------------------- host-side planning
struct Tile {
  int id;       // index into kTiles, -1 = simple kernel
  int bm, bn, nt;
  int bk;       // K step: 32, or 128 for long-K problems that leave SIMDs under-occupied
};

// (WAVES_M, WAVES_N, WM, WN) configurations compiled below, and their tile sizes.
constexpr Tile kTiles[] = {
    {0, 128, 128, 256, 32},  // <2,2,2,2>
    {1, 64, 128, 256, 32},   // <2,2,1,2>
    {2, 128, 64, 256, 32},   // <2,2,2,1>
    {3, 64, 64, 256, 32},    // <2,2,1,1>
    {4, 96, 128, 256, 32},   // <1,4,3,1>
    {5, 96, 64, 128, 32},    // <1,2,3,1>
    {6, 32, 64, 128, 32},    // <1,2,1,1>
};

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

bool mfma_ok(const GemmArgs& a) {
  if (a.K % 4 != 0 || a.lda % 4 != 0 || a.sA % 4 != 0 || !aligned16(a.A)) return false;
  if (a.blayout == B_NK && (a.ldb % 4 != 0 || a.sB % 4 != 0 || !aligned16(a.B))) return false;
  if (a.glu && (a.M % 32 != 0)) return false;
  return true;
}

// The operand mode actually launched (vectorised / windowed forms when the operands allow).
int effective_layout(const GemmArgs& a) {
  if (a.blayout == B_KN && a.ldb % 4 == 0 && a.sB % 4 == 0 && aligned16(a.B) &&
      a.ldb >= ((a.N + 3) / 4) * 4)
    return B_KN4;
  if (a.blayout == B_CONV && a.conv_ks == 8 && a.conv_stride == 4 && a.conv_dil == 1 &&
      a.K % 32 == 0 && a.conv_pad < a.conv_L)
    return B_CONVW;
  return a.blayout;
}

// Per-CU critical path in MFMA units: tiles per CU x tile area x K, divided by an efficiency
// that grows with the number of waves a SIMD can interleave (and with the K step depth, which
// hides memory latency when there are few waves); plus the operand traffic.
int forced_tile() {
  static const int v = [] {
    const char* e = std::getenv("MNN_GEMM_TILE");
    return e ? std::atoi(e) : -1;
  }();
  return v;
}

Tile choose_tiles(const GemmArgs& a) {
  if (!mfma_ok(a)) return {-1, 16, 16, 256, 32};
  if (const int f = forced_tile(); f >= 0 && f < (int)(sizeof(kTiles) / sizeof(kTiles[0]))) {
    const Tile& t = kTiles[f];
    const bool ok = !(a.glu && t.bm % 32) &&
                    !(t.bm == 96 && a.M % 96) &&
                    !(a.blayout == B_CONVREC && !(t.id == 3 || t.id == 4 || t.id == 5));
    if (ok) return t;
  }
  const int lay = effective_layout(a);
  const int cus = 256;
  double best = 1e300;
  Tile pick = kTiles[0];
  for (const Tile& t0 : kTiles) {
    if (a.glu && t0.bm % 32 != 0) continue;
    if (t0.bm == 96 && !(a.M % 96 == 0 && a.M <= 192)) continue;
    if (lay == B_CONVREC && !(t0.id == 4 || t0.id == 5 || t0.id == 3)) continue;
    for (int bk : {32}) {  // 128-deep steps are built but not chosen (slower on the encoder shapes)
      Tile t = t0;
      t.bk = bk;
      if (bk == 128) {
        // deep steps only on the small-tile configurations, for the modes instantiated with them
        if (!(t.id == 3 || t.id == 6)) continue;
        if (!(lay == B_NK || lay == B_KN4 || lay == B_CONVW)) continue;
        if (a.K < 256) continue;
        if (lay == B_CONVW && a.K % 128 != 0) continue;
      }
      const int64_t tiles =
          (int64_t)((a.M + t.bm - 1) / t.bm) * ((a.N + t.bn - 1) / t.bn) * a.batch;
      const int64_t per_cu = (tiles + cus - 1) / cus;
      const int waves_wg = t.nt / 64;
      const double waves_simd = std::min<double>((double)per_cu, 4.0) * waves_wg / 4.0;
      double eff = waves_simd >= 3 ? 1.0 : waves_simd >= 2 ? 0.9 : waves_simd >= 1 ? 0.65 : 0.35;
      if (bk == 128) eff = std::min(1.0, eff + (waves_simd >= 1 ? 0.2 : 0.3));
      const double work = (double)per_cu * t.bm * t.bn;
      const double traffic = (double)per_cu * (t.bm + t.bn) * 8.0;
      const double cost = (work / eff + traffic) * (double)a.K;
      if (cost < best * 0.999) {
        best = cost;
        pick = t;
      }
    }
  }
  return pick;
}

template <int WAVES_M, int WAVES_N, int WM, int WN, int BK>
void launch_mode(const LaunchCtx& c, const GemmArgs& a, dim3 grid, dim3 block, int lay,
                 int m_fastest) {
  if (a.precision == MNN_PRECISION_BF16 && BK == 32 &&
      (lay == B_NK || lay == B_KN4 || lay == B_CONVW)) {
    switch (lay) {
      case B_NK:
        return launch(c, "gemm_bf16_mfma_nk",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_NK, 32, true>, grid, block,
                      0, a, m_fastest);
      case B_KN4:
        return launch(c, "gemm_bf16_mfma_kn",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_KN4, 32, true>, grid,
                      block, 0, a, m_fastest);
      default:
        return launch(c, "gemm_bf16_mfma_conv",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_CONVW, 32, true>, grid,
                      block, 0, a, m_fastest);
    }
  }
  if constexpr (BK == 128) {
    switch (lay) {
      case B_NK:
        return launch(c, "gemm_f32_mfma_nk",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_NK, 128>, grid, block, 0,
                      a, m_fastest);
      case B_KN4:
        return launch(c, "gemm_f32_mfma_kn",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_KN4, 128>, grid, block, 0,
                      a, m_fastest);
      default:
        return launch(c, "gemm_f32_mfma_conv",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_CONVW, 128>, grid, block,
                      0, a, m_fastest);
    }
  } else {
    switch (lay) {
      case B_NK:
        return launch(c, "gemm_f32_mfma_nk",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_NK, 32>, grid, block, 0, a,
                      m_fastest);
      case B_KN4:
        return launch(c, "gemm_f32_mfma_kn",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_KN4, 32>, grid, block, 0,
                      a, m_fastest);
      case B_KN:
        return launch(c, "gemm_f32_mfma_kn",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_KN, 32>, grid, block, 0, a,
                      m_fastest);
      case B_CONVW:
        return launch(c, "gemm_f32_mfma_conv",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_CONVW, 32>, grid, block, 0,
                      a, m_fastest);
      case B_CONVREC:
        if constexpr ((WAVES_M == 2 && WAVES_N == 2 && WM == 1 && WN == 1) ||
                      (WAVES_M == 1 && WM == 3 && WN == 1))
          return launch(c, "gemm_f32_mfma_convrec",
                        gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_CONVREC, 32>, grid, block,
                        0, a, m_fastest);
        fail(MNN_ERR_INVALID_CONFIGURATION, "conv-recompute GEMM: unsupported tile");
      default:
        return launch(c, "gemm_f32_mfma_conv",
                      gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_CONV, 32>, grid, block, 0,
                      a, m_fastest);
    }
  }
}

template <int WAVES_M, int WAVES_N, int WM, int WN>
void launch_cfg(const LaunchCtx& c, const GemmArgs& a, const Tile& t) {
  dim3 grid(cdiv(a.N, t.bn), cdiv(a.M, t.bm), a.batch), block(WAVES_M * WAVES_N * 64);
  const int lay = effective_layout(a);
  const int m_fastest = lay != B_NK;  // activation-sized B: neighbours share the B panel
  if (t.bk == 128) {
    if constexpr ((WAVES_M == 2 && WAVES_N == 2 && WM == 1 && WN == 1) ||
                  (WAVES_M == 1 && WAVES_N == 2 && WM == 1 && WN == 1))
      return launch_mode<WAVES_M, WAVES_N, WM, WN, 128>(c, a, grid, block, lay, m_fastest);
    fail(MNN_ERR_INVALID_CONFIGURATION, "gemm: 128-deep K step not built for this tile");
  }
  launch_mode<WAVES_M, WAVES_N, WM, WN, 32>(c, a, grid, block, lay, m_fastest);
}

}  // namespace

int gemm_num_tiles(const GemmArgs& a) {
  MNN_REQUIRE(!gemm_nk_lds_supported(a), MNN_ERR_INVALID_ARGUMENT,
              "gemm_num_tiles: only GEMMs with per-tile statistics have a tile count");
  const Tile t = choose_tiles(a);
  return (int)(cdiv(a.N, t.bn) * cdiv(a.M, t.bm));
}

void gemm(const LaunchCtx& c, const GemmArgs& a) {
  if (a.M <= 0 || a.N <= 0 || a.batch <= 0) return;
  MNN_REQUIRE(a.K > 0, MNN_ERR_INVALID_ARGUMENT, "gemm: K must be positive");
  if (gemm_nk_lds_supported(a)) return gemm_nk_lds(c, a);
  MNN_REQUIRE(!a.ln_parts && !a.row_parts, MNN_ERR_INVALID_CONFIGURATION,
              "gemm: folded LayerNorm / row statistics need the LDS-DMA path's operand contract");
  const Tile t = choose_tiles(a);
  MNN_REQUIRE(!(a.glu && t.id < 0), MNN_ERR_INVALID_CONFIGURATION,
              "gemm: GLU epilogue needs M % 32 == 0 and 16-byte aligned operands");
  MNN_REQUIRE(!(a.blayout == B_CONVREC && (t.id < 0 || a.K > 96)), MNN_ERR_INVALID_CONFIGURATION,
              "gemm: conv-recompute operand needs 16-byte aligned weights, K % 4 == 0, K <= 96");
  MNN_REQUIRE(!(a.pro_stats && t.id < 0), MNN_ERR_INVALID_CONFIGURATION,
              "gemm: GroupNorm statistics prologue needs the matrix-core path");
  switch (t.id) {
    case 0: return launch_cfg<2, 2, 2, 2>(c, a, t);
    case 1: return launch_cfg<2, 2, 1, 2>(c, a, t);
    case 2: return launch_cfg<2, 2, 2, 1>(c, a, t);
    case 3: return launch_cfg<2, 2, 1, 1>(c, a, t);
    case 4: return launch_cfg<1, 4, 3, 1>(c, a, t);
    case 5: return launch_cfg<1, 2, 3, 1>(c, a, t);
    case 6: return launch_cfg<1, 2, 1, 1>(c, a, t);
    default: {
      dim3 grid(cdiv(a.N, 16), cdiv(a.M, 16), a.batch);
      return launch(c, "gemm_f32_simple", gemm_f32_simple_kernel, grid, dim3(256), 0, a);
    }
  }
}

}  // namespace k
}  // namespace mnn
