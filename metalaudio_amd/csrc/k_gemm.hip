// GEMM on the CDNA4 matrix cores, fp32 operands (v_mfma_f32_32x32x2_f32), fp32 accumulation.
//
// C[b] = epilogue(A[b] * B[b]) with A [M][K] row-major and three operand modes for B:
//   B_NK   : B^T stored [N][K] (Linear / attention projections, PyTorch weight layout,
//            Linear.swift:337-352 computes y = x W^T + b),
//   B_KN   : B stored [K][N] (1x1 convolution over [C][L] activations),
//   B_CONV : implicit im2col of a [Cin][L] signal (strided Conv1D with zero or reflect padding,
//            DynamicConv1D.swift:288-324,358-401), never materialised in HBM.
// Fusions: a per-k affine + activation on B while it is loaded (GroupNorm-apply + GELU of the
// producer), and epilogues bias (per N or per M), activation, GLU over row pairs, residual with
// per-column LayerScale, and GroupNorm(1) partial statistics of the output.
//
// Tiling: workgroup = WAVES_M x WAVES_N waves, each wave owns WM x WN blocks of 32x32 outputs.
// K advances in steps of 32 through double-buffered LDS with one barrier per step; the next
// step's global loads are in flight while the matrix cores work on the current one.
// Within a K step, lane group g = lane/32 owns k in [16g, 16g+16): the MFMA's two k slots are
// fed k = s and 16 + s in sub-step s. A and B use the same assignment, so the sum over k is
// unchanged, and each lane reads its 16 k values of a row with four 16-byte LDS reads.
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int BK = 32;
constexpr int PADK = 4;  // LDS row padding (floats) for [row][k] tiles

template <int WAVES_M, int WAVES_N, int WM, int WN, int BMODE>
struct GemmCfg {
  static constexpr int BM = WAVES_M * WM * 32;
  static constexpr int BN = WAVES_N * WN * 32;
  static constexpr int NT = WAVES_M * WAVES_N * 64;
  static constexpr int LDA = BK + PADK;
  static constexpr int LDB = (BMODE == B_KN) ? (BN + 4) : (BK + PADK);
  static constexpr int A_FLOATS = BM * LDA;
  static constexpr int B_FLOATS = (BMODE == B_KN) ? BK * LDB : BN * LDB;
  static constexpr int A_V4 = BM * BK / 4 / NT;  // float4 per thread per stage
  static constexpr int B_V4 = (BMODE == B_NK) ? BN * BK / 4 / NT : 0;
  static constexpr int B_SC = (BMODE != B_NK) ? BN * BK / NT : 0;  // scalars per thread
  static_assert(BM * BK / 4 % NT == 0, "A tile must split evenly over threads");
  static_assert(BN * BK / 4 % NT == 0, "B tile must split evenly over threads");
};

template <int WAVES_M, int WAVES_N, int WM, int WN, int BMODE>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64, 2) void gemm_f32_mfma_kernel(GemmArgs a) {
  using Cfg = GemmCfg<WAVES_M, WAVES_N, WM, WN, BMODE>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NT = Cfg::NT, LDA = Cfg::LDA, LDB = Cfg::LDB;
  __shared__ __attribute__((aligned(16))) float As[2][Cfg::A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs[2][Cfg::B_FLOATS];
  __shared__ float red[3 * (NT / 64)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int bz = blockIdx.z;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int M = a.M, N = a.N, K = a.K;
  const float* __restrict__ A = a.A + (int64_t)bz * a.sA;
  const float* __restrict__ B = a.B + (int64_t)bz * a.sB;
  const float* __restrict__ coef = a.pro_coef ? a.pro_coef + (int64_t)bz * 2 * K : nullptr;

  float4 ra[Cfg::A_V4];
  float4 rb4[Cfg::B_V4 > 0 ? Cfg::B_V4 : 1];
  float rbs[Cfg::B_SC > 0 ? Cfg::B_SC : 1];

  auto load_tiles = [&](int k0) {
#pragma unroll
    for (int i = 0; i < Cfg::A_V4; ++i) {
      const int idx = tid + i * NT;
      const int row = idx / (BK / 4), kc = idx % (BK / 4);
      const int gm = m0 + row, gk = k0 + kc * 4;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const float4*>(A + (int64_t)gm * a.lda + gk)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if constexpr (BMODE == B_NK) {
#pragma unroll
      for (int i = 0; i < Cfg::B_V4; ++i) {
        const int idx = tid + i * NT;
        const int row = idx / (BK / 4), kc = idx % (BK / 4);
        const int gn = n0 + row, gk = k0 + kc * 4;
        rb4[i] = (gn < N && gk < K)
                     ? *reinterpret_cast<const float4*>(B + (int64_t)gn * a.ldb + gk)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
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
          if (coef) v = apply_act(fmaf(v, coef[2 * gk], coef[2 * gk + 1]), a.pro_act);
        }
        rbs[i] = v;
      }
    } else {  // B_CONV
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int idx = tid + i * NT;
        const int kc = idx % BK, nr = idx / BK;
        const int gk = k0 + kc, gn = n0 + nr;
        float v = 0.f;
        if (gk < K && gn < N) {
          const int ci = gk / a.conv_ks, kk = gk - ci * a.conv_ks;
          int pos = gn * a.conv_stride - a.conv_pad + kk * a.conv_dil;
          if (a.conv_reflect) {
            pos = pos < 0 ? -pos : pos;
            pos = pos >= a.conv_L ? 2 * (a.conv_L - 1) - pos : pos;
            v = B[(int64_t)ci * a.ldb + pos];
          } else if (pos >= 0 && pos < a.conv_L) {
            v = B[(int64_t)ci * a.ldb + pos];
          }
        }
        rbs[i] = v;
      }
    }
  };

  auto store_tiles = [&](int buf) {
    float* as = As[buf];
    float* bs = Bs[buf];
#pragma unroll
    for (int i = 0; i < Cfg::A_V4; ++i) {
      const int idx = tid + i * NT;
      const int row = idx / (BK / 4), kc = idx % (BK / 4);
      *reinterpret_cast<float4*>(as + row * LDA + kc * 4) = ra[i];
    }
    if constexpr (BMODE == B_NK) {
#pragma unroll
      for (int i = 0; i < Cfg::B_V4; ++i) {
        const int idx = tid + i * NT;
        const int row = idx / (BK / 4), kc = idx % (BK / 4);
        *reinterpret_cast<float4*>(bs + row * LDB + kc * 4) = rb4[i];
      }
    } else if constexpr (BMODE == B_KN) {
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int idx = tid + i * NT;
        bs[(idx / BN) * LDB + (idx % BN)] = rbs[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < Cfg::B_SC; ++i) {
        const int idx = tid + i * NT;
        bs[(idx / BK) * LDB + (idx % BK)] = rbs[i];
      }
    }
  };

  floatx16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int g = lane >> 5, l32 = lane & 31;
  const int arow0 = wm * WM * 32 + l32;
  const int bcol0 = wn * WN * 32 + l32;

  const int nk = (K + BK - 1) / BK;
  load_tiles(0);
  store_tiles(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles((kt + 1) * BK);

    const float* as = As[cur];
    const float* bs = Bs[cur];
    float af[WM][16];
    float bf[WN][16];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const float* p = as + (arow0 + i * 32) * LDA + 16 * g;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float4 t = *reinterpret_cast<const float4*>(p + 4 * q);
        af[i][4 * q + 0] = t.x; af[i][4 * q + 1] = t.y;
        af[i][4 * q + 2] = t.z; af[i][4 * q + 3] = t.w;
      }
    }
    if constexpr (BMODE == B_KN) {
#pragma unroll
      for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int s = 0; s < 16; ++s) bf[j][s] = bs[(16 * g + s) * LDB + bcol0 + j * 32];
    } else {
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const float* p = bs + (bcol0 + j * 32) * LDB + 16 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float4 t = *reinterpret_cast<const float4*>(p + 4 * q);
          bf[j][4 * q + 0] = t.x; bf[j][4 * q + 1] = t.y;
          bf[j][4 * q + 2] = t.z; bf[j][4 * q + 3] = t.w;
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);

    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  // accumulator layout (32x32 block): lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32
  float* __restrict__ Cp = a.C + (int64_t)bz * a.sC;
  const float* __restrict__ Rp = a.R ? a.R + (int64_t)bz * a.sR : nullptr;
  float sn = 0.f, smean = 0.f, sm2 = 0.f;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int mblk = m0 + wm * WM * 32 + i * 32;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int gn = n0 + wn * WN * 32 + j * 32 + l32;
      if (a.glu) {
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int r = 8 * (v / 4) + 4 * g + (v % 4);  // < 16
          const int gm = mblk + r;
          if (gm < M && gn < N) {
            float va = acc[i][j][v], vb = acc[i][j][v + 8];
            if (a.bias_mode == BIAS_M) {
              va += a.bias[gm];
              vb += a.bias[gm + 16];
            } else if (a.bias_mode == BIAS_N) {
              va += a.bias[gn];
              vb += a.bias[gn];
            }
            const int orow = (mblk / 32) * 16 + r;
            Cp[(int64_t)orow * a.ldc + gn] = va * stable_sigmoid(vb);
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
          if (gm < M && gn < N) {
            float val = acc[i][j][v];
            if (a.bias_mode == BIAS_N) val += a.bias[gn];
            else if (a.bias_mode == BIAS_M) val += a.bias[gm];
            if (a.stats) {
              sn += 1.f;
              float d = val - smean;
              smean += d / sn;
              sm2 += d * (val - smean);
            }
            val = apply_act(val, a.act);
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
    block_welford(sn, smean, sm2, red);
    if (tid == 0) {
      const int tiles = gridDim.x * gridDim.y;
      float* o = a.stats + ((int64_t)bz * tiles + blockIdx.y * gridDim.x + blockIdx.x) * 3;
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
      } else if (a.blayout == B_KN) {
        bv = B[(int64_t)kk * a.ldb + gn];
        if (coef) bv = apply_act(fmaf(bv, coef[2 * kk], coef[2 * kk + 1]), a.pro_act);
      } else {
        const int ci = kk / a.conv_ks, t = kk - ci * a.conv_ks;
        int pos = gn * a.conv_stride - a.conv_pad + t * a.conv_dil;
        if (a.conv_reflect) {
          pos = pos < 0 ? -pos : pos;
          pos = pos >= a.conv_L ? 2 * (a.conv_L - 1) - pos : pos;
          bv = B[(int64_t)ci * a.ldb + pos];
        } else {
          bv = (pos >= 0 && pos < a.conv_L) ? B[(int64_t)ci * a.ldb + pos] : 0.f;
        }
      }
      acc = fmaf(A[(int64_t)gm * a.lda + kk], bv, acc);
    }
    if (a.bias_mode == BIAS_N) acc += a.bias[gn];
    else if (a.bias_mode == BIAS_M) acc += a.bias[gm];
    if (a.stats) {
      sn = 1.f;
      smean = acc;
    }
    acc = apply_act(acc, a.act);
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

struct TileChoice {
  int id;  // 0: 128x128, 1: 64x128, 2: 64x64, 3: 96x128, 4: 32x64, -1: simple
  int bm, bn;
};

bool mfma_ok(const GemmArgs& a) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (a.K % 4 != 0 || a.lda % 4 != 0 || a.sA % 4 != 0 || !al(a.A)) return false;
  if (a.blayout == B_NK && (a.ldb % 4 != 0 || a.sB % 4 != 0 || !al(a.B))) return false;
  if (a.glu && (a.M % 32 != 0)) return false;
  return true;
}

TileChoice choose_tiles(const GemmArgs& a) {
  if (!mfma_ok(a)) return {-1, 16, 16};
  if (a.glu && a.M % 32 != 0) return {-1, 16, 16};
  const int64_t target = 512;  // two workgroups per CU on 256 CUs
  auto tiles = [&](int bm, int bn) {
    return (int64_t)((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn) * a.batch;
  };
  if (a.M == 96 || (a.M % 96 == 0 && a.M <= 192 && a.M % 128 != 0)) {
    if (tiles(96, 128) >= target / 2) return {3, 96, 128};
  }
  const TileChoice order[] = {{0, 128, 128}, {1, 64, 128}, {2, 64, 64}, {4, 32, 64}};
  for (const auto& t : order)
    if (tiles(t.bm, t.bn) >= target) return t;
  return {4, 32, 64};
}

template <int WAVES_M, int WAVES_N, int WM, int WN>
void launch_cfg(const LaunchCtx& c, const GemmArgs& a, int bm, int bn) {
  dim3 grid(cdiv(a.N, bn), cdiv(a.M, bm), a.batch), block(WAVES_M * WAVES_N * 64);
  switch (a.blayout) {
    case B_NK:
      return launch(c, "gemm_f32_mfma_nk", gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_NK>,
                    grid, block, 0, a);
    case B_KN:
      return launch(c, "gemm_f32_mfma_kn", gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_KN>,
                    grid, block, 0, a);
    default:
      return launch(c, "gemm_f32_mfma_conv",
                    gemm_f32_mfma_kernel<WAVES_M, WAVES_N, WM, WN, B_CONV>, grid, block, 0, a);
  }
}

}  // namespace

int gemm_num_tiles(const GemmArgs& a) {
  TileChoice t = choose_tiles(a);
  return (int)(cdiv(a.N, t.bn) * cdiv(a.M, t.bm));
}

void gemm(const LaunchCtx& c, const GemmArgs& a) {
  if (a.M <= 0 || a.N <= 0 || a.batch <= 0) return;
  MNN_REQUIRE(a.K > 0, MNN_ERR_INVALID_ARGUMENT, "gemm: K must be positive");
  TileChoice t = choose_tiles(a);
  MNN_REQUIRE(!(a.glu && t.id < 0), MNN_ERR_INVALID_CONFIGURATION,
              "gemm: GLU epilogue needs M % 32 == 0 and 16-byte aligned operands");
  switch (t.id) {
    case 0: return launch_cfg<2, 2, 2, 2>(c, a, t.bm, t.bn);
    case 1: return launch_cfg<2, 2, 1, 2>(c, a, t.bm, t.bn);
    case 2: return launch_cfg<2, 2, 1, 1>(c, a, t.bm, t.bn);
    case 3: return launch_cfg<1, 4, 3, 1>(c, a, t.bm, t.bn);
    case 4: return launch_cfg<1, 2, 1, 1>(c, a, t.bm, t.bn);
    default: {
      dim3 grid(cdiv(a.N, 16), cdiv(a.M, 16), a.batch);
      return launch(c, "gemm_f32_simple", gemm_f32_simple_kernel, grid, dim3(256), 0, a);
    }
  }
}

}  // namespace k
}  // namespace mnn
