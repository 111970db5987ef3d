// Encoder-level kernels on the matrix cores (v_mfma_f32_32x32x2_f32) with LDS-DMA staging:
//
//   enc_conv     strided Conv1D, kernel 8 / stride 4 / dilation 1 / groups 1, zero or reflect
//                padding < 4 (DynamicConv1D.swift:288-324,358-401; UNet.swift:52), as an implicit
//                GEMM C[co][t] = bias[co] + sum_{ci,k} W[co][ci*8+k] * x[ci][4t - pad + k], with
//                per-workgroup GroupNorm(1) statistics partials of C (Normalization.swift:479-597:
//                biased variance);
//   enc_rewrite  the 1x1 rewrite conv C -> 2C as a GEMM over the conv output read through
//                GroupNorm + GELU (statistics merged once per workgroup, applied to the operand
//                fragments in registers), with GLU (NN.metal:1012-1023) in the epilogue.
//
// Both kernels are persistent (one or two workgroups per CU, each walking a set of output tiles).
// The statistics hand-off needs no cross-workgroup synchronisation inside the conv: a
// device-scope fence there writes back and invalidates the XCD's L2 under the other workgroups.
//
// Both stage their operands in a ring of S LDS buffers filled by LDS-DMA loads (lds_dma.hpp) and
// meet at one barrier per stage. A (the weights, [M][K] rows) uses the swizzled [rows][32 floats]
// layout of the transformer GEMM. The conv's B operand is the raw input: per stage 4 channels x
// (4*BN + 4) consecutive samples, fetched as 16-byte chunks from 4-byte aligned addresses; im2col
// exists neither in HBM nor in LDS, and lane (t, k) reads its 4 taps x[ci][4t + k..k+3] as one
// 16-byte LDS read. Chunks that cross the signal ends are rewritten in LDS with their reflect /
// zero values after they land (first and last tiles only). The rewrite's B operand is [K][N] rows
// with a 16-byte pitch; row r's chunk j sits at slot j ^ 8*((r/16) mod 2), which keeps the two
// lane halves (k and k + 16) on different banks.
//
// Deep, narrow levels (few output tiles, long K) split K inside the workgroup: KG groups of waves
// each own a 32-deep slice of every stage, and their accumulators are summed through LDS at the
// end, so a 32x64 tile still keeps 8 waves busy on its CU.
#include "device_utils.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

enum { ENC_CONV = 0, ENC_RW = 1 };
constexpr int kMaxM = 1024;  // output rows (bias staged in LDS)
constexpr int kMaxK = 512;   // rewrite operand rows (GroupNorm coefficients staged in LDS)

template <int MODE, int WMW, int WNW, int WM, int WN, int KG, int S>
struct EncCfg {
  static constexpr int BM = WMW * WM * 32, BN = WNW * WN * 32;
  static constexpr int NWO = WMW * WNW;  // waves per k-group: one output tile
  static constexpr int NW = NWO * KG, NT = NW * 64;
  static constexpr int BK = 32 * KG;  // k per stage
  static constexpr int A_FLOATS = KG * BM * 32;
  static constexpr int A_INS = KG * BM / 8;  // 8 rows of 32 floats per wave load
  static constexpr int WCH = BN + 1;         // conv: 16-byte chunks per channel window
  static constexpr int B_RAW = MODE == ENC_CONV ? KG * 4 * WCH : KG * 32 * BN / 4;
  static constexpr int B_INS = (B_RAW + 64 * NW - 1) / (64 * NW) * NW;
  static constexpr int B_FLOATS = B_INS * 256;
  static constexpr int A_INS_W = A_INS / NW, B_INS_W = B_INS / NW;
  static constexpr int L = A_INS_W + B_INS_W;  // loads per wave per stage
  static constexpr int STAGE = A_FLOATS + B_FLOATS;
  static constexpr int RED = (KG - 1) * BM * BN;  // k-group reduction area after the ring
  static_assert(A_INS % NW == 0, "A loads must split evenly over the waves");
  static_assert(MODE == ENC_CONV || BN >= 64, "rewrite B swizzle needs 16 chunks per row");
  static_assert((S - 2) * L < 64, "vmcnt range");
  static_assert(S >= 2, "ring depth");
};

struct EncArgs {
  int M = 0, N = 0, K = 0, batch = 1;
  const float* A = nullptr;  // weights [M][K], row stride lda
  int64_t lda = 0;
  // conv: input x[b][ci][L] (batch stride x_bs)
  const float* x = nullptr;
  int64_t x_bs = 0;
  int Cin = 0;  // real input channels; K = 8 * Cin rounded up to 4 channels (zero weights)
  int L = 0, pad = 0;
  bool reflect = false;
  // rewrite: B rows [K][ldb] (ldb % 4 == 0, >= N rounded up to 4), batch stride sB
  const float* Bm = nullptr;
  int64_t ldb = 0, sB = 0;
  const float* coef = nullptr;  // [batch][K][2] (scale, shift) per operand row, or null and ...
  const float* gamma = nullptr;
  const float* beta = nullptr;
  // output: C[b][m][n] (conv) or GLU rows C[b][m/2][n] (rewrite), row stride ldc
  float* C = nullptr;
  int64_t ldc = 0, sC = 0;
  const float* bias = nullptr;  // per row m
  // ... GroupNorm(1) statistics partials (count, mean, M2): written by the conv (one per
  // workgroup, nparts per batch), merged by the rewrite
  float* parts = nullptr;
  int nparts = 0;
  float eps = 1e-5f;
};

__device__ __forceinline__ int reflect_or_clamp(int p, int L) {
  p = p < 0 ? -p : p;
  p = p >= L ? 2 * (L - 1) - p : p;
  return min(max(p, 0), L - 1);  // columns past the output never need more than a valid sample
}

template <int MODE, int WMW, int WNW, int WM, int WN, int KG, int S>
__global__ __launch_bounds__(WMW* WNW* KG * 64) void enc_gemm_kernel(EncArgs a) {
  using Cfg = EncCfg<MODE, WMW, WNW, WM, WN, KG, S>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, NWO = Cfg::NWO, NT = Cfg::NT, BK = Cfg::BK;
  constexpr int STAGE = Cfg::STAGE, WCH = Cfg::WCH;
  __shared__ __attribute__((aligned(1024))) float smem[S * STAGE + Cfg::RED];
  __shared__ float2 coef_s[MODE == ENC_RW ? kMaxK : 1];
  __shared__ float bias_s[kMaxM];
  __shared__ float red[3 * (NT / 64)];
  __shared__ double redd[3 * (NT / 64)];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave / NWO, wo = wave % NWO;
  const int wm = wo / WNW, wn = wo % WNW;
  const int b = blockIdx.z;
  const int M = a.M, N = a.N, K = a.K;
  const int mt = (M + BM - 1) / BM, ntl = (N + BN - 1) / BN;
  const int tiles = mt * ntl;  // per batch
  const int G = gridDim.x;
  // persistent: workgroup wg takes tiles wg, wg + G, ...; workgroups of one XCD get consecutive
  // ids, so the tiles in flight on an XCD are neighbours (M fastest: they share a B panel)
  const int wg = xcd_logical_tile(blockIdx.x, G);
  const int my_tiles = wg < tiles ? (tiles - 1 - wg) / G + 1 : 0;
  const int nk = (K + BK - 1) / BK;
  const int iters = my_tiles * nk;

  // ------------------------------------------------ per-lane, tile-independent load geometry
  int arow[Cfg::A_INS_W], acol[Cfg::A_INS_W];
#pragma unroll
  for (int i = 0; i < Cfg::A_INS_W; ++i) {
    const int ins = wave * Cfg::A_INS_W + i;
    const int kgi = ins / (BM / 8), r = (ins % (BM / 8)) * 8 + (lane >> 3);
    arow[i] = r;
    acol[i] = kgi * 32 + 4 * ((lane & 7) ^ chunk_swizzle(r));
  }
  // conv: channel within the stage and window chunk; rewrite: row within the stage and chunk
  int bsel[Cfg::B_INS_W], bchk[Cfg::B_INS_W];
  bool bval[Cfg::B_INS_W];
#pragma unroll
  for (int i = 0; i < Cfg::B_INS_W; ++i) {
    const int e = (wave * Cfg::B_INS_W + i) * 64 + lane;
    bval[i] = e < Cfg::B_RAW;
    const int ee = bval[i] ? e : 0;  // padding chunks load a valid, unused address
    if constexpr (MODE == ENC_CONV) {
      bsel[i] = ee / WCH;  // kg * 4 + channel within the slice
      bchk[i] = ee % WCH;
    } else {
      const int kgi = ee / (8 * BN), rem = ee % (8 * BN);
      const int r = rem / (BN / 4);
      bchk[i] = (rem % (BN / 4)) ^ (8 * ((r >> 4) & 1));
      bsel[i] = r + 32 * kgi;
    }
  }
  const float* bbase = MODE == ENC_CONV ? a.x + (int64_t)b * a.x_bs : a.Bm + (int64_t)b * a.sB;
  auto tile_mn = [&](int ti, int& m0, int& n0) {
    const int t = wg + ti * G;
    m0 = (t % mt) * BM;
    n0 = (t / mt) * BN;
  };
  const unsigned lds0 = lds_address(smem);
  auto issue = [&](int it) {
    const int ti = it / nk, kt = it - ti * nk;
    int m0, n0;
    tile_mn(ti, m0, n0);
    const unsigned base = lds0 + 4u * (unsigned)((it % S) * STAGE);
#pragma unroll
    for (int i = 0; i < Cfg::A_INS_W; ++i) {
      const int ins = wave * Cfg::A_INS_W + i;
      // chunks past K (rewrite tail) are clamped into the row; their B rows are zero
      const float* src = a.A + (int64_t)min(m0 + arow[i], M - 1) * a.lda +
                         min(kt * BK + acol[i], K - 4);
      lds_dma16(src, __builtin_amdgcn_readfirstlane(base + 4u * (ins * 256)));
    }
#pragma unroll
    for (int i = 0; i < Cfg::B_INS_W; ++i) {
      const int ins = wave * Cfg::B_INS_W + i;
      const unsigned dst =
          __builtin_amdgcn_readfirstlane(base + 4u * (Cfg::A_FLOATS + ins * 256));
      if constexpr (MODE == ENC_CONV) {
        // channels past Cin (zero weights) read the last real channel
        const int chan = min(kt * 4 * KG + bsel[i], a.Cin - 1);
        const int pos = min(max(4 * n0 - a.pad + 4 * bchk[i], 0), a.L - 4);
        lds_dma16(bbase + (int64_t)chan * a.L + pos, dst);
      } else {
        const int row = min(kt * BK + bsel[i], K - 1);
        lds_dma16(bbase + (int64_t)row * a.ldb + min((int64_t)(n0 + 4 * bchk[i]), a.ldb - 4),
                  dst);
      }
    }
  };
  // conv: chunks crossing the signal ends get their padded values once the stage has landed
  auto fix_edges = [&](int it) {
    if constexpr (MODE == ENC_CONV) {
      const int ti = it / nk, kt = it - ti * nk;
      int m0, n0;
      tile_mn(ti, m0, n0);
      float* stage = smem + (it % S) * STAGE + Cfg::A_FLOATS;
#pragma unroll
      for (int i = 0; i < Cfg::B_INS_W; ++i) {
        const int pos = 4 * n0 - a.pad + 4 * bchk[i];
        if (bval[i] && (pos < 0 || pos + 3 > a.L - 1)) {
          const int e = (wave * Cfg::B_INS_W + i) * 64 + lane;
          const float* row = bbase + (int64_t)min(kt * 4 * KG + bsel[i], a.Cin - 1) * a.L;
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int p = pos + t;
            if (a.reflect) v[t] = row[reflect_or_clamp(p, a.L)];
            else v[t] = (p >= 0 && p < a.L) ? row[p] : 0.f;
          }
          *reinterpret_cast<float4*>(stage + 4 * e) = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
    }
  };

  // first stages in flight while the coefficients are prepared
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < iters) issue(s);
  for (int m = tid; m < M; m += NT) bias_s[m] = a.bias ? a.bias[m] : 0.f;
  // rewrite: GroupNorm coefficients of the operand rows (zero past K); with statistics
  // partials of the producer, every workgroup merges them the same way (fixed order, fp64)
  if constexpr (MODE == ENC_RW) {
    float mean = 0.f, rstd = 0.f;
    if (!a.coef) {
      const float2 ms =
          gn1_merge_one_round(a.parts + (int64_t)b * a.nparts * 3, a.nparts, a.eps, redd);
      mean = ms.x;
      rstd = ms.y;
    }
    for (int k = tid; k < nk * BK; k += NT) {
      float2 cf = make_float2(0.f, 0.f);
      if (k < K) {
        if (a.coef) {
          cf = *reinterpret_cast<const float2*>(a.coef + ((int64_t)b * K + k) * 2);
        } else {
          const float sc = (a.gamma ? a.gamma[k] : 1.f) * rstd;
          cf = make_float2(sc, (a.beta ? a.beta[k] : 0.f) - mean * sc);
        }
      }
      coef_s[k] = cf;
    }
  }
  wait_lgkmcnt0();
  stage_barrier();  // coefficients and bias visible; no memory fence (the stages stay in flight)

  floatx16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int g = lane >> 5, l32 = lane & 31;
  int aoff[WM], asw[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int r = wm * WM * 32 + 32 * i + l32;
    aoff[i] = kg * BM * 32 + r * 32;
    asw[i] = chunk_swizzle(r);
  }
  int bcol[WN];
#pragma unroll
  for (int j = 0; j < WN; ++j) bcol[j] = wn * WN * 32 + 32 * j + l32;

  ShiftedStats st;  // conv: statistics of every output this thread stores
  float* __restrict__ Cp = a.C + (int64_t)b * a.sC;

  int kt = 0, ti = 0;
  for (int it = 0; it < iters; ++it) {
    if (it + S - 2 < iters) wait_vmcnt<(S - 2) * Cfg::L>();
    else wait_vmcnt<0>();
    fix_edges(it);
    if constexpr (MODE == ENC_CONV) wait_lgkmcnt0();
    stage_barrier();  // stage it is complete everywhere; stage it-1 is no longer read
    if (it + S - 1 < iters) issue(it + S - 1);
    const float* As = smem + (it % S) * STAGE;
    const float* Bs = As + Cfg::A_FLOATS;
    // all fragment reads of the stage first, so their latency overlaps the matrix work
    float4 fa[4][WM], fb[4][WN];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int c = 4 * g + q4;
#pragma unroll
      for (int i = 0; i < WM; ++i)
        fa[q4][i] = *reinterpret_cast<const float4*>(As + aoff[i] + 4 * (c ^ asw[i]));
      if constexpr (MODE == ENC_CONV) {
        // k = 16g + 4q (within the slice): channel kg*4 + 2g + q/2, taps 4(q%2)..+3
        const int chan = kg * 4 + 2 * g + (q4 >> 1);
#pragma unroll
        for (int j = 0; j < WN; ++j)
          fb[q4][j] = *reinterpret_cast<const float4*>(Bs + chan * (4 * WCH) + 4 * bcol[j] +
                                                       4 * (q4 & 1));
      } else {
        const float* rowp = Bs + (kg * 32 + 16 * g + 4 * q4) * BN;
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const int col = 4 * ((bcol[j] >> 2) ^ (8 * g)) + (bcol[j] & 3);
          fb[q4][j] = make_float4(rowp[col], rowp[BN + col], rowp[2 * BN + col],
                                  rowp[3 * BN + col]);
        }
      }
    }
    // keep the reads ahead of the matrix work (the scheduler would otherwise sink each read next
    // to its first use to save registers, exposing the LDS latency every four MFMAs)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (MODE == ENC_RW) {
      // GroupNorm + GELU of the operand rows this lane holds (row k = 16g + 4q + s)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int kglob = kt * BK + kg * 32 + 16 * g + 4 * q4;
        float2 cf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) cf[s] = coef_s[kglob + s];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          fb[q4][j].x = gelu_tanh_fast(fmaf(fb[q4][j].x, cf[0].x, cf[0].y));
          fb[q4][j].y = gelu_tanh_fast(fmaf(fb[q4][j].y, cf[1].x, cf[1].y));
          fb[q4][j].z = gelu_tanh_fast(fmaf(fb[q4][j].z, cf[2].x, cf[2].y));
          fb[q4][j].w = gelu_tanh_fast(fmaf(fb[q4][j].w, cf[3].x, cf[3].y));
        }
      }
    }
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j) {
            const float av = s == 0 ? fa[q4][i].x : s == 1 ? fa[q4][i].y : s == 2 ? fa[q4][i].z : fa[q4][i].w;
            const float bv = s == 0 ? fb[q4][j].x : s == 1 ? fb[q4][j].y : s == 2 ? fb[q4][j].z : fb[q4][j].w;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[i][j], 0, 0, 0);
          }

    if (kt == nk - 1) {
      // ---------------------------------------------- tile done: k-group reduction, epilogue
      int m0, n0;
      tile_mn(ti, m0, n0);
      if constexpr (KG > 1) {
        // the reduction area is outside the ring (the next tile's stages are in flight); the
        // previous tile's reads of it are separated from these writes by a stage barrier
        float* redf = smem + S * STAGE;
        if (kg > 0) {
          float* dst = redf + ((kg - 1) * NWO + wo) * (WM * WN * 1024);
#pragma unroll
          for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
              for (int v = 0; v < 16; ++v) dst[((i * WN + j) * 16 + v) * 64 + lane] = acc[i][j][v];
        }
        wait_lgkmcnt0();
        stage_barrier();
        if (kg == 0) {
#pragma unroll
          for (int q = 1; q < KG; ++q) {
            const float* src = redf + ((q - 1) * NWO + wo) * (WM * WN * 1024);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
              for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                  acc[i][j][v] += src[((i * WN + j) * 16 + v) * 64 + lane];
          }
        }
      }
      // accumulator layout (32x32 block): lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4,
      // column l%32
      if (kg == 0) {
        if constexpr (MODE == ENC_RW) {
#pragma unroll
          for (int i = 0; i < WM; ++i) {
            const int mblk = m0 + wm * WM * 32 + i * 32;
            if (mblk >= M) continue;
#pragma unroll
            for (int j = 0; j < WN; ++j) {
              const int gn = n0 + bcol[j];
              if (gn >= N) continue;
#pragma unroll
              for (int v = 0; v < 8; ++v) {
                const int rr = 8 * (v / 4) + 4 * g + (v % 4);  // < 16
                const float va = acc[i][j][v] + bias_s[mblk + rr];
                const float vb = acc[i][j][v + 8] + bias_s[mblk + 16 + rr];
                Cp[(int64_t)((mblk >> 5) * 16 + rr) * a.ldc + gn] = va * stable_sigmoid(vb);
              }
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < WM; ++i) {
            const int mblk = m0 + wm * WM * 32 + i * 32;
#pragma unroll
            for (int j = 0; j < WN; ++j) {
              const int gn = n0 + bcol[j];
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
                if (gm < M && gn < N) {
                  const float val = acc[i][j][v] + bias_s[gm];
                  st.add(val);
                  Cp[(int64_t)gm * a.ldc + gn] = val;
                }
              }
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
      kt = 0;
      ++ti;
    } else {
      ++kt;
    }
  }

  // ------------------------------------------------ conv: GroupNorm(1) statistics partial
  if constexpr (MODE == ENC_CONV) {
    if (a.parts) {
      float sn, smean, sm2;
      st.finish(sn, smean, sm2);
      block_welford(sn, smean, sm2, red);
      if (tid == 0) {
        float* o = a.parts + ((int64_t)b * G + wg) * 3;
        o[0] = sn;
        o[1] = smean;
        o[2] = sm2;
      }
    }
  }
}

// ---------------------------------------------------------------- host-side selection
struct EncTile {
  int id, bm, bn, kg, nw, lds_kb;
};
// conv configurations (id -> template arguments in enc_conv); lds_kb: LDS per workgroup as
// compiled, which bounds the resident workgroups per CU
// (KiB, rounded up; 160 KiB per CU)
constexpr EncTile kConvTiles[] = {
    {0, 32, 64, 1, 2, 75},   // <1,2,1,1> KG1 S7
    {1, 32, 64, 2, 4, 133},  // <1,2,1,1> KG2 S6
    {2, 64, 64, 2, 8, 149},  // <2,2,1,1> KG2 S4
    {3, 32, 64, 4, 8, 149},  // <1,2,1,1> KG4 S3
    {4, 64, 64, 1, 4, 101},  // <2,2,1,1> KG1 S6
};
constexpr EncTile kRwTiles[] = {
    {0, 64, 64, 1, 4, 105},  // <2,2,1,1> KG1 S6
    {1, 32, 64, 1, 2, 69},   // <1,2,1,1> KG1 S5
    {2, 64, 64, 2, 8, 153},  // <2,2,1,1> KG2 S4
    {3, 32, 64, 2, 4, 137},  // <1,2,1,1> KG2 S5
};
constexpr int kCUs = 256;

int env_int(const char* name) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : -1;
}

int occupancy(const EncTile& t) { return std::max(1, std::min(160 / t.lds_kb, 32 / t.nw)); }

// Persistent grid: workgroups per batch.
int grid_per_batch(const EncTile& t, int tiles, int batch) {
  return std::max(1, std::min(tiles, kCUs * occupancy(t) / std::max(batch, 1)));
}

// Critical path in MFMA units per SIMD: tiles per workgroup x waves sharing a SIMD x per-wave
// work per tile (block area x K / k-groups), over an efficiency that grows with the waves a SIMD
// can interleave.
// whole_stages: K must be a multiple of the stage depth 32 * kg (the conv has no K tail).
template <size_t NT>
const EncTile& choose(const EncTile (&tiles)[NT], int M, int N, int K, int batch, int forced,
                      bool whole_stages) {
  auto fits = [&](const EncTile& t) { return !whole_stages || K % (32 * t.kg) == 0; };
  if (forced >= 0 && forced < (int)NT && fits(tiles[forced])) return tiles[forced];
  const EncTile* best = nullptr;
  double best_cost = 1e300;
  for (const EncTile& t : tiles) {
    if (!fits(t)) continue;
    const int per_b = (int)(cdiv(M, t.bm) * cdiv(N, t.bn));
    const int64_t total = (int64_t)per_b * batch;
    const int64_t wgs = (int64_t)grid_per_batch(t, per_b, batch) * batch;
    const double tiles_per_wg = std::ceil((double)total / wgs);
    const double waves_simd = (double)wgs * t.nw / (4.0 * kCUs);
    const double eff = waves_simd >= 2 ? 1.0 : waves_simd >= 1 ? 0.8 : 0.55;
    const double per_wave = (double)t.bm * t.bn / (t.nw / t.kg) * ((double)K / t.kg);
    const double cost = tiles_per_wg * std::max(1.0, waves_simd) * per_wave / eff;
    if (!best || cost < best_cost * 0.999) {
      best_cost = cost;
      best = &t;
    }
  }
  MNN_REQUIRE(best, MNN_ERR_INVALID_ARGUMENT, "enc: no tile configuration fits K = " << K);
  return *best;
}

template <int MODE, int WMW, int WNW, int WM, int WN, int KG, int S>
void launch_enc(const LaunchCtx& c, const EncArgs& a, const EncTile& t, const char* name) {
  using Cfg = EncCfg<MODE, WMW, WNW, WM, WN, KG, S>;
  static_assert(Cfg::BM > 0, "");
  const int per_b = (int)(cdiv(a.M, Cfg::BM) * cdiv(a.N, Cfg::BN));
  dim3 grid(grid_per_batch(t, per_b, a.batch), 1, a.batch), block(Cfg::NT);
  launch(c, name, enc_gemm_kernel<MODE, WMW, WNW, WM, WN, KG, S>, grid, block, 0, a);
}

}  // namespace

bool enc_conv_supported(int Cin, int Cout, int ks, int stride, int dil, int groups, int pad,
                        int64_t L) {
  return Cin > 0 && Cout > 0 && ks == 8 && stride == 4 && dil == 1 && groups == 1 && pad >= 0 &&
         pad < 4 && L >= 8 && L < (1LL << 30) / std::max(Cin, 4);
}

int enc_conv_padded_cin(int Cin) { return (Cin + 3) / 4 * 4; }

int enc_conv_parts(int Cout, int64_t Lout, int K, int batch) {
  const EncTile& t =
      choose(kConvTiles, Cout, (int)Lout, K, batch, env_int("MNN_ENC_CONV_TILE"), true);
  return grid_per_batch(t, (int)(cdiv(Cout, t.bm) * cdiv(Lout, t.bn)), batch);
}

void enc_conv(const LaunchCtx& c, const EncConvArgs& p) {
  EncArgs a;
  a.M = p.Cout;
  a.N = (int)p.Lout;
  a.K = enc_conv_padded_cin(p.Cin) * 8;
  a.batch = p.B;
  a.A = p.w;
  a.lda = a.K;
  a.x = p.x;
  a.x_bs = (int64_t)p.Cin * p.L;
  a.Cin = p.Cin;
  a.L = (int)p.L;
  a.pad = p.pad;
  a.reflect = p.reflect;
  a.C = p.y;
  a.ldc = p.ldy;
  a.sC = (int64_t)p.Cout * p.ldy;
  a.bias = p.bias;
  a.parts = p.parts;
  MNN_REQUIRE(enc_conv_supported(p.Cin, p.Cout, 8, 4, 1, 1, p.pad, p.L) && a.K % 32 == 0 &&
                  p.ldy >= p.Lout && p.Cout <= kMaxM,
              MNN_ERR_INVALID_ARGUMENT, "enc_conv: unsupported configuration");
  const EncTile& t =
      choose(kConvTiles, a.M, a.N, a.K, a.batch, env_int("MNN_ENC_CONV_TILE"), true);
  switch (t.id) {
    case 0: return launch_enc<ENC_CONV, 1, 2, 1, 1, 1, 7>(c, a, t, "enc_conv_f32");
    case 1: return launch_enc<ENC_CONV, 1, 2, 1, 1, 2, 6>(c, a, t, "enc_conv_f32");
    case 2: return launch_enc<ENC_CONV, 2, 2, 1, 1, 2, 4>(c, a, t, "enc_conv_f32");
    case 3: return launch_enc<ENC_CONV, 1, 2, 1, 1, 4, 3>(c, a, t, "enc_conv_f32");
    default: return launch_enc<ENC_CONV, 2, 2, 1, 1, 1, 6>(c, a, t, "enc_conv_f32");
  }
}

void enc_rewrite(const LaunchCtx& c, const EncRewriteArgs& p) {
  EncArgs a;
  a.M = 2 * p.C;
  a.N = (int)p.Lout;
  a.K = p.C;
  a.batch = p.B;
  a.A = p.w;
  a.lda = p.C;
  a.Bm = p.y;
  a.ldb = p.ldy;
  a.sB = (int64_t)p.C * p.ldy;
  a.parts = const_cast<float*>(p.parts);
  a.nparts = p.nparts;
  a.eps = p.eps;
  a.coef = p.coef;
  a.gamma = p.gamma;
  a.beta = p.beta;
  a.C = p.out;
  a.ldc = p.ldo;
  a.sC = (int64_t)p.C * p.ldo;
  a.bias = p.bias;
  MNN_REQUIRE(p.C % 16 == 0 && p.C >= 32 && p.C <= kMaxK && 2 * p.C <= kMaxM && p.ldy % 4 == 0 &&
                  p.ldy >= (p.Lout + 3) / 4 * 4 && ((p.parts && p.nparts > 0) || p.coef) && p.bias,
              MNN_ERR_INVALID_ARGUMENT, "enc_rewrite: unsupported configuration");
  const EncTile& t = choose(kRwTiles, a.M, a.N, a.K, a.batch, env_int("MNN_ENC_RW_TILE"), false);
  switch (t.id) {
    case 0: return launch_enc<ENC_RW, 2, 2, 1, 1, 1, 6>(c, a, t, "enc_rewrite_f32");
    case 1: return launch_enc<ENC_RW, 1, 2, 1, 1, 1, 5>(c, a, t, "enc_rewrite_f32");
    case 2: return launch_enc<ENC_RW, 2, 2, 1, 1, 2, 4>(c, a, t, "enc_rewrite_f32");
    default: return launch_enc<ENC_RW, 1, 2, 1, 1, 2, 5>(c, a, t, "enc_rewrite_f32");
  }
}

}  // namespace k
}  // namespace mnn
