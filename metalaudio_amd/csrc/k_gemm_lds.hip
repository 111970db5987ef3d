// fp32 GEMM C = epilogue(A * B^T) for B stored [N][K] (Linear / attention projections / FFN,
// PyTorch weight layout; Linear.swift:337-352 computes y = x W^T + b), on v_mfma_f32_32x32x2_f32.
//
// Operand tiles move from HBM to LDS with the CDNA4 LDS-DMA load (global_load_lds_dwordx4): the
// data never passes through VGPRs and no ds_write is issued, so the only per-step work besides
// the matrix cores is one s_barrier and the wave's fragment reads. K advances in 32-deep stages
// held in a ring of S LDS buffers; the loads of stage kt+S are issued once every wave has read
// stage kt into registers, so up to S-1 stages of HBM/L2 latency are in flight behind the
// matrix work.
//
// LDS layout of one stage: A rows [BM][32 floats] then B rows [BN][32 floats], unpadded
// (LDS-DMA writes each wave's 64 x 16 bytes contiguously). A row's 16-byte chunk c is stored at
// slot c ^ f(r), f(r) = (r + r/8) mod 8; the lane that fills slot s of row r fetches chunk s ^ f(r)
// from global memory (the 8 lanes of a row still read one contiguous 128-byte segment). The
// fragment reads (32 rows x one chunk per lane group) then hit distinct banks for 32- and 64-bank
// LDS alike.
//
// The loads are issued by inline asm: the compiler's own tracking of LDS-DMA would make every
// LDS read wait for all outstanding loads (it cannot tell the ring buffers apart), and a
// __syncthreads would wait for them at every barrier. Here the kernel waits itself for exactly the
// stage it is about to read (s_waitcnt vmcnt((S-2) * loads per stage)) before the barrier.
// S = 2 is allowed: the slot of stage kt is refilled as soon as its fragments are in registers.
//
// Within a stage, lane group g = lane/32 owns k in [16g, 16g+16): the MFMA's two k slots are fed
// k = 16g + 4q + s in sub-step (q, s). A and B use the same assignment, so the sum over k is
// unchanged, and each lane reads its 4 consecutive k of a row with one 16-byte LDS read.
#include "device_utils.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int BK = 32;

template <int WMW, int WNW, int WM, int WN, int S>
struct LdsCfg {
  static constexpr int BM = WMW * WM * 32, BN = WNW * WN * 32;
  static constexpr int NW = WMW * WNW, NT = NW * 64;
  static constexpr int A_INS = BM / 8 / NW, B_INS = BN / 8 / NW;  // 8 rows per wave load
  static constexpr int L = A_INS + B_INS;                         // loads per wave per stage
  static constexpr int STAGE = (BM + BN) * BK;                    // floats
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "tile rows must split over waves");
  static_assert((S - 1) * L < 64, "vmcnt range");
};

// C = R + rscale[n] * act(acc + bias) (R, rscale optional). ACT = -1: activation code at run time.
// Accumulator layout of a 32x32 block: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4,
// column l%32; each store instruction writes two 128-byte row segments.
//
// The values the stores depend on are loaded before the stores, and one explicit wait separates
// them. The vector memory counter counts stores as well as loads, so a load issued between stores
// (or one the compiler cannot track through a branch) makes each later store wait for every
// earlier store, and the epilogue would run at one memory latency per store. R may be C itself
// (in-place residual, element for element); no lane stores an element another lane reads, so
// loading before storing is exact. FAST (no bias along M, no residual): the few loads of the tile
// come first. Otherwise one 32-row block at a time: its loads, a wait, its stores (holding every
// residual of the tile at once would push the kernel past the register budget of two workgroups
// per CU).
template <int WMW, int WNW, int WM, int WN, int ACT, bool RES, bool FAST>
__device__ __forceinline__ void store_tile(const GemmArgs& a, const floatx16 (&acc)[WM][WN], int m0,
                                           int n0, int wm, int wn, int lane) {
  const int g = lane >> 5, l32 = lane & 31;
  const int bz = blockIdx.z;
  float* __restrict__ Cp = a.C + (int64_t)bz * a.sC;
  const float* Rp = RES && a.R ? a.R + (int64_t)bz * a.sR : nullptr;
  const bool full_m = m0 + WMW * WM * 32 <= a.M;
  constexpr int RI = FAST ? WM : 1;  // 32-row blocks whose residuals are held at once
  float bnv[WN], rsv[WN];
  float rv[RES ? RI : 1][RES ? WN : 1][16];
  if (a.bias_mode == BIAS_N) {
#pragma unroll
    for (int j = 0; j < WN; ++j) bnv[j] = a.bias[min(n0 + wn * WN * 32 + j * 32 + l32, a.N - 1)];
  } else {
#pragma unroll
    for (int j = 0; j < WN; ++j) bnv[j] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < WN; ++j)
    rsv[j] = RES && Rp && a.rscale ? a.rscale[min(n0 + wn * WN * 32 + j * 32 + l32, a.N - 1)] : 1.f;
  // residuals of blocks [i0, i0 + RI)
  auto load_res = [&](int i0) {
    if constexpr (RES) {
#pragma unroll
      for (int ii = 0; ii < RI; ++ii)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const int gn = min(n0 + wn * WN * 32 + j * 32 + l32, a.N - 1);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int gm =
                min(m0 + wm * WM * 32 + (i0 + ii) * 32 + 8 * (v / 4) + 4 * g + (v % 4), a.M - 1);
            rv[ii][j][v] = Rp ? Rp[(int64_t)gm * a.ldr + gn] : 0.f;
          }
        }
    }
  };
  if constexpr (FAST) {
    load_res(0);
    wait_vmcnt<0>();
  }
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int mblk = m0 + wm * WM * 32 + i * 32;
    float bmv[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) bmv[v] = 0.f;
    if constexpr (!FAST) {
      if (a.bias_mode == BIAS_M) {
#pragma unroll
        for (int v = 0; v < 16; ++v) bmv[v] = a.bias[min(mblk + 8 * (v / 4) + 4 * g + (v % 4), a.M - 1)];
      }
      load_res(i);
      wait_vmcnt<0>();
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int gn = n0 + wn * WN * 32 + j * 32 + l32;
      if (gn >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
        if (full_m || gm < a.M) {
          float val = acc[i][j][v] + bnv[j] + bmv[v];
          val = ACT < 0 ? apply_act(val, a.act, a.act_alpha) : apply_act(val, ACT);
          if constexpr (RES) val = rv[FAST ? i : 0][j][v] + rsv[j] * val;
          Cp[(int64_t)gm * a.ldc + gn] = val;
        }
      }
    }
  }
}

// Folded LayerNorm of A's rows: (rstd, -rstd * mean) of row m merged from its K / 64 partials
// (mean, M2) of 64 features each (Chan's formula for equal counts, a fixed order; K <= 64 *
// kLnMaxParts). ln_row_load issues the loads before the main loop, so they complete under it
// (GEMMs without a folded LayerNorm read a zero dummy, so no load sits under a branch), and
// ln_row_merge combines them in the epilogue.
constexpr int kLnMaxParts = 8;
struct LnRow {
  float2 q[kLnMaxParts];
};

__device__ float2 ln_dummy_parts[kLnMaxParts];

__device__ __forceinline__ LnRow ln_row_load(const GemmArgs& a, int m) {
  const bool on = a.ln_parts != nullptr;
  const int P = on ? a.K / 64 : 1;
  const float2* pp =
      on ? reinterpret_cast<const float2*>(a.ln_parts) + (int64_t)min(m, a.M - 1) * P
         : ln_dummy_parts;
  LnRow r;
#pragma unroll
  for (int p = 0; p < kLnMaxParts; ++p) r.q[p] = pp[min(p, P - 1)];
  return r;
}

__device__ __forceinline__ float2 ln_row_merge(const GemmArgs& a, const LnRow& r) {
  const int P = a.K / 64;
  float mean = r.q[0].x, m2 = r.q[0].y;
#pragma unroll
  for (int p = 1; p < kLnMaxParts; ++p) {
    if (p < P) {
      const float d = r.q[p].x - mean;
      mean += d * (1.f / (float)(p + 1));
      m2 += r.q[p].y + d * d * (64.f * (float)p / (float)(p + 1));
    }
  }
  const float rstd = 1.f / sqrtf(m2 / (float)a.K + a.ln_eps);
  return make_float2(rstd, -rstd * mean);
}

// The same epilogue with the tile transposed through LDS into row order, for outputs whose rows
// are 16-byte aligned (N % 4 == 0, ldc % 4 == 0; residual likewise): the accumulators are written
// to LDS ([rows][BN + 8 floats]: rows four apart, which the two lane groups write together, sit 32
// banks apart), read back as float4 along rows and stored so that consecutive lanes cover
// consecutive 16-byte pieces of a row — 512-byte row runs per half-wave for BN = 128 instead of the
// accumulator layout's 128-byte pieces of 32 rows, which the memory system served at about 2 TB/s.
// Bias (along N), activation, residual and LayerScale apply in row order. Tiles whose rows do not
// fit the LDS ring at once go in passes of whole wave rows. The caller has synchronised the
// workgroup after its last LDS read of the main loop.
template <int WMW, int WNW, int WM, int WN, int ACT, bool RES, int LDS_FLOATS>
__device__ __forceinline__ void store_tile_lds(const GemmArgs& a, const floatx16 (&acc)[WM][WN],
                                               int m0, int n0, int wm, int wn, int lane,
                                               float* smem, const LnRow& lnr) {
  constexpr int BM = WMW * WM * 32, BN = WNW * WN * 32, NT = WMW * WNW * 64;
  constexpr int PITCH = BN + 8;
  constexpr int WROWS = WM * 32;  // rows per wave row
  constexpr int PASS_WM = (BM * PITCH <= LDS_FLOATS) ? WMW : 1;  // wave rows per pass
  constexpr int PROWS = PASS_WM * WROWS;                          // rows per pass
  static_assert(PROWS * PITCH <= LDS_FLOATS, "epilogue tile does not fit the LDS ring");
  constexpr int C4 = BN / 4;                  // float4 per row
  constexpr int RPI = NT / C4;                // rows per thread iteration
  constexpr int IT = PROWS / RPI;             // iterations per pass
  static_assert(NT % C4 == 0 && PROWS % RPI == 0, "epilogue thread layout");
  const int g = lane >> 5, l32 = lane & 31;
  const int tid = threadIdx.x;
  const int bz = blockIdx.z;
  float* __restrict__ Cp = a.C + (int64_t)bz * a.sC;
  const float* Rp = RES && a.R ? a.R + (int64_t)bz * a.sR : nullptr;
  const int c4 = tid % C4, rr0 = tid / C4;
  const int gn = n0 + 4 * c4;
  const bool col_ok = gn < a.N;  // N % 4 == 0: a float4 is all in or all out
  float4 bn = make_float4(0.f, 0.f, 0.f, 0.f), rs = make_float4(1.f, 1.f, 1.f, 1.f);
  if (col_ok && a.bias_mode == BIAS_N) bn = *reinterpret_cast<const float4*>(a.bias + gn);
  if (RES && Rp && a.rscale && col_ok) rs = *reinterpret_cast<const float4*>(a.rscale + gn);
  // Folded LayerNorm: thread r < BM merges row m0 + r's partials (loaded before the main loop)
  // into (rstd, -rstd * mean), kept at the end of the LDS ring past the rows the passes below
  // write; the first pass's barrier makes them visible.
  static_assert(PROWS * PITCH + 2 * BM <= LDS_FLOATS, "epilogue tile and row coefficients");
  static_assert(BM <= NT, "one row coefficient per thread");
  float2* lnrow = reinterpret_cast<float2*>(smem + LDS_FLOATS - 2 * BM);
  const bool ln = a.ln_parts != nullptr;
  float4 lc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (ln) {
    if (col_ok) lc = *reinterpret_cast<const float4*>(a.ln_c + gn);
    if (tid < BM) lnrow[tid] = ln_row_merge(a, lnr);
  }
  const bool rstats = a.row_parts != nullptr;
#pragma unroll
  for (int pass = 0; pass < WMW / PASS_WM; ++pass) {
    if (pass > 0) __syncthreads();  // the previous pass's reads are done
    if (wm / PASS_WM == pass) {
      const int wr0 = (wm % PASS_WM) * WROWS;
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int r = wr0 + 32 * i + 8 * (v / 4) + 4 * g + (v % 4);
            const int c = wn * WN * 32 + 32 * j + l32;
            smem[r * PITCH + c] = acc[i][j][v];
          }
    }
    __syncthreads();
    const int prow0 = m0 + pass * PROWS;
    // residual rows first (loads before any store), then the stores
    float4 rv[RES ? IT : 1];
    if constexpr (RES) {
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int gm = min(prow0 + rr0 + it * RPI, a.M - 1);
        rv[it] = (Rp && col_ok) ? *reinterpret_cast<const float4*>(Rp + (int64_t)gm * a.ldr + gn)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      wait_vmcnt<0>();
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int r = rr0 + it * RPI;
      const int gm = prow0 + r;
      float4 v = *reinterpret_cast<const float4*>(smem + r * PITCH + 4 * c4);
      if (ln) {
        const float2 rc = lnrow[pass * PROWS + r];
        v.x = rc.x * v.x + rc.y * lc.x;
        v.y = rc.x * v.y + rc.y * lc.y;
        v.z = rc.x * v.z + rc.y * lc.z;
        v.w = rc.x * v.w + rc.y * lc.w;
      }
      v.x += bn.x;
      v.y += bn.y;
      v.z += bn.z;
      v.w += bn.w;
      if (ACT < 0) {
        v.x = apply_act(v.x, a.act, a.act_alpha);
        v.y = apply_act(v.y, a.act, a.act_alpha);
        v.z = apply_act(v.z, a.act, a.act_alpha);
        v.w = apply_act(v.w, a.act, a.act_alpha);
      } else if (ACT > 0) {
        v.x = apply_act(v.x, ACT);
        v.y = apply_act(v.y, ACT);
        v.z = apply_act(v.z, ACT);
        v.w = apply_act(v.w, ACT);
      }
      if constexpr (RES) {
        if (Rp) {
          v.x = rv[it].x + rs.x * v.x;
          v.y = rv[it].y + rs.y * v.y;
          v.z = rv[it].z + rs.z * v.z;
          v.w = rv[it].w + rs.w * v.w;
        }
      }
      if (rstats) {
        // (mean, M2) of the row's 64 columns held by this lane's 16-lane group (N % 64 == 0, so
        // col_ok is uniform over the group)
        const bool ok = col_ok && gm < a.M;
        const float mean = row16_sum(ok ? (v.x + v.y) + (v.z + v.w) : 0.f) * (1.f / 64.f);
        const float dx = v.x - mean, dy = v.y - mean, dz = v.z - mean, dw = v.w - mean;
        const float m2 = row16_sum(ok ? (dx * dx + dy * dy) + (dz * dz + dw * dw) : 0.f);
        if (ok && (c4 & 15) == 0)
          *reinterpret_cast<float2*>(a.row_parts + ((int64_t)gm * (a.N / 64) + gn / 64) * 2) =
              make_float2(mean, m2);
      }
      if (col_ok && gm < a.M) *reinterpret_cast<float4*>(Cp + (int64_t)gm * a.ldc + gn) = v;
    }
  }
}

// GLU epilogue: rows come in 32-row blocks [a0..a15 | b0..b15] (weights regrouped by the caller);
// output row 16*blk + r = (a_r + bias) * sigmoid(b_r + bias). In the accumulator layout register v
// (< 8) holds row rr = 8*(v/4) + 4*(l/32) + v%4 < 16 and register v + 8 holds row rr + 16, so every
// lane has both GLU partners.
template <int WMW, int WNW, int WM, int WN>
__device__ __forceinline__ void store_glu(const GemmArgs& a, const floatx16 (&acc)[WM][WN], int m0,
                                          int n0, int wm, int wn, int lane) {
  const int g = lane >> 5, l32 = lane & 31;
  float* __restrict__ Cp = a.C + (int64_t)blockIdx.z * a.sC;
  // bias values first (the compiler may not move these loads past the stores)
  float ba[WM][8], bb[WM][8];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int mblk = min(m0 + wm * WM * 32 + i * 32, a.M - 32);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int rr = 8 * (v / 4) + 4 * g + (v % 4);
      ba[i][v] = a.bias ? a.bias[mblk + rr] : 0.f;
      bb[i][v] = a.bias ? a.bias[mblk + 16 + rr] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int mblk = m0 + wm * WM * 32 + i * 32;
    if (mblk >= a.M) continue;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int gn = n0 + wn * WN * 32 + j * 32 + l32;
      if (gn >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int rr = 8 * (v / 4) + 4 * g + (v % 4);
        const float va = acc[i][j][v] + ba[i][v];
        const float vb = acc[i][j][v + 8] + bb[i][v];
        Cp[(int64_t)((mblk >> 5) * 16 + rr) * a.ldc + gn] = va * stable_sigmoid(vb);
      }
    }
  }
}

// Transposed-conv epilogue: row m = s*oc + r (phase r of output channel oc), column n = q; the value
// (+ bias[oc]) belongs at output position o = s*q + r - ct_pad of channel oc:
// C[oc * ldc + o] when 0 <= o < ct_len. A lane holds the s phases of one (oc, q) in registers
// v..v+s-1 (s = 4: rows 4i..4i+3 of a 32-row block), so consecutive lanes cover consecutive
// 4-sample runs of one output row. Bias values are loaded first (see store_tile). Every output
// sample is stored by exactly one (row, column), so with a.stats each workgroup also writes the
// GroupNorm(1) partial (count, mean, M2) of the samples it stored at
// stats[(batch * tiles + blockIdx.y * gridDim.x + blockIdx.x) * 3], tiles = gridDim.x * gridDim.y.
template <int WMW, int WNW, int WM, int WN>
__device__ __forceinline__ void store_ct(const GemmArgs& a, const floatx16 (&acc)[WM][WN], int m0,
                                         int n0, int wm, int wn, int lane) {
  const int g = lane >> 5, l32 = lane & 31;
  float* __restrict__ Cp = a.C + (int64_t)blockIdx.z * a.sC;
  const int s = a.ct_stride;
  float bmv[WM][16];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int gm = min(m0 + wm * WM * 32 + i * 32 + 8 * (v / 4) + 4 * g + (v % 4), a.M - 1);
      bmv[i][v] = a.bias ? a.bias[gm / s] : 0.f;
    }
  wait_vmcnt<0>();
  // four statistics accumulators, so the per-sample updates are not one dependent chain
  ShiftedStats st[4];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int mblk = m0 + wm * WM * 32 + i * 32;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int q = n0 + wn * WN * 32 + j * 32 + l32;
      if (q >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
        const int oc = gm / s, o = s * q + (gm - oc * s) - a.ct_pad;
        if (gm < a.M && o >= 0 && o < a.ct_len) {
          const float val = acc[i][j][v] + bmv[i][v];
          if (a.stats) st[v & 3].add(val);
          Cp[(int64_t)oc * a.ldc + o] = val;
        }
      }
    }
  }
  if (a.stats) {
    __shared__ float red[3 * WMW * WNW];
    float sn, smean, sm2;
    st[0].finish(sn, smean, sm2);
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      float n2, mean2, m22;
      st[k].finish(n2, mean2, m22);
      welford_combine(sn, smean, sm2, n2, mean2, m22);
    }
    block_welford(sn, smean, sm2, red);
    if (threadIdx.x == 0) {
      float* o = a.stats + ((int64_t)blockIdx.z * gridDim.x * gridDim.y + blockIdx.y * gridDim.x +
                            blockIdx.x) * 3;
      o[0] = sn;
      o[1] = smean;
      o[2] = sm2;
    }
  }
}

// K-split partial: the raw accumulators of K part p of batch b go to
// ws[((b * ksplit + p) * M + m) * N + n]; the caller reduces the parts (and applies the epilogue).
template <int WMW, int WNW, int WM, int WN>
__device__ __forceinline__ void store_part(const GemmArgs& a, const floatx16 (&acc)[WM][WN], int m0,
                                           int n0, int wm, int wn, int lane) {
  const int g = lane >> 5, l32 = lane & 31;
  float* __restrict__ wp = a.ws + (int64_t)blockIdx.z * a.M * a.N;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int mblk = m0 + wm * WM * 32 + i * 32;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int gn = n0 + wn * WN * 32 + j * 32 + l32;
      if (gn >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gm = mblk + 8 * (v / 4) + 4 * g + (v % 4);
        if (gm < a.M) wp[(int64_t)gm * a.N + gn] = acc[i][j][v];
      }
    }
  }
}

// EPI: 0 bias / activation / residual (store_tile), 1 GLU (store_glu: only the encoder's rewrite
// GEMMs use it), 2 transposed-conv scatter (store_ct), 3 K-split partials (store_part); each a
// separate instantiation.
//
// BF: A and B hold bf16 values (lda / ldb / sA / sB count bf16 elements). A stage is still 128
// bytes per row — 64 k — with the same swizzle; a lane's 16-byte fragment read is then 8
// consecutive k, exactly the operand of one v_mfma_f32_32x32x16_bf16 (lane group g supplies k
// slots 8g..8g+7), so chunk c = 4g + q4 of a stage feeds MFMA step q4 for A and B alike.
// The second launch bound asks for two workgroups per CU where two rings fit the 160 KB of LDS.
// BKN: B is k-major, [K][N] rows of stride ldb (the input of a transposed 2-D conv read in place,
// with a second matrix for rows kc1 .. kvalid - 1: the decoder's skip concat; rows past kvalid
// repeat the last valid one, whose products the zero columns of A cancel). A stage then holds
// B as [32 k rows][BN n], 16-byte chunk c of row r stored at slot c ^ (8 * ((r / 16) mod 2)), so
// the two lane groups (rows r and r + 16) read opposite halves of the 64 banks; each lane reads
// its 4 k of column n with four 4-byte LDS reads at row offsets that are immediates.
template <int WMW, int WNW, int WM, int WN, int S, int EPI, bool BF = false, bool BKN = false>
__global__ __launch_bounds__(WMW* WNW * 64,
                             (2 * S * (WMW * WM + WNW * WN) * 32 * BK * 4 <= 160 * 1024) ? 2 : 1)
void gemm_nk_lds_kernel(GemmArgs a) {
  using Cfg = LdsCfg<WMW, WNW, WM, WN, S>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN, A_INS = Cfg::A_INS, B_INS = Cfg::B_INS;
  constexpr int STAGE = Cfg::STAGE;
  constexpr int ES = BF ? 2 : 4;           // operand element bytes
  constexpr int BKE = BF ? 2 * BK : BK;    // k per 128-byte stage row
  __shared__ __attribute__((aligned(1024))) float smem[S * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNW, wn = wave % WNW;
  // blockIdx.z = batch * ksplit + K part (ksplit = 1 unless EPI == 3)
  const int ks = EPI == 3 ? a.ksplit : 1;
  const int bz = blockIdx.z / ks;
  // XCD-aware renumbering (workgroups go round robin over the 8 XCDs): consecutive logical tiles,
  // N fastest, land on one XCD and share the A panel in its L2.
  const int gx = gridDim.x;
  const int logical = xcd_logical_tile(blockIdx.x + gx * blockIdx.y, gx * gridDim.y);
  const int tn = logical % gx, tm = logical / gx;
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = a.M, N = a.N, K = a.K;
  const int nk = K / BKE / ks, kt0 = (int)(blockIdx.z % ks) * nk;  // this workgroup's stages
  // a folded LayerNorm's row partials (thread r: row m0 + r % BM)
  LnRow lnr;
  if constexpr (EPI == 0 && !BF) lnr = ln_row_load(a, m0 + tid % BM);
  const char* __restrict__ A = reinterpret_cast<const char*>(a.A) + (int64_t)bz * a.sA * ES;
  const char* __restrict__ B = reinterpret_cast<const char*>(a.B) + (int64_t)bz * a.sB * ES;

  // Per-lane byte offsets of this wave's stage loads from the operand base (rows past M / N are
  // clamped to the last row: they are read but their products are never stored). The base moves
  // by one stage per load round in SGPRs, so the loads need no per-stage VALU address work.
  const int lr = lane >> 3, ls = lane & 7;
  unsigned aoffg[A_INS], boffg[B_INS];
#pragma unroll
  for (int i = 0; i < A_INS; ++i) {
    const int rr = (wave * A_INS + i) * 8 + lr;
    const int gm = min(m0 + rr, M - 1);
    aoffg[i] = (unsigned)(ES * gm * a.lda + 16 * (ls ^ chunk_swizzle(rr)));
  }
#pragma unroll
  for (int i = 0; i < B_INS; ++i) {
    const int rr = (wave * B_INS + i) * 8 + lr;
    const int gn = min(n0 + rr, N - 1);
    boffg[i] = (unsigned)(ES * gn * a.ldb + 16 * (ls ^ chunk_swizzle(rr)));
  }
  // BKN: instruction i of this wave fills stage rows (wave * B_INS + i) * RPI + lane / CPR
  // (CPR 16-byte chunks per row), slot lane % CPR: that row's column chunk slot ^ swizzle,
  // clamped to the last whole chunk of the row (columns past N are never stored)
  constexpr int CPR = BN / 4, RPI = 64 / CPR;
  static_assert(!BKN || (BN >= 64 && !BF && EPI == 0), "k-major B: 64+ columns, fp32, plain epilogue");
  int bkr[BKN ? B_INS : 1], bkc[BKN ? B_INS : 1];
  if constexpr (BKN) {
#pragma unroll
    for (int i = 0; i < B_INS; ++i) {
      const int r = (wave * B_INS + i) * RPI + lane / CPR, slot = lane % CPR;
      bkr[i] = r;
      bkc[i] = min(n0 + 4 * (slot ^ (8 * ((r >> 4) & 1))), N - 4);
    }
  }
  const float* B1 = a.B + (int64_t)bz * a.sB;
  const float* B2 = a.B2 ? a.B2 + (int64_t)bz * a.sB2 : B1;
  const unsigned lds0 = lds_address(smem);
  auto issue = [&](int kt, int slot) {
    const unsigned base = lds0 + 4u * (unsigned)(slot * STAGE);
    const float* ak = reinterpret_cast<const float*>(A + (int64_t)(kt0 + kt) * BKE * ES);
    const float* bk = reinterpret_cast<const float*>(B + (int64_t)(kt0 + kt) * BKE * ES);
#pragma unroll
    for (int i = 0; i < A_INS; ++i)
      lds_dma16_s(ak, aoffg[i],
                  __builtin_amdgcn_readfirstlane(base + 4u * ((wave * A_INS + i) * 8 * BK)));
    if constexpr (BKN) {
#pragma unroll
      for (int i = 0; i < B_INS; ++i) {
        const int k = min((kt0 + kt) * BK + bkr[i], a.kvalid - 1);
        const float* src = (k < a.kc1 ? B1 + (int64_t)k * a.ldb
                                      : B2 + (int64_t)(k - a.kc1) * a.ldb) + bkc[i];
        lds_dma16(src, __builtin_amdgcn_readfirstlane(
                           base + 4u * (BM * BK + (wave * B_INS + i) * 8 * BK)));
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_INS; ++i)
        lds_dma16_s(bk, boffg[i], __builtin_amdgcn_readfirstlane(
                                      base + 4u * (BM * BK + (wave * B_INS + i) * 8 * BK)));
    }
  };

  floatx16 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // LDS word offsets of this lane's fragment rows in slot 0 (other slots: a constant offset)
  const int g = lane >> 5, l32 = lane & 31;
  int aoff[WM], boff[WN], asw[WM], bsw[WN];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int rr = wm * WM * 32 + 32 * i + l32;
    aoff[i] = rr * BK;
    asw[i] = chunk_swizzle(rr);
  }
#pragma unroll
  for (int j = 0; j < WN; ++j) {
    const int rr = wn * WN * 32 + 32 * j + l32;
    if constexpr (BKN) {  // column rr of row 16 g of the stage's B
      boff[j] = BM * BK + 16 * g * BN + ((((rr >> 2) ^ (8 * g)) << 2) | (rr & 3));
      bsw[j] = 0;
    } else {
      boff[j] = BM * BK + rr * BK;
      bsw[j] = chunk_swizzle(rr);
    }
  }

  // Software pipeline: the fragments of stage kt sit in registers while the matrix cores work on
  // them. Halfway through stage kt (after the MFMAs of its first two 8-deep k slices) the waves
  // meet at the barrier that makes stage kt+1 visible and frees the slot of stage kt, issue the
  // loads of stage kt+S into that slot, and read stage kt+1's fragments interleaved with the
  // second half's MFMAs, so neither the barrier nor the LDS latency stalls the matrix pipe.
  // The stage loop is unrolled by U (a multiple of S and of 2), so every ring slot and the two
  // fragment register sets are compile-time choices: no address arithmetic and no register copies
  // between stages.
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < nk) issue(s, s);
  float4 fa[2][4][WM], fb[2][4][WN];
  auto read_frags = [&](int slot, float4 (&xa)[4][WM], float4 (&xb)[4][WN]) {
    const float* base = smem + slot * STAGE;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int c = 4 * g + q4;
#pragma unroll
      for (int i = 0; i < WM; ++i)
        xa[q4][i] = *reinterpret_cast<const float4*>(base + aoff[i] + 4 * (c ^ asw[i]));
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        if constexpr (BKN) {  // k = 16 g + 4 q4 + s: rows 4 q4 + s below the lane's row base
          const float* bp = base + boff[j] + 4 * q4 * BN;
          xb[q4][j] = make_float4(bp[0], bp[BN], bp[2 * BN], bp[3 * BN]);
        } else {
          xb[q4][j] = *reinterpret_cast<const float4*>(base + boff[j] + 4 * (c ^ bsw[j]));
        }
      }
    }
  };
  auto mfma_slice = [&](const float4 (&xa)[4][WM], const float4 (&xb)[4][WN], int q4) {
    if constexpr (BF) {
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, xa[q4][i]), __builtin_bit_cast(bf16x8, xb[q4][j]),
              acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
          for (int j = 0; j < WN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[q4][i][s], xb[q4][j][s],
                                                             acc[i][j], 0, 0, 0);
    }
  };
  // stage 0: at most the S-1 newer stages may still be in flight
  if (S - 1 < nk) wait_vmcnt<(S - 1) * Cfg::L>();
  else wait_vmcnt<0>();
  stage_barrier();
  read_frags(0, fa[0], fb[0]);
  constexpr int U = S % 2 == 0 ? S : 2 * S;
  for (int kt0 = 0; kt0 + 1 < nk; kt0 += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kt = kt0 + u;
      if (kt + 1 < nk) {
        const int cur = u % 2, nxt = 1 - u % 2;
        mfma_slice(fa[cur], fb[cur], 0);
        mfma_slice(fa[cur], fb[cur], 1);
        __builtin_amdgcn_sched_barrier(0);  // the first half's MFMAs stay ahead of the barrier
        // stage kt+1 is complete for this wave once at most the S-2 newer stages are outstanding
        if (kt + S - 1 < nk) wait_vmcnt<(S - 2) * Cfg::L>();
        else wait_vmcnt<0>();
        stage_barrier();  // ... and for every wave; every wave's reads of stage kt are done
        if (kt + S < nk) issue(kt + S, u % S);  // stage kt+S goes to the slot stage kt frees
        read_frags((u + 1) % S, fa[nxt], fb[nxt]);
        mfma_slice(fa[cur], fb[cur], 2);
        mfma_slice(fa[cur], fb[cur], 3);
        // fragment reads alternate with the first MFMAs of the second half, so the last read has
        // the remaining MFMAs to complete before the next stage needs it
        constexpr int kReads = 4 * WM + (BKN ? 16 : 4) * WN, kMfma = 8 * WM * WN;
        if constexpr (BF) {
          // bf16: one MFMA per fragment pair and k step, 2 * WM * WN in the second half; the
          // reads are spread over them
          constexpr int kM = 2 * WM * WN, kR = (kReads + kM - 1) / kM;
#pragma unroll
          for (int r = 0; r < kM; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x100, kR, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          }
        } else {
#pragma unroll
          for (int r = 0; r < kReads; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          }
          __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
        }
      }
    }
  }
  // last stage: its fragments are in set (nk - 1) % 2 (moved to set 0 once, so a single copy of
  // the MFMAs owns the accumulators)
  if ((nk - 1) & 1) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
#pragma unroll
      for (int i = 0; i < WM; ++i) fa[0][q4][i] = fa[1][q4][i];
#pragma unroll
      for (int j = 0; j < WN; ++j) fb[0][q4][j] = fb[1][q4][j];
    }
  }
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) mfma_slice(fa[0], fb[0], q4);

  // ---------------------------------------------------------------- epilogue
  // The activation and residual form are uniform: one specialised copy of the store loop each
  // for the forms the transformer uses, a generic one for the rest.
  const bool res = a.R != nullptr, bm = a.bias_mode == BIAS_M;
  // row-ordered stores through LDS where rows are 16-byte aligned (see store_tile_lds)
  const bool rows16 = (a.N % 4 == 0) && (a.ldc % 4 == 0) && (a.sC % 4 == 0) &&
                      ((reinterpret_cast<uintptr_t>(a.C) & 15) == 0) &&
                      (!res || ((a.ldr % 4 == 0) && (a.sR % 4 == 0) &&
                                (reinterpret_cast<uintptr_t>(a.R) & 15) == 0)) &&
                      (a.bias_mode != BIAS_N || (reinterpret_cast<uintptr_t>(a.bias) & 15) == 0) &&
                      (!a.rscale || (reinterpret_cast<uintptr_t>(a.rscale) & 15) == 0);
  if constexpr (EPI == 0) {
    if (rows16 && !bm) {
      __syncthreads();  // every wave's last fragment reads of the LDS ring are done
      if (a.act == 0 && !res)
        store_tile_lds<WMW, WNW, WM, WN, 0, false, S * STAGE>(a, acc, m0, n0, wm, wn, lane, smem,
                                                              lnr);
      else if (a.act == 0)
        store_tile_lds<WMW, WNW, WM, WN, 0, true, S * STAGE>(a, acc, m0, n0, wm, wn, lane, smem,
                                                             lnr);
      else if (a.act == 3 && !res)
        store_tile_lds<WMW, WNW, WM, WN, 3, false, S * STAGE>(a, acc, m0, n0, wm, wn, lane, smem,
                                                              lnr);
      else
        store_tile_lds<WMW, WNW, WM, WN, -1, true, S * STAGE>(a, acc, m0, n0, wm, wn, lane, smem,
                                                              lnr);
      return;
    }
  }
  if constexpr (EPI == 1) store_glu<WMW, WNW, WM, WN>(a, acc, m0, n0, wm, wn, lane);
  else if constexpr (EPI == 2) store_ct<WMW, WNW, WM, WN>(a, acc, m0, n0, wm, wn, lane);
  else if constexpr (EPI == 3) store_part<WMW, WNW, WM, WN>(a, acc, m0, n0, wm, wn, lane);
  else if (a.act == 0 && !res && !bm)
    store_tile<WMW, WNW, WM, WN, 0, false, true>(a, acc, m0, n0, wm, wn, lane);
  else if (a.act == 0 && !bm)
    store_tile<WMW, WNW, WM, WN, 0, true, false>(a, acc, m0, n0, wm, wn, lane);
  else if (a.act == 3 && !res && !bm)
    store_tile<WMW, WNW, WM, WN, 3, false, true>(a, acc, m0, n0, wm, wn, lane);
  else store_tile<WMW, WNW, WM, WN, -1, true, false>(a, acc, m0, n0, wm, wn, lane);
}

struct LdsTile {
  int id, bm, bn;
  double eff;  // relative matrix-core efficiency of the tile shape (measured)
};
constexpr LdsTile kLdsTiles[] = {
    {0, 128, 128, 1.00},  // <2,2,2,2> S2, 64 KB LDS, 2 workgroups per CU
    {1, 128, 64, 0.93},   // <2,2,2,1> S3
    {2, 64, 128, 0.93},   // <2,2,1,2> S3
    {3, 64, 64, 0.88},    // <2,2,1,1> S4
};

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int forced_lds_tile() {
  static const int v = [] {
    const char* e = std::getenv("MNN_GEMM_LDS_TILE");
    return e ? std::atoi(e) : -1;
  }();
  return v;
}

// Per-CU critical path: the most tiles any CU runs x tile area / shape efficiency. A CU that holds a
// single workgroup runs it at about 0.6 of the rate of two co-resident ones (the issuing wave waits
// for each LDS-DMA load to be accepted, and no other workgroup's MFMAs fill those cycles; measured on
// the transformer shapes), so a grid of at most one tile per CU is charged 1/0.6.
const LdsTile& choose_lds_tile(const GemmArgs& a) {
  const int f = forced_lds_tile();
  if (f >= 0 && f < (int)(sizeof(kLdsTiles) / sizeof(kLdsTiles[0]))) return kLdsTiles[f];
  const LdsTile* best = &kLdsTiles[0];
  double best_cost = 1e300;
  for (const LdsTile& t : kLdsTiles) {
    const int64_t tiles = (int64_t)cdiv(a.M, t.bm) * cdiv(a.N, t.bn) * a.batch * a.ksplit;
    const int64_t per_cu = cdiv(tiles, (int64_t)256);
    const double cost = (double)per_cu * t.bm * t.bn / t.eff / (per_cu == 1 ? 0.6 : 1.0);
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = &t;
    }
  }
  return *best;
}

template <int WMW, int WNW, int WM, int WN, int S, bool BF = false>
void launch_lds(const LaunchCtx& c, const GemmArgs& a) {
  using Cfg = LdsCfg<WMW, WNW, WM, WN, S>;
  dim3 grid(cdiv(a.N, Cfg::BN), cdiv(a.M, Cfg::BM), a.batch * a.ksplit), block(Cfg::NT);
  if constexpr (BF) {  // bf16 operands: bias / activation / residual epilogue only
    launch(c, a.name ? a.name : "gemm_bf16_mfma_nk",
           gemm_nk_lds_kernel<WMW, WNW, WM, WN, S, 0, true>, grid, block, 0, a);
  } else {
    const char* name = a.name ? a.name : "gemm_f32_mfma_nk";
    if (a.blayout == B_KN)
      launch(c, name, gemm_nk_lds_kernel<WMW, WNW, WM, WN, S, 0, false, true>, grid, block, 0, a);
    else if (a.ksplit > 1)
      launch(c, name, gemm_nk_lds_kernel<WMW, WNW, WM, WN, S, 3>, grid, block, 0, a);
    else if (a.glu) launch(c, name, gemm_nk_lds_kernel<WMW, WNW, WM, WN, S, 1>, grid, block, 0, a);
    else if (a.ct_stride > 0)
      launch(c, name, gemm_nk_lds_kernel<WMW, WNW, WM, WN, S, 2>, grid, block, 0, a);
    else launch(c, name, gemm_nk_lds_kernel<WMW, WNW, WM, WN, S, 0>, grid, block, 0, a);
  }
}

}  // namespace

namespace {
// The folded-LayerNorm and row-statistics epilogue forms exist in the row-ordered store only:
// the conditions under which the kernel takes it (fp32, plain epilogue, 16-byte aligned rows),
// batch 1, and whole 64-column groups.
bool ln_fold_epilogue_ok(const GemmArgs& a) {
  const bool res = a.R != nullptr;
  const bool rows16 = a.N % 4 == 0 && a.ldc % 4 == 0 && aligned16(a.C) &&
                      (!res || (a.ldr % 4 == 0 && aligned16(a.R))) &&
                      (a.bias_mode != BIAS_N || aligned16(a.bias)) &&
                      (!a.rscale || aligned16(a.rscale));
  return rows16 && a.batch == 1 && !a.ab_bf16 && !a.glu && a.ct_stride == 0 && a.ksplit == 1 &&
         a.stats == nullptr && a.bias_mode != BIAS_M &&
         (!a.ln_parts || (a.K % 64 == 0 && a.K <= 64 * kLnMaxParts && a.ln_c &&
                          aligned16(a.ln_c) && aligned16(a.ln_parts))) &&
         (!a.row_parts || (a.N % 64 == 0 && (reinterpret_cast<uintptr_t>(a.row_parts) & 7) == 0));
}
}  // namespace

bool gemm_nk_lds_supported(const GemmArgs& a) {
  if (a.ab_bf16) {
    // bf16 operands: 64 k per stage, rows 16-byte aligned (8 elements), plain epilogue
    const bool off32 = ((int64_t)(a.M - 1) * a.lda + a.K) * 2 < ((int64_t)1 << 32) &&
                       ((int64_t)(a.N - 1) * a.ldb + a.K) * 2 < ((int64_t)1 << 32);
    return off32 && a.blayout == B_NK && a.precision == MNN_PRECISION_BF16 &&
           a.K % (2 * BK) == 0 && a.lda % 8 == 0 && a.ldb % 8 == 0 && a.sA % 8 == 0 &&
           a.sB % 8 == 0 && aligned16(a.A) && aligned16(a.B) && a.stats == nullptr &&
           a.pro_coef == nullptr && a.pro_stats == nullptr && !a.glu && a.ct_stride == 0 &&
           a.ksplit == 1 && a.bias_mode != BIAS_M;
  }
  // per-lane load offsets are 32-bit byte offsets from the operand (batch) base
  const bool off32 = ((int64_t)(a.M - 1) * a.lda + a.K) * 4 < ((int64_t)1 << 32) &&
                     ((int64_t)(a.N - 1) * a.ldb + a.K) * 4 < ((int64_t)1 << 32);
  if (a.blayout == B_KN) {
    // k-major B read in place (opt-in): plain epilogue, whole 16-byte chunks per row
    return a.bkn_lds && a.precision == MNN_PRECISION_F32 && a.K % BK == 0 && a.N >= 4 &&
           a.N % 4 == 0 && a.ldb % 4 == 0 && a.sB % 4 == 0 && a.sB2 % 4 == 0 && aligned16(a.B) &&
           (!a.B2 || aligned16(a.B2)) && a.kvalid >= 1 && a.kc1 >= 0 && a.kc1 <= a.kvalid &&
           ((int64_t)(a.M - 1) * a.lda + a.K) * 4 < ((int64_t)1 << 32) && a.lda % 4 == 0 &&
           a.sA % 4 == 0 && aligned16(a.A) && a.pro_coef == nullptr && a.pro_stats == nullptr &&
           !a.glu && a.ct_stride == 0 && a.ksplit == 1 && a.stats == nullptr && !a.ln_parts &&
           !a.row_parts && a.bias_mode != BIAS_M && a.R == nullptr && a.act == 0;
  }
  return off32 && a.blayout == B_NK && a.precision == MNN_PRECISION_F32 && a.K % BK == 0 &&
         a.lda % 4 == 0 && a.ldb % 4 == 0 && a.sA % 4 == 0 && a.sB % 4 == 0 && aligned16(a.A) &&
         aligned16(a.B) && a.pro_coef == nullptr && a.pro_stats == nullptr &&
         (!a.glu || (a.M % 32 == 0 && a.bias_mode != BIAS_N && a.R == nullptr && a.act == 0)) &&
         (a.ct_stride == 0 || (!a.glu && a.R == nullptr && a.act == 0 && a.bias_mode != BIAS_N)) &&
         a.ksplit >= 1 && (a.K / BK) % a.ksplit == 0 &&
         (a.ksplit == 1 || (a.ws != nullptr && !a.glu)) &&
         (a.stats == nullptr || (a.ct_stride > 0 && a.ksplit == 1)) &&
         ((!a.ln_parts && !a.row_parts) || ln_fold_epilogue_ok(a));
}

int64_t gemm_nk_lds_tiles(const GemmArgs& a) {
  if (a.ab_bf16) return -1;
  const LdsTile& t = choose_lds_tile(a);
  return (int64_t)cdiv(a.M, t.bm) * cdiv(a.N, t.bn);
}

void gemm_nk_lds(const LaunchCtx& c, const GemmArgs& a) {
  MNN_REQUIRE(gemm_nk_lds_supported(a), MNN_ERR_INVALID_ARGUMENT,
              "gemm_nk_lds: operands outside the LDS-DMA path's contract");
  if (a.ab_bf16) {
    // bf16: a stage holds 64 k, so its matrix work is an eighth of the fp32 kernel's while its
    // loads are as large: four-stage rings keep more load latency in flight. 128x128 tiles where
    // they fill the CUs, 64x64 tiles for grids of fewer than 256 of them.
    const int f = forced_lds_tile();
    const int64_t big = (int64_t)cdiv(a.M, 128) * cdiv(a.N, 128) * a.batch;
    if (f == 3 || (f < 0 && big < 256)) return launch_lds<2, 2, 1, 1, 4, true>(c, a);
    return launch_lds<2, 2, 2, 2, 4, true>(c, a);
  }
  switch (choose_lds_tile(a).id) {
    case 0: return launch_lds<2, 2, 2, 2, 2>(c, a);
    case 1: return launch_lds<2, 2, 2, 1, 3>(c, a);
    case 2: return launch_lds<2, 2, 1, 2, 3>(c, a);
    default: return launch_lds<2, 2, 1, 1, 4>(c, a);
  }
}

}  // namespace k
}  // namespace mnn
