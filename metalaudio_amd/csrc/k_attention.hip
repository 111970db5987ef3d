// Fused multi-head attention forward: O = softmax(Q K^T * scale) V per (batch, head), with an
// online softmax so the [Sq, Sk] score matrix never leaves registers. Replaces the reference's
// attention_scores / attention_softmax / attention_output kernels, which write fp32 [H, Sq, Sk]
// scores to memory (Attention.swift:301-327, 675-705, 744-768). Semantics follow the reference
// CPU restatement (Attention.swift:840-976): head h uses columns [h*hd, (h+1)*hd) of the packed
// projections, scale = 1/sqrt(hd), P = exp(s - max) / (sum + 1e-10), O is written [S, H*hd].
//
// Matrix-core formulation (v_mfma_f32_16x16x4_f32, fp32 operands): each wave owns QW query
// columns and computes the TRANSPOSED scores S^T = K Q^T for a block of 64 keys. The accumulator
// layout of S^T (lane l holds keys 4*(l/16)+r, query l%16) is exactly the B-operand layout the
// next product O^T += V^T P^T needs when its k-slots are assigned the same keys, so P goes from
// the softmax straight into the PV matrix product without a trip through LDS. Per query, the
// running max is shared across the four lane groups with two xor-shuffles; running sums stay
// per lane and are combined once at the end. Q is pre-multiplied by scale*log2(e) so the
// exponentials are exp2. K/V blocks move HBM -> LDS by LDS-DMA (lds_dma.hpp) into two-slot K and
// V rings, with one barrier per block.
#include "device_utils.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

#include <algorithm>
#include <type_traits>

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int BKV = 64;

// LDS layout: two K slots then two V slots, each one 64-key block of HD/4 16-byte chunks per row
// plus one padding chunk (row pitch HD + 4 floats keeps 16 consecutive rows on distinct banks).
// One LDS-DMA instruction fills 64 consecutive chunks, so a slot is PC instructions; the padding
// chunk is loaded as a harmless duplicate of the row's last chunk.
template <int HD>
struct AttnCfg {
  static constexpr int PC = HD / 4 + 1;       // chunks per padded row
  static constexpr int LDK = PC * 4;          // floats per padded row
  static constexpr int SLOT = PC * 256;       // floats per slot (64 rows)
  // workgroups per CU the LDS allows (160 KiB per CU); head dim 48 fits three
  static constexpr int OCC = (4 * SLOT * 4) * 3 <= 160 * 1024 ? 3 : 2;
};

// Pipeline per 64-key block j: the K fragments of block j are already in registers, so the
// scores S^T = K Q^T and the softmax run without touching LDS; then the waves meet at the one
// barrier of the block, which makes V(j) and K(j+1) visible and frees the slots of K(j) and
// V(j-1); the loads of K(j+2) and V(j+1) go into those slots, and the PV product of block j runs
// with V(j)'s fragment reads in front of it and K(j+1)'s fragment reads interleaved with it.
template <int HD, int QW>
__global__ __launch_bounds__(256, AttnCfg<HD>::OCC) void attn_fwd_f32_kernel(AttnArgs a) {
  using Cfg = AttnCfg<HD>;
  constexpr int NW = 4, BQ = NW * QW, NU = QW / 16, HS = HD / 4, ND = HD / 16;
  constexpr int LDK = Cfg::LDK, PC = Cfg::PC, SLOT = Cfg::SLOT;
  constexpr int LW = (PC + NW - 1) / NW;  // wave loads per wave and slot (the last may be idle)
  __shared__ __attribute__((aligned(1024))) float smem[4 * SLOT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, l16 = lane & 15;
  // XCD-aware numbering (workgroups go round robin over the 8 XCDs): consecutive logical work
  // units, query blocks fastest, land on one XCD, so the query blocks of one (batch, head) share
  // its K and V in that XCD's L2 instead of every XCD streaming every head's K and V
  const int nq = gridDim.x, nh = gridDim.y;
  const int unit = xcd_logical_tile(blockIdx.x + nq * (blockIdx.y + nh * blockIdx.z),
                                    nq * nh * gridDim.z);
  const int qblk = unit % nq, h = (unit / nq) % nh, bz = unit / (nq * nh);
  const int ns = a.nsplit, b = bz / ns, sp = bz % ns;
  const int qw0 = qblk * BQ + wave * QW;
  // key blocks [kb0, kb0 + nl) of this workgroup's key range (all of them without a key split)
  const int nblk_all = (a.Sk + BKV - 1) / BKV;
  const int kb0 = (int)((int64_t)sp * nblk_all / ns);
  const int nblk = (int)((int64_t)(sp + 1) * nblk_all / ns) - kb0;

  const float* __restrict__ qb = a.q + (int64_t)b * a.q_bs + h * HD;
  const float* __restrict__ kb = a.k + (int64_t)b * a.kv_bs + h * HD;
  const float* __restrict__ vb = a.v + (int64_t)b * a.kv_bs + h * HD;

  // wave load j = i*NW + wave of a slot covers chunks [64j, 64j+64); lane byte offsets
  // (row * kv_rs + 4 * chunk) * 4 of a full block are the same for K and V and computed once
  unsigned soff[LW];
#pragma unroll
  for (int i = 0; i < LW; ++i) {
    const int e = min(i * NW + wave, PC - 1) * 64 + lane;
    soff[i] = 4u * (unsigned)((e / PC) * (int)a.kv_rs + 4 * min(e % PC, PC - 2));
  }
  const unsigned lds0 = lds_address(smem);
  // K block blk -> slot blk % 2, V block blk -> slot 2 + blk % 2 (`par` = blk % 2, compile-time at
  // the call sites in the block loop)
  auto issue = [&](int blk, bool isv, int par) {
    const unsigned base = lds0 + 4u * (unsigned)(((isv ? 2 : 0) + par) * SLOT);
    const float* src = (isv ? vb : kb) + (int64_t)blk * BKV * a.kv_rs;
    // The tail block's clamped offsets are computed in a branch of their own, around their own
    // loads: with only the offset under the branch the compiler if-converted it, and every block
    // paid the clamp arithmetic (~50 VALU instructions per 64-key block, beside 96 MFMAs).
    if (blk * BKV + BKV > a.Sk) {  // rows past the last key re-read the last key (scores masked)
#pragma unroll
      for (int i = 0; i < LW; ++i) {
        const int j = i * NW + wave;
        if (j < PC) {
          const int e = j * 64 + lane;
          const unsigned off = 4u * (unsigned)(min(e / PC, a.Sk - 1 - blk * BKV) * (int)a.kv_rs +
                                               4 * min(e % PC, PC - 2));
          lds_dma16_s(src, off, base + 4u * (unsigned)(j * 256));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < LW; ++i) {
        const int j = i * NW + wave;
        if (j < PC) lds_dma16_s(src, soff[i], base + 4u * (unsigned)(j * 256));
      }
    }
  };
  issue(kb0, false, 0);
  issue(kb0, true, 0);
  if (nblk > 1) issue(kb0 + 1, false, 1);

  // Q fragments: B operand of S^T = K Q^T; lane group G owns d in [G*HS, (G+1)*HS)
  const float qscale = a.scale * 1.4426950408889634f;
  float qf[NU][HS];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int q = qw0 + 16 * u + l16;
    if (q < a.Sq) {
      const float* p = qb + (int64_t)q * a.q_rs + G * HS;
#pragma unroll
      for (int s4 = 0; s4 < HS / 4; ++s4) {
        float4 t = *reinterpret_cast<const float4*>(p + 4 * s4);
        qf[u][4 * s4 + 0] = t.x * qscale; qf[u][4 * s4 + 1] = t.y * qscale;
        qf[u][4 * s4 + 2] = t.z * qscale; qf[u][4 * s4 + 3] = t.w * qscale;
      }
    } else {
#pragma unroll
      for (int s = 0; s < HS; ++s) qf[u][s] = 0.f;
    }
  }

  // O^T accumulators: MFMA w holds output rows d = dmap(i, w) (i = MFMA row). Head dim 64 uses
  // d = 4i + w: a lane's four values of one V row are one 16-byte LDS read and its outputs are
  // contiguous. Other head dims use d = i + 16w: a lane's values of one V row sit 16 floats apart,
  // so the reads of a key tile's four rows are all within the 8-bit offset range of paired LDS
  // reads from one base address (no per-read address arithmetic).
  floatx4 o[ND][NU];
  float mref[NU], lsum[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    mref[u] = 0.f;
    lsum[u] = 0.f;
#pragma unroll
    for (int w = 0; w < ND; ++w) o[w][u] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  // K fragments of key tile t: rows 16t + l16, d in [G*HS, (G+1)*HS)
  float4 kfr[HS / 4][4];
  auto read_k = [&](int par, float4 (&kr)[HS / 4][4]) {
    const float* ks = smem + par * SLOT;
#pragma unroll
    for (int s4 = 0; s4 < HS / 4; ++s4)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        kr[s4][t] = *reinterpret_cast<const float4*>(ks + (16 * t + l16) * LDK + G * HS + 4 * s4);
  };
  wait_vmcnt<0>();
  stage_barrier();
  read_k(0, kfr);

  // One 64-key block (blk counts from the start of the workgroup's key range); PAR = blk % 2
  // selects the ring slots at compile time, so every LDS address below is a lane base plus an
  // immediate offset. The block loop runs the two parities in turn.
  auto block_step = [&](int blk, auto parc) {
    constexpr int PAR = decltype(parc)::value;
    const int kv0 = (kb0 + blk) * BKV;
    // S^T tiles: 4 key tiles x NU query tiles, k-steps outermost so the 4*NU independent
    // accumulators interleave and no MFMA waits on the previous one
    // accumulators start at -mref, so the scores come out relative to the reference maximum
    floatx4 st[4][NU];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < NU; ++u) st[t][u] = floatx4{-mref[u], -mref[u], -mref[u], -mref[u]};
#pragma unroll
    for (int s4 = 0; s4 < HS / 4; ++s4)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int u = 0; u < NU; ++u) {
            const float kv = s == 0 ? kfr[s4][t].x : s == 1 ? kfr[s4][t].y : s == 2 ? kfr[s4][t].z : kfr[s4][t].w;
            st[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, qf[u][4 * s4 + s], st[t][u], 0, 0, 0);
          }
    // mask keys beyond Sk
    if (kv0 + BKV > a.Sk) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kv0 + 16 * t + 4 * G + r >= a.Sk)
#pragma unroll
            for (int u = 0; u < NU; ++u) st[t][u][r] = -INFINITY;
    }
    // Online softmax with a lazily moved reference: p = exp2(s - mref). The first block sets mref
    // to its maximum; later blocks move it (rescaling l and O) only when their maximum exceeds
    // it by more than kTau, so p <= 2^kTau and most blocks skip the rescale. l >= 1 always holds
    // (the block that set mref contributes exp2(0)), so nothing underflows.
    constexpr float kTau = 8.f;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[t][u][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      if (blk == 0 || mx > kTau) {  // uniform per query column
        const float alpha = __builtin_amdgcn_exp2f(-mx);
        lsum[u] *= alpha;
        mref[u] += mx;
#pragma unroll
        for (int w = 0; w < ND; ++w) o[w][u] *= alpha;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) st[t][u][r] -= mx;
      }
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(st[t][u][r]);
          st[t][u][r] = p;
          ps += p;
        }
      lsum[u] += ps;
    }
    __builtin_amdgcn_sched_barrier(0);  // scores and softmax stay ahead of the barrier
    // V(blk) and K(blk+1) have landed for this wave (they are the only loads in flight) ...
    wait_vmcnt<0>();
    stage_barrier();  // ... and for every wave; K(blk) and V(blk-1) are no longer read
    if (blk + 2 < nblk) issue(kb0 + blk + 2, false, PAR);
    if (blk + 1 < nblk) issue(kb0 + blk + 1, true, 1 - PAR);
    // PV in four key tiles t. The V rows of tile t+1 (key 16(t+1) + 4G + r, this lane's d) and
    // the K fragments of tile t of the next block are read while tile t's MFMAs run; the
    // scheduling barriers keep each tile's reads next to it, which bounds the live registers.
    const float* vs = smem + (2 + PAR) * SLOT;
    const float* ksn = smem + (1 - PAR) * SLOT;
    const bool next = blk + 1 < nblk;
    auto read_v = [&](int t, float (&vr)[4][ND]) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (ND == 4) {
          const float4 v4 =
              *reinterpret_cast<const float4*>(vs + (16 * t + 4 * G + r) * LDK + 4 * l16);
          vr[r][0] = v4.x; vr[r][1] = v4.y; vr[r][2] = v4.z; vr[r][3] = v4.w;
        } else {
          const float* vrow = vs + (16 * t + 4 * G + r) * LDK + l16;
#pragma unroll
          for (int w = 0; w < ND; ++w) vr[r][w] = vrow[16 * w];
        }
      }
    };
    float vf[2][4][ND];
    read_v(0, vf[0]);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < 4) read_v(t + 1, vf[(t + 1) & 1]);
      if (next) {
#pragma unroll
        for (int s4 = 0; s4 < HS / 4; ++s4)
          kfr[s4][t] = *reinterpret_cast<const float4*>(ksn + (16 * t + l16) * LDK + G * HS + 4 * s4);
      }
      // O^T += V^T P^T ; k-slot G of step (t, r) is key 16t + 4G + r
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int w = 0; w < ND; ++w)
#pragma unroll
          for (int u = 0; u < NU; ++u)
            o[w][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[t & 1][r][w], st[t][u][r], o[w][u],
                                                           0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int blk = 0;
  for (; blk + 1 < nblk; blk += 2) {
    block_step(blk, std::integral_constant<int, 0>{});
    block_step(blk + 1, std::integral_constant<int, 1>{});
  }
  if (blk < nblk) block_step(blk, std::integral_constant<int, 0>{});

  // normalise and write O[b][q][h*HD + d]; for query l16 a lane holds d = dmap(4G + r, w):
  // 16 consecutive values (head dim 64) or ND runs of 4 (d = 16w + 4G + r). With a key split the
  // unnormalised O of the range goes to its partial row, with the range's reference maximum and
  // sum (attn_combine_kernel merges the ranges).
  const bool part = ns > 1;
  const int64_t prow0 = (((int64_t)sp * a.B + b) * a.H + h) * a.Sq;  // partial row of query 0
  float* __restrict__ ob = part ? a.part + prow0 * HD : a.o + (int64_t)b * a.o_bs + h * HD;
  const int64_t ors = part ? HD : a.o_rs;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    float l = lsum[u];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = part ? 1.f : 1.f / (l + 1e-10f);
    const int q = qw0 + 16 * u + l16;
    if (q < a.Sq) {
      if (part && G == 0) {
        const int64_t ml = (int64_t)ns * a.B * a.H * a.Sq * HD;  // maxima, then sums
        a.part[ml + prow0 + q] = mref[u];
        a.part[ml + (int64_t)ns * a.B * a.H * a.Sq + prow0 + q] = l;
      }
      float* orow = ob + (int64_t)q * ors;
      if constexpr (ND == 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int w = 0; w < ND; ++w) orow[16 * G + 4 * r + w] = o[w][u][r] * inv;
      } else {
#pragma unroll
        for (int w = 0; w < ND; ++w)
#pragma unroll
          for (int r = 0; r < 4; ++r) orow[16 * w + 4 * G + r] = o[w][u][r] * inv;
      }
    }
  }
}

// Merges the key ranges of a key-split attention: with M_s, L_s and O_s the reference maximum
// (log2 units), sum and unnormalised output of range s, m = max_s M_s and w_s = 2^(M_s - m),
// O = sum_s w_s O_s / (sum_s w_s L_s + 1e-10). One thread per 4 consecutive d of one query.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  const int hd4 = a.hd / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  if (i >= (int64_t)a.Sq * hd4) return;
  const int q = (int)(i / hd4), d = 4 * (int)(i % hd4);
  const int ns = a.nsplit;
  const int64_t rows = (int64_t)a.B * a.H * a.Sq;  // partial rows per range
  const int64_t ml = rows * ns * a.hd, row = ((int64_t)b * a.H + h) * a.Sq + q;
  float m = -INFINITY;
  for (int sp = 0; sp < ns; ++sp) m = fmaxf(m, a.part[ml + sp * rows + row]);
  float l = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp = 0; sp < ns; ++sp) {
    const float w = __builtin_amdgcn_exp2f(a.part[ml + sp * rows + row] - m);
    l += w * a.part[ml + (int64_t)ns * rows + sp * rows + row];
    const float4 o = *reinterpret_cast<const float4*>(a.part + (sp * rows + row) * a.hd + d);
    acc.x += w * o.x;
    acc.y += w * o.y;
    acc.z += w * o.z;
    acc.w += w * o.w;
  }
  const float inv = 1.f / (l + 1e-10f);
  *reinterpret_cast<float4*>(a.o + (int64_t)b * a.o_bs + (int64_t)q * a.o_rs + h * a.hd + d) =
      make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

// Generic path for any head dimension: one wave per (b, h, query), scores staged in LDS,
// three passes (max, sum of exp, weighted sum of V), the reference's exact formula.
constexpr int kMaxGenericSk = 12288;
__global__ __launch_bounds__(64) void attn_generic_kernel(AttnArgs a) {
  __shared__ float sc[kMaxGenericSk];
  const int lane = threadIdx.x;
  const int q = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const float* qr = a.q + (int64_t)b * a.q_bs + (int64_t)q * a.q_rs + h * a.hd;
  const float* kb = a.k + (int64_t)b * a.kv_bs + h * a.hd;
  const float* vb = a.v + (int64_t)b * a.kv_bs + h * a.hd;
  float mx = -INFINITY;
  for (int kv = lane; kv < a.Sk; kv += 64) {
    const float* kr = kb + (int64_t)kv * a.kv_rs;
    float dot = 0.f;
    for (int d = 0; d < a.hd; ++d) dot = fmaf(qr[d], kr[d], dot);
    const float s = dot * a.scale;
    sc[kv] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int kv = lane; kv < a.Sk; kv += 64) {
    const float e = expf(sc[kv] - mx);
    sc[kv] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  __syncthreads();
  const float inv = 1.f / (sum + 1e-10f);
  float* orow = a.o + (int64_t)b * a.o_bs + (int64_t)q * a.o_rs + h * a.hd;
  for (int d = lane; d < a.hd; d += 64) {
    float acc = 0.f;
    for (int kv = 0; kv < a.Sk; ++kv) acc = fmaf(sc[kv], vb[(int64_t)kv * a.kv_rs + d], acc);
    orow[d] = acc * inv;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

bool fast_form(const AttnArgs& a) {
  return aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.o) &&
         a.q_rs % 4 == 0 && a.kv_rs % 4 == 0 && a.o_rs % 4 == 0 && a.q_bs % 4 == 0 &&
         a.kv_bs % 4 == 0 && a.o_bs % 4 == 0 && (a.hd == 48 || a.hd == 64);
}

template <int HD>
void launch_hd(const LaunchCtx& c, const AttnArgs& a) {
  if (a.nsplit > 1) {  // 16 queries per wave, key ranges along grid z, then the merge
    dim3 grid(cdiv(a.Sq, 64), a.H, a.B * a.nsplit);
    launch(c, HD == 64 ? "attn_fwd_f32_hd64_q16" : "attn_fwd_f32_hd48_q16",
           attn_fwd_f32_kernel<HD, 16>, grid, dim3(256), 0, a);
    launch(c, "attn_combine_f32", attn_combine_kernel,
           dim3((unsigned)cdiv((int64_t)a.Sq * (HD / 4), 256), a.H, a.B), dim3(256), 0, a);
    return;
  }
  // queries per wave: 32 or 16, whichever needs fewer workgroup rounds x queries per workgroup
  // over the chip's workgroup slots (fewer, longer rounds win ties: K fragments are reused twice).
  // At three workgroups per CU (head dim 48) the 32-query form does not fit the register budget.
  const int64_t slots = (int64_t)c.dev->props.multiProcessorCount * AttnCfg<HD>::OCC;
  const int64_t wg32 = (int64_t)cdiv(a.Sq, 128) * a.H * a.B;
  const int64_t wg16 = (int64_t)cdiv(a.Sq, 64) * a.H * a.B;
  const int64_t cost32 = (int64_t)cdiv(wg32, slots) * 2, cost16 = cdiv(wg16, slots);
  if constexpr (AttnCfg<HD>::OCC < 3) {
    if (cost32 <= cost16) {
      dim3 grid(cdiv(a.Sq, 128), a.H, a.B);
      return launch(c, "attn_fwd_f32_hd64_q32", attn_fwd_f32_kernel<HD, 32>, grid, dim3(256), 0,
                    a);
    }
  }
  dim3 grid(cdiv(a.Sq, 64), a.H, a.B);
  launch(c, HD == 64 ? "attn_fwd_f32_hd64_q16" : "attn_fwd_f32_hd48_q16",
         attn_fwd_f32_kernel<HD, 16>, grid, dim3(256), 0, a);
}

}  // namespace

bool attention_supported(int hd) { return hd > 0; }

// Key split where the query workgroups leave at least half of the device's workgroup slots idle:
// n ranges (the largest n <= 4 with n W <= S for W workgroups of 64 queries on S slots, at least 4
// key blocks per range) fill them. Grids of more than half the slots are not split: filling a
// last round's idle slots this way (e.g. 1344 workgroups on 768 slots as 4 ranges) lowered the
// attention's kernel time but made the two-stream transformer step ~1 % slower (the partial
// outputs' traffic and the merge launches). Config 3's 256 workgroups on 512 slots: 86 -> 78 us
// + 4 us merge. Tuning override: MNN_ATTN_SPLITS (1 disables).
int attention_key_splits(const LaunchCtx& c, const AttnArgs& a) {
  if (a.Sq <= 0 || a.B <= 0 || a.H <= 0 || a.Sk <= 0 || !fast_form(a)) return 1;
  const int nblk = (a.Sk + BKV - 1) / BKV;
  static const int forced = [] {
    const char* e = std::getenv("MNN_ATTN_SPLITS");
    return e ? std::atoi(e) : 0;
  }();
  if (forced > 0) return std::max(1, std::min({forced, 8, nblk}));
  const int occ = a.hd == 64 ? AttnCfg<64>::OCC : AttnCfg<48>::OCC;
  const int64_t slots = (int64_t)c.dev->props.multiProcessorCount * occ;
  const int64_t wg = (int64_t)cdiv(a.Sq, 64) * a.H * a.B;
  int best = 1;
  for (int ns = 2; ns <= 4 && nblk >= 4 * ns && wg * ns <= slots; ++ns) best = ns;
  return best;
}

int64_t attention_part_floats(const AttnArgs& a, int nsplit) {
  return nsplit <= 1 ? 0 : (int64_t)nsplit * a.B * a.H * a.Sq * (a.hd + 2);
}

void attention(const LaunchCtx& c, const AttnArgs& a) {
  if (a.Sq <= 0 || a.B <= 0 || a.H <= 0) return;
  MNN_REQUIRE(a.Sk > 0, MNN_ERR_INVALID_ARGUMENT, "attention: empty key sequence");
  const bool vec = fast_form(a);
  MNN_REQUIRE(a.nsplit >= 1 && (a.nsplit == 1 || (vec && a.part && a.nsplit <= 8 &&
                                                  a.nsplit <= (a.Sk + BKV - 1) / BKV &&
                                                  (int64_t)a.B * a.nsplit <= 65535)),
              MNN_ERR_INVALID_ARGUMENT, "attention: unsupported key split");
  if (vec && a.hd == 64) return launch_hd<64>(c, a);
  if (vec && a.hd == 48) return launch_hd<48>(c, a);
  MNN_REQUIRE(a.Sk <= kMaxGenericSk, MNN_ERR_INVALID_CONFIGURATION,
              "attention: head dim " << a.hd << " with " << a.Sk
                                     << " keys exceeds the generic kernel's limit");
  launch(c, "attn_generic_f32", attn_generic_kernel, dim3(a.Sq, a.H, a.B), dim3(64), 0, a);
}

}  // namespace k
}  // namespace mnn
