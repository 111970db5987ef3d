// Device-side helpers shared by the kernels: activations, wave64 reductions, bf16 rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mnn {
namespace dev {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short shortx8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// sigmoid with the +-88 clamp of the reference's stable_sigmoid (Shaders/NN.metal:32-47);
// 1/(1+e^-x) and e^x/(1+e^x) are the same number, so one branchless form suffices. The reciprocal
// is the hardware's (v_rcp_f32, about 1 ulp): an IEEE division is ten instructions, which the
// GLU epilogues of the matrix-core kernels pay in full beside their MFMAs.
__device__ __forceinline__ float stable_sigmoid(float x) {
  x = fminf(fmaxf(x, -88.f), 88.f);
  return __builtin_amdgcn_rcpf(1.f + __expf(-x));
}

// tanh-approximation GELU: 0.5 x (1 + tanh(u)), u = sqrt(2/pi)(x + 0.044715 x^3).
// Evaluated as x * sigmoid(2u), the same function (1 + tanh(u) = 2 sigmoid(2u)), which needs one
// exp and no cancellation near u = 0; the hardware reciprocal as in stable_sigmoid. For |x| large
// the exp saturates to 0 / inf and the result is x / -0, as the clamped reference form
// (Activations.swift:124-137) gives.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  const float u = k0 * fmaf(k1 * x, x * x, x);
  return x * __builtin_amdgcn_rcpf(1.f + __expf(-2.f * u));
}

// Reference GELU layer semantics: x > 10 -> x, x < -10 -> 0, else the tanh formula.
__device__ __forceinline__ float gelu_clamped(float x) {
  return x > 10.f ? x : (x < -10.f ? 0.f : gelu_tanh(x));
}

// Fused activation codes of mnn_activation; `alpha` is leaky ReLU's negative slope
// (FusedConv1D / FusedLinear leakyReluAlpha, default 0.01: Conv1D.swift:786, Linear.swift:495).
__device__ __forceinline__ float apply_act(float x, int act, float alpha = 0.01f) {
  switch (act) {
    case 1: return fmaxf(x, 0.f);
    case 2: return x >= 0.f ? x : alpha * x;
    case 3: return gelu_tanh(x);
    case 4: return x * stable_sigmoid(x);
    case 5: return stable_sigmoid(x);
    case 6: return tanhf(x);
    default: return x;
  }
}

// Every lane of the calling wave receives the merge of np >= 1 (count, mean, M2) partials, in
// fp64: n = sum n_j, mean = sum n_j mean_j / n, M2 = sum (M2_j + n_j (mean_j - mean)^2). Lane l
// takes partials l, l + 64, ...; the wave sums are xor butterflies, so every lane (and every wave
// and workgroup that merges the same partials) gets the identical value. Plain sums instead of
// Chan's pairwise merges leave no division inside the reduction, and the first 512 partials are
// loaded together (PartsBatch below).
__device__ __forceinline__ double wave_sum_xor_d(double v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int CTRL>
__device__ __forceinline__ double dpp_mov_d(double v) {
  const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, 0xF, 0xF, false);
  return __hiloint2double(hi, lo);
}

__device__ __forceinline__ double readlane_d(double v, int lane) {
  return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                          __builtin_amdgcn_readlane(__double2loint(v), lane));
}

// Sum over the whole wave of a double by DPP row sums (each step moves both halves) and the four
// rows' sums read from lanes 0, 16, 32 and 48, added in that fixed order: every lane returns the
// same bits. All 64 lanes must be active.
__device__ __forceinline__ double wave_sum_dpp_d(double v) {
  v += dpp_mov_d<0xB1>(v);
  v += dpp_mov_d<0x4E>(v);
  v += dpp_mov_d<0x141>(v);
  v += dpp_mov_d<0x140>(v);
  return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

// The first 64 * KB partials of a wave_merge_parts call, loaded by straight-line code (clamped
// addresses, no branch or loop) so that a kernel can put them in flight together with its other
// loads; merge() finishes from registers, re-reading only partials beyond the first batch.
// merge() (and BlockParts::reduce_waves below) sum over the wave with DPP: every lane of the
// wave must be active at the call.
template <int KB>
struct PartsBatch {
  float pn[KB], pm[KB], pq[KB];
  __device__ __forceinline__ void load(const float* __restrict__ p, int np) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const int jc = max(min(lane + 64 * k, np - 1), 0);
      pn[k] = p[3 * jc];
      pm[k] = p[3 * jc + 1];
      pq[k] = p[3 * jc + 2];
    }
  }
  __device__ __forceinline__ void merge(const float* __restrict__ p, int np, double& n,
                                        double& mean, double& m2) {
    const int lane = threadIdx.x & 63;
    // sum n_j, sum n_j mean_j, sum n_j mean_j^2, sum M2_j: four independent wave sums
    double sn = 0.0, sm = 0.0, sm2 = 0.0, sq = 0.0;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      if (lane + 64 * k < np) {
        const double c = pn[k], m = pm[k];
        sn += c;
        sm += c * m;
        sm2 += c * m * m;
        sq += (double)pq[k];
      }
    }
    for (int j = lane + 64 * KB; j < np; j += 64) {  // beyond the first batch
      const double c = p[3 * j], m = p[3 * j + 1];
      sn += c;
      sm += c * m;
      sm2 += c * m * m;
      sq += (double)p[3 * j + 2];
    }
    n = wave_sum_dpp_d(sn);
    sm = wave_sum_dpp_d(sm);
    sm2 = wave_sum_dpp_d(sm2);
    sq = wave_sum_dpp_d(sq);
    mean = n > 0.0 ? sm / n : 0.0;
    // M2 = sum M2_j + sum n_j (mean_j - mean)^2 = sum M2_j + sum n_j mean_j^2 - n mean^2; in fp64
    // the cancellation costs about mean^2 / var * 1e-16 relative, negligible below |mean| / std ~ 1e5
    m2 = n > 0.0 ? fmax(sq + (sm2 - sm * mean), 0.0) : 0.0;
  }
};

// Workgroup-wide merge of np partials (the formula of PartsBatch::merge): thread i of the
// workgroup loads partials i, i + blockDim, ... (PER of them, straight-line), so each partial is
// read once per workgroup; the four sums are reduced per wave, written to `sh` (4 doubles per wave)
// and, after the caller's next __syncthreads, finish() combines the waves in order, giving every
// thread the identical result.
template <int PER>
struct BlockParts {
  float pn[PER], pm[PER], pq[PER];
  __device__ __forceinline__ void load(const float* __restrict__ p, int np) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int jc = max(min((int)threadIdx.x + (int)blockDim.x * k, np - 1), 0);
      pn[k] = p[3 * jc];
      pm[k] = p[3 * jc + 1];
      pq[k] = p[3 * jc + 2];
    }
  }
  // per-wave sums into sh[wave * 4 + 0..3]; partials beyond PER * blockDim are read here
  __device__ __forceinline__ void reduce_waves(const float* __restrict__ p, int np, double* sh) {
    double sn = 0.0, sm = 0.0, sm2 = 0.0, sq = 0.0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      if ((int)threadIdx.x + (int)blockDim.x * k < np) {
        const double c = pn[k], m = pm[k];
        sn += c;
        sm += c * m;
        sm2 += c * m * m;
        sq += (double)pq[k];
      }
    }
    for (int j = threadIdx.x + blockDim.x * PER; j < np; j += blockDim.x) {
      const double c = p[3 * j], m = p[3 * j + 1];
      sn += c;
      sm += c * m;
      sm2 += c * m * m;
      sq += (double)p[3 * j + 2];
    }
    sn = wave_sum_dpp_d(sn);
    sm = wave_sum_dpp_d(sm);
    sm2 = wave_sum_dpp_d(sm2);
    sq = wave_sum_dpp_d(sq);
    if ((threadIdx.x & 63) == 0) {
      double* o = sh + 4 * (threadIdx.x >> 6);
      o[0] = sn;
      o[1] = sm;
      o[2] = sm2;
      o[3] = sq;
    }
  }
  static __device__ __forceinline__ void finish(const double* sh, double& n, double& mean,
                                                double& m2) {
    double sn = 0.0, sm = 0.0, sm2 = 0.0, sq = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
      sn += sh[4 * w];
      sm += sh[4 * w + 1];
      sm2 += sh[4 * w + 2];
      sq += sh[4 * w + 3];
    }
    n = sn;
    mean = n > 0.0 ? sm / n : 0.0;
    m2 = n > 0.0 ? fmax(sq + (sm2 - sm * mean), 0.0) : 0.0;
  }
};

__device__ __forceinline__ void wave_merge_parts(const float* __restrict__ p, int np, double& n,
                                                 double& mean, double& m2) {
  PartsBatch<8> pb;
  pb.load(p, np);
  pb.merge(p, np, n, mean, m2);
}

// Sum over each aligned group of 16 lanes (a DPP "row"), the total in every lane of the group, by
// DPP moves instead of LDS permutes: swap neighbours (quad_perm [1,0,3,2]), swap pairs
// ([2,3,0,1]), mirror within 8 lanes, mirror within 16. Each step adds a value to its partner's,
// and both partners compute the same sum (a + b = b + a), so every lane ends with the identical
// total.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return v;
}

// Workgroup barrier that orders LDS accesses only: global loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over the whole wave by DPP row sums and the four rows' sums read from lanes 0, 16, 32 and
// 48, added in that fixed order: every lane returns the same bits. All 64 lanes must be active.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = row16_sum(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Chan's merge of statistics (n2, mean2, m22) into (n, mean, m2).
__device__ __forceinline__ void welford_combine(float& n, float& mean, float& m2, float n2,
                                                float mean2, float m22) {
  const float nt = n + n2;
  if (nt > 0.f) {
    const float d = mean2 - mean;
    const float w = n2 / nt;
    mean = mean + d * w;
    m2 = m2 + m22 + d * d * n * w;
  }
  n = nt;
}

// Workgroup-wide (count, mean, M2) of per-thread values: the workgroup mean from DPP sums of the
// counts and of count * mean, then M2 = sum of (M2 + count * (mean - workgroup mean)^2), Chan's
// merge written about the final mean, so no term cancels. Two DPP wave sums and two LDS exchanges
// in a fixed order: a merge over the lanes (a division and an LDS permute chain per step) left
// every wave ~1 us at its end in short kernels.
// Each thread passes its own (n, mean, m2); thread 0 receives the workgroup result. Every lane of
// every wave must be active. `red` must hold 3 * (blockDim.x / 64) floats of LDS.
__device__ __forceinline__ void block_welford(float& n, float& mean, float& m2, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const float c = wave_sum_dpp(n), s = wave_sum_dpp(n * mean);
  if (lane == 0) {
    red[wid * 3 + 0] = c;
    red[wid * 3 + 1] = s;
  }
  __syncthreads();
  float C = 0.f, S = 0.f;
  for (int w = 0; w < nw; ++w) {
    C += red[w * 3 + 0];
    S += red[w * 3 + 1];
  }
  const float M = C > 0.f ? S / C : 0.f;
  const float d = mean - M;
  const float q = wave_sum_dpp(n > 0.f ? fmaf(n * d, d, m2) : 0.f);
  if (lane == 0) red[wid * 3 + 2] = q;
  __syncthreads();
  if (threadIdx.x == 0) {
    float Q = 0.f;
    for (int w = 0; w < nw; ++w) Q += red[w * 3 + 2];
    n = C;
    mean = M;
    m2 = Q;
  }
}

// Running (count, mean, M2) of a thread's values without a division per value: sums of
// (v - shift) and (v - shift)^2 around the thread's first value, converted once at the end.
struct ShiftedStats {
  float n = 0.f, shift = 0.f, s1 = 0.f, s2 = 0.f;
  __device__ __forceinline__ void add(float v) {
    if (n == 0.f) shift = v;
    const float d = v - shift;
    n += 1.f;
    s1 += d;
    s2 = fmaf(d, d, s2);
  }
  __device__ __forceinline__ void finish(float& cnt, float& mean, float& m2) const {
    cnt = n;
    if (n > 0.f) {
      const float md = s1 / n;
      mean = shift + md;
      m2 = fmaxf(s2 - s1 * md, 0.f);
    } else {
      mean = 0.f;
      m2 = 0.f;
    }
  }
};

// Block-wide fixed-order sum of one double per thread (wave shuffles, then the waves in order).
// `sh` needs blockDim.x / 64 doubles; every thread receives the total.
__device__ __forceinline__ double block_sum_d(double v, double* sh) {
  v = wave_sum_d(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) sh[wid] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < nw; ++w) t += sh[w];
  __syncthreads();
  return t;
}

// Merge of GroupNorm(1) partials (count, mean, M2) written by a previous kernel, by every thread
// of a workgroup: N = sum n_j, mean = sum n_j mean_j / N, M2 = sum (M2_j + n_j (mean_j - mean)^2),
// accumulated in fp64 in a fixed order, so every workgroup obtains the same (mean, rstd).
// `sh` needs blockDim.x / 64 doubles of LDS.
__device__ __forceinline__ float2 gn1_merge(const float* __restrict__ partials, int nparts,
                                           float eps, double* sh) {
  double n = 0.0, s1 = 0.0;
  for (int j = threadIdx.x; j < nparts; j += blockDim.x) {
    const float* p = partials + (int64_t)j * 3;
    n += p[0];
    s1 += (double)p[0] * (double)p[1];
  }
  const double ntot = block_sum_d(n, sh);
  const double mean = ntot > 0.0 ? block_sum_d(s1, sh) / ntot : 0.0;
  double m2 = 0.0;
  for (int j = threadIdx.x; j < nparts; j += blockDim.x) {
    const float* p = partials + (int64_t)j * 3;
    const double d = (double)p[1] - mean;
    m2 += (double)p[2] + (double)p[0] * d * d;
  }
  m2 = block_sum_d(m2, sh);
  const double var = ntot > 0.0 ? m2 / ntot : 0.0;  // biased (population) variance
  float rstd = (float)(1.0 / sqrt(var + (double)eps));
  if (!isfinite(rstd)) rstd = 0.f;  // reference CPU path guard (Normalization.swift:695-699)
  return make_float2((float)mean, rstd);
}

// One-round variant for consumers that merge at every workgroup: each thread sums, in fp64 and in
// a fixed order, N = sum n_j, S1 = sum n_j mean_j and S2 = sum (M2_j + n_j mean_j^2); one
// workgroup reduction of the three sums then gives mean = S1 / N and M2 = S2 - N mean^2 (the
// cancellation costs ~1e-16 * mean^2 / var relative to var in fp64). Uses only LDS barriers
// (no memory fence), so LDS-DMA loads issued earlier stay in flight. `sh` needs
// 3 * blockDim.x / 64 doubles of LDS. Returns (mean, rstd) to every thread.
__device__ __forceinline__ float2 gn1_merge_one_round(const float* __restrict__ partials,
                                                     int nparts, float eps, double* sh) {
  // each round loads kBatch partials per thread with every load in flight (clamped addresses;
  // out-of-range values are loaded but not used), instead of one dependent load per partial
  constexpr int kBatch = 8;
  double n = 0.0, s1 = 0.0, s2 = 0.0;
  for (int j0 = 0; j0 < nparts; j0 += kBatch * (int)blockDim.x) {
    float pn[kBatch], pm[kBatch], pq[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const float* p = partials + 3 * (int64_t)min(j0 + k * (int)blockDim.x + (int)threadIdx.x,
                                                   nparts - 1);
      pn[k] = p[0];
      pm[k] = p[1];
      pq[k] = p[2];
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (j0 + k * (int)blockDim.x + (int)threadIdx.x < nparts) {
        const double c = pn[k], m = pm[k];
        n += c;
        s1 += c * m;
        s2 += (double)pq[k] + c * m * m;
      }
    }
  }
  n = wave_sum_d(n);
  s1 = wave_sum_d(s1);
  s2 = wave_sum_d(s2);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) {
    sh[3 * wid] = n;
    sh[3 * wid + 1] = s1;
    sh[3 * wid + 2] = s2;
  }
  __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4));  // this wave's LDS writes done
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  double N = 0.0, S1 = 0.0, S2 = 0.0;
  for (int w = 0; w < nw; ++w) {
    N += sh[3 * w];
    S1 += sh[3 * w + 1];
    S2 += sh[3 * w + 2];
  }
  const double mean = N > 0.0 ? S1 / N : 0.0;
  const double var = N > 0.0 ? fmax(S2 - N * mean * mean, 0.0) / N : 0.0;  // biased variance
  float rstd = (float)(1.0 / sqrt(var + (double)eps));
  if (!isfinite(rstd)) rstd = 0.f;  // reference CPU path guard (Normalization.swift:695-699)
  return make_float2((float)mean, rstd);
}

// ---------------------------------------------------------------- grid-wide statistics exchange
// One-launch GroupNorm: every workgroup of a grid that the device holds at once publishes the
// (mean, M2) of its tile, and the batch's statistics are merged from all of them (xch_merge)
// before any workgroup normalises. No cache maintenance is used (an agent-scope acquire fence
// per wave and a release fence per workgroup cost more than the rest of such kernels): a
// partial is two 64-bit words (tag << 32 | mean bits), (tag << 32 | M2 bits), each stored and
// loaded as one relaxed device-scope atomic, so a reader sees either a whole word of this launch
// or one with another tag. The count of a partial follows from the geometry and is not exchanged.
//
// Two ways to collect, by grid size. With up to a few hundred workgroups every workgroup polls
// every partial and merges them itself (fewest round trips). With more, that polling makes
// traffic at the coherence point that grows with the square of the grid (each 8-byte
// device-scope load is a transaction of its own), so workgroup 0 of each batch is the merger:
// it polls the partials, merges them and publishes one result pair (mean, rstd), which is all
// the others poll. Neither keeps a count by read-modify-writes on one word: those are
// serialised where the word lives (tens of ns each), microseconds at these grids.

// Merge of the collected (mean, M2) partials in a fixed order, in every wave of the caller (no
// barrier): fp64 sums over the partials by lane, then over the wave; count(v) is partial v's
// element count and ntot their sum. Every lane of every wave returns the same bits.
template <class CountFn>
__device__ __forceinline__ float2 xch_merge(const float2* sp, int nparts, CountFn count,
                                            double ntot, float eps) {
  double sm = 0.0, sm2 = 0.0, sq = 0.0;
  for (int v = threadIdx.x & 63; v < nparts; v += 64) {
    const double c = count(v);
    const double m = sp[v].x;
    sm += c * m;
    sm2 += c * m * m;
    sq += (double)sp[v].y;
  }
  sm = wave_sum_dpp_d(sm);
  sm2 = wave_sum_dpp_d(sm2);
  sq = wave_sum_dpp_d(sq);
  const double mean = sm / ntot;
  const double var = fmax(sq + (sm2 - sm * mean), 0.0) / ntot;
  float rstd = (float)(1.0 / sqrt(var + (double)eps));
  if (!isfinite(rstd)) rstd = 0.f;
  return make_float2((float)mean, rstd);
}

// Epoch tags: words carry a per-batch epoch tag instead of being cleared. Every workgroup reads
// the batch's epoch E at its start and tags its words (E mod 2^31) + 1. Once workgroup 0 of the
// batch has seen every partial, every workgroup has read E, so it advances the epoch then (the
// merger; in the poll-everything form, workgroup 0 as well). Stale words of earlier launches
// (graph replays included) never carry the current tag, so nothing is cleared and no workgroup
// counts out.
//
// Termination: every workgroup publishes before it waits, and the waits of all but workgroup 0
// are bounded (a workgroup whose wait runs out computes every partial itself, by the same code
// as their owners, so the same bits). So workgroup 0's wait, which is not bounded (it must see
// every partial before it may advance the epoch), ends once every workgroup has run: if the grid
// is not resident at once, the bounded waiters finish and free their slots for the rest.
//
// Buffer layout (64-bit words): batch b's epoch at word 4 b (low half), its result at 4 b + 2
// (tag | mean bits) and 4 b + 3 (tag | rstd bits); partial slots from word 4 * kXmMaxBatch, two
// per partial, batch b's partial v at slot b * nparts + v. The buffer is zero before the first
// launch. Launches that share a buffer must not overlap.
constexpr int kXmMaxBatch = 64;

__device__ __forceinline__ unsigned long long* xm_batch(unsigned long long* xch, int b) {
  return xch + 4 * b;
}
__device__ __forceinline__ unsigned long long* xm_slots(unsigned long long* xch, int b,
                                                        int nparts) {
  return xch + 4 * kXmMaxBatch + 2 * (int64_t)b * nparts;
}

// The tag of this launch's words for batch b.
__device__ __forceinline__ unsigned xm_tag(unsigned long long* xch, int b) {
  const unsigned e = (unsigned)__hip_atomic_load(xm_batch(xch, b), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
  return (e & 0x7fffffffu) + 1u;
}

__device__ __forceinline__ void put_tag(unsigned long long* s, unsigned tag, float lo) {
  __hip_atomic_store(s, ((unsigned long long)tag << 32) | __float_as_uint(lo), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Publishes partial v of batch b (thread 0).
__device__ __forceinline__ void xm_put(unsigned long long* xch, int b, int nparts, int v,
                                       unsigned tag, float mean, float m2) {
  unsigned long long* sl = xm_slots(xch, b, nparts) + 2 * v;
  put_tag(sl, tag, mean);
  put_tag(sl + 1, tag, m2);
}

// Polls the nparts partials of batch b into sp[] (NT threads, PER per thread, loaded together)
// until every one carries this launch's tag; spin_limit < 0: without bound (the merger, which
// must see every partial before it may advance the epoch). Returns false when spin_limit polls
// passed without that (the caller then computes the partials itself); every thread returns the
// same value.
template <int NT, int PER>
__device__ __forceinline__ bool xm_collect(unsigned long long* xch, int b, int nparts,
                                           unsigned tag, float2* sp, int spin_limit = -1) {
  const unsigned long long* slots = xm_slots(xch, b, nparts);
  for (int polls = 0;; ++polls) {
    bool ok = true;
    for (int v0 = 0; v0 < nparts; v0 += NT * PER) {
      unsigned long long a[PER], c[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int v = min(v0 + (int)threadIdx.x + i * NT, nparts - 1);
        a[i] = __hip_atomic_load(slots + 2 * v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        c[i] = __hip_atomic_load(slots + 2 * v + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int v = v0 + (int)threadIdx.x + i * NT;
        if (v < nparts) {
          ok = ok && (unsigned)(a[i] >> 32) == tag && (unsigned)(c[i] >> 32) == tag;
          sp[v] = make_float2(__uint_as_float((unsigned)a[i]), __uint_as_float((unsigned)c[i]));
        }
      }
    }
    if (!__syncthreads_or(!ok)) return true;
    if (spin_limit >= 0 && polls >= spin_limit) return false;
    __builtin_amdgcn_s_sleep(1);
  }
}

// Advances batch b's epoch (thread 0 of a workgroup that has seen every partial of the launch).
__device__ __forceinline__ void xm_advance(unsigned long long* xch, int b, unsigned tag) {
  __hip_atomic_store(reinterpret_cast<unsigned*>(xm_batch(xch, b)), tag & 0x7fffffffu,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The merger, with the merged result: publishes it and advances the batch's epoch (thread 0).
__device__ __forceinline__ void xm_publish(unsigned long long* xch, int b, unsigned tag,
                                           float2 mr) {
  unsigned long long* w = xm_batch(xch, b);
  put_tag(w + 2, tag, mr.x);
  put_tag(w + 3, tag, mr.y);
  xm_advance(xch, b, tag);
}

// Every other workgroup: polls batch b's result pair (one thread, broadcast through `s_res`)
// until it carries this launch's tag; false when spin_limit polls passed without it.
__device__ __forceinline__ bool xm_wait(unsigned long long* xch, int b, unsigned tag,
                                        int spin_limit, float2* s_res) {
  const unsigned long long* w = xm_batch(xch, b);
  if (threadIdx.x == 0) {
    float2 r = make_float2(0.f, -1.f);  // rstd < 0: not seen
    for (int polls = 0;; ++polls) {
      const unsigned long long m = __hip_atomic_load(w + 2, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
      const unsigned long long q = __hip_atomic_load(w + 3, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
      if ((unsigned)(m >> 32) == tag && (unsigned)(q >> 32) == tag) {
        r = make_float2(__uint_as_float((unsigned)m), __uint_as_float((unsigned)q));
        break;
      }
      if (polls >= spin_limit) break;
      __builtin_amdgcn_s_sleep(1);
    }
    *s_res = r;
  }
  lds_barrier();
  return s_res->y >= 0.f;
}

}  // namespace dev
}  // namespace mnn
