// Short-time Fourier transform of the frequency branch (STFT.swift:40-80 and :384-533 over the
// FFT of FFT.swift): analysis frames of N samples every `hop` samples (no centring padding), the
// window applied, a full N-point DFT without scaling; the inverse takes the real part of each
// frame's inverse DFT scaled by 1/N, applies the window again, overlap-adds the frames and
// divides by the overlap-added squared window floored at `floor` (values below FLT_MIN counted as
// zero first).
//
// A real N-point DFT is computed as a complex M = N/2-point FFT of z[m] = x[2m] + i x[2m+1] and
// the split step
//   X[k] = (Z[k] + conj Z[M-k]) / 2 - i e^{-2 pi i k / N} (Z[k] - conj Z[M-k]) / 2,  0 <= k <= M
// (X[N-k] = conj X[k] for the full spectrum). For 128 <= N <= 8192 the M-point FFT is
// register-resident (Stockham passes of radix 16, each thread holding 16 values, the LDS only
// between passes; several frames per workgroup); other sizes run one workgroup per frame with
// radix-2 decimation in time in LDS (input stored bit-reversed, two stages per barrier). Twiddles
// come from tables computed on the host in double precision. The inverse runs the same steps
// backwards (Hermitian fold of the input, merge into Z, inverse FFT with conjugate twiddles,
// 1/M); the overlap-add is a gather over the frames that cover each output sample, in increasing
// frame order, so it needs no atomics.
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int kThreads = 256;
constexpr int kStftLdsTwMaxN = 8192;  // LDS twiddles up to 68 KiB of LDS per workgroup (padded)
constexpr int kStftStageMaxN = 4096;  // inverse with the spectrum staged in LDS: 51 KiB

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// LDS slot of complex element i of an LDS array (z, the twiddles in LDS): one padding slot per
// 16 elements. The butterfly passes and the bit-reversed stores access 8-byte elements at
// power-of-two strides, which without padding fall on a few of the LDS banks (counters showed
// twice as many bank-conflict cycles as LDS instruction cycles).
__device__ __forceinline__ int zp(int i) { return i + (i >> 4); }
constexpr int zslots(int m) { return m + m / 16; }

// In-place radix-2 DIT FFT of z[0..M) (bit-reversed input order) in LDS; inverse uses conjugate
// twiddles (no scaling). tw[k] = e^{-2 pi i k / N}, N = 2M. Two consecutive stages h and 2h run
// per barrier: a thread takes the group i0 + {0, h, 2h, 3h} (i0 = 4h q + p, p < h) through stage
// h (pairs (i0, i0+h), (i0+2h, i0+3h), twiddle W_2h^p) and stage 2h (pairs (i0, i0+2h) with
// W_4h^p, (i0+h, i0+3h) with W_4h^(p+h)), the same operations in the same order as two radix-2
// passes; an odd stage count ends with one radix-2 pass. z is addressed through zp(); TWP: tw is
// the padded LDS copy (zp()), else the plain global table.
template <bool TWP>
__device__ void fft_lds(float2* z, int M, const float2* __restrict__ tw, bool inverse) {
  const int lt = threadIdx.x;
  auto twd = [&](int i) { return tw[TWP ? zp(i) : i]; };
  int h = 1;
  for (; 2 * h < M; h <<= 2) {
    const int s1 = M / h, s2 = M / (2 * h);  // W_2h^p = tw[p * s1], W_4h^p = tw[p * s2]
    for (int t = lt; t < M / 4; t += kThreads) {
      const int p = t & (h - 1);
      const int i0 = ((t - p) << 2) + p;
      float2 w1 = twd(p * s1), w2 = twd(p * s2), w3 = twd(p * s2 + M / 2);
      if (inverse) {
        w1.y = -w1.y;
        w2.y = -w2.y;
        w3.y = -w3.y;
      }
      float2 a0 = z[zp(i0)], a1 = z[zp(i0 + h)], a2 = z[zp(i0 + 2 * h)], a3 = z[zp(i0 + 3 * h)];
      float2 bb = cmul(a1, w1);
      a1 = make_float2(a0.x - bb.x, a0.y - bb.y);
      a0 = make_float2(a0.x + bb.x, a0.y + bb.y);
      bb = cmul(a3, w1);
      a3 = make_float2(a2.x - bb.x, a2.y - bb.y);
      a2 = make_float2(a2.x + bb.x, a2.y + bb.y);
      bb = cmul(a2, w2);
      z[zp(i0 + 2 * h)] = make_float2(a0.x - bb.x, a0.y - bb.y);
      z[zp(i0)] = make_float2(a0.x + bb.x, a0.y + bb.y);
      bb = cmul(a3, w3);
      z[zp(i0 + 3 * h)] = make_float2(a1.x - bb.x, a1.y - bb.y);
      z[zp(i0 + h)] = make_float2(a1.x + bb.x, a1.y + bb.y);
    }
    __syncthreads();
  }
  if (h < M) {
    const int stride = M / h;  // W_{2h}^p = tw[p * M / h]
    for (int t = lt; t < M / 2; t += kThreads) {
      const int p = t & (h - 1);
      const int i0 = ((t - p) << 1) + p, i1 = i0 + h;
      float2 w = twd(p * stride);
      if (inverse) w.y = -w.y;
      const float2 a = z[zp(i0)], b = cmul(z[zp(i1)], w);
      z[zp(i0)] = make_float2(a.x + b.x, a.y + b.y);
      z[zp(i1)] = make_float2(a.x - b.x, a.y - b.y);
    }
    __syncthreads();
  }
}

// Frame of this workgroup. Workgroups are dealt to the 8 XCDs round robin; numbering the frames
// so that consecutive frames run on one XCD lets the bin-major layout's writes (consecutive
// frames of one bin share a cache line) merge in that XCD's L2. The grid is padded to a multiple
// of 8 (frames past the end return before any barrier).
__device__ __forceinline__ int64_t frame_of_block(int64_t frames) {
  const unsigned per = gridDim.x / 8;
  return (int64_t)(blockIdx.x % 8) * per + blockIdx.x / 8;
}

__device__ __forceinline__ int bitrev(int m, int logM) {
  return logM == 0 ? 0 : (int)(__brev((unsigned)m) >> (32 - logM));
}

// With LDS_TW the twiddle table is copied to LDS with the input (one global-latency exposure
// instead of one per butterfly pass); LDS holds z then the table (N/2 float2 each).
template <bool LDS_TW>
__global__ __launch_bounds__(kThreads) void stft_forward_kernel(StftArgs a) {
  extern __shared__ float2 z[];
  const int64_t f = frame_of_block(a.frames);
  const int b = blockIdx.y;
  if (f >= a.frames) return;
  const int M = a.N / 2;
  float2* tws = z + zslots(M);
  const float* xs = a.x + (int64_t)b * a.n + (int64_t)f * a.hop;
  // every load of a batch of 8 samples pairs per thread (clamped indices) before any LDS store
  for (int m0 = threadIdx.x; m0 < M; m0 += 8 * kThreads) {
    float xe[8], xo[8], we[8], wo[8];
    float2 tv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int m = min(m0 + u * kThreads, M - 1);
      xe[u] = xs[2 * m];
      xo[u] = xs[2 * m + 1];
      we[u] = a.win[2 * m];
      wo[u] = a.win[2 * m + 1];
      if (LDS_TW) tv[u] = a.tw[m];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int m = m0 + u * kThreads;
      if (m < M) {
        z[zp(bitrev(m, a.logM))] = make_float2(xe[u] * we[u], xo[u] * wo[u]);
        if (LDS_TW) tws[zp(m)] = tv[u];
      }
    }
  }
  __syncthreads();
  fft_lds<LDS_TW>(z, M, LDS_TW ? tws : a.tw, false);
  const int bins = a.onesided ? M + 1 : a.N;
  const int64_t base = (int64_t)b * a.frames * bins;
  for (int k = threadIdx.x; k <= M; k += kThreads) {
    const float2 zk = z[zp(k == M ? 0 : k)];
    const float2 zc = z[zp(k == 0 ? 0 : M - k)];  // Z[M-k], conjugated below
    const float2 fe = make_float2(0.5f * (zk.x + zc.x), 0.5f * (zk.y - zc.y));
    const float2 d = make_float2(0.5f * (zk.x - zc.x), 0.5f * (zk.y + zc.y));  // (Zk - conj Zc)/2
    const float2 fo = make_float2(d.y, -d.x);                                    // -i * d
    const float2 w = k == M ? make_float2(-1.f, 0.f) : (LDS_TW ? tws[zp(k)] : a.tw[min(k, M - 1)]);
    const float2 t = cmul(w, fo);
    const float re = fe.x + t.x, im = fe.y + t.y;
    auto put = [&](int kk, float r, float i) {
      const int64_t o = a.layout == 0 ? base + (int64_t)f * bins + kk
                                      : base + (int64_t)kk * a.frames + f;
      a.re[o] = r;
      a.im[o] = i;
    };
    put(k, re, im);
    if (!a.onesided && k > 0 && k < M) put(a.N - k, re, -im);
  }
}

// STAGE (one-sided spectra, twiddles in LDS): each bin is loaded from global memory once into
// LDS (the M + 1 float2 after the twiddles) and read back for both members of its Hermitian pair
// (k and M - k), instead of being loaded twice.
template <bool LDS_TW, bool STAGE>
__global__ __launch_bounds__(kThreads) void stft_inverse_kernel(StftArgs a) {
  extern __shared__ float2 z[];
  const int64_t f = frame_of_block(a.frames);
  const int b = blockIdx.y;
  if (f >= a.frames) return;
  const int M = a.N / 2;
  float2* tws = z + zslots(M);
  const int bins = a.onesided ? M + 1 : a.N;
  const int64_t base = (int64_t)b * a.frames * bins;
  auto get = [&](int kk) {
    const int64_t o = a.layout == 0 ? base + (int64_t)f * bins + kk
                                    : base + (int64_t)kk * a.frames + f;
    return make_float2(a.cre[o], a.cim[o]);
  };
  // Hermitian part H[k] of the input spectrum, k in [0, M], from X[k] (g) and X[N-k] (c, full
  // spectra only): the real part of the inverse DFT depends on nothing else.
  auto herm = [&](int kk, float2 g, float2 c) {
    float2 h = g;
    if (!a.onesided && kk > 0 && kk < M) h = make_float2(0.5f * (g.x + c.x), 0.5f * (g.y - c.y));
    if (kk == 0 || kk == M) h.y = 0.f;
    return h;
  };
  if constexpr (STAGE) {
    float2* xs = z + 2 * zslots(M);  // X[0 .. M]
    // every load of a batch of 4 bins per thread (clamped indices) before any LDS store
    for (int k0 = threadIdx.x; k0 <= M; k0 += 4 * kThreads) {
      float2 g[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) g[u] = get(min(k0 + u * kThreads, M));
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k0 + u * kThreads <= M) xs[k0 + u * kThreads] = g[u];
    }
    __syncthreads();
    for (int k = threadIdx.x; k < M; k += kThreads) {
      const float2 zero = make_float2(0.f, 0.f);
      const float2 hk = herm(k, xs[k], zero), hc = herm(M - k, xs[M - k], zero);
      const float2 fe = make_float2(0.5f * (hk.x + hc.x), 0.5f * (hk.y - hc.y));
      const float2 d = make_float2(0.5f * (hk.x - hc.x), 0.5f * (hk.y + hc.y));
      const float2 t = a.tw[k];
      tws[zp(k)] = t;
      const float2 w = make_float2(t.x, -t.y);  // e^{+2 pi i k / N}
      const float2 fo = cmul(d, w);
      z[zp(bitrev(k, a.logM))] = make_float2(fe.x - fo.y, fe.y + fo.x);  // Fe + i Fo
    }
  }
  // every load of a batch of 4 bins per thread (clamped indices) before any LDS store
  for (int k0 = threadIdx.x; !STAGE && k0 < M; k0 += 4 * kThreads) {
    float2 gk[4], gc[4], ck[4], cc[4], tv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = min(k0 + u * kThreads, M - 1), kc = M - k;
      gk[u] = get(k);
      gc[u] = get(kc);
      if (!a.onesided) {
        ck[u] = get(k > 0 ? a.N - k : k);
        cc[u] = get(kc < M ? a.N - kc : kc);
      } else {
        ck[u] = cc[u] = make_float2(0.f, 0.f);  // not read for one-sided spectra
      }
      tv[u] = a.tw[k];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = k0 + u * kThreads;
      if (k >= M) continue;
      const float2 hk = herm(k, gk[u], ck[u]), hc = herm(M - k, gc[u], cc[u]);
      const float2 fe = make_float2(0.5f * (hk.x + hc.x), 0.5f * (hk.y - hc.y));
      const float2 d = make_float2(0.5f * (hk.x - hc.x), 0.5f * (hk.y + hc.y));
      const float2 t = tv[u];
      if (LDS_TW) tws[zp(k)] = t;
      const float2 w = make_float2(t.x, -t.y);  // e^{+2 pi i k / N}
      const float2 fo = cmul(d, w);
      z[zp(bitrev(k, a.logM))] = make_float2(fe.x - fo.y, fe.y + fo.x);  // Fe + i Fo
    }
  }
  __syncthreads();
  fft_lds<LDS_TW>(z, M, LDS_TW ? tws : a.tw, true);
  const float s = 1.f / (float)M;
  float* out = a.frames_buf + ((int64_t)b * a.frames + f) * a.N;
  for (int m = threadIdx.x; m < M; m += kThreads) {
    const float2 v = z[zp(m)];
    out[2 * m] = (v.x * s) * a.win[2 * m];
    out[2 * m + 1] = (v.y * s) * a.win[2 * m + 1];
  }
}

// ------------------------------------------------------------ register-resident Stockham FFT
// A thread holds 16 complex values and runs each pass's radix-R DFTs (R = 16, or the last pass's
// smaller radix, 16 / R of them) in registers; the LDS carries the data between passes only
// (M = 2048: 3 passes, against 11 radix-2 stages in LDS). Pass p with radix R after L points
// are combined (Stockham, natural order in and out):
//   v_r = in[j + r M / R] * W_{L R}^{r k},  k = j mod L,  r < R
//   out[(j - k) R + k + s L] = sum_r v_r W_R^{r s},  s < R
// for the butterflies j < M / R. Pass 0 (L = 1) has no twiddles; the others read them from the
// plan's table staged in LDS (M - 16 entries, [pass][r - 1][k], computed on the host in double).
// The inverse uses conjugate twiddles throughout.

constexpr float kC1 = 0.92387953251128674f;  // cos(pi / 8)
constexpr float kC2 = 0.70710678118654752f;  // cos(pi / 4)
constexpr float kC3 = 0.38268343236508978f;  // cos(3 pi / 8)

// v * W_16^q (forward, e^{-2 pi i q / 16}) or v * conj(W_16^q) (INV), q < 8 (a constant after
// unrolling)
template <bool INV>
__device__ __forceinline__ float2 w16(float2 v, int q) {
  if (q == 0) return v;
  if (q == 4) return INV ? make_float2(-v.y, v.x) : make_float2(v.y, -v.x);
  const float c = q == 1 ? kC1 : q == 2 ? kC2 : q == 3 ? kC3 : q == 5 ? -kC3 : q == 6 ? -kC2 : -kC1;
  const float s = q == 1 ? kC3 : q == 2 ? kC2 : q == 3 ? kC1 : q == 5 ? kC1 : q == 6 ? kC2 : kC3;
  return INV ? make_float2(v.x * c - v.y * s, v.x * s + v.y * c)
             : make_float2(v.x * c + v.y * s, v.y * c - v.x * s);
}

constexpr int brev_c(int s, int bits) {
  int r = 0;
  for (int i = 0; i < bits; ++i) r |= ((s >> i) & 1) << (bits - 1 - i);
  return r;
}

// In-register R-point DFT of v[0..R) (natural order in and out): radix-2 decimation in
// frequency (stage of half-size h: v_p + v_{p+h}, (v_p - v_{p+h}) W_{2h}^p), then the
// bit-reversal permutation, which costs nothing after unrolling.
template <int R, bool INV>
__device__ __forceinline__ void dft_reg(float2* v) {
#pragma unroll
  for (int h = R / 2; h >= 1; h /= 2) {
#pragma unroll
    for (int i0 = 0; i0 < R; i0 += 2 * h) {
#pragma unroll
      for (int p = 0; p < h; ++p) {
        const float2 x = v[i0 + p], y = v[i0 + p + h];
        v[i0 + p] = make_float2(x.x + y.x, x.y + y.y);
        v[i0 + p + h] = w16<INV>(make_float2(x.x - y.x, x.y - y.y), p * 8 / h);
      }
    }
  }
  constexpr int bits = R == 16 ? 4 : R == 8 ? 3 : R == 4 ? 2 : R == 2 ? 1 : 0;
  float2 t[R];
#pragma unroll
  for (int s = 0; s < R; ++s) t[s] = v[brev_c(s, bits)];
#pragma unroll
  for (int s = 0; s < R; ++s) v[s] = t[s];
}

template <int LOGM>
struct SkCfg {
  static constexpr int M = 1 << LOGM, T = M / 16;    // threads per transform
  static constexpr int P = stft_sk_passes(LOGM);
  static constexpr int RL = stft_sk_radix(LOGM, P - 1);  // last pass's radix
  static constexpr int F = 256 / T < 16 ? 256 / T : 16;  // transforms (frames) per workgroup
  static constexpr int NT = F * T;
  static constexpr int ZS = M + M / 16;  // zslots(M)
  static constexpr int NSTW = M - 16;
  static constexpr size_t LDS = sizeof(float2) * ((size_t)F * ZS + NSTW);
  static_assert(LOGM >= kStftSkMinLogM && LOGM <= kStftSkMaxLogM && P >= 2 && P <= 3, "plan");
};

// Pass (R, L >= 16) of one transform in LDS: every read of the pass, the twiddles and the DFTs,
// a barrier, then the writes (in place) and a barrier.
template <int LOGM, int R, int L, bool INV>
__device__ __forceinline__ void sk_pass(float2* zg, const float2* stwl, int lt) {
  constexpr int M = 1 << LOGM, T = M / 16, NB = 16 / R;
  float2 v[16];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) v[b * R + r] = zg[zp(lt + b * T + r * (M / R))];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int k = (lt + b * T) & (L - 1);
#pragma unroll
    for (int r = 1; r < R; ++r) {
      float2 w = stwl[(L - 16) + (r - 1) * L + k];
      if (INV) w.y = -w.y;
      v[b * R + r] = cmul(v[b * R + r], w);
    }
    dft_reg<R, INV>(v + b * R);
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int jj = lt + b * T, k = jj & (L - 1);
#pragma unroll
    for (int s = 0; s < R; ++s) zg[zp((jj - k) * R + k + s * L)] = v[b * R + s];
  }
  __syncthreads();
}

// Forward STFT on the register-resident FFT: F frames per workgroup (one per group of T
// threads). Pass 0 reads the windowed samples from global memory; the last pass leaves Z in LDS
// in natural order for the split step. Output: frame-major rows (consecutive threads along bins)
// or bin-major rows (bin k of the workgroup's frames as one vector of up to 4 floats). Frames
// past the end run on the last frame and store nothing; with a frame count that is not a
// multiple of F the bin-major vectors are written as scalars.
template <int LOGM>
__global__ __launch_bounds__(SkCfg<LOGM>::NT) void stft_forward_sk_kernel(StftArgs a) {
  using C = SkCfg<LOGM>;
  constexpr int M = C::M, T = C::T, F = C::F, ZS = C::ZS, NT = C::NT;
  extern __shared__ float2 z[];
  float2* stwl = z + F * ZS;
  const int g = threadIdx.x / T, lt = threadIdx.x % T;
  const int64_t nblk = (a.frames + F - 1) / F;
  const int64_t fb = frame_of_block(nblk);
  const int b = blockIdx.y;
  if (fb >= nblk) return;
  const int64_t f0 = fb * F, f = min(f0 + g, a.frames - 1);
  float2* zg = z + g * ZS;
  for (int i = threadIdx.x; i < C::NSTW; i += NT) stwl[i] = a.stw[i];
  // the split step's twiddles W_N^k, loaded now so that their latency hides behind the FFT
  constexpr int VW = F < 4 ? F : 4, CH = F / VW;
  constexpr int KW = ((M + 1) * CH + NT - 1) / NT;  // work items per thread (at most)
  const bool vec = a.frames % F == 0;  // then every block's F frames exist
  float2 wpre[KW];
#pragma unroll
  for (int t = 0; t < KW; ++t) {
    const int i = threadIdx.x + t * NT;
    const int k = min(a.layout == 0 ? i : i / CH, M);
    const float2 tk = a.tw[min(k, M - 1)];  // the table has M entries; W_N^M = -1
    wpre[t] = k == M ? make_float2(-1.f, 0.f) : tk;
  }
  {
    const float* xs = a.x + (int64_t)b * a.n + f * a.hop;
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = lt + r * T;
      const float2 w = *reinterpret_cast<const float2*>(a.win + 2 * m);
      v[r] = make_float2(xs[2 * m] * w.x, xs[2 * m + 1] * w.y);
    }
    dft_reg<16, false>(v);
#pragma unroll
    for (int s = 0; s < 16; ++s) zg[zp(lt * 16 + s)] = v[s];
  }
  __syncthreads();
  if constexpr (C::P == 2) {
    sk_pass<LOGM, C::RL, 16, false>(zg, stwl, lt);
  } else {
    sk_pass<LOGM, 16, 16, false>(zg, stwl, lt);
    sk_pass<LOGM, C::RL, 256, false>(zg, stwl, lt);
  }
  // split step: X[k] = (Z[k] + conj Z[M-k]) / 2 - i W_N^k (Z[k] - conj Z[M-k]) / 2; a work item
  // is bin k of all F frames (frame-major) or of VW of them (bin-major chunk c)
  const int bins = a.onesided ? M + 1 : a.N;
  const int64_t base = (int64_t)b * a.frames * bins;
  auto xk = [&](int j, int k, float2 w) {
    const float2 zk = z[j * ZS + zp(k == M ? 0 : k)];
    const float2 zc = z[j * ZS + zp(k == 0 ? 0 : M - k)];  // Z[M-k], conjugated below
    const float2 fe = make_float2(0.5f * (zk.x + zc.x), 0.5f * (zk.y - zc.y));
    const float2 d = make_float2(0.5f * (zk.x - zc.x), 0.5f * (zk.y + zc.y));
    const float2 t = cmul(w, make_float2(d.y, -d.x));  // w * (-i d)
    return make_float2(fe.x + t.x, fe.y + t.y);
  };
  const bool fm = a.layout == 0;
  const int items = fm ? M + 1 : (M + 1) * CH;
#pragma unroll
  for (int t = 0; t < KW; ++t) {
    const int i = threadIdx.x + t * NT;
    if (i >= items) break;
    const int k = fm ? i : i / CH, c = fm ? 0 : i % CH;
    const float2 w = wpre[t];
    if (fm) {
#pragma unroll
      for (int j = 0; j < F; ++j) {
        if (f0 + j >= a.frames) break;
        const float2 x = xk(j, k, w);
        const int64_t o = base + (f0 + j) * bins;
        a.re[o + k] = x.x;
        a.im[o + k] = x.y;
        if (!a.onesided && k > 0 && k < M) {
          a.re[o + a.N - k] = x.x;
          a.im[o + a.N - k] = -x.y;
        }
      }
      continue;
    }
    float re[VW], im[VW];
#pragma unroll
    for (int u = 0; u < VW; ++u) {
      const float2 x = xk(c * VW + u, k, w);
      re[u] = x.x;
      im[u] = x.y;
    }
    auto put = [&](int kk, bool conj) {
      float* pr = a.re + base + (int64_t)kk * a.frames + f0 + c * VW;
      float* pi = a.im + base + (int64_t)kk * a.frames + f0 + c * VW;
      if (vec && VW == 4) {
        *reinterpret_cast<float4*>(pr) = make_float4(re[0], re[1 % VW], re[2 % VW], re[3 % VW]);
        *reinterpret_cast<float4*>(pi) =
            conj ? make_float4(-im[0], -im[1 % VW], -im[2 % VW], -im[3 % VW])
                 : make_float4(im[0], im[1 % VW], im[2 % VW], im[3 % VW]);
      } else if (vec && VW == 2) {
        *reinterpret_cast<float2*>(pr) = make_float2(re[0], re[1 % VW]);
        *reinterpret_cast<float2*>(pi) = conj ? make_float2(-im[0], -im[1 % VW])
                                              : make_float2(im[0], im[1 % VW]);
      } else {
#pragma unroll
        for (int u = 0; u < VW; ++u)
          if (f0 + c * VW + u < a.frames) {
            pr[u] = re[u];
            pi[u] = conj ? -im[u] : im[u];
          }
      }
    };
    put(k, false);
    if (!a.onesided && k > 0 && k < M) put(a.N - k, true);
  }
}

// Inverse frames on the register-resident FFT: F frames per workgroup. The Hermitian fold
// writes Z in natural order to LDS (a work item loads the pair (k, M - k), and X[N - k],
// X[N - (M - k)] for full spectra, of one frame, or of up to 4 frames as vectors in the bin-major
// layout, so every bin is read once); the passes run from LDS and the last one writes the scaled,
// windowed frame straight to the frame buffer.
template <int LOGM>
__global__ __launch_bounds__(SkCfg<LOGM>::NT) void stft_inverse_sk_kernel(StftArgs a) {
  using C = SkCfg<LOGM>;
  constexpr int M = C::M, T = C::T, F = C::F, ZS = C::ZS, NT = C::NT;
  extern __shared__ float2 z[];
  float2* stwl = z + F * ZS;
  const int g = threadIdx.x / T, lt = threadIdx.x % T;
  const int64_t nblk = (a.frames + F - 1) / F;
  const int64_t fb = frame_of_block(nblk);
  const int b = blockIdx.y;
  if (fb >= nblk) return;
  const int64_t f0 = fb * F;
  for (int i = threadIdx.x; i < C::NSTW; i += NT) stwl[i] = a.stw[i];
  // the last pass (radix R, L = M / R) gives thread lt out[j + s L] for its butterflies
  // j = lt + bb T < L; their window values are loaded now, off the critical path
  constexpr int R = C::RL, L = M / C::RL, NB = 16 / R;
  float2 wv[16];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb)
#pragma unroll
    for (int s = 0; s < R; ++s)
      wv[bb * R + s] = *reinterpret_cast<const float2*>(a.win + 2 * (lt + bb * T + s * L));
  const int bins = a.onesided ? M + 1 : a.N;
  const int64_t base = (int64_t)b * a.frames * bins;
  auto herm = [&](int kk, float2 gv, float2 cv) {  // cv = X[N - kk] (full spectra)
    float2 h = gv;
    if (!a.onesided && kk > 0 && kk < M)
      h = make_float2(0.5f * (gv.x + cv.x), 0.5f * (gv.y - cv.y));
    if (kk == 0 || kk == M) h.y = 0.f;
    return h;
  };
  auto fold = [&](float2 hk, float2 hc, float2 t) {  // Z[k] from H[k], H[M - k]
    const float2 fe = make_float2(0.5f * (hk.x + hc.x), 0.5f * (hk.y - hc.y));
    const float2 d = make_float2(0.5f * (hk.x - hc.x), 0.5f * (hk.y + hc.y));
    const float2 w = make_float2(t.x, -t.y);  // e^{+2 pi i k / N}
    const float2 fo = cmul(d, w);
    return make_float2(fe.x - fo.y, fe.y + fo.x);  // Fe + i Fo
  };
  // Z[k] and Z[M - k] of frame slot j from the bins of the pair
  auto put_pair = [&](int j, int k, float2 gk, float2 gc, float2 ck, float2 cc) {
    const int kc = M - k;
    const float2 hk = herm(k, gk, ck), hc = herm(kc, gc, cc);
    z[j * ZS + zp(k)] = fold(hk, hc, a.tw[k]);
    if (kc < M && kc != k) z[j * ZS + zp(kc)] = fold(hc, hk, a.tw[kc]);
  };
  const float2 zero = make_float2(0.f, 0.f);
  if (a.layout == 0) {
    for (int i = threadIdx.x; i < (M / 2 + 1) * F; i += NT) {
      const int j = i / (M / 2 + 1), k = i - j * (M / 2 + 1), kc = M - k;
      const int64_t o = base + min(f0 + j, a.frames - 1) * bins;
      const float2 gk = make_float2(a.cre[o + k], a.cim[o + k]);
      const float2 gc = make_float2(a.cre[o + kc], a.cim[o + kc]);
      float2 ck = zero, cc = zero;
      if (!a.onesided) {
        const int nk = k > 0 ? a.N - k : k, nc = kc < M ? a.N - kc : kc;
        ck = make_float2(a.cre[o + nk], a.cim[o + nk]);
        cc = make_float2(a.cre[o + nc], a.cim[o + nc]);
      }
      put_pair(j, k, gk, gc, ck, cc);
    }
  } else {
    constexpr int VW = F < 4 ? F : 4, CH = F / VW;
    const bool vec = a.frames % F == 0;  // then every block's F frames exist
    auto get = [&](int kk, int c, float2 (&x)[VW]) {  // X[kk] of frames c VW .. c VW + VW - 1
      const float* pr = a.cre + base + (int64_t)kk * a.frames + f0 + c * VW;
      const float* pi = a.cim + base + (int64_t)kk * a.frames + f0 + c * VW;
      if (vec && VW == 4) {
        const float4 r = *reinterpret_cast<const float4*>(pr);
        const float4 q = *reinterpret_cast<const float4*>(pi);
        const float rr[4] = {r.x, r.y, r.z, r.w}, qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int u = 0; u < VW; ++u) x[u] = make_float2(rr[u], qq[u]);
      } else if (vec && VW == 2) {
        const float2 r = *reinterpret_cast<const float2*>(pr);
        const float2 q = *reinterpret_cast<const float2*>(pi);
        const float rr[2] = {r.x, r.y}, qq[2] = {q.x, q.y};
#pragma unroll
        for (int u = 0; u < VW; ++u) x[u] = make_float2(rr[u], qq[u]);
      } else {
#pragma unroll
        for (int u = 0; u < VW; ++u) {
          const int64_t o = min(f0 + c * VW + u, a.frames - 1) - (f0 + c * VW);
          x[u] = make_float2(pr[o], pi[o]);
        }
      }
    };
    for (int i = threadIdx.x; i < (M / 2 + 1) * CH; i += NT) {
      const int k = i / CH, c = i % CH, kc = M - k;
      float2 gk[VW], gc[VW], ck[VW], cc[VW];
      get(k, c, gk);
      get(kc, c, gc);
      if (!a.onesided) {
        get(k > 0 ? a.N - k : k, c, ck);
        get(kc < M ? a.N - kc : kc, c, cc);
      }
#pragma unroll
      for (int u = 0; u < VW; ++u)
        put_pair(c * VW + u, k, gk[u], gc[u], a.onesided ? zero : ck[u],
                 a.onesided ? zero : cc[u]);
    }
  }
  __syncthreads();
  float2* zg = z + g * ZS;
  {
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = zg[zp(lt + r * T)];
    dft_reg<16, true>(v);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 16; ++s) zg[zp(lt * 16 + s)] = v[s];
    __syncthreads();
  }
  if constexpr (C::P == 3) sk_pass<LOGM, 16, 16, true>(zg, stwl, lt);
  // last pass, into registers
  float2 v[16];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb)
#pragma unroll
    for (int r = 0; r < R; ++r) v[bb * R + r] = zg[zp(lt + bb * T + r * L)];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) {
    const int k = lt + bb * T;  // < L
#pragma unroll
    for (int r = 1; r < R; ++r) {
      float2 w = stwl[(L - 16) + (r - 1) * L + k];
      w.y = -w.y;
      v[bb * R + r] = cmul(v[bb * R + r], w);
    }
    dft_reg<R, true>(v + bb * R);
  }
  const int64_t f = f0 + g;
  if (f >= a.frames) return;
  const float sc = 1.f / (float)M;
  float* out = a.frames_buf + ((int64_t)b * a.frames + f) * a.N;
#pragma unroll
  for (int bb = 0; bb < NB; ++bb)
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int m = lt + bb * T + s * L;
      const float2 w = wv[bb * R + s];
      const float2 x = v[bb * R + s];
      *reinterpret_cast<float2*>(out + 2 * m) = make_float2((x.x * sc) * w.x, (x.y * sc) * w.y);
    }
}

__global__ __launch_bounds__(kThreads) void stft_overlap_add_kernel(StftArgs a) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int b = blockIdx.y;
  const int64_t L = (int64_t)(a.frames - 1) * a.hop + a.N;
  if (t >= L) return;
  int64_t f0 = t - a.N + 1 <= 0 ? 0 : (t - a.N + 1 + a.hop - 1) / a.hop;
  int64_t f1 = t / a.hop;
  if (f1 > a.frames - 1) f1 = a.frames - 1;
  float acc = 0.f, ws = 0.f;
  const float* fr = a.frames_buf + (int64_t)b * a.frames * a.N;
  for (int64_t f = f0; f <= f1; ++f) {
    const int n = (int)(t - f * a.hop);
    acc += fr[f * a.N + n];
    const float w = a.win[n];
    ws += w * w;
  }
  if (ws < 1.17549435e-38f) ws = 0.f;  // FLT_MIN: denormal sums count as zero
  ws = fmaxf(ws, a.floor);
  a.y[(int64_t)b * L + t] = acc / ws;
}

void check(const StftArgs& a) {
  MNN_REQUIRE(a.N >= 4 && a.N <= kStftMaxN && (a.N & (a.N - 1)) == 0 && a.hop > 0 &&
                  a.batch > 0 && a.batch <= 65535 && a.frames > 0 && a.frames <= 2147483640 &&
                  a.win && a.tw,
              MNN_ERR_INVALID_ARGUMENT, "stft: invalid configuration");
}

// Register-resident FFT kernels by log2 M (M = N / 2); null outside their range. Tuning
// override MNN_STFT_SK=0 keeps the LDS radix-2 kernels.
bool use_sk(const StftArgs& a) {
  static const bool on = [] {
    const char* e = std::getenv("MNN_STFT_SK");
    return !e || std::atoi(e) != 0;
  }();
  return on && a.stw && a.logM >= kStftSkMinLogM && a.logM <= kStftSkMaxLogM;
}

template <int LOGM>
void launch_sk(const LaunchCtx& c, const StftArgs& a, bool inverse) {
  using C = SkCfg<LOGM>;
  const dim3 grid((unsigned)(8 * cdiv(cdiv(a.frames, C::F), 8)), (unsigned)a.batch);
  if (inverse)
    launch(c, "istft_frames_f32", stft_inverse_sk_kernel<LOGM>, grid, dim3(C::NT), C::LDS, a);
  else
    launch(c, "stft_forward_f32", stft_forward_sk_kernel<LOGM>, grid, dim3(C::NT), C::LDS, a);
}

void run_sk(const LaunchCtx& c, const StftArgs& a, bool inverse) {
  switch (a.logM) {
    case 6: return launch_sk<6>(c, a, inverse);
    case 7: return launch_sk<7>(c, a, inverse);
    case 8: return launch_sk<8>(c, a, inverse);
    case 9: return launch_sk<9>(c, a, inverse);
    case 10: return launch_sk<10>(c, a, inverse);
    case 11: return launch_sk<11>(c, a, inverse);
    case 12: return launch_sk<12>(c, a, inverse);
    default: fail(MNN_ERR_INVALID_ARGUMENT, "stft: no register-resident FFT for this size");
  }
}

}  // namespace

void stft_forward(const LaunchCtx& c, const StftArgs& a) {
  check(a);
  MNN_REQUIRE(a.x && a.re && a.im && a.n >= a.N &&
                  (int64_t)(a.frames - 1) * a.hop + a.N <= a.n,
              MNN_ERR_INVALID_ARGUMENT, "stft_forward: frames exceed the signal");
  const dim3 grid((unsigned)(8 * cdiv(a.frames, 8)), (unsigned)a.batch);
  const int zs = zslots(a.N / 2);
  if (use_sk(a)) return run_sk(c, a, false);
  if (a.N <= kStftLdsTwMaxN)
    launch(c, "stft_forward_f32", stft_forward_kernel<true>, grid, dim3(kThreads),
           sizeof(float2) * 2 * zs, a);
  else
    launch(c, "stft_forward_f32", stft_forward_kernel<false>, grid, dim3(kThreads),
           sizeof(float2) * zs, a);
}

void stft_inverse(const LaunchCtx& c, const StftArgs& a) {
  check(a);
  MNN_REQUIRE(a.cre && a.cim && a.frames_buf && a.y, MNN_ERR_INVALID_ARGUMENT,
              "stft_inverse: missing buffers");
  const dim3 grid((unsigned)(8 * cdiv(a.frames, 8)), (unsigned)a.batch);
  const int zs = zslots(a.N / 2);
  if (use_sk(a))
    run_sk(c, a, true);
  else if (a.onesided && a.N <= kStftStageMaxN)
    launch(c, "istft_frames_f32", stft_inverse_kernel<true, true>, grid, dim3(kThreads),
           sizeof(float2) * (2 * zs + a.N / 2 + 1), a);
  else if (a.N <= kStftLdsTwMaxN)
    launch(c, "istft_frames_f32", stft_inverse_kernel<true, false>, grid, dim3(kThreads),
           sizeof(float2) * 2 * zs, a);
  else
    launch(c, "istft_frames_f32", stft_inverse_kernel<false, false>, grid, dim3(kThreads),
           sizeof(float2) * zs, a);
  const int64_t L = (int64_t)(a.frames - 1) * a.hop + a.N;
  launch(c, "istft_overlap_add_f32", stft_overlap_add_kernel,
         dim3((unsigned)cdiv(L, kThreads), (unsigned)a.batch), dim3(kThreads), 0, a);
}

}  // namespace k
}  // namespace mnn
