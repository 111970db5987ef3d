// Short-time Fourier transform of the frequency branch (STFT.swift:40-80 and :384-533 over the
// FFT of FFT.swift): analysis frames of N samples every `hop` samples (no centring padding), the
// window applied, a full N-point DFT without scaling; the inverse takes the real part of each
// frame's inverse DFT scaled by 1/N, applies the window again, overlap-adds the frames and
// divides by the overlap-added squared window floored at `floor` (values below FLT_MIN counted as
// zero first).
//
// One workgroup per (signal, frame). A real N-point DFT is computed as a complex M = N/2-point
// FFT of z[m] = x[2m] + i x[2m+1] and the split step
//   X[k] = (Z[k] + conj Z[M-k]) / 2 - i e^{-2 pi i k / N} (Z[k] - conj Z[M-k]) / 2,  0 <= k <= M
// (X[N-k] = conj X[k] for the full spectrum). The M-point FFT is radix-2 decimation in time in
// LDS (input stored bit-reversed, log2 M butterfly passes, one barrier each). Twiddles
// e^{-2 pi i k / N}, k < M, come from a table computed on the host in double precision.
// The inverse runs the same steps backwards (Hermitian fold of the input, merge into Z, inverse
// FFT with conjugate twiddles, 1/M); the overlap-add is a gather over the frames that cover each
// output sample, in increasing frame order, so it needs no atomics.
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
  auto twd = [&](int i) { return tw[TWP ? zp(i) : i]; };
  int h = 1;
  for (; 2 * h < M; h <<= 2) {
    const int s1 = M / h, s2 = M / (2 * h);  // W_2h^p = tw[p * s1], W_4h^p = tw[p * s2]
    for (int t = threadIdx.x; t < M / 4; t += kThreads) {
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
    for (int t = threadIdx.x; t < M / 2; t += kThreads) {
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
    const float2 w = k == M ? make_float2(-1.f, 0.f) : (LDS_TW ? tws[zp(k)] : a.tw[k]);
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

}  // namespace

void stft_forward(const LaunchCtx& c, const StftArgs& a) {
  check(a);
  MNN_REQUIRE(a.x && a.re && a.im && a.n >= a.N &&
                  (int64_t)(a.frames - 1) * a.hop + a.N <= a.n,
              MNN_ERR_INVALID_ARGUMENT, "stft_forward: frames exceed the signal");
  const dim3 grid((unsigned)(8 * cdiv(a.frames, 8)), (unsigned)a.batch);
  const int zs = zslots(a.N / 2);
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
  if (a.onesided && a.N <= kStftStageMaxN)
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
