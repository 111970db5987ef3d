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
constexpr int kStftLdsTwMaxN = 8192;  // LDS twiddles up to 64 KB of LDS per workgroup

__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}

// In-place radix-2 DIT FFT of z[0..M) (bit-reversed input order) in LDS; inverse uses conjugate
// twiddles (no scaling). tw[k] = e^{-2 pi i k / N}, N = 2M.
__device__ void fft_lds(float2* z, int M, const float2* __restrict__ tw, bool inverse) {
  for (int h = 1; h < M; h <<= 1) {
    const int stride = M / h;  // W_{2h}^p = tw[p * M / h]
    for (int t = threadIdx.x; t < M / 2; t += kThreads) {
      const int p = t & (h - 1);
      const int i0 = ((t - p) << 1) + p, i1 = i0 + h;
      float2 w = tw[p * stride];
      if (inverse) w.y = -w.y;
      const float2 a = z[i0], b = cmul(z[i1], w);
      z[i0] = make_float2(a.x + b.x, a.y + b.y);
      z[i1] = make_float2(a.x - b.x, a.y - b.y);
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
  float2* tws = z + M;
  const float* xs = a.x + (int64_t)b * a.n + (int64_t)f * a.hop;
  for (int m = threadIdx.x; m < M; m += kThreads) {
    const float e = xs[2 * m] * a.win[2 * m], o = xs[2 * m + 1] * a.win[2 * m + 1];
    z[bitrev(m, a.logM)] = make_float2(e, o);
    if (LDS_TW) tws[m] = a.tw[m];
  }
  __syncthreads();
  fft_lds(z, M, LDS_TW ? tws : a.tw, false);
  const int bins = a.onesided ? M + 1 : a.N;
  const int64_t base = (int64_t)b * a.frames * bins;
  for (int k = threadIdx.x; k <= M; k += kThreads) {
    const float2 zk = z[k == M ? 0 : k];
    const float2 zc = z[k == 0 ? 0 : M - k];  // Z[M-k], conjugated below
    const float2 fe = make_float2(0.5f * (zk.x + zc.x), 0.5f * (zk.y - zc.y));
    const float2 d = make_float2(0.5f * (zk.x - zc.x), 0.5f * (zk.y + zc.y));  // (Zk - conj Zc)/2
    const float2 fo = make_float2(d.y, -d.x);                                    // -i * d
    const float2 w = k == M ? make_float2(-1.f, 0.f) : (LDS_TW ? tws[k] : a.tw[k]);
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

template <bool LDS_TW>
__global__ __launch_bounds__(kThreads) void stft_inverse_kernel(StftArgs a) {
  extern __shared__ float2 z[];
  const int64_t f = frame_of_block(a.frames);
  const int b = blockIdx.y;
  if (f >= a.frames) return;
  const int M = a.N / 2;
  float2* tws = z + M;
  const int bins = a.onesided ? M + 1 : a.N;
  const int64_t base = (int64_t)b * a.frames * bins;
  auto get = [&](int kk) {
    const int64_t o = a.layout == 0 ? base + (int64_t)f * bins + kk
                                    : base + (int64_t)kk * a.frames + f;
    return make_float2(a.cre[o], a.cim[o]);
  };
  // Hermitian part H[k] of the input spectrum, k in [0, M]: the real part of the inverse DFT
  // depends on nothing else.
  auto herm = [&](int kk) {
    float2 h = get(kk);
    if (!a.onesided && kk > 0 && kk < M) {
      const float2 c = get(a.N - kk);
      h = make_float2(0.5f * (h.x + c.x), 0.5f * (h.y - c.y));
    }
    if (kk == 0 || kk == M) h.y = 0.f;
    return h;
  };
  for (int k = threadIdx.x; k < M; k += kThreads) {
    const float2 hk = herm(k), hc = herm(M - k);
    const float2 fe = make_float2(0.5f * (hk.x + hc.x), 0.5f * (hk.y - hc.y));
    const float2 d = make_float2(0.5f * (hk.x - hc.x), 0.5f * (hk.y + hc.y));
    const float2 t = a.tw[k];
    if (LDS_TW) tws[k] = t;
    const float2 w = make_float2(t.x, -t.y);  // e^{+2 pi i k / N}
    const float2 fo = cmul(d, w);
    z[bitrev(k, a.logM)] = make_float2(fe.x - fo.y, fe.y + fo.x);  // Fe + i Fo
  }
  __syncthreads();
  fft_lds(z, M, LDS_TW ? tws : a.tw, true);
  const float s = 1.f / (float)M;
  float* out = a.frames_buf + ((int64_t)b * a.frames + f) * a.N;
  for (int m = threadIdx.x; m < M; m += kThreads) {
    const float2 v = z[m];
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
  if (a.N <= kStftLdsTwMaxN)
    launch(c, "stft_forward_f32", stft_forward_kernel<true>, grid, dim3(kThreads),
           sizeof(float2) * a.N, a);
  else
    launch(c, "stft_forward_f32", stft_forward_kernel<false>, grid, dim3(kThreads),
           sizeof(float2) * (a.N / 2), a);
}

void stft_inverse(const LaunchCtx& c, const StftArgs& a) {
  check(a);
  MNN_REQUIRE(a.cre && a.cim && a.frames_buf && a.y, MNN_ERR_INVALID_ARGUMENT,
              "stft_inverse: missing buffers");
  const dim3 grid((unsigned)(8 * cdiv(a.frames, 8)), (unsigned)a.batch);
  if (a.N <= kStftLdsTwMaxN)
    launch(c, "istft_frames_f32", stft_inverse_kernel<true>, grid, dim3(kThreads),
           sizeof(float2) * a.N, a);
  else
    launch(c, "istft_frames_f32", stft_inverse_kernel<false>, grid, dim3(kThreads),
           sizeof(float2) * (a.N / 2), a);
  const int64_t L = (int64_t)(a.frames - 1) * a.hop + a.N;
  launch(c, "istft_overlap_add_f32", stft_overlap_add_kernel,
         dim3((unsigned)cdiv(L, kThreads), (unsigned)a.batch), dim3(kThreads), 0, a);
}

}  // namespace k
}  // namespace mnn
