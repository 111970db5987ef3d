// STFT plan: host tables and shape checks around the kernels of k_stft.hip.
#include "stft.hpp"

#include <cmath>

namespace mnn {

float window_coefficient(int window, int index, int length) {
  if (length <= 1) return 1.f;
  const double n = index, d = (double)length - 1.0, pi = 3.14159265358979323846;
  switch (window) {
    case 0: return 1.f;
    case 1: return (float)(0.5 * (1.0 - std::cos(2.0 * pi * n / d)));
    case 2: return (float)(0.54 - 0.46 * std::cos(2.0 * pi * n / d));
    case 3:
      return (float)(0.42 - 0.5 * std::cos(2.0 * pi * n / d) + 0.08 * std::cos(4.0 * pi * n / d));
    default: fail(MNN_ERR_INVALID_ARGUMENT, "unknown window type " + std::to_string(window));
  }
  return 0.f;
}

float stft_effective_floor(float f) {
  if (!(f >= 1e-10f)) return 1e-6f;
  if (f > 0.1f) return 0.1f;
  return f;
}

StftPlan::StftPlan(Device* d, int fft_size, int hop, int window)
    : dev_(d), N_(fft_size), hop_(hop), window_(window) {
  MNN_REQUIRE(fft_size >= 4 && fft_size <= k::kStftMaxN && (fft_size & (fft_size - 1)) == 0,
              MNN_ERR_INVALID_CONFIGURATION,
              "FFT size must be a power of 2 in [4, " << k::kStftMaxN << "], got " << fft_size);
  MNN_REQUIRE(hop > 0, MNN_ERR_INVALID_CONFIGURATION, "hop size must be positive");
  MNN_REQUIRE(window >= 0 && window <= 3, MNN_ERR_INVALID_CONFIGURATION, "unknown window type");
  win_host_.resize(N_);
  for (int i = 0; i < N_; ++i) win_host_[i] = window_coefficient(window, i, N_);
  std::vector<float> tw((size_t)N_);  // N/2 complex
  const double pi = 3.14159265358979323846;
  for (int k = 0; k < N_ / 2; ++k) {
    tw[2 * k] = (float)std::cos(-2.0 * pi * k / N_);
    tw[2 * k + 1] = (float)std::sin(-2.0 * pi * k / N_);
  }
  // Stockham pass twiddles W_{L R}^{r k} = e^{-2 pi i r k / (L R)}, pass by pass, [r - 1][k]
  std::vector<float> stw;
  int logm = 0;
  while ((2 << logm) < N_) ++logm;
  if (logm >= k::kStftSkMinLogM && logm <= k::kStftSkMaxLogM) {
    int L = k::stft_sk_radix(logm, 0);
    for (int p = 1; p < k::stft_sk_passes(logm); ++p) {
      const int R = k::stft_sk_radix(logm, p);
      for (int r = 1; r < R; ++r)
        for (int kk = 0; kk < L; ++kk) {
          stw.push_back((float)std::cos(-2.0 * pi * r * kk / ((double)L * R)));
          stw.push_back((float)std::sin(-2.0 * pi * r * kk / ((double)L * R)));
        }
      L *= R;
    }
    MNN_REQUIRE(stw.size() == 2 * (size_t)(N_ / 2 - 16), MNN_ERR_INVALID_CONFIGURATION,
                "Stockham twiddle table size");
  }
  d->make_current();
  win_.reserve(sizeof(float) * N_);
  tw_.reserve(sizeof(float) * N_);
  HIP_CHECK(hipMemcpy(win_.ptr, win_host_.data(), sizeof(float) * N_, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(tw_.ptr, tw.data(), sizeof(float) * N_, hipMemcpyHostToDevice));
  if (!stw.empty()) {
    stw_.reserve(sizeof(float) * stw.size());
    HIP_CHECK(hipMemcpy(stw_.ptr, stw.data(), sizeof(float) * stw.size(), hipMemcpyHostToDevice));
  }
}

int64_t StftPlan::frame_count(int64_t n) const {
  MNN_REQUIRE(n >= N_, MNN_ERR_INVALID_ARGUMENT,
              "input of " << n << " samples is shorter than the FFT size " << N_);
  return (n - N_) / hop_ + 1;
}

int64_t StftPlan::output_length(int64_t frames) const {
  MNN_REQUIRE(frames > 0 && frames - 1 <= (INT64_MAX - N_) / hop_, MNN_ERR_INVALID_ARGUMENT,
              "iSTFT output length overflows for " << frames << " frames");
  return (frames - 1) * hop_ + N_;
}

Shape StftPlan::spectrum_shape(int64_t B, bool batched, int64_t frames, bool onesided,
                               int layout) const {
  const int64_t bins = onesided ? N_ / 2 + 1 : N_;
  Shape s = layout == 0 ? Shape{frames, bins} : Shape{bins, frames};
  if (batched) s.insert(s.begin(), B);
  return s;
}

namespace {
int log2i(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}
}  // namespace

void StftPlan::forward(const Tensor& x, Tensor& re, Tensor& im, bool onesided, int layout,
                       Stream& s) {
  MNN_REQUIRE(layout == 0 || layout == 1, MNN_ERR_INVALID_ARGUMENT, "layout must be 0 or 1");
  MNN_REQUIRE(x.dtype == MNN_F32 && re.dtype == MNN_F32 && im.dtype == MNN_F32,
              MNN_ERR_INVALID_ARGUMENT, "STFT tensors must be f32");
  MNN_REQUIRE(x.shape.size() == 1 || x.shape.size() == 2, MNN_ERR_SHAPE_MISMATCH,
              "STFT input must be [n] or [B, n], got " << shape_str(x.shape));
  const bool batched = x.shape.size() == 2;
  const int64_t B = batched ? x.shape[0] : 1, n = x.shape.back();
  const int64_t F = frame_count(n);
  const Shape want = spectrum_shape(B, batched, F, onesided, layout);
  MNN_REQUIRE(re.shape == want && im.shape == want, MNN_ERR_SHAPE_MISMATCH,
              "STFT outputs must be " << shape_str(want));
  k::StftArgs a;
  a.N = N_;
  a.logM = log2i(N_ / 2);
  a.hop = hop_;
  a.batch = (int)B;
  a.onesided = onesided;
  a.layout = layout;
  a.n = n;
  a.frames = F;
  a.win = win_.f32();
  a.tw = static_cast<const float2*>(tw_.ptr);
  a.stw = static_cast<const float2*>(stw_.ptr);
  a.x = x.f32();
  a.re = re.f32();
  a.im = im.f32();
  k::stft_forward(LaunchCtx{s.dev, s.s}, a);
}

void StftPlan::inverse(const Tensor& re, const Tensor& im, bool onesided, int layout,
                       float floor, Tensor& y, Stream& s) {
  MNN_REQUIRE(layout == 0 || layout == 1, MNN_ERR_INVALID_ARGUMENT, "layout must be 0 or 1");
  MNN_REQUIRE(re.dtype == MNN_F32 && im.dtype == MNN_F32 && y.dtype == MNN_F32,
              MNN_ERR_INVALID_ARGUMENT, "iSTFT tensors must be f32");
  MNN_REQUIRE((re.shape.size() == 2 || re.shape.size() == 3) && re.shape == im.shape,
              MNN_ERR_SHAPE_MISMATCH, "iSTFT real/imag must match and be 2-D or 3-D");
  const bool batched = re.shape.size() == 3;
  const int64_t B = batched ? re.shape[0] : 1;
  const int64_t bins = onesided ? N_ / 2 + 1 : N_;
  const int64_t F = layout == 0 ? re.shape[re.shape.size() - 2] : re.shape.back();
  const int64_t got_bins = layout == 0 ? re.shape.back() : re.shape[re.shape.size() - 2];
  MNN_REQUIRE(got_bins == bins && F > 0, MNN_ERR_SHAPE_MISMATCH,
              "iSTFT input has " << got_bins << " bins, expected " << bins);
  const int64_t L = output_length(F);
  const Shape want = batched ? Shape{B, L} : Shape{L};
  MNN_REQUIRE(y.shape == want, MNN_ERR_SHAPE_MISMATCH,
              "iSTFT output must be " << shape_str(want));
  frames_.reserve(sizeof(float) * B * F * N_);
  k::StftArgs a;
  a.N = N_;
  a.logM = log2i(N_ / 2);
  a.hop = hop_;
  a.batch = (int)B;
  a.onesided = onesided;
  a.layout = layout;
  a.frames = F;
  a.win = win_.f32();
  a.tw = static_cast<const float2*>(tw_.ptr);
  a.stw = static_cast<const float2*>(stw_.ptr);
  a.cre = re.f32();
  a.cim = im.f32();
  a.frames_buf = frames_.f32();
  a.y = y.f32();
  a.floor = stft_effective_floor(floor);
  k::stft_inverse(LaunchCtx{s.dev, s.s}, a);
}

}  // namespace mnn
