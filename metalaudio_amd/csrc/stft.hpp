// STFT plan (FFT.Config + STFT, FFT.swift:150-300 and STFT.swift:20-533): FFT size, hop, window
// and the device tables (window, twiddles) and the inverse's frame workspace.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace mnn {

class StftPlan {
 public:
  // window: 0 none, 1 Hann, 2 Hamming, 3 Blackman (WindowType.coefficient, symmetric, N - 1
  // denominator, evaluated in double and rounded to float).
  StftPlan(Device* d, int fft_size, int hop, int window);
  int fft_size() const { return N_; }
  int hop() const { return hop_; }
  const std::vector<float>& window() const { return win_host_; }
  int64_t frame_count(int64_t samples) const;    // (n - N) / hop + 1; error if n < N
  int64_t output_length(int64_t frames) const;   // (frames - 1) * hop + N, overflow-checked
  // x [n] or [B, n] -> re/im [B?, frames, bins] (layout 0) or [B?, bins, frames] (layout 1)
  void forward(const Tensor& x, Tensor& re, Tensor& im, bool onesided, int layout, Stream& s);
  void inverse(const Tensor& re, const Tensor& im, bool onesided, int layout, float floor,
               Tensor& y, Stream& s);
  Device* device() const { return dev_; }

 private:
  Shape spectrum_shape(int64_t B, bool batched, int64_t frames, bool onesided, int layout) const;
  Device* dev_;
  int N_, hop_, window_;
  std::vector<float> win_host_;
  DevBuf win_, tw_, stw_, frames_;
};

float window_coefficient(int window, int index, int length);
// The floor the inverse divides by (STFT.swift:491-501): below 1e-10 -> 1e-6, above 0.1 -> 0.1.
float stft_effective_floor(float configured);

}  // namespace mnn
