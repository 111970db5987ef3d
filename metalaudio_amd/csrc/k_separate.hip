// Time-domain separation around the U-Net (HTDemucs.separate, HTDemucs.swift:617-691) and the
// long-audio segment driver: de-interleave + zero padding of one segment of interleaved audio
// into the network's planar input, and the write-back of each stem into the interleaved output
// with a linear crossfade over the frames a segment shares with the previous one.
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mnn {
namespace k {

namespace {

constexpr int kThreads = 256;

// xp[ch][t] = x[(start + t - lp) * C + ch] for lp <= t < lp + len, zero elsewhere (t < Lp).
__global__ __launch_bounds__(kThreads) void deinterleave_pad_kernel(SegmentArgs a) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int ch = blockIdx.y;
  if (t >= a.Lp) return;
  const int64_t i = t - a.lp;
  float v = 0.f;
  if (i >= 0 && i < a.len) v = a.x[(a.start + i) * a.C + ch];
  a.xp[(int64_t)ch * a.Lp + t] = v;
}

// out[s][(start + i) * C + ch] from y[s][ch][lp + i], i < len; the first `fade` frames blend
// with what the previous segment wrote: out = out * (1 - w) + y * w, w = (i + 1) / (fade + 1).
__global__ __launch_bounds__(kThreads) void crossfade_store_kernel(SegmentArgs a) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int ch = blockIdx.y, s = blockIdx.z;
  if (i >= a.len) return;
  const float y = a.y[((int64_t)s * a.C + ch) * a.Lp + a.lp + i];
  float* o = a.out + (int64_t)s * a.n * a.C + (a.start + i) * a.C + ch;
  if (i < a.fade) {
    const float w = (float)(i + 1) / (float)(a.fade + 1);
    *o = *o * (1.f - w) + y * w;
  } else {
    *o = y;
  }
}

}  // namespace

void segment_deinterleave_pad(const LaunchCtx& c, const SegmentArgs& a) {
  MNN_REQUIRE(a.x && a.xp && a.C > 0 && a.C <= 65535 && a.lp >= 0 && a.len > 0 &&
                  a.lp + a.len <= a.Lp && a.start >= 0 && a.start + a.len <= a.n,
              MNN_ERR_INVALID_ARGUMENT, "segment: invalid de-interleave arguments");
  launch(c, "deinterleave_pad_f32", deinterleave_pad_kernel,
         dim3((unsigned)cdiv(a.Lp, kThreads), (unsigned)a.C), dim3(kThreads), 0, a);
}

void segment_crossfade_store(const LaunchCtx& c, const SegmentArgs& a) {
  MNN_REQUIRE(a.y && a.out && a.C > 0 && a.C <= 65535 && a.S > 0 && a.S <= 65535 &&
                  a.len > 0 && a.lp + a.len <= a.Lp && a.start >= 0 && a.start + a.len <= a.n &&
                  a.fade >= 0 && a.fade <= a.len,
              MNN_ERR_INVALID_ARGUMENT, "segment: invalid store arguments");
  launch(c, "crossfade_store_f32", crossfade_store_kernel,
         dim3((unsigned)cdiv(a.len, kThreads), (unsigned)a.C, (unsigned)a.S), dim3(kThreads), 0,
         a);
}

}  // namespace k
}  // namespace mnn
