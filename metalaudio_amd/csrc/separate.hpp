// Time-domain HTDemucs separation (HTDemucs.swift: buildTimeUNet :260-293, output heads
// :333-350, forward :376-392, forwardTimeUNet :521-548, separate :617-691) and the long-audio
// segment driver (docs/guides/HTDEMUCS_GUIDE.md:170-191).
#pragma once

#include "layers.hpp"
#include "safetensors.hpp"
#include "weight_names.hpp"

namespace mnn {

class TimeSeparator {
 public:
  TimeSeparator(Device* d, const mnn_separator_desc& desc);
  // "time_encoder.{i}.*" (level i), "time_decoder.{j}.*" (j = 0 is the deepest level, as the
  // reference's timeDecoders array), "time_output_heads.{s}.weight|bias" (the reference's name,
  // HTDemucs.swift:1021; "output_heads.{s}" is accepted as well).
  void load(const std::string& name, const float* data, size_t n);
  // HTDemucs.loadWeights(from:) for the time-domain model: every tensor of the file whose name,
  // mapped to the MetalAudio convention, addresses this model is read as fp32 and loaded; other
  // tensors (the frequency branch, the transformer) are skipped. Returns the number loaded.
  // MNN_ERR_TENSOR_NOT_FOUND (nothing loaded) when a tensor the reference requires is absent.
  int load_safetensors(const SafeTensorsFile& f, WeightConvention conv);
  // x: interleaved [n * C]; out: [S, n * C] interleaved stems
  void separate(const Tensor& x, Tensor& out, Stream& s);
  // Segments of `segment` frames every segment - overlap frames, crossfaded over the frames a
  // segment shares with the previous one.
  void separate_long(const Tensor& x, Tensor& out, int64_t segment, int64_t overlap, Stream& s);
  Device* device() const { return dev_; }

 private:
  void run_segment(const float* x, int64_t n, int64_t start, int64_t len, int64_t fade,
                   float* out, Stream& s);
  void plan(int64_t Lp);
  Device* dev_;
  mnn_separator_desc d_;
  std::vector<std::unique_ptr<Layer>> enc_, dec_, heads_;
  int64_t planned_ = -1;
  DevBuf xp_, y_;
  std::vector<std::unique_ptr<DevBuf>> enc_out_, dec_out_;
  std::vector<Tensor> enc_t_, dec_t_, head_t_;
  Tensor xp_t_;
};

}  // namespace mnn
