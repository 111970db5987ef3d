// Time-domain separation: the U-Net and output heads as library layers, per-length activation
// buffers, and the segment loop of the long-audio driver. Everything stays on the device.
#include "separate.hpp"

namespace mnn {

namespace {

Tensor view(Device* d, void* p, Shape shape) {
  Tensor t;
  t.dev = d;
  t.dtype = MNN_F32;
  t.shape = std::move(shape);
  t.data = p;
  t.bytes = sizeof(float) * numel(t.shape);
  t.owns = false;
  return t;
}

int64_t pad_divisor(int levels, int stride) {
  int64_t d = 1;
  for (int i = 0; i < levels; ++i) {
    MNN_REQUIRE(d <= INT64_MAX / stride, MNN_ERR_INVALID_CONFIGURATION, "stride^levels overflows");
    d *= stride;
  }
  return d;
}

}  // namespace

TimeSeparator::TimeSeparator(Device* d, const mnn_separator_desc& desc) : dev_(d), d_(desc) {
  MNN_REQUIRE(desc.input_channels > 0 && desc.num_stems > 0 && desc.levels > 0 &&
                  desc.levels <= 8 && desc.kernel_size > 0 && desc.stride > 1 &&
                  desc.num_groups > 0,
              MNN_ERR_INVALID_CONFIGURATION, "separator: invalid configuration");
  std::vector<int> ch{desc.input_channels};
  for (int i = 0; i < desc.levels; ++i) {
    MNN_REQUIRE(desc.channels[i] > 0, MNN_ERR_INVALID_CONFIGURATION,
                "separator: channel count of level " << i << " must be positive");
    ch.push_back(desc.channels[i]);
  }
  for (int i = 0; i < desc.levels; ++i) {
    mnn_encoder_block_desc e{};
    e.in_channels = ch[i];
    e.out_channels = ch[i + 1];
    e.kernel_size = desc.kernel_size;
    e.stride = desc.stride;
    e.num_groups = i == 0 ? std::min(desc.num_groups, ch[i]) : desc.num_groups;
    e.rewrite = 0;
    e.precision = MNN_PRECISION_F32;
    enc_.push_back(make_encoder_block(d, e));
  }
  for (int i = desc.levels - 1; i >= 0; --i) {
    mnn_decoder_block_desc c{};
    c.in_channels = ch[i + 1];
    c.skip_channels = ch[i + 1];
    c.out_channels = i == 0 ? desc.input_channels : ch[i];
    c.kernel_size = desc.kernel_size;
    c.stride = desc.stride;
    c.num_groups = std::max(1, i == 0 ? std::min(desc.num_groups, c.out_channels) : desc.num_groups);
    dec_.push_back(make_decoder_block(d, c));
  }
  for (int s = 0; s < desc.num_stems; ++s) {
    mnn_conv1d_desc h{};
    h.in_channels = h.out_channels = desc.input_channels;
    h.kernel_size = h.stride = h.dilation = h.groups = 1;
    h.use_bias = 1;
    h.padding_mode = MNN_PAD_VALID;
    h.activation = MNN_ACT_NONE;
    h.precision = MNN_PRECISION_F32;
    heads_.push_back(make_conv1d(d, h));
  }
}

void TimeSeparator::load(const std::string& name, const float* data, size_t n) {
  auto indexed = [&](const char* prefix, std::vector<std::unique_ptr<Layer>>& v) -> bool {
    const std::string p = prefix;
    if (name.rfind(p, 0) != 0) return false;
    const size_t dot = name.find('.', p.size());
    MNN_REQUIRE(dot != std::string::npos && dot > p.size(), MNN_ERR_INVALID_ARGUMENT,
                "separator: malformed parameter name '" << name << "'");
    int idx = -1;
    try {
      idx = std::stoi(name.substr(p.size(), dot - p.size()));
    } catch (...) {
      idx = -1;
    }
    MNN_REQUIRE(idx >= 0 && idx < (int)v.size(), MNN_ERR_INVALID_ARGUMENT,
                "separator: no layer for parameter '" << name << "'");
    v[idx]->load(name.substr(dot + 1), data, n);
    return true;
  };
  dev_->make_current();
  // heads: the reference's name (HTDemucs.swift:1021) and this library's earlier short form
  if (indexed("time_encoder.", enc_) || indexed("time_decoder.", dec_) ||
      indexed("time_output_heads.", heads_) || indexed("output_heads.", heads_))
    return;
  fail(MNN_ERR_INVALID_ARGUMENT, "separator: unknown parameter '" + name + "'");
}

namespace {
bool separator_tensor(const std::string& m) {
  return m.rfind("time_encoder.", 0) == 0 || m.rfind("time_decoder.", 0) == 0 ||
         m.rfind("time_output_heads.", 0) == 0 || m.rfind("output_heads.", 0) == 0;
}
}  // namespace

int TimeSeparator::load_safetensors(const SafeTensorsFile& f, WeightConvention conv) {
  // The tensors HTDemucs.loadWeights(from:mapper:) requires (HTDemucs.swift:892-937): every
  // encoder conv weight and GroupNorm weight / bias, every decoder transposed-conv weight and
  // GroupNorm weight / bias. Conv biases are optional (loadConv1DWeights,
  // SafeTensorsLoader.swift:238-258) and so are the output heads (:1017-1029). All of them are
  // checked before anything is loaded, so a file that lacks one leaves the model unchanged.
  std::map<std::string, std::string> by_ma;  // MetalAudio name -> the file's own name
  for (const std::string& name : f.names()) {
    const std::string m = to_metalaudio(conv, name);
    if (separator_tensor(m)) by_ma[m] = name;
  }
  auto need = [&](const std::string& a, const std::string& b = std::string()) {
    if (by_ma.count(a) || (!b.empty() && by_ma.count(b))) return;
    fail(MNN_ERR_TENSOR_NOT_FOUND, "separator: tensor '" + a + "' not found in the file");
  };
  for (size_t i = 0; i < enc_.size(); ++i) {
    const std::string p = "time_encoder." + std::to_string(i) + ".";
    need(p + "conv.weight");
    need(p + "norm.weight");
    need(p + "norm.bias");
  }
  for (size_t j = 0; j < dec_.size(); ++j) {
    const std::string p = "time_decoder." + std::to_string(j) + ".";
    need(p + "conv_transpose.weight", p + "conv_tr.weight");
    need(p + "norm.weight");
    need(p + "norm.bias");
  }
  std::vector<float> buf;
  for (const auto& kv : by_ma) {
    const int64_t n = f.info(kv.second).count();
    buf.resize((size_t)n);
    f.read_f32(kv.second, buf.data(), buf.size());
    load(kv.first, buf.data(), buf.size());
  }
  return (int)by_ma.size();
}

void TimeSeparator::plan(int64_t Lp) {
  if (planned_ == Lp) return;
  const int C = d_.input_channels, S = d_.num_stems, Lv = d_.levels;
  xp_.reserve(sizeof(float) * C * Lp);
  xp_t_ = view(dev_, xp_.ptr, {1, C, Lp});
  while ((int)enc_out_.size() < Lv) enc_out_.push_back(std::make_unique<DevBuf>());
  while ((int)dec_out_.size() < Lv) dec_out_.push_back(std::make_unique<DevBuf>());
  enc_t_.clear();
  dec_t_.clear();
  int64_t L = Lp;
  for (int i = 0; i < Lv; ++i) {
    L /= d_.stride;
    enc_out_[i]->reserve(sizeof(float) * d_.channels[i] * L);
    enc_t_.push_back(view(dev_, enc_out_[i]->ptr, {1, d_.channels[i], L}));
  }
  for (int j = 0; j < Lv; ++j) {
    const int i = Lv - 1 - j;
    L *= d_.stride;
    const int co = i == 0 ? C : d_.channels[i - 1];
    dec_out_[j]->reserve(sizeof(float) * co * L);
    dec_t_.push_back(view(dev_, dec_out_[j]->ptr, {1, co, L}));
  }
  MNN_REQUIRE(L == Lp, MNN_ERR_INVALID_CONFIGURATION,
              "separator: decoder output length " << L << " differs from the padded input " << Lp);
  y_.reserve(sizeof(float) * S * C * Lp);
  head_t_.clear();
  for (int s = 0; s < S; ++s)
    head_t_.push_back(view(dev_, static_cast<float*>(y_.ptr) + (int64_t)s * C * Lp, {1, C, Lp}));
  planned_ = Lp;
}

void TimeSeparator::run_segment(const float* x, int64_t n, int64_t start, int64_t len,
                                int64_t fade, float* out, Stream& s) {
  const int64_t div = pad_divisor(d_.levels, d_.stride);
  const int64_t rem = len % div, total = rem == 0 ? 0 : div - rem;
  const int64_t lp = total / 2, Lp = len + total;
  plan(Lp);
  const LaunchCtx c{s.dev, s.s};
  k::SegmentArgs a;
  a.C = d_.input_channels;
  a.S = d_.num_stems;
  a.n = n;
  a.start = start;
  a.len = len;
  a.Lp = Lp;
  a.lp = lp;
  a.fade = fade;
  a.x = x;
  a.xp = xp_.f32();
  a.y = y_.f32();
  a.out = out;
  k::segment_deinterleave_pad(c, a);
  const Tensor* cur = &xp_t_;
  for (size_t i = 0; i < enc_.size(); ++i) {
    enc_[i]->forward(*cur, enc_t_[i], s);
    cur = &enc_t_[i];
  }
  for (size_t j = 0; j < dec_.size(); ++j) {
    const Tensor& skip = enc_t_[enc_.size() - 1 - j];
    dec_[j]->forward_cross(cur, &skip, &dec_t_[j], nullptr, s);
    cur = &dec_t_[j];
  }
  for (size_t h = 0; h < heads_.size(); ++h) heads_[h]->forward(*cur, head_t_[h], s);
  k::segment_crossfade_store(c, a);
}

void TimeSeparator::separate(const Tensor& x, Tensor& out, Stream& s) {
  separate_long(x, out, 0, 0, s);
}

void TimeSeparator::separate_long(const Tensor& x, Tensor& out, int64_t segment, int64_t overlap,
                                  Stream& s) {
  const int C = d_.input_channels, S = d_.num_stems;
  MNN_REQUIRE(x.dtype == MNN_F32 && out.dtype == MNN_F32, MNN_ERR_INVALID_ARGUMENT,
              "separator: tensors must be f32");
  MNN_REQUIRE(x.shape.size() == 1 && x.shape[0] % C == 0 && x.shape[0] > 0,
              MNN_ERR_SHAPE_MISMATCH,
              "separator: input must be interleaved [n * " << C << "], got " << shape_str(x.shape));
  const int64_t n = x.shape[0] / C;
  MNN_REQUIRE(out.shape == Shape({S, n * C}), MNN_ERR_SHAPE_MISMATCH,
              "separator: output must be [" << S << ", " << n * C << "]");
  if (segment <= 0 || segment >= n) {  // one pass over the whole input
    run_segment(x.f32(), n, 0, n, 0, out.f32(), s);
    return;
  }
  MNN_REQUIRE(overlap >= 0 && overlap < segment, MNN_ERR_INVALID_ARGUMENT,
              "separator: overlap must be in [0, segment)");
  int64_t prev_end = 0;
  for (int64_t start = 0; start < n; start += segment - overlap) {
    const int64_t end = std::min(start + segment, n);
    run_segment(x.f32(), n, start, end - start, std::max<int64_t>(0, prev_end - start),
                out.f32(), s);
    prev_end = end;
    if (end == n) break;
  }
}

}  // namespace mnn
