// Hot-path layers of the MetalNN stack on MI355X. Each class states the reference type it
// stands in for; the arithmetic lives in the k_*.hip kernels, this file only plans launches.
#include "layers.hpp"

#include <algorithm>
#include <cmath>

namespace mnn {

namespace {

LaunchCtx ctx(Stream& s) { return LaunchCtx{s.dev, s.s}; }

// [C, L] / [B, C, L] -> (B, C, L)
void split_bcl(const Shape& s, int64_t& B, int64_t& C, int64_t& L) {
  MNN_REQUIRE(s.size() == 2 || s.size() == 3, MNN_ERR_SHAPE_MISMATCH,
              "expected [C, L] or [B, C, L], got " << shape_str(s));
  B = s.size() == 3 ? s[0] : 1;
  C = s[s.size() - 2];
  L = s[s.size() - 1];
}

// [S, E] / [B, S, E] -> (B, S, E); a 1-D [E] is one row.
void split_bse(const Shape& s, int64_t& B, int64_t& S, int64_t& E) {
  MNN_REQUIRE(s.size() >= 1 && s.size() <= 3, MNN_ERR_SHAPE_MISMATCH,
              "expected [E], [S, E] or [B, S, E], got " << shape_str(s));
  E = s.back();
  S = s.size() >= 2 ? s[s.size() - 2] : 1;
  B = s.size() == 3 ? s[0] : 1;
}

Shape with_last(Shape s, int64_t last) {
  s.back() = last;
  return s;
}

}  // namespace

// ------------------------------------------------------------------ Layer base
void Layer::forward_cross(const Tensor*, const Tensor*, Tensor*, Tensor*, Stream&) {
  fail(MNN_ERR_INVALID_CONFIGURATION, std::string(kind()) + " has no two-input forward");
}

Param& Layer::add_param(const std::string& name, int64_t count, float fill) {
  auto p = std::make_unique<Param>();
  p->name = name;
  p->count = count;
  dev_->make_current();
  p->buf.reserve(sizeof(float) * std::max<int64_t>(count, 1));
  std::vector<float> init(std::max<int64_t>(count, 1), fill);
  HIP_CHECK(hipMemcpy(p->buf.ptr, init.data(), sizeof(float) * count, hipMemcpyHostToDevice));
  params_.push_back(std::move(p));
  return *params_.back();
}

Param* Layer::find_param(const std::string& name) {
  std::string n = name;
  auto a = aliases_.find(n);
  if (a != aliases_.end()) n = a->second;
  for (auto& p : params_)
    if (p->name == n) return p.get();
  return nullptr;
}

void Layer::load(const std::string& name, const float* data, size_t n) {
  Param* p = find_param(name);
  MNN_REQUIRE(p, MNN_ERR_INVALID_ARGUMENT, kind() << ": unknown parameter '" << name << "'");
  MNN_REQUIRE((int64_t)n == p->count, MNN_ERR_BUFFER_SIZE_MISMATCH,
              kind() << " parameter '" << name << "': expected " << p->count << " values, got "
                     << n);
  MNN_REQUIRE(data || n == 0, MNN_ERR_INVALID_ARGUMENT, "null data");
  for (size_t i = 0; i < n; ++i) {
    MNN_REQUIRE(!std::isnan(data[i]), MNN_ERR_INVALID_CONFIGURATION,
                name << " contain NaN values - model file may be corrupted");
    MNN_REQUIRE(!std::isinf(data[i]), MNN_ERR_INVALID_CONFIGURATION,
                name << " contain Inf values - possible exploding gradients during training");
  }
  dev_->make_current();
  HIP_CHECK(hipMemcpy(p->buf.ptr, data, sizeof(float) * n, hipMemcpyHostToDevice));
  p->loaded = true;
  ++p->version;
  on_loaded(p->name, data, n);
}

void Layer::check_out(const Tensor& out, const Shape& expect) const {
  MNN_REQUIRE(out.count() == numel(expect), MNN_ERR_BUFFER_SIZE_MISMATCH,
              kind() << ": output holds " << out.count() << " elements, expected "
                     << shape_str(expect));
  MNN_REQUIRE(out.dtype == MNN_F32, MNN_ERR_INVALID_ARGUMENT, kind() << ": output must be f32");
}

// ------------------------------------------------------------------ Conv1D / DynamicConv1D
// Conv1D (Conv1D.swift:11-514), DynamicConv1D (DynamicConv1D.swift:35-403) and FusedConv1D's
// activation epilogue (Conv1D.swift:742-1028). Dense contractions (Cin*K >= 64) run as an
// implicit GEMM on the matrix cores; small ones on the direct kernel.
class Conv1DLayer : public Layer {
 public:
  Conv1DLayer(Device* d, const mnn_conv1d_desc& desc, float leaky_alpha = 0.01f)
      : Layer(d), p_(desc), alpha_(leaky_alpha) {
    MNN_REQUIRE(std::isfinite(leaky_alpha), MNN_ERR_INVALID_CONFIGURATION,
                "FusedConv1D: leakyReluAlpha must be finite");
    MNN_REQUIRE(p_.in_channels > 0 && p_.out_channels > 0 && p_.kernel_size > 0 &&
                    p_.stride > 0 && p_.dilation > 0 && p_.groups > 0,
                MNN_ERR_INVALID_CONFIGURATION, "Conv1D: sizes must be positive");
    MNN_REQUIRE(p_.in_channels % p_.groups == 0 && p_.out_channels % p_.groups == 0,
                MNN_ERR_INVALID_CONFIGURATION, "Conv1D: channels must be divisible by groups");
    MNN_REQUIRE(p_.padding >= 0, MNN_ERR_INVALID_CONFIGURATION, "Conv1D: negative padding");
    w_ = &add_param("weight",
                    (int64_t)p_.out_channels * (p_.in_channels / p_.groups) * p_.kernel_size);
    if (p_.use_bias) b_ = &add_param("bias", p_.out_channels);
    if (p_.input_length > 0)
      MNN_REQUIRE(out_len(p_.input_length) > 0, MNN_ERR_INVALID_CONFIGURATION,
                  "Conv1D: output length would be <= 0");
  }
  const char* kind() const override { return p_.input_length > 0 ? "Conv1D" : "DynamicConv1D"; }
  Shape input_shape() const override { return {p_.in_channels, p_.input_length}; }
  Shape output_shape() const override {
    return {p_.out_channels, p_.input_length > 0 ? out_len(p_.input_length) : 0};
  }
  int pad_for(int64_t L) const {
    switch (p_.padding_mode) {
      case MNN_PAD_VALID: return 0;
      case MNN_PAD_SAME: {  // DynamicConv1D.swift:167-173
        const int64_t eff = (int64_t)(p_.kernel_size - 1) * p_.dilation + 1;
        const int64_t outl = (L + p_.stride - 1) / p_.stride;
        const int64_t total = std::max<int64_t>(0, (outl - 1) * p_.stride + eff - L);
        return (int)(total / 2);
      }
      default: return p_.padding;
    }
  }
  // output = floor((L + 2p - ((k-1)d + 1)) / s) + 1 (DynamicConv1D.swift:153-161)
  int64_t out_len(int64_t L) const {
    const int64_t eff = (int64_t)(p_.kernel_size - 1) * p_.dilation + 1;
    const int64_t num = L + 2 * pad_for(L) - eff;
    return num < 0 ? 0 : num / p_.stride + 1;
  }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, L;
    split_bcl(in, B, C, L);
    MNN_REQUIRE(C == p_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                kind() << ": expected " << p_.in_channels << " input channels, got " << C);
    if (p_.input_length > 0)
      MNN_REQUIRE(L == p_.input_length, MNN_ERR_SHAPE_MISMATCH,
                  "Conv1D: expected input length " << p_.input_length << ", got " << L);
    const int64_t lo = out_len(L);
    MNN_REQUIRE(lo > 0, MNN_ERR_SHAPE_MISMATCH, kind() << ": input length " << L << " too short");
    if (p_.padding_mode == MNN_PAD_REFLECT)
      MNN_REQUIRE(pad_for(L) < L, MNN_ERR_SHAPE_MISMATCH,
                  "reflect padding " << pad_for(L) << " needs input length > padding");
    Shape o = in;
    o[o.size() - 2] = p_.out_channels;
    o.back() = lo;
    return o;
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    forward_residual(in, nullptr, out, s);
  }
  // FusedConv1D.forwardWithResidual (Conv1D.swift:857-900): out = act(conv + bias) + residual,
  // the residual added after the activation (:1016-1023). residual may be null or alias out.
  void forward_residual(const Tensor& in, const Tensor* res, Tensor& out, Stream& s) {
    const Shape os = infer_output(in.shape);
    check_out(out, os);
    if (res) {
      MNN_REQUIRE(res->count() == numel(os) && res->dtype == MNN_F32,
                  MNN_ERR_BUFFER_SIZE_MISMATCH,
                  kind() << ": residual holds " << res->count() << " elements, expected "
                         << shape_str(os));
    }
    int64_t B, C, L;
    split_bcl(in.shape, B, C, L);
    run(in.f32(), (int)B, (int)L, out.f32(), p_.activation, nullptr, s, 0,
        res ? res->f32() : nullptr);
  }
  bool uses_mfma() const {
    const int ck = p_.in_channels * p_.kernel_size;
    return p_.groups == 1 && ck % 4 == 0 && ck >= 64 && p_.out_channels >= 32;
  }
  // Implicit-GEMM arguments of the matrix-core path (one place, so the statistics partial
  // count and the launch always agree).
  const float* weight_ptr() const { return w_->ptr(); }
  const float* bias_ptr() const { return b_ ? b_->ptr() : nullptr; }
  // The small direct conv can be recomputed inside a consumer GEMM's operand loader
  // (B_CONVREC). Measured slower than storing the conv output on MI355X for the 2-channel
  // encoder level, so the encoder does not select it; kept for shapes where it pays.
  bool recompute_ok(int B, int L) const {
    (void)B;
    (void)L;
    return false;
  }
  k::GemmArgs gemm_args(const float* x, int B, int L, float* y, int act, float* stats,
                        int64_t ldy = 0, const float* res = nullptr) const {
    const int lo = (int)out_len(L);
    if (ldy == 0) ldy = lo;
    k::GemmArgs g;
    g.M = p_.out_channels;
    g.N = lo;
    g.K = p_.in_channels * p_.kernel_size;
    g.batch = B;
    g.A = w_->ptr();
    g.lda = g.K;
    g.B = x;
    g.ldb = L;
    g.sB = (int64_t)p_.in_channels * L;
    g.blayout = k::B_CONV;
    g.conv_L = L;
    g.conv_ks = p_.kernel_size;
    g.conv_stride = p_.stride;
    g.conv_pad = pad_for(L);
    g.conv_dil = p_.dilation;
    g.conv_reflect = p_.padding_mode == MNN_PAD_REFLECT;
    g.C = y;
    g.ldc = ldy;
    g.sC = (int64_t)p_.out_channels * ldy;
    g.bias = b_ ? b_->ptr() : nullptr;
    g.bias_mode = b_ ? k::BIAS_M : k::BIAS_NONE;
    g.act = act;
    g.act_alpha = alpha_;
    g.stats = stats;
    if (res) {
      g.R = res;
      g.ldr = ldy;
      g.sR = g.sC;
    }
    g.precision = p_.precision;
    return g;
  }
  k::ConvParams direct_params(int B, int L, int64_t ldy = 0, const float* res = nullptr) const {
    k::ConvParams c{B, p_.in_channels, p_.out_channels, L, (int)out_len(L), p_.kernel_size,
                    p_.stride, pad_for(L), p_.dilation, p_.groups,
                    p_.padding_mode == MNN_PAD_REFLECT, ldy};
    c.alpha = alpha_;
    c.res = res;
    return c;
  }
  // Number of GroupNorm(1) statistics partials per batch that run() writes for this input.
  int stats_chunks(int B, int L) const {
    if (uses_mfma()) return k::gemm_num_tiles(gemm_args(nullptr, B, L, nullptr, 0, nullptr));
    return k::conv1d_direct_num_chunks(direct_params(B, L));
  }
  // Runs the convolution; `stats` (GroupNorm(1) partials of the pre-activation output) is
  // optional and must hold 3 * B * stats_chunks(B, L) floats. Output rows are `ldy` apart
  // (0 = contiguous); `res` (same layout as y) is added after the activation.
  // y may be null on the direct path (statistics only).
  void run(const float* x, int B, int L, float* y, int act, float* stats, Stream& s,
           int64_t ldy = 0, const float* res = nullptr) {
    if (uses_mfma()) {
      k::gemm(ctx(s), gemm_args(x, B, L, y, act, stats, ldy, res));
      return;
    }
    k::conv1d_direct(ctx(s), direct_params(B, L, ldy, res), x, w_->ptr(),
                     b_ ? b_->ptr() : nullptr, y, act, stats, nullptr);
  }
  const mnn_conv1d_desc& desc() const { return p_; }
  // The direct register-window kernel family applies (groups 1, Cin * K <= 32, few channels).
  bool register_window(int B, int L) const {
    return !uses_mfma() && k::conv1d_direct_fusable(direct_params(B, L));
  }
  const float* weight() const { return w_->ptr(); }
  const float* bias() const { return b_ ? b_->ptr() : nullptr; }

 private:
  mnn_conv1d_desc p_;
  float alpha_ = 0.01f;
  Param* w_ = nullptr;
  Param* b_ = nullptr;
};

// ------------------------------------------------------------------ GroupNorm
// GroupNorm (Normalization.swift:32-725): population variance, eps 1e-5, per-channel affine.
class GroupNormLayer : public Layer {
 public:
  GroupNormLayer(Device* d, int groups, int channels, float eps, bool affine, int act)
      : Layer(d), G_(groups), C_(channels), eps_(eps), act_(act) {
    MNN_REQUIRE(groups > 0 && channels > 0 && channels % groups == 0,
                MNN_ERR_INVALID_CONFIGURATION,
                "numChannels (" << channels << ") must be divisible by numGroups (" << groups
                                << ")");
    if (affine) {
      gamma_ = &add_param("weight", channels, 1.f);
      beta_ = &add_param("bias", channels, 0.f);
      aliases_["gamma"] = "weight";
      aliases_["beta"] = "bias";
    }
  }
  const char* kind() const override { return "GroupNorm"; }
  Shape input_shape() const override { return {C_, 0}; }
  Shape output_shape() const override { return {C_, 0}; }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, L;
    split_bcl(in, B, C, L);
    MNN_REQUIRE(C == C_, MNN_ERR_SHAPE_MISMATCH,
                "GroupNorm: expected " << C_ << " channels, got " << C);
    return in;
  }
  // Two launches: per-chunk statistics partials, then the apply step whose workgroups merge
  // their group's partials themselves (no separate finalize pass).
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    int64_t B, C, L;
    split_bcl(in.shape, B, C, L);
    const int nchunk = k::gn_num_chunks(C_, G_, L);
    partials_.reserve(sizeof(float) * 3 * B * G_ * nchunk);
    k::gn_stats_partial(ctx(s), in.f32(), (int)B, C_, L, G_, partials_.f32(), nchunk);
    apply_parts(s, in.f32(), out.f32(), (int)B, L, partials_.f32(), nchunk, act_);
  }
  // forward() without any allocation: the partials go to the GPU's fixed scratch array.
  void forward_noalloc(const Tensor& in, Tensor& out, Stream& s) {
    check_out(out, infer_output(in.shape));
    int64_t B, C, L;
    split_bcl(in.shape, B, C, L);
    const int nchunk = k::gn_num_chunks(C_, G_, L);
    const int64_t need = 3 * B * G_ * (int64_t)nchunk;
    MNN_REQUIRE(need <= k::kGnScratchFloats, MNN_ERR_INVALID_CONFIGURATION,
                "GroupNorm without allocation: batch * groups * ceil(C / groups * L / 4096) = "
                    << need / 3 << " statistics partials exceed the scratch's "
                    << k::kGnScratchFloats / 3);
    float* parts = k::gn_scratch(dev_->ordinal);
    k::gn_stats_partial(ctx(s), in.f32(), (int)B, C_, L, G_, parts, nchunk);
    apply_parts(s, in.f32(), out.f32(), (int)B, L, parts, nchunk, act_);
  }
  // y = act(GroupNorm(x)) from statistics partials (nparts per (b, g)).
  void apply_parts(Stream& s, const float* x, float* y, int B, int64_t L, const float* parts,
                   int nparts, int act) const {
    k::gn_apply_parts(ctx(s), x, y, B, C_, L, G_, parts, nparts, gamma(), beta(), eps_, act);
  }
  float* reserve_partials(int64_t floats) {
    partials_.reserve(sizeof(float) * std::max<int64_t>(floats, 1));
    return partials_.f32();
  }
  // Exchange buffer of a one-launch chain (tags, a counter, the statistics partials), zeroed on
  // the stream when allocated; each launch leaves it ready for the next.
  void* exchange(Stream& s) {
    if (!xch_.ptr) {
      const size_t bytes = k::conv_gn_oneshot_exchange_bytes();
      xch_.reserve(bytes);
      k::zero_u32(ctx(s), xch_.as<unsigned>(), (int64_t)(bytes / 4));
    }
    return xch_.ptr;
  }
  // Turns partials into per-(b, c) coefficients held in coef().
  void finalize(Stream& s, int B, int nchunk, const float* partials) {
    coef_.reserve(sizeof(float) * 2 * B * C_);
    k::gn_finalize(ctx(s), partials, B, C_, G_, nchunk, eps_, gamma_ ? gamma_->ptr() : nullptr,
                   beta_ ? beta_->ptr() : nullptr, coef_.f32());
  }
  const float* coef() const { return coef_.f32(); }
  float* reserve_coef(int B) {
    coef_.reserve(sizeof(float) * 2 * B * C_);
    return coef_.f32();
  }
  float eps() const { return eps_; }
  const float* gamma() const { return gamma_ ? gamma_->ptr() : nullptr; }
  const float* beta() const { return beta_ ? beta_->ptr() : nullptr; }
  int groups() const { return G_; }
  int act() const { return act_; }

 private:
  int G_, C_;
  float eps_;
  int act_;
  Param* gamma_ = nullptr;
  Param* beta_ = nullptr;
  DevBuf partials_, coef_, xch_;
};

// ------------------------------------------------------------------ LayerNorm
// LayerNorm (Normalization.swift:734-964) over the last dimension.
class LayerNormLayer : public Layer {
 public:
  LayerNormLayer(Device* d, int features, float eps) : Layer(d), F_(features), eps_(eps) {
    MNN_REQUIRE(features > 0, MNN_ERR_INVALID_CONFIGURATION, "LayerNorm: featureSize <= 0");
    gamma_ = &add_param("gamma", features, 1.f);
    beta_ = &add_param("beta", features, 0.f);
    aliases_["weight"] = "gamma";
    aliases_["bias"] = "beta";
  }
  const char* kind() const override { return "LayerNorm"; }
  Shape input_shape() const override { return {F_}; }
  Shape output_shape() const override { return {F_}; }
  Shape infer_output(const Shape& in) const override {
    MNN_REQUIRE(!in.empty() && numel(in) % F_ == 0, MNN_ERR_SHAPE_MISMATCH,
                "LayerNorm: element count of " << shape_str(in) << " not a multiple of " << F_);
    return in;
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    run(in.f32(), in.count() / F_, out.f32(), s);
  }
  void run(const float* x, int64_t rows, float* y, Stream& s) {
    k::layernorm(ctx(s), x, y, rows, F_, gamma_->ptr(), beta_->ptr(), eps_);
  }
  // this LayerNorm into y and `other` (same feature size) into y2, reading x once
  void run_pair(const LayerNormLayer& other, const float* x, int64_t rows, float* y, float* y2,
                Stream& s) {
    MNN_REQUIRE(other.F_ == F_, MNN_ERR_SHAPE_MISMATCH, "LayerNorm pair: feature sizes differ");
    k::layernorm2(ctx(s), x, rows, F_, y, gamma_->ptr(), beta_->ptr(), eps_, y2,
                  other.gamma_->ptr(), other.beta_->ptr(), other.eps_);
  }
  int features() const { return F_; }
  float eps() const { return eps_; }
  const Param& gamma() const { return *gamma_; }
  const Param& beta() const { return *beta_; }

 private:
  int F_;
  float eps_;
  Param* gamma_;
  Param* beta_;
};

// ------------------------------------------------------------------ GELU
// GELU layer (Activations.swift:89-205): tanh approximation, x > 10 -> x, x < -10 -> 0.
class GELULayer : public Layer {
 public:
  GELULayer(Device* d, const Shape& s) : Layer(d), shape_(s) {}
  const char* kind() const override { return "GELU"; }
  Shape input_shape() const override { return shape_; }
  Shape output_shape() const override { return shape_; }
  Shape infer_output(const Shape& in) const override { return in; }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, in.shape);
    k::gelu(ctx(s), in.f32(), out.f32(), in.count(), true);
  }

 private:
  Shape shape_;
};

// ------------------------------------------------------------------ GLU
// glu kernel (Shaders/NN.metal:1012-1023) as a layer over the channel dimension.
class GLULayer : public Layer {
 public:
  GLULayer(Device* d, int c) : Layer(d), C_(c) {
    MNN_REQUIRE(c > 0, MNN_ERR_INVALID_CONFIGURATION, "GLU: channels <= 0");
  }
  const char* kind() const override { return "GLU"; }
  Shape input_shape() const override { return {2 * C_, 0}; }
  Shape output_shape() const override { return {C_, 0}; }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, L;
    split_bcl(in, B, C, L);
    MNN_REQUIRE(C == 2 * C_, MNN_ERR_SHAPE_MISMATCH,
                "GLU: expected " << 2 * C_ << " channels, got " << C);
    Shape o = in;
    o[o.size() - 2] = C_;
    return o;
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    int64_t B, C, L;
    split_bcl(in.shape, B, C, L);
    k::glu(ctx(s), in.f32(), out.f32(), B, (int64_t)C_ * L);
  }

 private:
  int C_;
};

// ------------------------------------------------------------------ Linear
// Linear / FusedLinear / HalfLinear (Linear.swift:27-672; HalfPrecisionLinear.swift:60-212):
// y = act(x W^T + b), W [out, in].
class LinearLayer : public Layer {
 public:
  LinearLayer(Device* d, int in, int out, bool bias, int act, mnn_precision prec,
              float leaky_alpha = 0.01f)
      : Layer(d), in_(in), out_(out), act_(act), prec_(prec), alpha_(leaky_alpha) {
    MNN_REQUIRE(in > 0 && out > 0, MNN_ERR_INVALID_CONFIGURATION, "Linear: sizes must be > 0");
    MNN_REQUIRE(std::isfinite(leaky_alpha), MNN_ERR_INVALID_CONFIGURATION,
                "FusedLinear: leakyReluAlpha must be finite");
    w_ = &add_param("weight", (int64_t)in * out);
    if (bias) b_ = &add_param("bias", out);
    if (prec == MNN_PRECISION_BF16) {  // zero weights until loaded, as the f32 parameter
      std::vector<float> z((size_t)in * out, 0.f);
      on_loaded("weight", z.data(), z.size());
    }
  }
  const char* kind() const override { return "Linear"; }
  Shape input_shape() const override { return {in_}; }
  Shape output_shape() const override { return {out_}; }
  Shape infer_output(const Shape& in) const override {
    MNN_REQUIRE(!in.empty() && in.back() == in_, MNN_ERR_SHAPE_MISMATCH,
                "Linear: expected last dimension " << in_ << ", got " << shape_str(in));
    return with_last(in, out_);
  }
  bool accepts_bf16() const override { return true; }
  // Input f32 or bf16 (HalfLinear's half-precision input, HalfPrecisionLinear.swift:60-212).
  // Precision BF16 with in_features % 64 == 0 runs the LDS-DMA GEMM on bf16 operands (an f32
  // input is rounded to bf16 first, the weights were rounded when loaded); a bf16 input under
  // precision F32 is widened to f32 (exact).
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    const int64_t rows = in.count() / in_;
    const bool lds16 = prec_ == MNN_PRECISION_BF16 && in_ % 64 == 0;
    if (in.dtype == MNN_BF16) {
      if (lds16) return run_bf16(static_cast<const uint16_t*>(in.data), rows, out.f32(), s);
      x32_.reserve(sizeof(float) * rows * in_);
      k::bf16_to_f32(ctx(s), static_cast<const uint16_t*>(in.data), x32_.f32(), rows * in_);
      return run(x32_.f32(), rows, out.f32(), act_, nullptr, nullptr, s);
    }
    if (lds16) {
      x16_.reserve(sizeof(uint16_t) * rows * in_);
      k::f32_to_bf16(ctx(s), in.f32(), static_cast<uint16_t*>(x16_.ptr), rows * in_);
      return run_bf16(static_cast<const uint16_t*>(x16_.ptr), rows, out.f32(), s);
    }
    run(in.f32(), rows, out.f32(), act_, nullptr, nullptr, s);
  }
  // bf16 operands on the LDS-DMA kernel: x [rows][in] bf16, the weights' bf16 copy.
  void run_bf16(const uint16_t* x, int64_t rows, float* y, Stream& s) {
    k::GemmArgs g;
    g.M = (int)rows;
    g.N = out_;
    g.K = in_;
    g.A = reinterpret_cast<const float*>(x);
    g.lda = in_;
    g.B = reinterpret_cast<const float*>(w16_.ptr);
    g.ldb = in_;
    g.blayout = k::B_NK;
    g.C = y;
    g.ldc = out_;
    g.bias = b_ ? b_->ptr() : nullptr;
    g.bias_mode = b_ ? k::BIAS_N : k::BIAS_NONE;
    g.act = act_;
    g.act_alpha = alpha_;
    g.precision = MNN_PRECISION_BF16;
    g.ab_bf16 = true;
    MNN_REQUIRE(k::gemm_nk_lds_supported(g), MNN_ERR_INVALID_CONFIGURATION,
                "Linear: bf16 operands outside the matrix-core kernel's contract");
    k::gemm_nk_lds(ctx(s), g);
  }
  // y = R + rscale * act(x W^T + b) when R is given (R may alias y).
  void run(const float* x, int64_t rows, float* y, int act, const float* R, const float* rscale,
           Stream& s) {
    k::GemmArgs g;
    g.M = (int)rows;
    g.N = out_;
    g.K = in_;
    g.A = x;
    g.lda = in_;
    g.B = w_->ptr();
    g.ldb = in_;
    g.blayout = k::B_NK;
    g.C = y;
    g.ldc = out_;
    g.bias = b_ ? b_->ptr() : nullptr;
    g.bias_mode = b_ ? k::BIAS_N : k::BIAS_NONE;
    g.act = act;
    g.act_alpha = alpha_;
    g.R = R;
    g.ldr = out_;
    g.rscale = rscale;
    g.precision = prec_;
    k::gemm(ctx(s), g);
  }
  int in_features() const { return in_; }
  int out_features() const { return out_; }

 protected:
  // precision BF16: keep a bf16 (round to nearest even) copy of the weights for the bf16 kernel
  void on_loaded(const std::string& name, const float* data, size_t n) override {
    if (prec_ != MNN_PRECISION_BF16 || name != "weight") return;
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = bf16_bits_rne(data[i]);
    w16_.reserve(sizeof(uint16_t) * n);
    HIP_CHECK(hipMemcpy(w16_.ptr, h.data(), n * sizeof(uint16_t), hipMemcpyHostToDevice));
  }

 private:
  static uint16_t bf16_bits_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  }
  int in_, out_, act_;
  mnn_precision prec_;
  float alpha_ = 0.01f;
  DevBuf w16_, x16_, x32_;
  Param* w_ = nullptr;
  Param* b_ = nullptr;
};

// ------------------------------------------------------------------ folded LayerNorm
// A LayerNorm whose output only feeds a linear map y = LN(x) W^T + b runs inside that map's GEMM:
// the GEMM reads the raw rows x against W * diag(gamma), and its epilogue forms
// rstd * acc - rstd * mean * c + b' (c[n] = sum_k W[n][k] gamma[k], b' = b + W beta), the rows'
// mean and rstd merged from (mean, M2) partials over 64-feature groups that the producer of x
// wrote (a residual GEMM's epilogue, or ln_row_parts). No normalised copy of x is written or read.
struct LnFold {
  const float* w = nullptr;      // W * diag(gamma), [N][K]
  const float* c = nullptr;      // [N]
  const float* b = nullptr;      // [N]
  const float* parts = nullptr;  // row partials of x, [rows][K / 64][2]
  float eps = 1e-5f;
};

// Folded weights of one (LayerNorm, linear map) pair: derived data, rebuilt on the stream of the
// call when a load has changed W, b, gamma or beta since they were built.
class LnFoldCache {
 public:
  // rows [row0, row0 + N) of W (row length K) and the same entries of b (b may be null)
  LnFold get(const LaunchCtx& c, const Param& w, int64_t row0, int N, int K, const Param* b,
             const LayerNormLayer& ln, const float* parts) {
    const uint64_t key[4] = {w.version, b ? b->version : 0, ln.gamma().version,
                             ln.beta().version};
    if (!valid_ || !std::equal(key, key + 4, key_)) {
      wf_.reserve(sizeof(float) * N * K);
      c_.reserve(sizeof(float) * N);
      b_.reserve(sizeof(float) * N);
      k::ln_fold(c, w.ptr() + row0 * K, b ? b->ptr() + row0 : nullptr, ln.gamma().ptr(),
                 ln.beta().ptr(), N, K, wf_.f32(), c_.f32(), b_.f32());
      std::copy(key, key + 4, key_);
      valid_ = true;
    }
    return LnFold{wf_.f32(), c_.f32(), b_.f32(), parts, ln.eps()};
  }

 private:
  DevBuf wf_, c_, b_;
  uint64_t key_[4] = {};
  bool valid_ = false;
};

// ------------------------------------------------------------------ MultiHeadAttention
// MultiHeadAttention / CrossAttention (Attention.swift:15-1063). Q, K, V come from one packed
// projection GEMM (self) or a Q GEMM plus a KV GEMM over rows E..3E of in_proj (cross); the
// fused attention kernel reads them in place with row strides, and the output projection can
// fuse a residual with LayerScale. The layer's precision applies to the projection GEMMs; the
// attention core (scores, softmax, P.V) always runs in fp32.
class MHALayer : public Layer {
 public:
  MHALayer(Device* d, int embed, int heads, bool bias, mnn_precision prec)
      : Layer(d), E_(embed), H_(heads), prec_(prec) {
    MNN_REQUIRE(embed > 0 && heads > 0 && embed % heads == 0, MNN_ERR_INVALID_CONFIGURATION,
                "embedDim (" << embed << ") must be divisible by numHeads (" << heads << ")");
    hd_ = embed / heads;
    win_ = &add_param("in_proj_weight", 3LL * embed * embed);
    wout_ = &add_param("out_proj_weight", (int64_t)embed * embed);
    if (bias) {
      bin_ = &add_param("in_proj_bias", 3LL * embed);
      bout_ = &add_param("out_proj_bias", embed);
    }
    // the names SafeTensorsLoader.loadAttentionWeights reads (SafeTensorsLoader.swift:335-339)
    aliases_["out_proj.weight"] = "out_proj_weight";
    aliases_["out_proj.bias"] = "out_proj_bias";
    // Default weights: identity-like Q/K/V/out projections (Attention.swift initializeDefaultWeights)
    std::vector<float> wi(3LL * embed * embed, 0.f), wo((int64_t)embed * embed, 0.f);
    for (int p = 0; p < 3; ++p)
      for (int i = 0; i < embed; ++i) wi[((int64_t)p * embed + i) * embed + i] = 1.f;
    for (int i = 0; i < embed; ++i) wo[(int64_t)i * embed + i] = 1.f;
    d->make_current();
    HIP_CHECK(hipMemcpy(win_->buf.ptr, wi.data(), wi.size() * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(wout_->buf.ptr, wo.data(), wo.size() * 4, hipMemcpyHostToDevice));
  }
  const char* kind() const override { return "MultiHeadAttention"; }
  Shape input_shape() const override { return {0, E_}; }
  Shape output_shape() const override { return {0, E_}; }
  Shape infer_output(const Shape& in) const override {
    MNN_REQUIRE((in.size() == 2 || in.size() == 3) && in.back() == E_, MNN_ERR_SHAPE_MISMATCH,
                "MultiHeadAttention: expected [S, " << E_ << "] or [B, S, " << E_ << "], got "
                                                    << shape_str(in));
    return in;
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    int64_t B, S, E;
    split_bse(in.shape, B, S, E);
    run(in.f32(), (int)S, nullptr, 0, (int)B, out.f32(), nullptr, nullptr, s);
  }
  void forward_cross(const Tensor* q, const Tensor* kv, Tensor* out, Tensor*, Stream& s) override {
    MNN_REQUIRE(q && kv && out, MNN_ERR_INVALID_ARGUMENT, "cross-attention needs query, keyValue, output");
    check_out(*out, infer_output(q->shape));
    infer_output(kv->shape);
    int64_t B, Sq, E, Bk, Sk, Ek;
    split_bse(q->shape, B, Sq, E);
    split_bse(kv->shape, Bk, Sk, Ek);
    MNN_REQUIRE(B == Bk, MNN_ERR_SHAPE_MISMATCH, "cross-attention: batch sizes differ");
    run(q->f32(), (int)Sq, kv->f32(), (int)Sk, (int)B, out->f32(), nullptr, nullptr, s);
  }
  // xkv == nullptr: self-attention. out = R + rscale * MHA(...) when R is given.
  void run(const float* xq, int Sq, const float* xkv, int Sk, int B, float* out, const float* R,
           const float* rscale, Stream& s) {
    project(xq, Sq, xkv, Sk, B, nullptr, nullptr, s);
    finish(Sq, xkv ? Sk : Sq, xkv != nullptr, B, out, R, rscale, nullptr, s);
  }
  // The Q / K / V projections (packed, or Q and KV for cross-attention). fq / fkv: LayerNorms
  // folded into them (xq / xkv are then the raw rows whose statistics the folds carry).
  void project(const float* xq, int Sq, const float* xkv, int Sk, int B, const LnFold* fq,
               const LnFold* fkv, Stream& s) {
    const int E = E_;
    const int64_t rq = (int64_t)B * Sq;
    if (!xkv) {
      qkv_.reserve(sizeof(float) * rq * 3 * E);
      proj(xq, rq, win_->ptr(), bin_ ? bin_->ptr() : nullptr, 3 * E, qkv_.f32(), fq, s);
    } else {
      project_q(xq, Sq, Sk, B, fq, s);
      project_kv(xkv, Sq, Sk, B, fkv, s);
    }
  }
  // The two halves of a cross-attention's projections (either order; same shapes for both):
  // queries from xq, keys / values from xkv.
  void project_q(const float* xq, int Sq, int Sk, int B, const LnFold* fq, Stream& s) {
    const int E = E_;
    const int64_t rq = (int64_t)B * Sq, rk = (int64_t)B * Sk;
    qkv_.reserve(sizeof(float) * (rq * E + rk * 2 * E));
    proj(xq, rq, win_->ptr(), bin_ ? bin_->ptr() : nullptr, E, qkv_.f32(), fq, s);
  }
  void project_kv(const float* xkv, int Sq, int Sk, int B, const LnFold* fkv, Stream& s) {
    const int E = E_;
    const int64_t rq = (int64_t)B * Sq, rk = (int64_t)B * Sk;
    qkv_.reserve(sizeof(float) * (rq * E + rk * 2 * E));
    proj(xkv, rk, win_->ptr() + (int64_t)E * E, bin_ ? bin_->ptr() + E : nullptr, 2 * E,
         qkv_.f32() + rq * E, fkv, s);
  }
  // Attention over the projections of the last project() call with the same shapes, then the
  // output projection (+ residual / LayerScale); row_parts receives the output rows' statistics
  // for a LayerNorm folded into the next GEMM.
  void finish(int Sq, int Sk, bool cross, int B, float* out, const float* R, const float* rscale,
              float* row_parts, Stream& s) {
    attend(Sq, Sk, cross, B, s);
    out_proj(Sq, B, out, R, rscale, row_parts, s);
  }
  void attend(int Sq, int Sk, bool cross, int B, Stream& s) {
    const int E = E_;
    const int64_t rq = (int64_t)B * Sq;
    k::AttnArgs at;
    at.B = B;
    at.H = H_;
    at.Sq = Sq;
    at.hd = hd_;
    at.scale = 1.f / std::sqrt((float)hd_);
    at.Sk = Sk;
    if (!cross) {
      at.q = qkv_.f32();
      at.q_rs = 3 * E;
      at.q_bs = (int64_t)Sq * 3 * E;
      at.k = qkv_.f32() + E;
      at.v = qkv_.f32() + 2 * E;
      at.kv_rs = 3 * E;
      at.kv_bs = (int64_t)Sq * 3 * E;
    } else {
      float* qb = qkv_.f32();
      float* kvb = qb + rq * E;
      at.q = qb;
      at.q_rs = E;
      at.q_bs = (int64_t)Sq * E;
      at.k = kvb;
      at.v = kvb + E;
      at.kv_rs = 2 * E;
      at.kv_bs = (int64_t)Sk * 2 * E;
    }
    attn_.reserve(sizeof(float) * rq * E);
    at.o = attn_.f32();
    at.o_rs = E;
    at.o_bs = (int64_t)Sq * E;
    const int ns = k::attention_key_splits(ctx(s), at);
    if (ns > 1) {
      part_.reserve(sizeof(float) * k::attention_part_floats(at, ns));
      at.nsplit = ns;
      at.part = part_.f32();
    }
    k::attention(ctx(s), at);
  }
  // output projection of the last attend() (+ residual / LayerScale)
  void out_proj(int Sq, int B, float* out, const float* R, const float* rscale, float* row_parts,
                Stream& s) {
    const int E = E_;
    const int64_t rq = (int64_t)B * Sq;
    k::GemmArgs g;
    g.M = (int)rq;
    g.N = E;
    g.K = E;
    g.A = attn_.f32();
    g.lda = E;
    g.B = wout_->ptr();
    g.ldb = E;
    g.blayout = k::B_NK;
    g.C = out;
    g.ldc = E;
    g.bias = bout_ ? bout_->ptr() : nullptr;
    g.bias_mode = bout_ ? k::BIAS_N : k::BIAS_NONE;
    g.R = R;
    g.ldr = E;
    g.rscale = rscale;
    g.row_parts = row_parts;
    g.precision = prec_;
    k::gemm(ctx(s), g);
  }
  mnn_precision precision() const { return prec_; }
  const Param& in_w() const { return *win_; }
  const Param* in_b() const { return bin_; }

 private:
  void proj(const float* x, int64_t rows, const float* w, const float* b, int nout, float* y,
            const LnFold* f, Stream& s) {
    k::GemmArgs g;
    g.M = (int)rows;
    g.N = nout;
    g.K = E_;
    g.A = x;
    g.lda = E_;
    g.B = f ? f->w : w;
    g.ldb = E_;
    g.blayout = k::B_NK;
    g.C = y;
    g.ldc = nout;
    g.bias = f ? f->b : b;
    g.bias_mode = (f || b) ? k::BIAS_N : k::BIAS_NONE;
    if (f) {
      g.ln_parts = f->parts;
      g.ln_c = f->c;
      g.ln_eps = f->eps;
    }
    g.precision = prec_;
    k::gemm(ctx(s), g);
  }

  int E_, H_, hd_;
  mnn_precision prec_;
  Param* win_ = nullptr;
  Param* wout_ = nullptr;
  Param* bin_ = nullptr;
  Param* bout_ = nullptr;
  DevBuf qkv_, attn_, part_;  // part_: key-split partial outputs
};

// ------------------------------------------------------------------ FeedForward
// FeedForward (Transformer.swift:7-364): Linear1 -> tanh-GELU -> Linear2, GELU fused into the
// first GEMM's epilogue, optional residual + LayerScale fused into the second.
class FeedForwardLayer : public Layer {
 public:
  FeedForwardLayer(Device* d, int in, int hidden, mnn_precision prec)
      : Layer(d), E_(in), Hd_(hidden), prec_(prec) {
    MNN_REQUIRE(in > 0 && hidden > 0, MNN_ERR_INVALID_CONFIGURATION, "FeedForward: sizes <= 0");
    w1_ = &add_param("linear1.weight", (int64_t)hidden * in);
    b1_ = &add_param("linear1.bias", hidden);
    w2_ = &add_param("linear2.weight", (int64_t)in * hidden);
    b2_ = &add_param("linear2.bias", in);
  }
  const char* kind() const override { return "FeedForward"; }
  Shape input_shape() const override { return {0, E_}; }
  Shape output_shape() const override { return {0, E_}; }
  Shape infer_output(const Shape& in) const override {
    MNN_REQUIRE(!in.empty() && in.back() == E_, MNN_ERR_SHAPE_MISMATCH,
                "FeedForward: expected last dimension " << E_ << ", got " << shape_str(in));
    return in;
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    run(in.f32(), in.count() / E_, out.f32(), nullptr, nullptr, s);
  }
  // f1: a LayerNorm folded into the first linear map (x are then the raw rows); row_parts: the
  // output rows' statistics for a LayerNorm folded into the next GEMM.
  void run(const float* x, int64_t rows, float* y, const float* R, const float* rscale,
           Stream& s, const LnFold* f1 = nullptr, float* row_parts = nullptr) {
    hidden_.reserve(sizeof(float) * rows * Hd_);
    k::GemmArgs g;
    g.M = (int)rows;
    g.N = Hd_;
    g.K = E_;
    g.A = x;
    g.lda = E_;
    g.B = f1 ? f1->w : w1_->ptr();
    g.ldb = E_;
    g.blayout = k::B_NK;
    g.C = hidden_.f32();
    g.ldc = Hd_;
    g.bias = f1 ? f1->b : b1_->ptr();
    g.bias_mode = k::BIAS_N;
    if (f1) {
      g.ln_parts = f1->parts;
      g.ln_c = f1->c;
      g.ln_eps = f1->eps;
    }
    g.act = MNN_ACT_GELU;
    g.precision = prec_;
    k::gemm(ctx(s), g);
    k::GemmArgs g2;
    g2.M = (int)rows;
    g2.N = E_;
    g2.K = Hd_;
    g2.A = hidden_.f32();
    g2.lda = Hd_;
    g2.B = w2_->ptr();
    g2.ldb = Hd_;
    g2.blayout = k::B_NK;
    g2.C = y;
    g2.ldc = E_;
    g2.bias = b2_->ptr();
    g2.bias_mode = k::BIAS_N;
    g2.R = R;
    g2.ldr = E_;
    g2.rscale = rscale;
    g2.row_parts = row_parts;
    g2.precision = prec_;
    k::gemm(ctx(s), g2);
  }
  mnn_precision precision() const { return prec_; }
  int hidden() const { return Hd_; }
  const Param& w1() const { return *w1_; }
  const Param& b1() const { return *b1_; }

 private:
  int E_, Hd_;
  mnn_precision prec_;
  Param *w1_, *b1_, *w2_, *b2_;
  DevBuf hidden_;
};

// ------------------------------------------------------------------ UNetEncoderBlock
// UNetEncoderBlock (UNet.swift:11-174): DynamicConv1D(reflect (k-1)/2) -> GroupNorm -> GELU,
// optionally followed by the HTDemucs rewrite 1x1 conv C -> 2C and GLU. Launch plan:
//   1. conv (+ bias) with GroupNorm partial statistics fused into its epilogue (G = 1),
//   2. statistics merge -> per-channel scale/shift,
//   3a. rewrite GEMM reading the conv output through GroupNorm+GELU, GLU in the epilogue, or
//   3b. (no rewrite) GroupNorm-apply + GELU.
class EncoderBlockLayer : public Layer {
 public:
  EncoderBlockLayer(Device* d, const mnn_encoder_block_desc& desc)
      : Layer(d), d_(desc) {
    MNN_REQUIRE(desc.in_channels > 0 && desc.out_channels > 0 && desc.kernel_size > 0 &&
                    desc.stride > 0 && desc.num_groups > 0,
                MNN_ERR_INVALID_CONFIGURATION, "UNetEncoderBlock: sizes must be positive");
    mnn_conv1d_desc cd{};
    cd.in_channels = desc.in_channels;
    cd.out_channels = desc.out_channels;
    cd.kernel_size = desc.kernel_size;
    cd.stride = desc.stride;
    cd.padding = (desc.kernel_size - 1) / 2;
    cd.dilation = 1;
    cd.groups = 1;
    cd.use_bias = 1;
    cd.input_length = 0;
    cd.padding_mode = MNN_PAD_REFLECT;
    cd.activation = MNN_ACT_NONE;
    cd.precision = desc.precision;
    conv_ = std::make_unique<Conv1DLayer>(d, cd);
    norm_ = std::make_unique<GroupNormLayer>(d, desc.num_groups, desc.out_channels, 1e-5f, true,
                                             MNN_ACT_GELU);
    const int C = desc.out_channels;
    if (desc.rewrite) {
      rw_ = &add_param("rewrite.weight", 2LL * C * C);
      rb_ = &add_param("rewrite.bias", 2LL * C);
      glu_fused_ = (C % 16 == 0);
      if (glu_fused_) {
        const int kp = k::enc_rewrite_kp(C);
        rw_perm_.reserve(sizeof(float) * 2 * C * C);
        rw_pad_.reserve(sizeof(float) * 2 * C * kp);
        rb_perm_.reserve(sizeof(float) * 2 * C);
        std::vector<float> z(std::max<int64_t>(2LL * C * kp, k::kEncL1PackFloats), 0.f);
        HIP_CHECK(hipMemcpy(rw_perm_.ptr, z.data(), 2LL * C * C * 4, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(rw_pad_.ptr, z.data(), 2LL * C * kp * 4, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(rb_perm_.ptr, z.data(), 2LL * C * 4, hipMemcpyHostToDevice));
        if (k::enc_l1_supported(desc.in_channels, C, desc.kernel_size, desc.stride, 1, 1,
                                (desc.kernel_size - 1) / 2, 8)) {
          l1_pack_.reserve(sizeof(float) * k::kEncL1PackFloats);
          HIP_CHECK(hipMemcpy(l1_pack_.ptr, z.data(), sizeof(float) * k::kEncL1PackFloats,
                              hipMemcpyHostToDevice));
        }
      }
    }
  }
  const char* kind() const override { return "UNetEncoderBlock"; }
  Shape input_shape() const override { return {d_.in_channels, 0}; }
  Shape output_shape() const override { return {d_.out_channels, 0}; }
  Shape infer_output(const Shape& in) const override { return conv_->infer_output(in); }
  void load(const std::string& name, const float* data, size_t n) override {
    if (name.rfind("conv.", 0) == 0) {
      conv_->load(name.substr(5), data, n);
      if (name == "conv.weight") pad_conv_weight(data);
      return;
    }
    if (name.rfind("norm.", 0) == 0) return norm_->load(name.substr(5), data, n);
    if (name == "rewrite.weight" || name == "rewrite.bias") {
      MNN_REQUIRE(d_.rewrite, MNN_ERR_INVALID_ARGUMENT, "block has no rewrite conv");
      return Layer::load(name, data, n);
    }
    fail(MNN_ERR_INVALID_ARGUMENT, "UNetEncoderBlock: unknown parameter '" + name + "'");
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    const Shape os = infer_output(in.shape);
    check_out(out, os);
    int64_t B, C, L;
    split_bcl(in.shape, B, C, L);
    const int Cout = d_.out_channels;
    const int64_t lo = os.back();
    const bool g1 = norm_->groups() == 1;
    if (d_.rewrite && g1 && glu_fused_ && d_.precision == MNN_PRECISION_F32 && l1_pack_.ptr &&
        k::enc_l1_supported(d_.in_channels, Cout, d_.kernel_size, d_.stride, 1, 1,
                            conv_->pad_for(L), L)) {
      // Few input channels (the first level): one launch whose workgroups exchange their
      // GroupNorm partials when the grid is resident at once, else a statistics pass and a fused
      // pass (conv recomputed with GroupNorm folded in); either way conv, GroupNorm, GELU,
      // rewrite and GLU in registers, only the output written.
      partials_.reserve(sizeof(float) * 3 * B * k::enc_l1_parts(lo));
      k::EncL1Args e;
      e.B = (int)B;
      e.Cin = d_.in_channels;
      e.C = Cout;
      e.pad = conv_->pad_for(L);
      e.L = L;
      e.Lout = lo;
      e.ldo = lo;
      e.reflect = conv_->desc().padding_mode == MNN_PAD_REFLECT;
      e.eps = norm_->eps();
      e.x = in.f32();
      e.w1 = conv_->weight_ptr();
      e.b1 = conv_->bias_ptr();
      e.gamma = norm_->gamma();
      e.beta = norm_->beta();
      e.parts = partials_.f32();
      e.a_rw = l1_pack_.f32();
      e.rb = rb_perm_.f32();
      e.out = out.f32();
      e.xch = exchange(s);
      e.spin_limit = s.dev->grid_spin_limit.load();
      k::enc_l1(ctx(s), e);
      return;
    }
    if (d_.rewrite && g1 && glu_fused_ && d_.precision == MNN_PRECISION_F32) {
      // Matrix-core path (k_enc.hip): the implicit-GEMM conv writes y and GroupNorm statistics
      // partials; the rewrite applies GroupNorm + GELU once (transposed into zt_) and runs the
      // LDS GEMM with GLU in its epilogue. A conv outside the implicit-GEMM kernel's contract
      // (kernel size other than 8 / stride 4) runs on the generic conv path.
      const auto& cd = conv_->desc();
      const int pad = conv_->pad_for(L);
      const int64_t pitch = (lo + 3) / 4 * 4;
      const int kp = k::enc_rewrite_kp(Cout);
      y_.reserve(sizeof(float) * B * Cout * pitch);
      zt_.reserve(sizeof(float) * B * lo * kp);
      k::EncRewriteArgs r;
      r.B = (int)B;
      r.C = Cout;
      r.Lout = lo;
      r.w = rw_pad_.f32();
      r.bias = rb_perm_.f32();
      r.y = y_.f32();
      r.ldy = pitch;
      r.gamma = norm_->gamma();
      r.beta = norm_->beta();
      r.eps = norm_->eps();
      r.zt = zt_.f32();
      r.kp = kp;
      r.out = out.f32();
      r.ldo = lo;
      const bool conv_ok = k::enc_conv_supported(cd.in_channels, Cout, cd.kernel_size, cd.stride,
                                                 cd.dilation, cd.groups, pad, L);
      if (conv_ok && k::enc_conv_gn_fits(ctx(s), cd.in_channels, Cout, L, lo, (int)B)) {
        // split-K conv, then one launch that sums the K parts, exchanges the GroupNorm
        // statistics between its workgroups and writes GELU(GroupNorm(y))^T: no y in HBM and no
        // separate normalisation pass
        const int K = k::enc_conv_padded_cin(cd.in_channels) * 8;
        ws_.reserve(sizeof(float) * k::enc_conv_ws_floats(Cout, lo, K, (int)B, true));
        k::EncConvArgs c;
        c.B = (int)B;
        c.Cin = cd.in_channels;
        c.Cout = Cout;
        c.L = L;
        c.Lout = lo;
        c.pad = pad;
        c.reflect = cd.padding_mode == MNN_PAD_REFLECT;
        c.x = in.f32();
        c.w = enc_conv_weight();
        c.bias = conv_->bias_ptr();
        c.ws = ws_.f32();
        c.zt = zt_.f32();
        c.gamma = norm_->gamma();
        c.beta = norm_->beta();
        c.eps = norm_->eps();
        c.xch = exchange(s);
        c.spin_limit = s.dev->grid_spin_limit.load();
        k::enc_conv(ctx(s), c);
        r.zt_ready = true;
      } else if (conv_ok) {
        const int K = k::enc_conv_padded_cin(cd.in_channels) * 8;
        const int nparts = k::enc_conv_parts(Cout, lo, K, (int)B);
        partials_.reserve(sizeof(float) * 3 * B * nparts);
        const int64_t wsf = k::enc_conv_ws_floats(Cout, lo, K, (int)B);
        if (wsf > 0) ws_.reserve(sizeof(float) * wsf);
        k::EncConvArgs c;
        c.B = (int)B;
        c.Cin = cd.in_channels;
        c.Cout = Cout;
        c.L = L;
        c.Lout = lo;
        c.pad = pad;
        c.reflect = cd.padding_mode == MNN_PAD_REFLECT;
        c.x = in.f32();
        c.w = enc_conv_weight();
        c.bias = conv_->bias_ptr();
        c.y = y_.f32();
        c.ldy = pitch;
        c.parts = partials_.f32();
        c.ws = wsf > 0 ? ws_.f32() : nullptr;
        k::enc_conv(ctx(s), c);
        r.parts = partials_.f32();
        r.nparts = nparts;
      } else {
        const int nchunk = conv_->stats_chunks((int)B, (int)L);
        partials_.reserve(sizeof(float) * 3 * B * nchunk);
        conv_->run(in.f32(), (int)B, (int)L, y_.f32(), MNN_ACT_NONE, partials_.f32(), s, pitch);
        r.parts = partials_.f32();
        r.nparts = nchunk;
      }
      k::enc_rewrite(ctx(s), r);
      return;
    }
    if (d_.rewrite && g1 && glu_fused_) {
      // Two launches: (1) conv writing GroupNorm statistics partials; (2) the rewrite GEMM,
      // whose workgroups merge the partials and read the conv output through GroupNorm + GELU,
      // GLU in the epilogue.
      const int nchunk = conv_->stats_chunks((int)B, (int)L);
      partials_.reserve(sizeof(float) * 3 * B * nchunk);
      k::GemmArgs g = rewrite_args((int)B, lo, out.f32());
      if (conv_->recompute_ok((int)B, (int)L)) {
        // small conv: statistics pass only; the GEMM recomputes the conv while loading
        conv_->run(in.f32(), (int)B, (int)L, nullptr, MNN_ACT_NONE, partials_.f32(), s, 0);
        const auto& cd = conv_->desc();
        g.blayout = k::B_CONVREC;
        g.B = in.f32();
        g.ldb = L;
        g.sB = (int64_t)cd.in_channels * L;
        g.conv_L = (int)L;
        g.conv_ks = cd.kernel_size;
        g.conv_stride = cd.stride;
        g.conv_pad = cd.padding;
        g.conv_dil = 1;
        g.conv_reflect = true;
        g.rc_w = conv_->weight_ptr();
        g.rc_b = conv_->bias_ptr();
      } else {
        // conv rows get a 16-byte pitch so the rewrite GEMM loads them as 16-byte vectors
        const int64_t pitch = (lo + 3) / 4 * 4;
        y_.reserve(sizeof(float) * B * Cout * pitch);
        conv_->run(in.f32(), (int)B, (int)L, y_.f32(), MNN_ACT_NONE, partials_.f32(), s, pitch);
        g.B = y_.f32();
        g.ldb = pitch;
        g.sB = (int64_t)Cout * pitch;
        g.blayout = k::B_KN;
      }
      g.pro_stats = partials_.f32();
      g.pro_nparts = nchunk;
      g.pro_gamma = norm_->gamma();
      g.pro_beta = norm_->beta();
      g.pro_eps = norm_->eps();
      k::gemm(ctx(s), g);
      return;
    }
    // General path (GroupNorm with several groups, no rewrite, or channel counts the fused GLU
    // epilogue does not take): conv -> statistics -> merge -> apply / GEMM (+ GLU kernel).
    y_.reserve(sizeof(float) * B * Cout * lo);
    int nchunk;
    if (g1) {
      nchunk = conv_->stats_chunks((int)B, (int)L);
      partials_.reserve(sizeof(float) * 3 * B * nchunk);
      conv_->run(in.f32(), (int)B, (int)L, y_.f32(), MNN_ACT_NONE, partials_.f32(), s);
    } else {
      conv_->run(in.f32(), (int)B, (int)L, y_.f32(), MNN_ACT_NONE, nullptr, s);
      nchunk = k::gn_num_chunks(Cout, norm_->groups(), lo);
      partials_.reserve(sizeof(float) * 3 * B * norm_->groups() * nchunk);
      k::gn_stats_partial(ctx(s), y_.f32(), (int)B, Cout, lo, norm_->groups(), partials_.f32(),
                          nchunk);
    }
    if (!d_.rewrite) {  // the apply pass merges the partials itself (no finalize launch)
      norm_->apply_parts(s, y_.f32(), out.f32(), (int)B, lo, partials_.f32(), nchunk,
                         MNN_ACT_GELU);
      return;
    }
    norm_->finalize(s, (int)B, nchunk, partials_.f32());
    k::GemmArgs g = rewrite_args((int)B, lo, out.f32());
    g.B = y_.f32();
    g.ldb = lo;
    g.sB = (int64_t)Cout * lo;
    g.blayout = k::B_KN;
    g.pro_coef = norm_->coef();
    if (glu_fused_) {
      k::gemm(ctx(s), g);
    } else {
      z_.reserve(sizeof(float) * B * 2 * Cout * lo);
      g.A = rw_->ptr();
      g.bias = rb_->ptr();
      g.glu = false;
      g.C = z_.f32();
      g.sC = 2LL * Cout * lo;
      k::gemm(ctx(s), g);
      k::glu(ctx(s), z_.f32(), out.f32(), B, (int64_t)Cout * lo);
    }
  }

 private:
  // The implicit-GEMM conv takes input channels in groups of 4: a conv with Cin % 4 != 0 (the
  // 2-channel first level) gets a copy of its weights with zero taps for the extra channels.
  void pad_conv_weight(const float* w) {
    const int cin = d_.in_channels, cip = k::enc_conv_padded_cin(cin), ks = d_.kernel_size;
    if (cip == cin || ks != 8) return;
    std::vector<float> p((size_t)d_.out_channels * cip * ks, 0.f);
    for (int co = 0; co < d_.out_channels; ++co)
      std::copy_n(w + (size_t)co * cin * ks, (size_t)cin * ks, p.data() + (size_t)co * cip * ks);
    wpad_.reserve(p.size() * sizeof(float));
    HIP_CHECK(hipMemcpy(wpad_.ptr, p.data(), p.size() * sizeof(float), hipMemcpyHostToDevice));
  }
  const float* enc_conv_weight() {
    if (k::enc_conv_padded_cin(d_.in_channels) == d_.in_channels) return conv_->weight_ptr();
    if (!wpad_.ptr) {  // weights never loaded: pad the layer's initial values
      std::vector<float> w((size_t)d_.out_channels * d_.in_channels * d_.kernel_size);
      HIP_CHECK(hipMemcpy(w.data(), conv_->weight_ptr(), w.size() * sizeof(float),
                          hipMemcpyDeviceToHost));
      pad_conv_weight(w.data());
    }
    return wpad_.f32();
  }
  // Rewrite 1x1 conv C -> 2C as a GEMM over the block's conv output (operand set by the caller).
  k::GemmArgs rewrite_args(int B, int64_t lo, float* out) const {
    const int Cout = d_.out_channels;
    k::GemmArgs g;
    g.M = 2 * Cout;
    g.N = (int)lo;
    g.K = Cout;
    g.batch = B;
    g.lda = Cout;
    g.A = glu_fused_ ? rw_perm_.f32() : rw_->ptr();
    g.bias = glu_fused_ ? rb_perm_.f32() : rb_->ptr();
    g.bias_mode = k::BIAS_M;
    g.glu = glu_fused_;
    g.pro_act = MNN_ACT_GELU;
    g.C = out;
    g.ldc = lo;
    g.sC = (int64_t)Cout * lo;
    g.precision = d_.precision;
    return g;
  }
 protected:
  // Rows of the rewrite weight are regrouped into 32-row blocks [a0..a15 | b0..b15] so the GLU
  // partner rows c and c + C meet in one accumulator block of the GEMM.
  void on_loaded(const std::string& name, const float* data, size_t n) override {
    if (!glu_fused_) return;
    const int C = d_.out_channels;
    if (name == "rewrite.weight") {
      std::vector<float> p(n);
      for (int blk = 0; blk < C / 16; ++blk)
        for (int j = 0; j < 16; ++j) {
          std::copy_n(data + (int64_t)(16 * blk + j) * C, C, p.data() + (int64_t)(32 * blk + j) * C);
          std::copy_n(data + (int64_t)(C + 16 * blk + j) * C, C,
                      p.data() + (int64_t)(32 * blk + 16 + j) * C);
        }
      HIP_CHECK(hipMemcpy(rw_perm_.ptr, p.data(), n * 4, hipMemcpyHostToDevice));
      // the same rows with the operand depth padded to a multiple of 32 (zero columns)
      const int kp = k::enc_rewrite_kp(C);
      std::vector<float> q(2LL * C * kp, 0.f);
      for (int r = 0; r < 2 * C; ++r)
        std::copy_n(p.data() + (int64_t)r * C, C, q.data() + (int64_t)r * kp);
      HIP_CHECK(hipMemcpy(rw_pad_.ptr, q.data(), q.size() * 4, hipMemcpyHostToDevice));
      if (l1_pack_.ptr) {  // the fused first-level kernel's register order
        std::vector<float> pk(k::kEncL1PackFloats);
        k::enc_l1_pack_rewrite(p.data(), pk.data());
        HIP_CHECK(hipMemcpy(l1_pack_.ptr, pk.data(), pk.size() * 4, hipMemcpyHostToDevice));
      }
    } else if (name == "rewrite.bias") {
      std::vector<float> p(n);
      for (int blk = 0; blk < C / 16; ++blk)
        for (int j = 0; j < 16; ++j) {
          p[32 * blk + j] = data[16 * blk + j];
          p[32 * blk + 16 + j] = data[C + 16 * blk + j];
        }
      HIP_CHECK(hipMemcpy(rb_perm_.ptr, p.data(), n * 4, hipMemcpyHostToDevice));
    }
  }

 private:
  mnn_encoder_block_desc d_;
  std::unique_ptr<Conv1DLayer> conv_;
  std::unique_ptr<GroupNormLayer> norm_;
  Param* rw_ = nullptr;
  Param* rb_ = nullptr;
  bool glu_fused_ = false;
  DevBuf rw_perm_, rb_perm_, rw_pad_, l1_pack_;
  DevBuf y_, partials_, z_, wpad_, ws_, zt_, xch_;
  // Exchange buffer of the one-launch GroupNorm forms (the first level, the split-K finish),
  // zeroed on the stream when allocated; its words carry per-launch epoch tags, so launches leave
  // nothing to clear. Forwards of one block that overlap (two streams) would share it, as they
  // share the workspaces.
  void* exchange(Stream& s) {
    if (!xch_.ptr) {
      const size_t bytes = k::enc_exchange_bytes();
      xch_.reserve(bytes);
      k::zero_u32(ctx(s), xch_.as<unsigned>(), (int64_t)(bytes / 4));
    }
    return xch_.ptr;
  }
};

// ------------------------------------------------------------------ ConvTranspose1D
// DynamicConvTranspose1D (DynamicConv1D.swift:411-645): weight [in, out/groups, k], bias [out];
// output length (L - 1) * stride - 2 * padding + dilation * (k - 1) + output_padding + 1
// (DynamicConv1D.swift:483-487). Groups 1, dilation 1 and k a multiple of the stride (1, 2 or 4
// taps per phase) run as a GEMM on the matrix cores (k_convt.hip: operand unfold + LDS GEMM with a
// scatter epilogue; the weights are repacked for it when loaded), except k 8 / stride 4 with at
// most 4 output channels, which runs a register kernel (a 64-row matrix tile would be mostly
// padding); every other configuration runs the reference's gather loop as one thread per output.
class ConvTranspose1DLayer : public Layer {
 public:
  ConvTranspose1DLayer(Device* d, const mnn_conv_transpose1d_desc& desc) : Layer(d), d_(desc) {
    MNN_REQUIRE(desc.in_channels > 0 && desc.out_channels > 0 && desc.kernel_size > 0 &&
                    desc.stride > 0 && desc.dilation > 0 && desc.groups > 0 &&
                    desc.padding >= 0 && desc.output_padding >= 0 &&
                    desc.in_channels % desc.groups == 0 && desc.out_channels % desc.groups == 0,
                MNN_ERR_INVALID_CONFIGURATION, "ConvTranspose1D: invalid configuration");
    w_ = &add_param("weight", (int64_t)desc.in_channels * (desc.out_channels / desc.groups) *
                                  desc.kernel_size);
    if (desc.use_bias) b_ = &add_param("bias", desc.out_channels);
    small_ = k::convt_small_supported(desc.in_channels, desc.out_channels, desc.kernel_size,
                                      desc.stride, desc.dilation, desc.groups);
    gemm_ = !small_ && k::convt_gemm_supported(desc.in_channels, desc.out_channels,
                                               desc.kernel_size, desc.stride, desc.dilation,
                                               desc.groups);
    if (gemm_) {
      std::vector<float> zero((size_t)w_->count, 0.f);
      pack(zero.data());
    }
  }
  const char* kind() const override { return "ConvTranspose1D"; }
  Shape input_shape() const override { return {d_.in_channels, 0}; }
  Shape output_shape() const override { return {d_.out_channels, 0}; }
  int64_t out_len(int64_t L) const {
    return (L - 1) * d_.stride - 2LL * d_.padding + (int64_t)d_.dilation * (d_.kernel_size - 1) +
           d_.output_padding + 1;
  }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, L;
    split_bcl(in, B, C, L);
    MNN_REQUIRE(C == d_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                "ConvTranspose1D: expected " << d_.in_channels << " channels, got " << C);
    MNN_REQUIRE(L > 0 && out_len(L) > 0, MNN_ERR_SHAPE_MISMATCH,
                "ConvTranspose1D: input length " << L << " gives no output");
    Shape o = in;
    o[o.size() - 2] = d_.out_channels;
    o.back() = out_len(L);
    return o;
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    int64_t B, C, L;
    split_bcl(in.shape, B, C, L);
    run(in.f32(), (int)C, nullptr, 0, (int)B, L, out.f32(), s);
  }
  // GroupNorm(1) statistics partials per batch that run() writes into `stats` (count, mean, M2
  // each, gn_apply_parts' layout for one group); 0 when this layer's path does not produce them.
  int stats_parts(int B, int64_t L, int G) const {
    if (!small_ && !gemm_) return 0;
    k::ConvTArgs a = args(d_.in_channels, 0, B, L);
    a.stat_groups = G;
    return k::convt_stats_parts(a);
  }
  // y [B][out][out_len(L)] from the channel concat [x1 (C1 channels); x2 (C2)], C1 + C2 = in;
  // with stats (stats_parts(B, L, G) > 0 only), the GroupNorm partials of y for G groups as well.
  void run(const float* x1, int C1, const float* x2, int C2, int B, int64_t L, float* y,
           Stream& s, float* stats = nullptr, int G = 1) {
    MNN_REQUIRE(C1 + C2 == d_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                "ConvTranspose1D: channel count mismatch");
    MNN_REQUIRE(!stats || stats_parts(B, L, G) > 0, MNN_ERR_INVALID_ARGUMENT,
                "ConvTranspose1D: this configuration writes no statistics partials");
    k::ConvTArgs a = args(C1, C2, B, L);
    a.x1 = x1;
    a.x2 = x2;
    a.w = w_->ptr();
    a.bias = b_ ? b_->ptr() : nullptr;
    a.y = y;
    a.stats = stats;
    a.stat_groups = G;
    if (small_) {
      k::convt_small(ctx(s), a);
    } else if (gemm_) {
      unfold_.reserve(sizeof(float) * k::convt_unfold_floats(B, d_.in_channels, d_.kernel_size,
                                                              d_.stride, d_.padding, a.Lout));
      const int64_t wsf = k::convt_split_ws_floats(B, d_.in_channels, d_.out_channels,
                                                   d_.kernel_size, d_.stride, d_.padding, a.Lout);
      if (wsf > 0) split_.reserve(sizeof(float) * wsf);
      k::convt_gemm(ctx(s), a, wpack_.f32(), unfold_.f32(), wsf > 0 ? split_.f32() : nullptr);
    } else {
      k::convt_direct(ctx(s), a);
    }
  }
  const mnn_conv_transpose1d_desc& desc() const { return d_; }

 protected:
  void on_loaded(const std::string& name, const float* data, size_t) override {
    if (name == "weight" && gemm_) pack(data);
  }

 private:
  k::ConvTArgs args(int C1, int C2, int B, int64_t L) const {
    k::ConvTArgs a;
    a.B = B;
    a.C1 = C1;
    a.C2 = C2;
    a.Cout = d_.out_channels;
    a.K = d_.kernel_size;
    a.stride = d_.stride;
    a.pad = d_.padding;
    a.dil = d_.dilation;
    a.groups = d_.groups;
    a.L = L;
    a.Lout = out_len(L);
    return a;
  }
  void pack(const float* w) {
    const int T = d_.kernel_size / d_.stride, Cp = k::convt_padded_cin(d_.in_channels);
    std::vector<float> h((size_t)d_.stride * d_.out_channels * T * Cp);
    k::convt_pack_weights(w, d_.in_channels, d_.out_channels, d_.kernel_size, d_.stride, h.data());
    dev_->make_current();
    wpack_.reserve(sizeof(float) * h.size());
    HIP_CHECK(hipMemcpy(wpack_.ptr, h.data(), sizeof(float) * h.size(), hipMemcpyHostToDevice));
  }
  mnn_conv_transpose1d_desc d_;
  Param* w_ = nullptr;
  Param* b_ = nullptr;
  bool small_ = false, gemm_ = false;
  DevBuf wpack_, unfold_, split_;
};

// ------------------------------------------------------------------ UNetDecoderBlock
// UNetDecoderBlock (UNet.swift:184-388): concat(input, skip) over channels -> ConvTranspose1D with
// padding (k - 1) / 2 and output_padding stride - 2 + k % 2 (UNet.swift:229-241; output length
// stride * L for even k) -> GroupNorm -> tanh-GELU. The concat is folded into the transposed
// conv's operand unfold, so no concatenated tensor is written (the reference copies both inputs
// through the CPU, UNet.swift:303-331). Two inputs: mnn_layer_forward_cross(input, skip, out).
class DecoderBlockLayer : public Layer {
 public:
  DecoderBlockLayer(Device* d, const mnn_decoder_block_desc& desc) : Layer(d), d_(desc) {
    MNN_REQUIRE(desc.in_channels > 0 && desc.skip_channels >= 0 && desc.out_channels > 0 &&
                    desc.kernel_size > 0 && desc.stride > 0 && desc.num_groups > 0,
                MNN_ERR_INVALID_CONFIGURATION, "UNetDecoderBlock: invalid configuration");
    mnn_conv_transpose1d_desc c{};
    c.in_channels = desc.in_channels + desc.skip_channels;
    c.out_channels = desc.out_channels;
    c.kernel_size = desc.kernel_size;
    c.stride = desc.stride;
    c.padding = (desc.kernel_size - 1) / 2;
    c.output_padding = desc.stride - 2 + desc.kernel_size % 2;
    c.dilation = 1;
    c.groups = 1;
    c.use_bias = 1;
    MNN_REQUIRE(c.output_padding >= 0, MNN_ERR_INVALID_CONFIGURATION,
                "UNetDecoderBlock: stride " << desc.stride << " gives a negative output padding");
    convt_ = std::make_unique<ConvTranspose1DLayer>(d, c);
    norm_ = std::make_unique<GroupNormLayer>(d, desc.num_groups, desc.out_channels, 1e-5f, true,
                                             MNN_ACT_GELU);
  }
  const char* kind() const override { return "UNetDecoderBlock"; }
  Shape input_shape() const override { return {d_.in_channels, 0}; }
  Shape output_shape() const override { return {d_.out_channels, 0}; }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, L;
    split_bcl(in, B, C, L);
    MNN_REQUIRE(C == d_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                "UNetDecoderBlock: expected " << d_.in_channels << " channels, got " << C);
    Shape o = in;
    o[o.size() - 2] = d_.out_channels;
    o.back() = convt_->out_len(L);
    return o;
  }
  void load(const std::string& name, const float* data, size_t n) override {
    if (name.rfind("conv_tr.", 0) == 0) return convt_->load(name.substr(8), data, n);
    if (name.rfind("conv_transpose.", 0) == 0) return convt_->load(name.substr(15), data, n);
    if (name.rfind("norm.", 0) == 0) return norm_->load(name.substr(5), data, n);
    fail(MNN_ERR_INVALID_ARGUMENT, "UNetDecoderBlock: unknown parameter '" + name + "'");
  }
  void forward(const Tensor&, Tensor&, Stream&) override {
    fail(MNN_ERR_INVALID_CONFIGURATION,
         "UNetDecoderBlock: forward takes (input, skip); use the two-input forward");
  }
  void forward_cross(const Tensor* in, const Tensor* skip, Tensor* out, Tensor*,
                     Stream& s) override {
    MNN_REQUIRE(in && skip && out, MNN_ERR_INVALID_ARGUMENT,
                "UNetDecoderBlock: input, skip and output are required");
    int64_t B, C, L, Bs, Cs, Ls;
    split_bcl(in->shape, B, C, L);
    split_bcl(skip->shape, Bs, Cs, Ls);
    MNN_REQUIRE(C == d_.in_channels && Cs == d_.skip_channels && Bs == B && Ls == L,
                MNN_ERR_SHAPE_MISMATCH,
                "UNetDecoderBlock: input " << shape_str(in->shape) << " and skip "
                                           << shape_str(skip->shape) << " do not match ["
                                           << d_.in_channels << "|" << d_.skip_channels
                                           << ", L]");
    const Shape os = infer_output(in->shape);
    check_out(*out, os);
    const int Cout = d_.out_channels;
    const int64_t lo = os.back();
    y_.reserve(sizeof(float) * B * Cout * lo);
    const int G = norm_->groups();
    if (const int np = convt_->stats_parts((int)B, L, G)) {
      // GroupNorm statistics from the transposed conv itself (GEMM epilogue, split-K reduce or
      // the few-channel kernel); the apply pass merges them (no statistics pass over y)
      partials_.reserve(sizeof(float) * 3 * B * G * np);
      convt_->run(in->f32(), (int)C, skip->f32(), (int)Cs, (int)B, L, y_.f32(), s,
                  partials_.f32(), G);
      norm_->apply_parts(s, y_.f32(), out->f32(), (int)B, lo, partials_.f32(), np,
                         MNN_ACT_GELU);
      return;
    }
    convt_->run(in->f32(), (int)C, skip->f32(), (int)Cs, (int)B, L, y_.f32(), s);
    const int nchunk = k::gn_num_chunks(Cout, G, lo);
    partials_.reserve(sizeof(float) * 3 * B * G * nchunk);
    k::gn_stats_partial(ctx(s), y_.f32(), (int)B, Cout, lo, G, partials_.f32(), nchunk);
    // the apply pass merges the partials itself (no finalize launch)
    norm_->apply_parts(s, y_.f32(), out->f32(), (int)B, lo, partials_.f32(), nchunk,
                       MNN_ACT_GELU);
  }

 private:
  mnn_decoder_block_desc d_;
  std::unique_ptr<ConvTranspose1DLayer> convt_;
  std::unique_ptr<GroupNormLayer> norm_;
  DevBuf y_, partials_;
};

// ------------------------------------------------------------------ 2-D convolutions
namespace {

// [C, H, W] / [B, C, H, W] -> (B, C, H, W)
void split_bchw(const Shape& s, int64_t& B, int64_t& C, int64_t& H, int64_t& W) {
  MNN_REQUIRE(s.size() == 3 || s.size() == 4, MNN_ERR_SHAPE_MISMATCH,
              "expected [C, H, W] or [B, C, H, W], got " << shape_str(s));
  B = s.size() == 4 ? s[0] : 1;
  C = s[s.size() - 3];
  H = s[s.size() - 2];
  W = s[s.size() - 1];
}

Shape with_chw(const Shape& in, int64_t C, int64_t H, int64_t W) {
  Shape o = in;
  o[o.size() - 3] = C;
  o[o.size() - 2] = H;
  o[o.size() - 1] = W;
  return o;
}

}  // namespace

// DynamicConv2D (DynamicConv2D.swift:37-592): valid / same / explicit / reflect padding, stride,
// dilation, groups. Output size floor((n + 2p - ((k-1)d + 1)) / s) + 1 (outputSize, :193-205),
// "same" padding total/2 on both sides for ceil(n / s) outputs (computePadding, :212-238).
class Conv2DLayer : public Layer {
 public:
  Conv2DLayer(Device* d, const mnn_conv2d_desc& desc) : Layer(d), d_(desc) {
    MNN_REQUIRE(desc.in_channels > 0 && desc.out_channels > 0 && desc.kernel_h > 0 &&
                    desc.kernel_w > 0 && desc.stride_h > 0 && desc.stride_w > 0 &&
                    desc.dilation_h > 0 && desc.dilation_w > 0 && desc.groups > 0 &&
                    desc.in_channels % desc.groups == 0 && desc.out_channels % desc.groups == 0 &&
                    desc.padding_mode >= MNN_PAD_VALID && desc.padding_mode <= MNN_PAD_REFLECT &&
                    desc.pad_h >= 0 && desc.pad_w >= 0,
                MNN_ERR_INVALID_CONFIGURATION, "Conv2D: invalid configuration");
    const int cpg = desc.in_channels / desc.groups;
    w_ = &add_param("weight",
                    (int64_t)desc.out_channels * cpg * desc.kernel_h * desc.kernel_w);
    if (desc.use_bias) b_ = &add_param("bias", desc.out_channels);
    gemm_ = desc.groups == 1;
    if (gemm_) {
      std::vector<float> zero((size_t)w_->count, 0.f);
      pack(zero.data());
    }
  }
  const char* kind() const override { return "Conv2D"; }
  Shape input_shape() const override { return {d_.in_channels, 0, 0}; }
  Shape output_shape() const override { return {d_.out_channels, 0, 0}; }
  std::pair<int, int> padding(int64_t H, int64_t W) const {
    switch (d_.padding_mode) {
      case MNN_PAD_VALID: return {0, 0};
      case MNN_PAD_SAME: {
        const int64_t ekh = (int64_t)(d_.kernel_h - 1) * d_.dilation_h + 1;
        const int64_t ekw = (int64_t)(d_.kernel_w - 1) * d_.dilation_w + 1;
        const int64_t oh = (H + d_.stride_h - 1) / d_.stride_h;
        const int64_t ow = (W + d_.stride_w - 1) / d_.stride_w;
        return {(int)(std::max<int64_t>(0, (oh - 1) * d_.stride_h + ekh - H) / 2),
                (int)(std::max<int64_t>(0, (ow - 1) * d_.stride_w + ekw - W) / 2)};
      }
      default: return {d_.pad_h, d_.pad_w};
    }
  }
  std::pair<int64_t, int64_t> out_size(int64_t H, int64_t W) const {
    const auto p = padding(H, W);
    const int64_t nh = H + 2LL * p.first - ((int64_t)(d_.kernel_h - 1) * d_.dilation_h + 1);
    const int64_t nw = W + 2LL * p.second - ((int64_t)(d_.kernel_w - 1) * d_.dilation_w + 1);
    if (nh < 0 || nw < 0) return {0, 0};
    return {nh / d_.stride_h + 1, nw / d_.stride_w + 1};
  }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, H, W;
    split_bchw(in, B, C, H, W);
    MNN_REQUIRE(C == d_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                "Conv2D: expected " << d_.in_channels << " channels, got " << C);
    const auto o = out_size(H, W);
    MNN_REQUIRE(H > 0 && W > 0 && o.first > 0 && o.second > 0, MNN_ERR_SHAPE_MISMATCH,
                "Conv2D: input " << H << "x" << W << " gives no output");
    return with_chw(in, d_.out_channels, o.first, o.second);
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    int64_t B, C, H, W;
    split_bchw(in.shape, B, C, H, W);
    run(in.f32(), (int)B, H, W, out.f32(), s);
  }
  // GroupNorm partials per (batch, group) that run() writes for G groups (0: this configuration
  // does not produce them; the caller runs a statistics pass).
  int stats_parts(int B, int64_t H, int64_t W, int G) const {
    k::Conv2DArgs a = args(nullptr, B, H, W, nullptr);
    if (k::conv2d_small_supported(a)) return k::conv2d_small_parts(a, G);
    if (!gemm_) return 0;
    a.stat_groups = G;
    return k::conv2d_gemm_stats_parts(a);
  }
  void run(const float* x, int B, int64_t H, int64_t W, float* y, Stream& s,
           float* stats = nullptr, int G = 0) {
    MNN_REQUIRE(H < (1 << 30) && W < (1 << 30), MNN_ERR_SHAPE_MISMATCH, "Conv2D: input too large");
    k::Conv2DArgs a = args(x, B, H, W, y);
    MNN_REQUIRE(!stats || stats_parts(B, H, W, G) > 0, MNN_ERR_INVALID_ARGUMENT,
                "Conv2D: this configuration writes no GroupNorm partials");
    if (k::conv2d_small_supported(a)) {
      k::conv2d_small(ctx(s), a, stats, G);
    } else if (gemm_) {
      a.stats = stats;
      a.stat_groups = G;
      const int64_t uf = k::conv2d_unfold_floats(a);
      if (uf > 0) unfold_.reserve(sizeof(float) * uf);
      const int64_t wf = k::conv2d_split_ws_floats(a);
      if (wf > 0) split_.reserve(sizeof(float) * wf);
      k::conv2d_gemm(ctx(s), a, wpack_.f32(), uf > 0 ? unfold_.f32() : nullptr,
                     wf > 0 ? split_.f32() : nullptr);
    } else {
      k::conv2d_direct(ctx(s), a);
    }
  }

 private:
  k::Conv2DArgs args(const float* x, int B, int64_t H, int64_t W, float* y) const {
    const auto o = out_size(H, W);
    const auto p = padding(H, W);
    k::Conv2DArgs a;
    a.B = B;
    a.Cin = d_.in_channels;
    a.Cout = d_.out_channels;
    a.H = (int)H;
    a.W = (int)W;
    a.Ho = (int)o.first;
    a.Wo = (int)o.second;
    a.KH = d_.kernel_h;
    a.KW = d_.kernel_w;
    a.sh = d_.stride_h;
    a.sw = d_.stride_w;
    a.ph = p.first;
    a.pw = p.second;
    a.dh = d_.dilation_h;
    a.dw = d_.dilation_w;
    a.groups = d_.groups;
    a.reflect = d_.padding_mode == MNN_PAD_REFLECT;
    a.x = x;
    a.w = w_->ptr();
    a.bias = b_ ? b_->ptr() : nullptr;
    a.y = y;
    return a;
  }

 protected:
  void on_loaded(const std::string& name, const float* data, size_t) override {
    if (name == "weight" && gemm_) pack(data);
  }

 private:
  void pack(const float* w) {
    const int Kp = k::conv2d_padded_k(d_.in_channels, d_.kernel_h, d_.kernel_w);
    std::vector<float> h((size_t)d_.out_channels * Kp);
    k::conv2d_pack_weights(w, d_.out_channels, d_.in_channels, d_.kernel_h, d_.kernel_w,
                           h.data());
    dev_->make_current();
    wpack_.reserve(sizeof(float) * h.size());
    HIP_CHECK(hipMemcpy(wpack_.ptr, h.data(), sizeof(float) * h.size(), hipMemcpyHostToDevice));
  }
  mnn_conv2d_desc d_;
  Param* w_ = nullptr;
  Param* b_ = nullptr;
  bool gemm_ = false;
  DevBuf wpack_, unfold_, split_;
};

// DynamicConvTranspose2D (DynamicConv2D.swift:598-959): output (n - 1)s - 2p + (k - 1)d + 1 + op
// per axis (outputSize, :727-736).
class ConvTranspose2DLayer : public Layer {
 public:
  ConvTranspose2DLayer(Device* d, const mnn_conv_transpose2d_desc& desc) : Layer(d), d_(desc) {
    MNN_REQUIRE(desc.in_channels > 0 && desc.out_channels > 0 && desc.kernel_h > 0 &&
                    desc.kernel_w > 0 && desc.stride_h > 0 && desc.stride_w > 0 &&
                    desc.dilation_h > 0 && desc.dilation_w > 0 && desc.groups > 0 &&
                    desc.pad_h >= 0 && desc.pad_w >= 0 && desc.output_pad_h >= 0 &&
                    desc.output_pad_w >= 0 && desc.in_channels % desc.groups == 0 &&
                    desc.out_channels % desc.groups == 0,
                MNN_ERR_INVALID_CONFIGURATION, "ConvTranspose2D: invalid configuration");
    w_ = &add_param("weight", (int64_t)desc.in_channels * (desc.out_channels / desc.groups) *
                                  desc.kernel_h * desc.kernel_w);
    if (desc.use_bias) b_ = &add_param("bias", desc.out_channels);
    gemm_ = desc.groups == 1;
    if (gemm_) {
      std::vector<float> zero((size_t)w_->count, 0.f);
      pack(zero.data());
    }
  }
  const char* kind() const override { return "ConvTranspose2D"; }
  Shape input_shape() const override { return {d_.in_channels, 0, 0}; }
  Shape output_shape() const override { return {d_.out_channels, 0, 0}; }
  std::pair<int64_t, int64_t> out_size(int64_t H, int64_t W) const {
    return {(H - 1) * d_.stride_h - 2LL * d_.pad_h + (int64_t)d_.dilation_h * (d_.kernel_h - 1) +
                d_.output_pad_h + 1,
            (W - 1) * d_.stride_w - 2LL * d_.pad_w + (int64_t)d_.dilation_w * (d_.kernel_w - 1) +
                d_.output_pad_w + 1};
  }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, H, W;
    split_bchw(in, B, C, H, W);
    MNN_REQUIRE(C == d_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                "ConvTranspose2D: expected " << d_.in_channels << " channels, got " << C);
    const auto o = out_size(H, W);
    MNN_REQUIRE(H > 0 && W > 0 && o.first > 0 && o.second > 0, MNN_ERR_SHAPE_MISMATCH,
                "ConvTranspose2D: input " << H << "x" << W << " gives no output");
    return with_chw(in, d_.out_channels, o.first, o.second);
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    int64_t B, C, H, W;
    split_bchw(in.shape, B, C, H, W);
    run(in.f32(), (int)C, nullptr, 0, (int)B, H, W, out.f32(), s);
  }
  // GroupNorm partials per (batch, group) that run() writes with stats for G groups (the
  // few-channel kernel or the matrix-core form's gather, gn_apply_parts' layout); 0 where it
  // writes none.
  int stats_parts(int B, int64_t H, int64_t W, int G) const {
    if (H >= (1 << 30) || W >= (1 << 30)) return 0;
    k::ConvT2DArgs a = args(nullptr, d_.in_channels, nullptr, 0, B, H, W, nullptr);
    a.stat_groups = G;
    if (!k::convt2d_small_supported(a) && !gemm_) return 0;
    return k::convt2d_stats_parts(a);
  }
  // y from the channel concat [x1 (C1); x2 (C2)], C1 + C2 = in_channels; with stats
  // (stats_parts(B, H, W, G) > 0 only), the GroupNorm partials of y for G groups as well.
  void run(const float* x1, int C1, const float* x2, int C2, int B, int64_t H, int64_t W,
           float* y, Stream& s, float* stats = nullptr, int G = 1) {
    MNN_REQUIRE(C1 + C2 == d_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                "ConvTranspose2D: channel count mismatch");
    MNN_REQUIRE(H < (1 << 30) && W < (1 << 30), MNN_ERR_SHAPE_MISMATCH,
                "ConvTranspose2D: input too large");
    MNN_REQUIRE(!stats || stats_parts(B, H, W, G) > 0, MNN_ERR_INVALID_ARGUMENT,
                "ConvTranspose2D: GroupNorm partials outside the matrix-core form");
    k::ConvT2DArgs a = args(x1, C1, x2, C2, B, H, W, y);
    a.stats = stats;
    a.stat_groups = G;
    if (k::convt2d_small_supported(a)) {
      k::convt2d_small(ctx(s), a);
    } else if (gemm_) {
      z_.reserve(sizeof(float) * k::convt2d_z_floats(a));
      unfold_.reserve(sizeof(float) * k::convt2d_unfold_floats(a));
      k::convt2d_gemm(ctx(s), a, wpack_.f32(), z_.f32(), unfold_.f32());
    } else {
      k::convt2d_direct(ctx(s), a);
    }
  }

 protected:
  void on_loaded(const std::string& name, const float* data, size_t) override {
    if (name == "weight" && gemm_) pack(data);
  }

 private:
  k::ConvT2DArgs args(const float* x1, int C1, const float* x2, int C2, int B, int64_t H,
                      int64_t W, float* y) const {
    const auto o = out_size(H, W);
    k::ConvT2DArgs a;
    a.B = B;
    a.C1 = C1;
    a.C2 = C2;
    a.Cout = d_.out_channels;
    a.H = (int)H;
    a.W = (int)W;
    a.Ho = (int)o.first;
    a.Wo = (int)o.second;
    a.KH = d_.kernel_h;
    a.KW = d_.kernel_w;
    a.sh = d_.stride_h;
    a.sw = d_.stride_w;
    a.ph = d_.pad_h;
    a.pw = d_.pad_w;
    a.dh = d_.dilation_h;
    a.dw = d_.dilation_w;
    a.groups = d_.groups;
    a.x1 = x1;
    a.x2 = x2;
    a.w = w_->ptr();
    a.bias = b_ ? b_->ptr() : nullptr;
    a.y = y;
    return a;
  }
  void pack(const float* w) {
    const int Cp = k::convt2d_padded_cin(d_.in_channels);
    std::vector<float> h((size_t)d_.out_channels * d_.kernel_h * d_.kernel_w * Cp);
    k::convt2d_pack_weights(w, d_.in_channels, d_.out_channels, d_.kernel_h, d_.kernel_w,
                            h.data());
    dev_->make_current();
    wpack_.reserve(sizeof(float) * h.size());
    HIP_CHECK(hipMemcpy(wpack_.ptr, h.data(), sizeof(float) * h.size(), hipMemcpyHostToDevice));
  }
  mnn_conv_transpose2d_desc d_;
  Param* w_ = nullptr;
  Param* b_ = nullptr;
  bool gemm_ = false;
  DevBuf wpack_, z_, unfold_;
};

// FreqUNetEncoderBlock2D (FreqUNet2D.swift:12-192): Conv2D (reflect padding ((k-1)/2 per axis),
// stride) -> GroupNorm over [C, H*W] -> tanh-GELU. Parameters "conv.weight", "conv.bias",
// "norm.weight", "norm.bias".
class FreqEncoderBlockLayer : public Layer {
 public:
  FreqEncoderBlockLayer(Device* d, const mnn_freq_block_desc& desc) : Layer(d), d_(desc) {
    MNN_REQUIRE(desc.in_channels > 0 && desc.out_channels > 0 && desc.kernel_h > 0 &&
                    desc.kernel_w > 0 && desc.stride_h > 0 && desc.stride_w > 0 &&
                    desc.num_groups > 0 && desc.skip_channels == 0,
                MNN_ERR_INVALID_CONFIGURATION, "FreqUNetEncoderBlock2D: invalid configuration");
    mnn_conv2d_desc c{};
    c.in_channels = desc.in_channels;
    c.out_channels = desc.out_channels;
    c.kernel_h = desc.kernel_h;
    c.kernel_w = desc.kernel_w;
    c.stride_h = desc.stride_h;
    c.stride_w = desc.stride_w;
    c.padding_mode = MNN_PAD_REFLECT;
    c.pad_h = (desc.kernel_h - 1) / 2;
    c.pad_w = (desc.kernel_w - 1) / 2;
    c.dilation_h = c.dilation_w = 1;
    c.groups = 1;
    c.use_bias = 1;
    conv_ = std::make_unique<Conv2DLayer>(d, c);
    norm_ = std::make_unique<GroupNormLayer>(d, desc.num_groups, desc.out_channels, 1e-5f, true,
                                             MNN_ACT_GELU);
  }
  const char* kind() const override { return "FreqUNetEncoderBlock2D"; }
  Shape input_shape() const override { return {d_.in_channels, 0, 0}; }
  Shape output_shape() const override { return {d_.out_channels, 0, 0}; }
  Shape infer_output(const Shape& in) const override { return conv_->infer_output(in); }
  void load(const std::string& name, const float* data, size_t n) override {
    if (name.rfind("conv.", 0) == 0) return conv_->load(name.substr(5), data, n);
    if (name.rfind("norm.", 0) == 0) return norm_->load(name.substr(5), data, n);
    fail(MNN_ERR_INVALID_ARGUMENT, "FreqUNetEncoderBlock2D: unknown parameter '" + name + "'");
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    const Shape os = infer_output(in.shape);
    check_out(out, os);
    int64_t B, C, H, W;
    split_bchw(in.shape, B, C, H, W);
    const int Cout = d_.out_channels;
    const int64_t L = os[os.size() - 2] * os.back();
    y_.reserve(sizeof(float) * B * Cout * L);
    const int G = norm_->groups();
    if (const int np = conv_->stats_parts((int)B, H, W, G)) {
      // the direct conv (few input channels) or the implicit GEMM's split-K reduce writes the
      // GroupNorm partials (no statistics pass)
      partials_.reserve(sizeof(float) * 3 * B * G * np);
      conv_->run(in.f32(), (int)B, H, W, y_.f32(), s, partials_.f32(), G);
      norm_->apply_parts(s, y_.f32(), out.f32(), (int)B, L, partials_.f32(), np, MNN_ACT_GELU);
      return;
    }
    conv_->run(in.f32(), (int)B, H, W, y_.f32(), s);
    gn_gelu(norm_.get(), partials_, y_.f32(), out.f32(), (int)B, Cout, L, s);
  }

  static void gn_gelu(GroupNormLayer* norm, DevBuf& partials, const float* y, float* out, int B,
                      int C, int64_t L, Stream& s) {
    const int G = norm->groups();
    const int nchunk = k::gn_num_chunks(C, G, L);
    partials.reserve(sizeof(float) * 3 * B * G * nchunk);
    k::gn_stats_partial(ctx(s), y, B, C, L, G, partials.f32(), nchunk);
    // the apply pass merges the partials itself (no finalize launch)
    norm->apply_parts(s, y, out, B, L, partials.f32(), nchunk, MNN_ACT_GELU);
  }

 private:
  mnn_freq_block_desc d_;
  std::unique_ptr<Conv2DLayer> conv_;
  std::unique_ptr<GroupNormLayer> norm_;
  DevBuf y_, partials_;
};

// FreqUNetDecoderBlock2D (FreqUNet2D.swift:198-428): concat(input, skip) over channels ->
// ConvTranspose2D (padding (k-1)/2, output padding stride-1 per axis) -> GroupNorm -> tanh-GELU.
// The concat is folded into the transposed conv's operand pack, so no concatenated tensor is
// written. Parameters "conv_tr.*" (or "conv_transpose.*") and "norm.*".
class FreqDecoderBlockLayer : public Layer {
 public:
  FreqDecoderBlockLayer(Device* d, const mnn_freq_block_desc& desc) : Layer(d), d_(desc) {
    MNN_REQUIRE(desc.in_channels > 0 && desc.skip_channels >= 0 && desc.out_channels > 0 &&
                    desc.kernel_h > 0 && desc.kernel_w > 0 && desc.stride_h > 0 &&
                    desc.stride_w > 0 && desc.num_groups > 0,
                MNN_ERR_INVALID_CONFIGURATION, "FreqUNetDecoderBlock2D: invalid configuration");
    mnn_conv_transpose2d_desc c{};
    c.in_channels = desc.in_channels + desc.skip_channels;
    c.out_channels = desc.out_channels;
    c.kernel_h = desc.kernel_h;
    c.kernel_w = desc.kernel_w;
    c.stride_h = desc.stride_h;
    c.stride_w = desc.stride_w;
    c.pad_h = (desc.kernel_h - 1) / 2;
    c.pad_w = (desc.kernel_w - 1) / 2;
    c.output_pad_h = desc.stride_h - 1;
    c.output_pad_w = desc.stride_w - 1;
    c.dilation_h = c.dilation_w = 1;
    c.groups = 1;
    c.use_bias = 1;
    convt_ = std::make_unique<ConvTranspose2DLayer>(d, c);
    norm_ = std::make_unique<GroupNormLayer>(d, desc.num_groups, desc.out_channels, 1e-5f, true,
                                             MNN_ACT_GELU);
  }
  const char* kind() const override { return "FreqUNetDecoderBlock2D"; }
  Shape input_shape() const override { return {d_.in_channels, 0, 0}; }
  Shape output_shape() const override { return {d_.out_channels, 0, 0}; }
  Shape infer_output(const Shape& in) const override {
    int64_t B, C, H, W;
    split_bchw(in, B, C, H, W);
    MNN_REQUIRE(C == d_.in_channels, MNN_ERR_SHAPE_MISMATCH,
                "FreqUNetDecoderBlock2D: expected " << d_.in_channels << " channels, got " << C);
    const auto o = convt_->out_size(H, W);
    MNN_REQUIRE(H > 0 && W > 0 && o.first > 0 && o.second > 0, MNN_ERR_SHAPE_MISMATCH,
                "FreqUNetDecoderBlock2D: input gives no output");
    return with_chw(in, d_.out_channels, o.first, o.second);
  }
  void load(const std::string& name, const float* data, size_t n) override {
    if (name.rfind("conv_tr.", 0) == 0) return convt_->load(name.substr(8), data, n);
    if (name.rfind("conv_transpose.", 0) == 0) return convt_->load(name.substr(15), data, n);
    if (name.rfind("norm.", 0) == 0) return norm_->load(name.substr(5), data, n);
    fail(MNN_ERR_INVALID_ARGUMENT, "FreqUNetDecoderBlock2D: unknown parameter '" + name + "'");
  }
  void forward(const Tensor&, Tensor&, Stream&) override {
    fail(MNN_ERR_INVALID_CONFIGURATION,
         "FreqUNetDecoderBlock2D: forward takes (input, skip); use the two-input forward");
  }
  void forward_cross(const Tensor* in, const Tensor* skip, Tensor* out, Tensor*,
                     Stream& s) override {
    MNN_REQUIRE(in && skip && out, MNN_ERR_INVALID_ARGUMENT,
                "FreqUNetDecoderBlock2D: input, skip and output are required");
    int64_t B, C, H, W, Bs, Cs, Hs, Ws;
    split_bchw(in->shape, B, C, H, W);
    split_bchw(skip->shape, Bs, Cs, Hs, Ws);
    MNN_REQUIRE(C == d_.in_channels && Cs == d_.skip_channels && Bs == B && Hs == H && Ws == W,
                MNN_ERR_SHAPE_MISMATCH,
                "FreqUNetDecoderBlock2D: input " << shape_str(in->shape) << " and skip "
                                                 << shape_str(skip->shape) << " do not match");
    const Shape os = infer_output(in->shape);
    check_out(*out, os);
    const int Cout = d_.out_channels;
    const int64_t L = os[os.size() - 2] * os.back();
    y_.reserve(sizeof(float) * B * Cout * L);
    const int G = norm_->groups();
    if (const int np = convt_->stats_parts((int)B, H, W, G)) {
      // the transposed conv (its few-channel kernel or its gather) writes the GroupNorm partials
      // (no statistics pass over y)
      partials_.reserve(sizeof(float) * 3 * B * G * np);
      convt_->run(in->f32(), (int)C, skip->f32(), (int)Cs, (int)B, H, W, y_.f32(), s,
                  partials_.f32(), G);
      norm_->apply_parts(s, y_.f32(), out->f32(), (int)B, L, partials_.f32(), np, MNN_ACT_GELU);
      return;
    }
    convt_->run(in->f32(), (int)C, skip->f32(), (int)Cs, (int)B, H, W, y_.f32(), s);
    FreqEncoderBlockLayer::gn_gelu(norm_.get(), partials_, y_.f32(), out->f32(), (int)B, Cout, L,
                                   s);
  }

 private:
  mnn_freq_block_desc d_;
  std::unique_ptr<ConvTranspose2DLayer> convt_;
  std::unique_ptr<GroupNormLayer> norm_;
  DevBuf y_, partials_;
};

// ------------------------------------------------------------------ transformer building blocks
namespace {

// One pre-norm branch of a transformer layer. Self: x += g1*MHA(LN1 x); x += g2*FFN(LN2 x).
// Cross: x += g1*MHA(LN1 x, LN2 other); x += g2*FFN(LN3 x). LayerScale g = layer_scale * 1
// unless loaded; layer_scale <= 0 disables it.
struct Branch {
  std::unique_ptr<LayerNormLayer> norm1, norm2, norm3;
  std::unique_ptr<MHALayer> attn;
  std::unique_ptr<FeedForwardLayer> ffn;
  std::unique_ptr<LinearLayer> dummy;
  bool cross = false;
  bool use_ls = false;
  DevBuf g1, g2;
  int E = 0;
  // folded weights: attention input projection (packed QKV, or Q for cross layers), the cross
  // layer's KV projection, the FFN's first linear map
  LnFoldCache fold_in, fold_kv, fold_ffn;

  Branch(Device* d, int embed, int heads, int ffn_dim, bool is_cross, float ls,
         mnn_precision prec)
      : cross(is_cross), E(embed) {
    norm1 = std::make_unique<LayerNormLayer>(d, embed, 1e-5f);
    norm2 = std::make_unique<LayerNormLayer>(d, embed, 1e-5f);
    if (is_cross) norm3 = std::make_unique<LayerNormLayer>(d, embed, 1e-5f);
    attn = std::make_unique<MHALayer>(d, embed, heads, true, prec);
    ffn = std::make_unique<FeedForwardLayer>(d, embed, ffn_dim, prec);
    use_ls = ls > 0.f;
    if (use_ls) {
      std::vector<float> v(embed, ls);
      g1.reserve(embed * 4);
      g2.reserve(embed * 4);
      HIP_CHECK(hipMemcpy(g1.ptr, v.data(), embed * 4, hipMemcpyHostToDevice));
      HIP_CHECK(hipMemcpy(g2.ptr, v.data(), embed * 4, hipMemcpyHostToDevice));
    }
  }
  LayerNormLayer* ffn_norm() { return cross ? norm3.get() : norm2.get(); }
  // LayerNorms foldable into the GEMMs after them: fp32, whole 64-feature groups (at most 8),
  // FFN width a multiple of the GEMM's k step
  bool foldable() const {
    return attn->precision() == MNN_PRECISION_F32 && ffn->precision() == MNN_PRECISION_F32 &&
           E % 64 == 0 && E <= 512 && ffn->hidden() % 32 == 0;
  }
  // returns true if the name was consumed
  bool load(const std::string& name, const float* data, size_t n) {
    auto starts = [&](const char* p) { return name.rfind(p, 0) == 0; };
    if (starts("norm1.")) return norm1->load(name.substr(6), data, n), true;
    if (starts("norm2.")) return norm2->load(name.substr(6), data, n), true;
    if (starts("norm3.")) {
      MNN_REQUIRE(cross, MNN_ERR_INVALID_ARGUMENT, "norm3 exists only in cross layers");
      return norm3->load(name.substr(6), data, n), true;
    }
    if (starts("attn.") || starts("self_attn.") || starts("cross_attn.")) {
      const size_t dot = name.find('.');
      return attn->load(name.substr(dot + 1), data, n), true;
    }
    if (starts("linear1.") || starts("linear2.")) return ffn->load(name, data, n), true;
    if (name == "gamma_1.scale" || name == "gamma_2.scale") {
      MNN_REQUIRE(use_ls, MNN_ERR_INVALID_ARGUMENT, "LayerScale disabled for this layer");
      MNN_REQUIRE((int)n == E, MNN_ERR_BUFFER_SIZE_MISMATCH, name << ": expected " << E);
      for (size_t i = 0; i < n; ++i)
        MNN_REQUIRE(std::isfinite(data[i]), MNN_ERR_INVALID_CONFIGURATION, name << " not finite");
      HIP_CHECK(hipMemcpy((name[6] == '1' ? g1 : g2).ptr, data, n * 4, hipMemcpyHostToDevice));
      return true;
    }
    return false;
  }
  const float* ls1() const { return use_ls ? g1.f32() : nullptr; }
  const float* ls2() const { return use_ls ? g2.f32() : nullptr; }
};

}  // namespace

// Single-sequence pre-norm transformer layer (config: MHSA + FFN).
class TransformerLayerImpl : public Layer {
 public:
  TransformerLayerImpl(Device* d, int embed, int heads, int ffn, float ls, mnn_precision prec)
      : Layer(d), E_(embed), br_(d, embed, heads, ffn, false, ls, prec) {}
  const char* kind() const override { return "TransformerLayer"; }
  Shape input_shape() const override { return {0, E_}; }
  Shape output_shape() const override { return {0, E_}; }
  Shape infer_output(const Shape& in) const override {
    MNN_REQUIRE((in.size() == 2 || in.size() == 3) && in.back() == E_, MNN_ERR_SHAPE_MISMATCH,
                "TransformerLayer: expected [S, " << E_ << "] or [B, S, " << E_ << "]");
    return in;
  }
  void load(const std::string& name, const float* data, size_t n) override {
    MNN_REQUIRE(br_.load(name, data, n), MNN_ERR_INVALID_ARGUMENT,
                "TransformerLayer: unknown parameter '" << name << "'");
  }
  void forward(const Tensor& in, Tensor& out, Stream& s) override {
    check_out(out, infer_output(in.shape));
    int64_t B, S, E;
    split_bse(in.shape, B, S, E);
    const int64_t rows = B * S;
    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (br_.foldable() && a16(in.data) && a16(out.data) &&
        rows * std::max<int64_t>(3 * E, br_.ffn->hidden()) * 4 < ((int64_t)1 << 32)) {
      // both LayerNorms folded into the GEMMs after them: row statistics of the input from
      // ln_row_parts, of the attention block's output from the out-projection's epilogue (the
      // QKV GEMM has read the first set by then, so one buffer holds both in turn)
      parts_.reserve(sizeof(float) * rows * (E / 64) * 2);
      float* P = parts_.f32();
      k::ln_row_parts(ctx(s), in.f32(), nullptr, rows, (int)E, P);
      const LnFold fq = br_.fold_in.get(ctx(s), br_.attn->in_w(), 0, 3 * (int)E, (int)E,
                                        br_.attn->in_b(), *br_.norm1, P);
      br_.attn->project(in.f32(), (int)S, nullptr, 0, (int)B, &fq, nullptr, s);
      br_.attn->finish((int)S, (int)S, false, (int)B, out.f32(), in.f32(), br_.ls1(), P, s);
      const LnFold f1 = br_.fold_ffn.get(ctx(s), br_.ffn->w1(), 0, br_.ffn->hidden(), (int)E,
                                         &br_.ffn->b1(), *br_.norm2, P);
      br_.ffn->run(out.f32(), rows, out.f32(), out.f32(), br_.ls2(), s, &f1);
      return;
    }
    h_.reserve(sizeof(float) * rows * E);
    br_.norm1->run(in.f32(), rows, h_.f32(), s);
    br_.attn->run(h_.f32(), (int)S, nullptr, 0, (int)B, out.f32(), in.f32(), br_.ls1(), s);
    br_.norm2->run(out.f32(), rows, h_.f32(), s);
    br_.ffn->run(h_.f32(), rows, out.f32(), out.f32(), br_.ls2(), s);
  }

 private:
  int E_;
  Branch br_;
  DevBuf h_, parts_;
};

// Cross-domain transformer bottleneck (CrossTransformerEncoder, Transformer.swift:567-700) with
// the HTDemucs layer structure: even layers self-attention per branch, odd layers cross-attention
// in which both branches attend to the other branch's state from before this layer.
class CrossTransformerImpl : public Layer {
 public:
  CrossTransformerImpl(Device* d, int embed, int heads, int ffn, int layers, float ls,
                       mnn_precision prec)
      : Layer(d), E_(embed) {
    MNN_REQUIRE(layers > 0, MNN_ERR_INVALID_CONFIGURATION, "CrossTransformer: num_layers <= 0");
    for (int i = 0; i < layers; ++i) {
      const bool cross = (i % 2) == 1;
      time_.push_back(std::make_unique<Branch>(d, embed, heads, ffn, cross, ls, prec));
      freq_.push_back(std::make_unique<Branch>(d, embed, heads, ffn, cross, ls, prec));
    }
  }
  const char* kind() const override { return "CrossTransformerEncoder"; }
  Shape input_shape() const override { return {0, E_}; }
  Shape output_shape() const override { return {0, E_}; }
  Shape infer_output(const Shape& in) const override {
    MNN_REQUIRE((in.size() == 2 || in.size() == 3) && in.back() == E_, MNN_ERR_SHAPE_MISMATCH,
                "CrossTransformerEncoder: expected [S, " << E_ << "] or [B, S, " << E_ << "]");
    return in;
  }
  void load(const std::string& name, const float* data, size_t n) override {
    // layers.{i}.{time|freq}.rest
    MNN_REQUIRE(name.rfind("layers.", 0) == 0, MNN_ERR_INVALID_ARGUMENT,
                "CrossTransformerEncoder: unknown parameter '" << name << "'");
    const size_t p1 = name.find('.', 7);
    MNN_REQUIRE(p1 != std::string::npos, MNN_ERR_INVALID_ARGUMENT, "bad parameter name " << name);
    const int li = std::atoi(name.substr(7, p1 - 7).c_str());
    MNN_REQUIRE(li >= 0 && li < (int)time_.size(), MNN_ERR_INVALID_ARGUMENT,
                "layer index out of range in " << name);
    const size_t p2 = name.find('.', p1 + 1);
    MNN_REQUIRE(p2 != std::string::npos, MNN_ERR_INVALID_ARGUMENT, "bad parameter name " << name);
    const std::string br = name.substr(p1 + 1, p2 - p1 - 1);
    MNN_REQUIRE(br == "time" || br == "freq", MNN_ERR_INVALID_ARGUMENT,
                "branch must be time or freq in " << name);
    Branch& b = br == "time" ? *time_[li] : *freq_[li];
    MNN_REQUIRE(b.load(name.substr(p2 + 1), data, n), MNN_ERR_INVALID_ARGUMENT,
                "CrossTransformerEncoder: unknown parameter '" << name << "'");
  }
  void forward(const Tensor&, Tensor&, Stream&) override {
    fail(MNN_ERR_INVALID_CONFIGURATION,
         "CrossTransformerEncoder needs two inputs: use forward_cross(time, freq, ...)");
  }
  // The time and freq branches only meet at the cross-attention exchange, so they run on two
  // streams: freq on the caller's stream, time on a side stream forked from it, joined back at the
  // end. Kernels of one branch then fill the CUs the other branch's grid leaves idle. A cross layer
  // starts with a two-way sync (the exchange buffers of the previous cross layer are free again),
  // and each attention waits for the other branch's normalised state (with the LayerNorms folded
  // into the GEMMs: for the other branch's projections of this branch's state). With kernel timing
  // on, everything runs on the caller's stream so launch durations are not stretched by overlap.
  void forward_cross(const Tensor* t, const Tensor* f, Tensor* to, Tensor* fo,
                     Stream& s) override {
    MNN_REQUIRE(t && f && to && fo, MNN_ERR_INVALID_ARGUMENT,
                "CrossTransformerEncoder: time, freq, time_out and freq_out are required");
    check_out(*to, infer_output(t->shape));
    check_out(*fo, infer_output(f->shape));
    int64_t B, St, E, Bf, Sf, Ef;
    split_bse(t->shape, B, St, E);
    split_bse(f->shape, Bf, Sf, Ef);
    MNN_REQUIRE(B == Bf, MNN_ERR_SHAPE_MISMATCH, "time and freq batch sizes differ");
    const int64_t rt = B * St, rf = B * Sf;
    const bool two = !dev_->timing;
    next_event_ = 0;
    Stream side{s.dev, s.s, false};
    if (two) {
      side.s = side_stream();
      link(s, side);
    }
    Stream& ts = side;  // time branch
    Stream& fs = s;     // freq branch
    if (fold_ok(rt, rf, t->data, f->data, to->data, fo->data)) {
      run_folded(t, f, to, fo, B, St, Sf, ts, fs, two);
      if (two) link(ts, s);
      return;
    }
    ht_.reserve(sizeof(float) * rt * E * 2);
    hf_.reserve(sizeof(float) * rf * E * 2);
    if (to->data != t->data) k::copy_bytes(ctx(ts), t->data, to->data, rt * E * 4);
    if (fo->data != f->data) k::copy_bytes(ctx(fs), f->data, fo->data, rf * E * 4);
    float* T = to->f32();
    float* F = fo->f32();
    float* ht = ht_.f32();
    float* ht2 = ht + rt * E;
    float* hf = hf_.f32();
    float* hf2 = hf + rf * E;
    for (size_t i = 0; i < time_.size(); ++i) {
      Branch& bt = *time_[i];
      Branch& bf = *freq_[i];
      if (!bt.cross) {
        bt.norm1->run(T, rt, ht, ts);
        bt.attn->run(ht, (int)St, nullptr, 0, (int)B, T, T, bt.ls1(), ts);
        bt.norm2->run(T, rt, ht, ts);
        bt.ffn->run(ht, rt, T, T, bt.ls2(), ts);
        bf.norm1->run(F, rf, hf, fs);
        bf.attn->run(hf, (int)Sf, nullptr, 0, (int)B, F, F, bf.ls1(), fs);
        bf.norm2->run(F, rf, hf, fs);
        bf.ffn->run(hf, rf, F, F, bf.ls2(), fs);
      } else {
        if (two) {
          link(ts, fs);
          link(fs, ts);
        }
        // all four normalisations read the states from before this layer; the two of each
        // state in one pass: time queries and time as freq's keys/values, freq queries and freq
        // as time's keys/values
        bt.norm1->run_pair(*bf.norm2, T, rt, ht, ht2, ts);
        bf.norm1->run_pair(*bt.norm2, F, rf, hf, hf2, fs);
        if (two) {
          link(fs, ts);  // hf2 ready
          link(ts, fs);  // ht2 ready
        }
        bt.attn->run(ht, (int)St, hf2, (int)Sf, (int)B, T, T, bt.ls1(), ts);
        bf.attn->run(hf, (int)Sf, ht2, (int)St, (int)B, F, F, bf.ls1(), fs);
        bt.ffn_norm()->run(T, rt, ht, ts);
        bt.ffn->run(ht, rt, T, T, bt.ls2(), ts);
        bf.ffn_norm()->run(F, rf, hf, fs);
        bf.ffn->run(hf, rf, F, F, bf.ls2(), fs);
      }
    }
    if (two) link(ts, s);
  }
  ~CrossTransformerImpl() override {
    if (side_) (void)hipStreamDestroy(side_);
    for (hipEvent_t e : events_) (void)hipEventDestroy(e);
  }

 private:
  static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
  // Every LayerNorm folded into the GEMM after it: fp32 branches, 64-feature groups, rows the
  // LDS-DMA GEMM addresses with 32-bit offsets, 16-byte aligned states.
  bool fold_ok(int64_t rt, int64_t rf, const void* t, const void* f, const void* to,
               const void* fo) const {
    if (!aligned16(t) || !aligned16(f) || !aligned16(to) || !aligned16(fo)) return false;
    int64_t widest = 3LL * E_;
    for (const auto* v : {&time_, &freq_})
      for (const auto& b : *v) {
        if (!b->foldable()) return false;
        widest = std::max<int64_t>(widest, b->ffn->hidden());
      }
    return std::max(rt, rf) * widest * 4 < ((int64_t)1 << 32);
  }
  // The layer loop with every LayerNorm folded into its consumer GEMM. Row statistics of the two
  // states (64-feature partials) come from ln_row_parts for the inputs (which also copies them to
  // the outputs) and from the residual GEMMs' epilogues after that. In a cross layer both
  // branches first project their queries and the other state's keys / values (reading both
  // states and both statistics buffers), and only after a two-way sync do the output projections
  // overwrite them.
  void run_folded(const Tensor* t, const Tensor* f, Tensor* to, Tensor* fo, int64_t B, int64_t St,
                  int64_t Sf, Stream& ts, Stream& fs, bool two) {
    const int E = E_;
    const int64_t rt = B * St, rf = B * Sf;
    pt_.reserve(sizeof(float) * rt * (E / 64) * 2);
    pf_.reserve(sizeof(float) * rf * (E / 64) * 2);
    float* T = to->f32();
    float* F = fo->f32();
    float* PT = pt_.f32();
    float* PF = pf_.f32();
    k::ln_row_parts(ctx(ts), t->f32(), to->data != t->data ? T : nullptr, rt, E, PT);
    k::ln_row_parts(ctx(fs), f->f32(), fo->data != f->data ? F : nullptr, rf, E, PF);
    for (size_t i = 0; i < time_.size(); ++i) {
      Branch& bt = *time_[i];
      Branch& bf = *freq_[i];
      const bool last = i + 1 == time_.size();  // no LayerNorm reads the final states
      if (!bt.cross) {
        for (int side = 0; side < 2; ++side) {
          Branch& b = side ? bf : bt;
          Stream& st = side ? fs : ts;
          float* X = side ? F : T;
          float* P = side ? PF : PT;
          const int64_t S = side ? Sf : St, rows = side ? rf : rt;
          const LnFold fq = b.fold_in.get(ctx(st), b.attn->in_w(), 0, 3 * E, E, b.attn->in_b(),
                                          *b.norm1, P);
          b.attn->project(X, (int)S, nullptr, 0, (int)B, &fq, nullptr, st);
          b.attn->finish((int)S, (int)S, false, (int)B, X, X, b.ls1(), P, st);
          const LnFold f1 = b.fold_ffn.get(ctx(st), b.ffn->w1(), 0, b.ffn->hidden(), E,
                                           &b.ffn->b1(), *b.norm2, P);
          b.ffn->run(X, rows, X, X, b.ls2(), st, &f1, last ? nullptr : P);
        }
      } else {
        if (two) {
          link(ts, fs);
          link(fs, ts);
        }
        for (int side = 0; side < 2; ++side) {
          Branch& b = side ? bf : bt;
          Stream& st = side ? fs : ts;
          const LnFold fq = b.fold_in.get(ctx(st), b.attn->in_w(), 0, E, E, b.attn->in_b(),
                                          *b.norm1, side ? PF : PT);
          const LnFold fkv = b.fold_kv.get(ctx(st), b.attn->in_w(), E, 2 * E, E,
                                           b.attn->in_b(), *b.norm2, side ? PT : PF);
          // queries: this branch's cross norm of its own state; keys / values: this branch's
          // second norm of the other state
          b.attn->project(side ? F : T, (int)(side ? Sf : St), side ? T : F,
                          (int)(side ? St : Sf), (int)B, &fq, &fkv, st);
        }
        if (two) {
          link(fs, ts);  // freq has read T and PT
          link(ts, fs);  // time has read F and PF
        }
        for (int side = 0; side < 2; ++side) {
          Branch& b = side ? bf : bt;
          Stream& st = side ? fs : ts;
          float* X = side ? F : T;
          float* P = side ? PF : PT;
          const int64_t S = side ? Sf : St, Sy = side ? St : Sf, rows = side ? rf : rt;
          b.attn->finish((int)S, (int)Sy, true, (int)B, X, X, b.ls1(), P, st);
          const LnFold f1 = b.fold_ffn.get(ctx(st), b.ffn->w1(), 0, b.ffn->hidden(), E,
                                           &b.ffn->b1(), *b.ffn_norm(), P);
          b.ffn->run(X, rows, X, X, b.ls2(), st, &f1, last ? nullptr : P);
        }
      }
    }
  }

  hipStream_t side_stream() {
    if (!side_) {
      dev_->make_current();
      HIP_CHECK(hipStreamCreateWithFlags(&side_, hipStreamNonBlocking));
    }
    return side_;
  }
  // `to` waits for the work queued so far on `from`. Each link of a forward has its own event
  // (next_event_ restarts at every forward), so no event is recorded twice within one forward.
  void link(Stream& from, Stream& to) { HIP_CHECK(hipStreamWaitEvent(to.s, mark(from), 0)); }
  // an event recorded after the work queued so far on `from` (one per call within a forward)
  hipEvent_t mark(Stream& from) {
    if (next_event_ == events_.size()) {
      hipEvent_t e;
      HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
      events_.push_back(e);
    }
    hipEvent_t e = events_[next_event_++];
    HIP_CHECK(hipEventRecord(e, from.s));
    return e;
  }

  int E_;
  std::vector<std::unique_ptr<Branch>> time_, freq_;
  DevBuf ht_, hf_, pt_, pf_;
  hipStream_t side_ = nullptr;
  std::vector<hipEvent_t> events_;
  size_t next_event_ = 0;
};

// ------------------------------------------------------------------ CrossTransformerEncoder
// CrossTransformerEncoder with the reference class's own layer structure (TransformerLayer,
// Transformer.swift:370-560; the encoder's layer loop :626-667). Per layer, in this order:
//   T += SA_t(LN_ts(T))       (:467-470)
//   F += SA_f(LN_fs(F))
//   tn = LN_tc(T); fn = LN_fc(F)
//   T += CA_t(tn, fn)         time queries, freq keys / values
//   F += CA_f(fn, tn)         freq queries; tn is the time state from before the line above
//   T += FFN_t(LN_tf(T)); F += FFN_f(LN_ff(F))
// One residual per sub-block (:467-495), no LayerScale: every residual goes through the GEMM
// epilogue of the sub-block's last linear map (out-projection, FFN second linear) as
// C = R + (acc + bias). Weight names follow
// TransformerLayer.loadWeights (:529-557): layers.{i}.{norm_time_self, norm_freq_self,
// norm_time_cross, norm_freq_cross, norm_time_ffn, norm_freq_ffn}.{weight,bias},
// layers.{i}.{self_attn_time, self_attn_freq, cross_attn_time, cross_attn_freq}.{in_proj_weight,
// in_proj_bias, out_proj.weight, out_proj.bias}, layers.{i}.{ffn_time, ffn_freq}.{linear1,
// linear2}.{weight,bias}. Batched inputs [B, S, E] run every batch element (the reference sizes its
// work buffers for one).
class CrossTransformerEncoderImpl : public Layer {
 public:
  CrossTransformerEncoderImpl(Device* d, int embed, int heads, int ffn, int layers,
                              mnn_precision prec)
      : Layer(d), E_(embed) {
    MNN_REQUIRE(layers > 0, MNN_ERR_INVALID_CONFIGURATION,
                "CrossTransformerEncoder: num_layers <= 0");
    for (int i = 0; i < layers; ++i) {
      auto L = std::make_unique<Lyr>();
      for (auto* n : {&L->nts, &L->nfs, &L->ntc, &L->nfc, &L->ntf, &L->nff})
        *n = std::make_unique<LayerNormLayer>(d, embed, 1e-5f);
      for (auto* a : {&L->sat, &L->saf, &L->cat, &L->caf})
        *a = std::make_unique<MHALayer>(d, embed, heads, true, prec);
      L->fft = std::make_unique<FeedForwardLayer>(d, embed, ffn, prec);
      L->fff = std::make_unique<FeedForwardLayer>(d, embed, ffn, prec);
      layers_.push_back(std::move(L));
    }
  }
  const char* kind() const override { return "CrossTransformerEncoder"; }
  Shape input_shape() const override { return {0, E_}; }
  Shape output_shape() const override { return {0, E_}; }
  Shape infer_output(const Shape& in) const override {
    MNN_REQUIRE((in.size() == 2 || in.size() == 3) && in.back() == E_, MNN_ERR_SHAPE_MISMATCH,
                "CrossTransformerEncoder: expected [S, " << E_ << "] or [B, S, " << E_ << "]");
    return in;
  }
  void load(const std::string& name, const float* data, size_t n) override {
    MNN_REQUIRE(name.rfind("layers.", 0) == 0, MNN_ERR_INVALID_ARGUMENT,
                "CrossTransformerEncoder: unknown parameter '" << name << "'");
    const size_t p1 = name.find('.', 7);
    MNN_REQUIRE(p1 != std::string::npos, MNN_ERR_INVALID_ARGUMENT, "bad parameter name " << name);
    const int li = std::atoi(name.substr(7, p1 - 7).c_str());
    MNN_REQUIRE(li >= 0 && li < (int)layers_.size(), MNN_ERR_INVALID_ARGUMENT,
                "layer index out of range in " << name);
    const std::string rest = name.substr(p1 + 1);
    const size_t dot = rest.find('.');
    MNN_REQUIRE(dot != std::string::npos, MNN_ERR_INVALID_ARGUMENT, "bad parameter name " << name);
    const std::string part = rest.substr(0, dot), tail = rest.substr(dot + 1);
    Lyr& L = *layers_[li];
    const std::map<std::string, Layer*> parts = {
        {"norm_time_self", L.nts.get()},  {"norm_freq_self", L.nfs.get()},
        {"norm_time_cross", L.ntc.get()}, {"norm_freq_cross", L.nfc.get()},
        {"norm_time_ffn", L.ntf.get()},   {"norm_freq_ffn", L.nff.get()},
        {"self_attn_time", L.sat.get()},  {"self_attn_freq", L.saf.get()},
        {"cross_attn_time", L.cat.get()}, {"cross_attn_freq", L.caf.get()},
        {"ffn_time", L.fft.get()},        {"ffn_freq", L.fff.get()}};
    const auto it = parts.find(part);
    MNN_REQUIRE(it != parts.end(), MNN_ERR_INVALID_ARGUMENT,
                "CrossTransformerEncoder: unknown parameter '" << name << "'");
    it->second->load(tail, data, n);
  }
  void forward(const Tensor&, Tensor&, Stream&) override {
    fail(MNN_ERR_INVALID_CONFIGURATION,
         "CrossTransformerEncoder needs two inputs: use forward_cross(time, freq, ...)");
  }
  void forward_cross(const Tensor* t, const Tensor* f, Tensor* to, Tensor* fo,
                     Stream& s) override {
    MNN_REQUIRE(t && f && to && fo, MNN_ERR_INVALID_ARGUMENT,
                "CrossTransformerEncoder: time, freq, time_out and freq_out are required");
    check_out(*to, infer_output(t->shape));
    check_out(*fo, infer_output(f->shape));
    int64_t B, St, E, Bf, Sf, Ef;
    split_bse(t->shape, B, St, E);
    split_bse(f->shape, Bf, Sf, Ef);
    MNN_REQUIRE(B == Bf, MNN_ERR_SHAPE_MISMATCH, "time and freq batch sizes differ");
    const int64_t rt = B * St, rf = B * Sf;
    ht_.reserve(sizeof(float) * rt * E);
    hf_.reserve(sizeof(float) * rf * E);
    if (to->data != t->data) k::copy_bytes(ctx(s), t->data, to->data, rt * E * 4);
    if (fo->data != f->data) k::copy_bytes(ctx(s), f->data, fo->data, rf * E * 4);
    float *T = to->f32(), *F = fo->f32(), *ht = ht_.f32(), *hf = hf_.f32();
    for (auto& Lp : layers_) {
      Lyr& L = *Lp;
      L.nts->run(T, rt, ht, s);
      L.sat->run(ht, (int)St, nullptr, 0, (int)B, T, T, nullptr, s);
      L.nfs->run(F, rf, hf, s);
      L.saf->run(hf, (int)Sf, nullptr, 0, (int)B, F, F, nullptr, s);
      L.ntc->run(T, rt, ht, s);
      L.nfc->run(F, rf, hf, s);
      L.cat->run(ht, (int)St, hf, (int)Sf, (int)B, T, T, nullptr, s);
      L.caf->run(hf, (int)Sf, ht, (int)St, (int)B, F, F, nullptr, s);
      L.ntf->run(T, rt, ht, s);
      L.fft->run(ht, rt, T, T, nullptr, s);
      L.nff->run(F, rf, hf, s);
      L.fff->run(hf, rf, F, F, nullptr, s);
    }
  }

 private:
  struct Lyr {
    std::unique_ptr<LayerNormLayer> nts, nfs, ntc, nfc, ntf, nff;
    std::unique_ptr<MHALayer> sat, saf, cat, caf;
    std::unique_ptr<FeedForwardLayer> fft, fff;
  };
  int E_;
  std::vector<std::unique_ptr<Lyr>> layers_;
  DevBuf ht_, hf_;
};

// ------------------------------------------------------------------ Sequential fusion
// Conv1D (no activation, no residual) -> GroupNorm(1 group) [-> GELU] inside a Sequential runs as
// one group. A small contraction (register-window conv) whose grid the device holds at once runs
// in one launch: each workgroup keeps its conv tile in registers and the workgroups exchange their
// statistics partials through the GroupNorm layer's own exchange buffer (tagged words, bounded
// wait); a larger grid takes a statistics pass and an apply pass that recomputes the conv. Other
// convs write their output and statistics partials from the conv's epilogue, then one apply pass
// writes act(GroupNorm(y)). Results are those of the layers run one by one (GELU's +-10 clamp and
// the tanh form agree to float precision beyond |x| = 10).
int fused_chain_length(const std::vector<Layer*>& v, size_t i) {
  if (i + 1 >= v.size()) return 1;
  auto* c = dynamic_cast<Conv1DLayer*>(v[i]);
  auto* g = dynamic_cast<GroupNormLayer*>(v[i + 1]);
  if (!c || !g || c->desc().activation != MNN_ACT_NONE || g->groups() != 1) return 1;
  if (i + 2 < v.size() && g->act() == MNN_ACT_NONE && dynamic_cast<GELULayer*>(v[i + 2]))
    return 3;
  return 2;
}

void run_fused_chain(const std::vector<Layer*>& v, size_t i, int n, const Tensor& in,
                     Tensor& y, Tensor& out, Stream& s) {
  auto* c = static_cast<Conv1DLayer*>(v[i]);
  auto* g = static_cast<GroupNormLayer*>(v[i + 1]);
  const Shape ys = c->infer_output(in.shape);
  MNN_REQUIRE(y.count() == numel(ys) && out.count() == numel(ys), MNN_ERR_BUFFER_SIZE_MISMATCH,
              "fused Conv1D -> GroupNorm: buffers do not hold " << shape_str(ys));
  int64_t B, C, L;
  split_bcl(in.shape, B, C, L);
  const int act = n == 3 ? MNN_ACT_GELU : g->act();
  // The plan may give the chain's last layer the buffer of the layer before the chain, i.e. the
  // chain's own input. The forms below that recompute the convolution from `in` while other
  // workgroups already write `out` then race, so an aliased output takes the y path.
  const char* ib = static_cast<const char*>(in.data);
  const char* ob = static_cast<const char*>(out.data);
  const bool aliased = ob < ib + in.count() * dtype_size(in.dtype) &&
                       ib < ob + out.count() * dtype_size(out.dtype);
  if (!aliased && c->register_window((int)B, (int)L)) {
    // small contraction: statistics pass, then a pass that recomputes the convolution and
    // writes the normalised output once (y is not used)
    k::ConvParams p = c->direct_params((int)B, (int)L);
    p.alpha = 0.01f;  // the activation is GroupNorm's: leaky ReLU slope 0.01
    if (k::conv_gn_oneshot_fits(ctx(s), p)) {
      // the grid fits the device at once: both passes in one launch
      k::conv_gn_oneshot(ctx(s), p, in.f32(), c->weight(), c->bias(), g->exchange(s),
                         s.dev->grid_spin_limit.load(), g->gamma(), g->beta(), g->eps(), act,
                         out.f32());
      return;
    }
    const int nparts = k::conv_gn_num_parts(p);
    float* parts = g->reserve_partials(3LL * B * nparts);
    k::conv_gn_stats(ctx(s), p, in.f32(), c->weight(), c->bias(), parts);
    k::conv_gn_apply(ctx(s), p, in.f32(), c->weight(), c->bias(), parts, nparts, g->gamma(),
                     g->beta(), g->eps(), act, out.f32());
    return;
  }
  const int nparts = c->stats_chunks((int)B, (int)L);
  float* parts = g->reserve_partials(3LL * B * nparts);
  c->run(in.f32(), (int)B, (int)L, y.f32(), MNN_ACT_NONE, parts, s);
  g->apply_parts(s, y.f32(), out.f32(), (int)B, ys.back(), parts, nparts, act);
}

void groupnorm_forward_noalloc(Layer* l, const Tensor& in, Tensor& out, Stream& s) {
  auto* g = dynamic_cast<GroupNormLayer*>(l);
  MNN_REQUIRE(g, MNN_ERR_INVALID_ARGUMENT,
              "allocation-free GroupNorm forward needs a GroupNorm layer, got " << l->kind());
  g->forward_noalloc(in, out, s);
}

// ------------------------------------------------------------------ factories
std::unique_ptr<Layer> make_conv1d(Device* d, const mnn_conv1d_desc& desc, float leaky_alpha) {
  return std::make_unique<Conv1DLayer>(d, desc, leaky_alpha);
}
void conv1d_forward_residual(Layer* l, const Tensor& in, const Tensor* res, Tensor& out,
                             Stream& s) {
  auto* c = dynamic_cast<Conv1DLayer*>(l);
  MNN_REQUIRE(c, MNN_ERR_INVALID_ARGUMENT,
              "forwardWithResidual needs a Conv1D layer, got " << l->kind());
  c->forward_residual(in, res, out, s);
}
std::unique_ptr<Layer> make_groupnorm(Device* d, int groups, int channels, float eps, bool affine,
                                      int act) {
  return std::make_unique<GroupNormLayer>(d, groups, channels, eps, affine, act);
}
std::unique_ptr<Layer> make_layernorm(Device* d, int features, float eps) {
  return std::make_unique<LayerNormLayer>(d, features, eps);
}
std::unique_ptr<Layer> make_gelu(Device* d, const Shape& shape) {
  return std::make_unique<GELULayer>(d, shape);
}
std::unique_ptr<Layer> make_glu(Device* d, int out_channels) {
  return std::make_unique<GLULayer>(d, out_channels);
}
std::unique_ptr<Layer> make_linear(Device* d, int in, int out, bool bias, int act,
                                   mnn_precision prec, float leaky_alpha) {
  return std::make_unique<LinearLayer>(d, in, out, bias, act, prec, leaky_alpha);
}
std::unique_ptr<Layer> make_mha(Device* d, int embed, int heads, bool bias, mnn_precision prec) {
  return std::make_unique<MHALayer>(d, embed, heads, bias, prec);
}
std::unique_ptr<Layer> make_feedforward(Device* d, int in, int hidden, mnn_precision prec) {
  return std::make_unique<FeedForwardLayer>(d, in, hidden, prec);
}
std::unique_ptr<Layer> make_encoder_block(Device* d, const mnn_encoder_block_desc& desc) {
  return std::make_unique<EncoderBlockLayer>(d, desc);
}
std::unique_ptr<Layer> make_conv_transpose1d(Device* d, const mnn_conv_transpose1d_desc& desc) {
  return std::make_unique<ConvTranspose1DLayer>(d, desc);
}
std::unique_ptr<Layer> make_conv2d(Device* d, const mnn_conv2d_desc& desc) {
  return std::make_unique<Conv2DLayer>(d, desc);
}
std::unique_ptr<Layer> make_conv_transpose2d(Device* d, const mnn_conv_transpose2d_desc& desc) {
  return std::make_unique<ConvTranspose2DLayer>(d, desc);
}
std::unique_ptr<Layer> make_freq_encoder_block(Device* d, const mnn_freq_block_desc& desc) {
  return std::make_unique<FreqEncoderBlockLayer>(d, desc);
}
std::unique_ptr<Layer> make_freq_decoder_block(Device* d, const mnn_freq_block_desc& desc) {
  return std::make_unique<FreqDecoderBlockLayer>(d, desc);
}
std::unique_ptr<Layer> make_decoder_block(Device* d, const mnn_decoder_block_desc& desc) {
  return std::make_unique<DecoderBlockLayer>(d, desc);
}
std::unique_ptr<Layer> make_transformer_layer(Device* d, int embed, int heads, int ffn,
                                              float layer_scale, mnn_precision prec) {
  return std::make_unique<TransformerLayerImpl>(d, embed, heads, ffn, layer_scale, prec);
}
std::unique_ptr<Layer> make_cross_transformer_encoder(Device* d, int embed, int heads, int ffn,
                                                     int layers, mnn_precision prec) {
  return std::make_unique<CrossTransformerEncoderImpl>(d, embed, heads, ffn, layers, prec);
}
std::unique_ptr<Layer> make_cross_transformer(Device* d, int embed, int heads, int ffn,
                                              int layers, float layer_scale, mnn_precision prec) {
  return std::make_unique<CrossTransformerImpl>(d, embed, heads, ffn, layers, layer_scale, prec);
}

}  // namespace mnn
