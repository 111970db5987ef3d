// C++ mirror of the reference's layer API: the NNLayer protocol (NNLayer.swift:12-16), the
// hot-path layers of Sources/MetalNN, and Sequential (Model.swift:65-357).
#pragma once

#include <condition_variable>
#include <functional>

#include "common.hpp"
#include "kernels.hpp"

namespace mnn {

// A named device parameter with validated host upload (validateWeights, NNLayer.swift:27-59).
struct Param {
  std::string name;
  int64_t count = 0;
  DevBuf buf;
  bool loaded = false;
  uint64_t version = 0;  // counts loads, so data derived from the parameter can tell it is stale
  const float* ptr() const { return buf.f32(); }
};

class Layer {
 public:
  explicit Layer(Device* d) : dev_(d) {}
  virtual ~Layer() = default;
  virtual const char* kind() const = 0;
  virtual Shape input_shape() const = 0;   // declared, 0 = dynamic dimension
  virtual Shape output_shape() const = 0;  // declared, 0 = dynamic dimension
  virtual Shape infer_output(const Shape& in) const = 0;  // concrete; throws on a bad input
  virtual void forward(const Tensor& in, Tensor& out, Stream& s) = 0;
  virtual void forward_cross(const Tensor* a, const Tensor* b, Tensor* out_a, Tensor* out_b,
                             Stream& s);
  // Whether forward() takes an MNN_BF16 input tensor (otherwise inputs must be f32).
  virtual bool accepts_bf16() const { return false; }
  // Loads a parameter by name; the default looks the name up in params_ (and aliases_).
  virtual void load(const std::string& name, const float* data, size_t n);
  Device* device() const { return dev_; }

 protected:
  Param& add_param(const std::string& name, int64_t count, float fill = 0.f);
  // Called after a successful load, for layers that derive device data from a parameter.
  virtual void on_loaded(const std::string& /*name*/, const float* /*data*/, size_t /*n*/) {}
  Param* find_param(const std::string& name);
  void check_out(const Tensor& out, const Shape& expect) const;

  Device* dev_;
  std::vector<std::unique_ptr<Param>> params_;
  std::map<std::string, std::string> aliases_;
};

// Layer factories (definitions in layers.cpp).
std::unique_ptr<Layer> make_conv1d(Device* d, const mnn_conv1d_desc& desc,
                                   float leaky_alpha = 0.01f);
// FusedConv1D.forwardWithResidual on a Conv1D layer (res may be null).
void conv1d_forward_residual(Layer* l, const Tensor& in, const Tensor* res, Tensor& out,
                             Stream& s);
std::unique_ptr<Layer> make_groupnorm(Device* d, int groups, int channels, float eps, bool affine,
                                      int act);
// GroupNorm forward with its statistics partials in the GPU's fixed scratch (no allocation).
void groupnorm_forward_noalloc(Layer* l, const Tensor& in, Tensor& out, Stream& s);
std::unique_ptr<Layer> make_layernorm(Device* d, int features, float eps);
std::unique_ptr<Layer> make_gelu(Device* d, const Shape& shape);
std::unique_ptr<Layer> make_glu(Device* d, int out_channels);
std::unique_ptr<Layer> make_linear(Device* d, int in, int out, bool bias, int act,
                                   mnn_precision prec, float leaky_alpha = 0.01f);
std::unique_ptr<Layer> make_mha(Device* d, int embed, int heads, bool bias, mnn_precision prec);
std::unique_ptr<Layer> make_feedforward(Device* d, int in, int hidden, mnn_precision prec);
std::unique_ptr<Layer> make_encoder_block(Device* d, const mnn_encoder_block_desc& desc);
std::unique_ptr<Layer> make_conv_transpose1d(Device* d, const mnn_conv_transpose1d_desc& desc);
std::unique_ptr<Layer> make_decoder_block(Device* d, const mnn_decoder_block_desc& desc);
std::unique_ptr<Layer> make_conv2d(Device* d, const mnn_conv2d_desc& desc);
std::unique_ptr<Layer> make_conv_transpose2d(Device* d, const mnn_conv_transpose2d_desc& desc);
std::unique_ptr<Layer> make_freq_encoder_block(Device* d, const mnn_freq_block_desc& desc);
std::unique_ptr<Layer> make_freq_decoder_block(Device* d, const mnn_freq_block_desc& desc);
std::unique_ptr<Layer> make_transformer_layer(Device* d, int embed, int heads, int ffn,
                                              float layer_scale, mnn_precision prec);
std::unique_ptr<Layer> make_cross_transformer(Device* d, int embed, int heads, int ffn,
                                              int layers, float layer_scale, mnn_precision prec);
// The reference CrossTransformerEncoder's own layer structure (self + cross + FFN in every layer).
std::unique_ptr<Layer> make_cross_transformer_encoder(Device* d, int embed, int heads, int ffn,
                                                     int layers, mnn_precision prec);

// Sequential fusion (layers.cpp): the number of layers from index i that run as one fused
// group (1 = no fusion), and the fused run (y: the first layer's buffer, out: the last one's).
int fused_chain_length(const std::vector<Layer*>& v, size_t i);
void run_fused_chain(const std::vector<Layer*>& v, size_t i, int n, const Tensor& in, Tensor& y,
                     Tensor& out, Stream& s);

// Sequential with the reference's ping-pong buffer plan (Model.swift:135-201).
class Sequential {
 public:
  // forwardAsync completion: status and the borrowed output (null on failure).
  using Completion = std::function<void(mnn_status, Tensor*)>;
  explicit Sequential(Device* d) : dev_(d) {}
  ~Sequential();
  void add(Layer* l, bool checked);
  void build();
  Tensor* forward(const Tensor& in, Stream& s);
  // Sequential.forwardAsync (Model.swift:271-346): enqueue the forward on s and return; `done`
  // runs once, on a library thread, after the GPU work completes. Throws (and never calls
  // `done`) when the forward cannot be enqueued.
  void forward_async(const Tensor& in, Stream& s, Completion done);
  std::pair<int, int> buffer_stats() const;
  int layer_count() const { return (int)layers_.size(); }
  // layer(at:) (Model.swift:354-357): null when out of range
  Layer* layer_at(int index) const;

 private:
  struct Plan {
    std::vector<Shape> shapes;       // per layer output shape
    std::vector<int> buffer_index;   // per layer buffer
    std::vector<Tensor*> buffers;    // owned
  };
  Plan* plan_for(const Shape& in);
  void free_plans();

  Device* dev_;
  std::vector<Layer*> layers_;
  bool built_ = false;
  std::map<Shape, Plan> plans_;
  const Plan* last_plan_ = nullptr;
  std::mutex forward_mu_;
  Tensor* forward_locked(const Tensor& in, Stream& s);
  // forwardAsync bookkeeping: one forward in flight at a time. The completion threads count
  // themselves in a state block they share with the model, so a thread whose completion
  // destroyed the model still finds the block alive; the destructor waits for every other
  // completion thread.
  struct AsyncState {
    std::mutex mu;
    std::condition_variable cv;
    int threads = 0;
  };
  std::atomic<bool> async_in_flight_{false};
  std::shared_ptr<AsyncState> async_ = std::make_shared<AsyncState>();
};

Tensor* tensor_create(Device* d, mnn_dtype dt, const Shape& shape);
void tensor_destroy(Tensor* t);

}  // namespace mnn
