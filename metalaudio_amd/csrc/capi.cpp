// extern "C" entry points of mnn.h: argument checks, exception -> status translation.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <thread>

#include "layers.hpp"
#include "mnn_debug.h"
#include "safetensors.hpp"
#include "stft.hpp"
#include "separate.hpp"
#include "weight_names.hpp"

using namespace mnn;

struct mnn_device_s {};
struct mnn_stream_s {};
struct mnn_tensor_s {};
struct mnn_layer_s {};
struct mnn_sequential_s {};
struct mnn_safetensors_s {};
struct mnn_mtla_s {};
struct mnn_stft_s {};
struct mnn_separator_s {};
struct mnn_mtla_writer_s {};

namespace {

thread_local std::string g_last_error;

template <class F>
mnn_status guard(F&& f) {
  try {
    f();
    g_last_error.clear();
    return MNN_OK;
  } catch (const Error& e) {
    g_last_error = e.msg;
    return e.code;
  } catch (const std::bad_alloc&) {
    g_last_error = "host allocation failed";
    return MNN_ERR_OUT_OF_MEMORY;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return MNN_ERR_GPU_EXECUTION;
  }
}

Device* D(mnn_device d) {
  MNN_REQUIRE(d, MNN_ERR_INVALID_ARGUMENT, "null device");
  return reinterpret_cast<Device*>(d);
}
Stream* S(mnn_stream s) {
  MNN_REQUIRE(s, MNN_ERR_INVALID_ARGUMENT, "null stream");
  return reinterpret_cast<Stream*>(s);
}
Tensor* T(mnn_tensor t) {
  MNN_REQUIRE(t, MNN_ERR_INVALID_ARGUMENT, "null tensor");
  return reinterpret_cast<Tensor*>(t);
}
Layer* L(mnn_layer l) {
  MNN_REQUIRE(l, MNN_ERR_INVALID_ARGUMENT, "null layer");
  return reinterpret_cast<Layer*>(l);
}
Sequential* Q(mnn_sequential q) {
  MNN_REQUIRE(q, MNN_ERR_INVALID_ARGUMENT, "null sequential");
  return reinterpret_cast<Sequential*>(q);
}

Shape to_shape(int rank, const int64_t* dims) {
  MNN_REQUIRE(rank >= 1 && rank <= MNN_MAX_RANK && dims, MNN_ERR_INVALID_ARGUMENT,
              "rank must be 1.." << MNN_MAX_RANK);
  return Shape(dims, dims + rank);
}

void put_shape(const Shape& s, int* rank, int64_t* dims) {
  MNN_REQUIRE(rank && dims, MNN_ERR_INVALID_ARGUMENT, "null shape output");
  *rank = (int)s.size();
  for (size_t i = 0; i < s.size(); ++i) dims[i] = s[i];
}

// The stream a call runs on: the given one or the device's default stream.
Stream resolve_stream(Device* d, mnn_stream s) {
  if (s) {
    Stream* st = S(s);
    MNN_REQUIRE(st->dev == d, MNN_ERR_INVALID_ARGUMENT, "stream belongs to another device");
    return *st;
  }
  return Stream{d, d->default_stream, false};
}

mnn_layer wrap(std::unique_ptr<Layer> l) { return reinterpret_cast<mnn_layer>(l.release()); }

template <class T>
const T& need(const T* p) {
  MNN_REQUIRE(p, MNN_ERR_INVALID_ARGUMENT, "null descriptor");
  return *p;
}

}  // namespace

extern "C" {

const char* mnn_last_error_message(void) { return g_last_error.c_str(); }

const char* mnn_status_string(mnn_status s) {
  switch (s) {
    case MNN_OK: return "ok";
    case MNN_ERR_INVALID_CONFIGURATION: return "invalid configuration";
    case MNN_ERR_BUFFER_SIZE_MISMATCH: return "buffer size mismatch";
    case MNN_ERR_PIPELINE_CREATION_FAILED: return "pipeline creation failed";
    case MNN_ERR_GPU_TIMEOUT: return "GPU timeout";
    case MNN_ERR_GPU_EXECUTION: return "GPU execution error";
    case MNN_ERR_DEVICE_LOST: return "device lost";
    case MNN_ERR_OUT_OF_MEMORY: return "out of memory";
    case MNN_ERR_SHAPE_MISMATCH: return "shape mismatch";
    case MNN_ERR_EMPTY_MODEL: return "empty model";
    case MNN_ERR_INPUT_SHAPE_MISMATCH: return "input shape mismatch";
    case MNN_ERR_NOT_BUILT: return "model not built";
    case MNN_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MNN_ERR_FILE_NOT_FOUND: return "file not found";
    case MNN_ERR_INVALID_FILE: return "invalid file";
    case MNN_ERR_TENSOR_NOT_FOUND: return "tensor not found";
  }
  return "unknown status";
}

const char* mnn_version(void) { return "mnn 0.1.0 (gfx950)"; }

// ------------------------------------------------------------------ device
mnn_status mnn_device_create(int ordinal, mnn_device* out) {
  return guard([&] {
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null output");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    MNN_REQUIRE(e == hipSuccess && n > 0, MNN_ERR_DEVICE_LOST,
                "no HIP device available (" << hipGetErrorString(e) << ")");
    MNN_REQUIRE(ordinal >= 0 && ordinal < n, MNN_ERR_INVALID_ARGUMENT,
                "device ordinal " << ordinal << " out of range (" << n << " devices)");
    auto d = std::make_unique<Device>();
    d->ordinal = ordinal;
    HIP_CHECK(hipSetDevice(ordinal));
    HIP_CHECK(hipGetDeviceProperties(&d->props, ordinal));
    MNN_REQUIRE(std::string(d->props.gcnArchName).rfind("gfx950", 0) == 0,
                MNN_ERR_PIPELINE_CREATION_FAILED,
                "kernels are built for gfx950, device is " << d->props.gcnArchName);
    HIP_CHECK(hipStreamCreateWithFlags(&d->default_stream, hipStreamNonBlocking));
    *out = reinterpret_cast<mnn_device>(d.release());
  });
}

mnn_status mnn_device_destroy(mnn_device dev) {
  return guard([&] {
    if (!dev) return;
    Device* d = D(dev);
    d->make_current();
    (void)hipDeviceSynchronize();
    for (auto& t : d->pending) {
      (void)hipEventDestroy(t.start);
      (void)hipEventDestroy(t.stop);
    }
    for (auto& p : d->event_pool) {
      (void)hipEventDestroy(p.first);
      (void)hipEventDestroy(p.second);
    }
    if (d->default_stream) (void)hipStreamDestroy(d->default_stream);
    delete d;
  });
}

mnn_status mnn_device_name(mnn_device dev, char* buf, size_t n) {
  return guard([&] {
    Device* d = D(dev);
    MNN_REQUIRE(buf && n > 0, MNN_ERR_INVALID_ARGUMENT, "null buffer");
    std::snprintf(buf, n, "%s [%s, %d CUs]", d->props.name[0] ? d->props.name : "AMD GPU", d->props.gcnArchName,
                  d->props.multiProcessorCount);
  });
}

mnn_status mnn_device_synchronize(mnn_device dev) {
  return guard([&] {
    Device* d = D(dev);
    d->check_alive();
    d->make_current();
    HIP_CHECK(hipDeviceSynchronize());
  });
}

mnn_status mnn_device_mark_lost(mnn_device dev) {
  return guard([&] { D(dev)->lost = true; });
}

mnn_status mnn_device_check_available(mnn_device dev, int timeout_ms) {
  return guard([&] {
    Device* d = D(dev);
    d->check_alive();
    d->make_current();
    hipEvent_t e;
    HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    HIP_CHECK(hipEventRecord(e, d->default_stream));
    const auto t0 = std::chrono::steady_clock::now();
    while (true) {
      hipError_t q = hipEventQuery(e);
      if (q == hipSuccess) break;
      if (q != hipErrorNotReady) {
        (void)hipEventDestroy(e);
        d->lost = true;
        fail(MNN_ERR_DEVICE_LOST, std::string("device check failed: ") + hipGetErrorString(q));
      }
      if (timeout_ms > 0 && std::chrono::steady_clock::now() - t0 >
                                std::chrono::milliseconds(timeout_ms)) {
        (void)hipEventDestroy(e);
        fail(MNN_ERR_GPU_TIMEOUT, "device did not answer within the timeout");
      }
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    (void)hipEventDestroy(e);
  });
}

mnn_status mnn_device_set_kernel_timing(mnn_device dev, int enable) {
  return guard([&] { D(dev)->timing = enable != 0; });
}

mnn_status mnn_device_kernel_timing(mnn_device dev, const char* sub, int64_t* launches,
                                    double* total_ms) {
  return guard([&] {
    Device* d = D(dev);
    MNN_REQUIRE(launches && total_ms, MNN_ERR_INVALID_ARGUMENT, "null output");
    d->make_current();
    d->resolve_timers();
    int64_t n = 0;
    double ms = 0.0;
    std::lock_guard<std::mutex> lk(d->timing_mu);
    for (auto& kv : d->stats)
      if (!sub || kv.first.find(sub) != std::string::npos) {
        n += kv.second.first;
        ms += kv.second.second;
      }
    *launches = n;
    *total_ms = ms;
  });
}

mnn_status mnn_device_reset_kernel_timing(mnn_device dev) {
  return guard([&] {
    Device* d = D(dev);
    d->make_current();
    d->resolve_timers();
    std::lock_guard<std::mutex> lk(d->timing_mu);
    d->stats.clear();
  });
}

// ------------------------------------------------------------------ stream
mnn_status mnn_stream_create(mnn_device dev, mnn_stream* out) {
  return guard([&] {
    Device* d = D(dev);
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null output");
    d->make_current();
    auto s = std::make_unique<Stream>();
    s->dev = d;
    s->owned = true;
    HIP_CHECK(hipStreamCreateWithFlags(&s->s, hipStreamNonBlocking));
    *out = reinterpret_cast<mnn_stream>(s.release());
  });
}

mnn_status mnn_stream_sync(mnn_stream st, int timeout_ms) {
  return guard([&] {
    Stream* s = S(st);
    s->dev->check_alive();
    s->dev->make_current();
    if (timeout_ms <= 0) {
      HIP_CHECK(hipStreamSynchronize(s->s));
      return;
    }
    const auto t0 = std::chrono::steady_clock::now();
    while (true) {
      hipError_t q = hipStreamQuery(s->s);
      if (q == hipSuccess) return;
      if (q != hipErrorNotReady)
        fail(MNN_ERR_GPU_EXECUTION, std::string("stream error: ") + hipGetErrorString(q));
      if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(timeout_ms))
        fail(MNN_ERR_GPU_TIMEOUT, "GPU work did not finish within " + std::to_string(timeout_ms) +
                                      " ms (it keeps running)");
      std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
  });
}

namespace {
// Timing marks of mnn_debug_stream_mark, per stream handle.
std::mutex g_marks_mu;
std::map<const Stream*, std::vector<hipEvent_t>> g_marks;
}  // namespace

mnn_status mnn_stream_destroy(mnn_stream st) {
  return guard([&] {
    if (!st) return;
    Stream* s = S(st);
    s->dev->make_current();
    if (s->owned && s->s) {
      (void)hipStreamSynchronize(s->s);
      (void)hipStreamDestroy(s->s);
    }
    {
      std::lock_guard<std::mutex> lk(g_marks_mu);
      auto it = g_marks.find(s);
      if (it != g_marks.end()) {
        for (hipEvent_t e : it->second) (void)hipEventDestroy(e);
        g_marks.erase(it);
      }
    }
    delete s;
  });
}

// ------------------------------------------------------------------ tensor
mnn_status mnn_tensor_create(mnn_device dev, mnn_dtype dtype, int rank, const int64_t* dims,
                             mnn_tensor* out) {
  return guard([&] {
    Device* d = D(dev);
    d->check_alive();
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null output");
    MNN_REQUIRE(dtype == MNN_F32 || dtype == MNN_BF16, MNN_ERR_INVALID_ARGUMENT, "bad dtype");
    *out = reinterpret_cast<mnn_tensor>(tensor_create(d, dtype, to_shape(rank, dims)));
  });
}

mnn_status mnn_tensor_destroy(mnn_tensor t) {
  return guard([&] {
    if (t) tensor_destroy(T(t));
  });
}

mnn_status mnn_tensor_shape(mnn_tensor t, int* rank, int64_t* dims) {
  return guard([&] { put_shape(T(t)->shape, rank, dims); });
}

mnn_status mnn_tensor_reshape(mnn_tensor t, int rank, const int64_t* dims) {
  return guard([&] {
    Tensor* x = T(t);
    Shape s = to_shape(rank, dims);
    MNN_REQUIRE(numel(s) == x->count(), MNN_ERR_BUFFER_SIZE_MISMATCH,
                "reshape " << shape_str(x->shape) << " -> " << shape_str(s)
                           << " changes the element count");
    x->shape = s;
  });
}

mnn_status mnn_tensor_upload(mnn_tensor t, const void* host, size_t bytes, mnn_stream st) {
  return guard([&] {
    Tensor* x = T(t);
    x->dev->check_alive();
    MNN_REQUIRE(host || bytes == 0, MNN_ERR_INVALID_ARGUMENT, "null host buffer");
    MNN_REQUIRE(bytes == x->bytes, MNN_ERR_BUFFER_SIZE_MISMATCH,
                "upload of " << bytes << " bytes into a tensor of " << x->bytes);
    Stream s = resolve_stream(x->dev, st);
    x->dev->make_current();
    HIP_CHECK(hipMemcpyAsync(x->data, host, bytes, hipMemcpyHostToDevice, s.s));
    HIP_CHECK(hipStreamSynchronize(s.s));
  });
}

mnn_status mnn_tensor_download(mnn_tensor t, void* host, size_t bytes, mnn_stream st) {
  return guard([&] {
    Tensor* x = T(t);
    x->dev->check_alive();
    MNN_REQUIRE(host || bytes == 0, MNN_ERR_INVALID_ARGUMENT, "null host buffer");
    MNN_REQUIRE(bytes == x->bytes, MNN_ERR_BUFFER_SIZE_MISMATCH,
                "download of " << bytes << " bytes from a tensor of " << x->bytes);
    Stream s = resolve_stream(x->dev, st);
    x->dev->make_current();
    HIP_CHECK(hipMemcpyAsync(host, x->data, bytes, hipMemcpyDeviceToHost, s.s));
    HIP_CHECK(hipStreamSynchronize(s.s));
  });
}

mnn_status mnn_tensor_copy(mnn_tensor dst, mnn_tensor src, mnn_stream st) {
  return guard([&] {
    Tensor* d = T(dst);
    Tensor* s = T(src);
    MNN_REQUIRE(d->dev == s->dev, MNN_ERR_INVALID_ARGUMENT, "tensors on different devices");
    d->dev->check_alive();
    MNN_REQUIRE(d->bytes == s->bytes, MNN_ERR_BUFFER_SIZE_MISMATCH,
                "copy between tensors of " << s->bytes << " and " << d->bytes << " bytes");
    Stream sv = resolve_stream(d->dev, st);
    d->dev->make_current();
    k::copy_bytes(LaunchCtx{d->dev, sv.s}, s->data, d->data, (int64_t)s->bytes);
  });
}

mnn_status mnn_tensor_device_ptr(mnn_tensor t, void** ptr) {
  return guard([&] {
    MNN_REQUIRE(ptr, MNN_ERR_INVALID_ARGUMENT, "null output");
    *ptr = T(t)->data;
  });
}

// ------------------------------------------------------------------ layers
#define MNN_CREATE(expr)                                         \
  return guard([&] {                                             \
    Device* d = D(dev);                                          \
    d->check_alive();                                            \
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null output");   \
    d->make_current();                                           \
    *out = wrap(expr);                                           \
  })

mnn_status mnn_conv1d_create(mnn_device dev, const mnn_conv1d_desc* desc, mnn_layer* out) {
  MNN_CREATE(make_conv1d(d, need(desc)));
}
mnn_status mnn_fused_conv1d_create(mnn_device dev, const mnn_conv1d_desc* desc,
                                   float leaky_relu_alpha, mnn_layer* out) {
  MNN_CREATE(make_conv1d(d, need(desc), leaky_relu_alpha));
}
mnn_status mnn_conv1d_forward_residual(mnn_layer layer, mnn_tensor input, mnn_tensor residual,
                                       mnn_tensor output, mnn_stream st) {
  return guard([&] {
    Layer* l = L(layer);
    Tensor* in = T(input);
    Tensor* out = T(output);
    Tensor* res = residual ? T(residual) : nullptr;
    MNN_REQUIRE(in->dev == l->device() && out->dev == l->device() &&
                    (!res || res->dev == l->device()),
                MNN_ERR_INVALID_ARGUMENT, "tensors must live on the layer's device");
    MNN_REQUIRE(in->dtype == MNN_F32 && out->dtype == MNN_F32 && (!res || res->dtype == MNN_F32),
                MNN_ERR_INVALID_ARGUMENT, "forwardWithResidual: tensors must be f32");
    in->dev->check_alive();
    Stream s = resolve_stream(in->dev, st);
    in->dev->make_current();
    conv1d_forward_residual(l, *in, res, *out, s);
  });
}
mnn_status mnn_groupnorm_create(mnn_device dev, int num_groups, int num_channels, float epsilon,
                                int affine, mnn_activation act, mnn_layer* out) {
  MNN_CREATE(make_groupnorm(d, num_groups, num_channels, epsilon, affine != 0, act));
}
mnn_status mnn_groupnorm_forward_noalloc(mnn_layer layer, mnn_tensor input, mnn_tensor output,
                                         mnn_stream st) {
  return guard([&] {
    Layer* l = L(layer);
    Tensor* in = T(input);
    Tensor* out = T(output);
    MNN_REQUIRE(in->dev == l->device() && out->dev == l->device(), MNN_ERR_INVALID_ARGUMENT,
                "tensors must live on the layer's device");
    MNN_REQUIRE(in->dtype == MNN_F32 && out->dtype == MNN_F32, MNN_ERR_INVALID_ARGUMENT,
                "GroupNorm: tensors must be f32");
    in->dev->check_alive();
    Stream s = resolve_stream(in->dev, st);
    in->dev->make_current();
    groupnorm_forward_noalloc(l, *in, *out, s);
  });
}
mnn_status mnn_layernorm_create(mnn_device dev, int feature_size, float epsilon, mnn_layer* out) {
  MNN_CREATE(make_layernorm(d, feature_size, epsilon));
}
mnn_status mnn_gelu_create(mnn_device dev, int rank, const int64_t* shape, mnn_layer* out) {
  MNN_CREATE(make_gelu(d, to_shape(rank, shape)));
}
mnn_status mnn_glu_create(mnn_device dev, int out_channels, mnn_layer* out) {
  MNN_CREATE(make_glu(d, out_channels));
}
mnn_status mnn_linear_create(mnn_device dev, int in_features, int out_features, int use_bias,
                             mnn_activation act, mnn_precision prec, mnn_layer* out) {
  MNN_CREATE(make_linear(d, in_features, out_features, use_bias != 0, act, prec));
}
mnn_status mnn_fused_linear_create(mnn_device dev, int in_features, int out_features,
                                   int use_bias, mnn_activation act, float leaky_relu_alpha,
                                   mnn_precision prec, mnn_layer* out) {
  MNN_CREATE(make_linear(d, in_features, out_features, use_bias != 0, act, prec,
                         leaky_relu_alpha));
}
mnn_status mnn_mha_create(mnn_device dev, int embed_dim, int num_heads, int use_bias,
                          mnn_precision prec, mnn_layer* out) {
  MNN_CREATE(make_mha(d, embed_dim, num_heads, use_bias != 0, prec));
}
mnn_status mnn_feedforward_create(mnn_device dev, int input_dim, int hidden_dim,
                                  mnn_precision prec, mnn_layer* out) {
  MNN_CREATE(make_feedforward(d, input_dim, hidden_dim, prec));
}
mnn_status mnn_encoder_block_create(mnn_device dev, const mnn_encoder_block_desc* desc,
                                    mnn_layer* out) {
  MNN_CREATE(make_encoder_block(d, need(desc)));
}
mnn_status mnn_conv_transpose1d_create(mnn_device dev, const mnn_conv_transpose1d_desc* desc,
                                       mnn_layer* out) {
  MNN_CREATE(make_conv_transpose1d(d, need(desc)));
}
mnn_status mnn_decoder_block_create(mnn_device dev, const mnn_decoder_block_desc* desc,
                                    mnn_layer* out) {
  MNN_CREATE(make_decoder_block(d, need(desc)));
}
mnn_status mnn_conv2d_create(mnn_device dev, const mnn_conv2d_desc* desc, mnn_layer* out) {
  MNN_CREATE(make_conv2d(d, need(desc)));
}
mnn_status mnn_conv_transpose2d_create(mnn_device dev, const mnn_conv_transpose2d_desc* desc,
                                       mnn_layer* out) {
  MNN_CREATE(make_conv_transpose2d(d, need(desc)));
}
mnn_status mnn_freq_encoder_block_create(mnn_device dev, const mnn_freq_block_desc* desc,
                                         mnn_layer* out) {
  MNN_CREATE(make_freq_encoder_block(d, need(desc)));
}
mnn_status mnn_freq_decoder_block_create(mnn_device dev, const mnn_freq_block_desc* desc,
                                         mnn_layer* out) {
  MNN_CREATE(make_freq_decoder_block(d, need(desc)));
}
namespace {
// Zero padding that makes n a multiple of stride^levels, split total/2 left, rest right.
void unet_pad(int64_t n, int levels, int stride, int64_t& left, int64_t& right, int64_t& out) {
  MNN_REQUIRE(n >= 0 && levels >= 0 && stride > 0, MNN_ERR_INVALID_ARGUMENT,
              "invalid padding query");
  int64_t divisor = 1;
  for (int i = 0; i < levels; ++i) {
    MNN_REQUIRE(divisor <= (INT64_MAX / stride), MNN_ERR_INVALID_ARGUMENT,
                "stride^levels overflows");
    divisor *= stride;
  }
  const int64_t rem = n % divisor;
  const int64_t total = rem == 0 ? 0 : divisor - rem;
  left = total / 2;
  right = total - total / 2;
  out = n + total;
}
int64_t unet_bottleneck(int64_t n, int levels, int stride) {
  MNN_REQUIRE(stride > 0 && levels >= 0, MNN_ERR_INVALID_ARGUMENT, "invalid bottleneck query");
  for (int i = 0; i < levels; ++i) n /= stride;
  return n;
}
}  // namespace

mnn_status mnn_unet_padding(int64_t input_length, int levels, int kernel_size, int stride,
                            int64_t* left_pad, int64_t* right_pad, int64_t* output_length) {
  return guard([&] {
    MNN_REQUIRE(left_pad && right_pad && output_length, MNN_ERR_INVALID_ARGUMENT,
                "null output pointer");
    MNN_REQUIRE(kernel_size > 0, MNN_ERR_INVALID_ARGUMENT, "invalid padding query");
    unet_pad(input_length, levels, stride, *left_pad, *right_pad, *output_length);
  });
}
mnn_status mnn_unet_bottleneck_length(int64_t input_length, int levels, int stride,
                                      int64_t* length) {
  return guard([&] {
    MNN_REQUIRE(length, MNN_ERR_INVALID_ARGUMENT, "invalid bottleneck query");
    *length = unet_bottleneck(input_length, levels, stride);
  });
}
mnn_status mnn_unet_padding_2d(int64_t height, int64_t width, int levels, int stride,
                               int64_t out[6]) {
  return guard([&] {
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null output pointer");
    int64_t o[6];
    unet_pad(height, levels, stride, o[0], o[1], o[4]);
    unet_pad(width, levels, stride, o[2], o[3], o[5]);
    std::copy(o, o + 6, out);
  });
}
mnn_status mnn_unet_bottleneck_2d(int64_t height, int64_t width, int levels, int stride,
                                  int64_t out[2]) {
  return guard([&] {
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null output pointer");
    const int64_t h = unet_bottleneck(height, levels, stride);
    out[1] = unet_bottleneck(width, levels, stride);
    out[0] = h;
  });
}
// ------------------------------------------------------------------ STFT
namespace {
StftPlan* SP(mnn_stft p) {
  MNN_REQUIRE(p, MNN_ERR_INVALID_ARGUMENT, "null STFT handle");
  return reinterpret_cast<StftPlan*>(p);
}
}  // namespace

mnn_status mnn_stft_create(mnn_device dev, int fft_size, int hop_size, int window, mnn_stft* out) {
  return guard([&] {
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null argument");
    Device* d = D(dev);
    d->check_alive();
    *out = reinterpret_cast<mnn_stft>(new StftPlan(d, fft_size, hop_size, window));
  });
}
mnn_status mnn_stft_destroy(mnn_stft plan) {
  return guard([&] {
    StftPlan* p = reinterpret_cast<StftPlan*>(plan);
    if (p) p->device()->make_current();
    delete p;
  });
}
mnn_status mnn_stft_window(mnn_stft plan, float* out, size_t count) {
  return guard([&] {
    const auto& w = SP(plan)->window();
    MNN_REQUIRE(out && count == w.size(), MNN_ERR_BUFFER_SIZE_MISMATCH,
                "window holds " << w.size() << " values");
    std::copy(w.begin(), w.end(), out);
  });
}
mnn_status mnn_stft_frame_count(mnn_stft plan, int64_t samples, int64_t* frames) {
  return guard([&] {
    MNN_REQUIRE(frames, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *frames = SP(plan)->frame_count(samples);
  });
}
mnn_status mnn_stft_output_length(mnn_stft plan, int64_t frames, int64_t* samples) {
  return guard([&] {
    MNN_REQUIRE(samples, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *samples = SP(plan)->output_length(frames);
  });
}
mnn_status mnn_stft_forward(mnn_stft plan, mnn_tensor input, mnn_tensor real, mnn_tensor imag,
                            int onesided, int layout, mnn_stream st) {
  return guard([&] {
    StftPlan* p = SP(plan);
    Tensor *x = T(input), *re = T(real), *im = T(imag);
    Device* d = p->device();
    d->check_alive();
    MNN_REQUIRE(x->dev == d && re->dev == d && im->dev == d, MNN_ERR_INVALID_ARGUMENT,
                "tensors and plan on different devices");
    Stream s = resolve_stream(d, st);
    d->make_current();
    p->forward(*x, *re, *im, onesided != 0, layout, s);
  });
}
mnn_status mnn_stft_inverse(mnn_stft plan, mnn_tensor real, mnn_tensor imag, int onesided,
                            int layout, float window_floor, mnn_tensor output, mnn_stream st) {
  return guard([&] {
    StftPlan* p = SP(plan);
    Tensor *re = T(real), *im = T(imag), *y = T(output);
    Device* d = p->device();
    d->check_alive();
    MNN_REQUIRE(y->dev == d && re->dev == d && im->dev == d, MNN_ERR_INVALID_ARGUMENT,
                "tensors and plan on different devices");
    Stream s = resolve_stream(d, st);
    d->make_current();
    p->inverse(*re, *im, onesided != 0, layout, window_floor, *y, s);
  });
}

// ------------------------------------------------------------------ separator
namespace {
TimeSeparator* SEP(mnn_separator p) {
  MNN_REQUIRE(p, MNN_ERR_INVALID_ARGUMENT, "null separator handle");
  return reinterpret_cast<TimeSeparator*>(p);
}
}  // namespace

mnn_status mnn_separator_create(mnn_device dev, const mnn_separator_desc* desc,
                                mnn_separator* out) {
  return guard([&] {
    MNN_REQUIRE(desc && out, MNN_ERR_INVALID_ARGUMENT, "null argument");
    Device* d = D(dev);
    d->check_alive();
    d->make_current();
    *out = reinterpret_cast<mnn_separator>(new TimeSeparator(d, *desc));
  });
}
mnn_status mnn_separator_destroy(mnn_separator sep) {
  return guard([&] {
    TimeSeparator* p = reinterpret_cast<TimeSeparator*>(sep);
    if (p) p->device()->make_current();
    delete p;
  });
}
mnn_status mnn_separator_load(mnn_separator sep, const char* name, const float* data, size_t n) {
  return guard([&] {
    MNN_REQUIRE(name && (data || n == 0), MNN_ERR_INVALID_ARGUMENT, "null argument");
    TimeSeparator* p = SEP(sep);
    p->device()->check_alive();
    p->load(name, data, n);
  });
}
namespace {
mnn_status separate_call(mnn_separator sep, mnn_tensor input, mnn_tensor output, int64_t seg,
                         int64_t ovl, mnn_stream st) {
  return guard([&] {
    TimeSeparator* p = SEP(sep);
    Tensor *x = T(input), *y = T(output);
    Device* d = p->device();
    d->check_alive();
    MNN_REQUIRE(x->dev == d && y->dev == d, MNN_ERR_INVALID_ARGUMENT,
                "tensors and separator on different devices");
    MNN_REQUIRE(x->data != y->data, MNN_ERR_INVALID_ARGUMENT, "input and output must differ");
    Stream s = resolve_stream(d, st);
    d->make_current();
    p->separate_long(*x, *y, seg, ovl, s);
  });
}
}  // namespace
mnn_status mnn_separator_separate(mnn_separator sep, mnn_tensor input, mnn_tensor output,
                                  mnn_stream stream) {
  return separate_call(sep, input, output, 0, 0, stream);
}
mnn_status mnn_separator_separate_long(mnn_separator sep, mnn_tensor input, mnn_tensor output,
                                       int64_t segment_frames, int64_t overlap_frames,
                                       mnn_stream stream) {
  return separate_call(sep, input, output, segment_frames <= 0 ? 0 : segment_frames,
                       overlap_frames, stream);
}

// ------------------------------------------------------------------ SafeTensors
namespace {
SafeTensorsFile* ST(mnn_safetensors s) {
  MNN_REQUIRE(s, MNN_ERR_INVALID_ARGUMENT, "null safetensors handle");
  return reinterpret_cast<SafeTensorsFile*>(s);
}
void put_string(const std::string& v, char* buf, size_t cap) {
  MNN_REQUIRE(buf && cap > v.size(), MNN_ERR_BUFFER_SIZE_MISMATCH,
              "buffer of " << cap << " bytes is too small for " << v.size() + 1);
  std::memcpy(buf, v.c_str(), v.size() + 1);
}
}  // namespace

mnn_status mnn_safetensors_open(const char* path, mnn_safetensors* out) {
  return guard([&] {
    MNN_REQUIRE(path && out, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *out = reinterpret_cast<mnn_safetensors>(new SafeTensorsFile(path));
  });
}
mnn_status mnn_safetensors_close(mnn_safetensors st) {
  return guard([&] { delete reinterpret_cast<SafeTensorsFile*>(st); });
}
mnn_status mnn_safetensors_tensor_count(mnn_safetensors st, int* count) {
  return guard([&] {
    MNN_REQUIRE(count, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *count = (int)ST(st)->names().size();
  });
}
mnn_status mnn_safetensors_tensor_name(mnn_safetensors st, int index, char* buf, size_t cap) {
  return guard([&] {
    const auto& n = ST(st)->names();
    MNN_REQUIRE(index >= 0 && index < (int)n.size(), MNN_ERR_INVALID_ARGUMENT,
                "tensor index " << index << " out of range");
    put_string(n[index], buf, cap);
  });
}
mnn_status mnn_safetensors_tensor_info(mnn_safetensors st, const char* name, mnn_st_dtype* dtype,
                                       int* rank, int64_t* dims, size_t* count) {
  return guard([&] {
    MNN_REQUIRE(name, MNN_ERR_INVALID_ARGUMENT, "null name");
    const StTensorInfo& ti = ST(st)->info(name);
    MNN_REQUIRE((int)ti.shape.size() <= MNN_MAX_RANK, MNN_ERR_INVALID_ARGUMENT,
                "tensor rank " << ti.shape.size() << " exceeds " << MNN_MAX_RANK);
    if (dtype) *dtype = (mnn_st_dtype)ti.dtype;
    if (rank) *rank = (int)ti.shape.size();
    if (dims)
      for (size_t i = 0; i < ti.shape.size(); ++i) dims[i] = ti.shape[i];
    if (count) *count = ti.end >= ti.begin ? (size_t)ti.count() : 0;
  });
}
mnn_status mnn_safetensors_read_f32(mnn_safetensors st, const char* name, float* out,
                                    size_t count) {
  return guard([&] {
    MNN_REQUIRE(name, MNN_ERR_INVALID_ARGUMENT, "null name");
    ST(st)->read_f32(name, out, count);
  });
}
mnn_status mnn_safetensors_metadata(mnn_safetensors st, const char* key, char* buf, size_t cap) {
  return guard([&] {
    MNN_REQUIRE(key, MNN_ERR_INVALID_ARGUMENT, "null key");
    const auto& m = ST(st)->metadata();
    auto it = m.find(key);
    MNN_REQUIRE(it != m.end(), MNN_ERR_TENSOR_NOT_FOUND, "metadata key '" << key << "' absent");
    put_string(it->second, buf, cap);
  });
}
mnn_status mnn_layer_load_safetensors(mnn_layer layer, mnn_safetensors st,
                                      const char* tensor_name, const char* param_name) {
  return guard([&] {
    Layer* l = L(layer);
    SafeTensorsFile* f = ST(st);
    MNN_REQUIRE(tensor_name && param_name, MNN_ERR_INVALID_ARGUMENT, "null name");
    const StTensorInfo& ti = f->info(tensor_name);
    MNN_REQUIRE(ti.end >= ti.begin, MNN_ERR_INVALID_FILE,
                "Tensor '" << tensor_name << "' has a negative byte range");
    std::vector<float> host((size_t)ti.count());
    f->read_f32(tensor_name, host.data(), host.size());
    l->device()->check_alive();
    l->device()->make_current();
    l->load(param_name, host.data(), host.size());
  });
}

// ------------------------------------------------------------------ weight names
namespace {
WeightConvention WCONV(int c) {
  MNN_REQUIRE(c >= WC_METALAUDIO && c <= WC_UNKNOWN, MNN_ERR_INVALID_ARGUMENT,
              "unknown naming convention " << c);
  return static_cast<WeightConvention>(c);
}
}  // namespace

mnn_status mnn_weight_convention_detect(const char* const* names, int count, int* convention) {
  return guard([&] {
    MNN_REQUIRE(convention && count >= 0 && (names || count == 0), MNN_ERR_INVALID_ARGUMENT,
                "invalid argument");
    std::vector<std::string> v;
    for (int i = 0; i < count; ++i) {
      MNN_REQUIRE(names[i], MNN_ERR_INVALID_ARGUMENT, "null name at " << i);
      v.emplace_back(names[i]);
    }
    *convention = detect_convention(v);
  });
}
mnn_status mnn_safetensors_detect_convention(mnn_safetensors st, int* convention) {
  return guard([&] {
    MNN_REQUIRE(convention, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *convention = detect_convention(ST(st)->names());
  });
}
mnn_status mnn_weight_name_to_metalaudio(int convention, const char* name, char* buf, size_t cap) {
  return guard([&] {
    MNN_REQUIRE(name, MNN_ERR_INVALID_ARGUMENT, "null name");
    put_string(to_metalaudio(WCONV(convention), name), buf, cap);
  });
}
mnn_status mnn_weight_name_from_metalaudio(const char* name, int target, char* buf, size_t cap) {
  return guard([&] {
    MNN_REQUIRE(name, MNN_ERR_INVALID_ARGUMENT, "null name");
    put_string(from_metalaudio(name, WCONV(target)), buf, cap);
  });
}
mnn_status mnn_weight_name_is_metalaudio(const char* name, int* out) {
  return guard([&] {
    MNN_REQUIRE(name && out, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *out = is_metalaudio_naming(name) ? 1 : 0;
  });
}
mnn_status mnn_weight_name_is_demucs(const char* name, int* out) {
  return guard([&] {
    MNN_REQUIRE(name && out, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *out = is_demucs_naming(name) ? 1 : 0;
  });
}
mnn_status mnn_safetensors_find_mapped(mnn_safetensors st, int convention,
                                       const char* metalaudio_name, char* buf, size_t cap) {
  return guard([&] {
    MNN_REQUIRE(metalaudio_name, MNN_ERR_INVALID_ARGUMENT, "null name");
    const std::string n = find_mapped(ST(st)->names(), WCONV(convention), metalaudio_name);
    MNN_REQUIRE(!n.empty(), MNN_ERR_TENSOR_NOT_FOUND,
                "Tensor '" << metalaudio_name << "' not found");
    put_string(n, buf, cap);
  });
}

mnn_status mnn_separator_load_safetensors(mnn_separator sep, mnn_safetensors st, int convention,
                                          int* loaded) {
  return guard([&] {
    TimeSeparator* p = SEP(sep);
    MNN_REQUIRE(convention >= WC_METALAUDIO && convention <= WC_UNKNOWN,
                MNN_ERR_INVALID_ARGUMENT, "unknown naming convention " << convention);
    p->device()->check_alive();
    const int n = p->load_safetensors(*ST(st), static_cast<WeightConvention>(convention));
    if (loaded) *loaded = n;
  });
}

// ------------------------------------------------------------------ MTLA
namespace {
MtlaFile* MT(mnn_mtla m) {
  MNN_REQUIRE(m, MNN_ERR_INVALID_ARGUMENT, "null model-file handle");
  return reinterpret_cast<MtlaFile*>(m);
}
using MtlaTensors = std::map<std::string, std::pair<std::vector<int64_t>, std::vector<float>>>;
MtlaTensors* MW(mnn_mtla_writer w) {
  MNN_REQUIRE(w, MNN_ERR_INVALID_ARGUMENT, "null writer handle");
  return reinterpret_cast<MtlaTensors*>(w);
}
}  // namespace

mnn_status mnn_mtla_open(const char* path, mnn_mtla* out) {
  return guard([&] {
    MNN_REQUIRE(path && out, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *out = reinterpret_cast<mnn_mtla>(new MtlaFile(path));
  });
}
mnn_status mnn_mtla_close(mnn_mtla m) {
  return guard([&] { delete reinterpret_cast<MtlaFile*>(m); });
}
mnn_status mnn_mtla_tensor_count(mnn_mtla m, int* count) {
  return guard([&] {
    MNN_REQUIRE(count, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *count = (int)MT(m)->names().size();
  });
}
mnn_status mnn_mtla_tensor_name(mnn_mtla m, int index, char* buf, size_t cap) {
  return guard([&] {
    const auto& n = MT(m)->names();
    MNN_REQUIRE(index >= 0 && index < (int)n.size(), MNN_ERR_INVALID_ARGUMENT,
                "tensor index " << index << " out of range");
    put_string(n[index], buf, cap);
  });
}
mnn_status mnn_mtla_tensor_info(mnn_mtla m, const char* name, int* rank, int64_t* dims,
                                size_t* count) {
  return guard([&] {
    MNN_REQUIRE(name, MNN_ERR_INVALID_ARGUMENT, "null name");
    const auto& sh = MT(m)->shape(name);
    MNN_REQUIRE((int)sh.size() <= MNN_MAX_RANK, MNN_ERR_INVALID_ARGUMENT,
                "tensor rank " << sh.size() << " exceeds " << MNN_MAX_RANK);
    if (rank) *rank = (int)sh.size();
    if (dims)
      for (size_t i = 0; i < sh.size(); ++i) dims[i] = sh[i];
    if (count) *count = MT(m)->data(name).size();
  });
}
mnn_status mnn_mtla_read_f32(mnn_mtla m, const char* name, float* out, size_t count) {
  return guard([&] {
    MNN_REQUIRE(name, MNN_ERR_INVALID_ARGUMENT, "null name");
    const auto& v = MT(m)->data(name);
    MNN_REQUIRE(v.size() == count, MNN_ERR_BUFFER_SIZE_MISMATCH,
                "Tensor '" << name << "' holds " << v.size() << " values, the destination "
                           << count);
    MNN_REQUIRE(out || count == 0, MNN_ERR_INVALID_ARGUMENT, "null destination");
    std::copy(v.begin(), v.end(), out);
  });
}
mnn_status mnn_layer_load_mtla(mnn_layer layer, mnn_mtla m, const char* tensor_name,
                               const char* param_name) {
  return guard([&] {
    Layer* l = L(layer);
    MNN_REQUIRE(tensor_name && param_name, MNN_ERR_INVALID_ARGUMENT, "null name");
    const auto& v = MT(m)->data(tensor_name);
    l->device()->check_alive();
    l->device()->make_current();
    l->load(param_name, v.data(), v.size());
  });
}
mnn_status mnn_mtla_writer_create(mnn_mtla_writer* out) {
  return guard([&] {
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null argument");
    *out = reinterpret_cast<mnn_mtla_writer>(new MtlaTensors());
  });
}
mnn_status mnn_mtla_writer_add(mnn_mtla_writer w, const char* name, int rank, const int64_t* dims,
                               const float* data) {
  return guard([&] {
    MNN_REQUIRE(name && rank >= 0 && rank <= 16 && (rank == 0 || dims), MNN_ERR_INVALID_ARGUMENT,
                "invalid tensor description");
    std::vector<int64_t> sh(dims, dims + rank);
    int64_t n = 1;
    for (int64_t d : sh) {
      MNN_REQUIRE(d >= 0 && d <= UINT32_MAX, MNN_ERR_INVALID_ARGUMENT, "bad dimension");
      n *= d;
    }
    MNN_REQUIRE(data || n == 0, MNN_ERR_INVALID_ARGUMENT, "null data");
    (*MW(w))[name] = {std::move(sh), std::vector<float>(data, data + n)};
  });
}
mnn_status mnn_mtla_writer_save(mnn_mtla_writer w, const char* path) {
  return guard([&] {
    MNN_REQUIRE(path, MNN_ERR_INVALID_ARGUMENT, "null path");
    mtla_write(path, *MW(w));
  });
}
mnn_status mnn_mtla_writer_destroy(mnn_mtla_writer w) {
  return guard([&] { delete reinterpret_cast<MtlaTensors*>(w); });
}

mnn_status mnn_transformer_layer_create(mnn_device dev, int embed_dim, int num_heads, int ffn_dim,
                                        float layer_scale, mnn_precision prec, mnn_layer* out) {
  MNN_CREATE(make_transformer_layer(d, embed_dim, num_heads, ffn_dim, layer_scale, prec));
}
mnn_status mnn_cross_transformer_create(mnn_device dev, int embed_dim, int num_heads, int ffn_dim,
                                        int num_layers, float layer_scale, mnn_precision prec,
                                        mnn_layer* out) {
  MNN_CREATE(
      make_cross_transformer(d, embed_dim, num_heads, ffn_dim, num_layers, layer_scale, prec));
}

mnn_status mnn_cross_transformer_encoder_create(mnn_device dev, int embed_dim, int num_heads,
                                                int ffn_dim, int num_layers, mnn_precision prec,
                                                mnn_layer* out) {
  MNN_CREATE(make_cross_transformer_encoder(d, embed_dim, num_heads, ffn_dim, num_layers, prec));
}

mnn_status mnn_layer_destroy(mnn_layer layer) {
  return guard([&] {
    if (!layer) return;
    Layer* l = L(layer);
    l->device()->make_current();
    (void)hipDeviceSynchronize();
    delete l;
  });
}

mnn_status mnn_layer_load_weights(mnn_layer layer, const char* name, const float* data,
                                  size_t count) {
  return guard([&] {
    Layer* l = L(layer);
    MNN_REQUIRE(name, MNN_ERR_INVALID_ARGUMENT, "null name");
    l->device()->check_alive();
    l->device()->make_current();
    l->load(name, data, count);
  });
}

mnn_status mnn_layer_forward(mnn_layer layer, mnn_tensor input, mnn_tensor output,
                             mnn_stream st) {
  return guard([&] {
    Layer* l = L(layer);
    Tensor* in = T(input);
    Tensor* o = T(output);
    Device* d = l->device();
    d->check_alive();
    MNN_REQUIRE(in->dev == d && o->dev == d, MNN_ERR_INVALID_ARGUMENT,
                "tensors and layer on different devices");
    MNN_REQUIRE(in->dtype == MNN_F32 || l->accepts_bf16(), MNN_ERR_INVALID_ARGUMENT,
                l->kind() << ": input must be f32");
    Stream s = resolve_stream(d, st);
    d->make_current();
    l->forward(*in, *o, s);
  });
}

mnn_status mnn_layer_forward_cross(mnn_layer layer, mnn_tensor a, mnn_tensor b, mnn_tensor out_a,
                                   mnn_tensor out_b, mnn_stream st) {
  return guard([&] {
    Layer* l = L(layer);
    Device* d = l->device();
    d->check_alive();
    Tensor* ta = a ? T(a) : nullptr;
    Tensor* tb = b ? T(b) : nullptr;
    Tensor* oa = out_a ? T(out_a) : nullptr;
    Tensor* ob = out_b ? T(out_b) : nullptr;
    for (Tensor* t : {ta, tb, oa, ob})
      if (t) {
        MNN_REQUIRE(t->dev == d, MNN_ERR_INVALID_ARGUMENT, "tensor on another device");
        MNN_REQUIRE(t->dtype == MNN_F32, MNN_ERR_INVALID_ARGUMENT, "tensors must be f32");
      }
    Stream s = resolve_stream(d, st);
    d->make_current();
    l->forward_cross(ta, tb, oa, ob, s);
  });
}

mnn_status mnn_layer_input_shape(mnn_layer layer, int* rank, int64_t* dims) {
  return guard([&] { put_shape(L(layer)->input_shape(), rank, dims); });
}

mnn_status mnn_layer_output_shape(mnn_layer layer, int* rank, int64_t* dims) {
  return guard([&] { put_shape(L(layer)->output_shape(), rank, dims); });
}

mnn_status mnn_layer_infer_output_shape(mnn_layer layer, int in_rank, const int64_t* in_dims,
                                        int* out_rank, int64_t* out_dims) {
  return guard([&] {
    put_shape(L(layer)->infer_output(to_shape(in_rank, in_dims)), out_rank, out_dims);
  });
}

// ------------------------------------------------------------------ sequential
mnn_status mnn_sequential_create(mnn_device dev, mnn_sequential* out) {
  return guard([&] {
    Device* d = D(dev);
    MNN_REQUIRE(out, MNN_ERR_INVALID_ARGUMENT, "null output");
    *out = reinterpret_cast<mnn_sequential>(new Sequential(d));
  });
}

mnn_status mnn_sequential_destroy(mnn_sequential seq) {
  return guard([&] {
    if (seq) delete Q(seq);
  });
}

mnn_status mnn_sequential_add(mnn_sequential seq, mnn_layer layer) {
  return guard([&] { Q(seq)->add(L(layer), true); });
}

mnn_status mnn_sequential_add_unchecked(mnn_sequential seq, mnn_layer layer) {
  return guard([&] { Q(seq)->add(L(layer), false); });
}

mnn_status mnn_sequential_build(mnn_sequential seq) {
  return guard([&] { Q(seq)->build(); });
}

mnn_status mnn_sequential_forward(mnn_sequential seq, mnn_tensor input, mnn_stream st,
                                  mnn_tensor* output) {
  return guard([&] {
    Sequential* q = Q(seq);
    Tensor* in = T(input);
    MNN_REQUIRE(output, MNN_ERR_INVALID_ARGUMENT, "null output");
    in->dev->check_alive();
    Stream s = resolve_stream(in->dev, st);
    in->dev->make_current();
    *output = reinterpret_cast<mnn_tensor>(q->forward(*in, s));
  });
}

mnn_status mnn_sequential_forward_async(mnn_sequential seq, mnn_tensor input, mnn_stream st,
                                        mnn_completion_fn completion, void* user) {
  if (!completion) {
    g_last_error = "null completion";
    return MNN_ERR_INVALID_ARGUMENT;
  }
  const mnn_status status = guard([&] {
    Sequential* q = Q(seq);
    Tensor* in = T(input);
    in->dev->check_alive();
    Stream s = resolve_stream(in->dev, st);
    in->dev->make_current();
    q->forward_async(*in, s, [completion, user](mnn_status status, Tensor* out) {
      completion(user, status, reinterpret_cast<mnn_tensor>(out));
    });
  });
  // not enqueued: the completion still runs exactly once, here, with the failure
  if (status != MNN_OK) completion(user, status, nullptr);
  return status;
}

mnn_status mnn_sequential_layer_at(mnn_sequential seq, int index, mnn_layer* layer) {
  return guard([&] {
    MNN_REQUIRE(layer, MNN_ERR_INVALID_ARGUMENT, "null output");
    *layer = reinterpret_cast<mnn_layer>(Q(seq)->layer_at(index));
  });
}

mnn_status mnn_sequential_buffer_stats(mnn_sequential seq, int* allocated, int* layers) {
  return guard([&] {
    MNN_REQUIRE(allocated && layers, MNN_ERR_INVALID_ARGUMENT, "null output");
    auto st = Q(seq)->buffer_stats();
    *allocated = st.first;
    *layers = st.second;
  });
}

mnn_status mnn_sequential_layer_count(mnn_sequential seq, int* count) {
  return guard([&] {
    MNN_REQUIRE(count, MNN_ERR_INVALID_ARGUMENT, "null output");
    *count = Q(seq)->layer_count();
  });
}

// ------------------------------------------------------------------ diagnostics
mnn_status mnn_debug_mfma_probe(mnn_device dev, int variant, const float* a, const float* b,
                                float* d_out) {
  return guard([&] {
    Device* d = D(dev);
    d->check_alive();
    MNN_REQUIRE(a && b && d_out, MNN_ERR_INVALID_ARGUMENT, "null buffer");
    MNN_REQUIRE(variant >= 0 && variant <= 3, MNN_ERR_INVALID_ARGUMENT, "variant must be 0..3");
    d->make_current();
    const int na = variant < 2 ? 1 : 8;
    const int nd = (variant == 0 || variant == 2) ? 16 : 4;
    float *da, *db, *dd;
    HIP_CHECK(hipMalloc(&da, 64 * na * 4));
    HIP_CHECK(hipMalloc(&db, 64 * na * 4));
    HIP_CHECK(hipMalloc(&dd, 64 * nd * 4));
    HIP_CHECK(hipMemcpy(da, a, 64 * na * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(db, b, 64 * na * 4, hipMemcpyHostToDevice));
    k::mfma_probe(LaunchCtx{d, d->default_stream}, variant, da, db, dd);
    HIP_CHECK(hipStreamSynchronize(d->default_stream));
    HIP_CHECK(hipMemcpy(d_out, dd, 64 * nd * 4, hipMemcpyDeviceToHost));
    (void)hipFree(da);
    (void)hipFree(db);
    (void)hipFree(dd);
  });
}

mnn_status mnn_debug_enc_conv_plan(int in_channels, int out_channels, int64_t out_length,
                                   int batch, int gn_finish, int* splits, int* tile_m,
                                   int* tile_n) {
  return guard([&] {
    MNN_REQUIRE(splits && tile_m && tile_n && in_channels > 0 && out_channels > 0 &&
                    out_length > 0 && batch > 0,
                MNN_ERR_INVALID_ARGUMENT, "invalid argument");
    k::enc_conv_plan_info(in_channels, out_channels, out_length, batch, gn_finish != 0, splits,
                          tile_m, tile_n);
  });
}

mnn_status mnn_debug_set_launch_log(mnn_device dev, int enable) {
  return guard([&] {
    Device* d = D(dev);
    std::lock_guard<std::mutex> lk(d->timing_mu);
    if (enable) d->launches.clear();
    d->launch_log.store(enable != 0);
  });
}

mnn_status mnn_debug_set_grid_spin_limit(mnn_device dev, int polls, int* previous) {
  return guard([&] {
    MNN_REQUIRE(polls >= 0, MNN_ERR_INVALID_ARGUMENT, "polls must be >= 0, got " << polls);
    Device* d = D(dev);
    const int old = d->grid_spin_limit.exchange(polls);
    if (previous) *previous = old;
  });
}

mnn_status mnn_debug_kernel_timing_table(mnn_device dev, char* buf, size_t cap, size_t* needed) {
  return guard([&] {
    MNN_REQUIRE(needed, MNN_ERR_INVALID_ARGUMENT, "needed is required");
    Device* d = D(dev);
    d->make_current();
    d->resolve_timers();
    std::ostringstream os;
    {
      std::lock_guard<std::mutex> lk(d->timing_mu);
      for (auto& kv : d->stats) os << kv.first << ' ' << kv.second.first << ' ' << kv.second.second << '\n';
    }
    const std::string text = os.str();
    *needed = text.size() + 1;
    if (!buf) return;
    MNN_REQUIRE(cap >= text.size() + 1, MNN_ERR_BUFFER_SIZE_MISMATCH,
                "kernel timing table needs " << text.size() + 1 << " bytes");
    std::memcpy(buf, text.c_str(), text.size() + 1);
  });
}

mnn_status mnn_debug_stream_mark(mnn_stream st, int index) {
  return guard([&] {
    MNN_REQUIRE(st, MNN_ERR_INVALID_ARGUMENT, "a stream is required");
    MNN_REQUIRE(index >= 0 && index < 65536, MNN_ERR_INVALID_ARGUMENT,
                "mark index must be in [0, 65536), got " << index);
    Stream* s = S(st);
    s->dev->make_current();
    std::lock_guard<std::mutex> lk(g_marks_mu);
    auto& v = g_marks[s];
    while ((int)v.size() <= index) {
      hipEvent_t e;
      HIP_CHECK(hipEventCreate(&e));
      v.push_back(e);
    }
    HIP_CHECK(hipEventRecord(v[index], s->s));
  });
}

mnn_status mnn_debug_stream_mark_elapsed(mnn_stream st, int from, int to, float* ms) {
  return guard([&] {
    MNN_REQUIRE(st && ms, MNN_ERR_INVALID_ARGUMENT, "a stream and an output are required");
    Stream* s = S(st);
    s->dev->make_current();
    std::lock_guard<std::mutex> lk(g_marks_mu);
    auto it = g_marks.find(s);
    MNN_REQUIRE(it != g_marks.end() && from >= 0 && to >= 0 && from < (int)it->second.size() &&
                    to < (int)it->second.size(),
                MNN_ERR_INVALID_ARGUMENT, "mark " << from << " or " << to << " never recorded");
    HIP_CHECK(hipEventSynchronize(it->second[to]));
    HIP_CHECK(hipEventElapsedTime(ms, it->second[from], it->second[to]));
  });
}

mnn_status mnn_debug_empty_launch(mnn_stream st) {
  return guard([&] {
    MNN_REQUIRE(st, MNN_ERR_INVALID_ARGUMENT, "a stream is required");
    Stream* s = S(st);
    s->dev->check_alive();
    s->dev->make_current();
    k::floor_empty(LaunchCtx{s->dev, s->s});
  });
}

mnn_status mnn_debug_stream_rw(mnn_tensor src, int64_t read_bytes, mnn_tensor dst,
                               int64_t write_bytes, mnn_stream st) {
  return guard([&] {
    Tensor* a = T(src);
    Tensor* b = T(dst);
    MNN_REQUIRE(a->dev == b->dev, MNN_ERR_INVALID_ARGUMENT, "tensors on different devices");
    MNN_REQUIRE(read_bytes >= 0 && write_bytes >= 0 && read_bytes % 16 == 0 &&
                    write_bytes % 16 == 0 && (size_t)read_bytes <= a->bytes &&
                    (size_t)write_bytes <= b->bytes,
                MNN_ERR_INVALID_ARGUMENT, "byte counts must be multiples of 16 within the tensors");
    a->dev->check_alive();
    Stream s = resolve_stream(a->dev, st);
    a->dev->make_current();
    k::floor_stream(LaunchCtx{s.dev, s.s}, a->data, read_bytes, b->data, write_bytes);
  });
}

mnn_status mnn_debug_device_allocations(int64_t* count) {
  return guard([&] {
    MNN_REQUIRE(count, MNN_ERR_INVALID_ARGUMENT, "count is required");
    *count = g_device_allocations.load();
  });
}

mnn_status mnn_debug_launch_log(mnn_device dev, char* buf, size_t cap, size_t* needed) {
  return guard([&] {
    MNN_REQUIRE(needed, MNN_ERR_INVALID_ARGUMENT, "needed is required");
    Device* d = D(dev);
    std::string all;
    {
      std::lock_guard<std::mutex> lk(d->timing_mu);
      for (const std::string& l : d->launches) all += l + "\n";
    }
    *needed = all.size() + 1;
    MNN_REQUIRE(buf && cap >= all.size() + 1, MNN_ERR_BUFFER_SIZE_MISMATCH,
                "launch log needs " << all.size() + 1 << " bytes");
    std::memcpy(buf, all.c_str(), all.size() + 1);
  });
}

}  // extern "C"
