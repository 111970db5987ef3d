// Device timing hooks, tensors and Sequential.
#include <algorithm>
#include <thread>

#include "layers.hpp"

namespace mnn {

size_t dtype_size(mnn_dtype t) { return t == MNN_BF16 ? 2 : 4; }

std::atomic<int64_t> g_device_allocations{0};

// ------------------------------------------------------------------ kernel timing
void timing_begin(const LaunchCtx& c, const char*, hipEvent_t* e0, hipEvent_t* e1) {
  Device* d = c.dev;
  std::lock_guard<std::mutex> lk(d->timing_mu);
  if (!d->event_pool.empty()) {
    *e0 = d->event_pool.back().first;
    *e1 = d->event_pool.back().second;
    d->event_pool.pop_back();
  } else {
    HIP_CHECK(hipEventCreate(e0));
    HIP_CHECK(hipEventCreate(e1));
  }
}

void timing_end(const LaunchCtx& c, const char* name, hipEvent_t e0, hipEvent_t e1) {
  Device* d = c.dev;
  std::lock_guard<std::mutex> lk(d->timing_mu);
  d->pending.push_back(KernelTimer{name, e0, e1});
}

void log_launch(const LaunchCtx& c, const char* name, dim3 grid, dim3 block) {
  Device* d = c.dev;
  std::lock_guard<std::mutex> lk(d->timing_mu);
  d->launches.push_back(std::string(name) + " " + std::to_string(grid.x) + " " +
                        std::to_string(grid.y) + " " + std::to_string(grid.z) + " " +
                        std::to_string(block.x));
}

void Device::resolve_timers() {
  std::lock_guard<std::mutex> lk(timing_mu);
  for (auto& t : pending) {
    HIP_CHECK(hipEventSynchronize(t.stop));
    float ms = 0.f;
    HIP_CHECK(hipEventElapsedTime(&ms, t.start, t.stop));
    auto& st = stats[t.name];
    st.first += 1;
    st.second += ms;
    event_pool.emplace_back(t.start, t.stop);
  }
  pending.clear();
}

// ------------------------------------------------------------------ tensors
Tensor* tensor_create(Device* d, mnn_dtype dt, const Shape& shape) {
  MNN_REQUIRE(!shape.empty() && shape.size() <= MNN_MAX_RANK, MNN_ERR_INVALID_ARGUMENT,
              "tensor rank must be 1.." << MNN_MAX_RANK);
  for (auto v : shape)
    MNN_REQUIRE(v >= 0, MNN_ERR_INVALID_ARGUMENT, "negative dimension in " << shape_str(shape));
  auto t = std::make_unique<Tensor>();
  t->dev = d;
  t->dtype = dt;
  t->shape = shape;
  t->bytes = (size_t)numel(shape) * dtype_size(dt);
  d->make_current();
  if (t->bytes) {
    HIP_CHECK(hipMalloc(&t->data, t->bytes));
    g_device_allocations.fetch_add(1, std::memory_order_relaxed);
    HIP_CHECK(hipMemsetAsync(t->data, 0, t->bytes, d->default_stream));
    HIP_CHECK(hipStreamSynchronize(d->default_stream));
  }
  return t.release();
}

void tensor_destroy(Tensor* t) {
  if (!t) return;
  if (t->owns && t->data) {
    t->dev->make_current();
    (void)hipFree(t->data);
  }
  delete t;
}

// ------------------------------------------------------------------ Sequential
namespace {
// The model whose forwardAsync completion runs on this thread, if any.
thread_local const Sequential* tl_completing = nullptr;
}  // namespace

Sequential::~Sequential() {
  {  // completion threads of forward_async use `this` until their callback has returned; a
     // completion that destroys its own model waits only for the model's other threads
    const int self = tl_completing == this ? 1 : 0;
    std::unique_lock<std::mutex> lk(async_->mu);
    async_->cv.wait(lk, [&] { return async_->threads <= self; });
  }
  free_plans();
}

void Sequential::free_plans() {
  for (auto& kv : plans_)
    for (Tensor* t : kv.second.buffers) tensor_destroy(t);
  plans_.clear();
  last_plan_ = nullptr;
}

// Model.swift:74-116: the new layer's input must match the previous output, 0 matching anything.
void Sequential::add(Layer* l, bool checked) {
  MNN_REQUIRE(l, MNN_ERR_INVALID_ARGUMENT, "null layer");
  std::lock_guard<std::mutex> lk(forward_mu_);
  if (checked && !layers_.empty()) {
    const Shape prev = layers_.back()->output_shape();
    const Shape next = l->input_shape();
    bool ok = prev.size() == next.size();
    for (size_t i = 0; ok && i < prev.size(); ++i)
      ok = prev[i] == next[i] || prev[i] == 0 || next[i] == 0;
    MNN_REQUIRE(ok, MNN_ERR_SHAPE_MISMATCH,
                "Layer " << layers_.size() << " shape mismatch: expected input " << shape_str(prev)
                         << ", got " << shape_str(next));
  }
  layers_.push_back(l);
  built_ = false;
  free_plans();
}

void Sequential::build() {
  std::lock_guard<std::mutex> lk(forward_mu_);
  free_plans();
  if (layers_.empty()) return;
  built_ = true;
  // Fully static models get their buffers now, like the reference; dynamic ones on first use.
  const Shape in = layers_[0]->input_shape();
  if (std::find(in.begin(), in.end(), 0) == in.end()) last_plan_ = plan_for(in);
}

Sequential::Plan* Sequential::plan_for(const Shape& in) {
  auto it = plans_.find(in);
  if (it != plans_.end()) return &it->second;
  Plan plan;
  Shape cur = in;
  for (Layer* l : layers_) {
    cur = l->infer_output(cur);
    plan.shapes.push_back(cur);
  }
  // Ping-pong reuse (Model.swift:157-195): reuse a same-shape buffer whose last user is at
  // least two layers back, else allocate.
  std::map<Shape, std::vector<std::pair<int, int>>> by_shape;  // shape -> (buffer, last use)
  for (int i = 0; i < (int)plan.shapes.size(); ++i) {
    auto& cands = by_shape[plan.shapes[i]];
    int reuse = -1;
    for (auto& c : cands)
      if (i - c.second >= 2) {
        reuse = c.first;
        c.second = i;
        break;
      }
    if (reuse < 0) {
      reuse = (int)plan.buffers.size();
      plan.buffers.push_back(tensor_create(dev_, MNN_F32, plan.shapes[i]));
      cands.emplace_back(reuse, i);
    }
    plan.buffer_index.push_back(reuse);
  }
  auto res = plans_.emplace(in, std::move(plan));
  return &res.first->second;
}

Tensor* Sequential::forward(const Tensor& in, Stream& s) {
  std::lock_guard<std::mutex> lk(forward_mu_);
  return forward_locked(in, s);
}

Tensor* Sequential::forward_locked(const Tensor& in, Stream& s) {
  MNN_REQUIRE(!layers_.empty(), MNN_ERR_EMPTY_MODEL, "Cannot run inference on empty model");
  // Model.swift:228-229 (and forwardAsync, :293-298): invalidConfiguration
  MNN_REQUIRE(built_, MNN_ERR_INVALID_CONFIGURATION, "Model not built. Call build() first.");
  // Model.swift:231-236 compares the whole shape; here leading batch dimensions are allowed
  // (layers take [C, L] or [B, C, L], [F] or [N, F]) and 0 in the declared shape is dynamic.
  const Shape expect = layers_[0]->input_shape();
  bool ok = in.shape.size() >= expect.size();
  const size_t off = ok ? in.shape.size() - expect.size() : 0;
  for (size_t i = 0; ok && i < expect.size(); ++i)
    ok = expect[i] == 0 || expect[i] == in.shape[off + i];
  MNN_REQUIRE(ok, MNN_ERR_INPUT_SHAPE_MISMATCH,
              "Model input shape mismatch: expected " << shape_str(expect) << ", got "
                                                      << shape_str(in.shape));
  Plan* p = plan_for(in.shape);
  last_plan_ = p;
  const Tensor* cur = &in;
  for (size_t i = 0; i < layers_.size();) {
    const int n = fused_chain_length(layers_, i);
    Tensor* out = p->buffers[p->buffer_index[i + n - 1]];
    if (n > 1) {
      run_fused_chain(layers_, i, n, *cur, *p->buffers[p->buffer_index[i]], *out, s);
    } else {
      layers_[i]->forward(*cur, *out, s);
    }
    cur = out;
    i += n;
  }
  return p->buffers[p->buffer_index.back()];
}

void Sequential::forward_async(const Tensor& in, Stream& s, Completion done) {
  bool expected = false;
  // Model.swift:272-283: concurrent forwardAsync calls would corrupt the shared buffers
  MNN_REQUIRE(async_in_flight_.compare_exchange_strong(expected, true),
              MNN_ERR_INVALID_CONFIGURATION,
              "Concurrent forwardAsync() calls not supported. Use separate Sequential instances.");
  Tensor* out = nullptr;
  hipEvent_t ev = nullptr;
  try {
    std::lock_guard<std::mutex> lk(forward_mu_);
    out = forward_locked(in, s);
    dev_->make_current();
    HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    HIP_CHECK(hipEventRecord(ev, s.s));
  } catch (...) {
    if (ev) (void)hipEventDestroy(ev);
    async_in_flight_ = false;
    throw;
  }
  const int ordinal = dev_->ordinal;
  std::shared_ptr<AsyncState> st = async_;
  {
    std::lock_guard<std::mutex> lk(st->mu);
    ++st->threads;
  }
  try {
    std::thread([this, st, ev, out, ordinal, done = std::move(done)]() {
      (void)hipSetDevice(ordinal);
      const hipError_t e = hipEventSynchronize(ev);
      (void)hipEventDestroy(ev);
      async_in_flight_ = false;  // as the reference, cleared before the completion runs
      tl_completing = this;
      done(e == hipSuccess ? MNN_OK : MNN_ERR_GPU_EXECUTION, e == hipSuccess ? out : nullptr);
      tl_completing = nullptr;
      // `this` may be gone now (the completion may destroy the model): only `st` is used
      std::lock_guard<std::mutex> lk(st->mu);
      --st->threads;
      st->cv.notify_all();
    }).detach();
  } catch (...) {  // no thread: undo the bookkeeping so the model stays usable and destroyable
    {
      std::lock_guard<std::mutex> lk(st->mu);
      --st->threads;
    }
    st->cv.notify_all();
    (void)hipEventDestroy(ev);
    async_in_flight_ = false;
    fail(MNN_ERR_INVALID_CONFIGURATION, "forwardAsync: could not start the completion thread");
  }
}

Layer* Sequential::layer_at(int index) const {
  return index >= 0 && index < (int)layers_.size() ? layers_[index] : nullptr;
}

std::pair<int, int> Sequential::buffer_stats() const {
  return {last_plan_ ? (int)last_plan_->buffers.size() : 0, (int)layers_.size()};
}

}  // namespace mnn
