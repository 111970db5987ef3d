// Runtime core shared by the kernels, the layers and the C ABI.
// Device / Stream / Tensor replace AudioDevice, ComputeContext and Tensor of the reference
// (Sources/MetalAudioKit/Core/AudioDevice.swift, Core/ComputeContext.swift, Buffers/Tensor.swift).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "mnn.h"

namespace mnn {

// ------------------------------------------------------------------ errors
struct Error {
  mnn_status code;
  std::string msg;
};

[[noreturn]] inline void fail(mnn_status code, const std::string& msg) { throw Error{code, msg}; }

// Number of device allocations the library has made (tensors, weights, workspaces), process-wide;
// read through mnn_debug_device_allocations so tests can check that a path allocates nothing.
extern std::atomic<int64_t> g_device_allocations;

#define MNN_REQUIRE(cond, code, msg_expr)                      \
  do {                                                         \
    if (!(cond)) {                                             \
      std::ostringstream _os;                                  \
      _os << msg_expr;                                         \
      ::mnn::fail(code, _os.str());                            \
    }                                                          \
  } while (0)

#define HIP_CHECK(expr)                                                                   \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess) {                                                               \
      ::mnn::fail(_e == hipErrorOutOfMemory ? MNN_ERR_OUT_OF_MEMORY : MNN_ERR_GPU_EXECUTION, \
                  std::string(#expr) + ": " + hipGetErrorString(_e));                    \
    }                                                                                     \
  } while (0)

using Shape = std::vector<int64_t>;

inline int64_t numel(const Shape& s) {
  int64_t n = 1;
  for (auto d : s) n *= d;
  return n;
}

inline std::string shape_str(const Shape& s) {
  std::ostringstream os;
  os << "[";
  for (size_t i = 0; i < s.size(); ++i) os << (i ? ", " : "") << s[i];
  os << "]";
  return os.str();
}

// ------------------------------------------------------------------ device
struct KernelTimer {
  std::string name;
  hipEvent_t start, stop;
};

struct Device {
  int ordinal = 0;
  hipDeviceProp_t props{};
  hipStream_t default_stream = nullptr;
  std::atomic<bool> lost{false};
  // kernel timing
  bool timing = false;
  std::mutex timing_mu;
  std::vector<KernelTimer> pending;                      // events not yet resolved
  std::map<std::string, std::pair<int64_t, double>> stats;  // name -> (launches, ms)
  std::vector<std::pair<hipEvent_t, hipEvent_t>> event_pool;
  // launch log (a profiling aid): one line per launch, "name grid.x grid.y grid.z block.x"
  std::atomic<bool> launch_log{false};
  std::vector<std::string> launches;  // guarded by timing_mu
  // polls a workgroup makes in a grid-wide wait before it computes what it waits for itself
  std::atomic<int> grid_spin_limit{1 << 16};

  void make_current() const { (void)hipSetDevice(ordinal); }
  void check_alive() const {
    MNN_REQUIRE(!lost.load(), MNN_ERR_DEVICE_LOST, "device " << ordinal << " marked lost");
  }
  void resolve_timers();  // waits for pending events and folds them into stats
};

struct Stream {
  Device* dev = nullptr;
  hipStream_t s = nullptr;
  bool owned = false;
};

// ------------------------------------------------------------------ tensor
struct Tensor {
  Device* dev = nullptr;
  mnn_dtype dtype = MNN_F32;
  Shape shape;
  void* data = nullptr;
  size_t bytes = 0;
  bool owns = true;

  int64_t count() const { return numel(shape); }
  float* f32() const { return static_cast<float*>(data); }
};

size_t dtype_size(mnn_dtype t);

// Device buffer with RAII ownership, used for weights and workspaces.
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  // Grows (never shrinks) to at least `n` bytes; contents are not preserved on growth.
  void reserve(size_t n) {
    if (n <= bytes) return;
    release();
    HIP_CHECK(hipMalloc(&ptr, n));
    g_device_allocations.fetch_add(1, std::memory_order_relaxed);
    bytes = n;
  }
  float* f32() const { return static_cast<float*>(ptr); }
  template <class T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

// ------------------------------------------------------------------ launches
// Every library kernel is launched through `launch`, which checks the launch and, when the
// device's kernel timing is on, brackets it with events on the launch stream.
struct LaunchCtx {
  Device* dev;
  hipStream_t stream;
};

// Kernel timing: timing_begin hands out a pair of events (pooled) that the launch passes to
// hipExtLaunchKernel, which stamps them at the kernel's start and end; timing_end queues the pair
// for resolution under `name`.
void timing_begin(const LaunchCtx& c, const char* name, hipEvent_t* ev_start, hipEvent_t* ev_stop);
void timing_end(const LaunchCtx& c, const char* name, hipEvent_t ev_start, hipEvent_t ev_stop);
void log_launch(const LaunchCtx& c, const char* name, dim3 grid, dim3 block);

template <typename Kernel, typename... Args>
inline void launch(const LaunchCtx& c, const char* name, Kernel k, dim3 grid, dim3 block,
                   size_t shmem, Args... args) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return;
  if (c.dev && c.dev->launch_log.load(std::memory_order_relaxed)) log_launch(c, name, grid, block);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (c.dev && c.dev->timing) {
    // the events take the kernel's own start / end timestamps (no extra packets around it)
    timing_begin(c, name, &e0, &e1);
    hipExtLaunchKernelGGL(k, grid, block, (std::uint32_t)shmem, c.stream, e0, e1, 0u, args...);
  } else {
    hipLaunchKernelGGL(k, grid, block, shmem, c.stream, args...);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    fail(err == hipErrorNoBinaryForGpu || err == hipErrorInvalidDeviceFunction
             ? MNN_ERR_PIPELINE_CREATION_FAILED
             : MNN_ERR_GPU_EXECUTION,
         std::string("launch of ") + name + " failed: " + hipGetErrorString(err));
  if (e0) timing_end(c, name, e0, e1);
}

inline unsigned cdiv(int64_t a, int64_t b) { return static_cast<unsigned>((a + b - 1) / b); }

}  // namespace mnn
