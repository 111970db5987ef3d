// Elementwise kernels: GELU, other activations, GLU, byte copy.
// HBM-bound: 16-byte vector loads/stores where the buffer allows, grid-stride loops,
// every access bounds-checked (the reference GELU kernel has no bounds check,
// Activations.swift:124-137; here the tail is handled explicitly).
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t items) {
  int64_t g = (items + kThreads - 1) / kThreads;
  if (g > 65535 * 8) g = 65535 * 8;  // grid-stride beyond this
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

__global__ __launch_bounds__(kThreads) void gelu_kernel(const float* __restrict__ x,
                                                        float* __restrict__ y, int64_t n,
                                                        int clamp10, int vec) {
  const int64_t n4 = vec ? (n >> 2) : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* y4 = reinterpret_cast<float4*>(y);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    float4 v = x4[i];
    if (clamp10) {
      v.x = gelu_clamped(v.x); v.y = gelu_clamped(v.y);
      v.z = gelu_clamped(v.z); v.w = gelu_clamped(v.w);
    } else {
      v.x = gelu_tanh(v.x); v.y = gelu_tanh(v.y);
      v.z = gelu_tanh(v.z); v.w = gelu_tanh(v.w);
    }
    y4[i] = v;
  }
  for (int64_t i = (n4 << 2) + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = clamp10 ? gelu_clamped(x[i]) : gelu_tanh(x[i]);
}

__global__ __launch_bounds__(kThreads) void act_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t n, int act) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = apply_act(x[i], act);
}

__global__ __launch_bounds__(kThreads) void glu_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t half) {
  const int64_t b = blockIdx.y;
  const float* xa = x + b * 2 * half;
  const float* xb = xa + half;
  float* yb = y + b * half;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < half; i += stride)
    yb[i] = xa[i] * stable_sigmoid(xb[i]);
}

__global__ __launch_bounds__(kThreads) void copy_kernel(const uint8_t* __restrict__ s,
                                                        uint8_t* __restrict__ d, int64_t bytes,
                                                        int vec) {
  const int64_t n16 = vec ? (bytes >> 4) : 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint4* s4 = reinterpret_cast<const uint4*>(s);
  uint4* d4 = reinterpret_cast<uint4*>(d);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    d4[i] = s4[i];
  for (int64_t i = (n16 << 4) + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes;
       i += stride)
    d[i] = s[i];
}

__global__ __launch_bounds__(kThreads) void zero_u32_kernel(unsigned* __restrict__ d, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) d[i] = 0u;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

__global__ __launch_bounds__(kThreads) void f32_to_bf16_kernel(const float* __restrict__ x,
                                                               uint16_t* __restrict__ y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = f32_to_bf16_bits(x[i]);
}

__global__ __launch_bounds__(kThreads) void bf16_to_f32_kernel(const uint16_t* __restrict__ x,
                                                               float* __restrict__ y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = __uint_as_float((uint32_t)x[i] << 16);
}

}  // namespace

void f32_to_bf16(const LaunchCtx& c, const float* x, uint16_t* y, int64_t n) {
  if (n <= 0) return;
  launch(c, "f32_to_bf16", f32_to_bf16_kernel, dim3(grid_for(n)), dim3(kThreads), 0, x, y, n);
}

void bf16_to_f32(const LaunchCtx& c, const uint16_t* x, float* y, int64_t n) {
  if (n <= 0) return;
  launch(c, "bf16_to_f32", bf16_to_f32_kernel, dim3(grid_for(n)), dim3(kThreads), 0, x, y, n);
}

void gelu(const LaunchCtx& c, const float* x, float* y, int64_t n, bool clamp10) {
  if (n <= 0) return;
  const int vec = aligned16(x) && aligned16(y);
  launch(c, "gelu_f32", gelu_kernel, dim3(grid_for(vec ? (n + 3) / 4 : n)), dim3(kThreads), 0, x,
         y, n, (int)clamp10, vec);
}

void activation(const LaunchCtx& c, const float* x, float* y, int64_t n, int act) {
  if (n <= 0) return;
  if (act == 3) return gelu(c, x, y, n, false);
  launch(c, "activation_f32", act_kernel, dim3(grid_for(n)), dim3(kThreads), 0, x, y, n, act);
}

void glu(const LaunchCtx& c, const float* x, float* y, int64_t batch, int64_t half) {
  if (half <= 0 || batch <= 0) return;
  unsigned gx = grid_for(half);
  if (gx > 65535) gx = 65535;
  launch(c, "glu_f32", glu_kernel, dim3(gx, (unsigned)batch), dim3(kThreads), 0, x, y, half);
}

// Floor kernels (measurement aids): an empty launch, and a streaming pass that reads rd and
// writes wr 16-byte vectors (a copy where both apply, zeros past the read range, reads past the
// write range kept alive by an empty asm use), four vectors per thread and iteration with every
// load issued before the stores.
__global__ void floor_empty_kernel() {}

__global__ __launch_bounds__(kThreads) void floor_stream_kernel(const float4* __restrict__ src,
                                                                int64_t rd,
                                                                float4* __restrict__ dst,
                                                                int64_t wr) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t n = rd > wr ? rd : wr;
  for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < n; i0 += 4 * stride) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = i0 + u * stride;
      v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (rd > 0) {
        const float4 t = src[i < rd ? i : rd - 1];
        if (i < rd) v[u] = t;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = i0 + u * stride;
      if (i < wr) dst[i] = v[u];
      else asm volatile("" ::"v"(v[u].x), "v"(v[u].y), "v"(v[u].z), "v"(v[u].w));
    }
  }
}

void floor_empty(const LaunchCtx& c) {
  launch(c, "floor_empty", floor_empty_kernel, dim3(1), dim3(64), 0);
}

void floor_stream(const LaunchCtx& c, const void* src, int64_t read_bytes, void* dst,
                  int64_t write_bytes) {
  const int64_t rd = read_bytes / 16, wr = write_bytes / 16;
  const int64_t n = rd > wr ? rd : wr;
  if (n <= 0) return;
  launch(c, "floor_stream", floor_stream_kernel, dim3(grid_for((n + 3) / 4)), dim3(kThreads), 0,
         static_cast<const float4*>(src), rd, static_cast<float4*>(dst), wr);
}

void zero_u32(const LaunchCtx& c, unsigned* d, int64_t n) {
  if (n <= 0) return;
  launch(c, "zero_u32", zero_u32_kernel, dim3(grid_for(n)), dim3(kThreads), 0, d, n);
}

void copy_bytes(const LaunchCtx& c, const void* src, void* dst, int64_t bytes) {
  if (bytes <= 0) return;
  const int vec = aligned16(src) && aligned16(dst);
  launch(c, "copy_bytes", copy_kernel, dim3(grid_for(vec ? (bytes + 15) / 16 : bytes)),
         dim3(kThreads), 0, static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), bytes,
         vec);
}

}  // namespace k
}  // namespace mnn
