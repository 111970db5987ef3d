// Device-side helpers shared by the kernels: activations, wave64 reductions, bf16 rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mnn {
namespace dev {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short shortx8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// sigmoid with the +-88 clamp of the reference's stable_sigmoid (Shaders/NN.metal:32-47);
// 1/(1+e^-x) and e^x/(1+e^x) are the same number, so one branchless form suffices.
__device__ __forceinline__ float stable_sigmoid(float x) {
  x = fminf(fmaxf(x, -88.f), 88.f);
  return 1.f / (1.f + __expf(-x));
}

// tanh-approximation GELU: 0.5 x (1 + tanh(u)), u = sqrt(2/pi)(x + 0.044715 x^3).
// Evaluated as x * sigmoid(2u), the same function (1 + tanh(u) = 2 sigmoid(2u)), which needs one
// exp and no cancellation near u = 0. For |x| large the exp saturates to 0 / inf and the result
// is x / -0, as the clamped reference form (Activations.swift:124-137) gives.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  float u = k0 * (x + k1 * x * x * x);
  return x / (1.f + __expf(-2.f * u));
}

// Reference GELU layer semantics: x > 10 -> x, x < -10 -> 0, else the tanh formula.
__device__ __forceinline__ float gelu_clamped(float x) {
  return x > 10.f ? x : (x < -10.f ? 0.f : gelu_tanh(x));
}

__device__ __forceinline__ float apply_act(float x, int act) {
  switch (act) {
    case 1: return fmaxf(x, 0.f);
    case 2: return x >= 0.f ? x : 0.01f * x;
    case 3: return gelu_tanh(x);
    case 4: return x * stable_sigmoid(x);
    case 5: return stable_sigmoid(x);
    case 6: return tanhf(x);
    default: return x;
  }
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Workgroup-wide (count, mean, M2) of per-thread values, merged with Chan's formula.
// Each thread passes its own (n, mean, m2); thread 0 receives the workgroup result.
// `red` must hold 3 * (blockDim.x / 64) floats of LDS.
__device__ __forceinline__ void block_welford(float& n, float& mean, float& m2, float* red) {
  // wave level: tree over lanes
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float n2 = __shfl_xor(n, off, kWave);
    float mean2 = __shfl_xor(mean, off, kWave);
    float m22 = __shfl_xor(m2, off, kWave);
    float nt = n + n2;
    if (nt > 0.f) {
      float d = mean2 - mean;
      float w = n2 / nt;
      mean = mean + d * w;
      m2 = m2 + m22 + d * d * n * w;
    }
    n = nt;
  }
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) {
    red[wid * 3 + 0] = n;
    red[wid * 3 + 1] = mean;
    red[wid * 3 + 2] = m2;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    n = red[0];
    mean = red[1];
    m2 = red[2];
    for (int w = 1; w < nw; ++w) {
      float n2 = red[w * 3 + 0], mean2 = red[w * 3 + 1], m22 = red[w * 3 + 2];
      float nt = n + n2;
      if (nt > 0.f) {
        float d = mean2 - mean;
        float wt = n2 / nt;
        mean = mean + d * wt;
        m2 = m2 + m22 + d * d * n * wt;
      }
      n = nt;
    }
  }
}

}  // namespace dev
}  // namespace mnn
