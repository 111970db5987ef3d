// One-wave MFMA probe: runs a single matrix instruction on per-lane operands and returns the
// raw accumulator registers, so tests can confirm the lane layouts the GEMM and attention
// kernels are written against.
#include "device_utils.hpp"
#include "kernels.hpp"

namespace mnn {
namespace k {

using namespace dev;

namespace {

__global__ __launch_bounds__(64) void mfma_probe_kernel(int variant, const float* __restrict__ a,
                                                        const float* __restrict__ b,
                                                        float* __restrict__ d) {
  const int l = threadIdx.x;
  if (variant == 0) {
    floatx16 acc = {};
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[l], b[l], acc, 0, 0, 0);
    for (int v = 0; v < 16; ++v) d[l * 16 + v] = acc[v];
  } else if (variant == 1) {
    floatx4 acc = {};
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[l], b[l], acc, 0, 0, 0);
    for (int v = 0; v < 4; ++v) d[l * 4 + v] = acc[v];
  } else {
    shortx8 av, bv;
    for (int j = 0; j < 8; ++j) {
      av[j] = (short)f32_to_bf16_bits(a[l * 8 + j]);
      bv[j] = (short)f32_to_bf16_bits(b[l * 8 + j]);
    }
    bf16x8 ab = __builtin_bit_cast(bf16x8, av);
    bf16x8 bb = __builtin_bit_cast(bf16x8, bv);
    if (variant == 2) {
      floatx16 acc = {};
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ab, bb, acc, 0, 0, 0);
      for (int v = 0; v < 16; ++v) d[l * 16 + v] = acc[v];
    } else {
      floatx4 acc = {};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, bb, acc, 0, 0, 0);
      for (int v = 0; v < 4; ++v) d[l * 4 + v] = acc[v];
    }
  }
}

}  // namespace

void mfma_probe(const LaunchCtx& c, int variant, const float* a, const float* b, float* d) {
  MNN_REQUIRE(variant >= 0 && variant <= 3, MNN_ERR_INVALID_ARGUMENT,
              "mfma probe variant must be 0..3");
  launch(c, "mfma_probe", mfma_probe_kernel, dim3(1), dim3(64), 0, variant, a, b, d);
}

}  // namespace k
}  // namespace mnn
