// Memory-bound helpers of the triangle-attention block: the additive mask
// bias, the standalone C128 pair LayerNorm and the sigmoid output gate.
#include "common.hpp"
#include "kernels.hpp"

#include <atomic>
#include <cmath>

namespace fpx {
namespace {

// mbias[i][k] (i < n, k < np) followed by zero rows [n, np) of each head of
// the triangle bias.  inf * (mask - 1) is evaluated as two rounded fp32 ops,
// as the native expression is (patches/protenix/0005-*.patch:36-39).
template <typename BiasT>
__global__ void mask_bias_kernel(const float* __restrict__ mask, int64_t ms_i, int64_t ms_j, int n,
                                 int np, float inf, float* __restrict__ mbias,
                                 BiasT* __restrict__ tri_bias) {
  const int64_t head_rows = (int64_t)(np - n) * np;
  const int64_t total = (int64_t)n * np + kHeads * head_rows;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    if (idx < (int64_t)n * np) {
      const int i = (int)(idx / np);
      const int k = (int)(idx % np);
      float v = -INFINITY;
      if (k < n) v = mask ? inf * (mask[i * ms_i + k * ms_j] - 1.0f) : 0.0f;
      mbias[idx] = v;
    } else {
      const int64_t r = idx - (int64_t)n * np;
      const int64_t h = r / head_rows;
      const int64_t rest = r % head_rows;
      tri_bias[(h * np + n) * np + rest] = (BiasT)0.0f;
    }
  }
}

// One wavefront per 128-channel row: lane holds channels 2*lane, 2*lane+1,
// one 512-byte coalesced read and write per row.  Mean, then the biased
// variance of the centred values, both as register-level wave reductions of
// pivot-shifted values (ln_stats_c128).
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* __restrict__ x,
                                                         int64_t rows_i, int64_t rows_j,
                                                         int64_t xs_i, int64_t xs_j,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ b, float eps,
                                                         float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows_i * rows_j) return;
  const int64_t i = row / rows_j;
  const int64_t j = row % rows_j;
  const f32x2 v = *(const f32x2*)(x + i * xs_i + j * xs_j + 2 * lane);
  float d0, d1, rstd;
  ln_stats_c128(v.x, v.y, eps, d0, d1, rstd);
  f32x2 gw = {1.f, 1.f}, gb = {0.f, 0.f};
  if (w) gw = *(const f32x2*)(w + 2 * lane);
  if (b) gb = *(const f32x2*)(b + 2 * lane);
  *(f32x2*)(y + row * kChannels + 2 * lane) =
      f32x2{d0 * rstd * gw.x + gb.x, d1 * rstd * gw.y + gb.y};
}

__global__ __launch_bounds__(256) void sigmoid_mul_kernel(const f32x4* __restrict__ gate,
                                                          const f32x4* __restrict__ value,
                                                          f32x4* __restrict__ out,
                                                          int64_t count4) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= count4) return;
  const f32x4 g = gate[idx];
  const f32x4 v = value[idx];
  out[idx] = f32x4{v.x * sigmoidf_(g.x), v.y * sigmoidf_(g.y), v.z * sigmoidf_(g.z),
                   v.w * sigmoidf_(g.w)};
}

}  // namespace

hipError_t launch_mask_bias(const float* mask, int64_t ms_i, int64_t ms_j, int n, int np,
                            float inf, float* mbias, void* tri_bias, bool bias_bf16,
                            hipStream_t stream) {
  const int64_t total = (int64_t)n * np + (int64_t)kHeads * (np - n) * np;
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = (int64_t)device_cu_count() * 16;
  if (blocks > cap) blocks = cap;
  if (bias_bf16) {
    hipLaunchKernelGGL(mask_bias_kernel<__bf16>, dim3((uint32_t)blocks), dim3(256), 0, stream, mask,
                       ms_i, ms_j, n, np, inf, mbias, static_cast<__bf16*>(tri_bias));
  } else {
    hipLaunchKernelGGL(mask_bias_kernel<float>, dim3((uint32_t)blocks), dim3(256), 0, stream, mask,
                       ms_i, ms_j, n, np, inf, mbias, static_cast<float*>(tri_bias));
  }
  return hipGetLastError();
}

hipError_t launch_layer_norm(const float* x, int64_t rows_i, int64_t rows_j, int64_t xs_i,
                             int64_t xs_j, const float* w, const float* b, float eps, float* y,
                             hipStream_t stream) {
  const int64_t rows = rows_i * rows_j;
  if (rows == 0) return hipSuccess;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL(layer_norm_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, x, rows_i,
                     rows_j, xs_i, xs_j, w, b, eps, y);
  return hipGetLastError();
}

hipError_t launch_sigmoid_mul(const float* gate, const float* value, float* out, int64_t count4,
                              hipStream_t stream) {
  if (count4 == 0) return hipSuccess;
  const int64_t blocks = (count4 + 255) / 256;
  if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sigmoid_mul_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream,
                     (const f32x4*)gate, (const f32x4*)value, (f32x4*)out, count4);
  return hipGetLastError();
}

int device_cu_count() {
  static std::atomic<int> cached[64];
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  int value = cached[device].load(std::memory_order_relaxed);
  if (value > 0) return value;
  int count = 0;
  if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      count <= 0)
    count = 256;
  cached[device].store(count, std::memory_order_relaxed);
  return count;
}

}  // namespace fpx
