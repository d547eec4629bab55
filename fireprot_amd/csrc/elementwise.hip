// Memory-bound helpers of the triangle-attention block: the additive mask
// bias, the standalone C128 pair LayerNorm and the sigmoid output gate.
#include "common.hpp"
#include "kernels.hpp"
#include "split.hpp"

#include <atomic>
#include <cmath>

namespace fpx {
namespace {

// One wavefront per row i < rows: mbias[i][k] for k < np and the row's tile
// flags.  Word w of part 0 (the first kTileFlagWords words) has bit t % 32 of
// tile t = 32w + t % 32 set when some key of that 32-key tile has a nonzero
// mask bias (-0 counts as zero, since s + -0 == s); part 1 does the same for
// "every key of the tile has a nonzero mask bias", part 2 for "every key of
// the tile has a mask bias <= -kSkipMask".  Padded keys (k >= n, -inf) count
// as masked in all three.  Part 3 holds the row's largest mask bias (word 0)
// and its smallest over the keys < n (word 1), as float bits, NaN-propagating.  kFromMask: the source is a {0, 1} mask and
// inf * (mask - 1) is evaluated as two rounded fp32 ops, as the native
// expression is (patches/protenix/0005-*.patch:36-39); otherwise the source
// already holds mask-bias values and is copied.  np is a multiple of 64.
// Work-group 0 also zeroes the magnitude record (nullable).
template <bool kFromMask>
__global__ __launch_bounds__(256) void mask_rows_kernel(const float* __restrict__ mask,
                                                        int64_t ms_i, int64_t ms_j, int rows,
                                                        int n, int np, float inf,
                                                        float* __restrict__ mbias,
                                                        uint32_t* __restrict__ flags,
                                                        uint32_t* __restrict__ magnitudes) {
  if (magnitudes != nullptr && blockIdx.x == 0 && threadIdx.x < kMagnitudeWords)
    magnitudes[threadIdx.x] = 0u;
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= rows) return;
  uint32_t part[kTileFlagParts][kTileFlagWords] = {};
  float vmax = -INFINITY;  // NaN-propagating max of the row's mask biases
  float vneg = -INFINITY;  // NaN-propagating max of -bias over the keys < n
  for (int k0 = 0; k0 < np; k0 += 64) {
    const int k = k0 + lane;
    float v = -INFINITY;
    if (k < n) {
      const float m = mask ? mask[i * ms_i + k * ms_j] : 0.0f;
      v = !mask ? 0.0f : kFromMask ? inf * (m - 1.0f) : m;
      vneg = __builtin_elementwise_maximum(vneg, -v);
    }
    vmax = __builtin_elementwise_maximum(vmax, v);
    mbias[(int64_t)i * np + k] = v;
    const uint64_t nz = __ballot(v != 0.0f);
    const uint64_t far = __ballot(v <= -kSkipMask);
    const int t = k0 >> 5;  // tiles t and t + 1 (t even)
    const uint32_t bits[kTileFlagParts] = {
        (uint32_t)((uint32_t)nz != 0u) | ((uint32_t)((nz >> 32) != 0u) << 1),
        (uint32_t)((uint32_t)nz == ~0u) | ((uint32_t)((nz >> 32) == ~0u) << 1),
        (uint32_t)((uint32_t)far == ~0u) | ((uint32_t)((far >> 32) == ~0u) << 1)};
#pragma unroll
    for (int wd = 0; wd < kTileFlagWords; ++wd) {
      if (wd == (t >> 5)) {
#pragma unroll
        for (int pt = 0; pt < kTileFlagParts; ++pt) part[pt][wd] |= bits[pt] << (t & 31);
      }
    }
  }
  part[kTileFlagMaxPart][0] = __builtin_bit_cast(uint32_t, wave_max(vmax));
  part[kTileFlagMaxPart][1] = __builtin_bit_cast(uint32_t, -wave_max(vneg));
  uint32_t* dst = flags + (int64_t)i * kTileFlagParts * kTileFlagWords;
#pragma unroll
  for (int pt = 0; pt < kTileFlagParts; ++pt)
#pragma unroll
    for (int wd = 0; wd < kTileFlagWords; ++wd)
      if (lane == pt * kTileFlagWords + wd) dst[pt * kTileFlagWords + wd] = part[pt][wd];
}

// Zero rows [n, np) of every head of the triangle bias (padded queries), in
// the FP32 or the BF16 fragment order, in each of `copies` consecutive
// [4][np][np] copies (the FP32 block keeps the bias and its log2(e) copy).
template <typename BiasT>
__global__ void bias_pad_kernel(int n, int np, BiasT* __restrict__ tri_bias, int copies) {
  const int64_t per_head = (int64_t)(np - n) * np;
  const int64_t total = kHeads * per_head;
  const int64_t copy_elems = (int64_t)kHeads * np * np;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int h = (int)(idx / per_head);
    const int64_t r = idx % per_head;
    const int q = n + (int)(r / np);
    const int k = (int)(r % np);
    const int64_t at = sizeof(BiasT) == 4 ? bias_frag_index(h, q, k, np)
                                          : bias_frag_index_bf16(h, q, k, np);
    for (int c = 0; c < copies; ++c) tri_bias[c * copy_elems + at] = (BiasT)0.0f;
  }
}

// Both fragment-order copies of a caller's [4][n][n] bias with any strides.
// One thread per 4 consecutive fragment floats (keys t..t+3 of one query, the
// inverse of bias_frag_index): coalesced 16-byte stores, gathered loads that
// the caches absorb (the bias is 4 n^2 floats, read once).
__global__ __launch_bounds__(256) void stage_bias_kernel(const float* __restrict__ bias,
                                                         int64_t sh, int64_t sq, int64_t sk,
                                                         int n, int np, float* __restrict__ frag,
                                                         float* __restrict__ frag_l2,
                                                         uint32_t* __restrict__ magnitudes) {
  const int64_t nt = np >> 5;
  const int64_t total4 = (int64_t)kHeads * np * np / 4;
  float vmax = 0.f;  // NaN-propagating max |bias| staged by this lane
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total4;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = idx * 4;
    const int64_t blk = f >> 10;
    const int within = (int)(f & 1023);
    const int slot = (within >> 2) & 63;
    const int q = (int)((blk / nt) % nt) * 32 + (slot & 31);
    const int k0 = (int)(blk % nt) * 32 + (within >> 8) * 8 + (slot >> 5) * 4;
    const int h = (int)(blk / (nt * nt));
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (bias != nullptr && q < n) {
      const float* row = bias + h * sh + (int64_t)q * sq;
      if (k0 + 0 < n) v.x = row[(int64_t)(k0 + 0) * sk];
      if (k0 + 1 < n) v.y = row[(int64_t)(k0 + 1) * sk];
      if (k0 + 2 < n) v.z = row[(int64_t)(k0 + 2) * sk];
      if (k0 + 3 < n) v.w = row[(int64_t)(k0 + 3) * sk];
    }
    *(f32x4*)(frag + f) = v;
    *(f32x4*)(frag_l2 + f) = v * kLog2e;
    vmax = __builtin_elementwise_maximum(
        vmax, __builtin_elementwise_maximum(
                  __builtin_elementwise_maximum(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                  __builtin_elementwise_maximum(__builtin_fabsf(v.z), __builtin_fabsf(v.w))));
  }
  if (magnitudes != nullptr) {
    // one atomic per work-group: atomics on one word serialise
    __shared__ float wmax[4];
    const float m = wave_max(vmax);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      const float bm = __builtin_elementwise_maximum(__builtin_elementwise_maximum(wmax[0], wmax[1]),
                                                     __builtin_elementwise_maximum(wmax[2], wmax[3]));
      atomicMax(&magnitudes[3], __builtin_bit_cast(uint32_t, bm));
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

// Thirty-two lanes per 128-channel row, one 16-byte vector per lane (the
// 32 lanes read the row's 512 contiguous bytes); a wave covers 2 rows and a
// work-group 8 rows that are consecutive along axis b, the axis whose rows
// are adjacent in memory (j for the contiguous pair, i for the transposed
// view), so each work-group reads 4 KB contiguously.  Row (a, r) is read at
// x + a*xs_a + r*xs_b and written at y + a*ys_a + r*ys_b.  Statistics as
// ln_stats_c128: values shifted by the row's first channel, their mean, then
// the biased variance of the centred values; row16_sum plus one xor-16
// exchange per reduction.
__global__ __launch_bounds__(256) void layer_norm32_kernel(const float* __restrict__ x,
                                                           int64_t rows_b, int64_t xs_a,
                                                           int64_t xs_b, int64_t ys_a,
                                                           int64_t ys_b,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ b, float eps,
                                                           float* __restrict__ y, int groups_b) {
  const int c32 = threadIdx.x & 31;
  const int r8 = threadIdx.x >> 5;
  const int g = blockIdx.x;
  const int64_t ra = g / groups_b;
  const int64_t rb = (int64_t)(g - (int)ra * groups_b) * 8 + r8;
  const bool valid = rb < rows_b;
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (valid) v = *(const f32x4*)(x + ra * xs_a + rb * xs_b + 4 * c32);
  const float pivot = __shfl(v.x, 0, 32);
  const f32x4 sh = v - pivot;
  float s = row16_sum((sh.x + sh.y) + (sh.z + sh.w));
  s += __shfl_xor(s, 16, 32);
  const float mean = s * (1.0f / kChannels);
  const f32x4 d = sh - mean;
  float q = row16_sum((d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w));
  q += __shfl_xor(q, 16, 32);
  const float rstd = __builtin_amdgcn_rsqf(q * (1.0f / kChannels) + eps);
  f32x4 gw = {1.f, 1.f, 1.f, 1.f}, gb = {0.f, 0.f, 0.f, 0.f};
  if (w) gw = *(const f32x4*)(w + 4 * c32);
  if (b) gb = *(const f32x4*)(b + 4 * c32);
  if (valid) *(f32x4*)(y + ra * ys_a + rb * ys_b + 4 * c32) = d * rstd * gw + gb;
}

// out = value * sigmoid(gate), one 16-byte vector per thread (a plain copy
// kernel of this shape streams fastest on this part: more vectors per thread
// measured slower).
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
                            float inf, float* mbias, uint32_t* tile_flags, void* tri_bias,
                            bool bias_bf16, uint32_t* magnitudes, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (np % 64 || np > kTileFlagWords * 32 * 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mask_rows_kernel<true>, dim3((uint32_t)((n + 3) / 4)), dim3(256), 0, stream,
                     mask, ms_i, ms_j, n, n, np, inf, mbias, tile_flags, magnitudes);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || np == n) return e;
  const int64_t total = (int64_t)kHeads * (np - n) * np;
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = (int64_t)device_cu_count() * 16;
  if (blocks > cap) blocks = cap;
  if (bias_bf16) {
    hipLaunchKernelGGL(bias_pad_kernel<__bf16>, dim3((uint32_t)blocks), dim3(256), 0, stream, n,
                       np, static_cast<__bf16*>(tri_bias), 1);
  } else {
    hipLaunchKernelGGL(bias_pad_kernel<float>, dim3((uint32_t)blocks), dim3(256), 0, stream, n,
                       np, static_cast<float*>(tri_bias), 2);
  }
  return hipGetLastError();
}

hipError_t launch_mask_rows(const float* values, int64_t vs_i, int64_t vs_k, int rows, int n,
                            int np, float* mbias, uint32_t* tile_flags, uint32_t* magnitudes,
                            hipStream_t stream) {
  if (rows <= 0 || n <= 0) return hipSuccess;
  if (np % 64 || np < n || np > kTileFlagWords * 32 * 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mask_rows_kernel<false>, dim3((uint32_t)((rows + 3) / 4)), dim3(256), 0,
                     stream, values, vs_i, vs_k, rows, n, np, 0.0f, mbias, tile_flags, magnitudes);
  return hipGetLastError();
}

hipError_t launch_stage_bias(const float* bias, int64_t sh, int64_t sq, int64_t sk, int n, int np,
                             float* frag, float* frag_l2, uint32_t* magnitudes,
                             hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (np % 32 || np < n) return hipErrorInvalidValue;
  const int64_t total4 = (int64_t)kHeads * np * np / 4;
  int64_t blocks = (total4 + 255) / 256;
  // a few work-groups per CU stream the copy; fewer keep the record's atomics few
  const int64_t cap = (int64_t)device_cu_count() * (magnitudes != nullptr ? 4 : 32);
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(stage_bias_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, bias, sh, sq,
                     sk, n, np, frag, frag_l2, magnitudes);
  return hipGetLastError();
}

hipError_t launch_layer_norm(const float* x, int64_t rows_i, int64_t rows_j, int64_t xs_i,
                             int64_t xs_j, const float* w, const float* b, float eps, float* y,
                             hipStream_t stream) {
  const int64_t rows = rows_i * rows_j;
  if (rows == 0) return hipSuccess;
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a16(x) && a16(y) && (w == nullptr || a16(w)) && (b == nullptr || a16(b)) && xs_i % 4 == 0 &&
      xs_j % 4 == 0) {
    // Group rows along the axis with the smaller input stride (b); a is the other.
    const bool along_i = rows_i > 1 && xs_i < xs_j;
    const int64_t rows_a = along_i ? rows_j : rows_i;
    const int64_t rows_b = along_i ? rows_i : rows_j;
    const int64_t groups_b = (rows_b + 7) / 8;
    const int64_t blocks = rows_a * groups_b;
    if (groups_b <= 0x7fffffffll && blocks <= 0x7fffffffll) {
      const int64_t ys_i = rows_j * kChannels, ys_j = kChannels;
      hipLaunchKernelGGL(layer_norm32_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, x,
                         rows_b, along_i ? xs_j : xs_i, along_i ? xs_i : xs_j,
                         along_i ? ys_j : ys_i, along_i ? ys_i : ys_j, w, b, eps, y,
                         (int)groups_b);
      return hipGetLastError();
    }
  }
  // Rows only 8-byte aligned: one wavefront per row.
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

// The fp16 (hi, lo) split behind every FP32-accurate product (split_f16),
// on count8 groups of 8 floats taken as given (the kernels scale each block
// by a power of two first): plane 0 = hi, plane 1 = lo, each [count8 * 8]
// fp16 bit patterns.
__global__ __launch_bounds__(256) void split_planes_kernel(const f32x4* __restrict__ x,
                                                           uint32_t* __restrict__ planes,
                                                           int64_t count8) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= count8) return;
  const f32x4 u = x[2 * g], v = x[2 * g + 1];
  bf16x8 hi, lo;
  split_f16(f32x8{u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w}, hi, lo);
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4* out = reinterpret_cast<u32x4*>(planes);
  out[g] = __builtin_bit_cast(u32x4, hi);
  out[count8 + g] = __builtin_bit_cast(u32x4, lo);
}

hipError_t launch_split_planes(const float* x, uint16_t* planes, int64_t count8,
                               hipStream_t stream) {
  if (count8 == 0) return hipSuccess;
  const int64_t blocks = (count8 + 255) / 256;
  if (blocks > 0x7fffffffll) return hipErrorInvalidValue;
  hipLaunchKernelGGL(split_planes_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream,
                     (const f32x4*)x, reinterpret_cast<uint32_t*>(planes), count8);
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
