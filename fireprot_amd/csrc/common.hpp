// Shared device helpers for the gfx950 triangle-attention kernels.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, the FP32 matrix-core
// instruction v_mfma_f32_32x32x2_f32, and an XCD-aware work-group remap for the
// 8 accelerator dies of an MI355X.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fpx {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;
constexpr int kHeads = 4;
constexpr int kHeadDim = 32;
constexpr int kChannels = 128;
constexpr int kHidden = kHeads * kHeadDim;  // 128
constexpr int kXcds = 8;
constexpr float kLog2e = 1.4426950408889634f;

// D = A x B + C for one 32x32x2 FP32 matrix-core step.
// Operand/result lane layouts (CDNA3/CDNA4 ISA, "32x32x2 f32", single block):
//   A[row][k]  : lane = row + 32*k                      (row 0..31, k 0..1)
//   B[k][col]  : lane = col + 32*k
//   D[row][col]: lane = col + 32*((row/4)%2), register = (row%4) + 4*(row/8)
// i.e. lane l, register r holds D[8*(r/4) + 4*(l/32) + r%4][l%32].
// tests/test_gpu_mfma_layout.py calibrates this on the device.
__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row index (0..31) of result register r in lane half `half` (= lane/32).
__device__ __forceinline__ int mfma_row(int r, int half) {
  return 8 * (r >> 2) + 4 * half + (r & 3);
}

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}

// Sum over the 64 lanes, returned in every lane, with no LDS traffic: DPP
// adds across lane pairs, quads, 8 and 16 lanes (quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror, row_mirror), then v_permlane16_swap and
// v_permlane32_swap across rows.  Every lane adds the same two partial sums,
// so all lanes hold the identical value.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  v = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_bit_cast(float, (unsigned)s[0]) + __builtin_bit_cast(float, (unsigned)s[1]);
}

// NaN-propagating maximum over the 64 lanes (v_maximum3 semantics), returned
// in every lane, with the reduction pattern of wave_sum.
__device__ __forceinline__ float wave_max(float v) {
  auto mx = [](float x, float y) { return __builtin_elementwise_maximum(x, y); };
  v = mx(v, dpp<0xB1>(v));
  v = mx(v, dpp<0x4E>(v));
  v = mx(v, dpp<0x141>(v));
  v = mx(v, dpp<0x140>(v));
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  v = mx(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
  const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return mx(__builtin_bit_cast(float, (unsigned)s[0]), __builtin_bit_cast(float, (unsigned)s[1]));
}

// NaN-propagating maximum over each 32-lane half of the wave (lanes 0-31 and
// 32-63 separately), returned in every lane of the half.
__device__ __forceinline__ float half_max(float v) {
  auto mx = [](float x, float y) { return __builtin_elementwise_maximum(x, y); };
  v = mx(v, dpp<0xB1>(v));
  v = mx(v, dpp<0x4E>(v));
  v = mx(v, dpp<0x141>(v));
  v = mx(v, dpp<0x140>(v));
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return mx(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}

// Two-pass LayerNorm statistics of a 128-channel row held as two values per
// lane.  Values are shifted by lane 0's first value before summing, so rows
// with |mean| >> std (e.g. 1000 + 0.001*c) keep their digits: the centred
// values are formed from small differences instead of from a rounded mean of
// large values.  Returns the centred values and 1/sqrt(biased var + eps).
__device__ __forceinline__ void ln_stats_c128(float a, float b, float eps, float& da, float& db,
                                              float& rstd) {
  const float pivot =
      __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, a)));
  const float sa = a - pivot;
  const float sb = b - pivot;
  const float mean_s = wave_sum(sa + sb) * (1.0f / kChannels);
  da = sa - mean_s;
  db = sb - mean_s;
  const float var = wave_sum(da * da + db * db) * (1.0f / kChannels);
  rstd = __builtin_amdgcn_rsqf(var + eps);  // v_rsq_f32, within 1 ulp
}

__device__ __forceinline__ float exp2_fast(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// 1 / (1 + e^-x) with v_exp_f32 and v_rcp_f32 (within 1 ulp each); the
// limits are exact: 1 / inf = 0 and 1 / 1 = 1.
__device__ __forceinline__ float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// Work-groups are dispatched round-robin over the XCDs: hardware block b runs
// on XCD b % 8.  Return a logical index such that each XCD receives one
// contiguous range of logical indices, so neighbouring tiles (which share
// K/V rows or bias rows) meet in the same 4 MB L2.  Bijective for any total.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t total) {
  const uint32_t per = total / kXcds;
  const uint32_t extra = total % kXcds;
  const uint32_t xcd = b % kXcds;
  const uint32_t slot = b / kXcds;
  return xcd < extra ? xcd * (per + 1) + slot
                     : extra * (per + 1) + (xcd - extra) * per + slot;
}

// [128 x 32] weight fragment (B operand of v_mfma_f32_32x32x2_f32) of output
// column col (this lane's l % 32) of a torch [out][in] weight with in
// stride ld: lane half h holds input channels 64h .. 64h + 63.
__device__ __forceinline__ void load_fragment(const float* w, int col, int half, float* wf,
                                              int64_t ld = kChannels) {
  const float* src = w + (int64_t)col * ld + 64 * half;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const f32x4 v = *(const f32x4*)(src + 4 * t);
    wf[4 * t + 0] = v.x;
    wf[4 * t + 1] = v.y;
    wf[4 * t + 2] = v.z;
    wf[4 * t + 3] = v.w;
  }
}

__host__ __device__ __forceinline__ int64_t round_up(int64_t x, int64_t m) {
  return (x + m - 1) / m * m;
}

// Position of triangle-bias element (head h, query q, key k) in the FP32
// block's fragment-major copy: for every (head, 32-query tile, 32-key tile)
// one contiguous 4 KB block laid out exactly as the S^T accumulator of
// v_mfma_f32_32x32x2_f32 (lane = q%32 + 32*((k%32/4)%2), register
// r = 4*(k%32/8) + k%4), so a wave loads its fragment with four coalesced
// 1 KB reads.  np is the padded extent (a multiple of 32).
// The BF16 block's bias copy (bf16-rounded values): for every (head, 32-query
// tile, 32-key tile) one contiguous 2 KB block in the same lane and register
// order as bias_frag_index, register r of lane l at (r / 8) * 512 + l * 8 +
// r % 8, so a wave loads its fragment with two coalesced 1 KB reads and widens
// each value to FP32 with one shift or mask.
__host__ __device__ __forceinline__ int64_t bias_frag_index_bf16(int h, int q, int k, int np) {
  const int64_t nt = np >> 5;
  const int t = k & 31;
  const int lane = (q & 31) + 32 * ((t >> 2) & 1);
  const int r = 4 * (t >> 3) + (t & 3);
  return (((int64_t)h * nt + (q >> 5)) * nt + (k >> 5)) * 1024 + (r >> 3) * 512 + lane * 8 +
         (r & 7);
}

__host__ __device__ __forceinline__ int64_t bias_frag_index(int h, int q, int k, int np) {
  const int64_t nt = np >> 5;
  const int t = k & 31;
  return (((int64_t)h * nt + (q >> 5)) * nt + (k >> 5)) * 1024 + (t >> 3) * 256 +
         ((q & 31) + 32 * ((t >> 2) & 1)) * 4 + (t & 3);
}

}  // namespace fpx
