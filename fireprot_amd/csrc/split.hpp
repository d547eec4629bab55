// FP32 values as power-of-two scaled fp16 (hi, lo) planes for the CDNA4
// 16-bit matrix cores, and the 32x32x16 / 16x16x32 MFMA steps on them.
//
// A block of values is scaled by one power of two 2^e so that its max |x|
// lies in [2^14, 2^15), then split: hi = fp16(x 2^e) (round to nearest even)
// and lo = fp16(x 2^e - hi), where the difference is exact in FP32.  hi + lo
// keeps about 22 significant bits; a product of two such operands over the
// three terms hi hi, hi lo, lo hi leaves a relative error of about 2^-22 per
// product, the level of an FP32 dot product.  Scaling by a power of two (and
// back) is exact.
//
// Operand lane layout of v_mfma_f32_32x32x16_{f16,bf16} (one block): lane l
// holds A[l % 32][8 * (l / 32) + e] and B[8 * (l / 32) + e][l % 32],
// e = 0..7, of one 16-deep k step; the FP32 result has the 32x32x2 f32 layout
// (common.hpp).
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace fpx {

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) + e] and
// B[8 (l / 16) + e][l % 16], e = 0..7, of one 32-deep k step, and result
// register r holds D[4 (l / 16) + r][l % 16] (checked on the device against a
// host product of small integers).
__device__ __forceinline__ f32x4 mfma16_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_f16 on fp16 bit patterns held in bf16x8 vectors (the
// planes share one storage type); the operand and result layouts are those
// of the bf16 instruction.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x16 mfma_f16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_f16 on fp16 bit patterns (layouts of mfma16_bf16).
__device__ __forceinline__ f32x4 mfma16_f16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Scaled fp16 planes.  A block of values whose max |x| is m is scaled by
// 2^e, e = plane_exp(m), so that m 2^e lies in [2^14, 2^15), and split into
// hi = fp16(x 2^e) and lo = fp16(x 2^e - hi) (round to nearest even; the
// difference is exact).  hi + lo keeps about 22 significant bits, and the
// three terms hi hi, hi lo, lo hi of a product leave a relative error of
// about 2^-22 per product term; values far below the block's max keep an
// absolute error below 2^-25 of the scaled unit.  The scaling is a power of
// two (ldexp), so it and its inverse are exact.  e = 0 for a zero or
// non-finite m (NaN and infinities then reach the products unscaled).
__device__ __forceinline__ int plane_exp(float m) {
  return (m > 0.f && m < INFINITY) ? 15 - __builtin_amdgcn_frexp_expf(m) : 0;
}
// Plane exponent of a v^T tile: plane_exp clamped to |e| <= kPlaneExpMax,
// and kPlaneExpMax for a zero tile, so that it never lowers the smallest
// exponent of a row (the attention scales each tile's weights by
// 2^(e_min - e_t) before the product: see attention_split.hip).
__device__ __forceinline__ int value_plane_exp(float m) {
  if (m == 0.f) return kPlaneExpMax;
  const int e = plane_exp(m);
  return e < -kPlaneExpMax ? -kPlaneExpMax : e > kPlaneExpMax ? kPlaneExpMax : e;
}
// e of a power-of-two inverse plane scale s = 2^-e (a normal float).
__device__ __forceinline__ int inv_scale_exp(float s) {
  return 1 - __builtin_amdgcn_frexp_expf(s);
}
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// -1.0f in an SGPR the optimiser cannot fold, for the residual fma(float(hi),
// -1, x) = x - hi of the fp16 splits below.
__device__ __forceinline__ float opaque_minus_one() {
  float m;
  asm("s_mov_b32 %0, 0xbf800000" : "=s"(m));
  return m;
}
// N values (N even) -> fp16 hi and lo planes, packed two per word.  hi is one
// v_cvt_pk_f16_f32 per pair; the residuals x - hi are one v_fma_mix_f32 each,
// fma(float(hi half), -1, x), exact in FP32, and lo is one more
// v_cvt_pk_f16_f32 per pair: lo = fp16(x - hi) with one rounding.  Measured on
// gfx950 at four waves per SIMD, v_fma_mix_f32 and v_cvt_pk_f16_f32 take about
// 1.9 ns per wave instruction and v_fma_mixlo_f16 / v_fma_mixhi_f16 (the
// residual rounded straight into a half of the word) about 3.8 ns, so three
// instructions per pair here cost less than the two half-word ones.
template <int N>
__device__ __forceinline__ void split_f16_words(const float* x, uint32_t* hi, uint32_t* lo) {
  const float m1 = opaque_minus_one();
#pragma unroll
  for (int i = 0; i < N / 2; ++i)
    hi[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x[2 * i], x[2 * i + 1]}, f16x2));
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    float r0, r1;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]"
        : "=v"(r0)
        : "v"(hi[i]), "s"(m1), "v"(x[2 * i]));
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(r1)
        : "v"(hi[i]), "s"(m1), "v"(x[2 * i + 1]));
    lo[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{r0, r1}, f16x2));
  }
}
// Already scaled values -> fp16 hi and lo planes (bit patterns in bf16x8/x4).
__device__ __forceinline__ void split_f16(f32x8 x, bf16x8& hi, bf16x8& lo) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const float v[8] = {x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
  uint32_t h[4], l[4];
  split_f16_words<8>(v, h, l);
  hi = __builtin_bit_cast(bf16x8, u32x4{h[0], h[1], h[2], h[3]});
  lo = __builtin_bit_cast(bf16x8, u32x4{l[0], l[1], l[2], l[3]});
}
__device__ __forceinline__ void split_f16(f32x4 x, bf16x4& hi, bf16x4& lo) {
  const float v[4] = {x.x, x.y, x.z, x.w};
  uint32_t h[2], l[2];
  split_f16_words<4>(v, h, l);
  hi = __builtin_bit_cast(bf16x4, u32x2{h[0], h[1]});
  lo = __builtin_bit_cast(bf16x4, u32x2{l[0], l[1]});
}
__device__ __forceinline__ f32x8 ldexp8(f32x8 x, int e) {
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = __builtin_ldexpf(x[i], e);
  return x;
}
__device__ __forceinline__ f32x4 ldexp4(f32x4 x, int e) {
  return f32x4{__builtin_ldexpf(x.x, e), __builtin_ldexpf(x.y, e), __builtin_ldexpf(x.z, e),
               __builtin_ldexpf(x.w, e)};
}

// Sum over each 16-lane row of the wave (DPP quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror, row_mirror), returned in all 16 lanes.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v;
}

// Lane 0 of each 16-lane row, broadcast to the row (DPP row_newbcast:0).
__device__ __forceinline__ float row16_first(float v) {
  return dpp<0x150>(v);
}

}  // namespace fpx
