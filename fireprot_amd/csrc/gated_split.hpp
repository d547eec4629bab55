// Gated pair-row projections on the CDNA4 16-bit matrix cores, FP32-accurate.
//
// The triangle multiplication's input projections produce, per channel c of
// a pair row x,
//
//   value_c = LN(x) . Wv[c] + bv[c]    gate_c = LN(x) . Wg[c] + bg[c]
//
// and combine the two:  (mask * sigmoid(gate)) * value.  Rows and weights are held as
// power-of-two scaled fp16 (hi, lo) planes (split.hpp): the LN rows by one
// 2^ex per launch from the LN affine (|y_c| <= sqrt(128) |ln_w_c| + |ln_b_c|,
// applied by pre-scaling ln_w and ln_b), each weight column by its own 2^ew;
// each 32 x 32 block sums the three terms hi hi, hi lo, lo hi on
// v_mfma_f32_32x32x16_f16 and is scaled back with ldexp, exactly.
//
// A wave's 32 B-operand columns are 16 value channels followed by the gate
// channels of the same 16 channels, so its two weight planes fit in 64
// VGPRs and the result of lane l (value) and lane l + 16 (gate) belong to one
// channel: one v_permlane16_swap per register pair hands each lane both.  A
// work-group (8 waves) covers 128 channels, one slice; the slices of a row
// tile are neighbouring work-groups in the XCD-aware order.
//
// The pipeline is that of projection_split_kernel<kProjBlock>: LayerNorm 16
// lanes per row, raw rows staged through LDS so that a row load is waited
// an iteration after its issue, and lead / trail waves running the k steps
// and the normalise-and-store half in opposite orders.
#pragma once

#include "common.hpp"
#include "kernels.hpp"
#include "split.hpp"

namespace fpx {

enum GatedMode { kGatedTriMul = 0 };

struct GatedArgs {
  const float* x;        // pair row (r, k) at x + r * xs_r + k * xs_k
  int64_t xs_r;
  int64_t xs_k;
  int rows_r;            // outer rows
  int rows_k;            // valid k extent
  int span_k;            // k extent covered by tiles (a multiple of 32, >= rows_k)
  const float* ln_w;     // nullable
  const float* ln_b;     // nullable
  float eps;
  const float* w_value[4];  // per slice: [128 out][128 in]
  const float* w_gate[4];
  const float* b_value[4];  // nullable
  const float* b_gate[4];   // nullable
  const float* mask;     // kGatedTriMul: nullable multiplier of row (r, k)
  int64_t ms_r;
  int64_t ms_k;
  float* out[4];         // per slice, see gated_split_kernel
  int np;                // kGatedTriMul: packed extent of the output
  uint32_t* rowmax;      // kGatedTriMul: [slice][128][np] max |out| over k per (channel, row),
                         // float bits; null: none
};

template <int MODE>
struct GatedTraits;
template <>
struct GatedTraits<kGatedTriMul> {
  static constexpr int kSlices = 2;  // a, b
};

constexpr int kGatedWaves = 8;
constexpr int kGatedRows = 32;
constexpr int kGatedPlaneRow = kChannels + 8;  // bf16 per LDS row: 272 bytes

// Outputs: kGatedTriMul writes, for all k < span_k (0 past rows_k), the
// channel-blocked layout
//   out[slice][(((c / 16) * (span_k / 32) + k / 32) * np + r) * 512 + (c % 16) * 32 + k % 32]
// (np = a.np >= rows_r): a wave's 16 channels x 32 keys of a tile are one
// contiguous 2 KB block, the blocks of consecutive rows r are adjacent, and
// channel c's row r is 32-key runs np * 512 floats apart, the contraction's
// operand layout.  Each work-group owns whole rows r (first, first +
// streams, ...), so the row maxima are plain stores, and the work-groups
// in flight write one run of adjacent blocks per channel group.
template <int MODE>
__global__ __launch_bounds__(kGatedWaves * 64, 1) void gated_split_kernel(GatedArgs a, int tiles_k,
                                                                          int ntiles,
                                                                          int streams) {
  constexpr int kSlices = GatedTraits<MODE>::kSlices;
  __shared__ __attribute__((aligned(16))) __bf16 xs[2][2][kGatedRows][kGatedPlaneRow];
  __shared__ __attribute__((aligned(16))) float raw[kGatedRows][kChannels + 4];
  __shared__ float ms[4][kGatedRows];  // mask of tile T_k's rows at [k & 3]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const uint32_t logical = xcd_remap(blockIdx.x, gridDim.x);
  const int slice = (int)(logical % kSlices);
  const int first = (int)(logical / kSlices);
  const bool odd = l32 >= 16;           // gate column (B operand) / odd 16-lane row
  const int ch = 16 * w + (l32 & 15);   // channel of this lane's column, within the slice

  // Weight planes of this lane's column, scaled by 2^ew (the column's max
  // |w| over both halves of the wave).
  bf16x8 wh[8], wl[8];
  int ew;
  {
    const float* src = (odd ? a.w_gate[slice] : a.w_value[slice]) + (int64_t)ch * kChannels +
                       8 * half;
    f32x8 wv[8];
    float m = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const f32x4 u = *(const f32x4*)(src + 16 * t);
      const f32x4 v = *(const f32x4*)(src + 16 * t + 4);
      wv[t] = f32x8{u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) m = __builtin_elementwise_maximum(m, __builtin_fabsf(wv[t][e]));
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, m),
                                                     __builtin_bit_cast(unsigned, m), false, false);
    m = __builtin_elementwise_maximum(__builtin_bit_cast(float, (unsigned)sw[0]),
                                      __builtin_bit_cast(float, (unsigned)sw[1]));
    ew = plane_exp(m);
#pragma unroll
    for (int t = 0; t < 8; ++t) split_f16(ldexp8(wv[t], ew), wh[t], wl[t]);
  }
  const float bv = a.b_value[slice] ? a.b_value[slice][ch] : 0.f;
  const float bg = a.b_gate[slice] ? a.b_gate[slice][ch] : 0.f;

  // LN: 16 lanes per row, lane c16 holding channels 8*c16 .. 8*c16 + 7 of
  // tile row lrow.
  const int c16 = lane & 15;
  const int lrow = 4 * w + (lane >> 4);
  f32x8 lnw, lnb;
  float bound = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    lnw[e] = a.ln_w ? a.ln_w[8 * c16 + e] : 1.f;
    lnb[e] = a.ln_b ? a.ln_b[8 * c16 + e] : 0.f;
    bound = __builtin_elementwise_maximum(
        bound, 11.3137085f * __builtin_fabsf(lnw[e]) + __builtin_fabsf(lnb[e]));
  }
  // |y_c| <= sqrt(128) |ln_w_c| + |ln_b_c| up to FP32 rounding; the margin
  // keeps |y| 2^ex below 2^15.
  const int ex = plane_exp(wave_max(bound) * (1.0f + 0x1p-10f));
  lnw = ldexp8(lnw, ex);
  lnb = ldexp8(lnb, ex);

  // This work-group's tiles, local index i < count (at least one).
  const int count = tiles_k * ((a.rows_r - first + streams - 1) / streams);
  auto origin = [&](int i, int& r, int& k0) {
    const int q = i / tiles_k;
    r = first + streams * q;
    k0 = (i - q * tiles_k) * kGatedRows;
  };

  // Row loads with no branches on the data path (tile clamped to the last
  // one, row to the last valid row); the mask is 0 past rows_k.
  f32x8 stage_ln;
  float stage_m = 0.f;
  auto fetch = [&](int i) {
    int r, k0;
    origin(i < count ? i : count - 1, r, k0);
    const int kk = k0 + lrow;
    const int k = min(kk, a.rows_k - 1);
    const float* src = a.x + (int64_t)r * a.xs_r + (int64_t)k * a.xs_k + 8 * c16;
    const f32x4 u = *(const f32x4*)src;
    const f32x4 v = *(const f32x4*)(src + 4);
    stage_ln = f32x8{u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
    if constexpr (MODE == kGatedTriMul) {
      const float m = a.mask ? a.mask[(int64_t)r * a.ms_r + (int64_t)k * a.ms_k] : 1.f;
      stage_m = kk < a.rows_k ? m : 0.f;
    }
  };

  auto ln_stats = [&](const f32x8& rawv, f32x8& d, float& rstd) {
    const float pivot = row16_first(rawv[0]);
    const f32x8 sh = rawv - pivot;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += sh[e];
    const float mean = row16_sum(s) * (1.0f / kChannels);
    d = sh - mean;
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) q += d[e] * d[e];
    rstd = __builtin_amdgcn_rsqf(row16_sum(q) * (1.0f / kChannels) + a.eps);
  };

  auto stage_split = [&](int buf, const f32x8& d, float rstd, int k0) {
    f32x8 y = d * rstd * lnw + lnb;  // scaled by 2^ex
    if (k0 + lrow >= a.rows_k) y = f32x8{};
    bf16x8 hi, lo;
    split_f16(y, hi, lo);
    *(bf16x8*)&xs[buf][0][lrow][8 * c16] = hi;
    *(bf16x8*)&xs[buf][1][lrow][8 * c16] = lo;
  };

  auto consume = [&](int i) {  // i: local index of the staged tile
    *(f32x8*)&raw[lrow][8 * c16] = stage_ln;
    if constexpr (MODE == kGatedTriMul) {
      if (c16 == 0) ms[i & 3][lrow] = stage_m;
    }
  };

  // Two accumulation chains, swapped every k step.
  auto mfma_step = [&](int buf, int t, f32x16& c0, f32x16& c1) {
    const int k = 16 * t + 8 * half;
    const bf16x8 xh = *(const bf16x8*)&xs[buf][0][l32][k];
    const bf16x8 xl = *(const bf16x8*)&xs[buf][1][l32][k];
    if (t & 1) {
      c1 = mfma_f16(xh, wh[t], c1);
      c0 = mfma_f16(xh, wl[t], c0);
      c1 = mfma_f16(xl, wh[t], c1);
    } else {
      c0 = mfma_f16(xh, wh[t], c0);
      c1 = mfma_f16(xh, wl[t], c1);
      c0 = mfma_f16(xl, wh[t], c0);
    }
  };
  auto k_steps = [&](int buf) -> f32x16 {
    f32x16 c0 = {}, c1 = {};
#pragma unroll
    for (int t = 0; t < 8; ++t) mfma_step(buf, t, c0, c1);
    f32x16 r = c0 + c1;
#pragma unroll
    for (int e = 0; e < 16; ++e) r[e] = __builtin_ldexpf(r[e], -(ex + ew));
    return r;
  };

  // Result of local tile i: lanes of even 16-lane
  // rows hold the value channel, odd rows the gate channel.  Swapping
  // register r with r + 8 across the row pair leaves every lane the value
  // and gate of its channel for registers r + (odd ? 8 : 0), r < 8, i.e.
  // tile rows 8 rr + 4 half + e for rr = (odd ? 2 : 0) + r / 4, e = r % 4.
  float row_max = 0.f;  // kGatedTriMul: max |value| of this lane's channel over the row so far
  auto store = [&](const f32x16& res, int i) {
    f32x8 val;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      // Elements are copied out first: __builtin_bit_cast of a vector
      // element reads element 0 with this compiler.
      const float lo_reg = res[r];
      const float hi_reg = res[r + 8];
      const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, lo_reg),
                                                      __builtin_bit_cast(unsigned, hi_reg),
                                                      false, false);
      const float p = __builtin_bit_cast(float, (unsigned)s[0]) + bv;
      const float g = __builtin_bit_cast(float, (unsigned)s[1]);
      const int row = 8 * ((odd ? 2 : 0) + (r >> 2)) + 4 * half + (r & 3);
      // native order: a = mask; a = a * sigmoid(g); a = a * p
      val[r] = (ms[i & 3][row] * sigmoidf_(g + bg)) * p;
    }
    int r_out, k0;
    origin(i, r_out, k0);
    const int rr0 = odd ? 2 : 0;
    if constexpr (MODE == kGatedTriMul) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
        row_max = __builtin_elementwise_maximum(row_max, __builtin_fabsf(val[r]));
      if (k0 + kGatedRows == a.span_k) {
        // the row's last tile: the channel's max over the row is the max of
        // this lane's, lane l ^ 16's (other register half) and lane l ^ 32's
        // (other tile rows)
        float m = row_max;
        row_max = 0.f;
        const auto s16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, m),
                                                          __builtin_bit_cast(unsigned, m), false, false);
        m = __builtin_elementwise_maximum(__builtin_bit_cast(float, (unsigned)s16[0]),
                                          __builtin_bit_cast(float, (unsigned)s16[1]));
        const auto s32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, m),
                                                          __builtin_bit_cast(unsigned, m), false, false);
        m = __builtin_elementwise_maximum(__builtin_bit_cast(float, (unsigned)s32[0]),
                                          __builtin_bit_cast(float, (unsigned)s32[1]));
        if (!odd && half == 0 && a.rowmax != nullptr)
          a.rowmax[((int64_t)slice * kChannels + ch) * a.np + r_out] =
              __builtin_bit_cast(uint32_t, m);
      }
      // the wave's 2 KB block of the channel-blocked layout
      float* dst = a.out[slice] +
                   (((int64_t)w * tiles_k + k0 / kGatedRows) * a.np + r_out) * 512 +
                   (l32 & 15) * 32 + 4 * half;
#pragma unroll
      for (int q = 0; q < 2; ++q)
        *(f32x4*)(dst + 8 * (rr0 + q)) =
            f32x4{val[4 * q + 0], val[4 * q + 1], val[4 * q + 2], val[4 * q + 3]};
    }
  };

  const bool lead = w < kGatedWaves / 2;
  fetch(0);
  {
    int r0, k00;
    origin(0, r0, k00);
    f32x8 d;
    float rstd;
    ln_stats(stage_ln, d, rstd);
    stage_split(0, d, rstd, k00);
    if constexpr (MODE == kGatedTriMul) {
      if (c16 == 0) ms[0][lrow] = stage_m;
    }
  }
  fetch(1);
  consume(1);
  fetch(2);
  __syncthreads();

  f32x16 res = {};
  int i = 0;
  for (int buf = 0; i < count; buf ^= 1) {
    if (lead) res = k_steps(buf);
    {
      // The other half: normalise T_{k+1} into the other planes, then the
      // iteration's global accesses (see projection_split_kernel).
      const bool more = i + 1 < count;
      if (more) {
        int rn, kn0;
        origin(i + 1, rn, kn0);
        f32x8 d;
        float rstd;
        ln_stats(*(const f32x8*)&raw[lrow][8 * c16], d, rstd);
        stage_split(buf ^ 1, d, rstd, kn0);
      }
      __builtin_amdgcn_sched_barrier(0);
      consume(i + 2);
      fetch(i + 3);
      if (lead)
        store(res, i);
      else if (i > 0)
        store(res, i - 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!lead) res = k_steps(buf);
    __syncthreads();
    ++i;
  }
  if (!lead) store(res, i - 1);
}

// Launches gated_split_kernel<MODE> over rows_r x span_k / 32 row tiles.
template <int MODE>
hipError_t launch_gated_split(const GatedArgs& a, hipStream_t stream) {
  constexpr int kSlices = GatedTraits<MODE>::kSlices;
  const int tiles_k = a.span_k / kGatedRows;
  const int64_t ntiles = (int64_t)a.rows_r * tiles_k;
  if (ntiles == 0) return hipSuccess;
  if (a.span_k % kGatedRows || a.span_k < a.rows_k || a.rows_k < 1 || ntiles > 0x7fffffffll)
    return hipErrorInvalidValue;
  if (a.rows_r > a.np) return hipErrorInvalidValue;
  int64_t cap = (int64_t)device_cu_count() / kSlices;
  if (cap >= 8) cap -= cap % 8;
  if (cap < 1) cap = 1;
  // whole rows per work-group
  const int streams = (int)(a.rows_r < cap ? a.rows_r : cap);
  hipLaunchKernelGGL(gated_split_kernel<MODE>, dim3(streams * kSlices), dim3(kGatedWaves * 64), 0,
                     stream, a, tiles_k, (int)ntiles, streams);
  return hipGetLastError();
}

}  // namespace fpx
