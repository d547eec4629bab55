// Pair-row projections on the CDNA4 16-bit matrix cores, FP32-accurate.
//
// kProjBlock fuses the pair LayerNorm into the prologue (one read of z, two
// register-level reductions per row on pivot-shifted values: mean, then the
// biased variance of the centred values) and the triangle-bias projection
// (4 wave reductions per row, DPP and lane-swap steps with no LDS traffic),
// and writes q (scaled by 1/sqrt(32)), k, v^T as scaled fp16 planes,
// sigmoid(g) and the bias (fragment order, bias_frag_index; once as is and
// once scaled by log2(e)) straight into the layouts the attention kernel
// reads.  The row addressing x + i*xs_i + j*xs_j makes the ending-node read
// of z^T free of copies.  kProjQkv and kProjOut are the plain row
// projections (q/k/v of the operator hook; the block's output projection).
#include "common.hpp"
#include "kernels.hpp"
#include "split.hpp"

#include <type_traits>

namespace fpx {
namespace {

constexpr int kRows = 32;            // pair rows per tile

// Stores one wave's 32 x 32 result tile.  Lane holds rows 4*half +
// 8*(r/4) + r%4 of the tile, column col_w of output group `group` (0 q, 1 k,
// 2 v, 3 g; kProjOut: always 0), head or column block hw.  Row offsets are
// compile-time constants once the lane's base includes its 4*half rows.
// e_head: the plane exponent of this wave's head (kProjBlock planes: every
// q, k and v^T tile of the head is scaled by 2^e_head, head_plane_exp).
template <int MODE>
__device__ __forceinline__ void store_tile(const ProjArgs& a, int tile, int tiles_j, int group,
                                           int hw, int col_w, float col_bias, int half, int l32,
                                           const f32x16& acc, int e_head) {
  const int i = tile / tiles_j;
  const int j0 = (tile % tiles_j) * kRows + 4 * half;
  if constexpr (MODE == kProjBlock) {
    // Plane layout (ProjArgs::qh): per (i, head) a slice of np * 128
    // bytes, the hi plane and then the lo plane of 16-bit values.
    const int64_t bh = (int64_t)i * kHeads + hw;
    const int64_t slice_bytes = (int64_t)a.np * 128;
    if (group == 0 || group == 1) {
      // q, k: scaled fp16 planes [np rows][32 channels] with the head's
      // inverse scale.
      const float scale = group == 0 ? a.q_scale : 1.0f;
      const int e = e_head;
      // (acc * scale) 2^e == acc * (scale 2^e): one rounding either way
      const float f = __builtin_ldexpf(scale, e);
      // Lane pairs (l32, l32 ^ 1) swap halves so that each lane stores one
      // 32-bit word per plane and row pair: the even lane channels l32 and
      // l32 + 1 of the pair's first row, the odd lane channels l32 - 1 and
      // l32 of its second row.
      const bool odd = l32 & 1;
      const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
      uint8_t* base = reinterpret_cast<uint8_t*>(group == 0 ? a.qh : a.kh) + bh * slice_bytes +
                      (int64_t)(j0 + odd) * 64 + (l32 - odd) * 2;
      typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const f32x2 x = {acc[r] * f, acc[r + 1] * f};
        const f16x2 hi = __builtin_convertvector(x, f16x2);
        const f16x2 lo = __builtin_convertvector(x - __builtin_convertvector(hi, f32x2), f16x2);
        const uint32_t hw_ = __builtin_bit_cast(uint32_t, hi), lw = __builtin_bit_cast(uint32_t, lo);
        const uint32_t ho = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hw_, 0xB1, 0xF, 0xF, false);
        const uint32_t lo_ = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lw, 0xB1, 0xF, 0xF, false);
        const int64_t row = 8 * (r >> 2) + (r & 3);
        *(uint32_t*)(base + row * 64) = __builtin_amdgcn_perm(ho, hw_, sel);
        *(uint32_t*)(base + (slice_bytes >> 1) + row * 64) = __builtin_amdgcn_perm(lo_, lw, sel);
      }
      if (half == 0 && l32 == 0)
        a.scales[(((int64_t)group * a.rows_i + i) * kHeads + hw) * (a.np >> 5) + tile % tiles_j] =
            __builtin_ldexpf(1.0f, -e);
    } else if (group == 2) {
      // v^T: fp16 planes [np / 32 tiles][32 channels][32 key positions],
      // every tile of the head scaled by 2^e_head, keys of a tile in the
      // order of the S^T accumulator registers (key group g of four at
      // position 16 (g / 4) + 4 (0, 2, 1, 3)[g % 4]).  This lane's keys
      // 8 rr + e + 4 half sit at positions 8 half + 4 rr + e (rr < 2) and
      // 16 + 8 half + 4 (rr - 2) + e.
      const int e = e_head;
      const float f = __builtin_ldexpf(1.0f, e);
      uint8_t* base = reinterpret_cast<uint8_t*>(a.vt) + bh * slice_bytes +
                      (int64_t)(tile % tiles_j) * 2048 + l32 * 64 + 16 * half;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        bf16x8 hi, lo;
        split_f16(f32x8{acc[8 * q + 0] * f, acc[8 * q + 1] * f, acc[8 * q + 2] * f,
                        acc[8 * q + 3] * f, acc[8 * q + 4] * f, acc[8 * q + 5] * f,
                        acc[8 * q + 6] * f, acc[8 * q + 7] * f},
                  hi, lo);
        *(bf16x8*)(base + 32 * q) = hi;
        *(bf16x8*)(base + (slice_bytes >> 1) + 32 * q) = lo;
      }
      if (half == 0 && l32 == 0)
        a.scales[(((int64_t)2 * a.rows_i + i) * kHeads + hw) * (a.np >> 5) + tile % tiles_j] =
            __builtin_ldexpf(1.0f, -e);
    } else {
      float* dst = a.gs + ((int64_t)i * a.np + j0) * kHidden + col_w;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        dst[(8 * (r >> 2) + (r & 3)) * kHidden] = sigmoidf_(acc[r] + col_bias);
    }
  } else {
    // Rows past rows_j exist only in the last tile of an outer row; the
    // branch is uniform, so full tiles store with no per-element tests.
    const bool full = (tile % tiles_j + 1) * kRows <= a.rows_j;
    float* dst;
    int64_t stride;
    float scale = 1.0f, add = 0.0f;
    if (MODE == kProjQkv) {
      const int64_t rows = (int64_t)a.rows_i * a.rows_j;
      dst = a.out + ((int64_t)group * rows + (int64_t)i * a.rows_j + j0) * kHidden + 32 * hw + l32;
      stride = kHidden;
      if (group == 0) scale = a.q_scale;
    } else {
      dst = a.out + (int64_t)i * a.os_i + (int64_t)j0 * a.os_j + col_w;
      stride = a.os_j;
      add = col_bias;
    }
    // The residual update adds the rounded update to the old value, as
    // the native z += dz does.
    const bool residual = MODE == kProjOut && a.accumulate != 0;
    auto put = [&](float* d, float v) { *d = residual ? *d + v : v; };
    if (full) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        put(dst + (int64_t)(8 * (r >> 2) + (r & 3)) * stride, acc[r] * scale + add);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dj = 8 * (r >> 2) + (r & 3);
        if (j0 + dj < a.rows_j) put(dst + (int64_t)dj * stride, acc[r] * scale + add);
      }
    }
  }
}

// The projections run on v_mfma_f32_32x32x16_f16 with every FP32 operand
// held as scaled fp16 (hi, lo) planes (split.hpp): the three terms hi hi,
// hi lo, lo hi take 24 MFMAs per 32 x 32 tile over the 128 input channels,
// against 64 v_mfma_f32_32x32x2_f32 of 8x less work each, with an error per
// product below an FP32 dot product's.  Scales are powers of two:
//   - each weight column by 2^ew, its max |w| in [2^14, 2^15);
//   - kProjBlock's q, k and v^T outputs by one 2^e per head (store_tile's
//     e_head, from a bound on the values of normalised rows);
//   - LN rows (kProjBlock) by one 2^ex per launch from the LN affine: the
//     centred, normalised row has 2-norm sqrt(128), so |y_c| <= sqrt(128)
//     |ln_w_c| + |ln_b_c|; ln_w and ln_b are pre-scaled, so the scaled row
//     costs nothing;
//   - other rows (kProjQkv, kProjOut) each by their own 2^er.
// Results are scaled back with ldexp, exactly.  A wave's two weight planes
// take 64 VGPRs and a work-group covers a slice of the output columns: the
// block's 512 q/k/v/g columns (and the 384 of kProjQkv) are cut into two
// slices of 8 (6) waves, one work-group per CU, and the two work-groups of a
// slice pair run on the same XCD over the same row tiles, so the second read
// of each row tile comes from L2.  Each slice normalises its rows itself
// (kProjBlock); slice s projects triangle-bias heads 2s and 2s + 1.  Row
// tiles are split into the planes once, on their way into LDS.
template <int MODE>
struct SplitTraits;
template <>
struct SplitTraits<kProjBlock> {
  static constexpr int kWaves = 8;  // 256 of q, k, v, g's 512 columns
  static constexpr int kSlices = 2;
  static constexpr int kMinBlocks = 1;
};
template <>
struct SplitTraits<kProjQkv> {
  static constexpr int kWaves = 6;  // 192 of q, k, v's 384 columns
  static constexpr int kSlices = 2;
  static constexpr int kMinBlocks = 2;
};
template <>
struct SplitTraits<kProjOut> {
  static constexpr int kWaves = 4;  // the 128 output channels
  static constexpr int kSlices = 1;
  static constexpr int kMinBlocks = 3;
};

constexpr int kPlaneRow = kChannels + 8;  // bf16 per LDS row: 272 bytes, conflict-free b128 reads
typedef __bf16 XPlane[kRows][kPlaneRow];

template <int MODE, bool kFew>
__global__ __launch_bounds__(SplitTraits<MODE>::kWaves * 64, SplitTraits<MODE>::kMinBlocks) void
projection_split_kernel(ProjArgs a, int tiles_j, int ntiles, int streams) {
  using T = SplitTraits<MODE>;
  constexpr int NW = T::kWaves;
  constexpr int kThreads = NW * 64;
  constexpr bool kLn = MODE == kProjBlock;
  static_assert(!kLn || NW * 4 == kRows, "LN mode: 4 rows per wave, 16 lanes per row");
  constexpr int kVecs = kRows * kChannels / 4;              // float4 per tile
  constexpr int kLoads = (kVecs + kThreads - 1) / kThreads; // kProjQkv, kProjOut
  // Two row tiles of two planes: the MFMAs read one while the next is
  // normalised and split into the other, so a tile needs one barrier.
  __shared__ __attribute__((aligned(16))) XPlane xs[2][2];
  // kProjQkv, kProjOut: each staged row's plane exponent er.
  __shared__ __attribute__((aligned(16))) int rexp[2][kRows];
  // LN mode: raw rows of the next tile.  Each wave reads and rewrites only
  // its own rows, so the buffer needs no barrier of its own.
  __shared__ __attribute__((aligned(16))) float raw[kLn ? kRows : 1][kChannels + 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  // Consecutive logical indices share an XCD: the slices of a stream are
  // neighbours (the grid is a multiple of 16 when the tiles allow it).
  const uint32_t logical = xcd_remap(blockIdx.x, gridDim.x);
  const int slice = (int)(logical % T::kSlices);
  const int first = (int)(logical / T::kSlices);
  const int cb = __builtin_amdgcn_readfirstlane(slice * NW + w);  // 32-column block
  const int group = cb >> 2;
  const int hw = cb & 3;

  // kProjBlock planes: one plane exponent per head for q, k and v^T (this
  // wave's 32 columns are one head of one group), from a bound on the
  // values instead of each tile's maximum.  Every LayerNorm output obeys
  // |y_c| <= sqrt(128) |ln_w_c| + |ln_b_c|, so a column's values obey
  // |x W^T| <= sum_c |W_c| (sqrt(128) |ln_w_c| + |ln_b_c|) (times 1/sqrt(32)
  // for q).  With every tile of a head at one scale, the attention's product
  // scale and v^T exponent are the same for every key tile.  Accuracy does
  // not depend on the scale: the fp16 planes keep 22 significant bits
  // relative to each value down to 2^-14 of the scaled unit, and the values
  // of normalised rows lie within a few binary orders of the bound.
  // Large launches sum the bound here, in a loop of its own loads; launches
  // of a few tiles per work-group (kFew), where this prologue is a visible
  // part of the run, sum the weights loaded for the planes below against a
  // table of the channel bounds in LDS, the same terms in the same order.
  const int e_loop = [&] {
    if (MODE != kProjBlock || group > 2 || kFew) return 0;
    const float* src = a.w[group] + (int64_t)(32 * hw + l32) * kChannels + 8 * half;
    float s = 0.f;
    // a loop, not unrolled: few registers live beside the weight planes
#pragma unroll 1
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 16 * t + 8 * half + e;
        const float yb = 11.3137085f * __builtin_fabsf(a.ln_w ? a.ln_w[c] : 1.f) +
                         __builtin_fabsf(a.ln_b ? a.ln_b[c] : 0.f);
        s = __builtin_fmaf(__builtin_fabsf(src[16 * t + e]), yb, s);
      }
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, s),
                                                     __builtin_bit_cast(unsigned, s), false, false);
    s = __builtin_bit_cast(float, (unsigned)sw[0]) + __builtin_bit_cast(float, (unsigned)sw[1]);
    // the margin covers the rounding of the LN output, the sums and q's scale
    const float bound = wave_max(s) * (group == 0 ? a.q_scale : 1.0f) * (1.0f + 0x1p-8f);
    if (group == 2) return value_plane_exp(bound);
    const int e = plane_exp(bound);
    return e < -kPlaneExpMax ? -kPlaneExpMax : e > kPlaneExpMax ? kPlaneExpMax : e;
  }();
  constexpr bool kTable = MODE == kProjBlock && kFew;
  __shared__ __attribute__((aligned(16))) float ybound[kTable ? kChannels : 1];
  if constexpr (kTable) {
    if (tid < kChannels)
      ybound[tid] = 11.3137085f * __builtin_fabsf(a.ln_w ? a.ln_w[tid] : 1.f) +
                    __builtin_fabsf(a.ln_b ? a.ln_b[tid] : 0.f);
    __syncthreads();
  }
  int e_table = 0;

  // Weight planes: B[k][col] for col = 32*hw + l32 of group `group`, lane
  // holding channels 16t + 8*half + e of k step t, scaled by 2^ew (the
  // column's max |w| over both halves of the wave).
  bf16x8 wh[8], wl[8];
  int ew;
  {
    const float* src = a.w[group] + (int64_t)(32 * hw + l32) * kChannels + 8 * half;
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
    if constexpr (kTable) {
      if (group <= 2) {
        float s = 0.f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const f32x8 yb = *(const f32x8*)&ybound[16 * t + 8 * half];
#pragma unroll
          for (int e = 0; e < 8; ++e) s = __builtin_fmaf(__builtin_fabsf(wv[t][e]), yb[e], s);
        }
        const auto ss = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, s),
                                                         __builtin_bit_cast(unsigned, s), false, false);
        s = __builtin_bit_cast(float, (unsigned)ss[0]) + __builtin_bit_cast(float, (unsigned)ss[1]);
        const float bound = wave_max(s) * (group == 0 ? a.q_scale : 1.0f) * (1.0f + 0x1p-8f);
        if (group == 2) {
          e_table = value_plane_exp(bound);
        } else {
          const int e = plane_exp(bound);
          e_table = e < -kPlaneExpMax ? -kPlaneExpMax : e > kPlaneExpMax ? kPlaneExpMax : e;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) split_f16(ldexp8(wv[t], ew), wh[t], wl[t]);
  }
  const int e_head = kFew ? e_table : e_loop;
  const int col_w = MODE == kProjOut ? 32 * w + l32 : 32 * hw + l32;
  const float col_bias = (MODE != kProjQkv && a.b_g != nullptr) ? a.b_g[col_w] : 0.f;

  // LN mode: 16 lanes per row, lane c16 = lane % 16 holding channels
  // 8*c16 .. 8*c16 + 7 of row 4*w + lane/16; the LN affine and this slice's
  // two triangle-bias heads for those channels.
  const int c16 = lane & 15;
  const int lrow = 4 * w + (lane >> 4);
  f32x8 lnw, lnb, wb0, wb1;
  int ex = 0;  // LN mode: plane exponent of every row
  if constexpr (kLn) {
    float bound = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lnw[e] = a.ln_w ? a.ln_w[8 * c16 + e] : 1.f;
      lnb[e] = a.ln_b ? a.ln_b[8 * c16 + e] : 0.f;
      wb0[e] = a.w_bias[(2 * slice) * kChannels + 8 * c16 + e];
      wb1[e] = a.w_bias[(2 * slice + 1) * kChannels + 8 * c16 + e];
      bound = __builtin_elementwise_maximum(
          bound, 11.3137085f * __builtin_fabsf(lnw[e]) + __builtin_fabsf(lnb[e]));
    }
    // |y_c| <= sqrt(128) |ln_w_c| + |ln_b_c| up to FP32 rounding (< 1e-5
    // relative); the margin keeps |y| 2^ex below 2^15.
    ex = plane_exp(wave_max(bound) * (1.0f + 0x1p-10f));
    lnw = ldexp8(lnw, ex);
    lnb = ldexp8(lnb, ex);
  }

  // kProjBlock: running max |result| of this wave's group (q unscaled, k, v)
  // and max |bias| of the values this lane stores, for the magnitude record.
  float out_max = 0.f, bias_max = 0.f;
  auto note = [&](const f32x16& r) {
    if (MODE == kProjBlock && group < 3 && a.magnitudes != nullptr) {
#pragma unroll
      for (int e = 0; e < 16; ++e) out_max = __builtin_elementwise_maximum(out_max, __builtin_fabsf(r[e]));
    }
  };

  // Row loads in flight (LN mode: the tile after next).
  f32x8 stage_ln;
  f32x4 stage_vec[kLn ? 1 : kLoads];

  // Outer row i and first pair row j0 of a tile.
  auto origin = [&](int tile, int& i, int& j0) {
    i = tile / tiles_j;
    j0 = (tile - i * tiles_j) * kRows;
  };

  // LN mode: loads with no branches (tile clamped to the last one, row to
  // the last valid row; stage_split zeroes rows past rows_j), so every
  // staged slot holds finished loads on every path.
  auto fetch_ln = [&](f32x8& slot, int tile) {
    int i, j0;
    origin(tile < ntiles ? tile : ntiles - 1, i, j0);
    const int j = min(j0 + lrow, a.rows_j - 1);
    const float* src = a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j + 8 * c16;
    const f32x4 u = *(const f32x4*)src;
    const f32x4 v = *(const f32x4*)(src + 4);
    slot = f32x8{u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
  };

  auto fetch = [&](int tile) {
    int i, j0;
    origin(tile, i, j0);
#pragma unroll
    for (int t = 0; t < kLoads; ++t) {
      const int idx = tid + t * kThreads;
      const int j = j0 + (idx >> 5);
      stage_vec[t] = (idx < kVecs && j < a.rows_j)
                         ? *(const f32x4*)(a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j +
                                           (idx & 31) * 4)
                         : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  // LayerNorm statistics of the staged rows (two-pass on values shifted by
  // the row's first channel, as ln_stats_c128), returning the centred values
  // and 1/sqrt(biased var + eps).
  auto ln_stats = [&](const f32x8& raw, f32x8& d, float& rstd) {
    const float pivot = row16_first(raw[0]);
    const f32x8 sh = raw - pivot;
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

  // Normalises, splits and writes the staged rows into planes `buf`;
  // returns this lane's triangle-bias value (head 2*slice + c16 for c16 < 2,
  // 0 for rows past rows_j), stored later by store_bias.
  // The normalised row comes out scaled by 2^ex (ln_w, ln_b pre-scaled):
  // every rounding of y and of the bias sum scales with it exactly.
  auto stage_split = [&](int buf, const f32x8& d, float rstd, int j0) -> float {
    const bool valid = j0 + lrow < a.rows_j;
    f32x8 y = d * rstd * lnw + lnb;
    if (!valid) y = f32x8{};
    bf16x8 hi, lo;
    split_f16(y, hi, lo);
    *(bf16x8*)&xs[buf][0][lrow][8 * c16] = hi;
    *(bf16x8*)&xs[buf][1][lrow][8 * c16] = lo;
    float p0 = 0.f, p1 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p0 += y[e] * wb0[e];
      p1 += y[e] * wb1[e];
    }
    p0 = row16_sum(p0);
    p1 = row16_sum(p1);
    return __builtin_ldexpf(c16 == 0 ? p0 : p1, -ex);
  };

  auto store_bias = [&](float v, int i, int j0) {
    if (c16 < 2) {
      bias_max = __builtin_elementwise_maximum(bias_max, __builtin_fabsf(v));
      const int j = j0 + lrow;
      const int64_t at = bias_frag_index(2 * slice + c16, i, j, a.np);
      a.tri_bias[at] = v;
      a.tri_bias_l2[at] = v * kLog2e;
    }
  };

  // A row's 32 float4 sit in one 32-lane half of a wave (whole waves skip
  // the idx >= kVecs slots), so the row max is a half-wave reduction.
  auto stage_vecs = [&](int buf) {
#pragma unroll
    for (int t = 0; t < kLoads; ++t) {
      const int idx = tid + t * kThreads;
      if (idx < kVecs) {
        const f32x4 x = stage_vec[t];
        const float m = half_max(__builtin_elementwise_maximum(
            __builtin_elementwise_maximum(__builtin_fabsf(x.x), __builtin_fabsf(x.y)),
            __builtin_elementwise_maximum(__builtin_fabsf(x.z), __builtin_fabsf(x.w))));
        const int er = plane_exp(m);
        bf16x4 hi, lo;
        split_f16(ldexp4(x, er), hi, lo);
        const int row = idx >> 5;
        const int c4 = (idx & 31) * 4;
        *(bf16x4*)&xs[buf][0][row][c4] = hi;
        *(bf16x4*)&xs[buf][1][row][c4] = lo;
        if ((idx & 31) == 0) rexp[buf][row] = er;
      }
    }
  };

  // Scales a wave's 32 x 32 result back: ldexp by -(row exponent + ew).
  auto unscale = [&](f32x16 r, int buf) -> f32x16 {
    if constexpr (kLn) {
#pragma unroll
      for (int e = 0; e < 16; ++e) r[e] = __builtin_ldexpf(r[e], -(ex + ew));
    } else {
      typedef int i32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const i32x4 er = *(const i32x4*)&rexp[buf][8 * rr + 4 * half];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[4 * rr + e] = __builtin_ldexpf(r[4 * rr + e], -(er[e] + ew));
      }
    }
    return r;
  };

  // One 16-deep k step of the 32 x 32 tile, A[row][k] = the row planes; two
  // accumulation chains, swapped every step, so consecutive MFMAs do not
  // wait on each other.
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

  __builtin_amdgcn_s_waitcnt(0);
  int tile = first;  // first < streams <= ntiles: every work-group has a tile
  int next = tile + streams;
  if constexpr (kLn) {
    // Iteration k computes tile T_k = first + k*streams from planes k&1 and
    // normalises T_{k+1} from the raw LDS rows into the other planes.  The
    // two waves sharing a SIMD run the iteration's halves in opposite
    // orders, so one issues its k steps while the other normalises and
    // stores: "lead" waves (0-3) run the k steps first; "trail" waves (4-7)
    // normalise first, run their k steps last and store the result in the
    // next iteration.  Per wave, the global accesses of an iteration are
    // issued together, in this order: the registers holding T_{k+2}'s rows
    // (loaded one iteration earlier) are copied to the raw rows, T_{k+3}'s
    // rows are loaded, then the bias and results are stored.  The copy waits
    // for all of the wave's earlier global accesses (loads and stores share
    // one counter), which were issued an iteration ago.
    const bool lead = w < NW / 2;
    int i0, j00;
    origin(tile, i0, j00);
    fetch_ln(stage_ln, tile);
    {
      f32x8 d;
      float rstd;
      ln_stats(stage_ln, d, rstd);
      store_bias(stage_split(0, d, rstd, j00), i0, j00);
    }
    fetch_ln(stage_ln, next);
    *(f32x8*)&raw[lrow][8 * c16] = stage_ln;
    fetch_ln(stage_ln, next + streams);
    __syncthreads();

    auto k_steps = [&](int buf) -> f32x16 {
      f32x16 c0 = {}, c1 = {};
#pragma unroll
      for (int t = 0; t < 8; ++t) mfma_step(buf, t, c0, c1);
      return unscale(c0 + c1, buf);
    };
    // Normalises T_{k+1} (when it exists) into planes buf ^ 1, then issues
    // the wave's global accesses; `result`/`result_tile` are stored last.
    auto other_half = [&](int buf, const f32x16& result, int result_tile) {
      const bool more = next < ntiles;
      int ni, nj0;
      origin(more ? next : tile, ni, nj0);
      float bias = 0.f;
      if (more) {
        f32x8 d;
        float rstd;
        ln_stats(*(const f32x8*)&raw[lrow][8 * c16], d, rstd);
        bias = stage_split(buf ^ 1, d, rstd, nj0);
      }
      __builtin_amdgcn_sched_barrier(0);
      *(f32x8*)&raw[lrow][8 * c16] = stage_ln;
      fetch_ln(stage_ln, next + 2 * streams);
      if (more) store_bias(bias, ni, nj0);
      if (result_tile >= 0) {
        note(result);
        store_tile<MODE>(a, result_tile, tiles_j, group, hw, col_w, col_bias, half, l32, result,
                         e_head);
      }
      __builtin_amdgcn_sched_barrier(0);
    };

    // Only the k steps sit in wave-dependent branches, so the row staging
    // keeps one register assignment on every path.  `res` is this tile's
    // result on lead waves and the previous tile's on trail waves.
    f32x16 res = {};
    for (int buf = 0; tile < ntiles; buf ^= 1) {
      if (lead) res = k_steps(buf);
      const int result_tile = lead ? tile : tile - streams;
      other_half(buf, res, result_tile >= first ? result_tile : -1);
      if (!lead) res = k_steps(buf);
      __syncthreads();
      tile = next;
      next += streams;
    }
    if (!lead && tile - streams >= first) {
      note(res);
      store_tile<MODE>(a, tile - streams, tiles_j, group, hw, col_w, col_bias, half, l32, res,
                       e_head);
    }
    if (a.magnitudes != nullptr) {
      const float om = wave_max(out_max), bm = wave_max(bias_max);
      if constexpr (!kFew) {
        // Wave maxima (NaN-propagating), one atomic per wave and record word.
        if (lane == 0) {
          if (group < 3)
            atomicMax(&a.magnitudes[group],
                      __builtin_bit_cast(uint32_t, group == 0 ? om * a.q_scale : om));
          atomicMax(&a.magnitudes[3], __builtin_bit_cast(uint32_t, bm));
          if (blockIdx.x == 0 && w == 0) a.magnitudes[4] = 1u;
        }
      } else {
        // The work-group's maxima first, then one atomic per record word:
        // waves 0-3 hold one group, waves 4-7 the next.  The work-groups of
        // a launch of few tiles finish together, and atomics from every
        // wave on the same words would wait on each other.
        __shared__ uint32_t wg_max[NW][2];
        if (lane == 0) {
          wg_max[w][0] = __builtin_bit_cast(uint32_t, group == 0 ? om * a.q_scale : om);
          wg_max[w][1] = __builtin_bit_cast(uint32_t, bm);
        }
        __syncthreads();
        if (tid < 3) {
          // Non-negative floats (and NaN above them) order as their bits.
          const int from = tid == 1 ? NW / 2 : 0, to = tid == 0 ? NW / 2 : NW;
          uint32_t r = 0;
          for (int v = from; v < to; ++v) r = max(r, wg_max[v][tid == 2]);
          const int word = tid == 2 ? 3 : (slice * NW + from) >> 2;
          if (word < 3 || tid == 2) atomicMax(&a.magnitudes[word], r);
          if (blockIdx.x == 0 && tid == 0) a.magnitudes[4] = 1u;
        }
      }
    }
  } else {
    fetch(tile);
    stage_vecs(0);
    if (next < ntiles) fetch(next);
    __syncthreads();
    for (int buf = 0; tile < ntiles; buf ^= 1) {
      f32x16 c0 = {}, c1 = {};
#pragma unroll
      for (int t = 0; t < 8; ++t) mfma_step(buf, t, c0, c1);
      if (next < ntiles) {
        stage_vecs(buf ^ 1);
        if (next + streams < ntiles) fetch(next + streams);
      }
      store_tile<MODE>(a, tile, tiles_j, group, hw, col_w, col_bias, half, l32, unscale(c0 + c1, buf),
                       e_head);
      __syncthreads();
      tile = next;
      next += streams;
    }
  }
}

template <int MODE>
hipError_t launch_split(const ProjArgs& a, hipStream_t stream) {
  using T = SplitTraits<MODE>;
  const int tiles_j = (int)(round_up(a.span_j, kRows) / kRows);
  const int64_t ntiles = (int64_t)a.rows_i * tiles_j;
  if (ntiles == 0) return hipSuccess;
  if (ntiles > 0x7fffffffll) return hipErrorInvalidValue;
  // Streams of row tiles: one work-group per slice each, as many as fit
  // (rounded down to a multiple of 8 so the grid spreads evenly over the
  // XCDs and slice pairs never straddle two of them).
  int64_t cap = (int64_t)device_cu_count() * T::kMinBlocks / T::kSlices;
  if (cap >= 8) cap -= cap % 8;
  const int streams = (int)(ntiles < cap ? ntiles : cap);
  // The block projection at up to 64 row tiles per work-group (N up to
  // about 512) takes the variant with the shorter prologue and epilogue
  // (kFew); larger launches keep the other, whose tile loop was tuned.
  if constexpr (MODE == kProjBlock) {
    if (ntiles <= (int64_t)64 * streams) {
      hipLaunchKernelGGL((projection_split_kernel<MODE, true>), dim3(streams * T::kSlices),
                         dim3(T::kWaves * 64), 0, stream, a, tiles_j, (int)ntiles, streams);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((projection_split_kernel<MODE, false>), dim3(streams * T::kSlices),
                     dim3(T::kWaves * 64), 0, stream, a, tiles_j, (int)ntiles, streams);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_projection(int mode, const ProjArgs& a, hipStream_t stream) {
  switch (mode) {
    case kProjBlock:
      if (a.scales == nullptr) return hipErrorInvalidValue;
      return launch_split<kProjBlock>(a, stream);
    case kProjQkv:
      return launch_split<kProjQkv>(a, stream);
    case kProjOut:
      return launch_split<kProjOut>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace fpx
