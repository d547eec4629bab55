// Triangle multiplicative update (outgoing and incoming) on the CDNA4 16-bit
// matrix cores, FP32-accurate (scaled fp16 hi/lo planes, three terms per
// product), c_z = c_hidden = 128.
//
//   a[r, k, c] = mask[r, k] * sigmoid(LN_in(z) W_a_g^T + b)[c] * (LN_in(z) W_a_p^T + b)[c]
//   b[r, k, c] = the same with the b weights
//   x[i, j, c] = sum_k a[i, k, c] b[j, k, c]
//   u[i, j, :] = sigmoid(LN_in(z[i, j]) W_g^T + b_g) * (LN_out(x[i, j]) W_z^T + b_z)
//   out        = u, or z + u (the residual update)
//
// in the contraction frame (r, k): z[r, k] for the outgoing update and
// z[k, r] for the incoming one, so both directions are one kernel chain; the
// incoming read of z^T goes through strides, with no transposed copy.
//
// Three launches:
//   gated_split_kernel<kGatedTriMul>
//                          LN_in, the four 128x128 projections, sigmoid gates
//                          and the mask; writes a and b channel-blocked (each
//                          channel's rows as 32-key runs, gated_split.hpp)
//                          with each (channel, row)'s max |value|
//   trimul_contract_kernel x_c = A_c B_c^T for the 128 channels: a batched
//                          GEMM on 128 x 128 output tiles, key stages
//                          double-buffered in LDS, XCD-aware tile order
//   trimul_finish_split_kernel
//                          LN_out(x) W_z^T and LN_in(z) W_g^T for 32 pairs
//                          per tile, the sigmoid gate and the in-place write
#include "common.hpp"
#include "gated_split.hpp"

#include "gemm.hpp"
#include "kernels.hpp"

namespace fpx {
namespace {

constexpr int kRows = 32;                 // pair rows per finish tile

// ----------------------------------------------------------- contraction
// One work-group = (channel c, 128 rows i, 128 columns j) of x_c = A_c B_c^T
// (gemm_nt_128_f16 over the np keys).  Work-groups of one channel are consecutive
// in the logical order, and xcd_remap gives each XCD a contiguous range, so
// the A and B row panels a range touches stay in that XCD's L2.
// gemm_nt_128_f16 (16-bit matrix cores, scaled fp16 planes), with each row's
// exponent from the row maxima the projection recorded, on the
// channel-blocked a and b of gated_split_kernel<kGatedTriMul> (channel c's
// row r at ((c / 16) np / 32 np + r) 512 + (c % 16) 32, rows 512 floats
// apart, 32-key runs np * 512 floats apart).
__global__ __launch_bounds__(256, 2) void trimul_contract_kernel(const float* __restrict__ pa,
                                                                 const float* __restrict__ pb,
                                                                 const uint32_t* __restrict__ rowmax,
                                                                 float* __restrict__ x, int n,
                                                                 int np, int tiles,
                                                                 uint32_t total) {
  __shared__ __attribute__((aligned(16))) F16Stage As[2];
  __shared__ __attribute__((aligned(16))) F16Stage Bs[2];
  __shared__ int ea[kGemmTile], eb[kGemmTile];

  const uint32_t logical = xcd_remap(blockIdx.x, total);
  const int per_channel = tiles * tiles;
  const int c = (int)(logical / per_channel);
  const int rem = (int)(logical % per_channel);
  const int i0 = (rem / tiles) * kGemmTile;
  const int j0 = (rem % tiles) * kGemmTile;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  f32x16 acc[2][2] = {};
  {
    const int t = threadIdx.x;
    const uint32_t* rm = rowmax + ((int64_t)(t >> 7) * kChannels + c) * np + ((t >> 7) ? j0 : i0);
    (t >> 7 ? eb : ea)[t & 127] = plane_exp(__builtin_bit_cast(float, rm[t & 127]));
    __syncthreads();
    const int64_t run = 512 * (int64_t)np;  // floats between a row's 32-key runs
    const int64_t cbase = (int64_t)(c >> 4) * (np / 32) * run + (c & 15) * 32;
    gemm_nt_128_f16(pa + cbase + 512 * (int64_t)i0, 512, pb + cbase + 512 * (int64_t)j0, 512,
                    run, np / kSplitK, As, Bs, ea, eb, acc);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int ej = eb[(w & 1) * 64 + 32 * cb + l32];
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[rb][cb][r] = __builtin_ldexpf(acc[rb][cb][r], -(ea[(w >> 1) * 64 + 32 * rb + mfma_row(r, half)] + ej));
      }
    }
  }

  // x is blocked [n][np / 32][128 channels][32 columns]: the finish kernel
  // reads one contiguous 16 KB block per 32-pair tile.
  const int64_t nb = np / 32;
  const int wi = (w >> 1) * 64;
  const int wj = (w & 1) * 64;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int j = j0 + wj + 32 * cb + l32;
    if (j >= n) continue;
    float* col = x + ((int64_t)(j >> 5) * kChannels + c) * 32 + (j & 31);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wi + 32 * rb + mfma_row(r, half);
        if (i < n) col[(int64_t)i * nb * kChannels * 32] = acc[rb][cb][r];
      }
    }
  }
}

// ---------------------------------------------------------------- finish
// The finish on v_mfma_f32_16x16x32_f16 with power-of-two scaled fp16 (hi,
// lo) planes of both normalised inputs and both weights (three terms, FP32
// rounding level).
// The 16 x 16 shape lets a wave hold W_z and W_g planes for 16 output
// channels in 96 VGPRs while the value (LN_out(x) W_z^T) and gate
// (LN_in(z) W_g^T) results of one channel land in the same lane, so a
// work-group of 8 waves covers all 128 channels of a 32-pair tile.
// Persistent, one work-group per CU, with the pipeline of the split
// projections: raw x (transposed on its way in) and z rows are staged
// through per-wave LDS rows and waited an iteration after their loads;
// waves 0-3 run their k steps first, waves 4-7 last.  With accumulate, the
// residual values are loaded an iteration ahead of their stores.
constexpr int kFinPlaneRow = kChannels + 8;  // bf16 per LDS row: 272 bytes

__global__ __launch_bounds__(512, 1) void trimul_finish_split_kernel(TriMulArgs a, int tiles_j,
                                                                     int ntiles) {
  __shared__ __attribute__((aligned(16))) __bf16 px[2][2][kRows][kFinPlaneRow];
  __shared__ __attribute__((aligned(16))) __bf16 pz[2][2][kRows][kFinPlaneRow];
  __shared__ __attribute__((aligned(16))) float raw_x[kRows][kChannels + 4];
  __shared__ __attribute__((aligned(16))) float raw_z[kRows][kChannels + 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15;
  const int g4 = lane >> 4;          // 16-lane group: k group of the operands, row group of D
  const int ch = 16 * w + l16;       // output channel of this lane
  const int n = a.n;
  const int64_t nb = a.np / 32;
  const bool residual = a.accumulate != 0;

  // Weight planes: B[k][c] = W[c][k], lane holding keys 32t + 8 g4 + e, as
  // fp16 (hi, lo) of W[c] 2^ew (each channel row's max |w| over the four
  // lanes l16 + 16 g4 that hold it).
  bf16x8 wz[2][4], wg[2][4];
  int ewz, ewg;
  {
    f32x8 vz[4], vg[4];
    float mz = 0.f, mg = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float* sz = a.w_z + (int64_t)ch * kChannels + 32 * t + 8 * g4;
      const float* sg = a.w_g + (int64_t)ch * kChannels + 32 * t + 8 * g4;
      const f32x4 z0 = *(const f32x4*)sz, z1 = *(const f32x4*)(sz + 4);
      const f32x4 g0 = *(const f32x4*)sg, g1 = *(const f32x4*)(sg + 4);
      vz[t] = f32x8{z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
      vg[t] = f32x8{g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        mz = __builtin_elementwise_maximum(mz, __builtin_fabsf(vz[t][e]));
        mg = __builtin_elementwise_maximum(mg, __builtin_fabsf(vg[t][e]));
      }
    }
    auto rows4_max = [](float v) {  // lanes l, l ^ 16, l ^ 32, l ^ 48
      const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v),
                                                      __builtin_bit_cast(unsigned, v), false, false);
      v = __builtin_elementwise_maximum(__builtin_bit_cast(float, (unsigned)s[0]),
                                        __builtin_bit_cast(float, (unsigned)s[1]));
      const auto u = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                      __builtin_bit_cast(unsigned, v), false, false);
      return __builtin_elementwise_maximum(__builtin_bit_cast(float, (unsigned)u[0]),
                                           __builtin_bit_cast(float, (unsigned)u[1]));
    };
    ewz = plane_exp(rows4_max(mz));
    ewg = plane_exp(rows4_max(mg));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      split_f16(ldexp8(vz[t], ewz), wz[0][t], wz[1][t]);
      split_f16(ldexp8(vg[t], ewg), wg[0][t], wg[1][t]);
    }
  }
  const float bz = a.b_z ? a.b_z[ch] : 0.f;
  const float bg = a.b_g ? a.b_g[ch] : 0.f;

  // LN lanes: 16 per row, lane c16 = l16 holding channels 8 c16 .. +7 of
  // tile row lrow.
  const int lrow = 4 * w + g4;
  f32x8 lnw_in, lnb_in, lnw_out, lnb_out;
  float bound_in = 0.f, bound_out = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c = 8 * l16 + e;
    lnw_in[e] = a.ln_in_w ? a.ln_in_w[c] : 1.f;
    lnb_in[e] = a.ln_in_b ? a.ln_in_b[c] : 0.f;
    lnw_out[e] = a.ln_out_w ? a.ln_out_w[c] : 1.f;
    lnb_out[e] = a.ln_out_b ? a.ln_out_b[c] : 0.f;
    bound_in = __builtin_elementwise_maximum(
        bound_in, 11.3137085f * __builtin_fabsf(lnw_in[e]) + __builtin_fabsf(lnb_in[e]));
    bound_out = __builtin_elementwise_maximum(
        bound_out, 11.3137085f * __builtin_fabsf(lnw_out[e]) + __builtin_fabsf(lnb_out[e]));
  }
  // LN rows as fp16 planes scaled by one power of two per input: |y_c| <=
  // sqrt(128) |ln_w_c| + |ln_b_c| up to FP32 rounding (pre-scaled affines).
  const int ex_in = plane_exp(wave_max(bound_in) * (1.0f + 0x1p-10f));
  const int ex_out = plane_exp(wave_max(bound_out) * (1.0f + 0x1p-10f));
  lnw_in = ldexp8(lnw_in, ex_in);
  lnb_in = ldexp8(lnb_in, ex_in);
  lnw_out = ldexp8(lnw_out, ex_out);
  lnb_out = ldexp8(lnb_out, ex_out);

  auto origin = [&](int tile, int& i, int& jb) {
    i = tile / tiles_j;
    jb = tile - i * tiles_j;
  };

  // Loads of one tile: x chunks x[c][4w .. 4w+3] for c = lane, lane + 64 of
  // the tile's contiguous 16 KB block (this wave's 4 rows, transposed at
  // the copy), and z row lrow (clamped to n - 1), channels 8 l16 .. +7.
  f32x4 sx[2];
  f32x8 sz_raw;
  auto fetch = [&](int tile) {
    int i, jb;
    origin(tile < ntiles ? tile : ntiles - 1, i, jb);
    const float* xb = a.x + ((int64_t)i * nb + jb) * kChannels * 32 + 4 * w;
    sx[0] = *(const f32x4*)(xb + (int64_t)lane * 32);
    sx[1] = *(const f32x4*)(xb + (int64_t)(lane + 64) * 32);
    const int j = min(jb * kRows + lrow, n - 1);
    const float* zr = a.z + (int64_t)i * a.zs_i + (int64_t)j * a.zs_j + 8 * l16;
    const f32x4 u = *(const f32x4*)zr;
    const f32x4 v = *(const f32x4*)(zr + 4);
    sz_raw = f32x8{u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
  };
  auto copy_raw = [&]() {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e) raw_x[4 * w + e][lane + 64 * q] = sx[q][e];
    }
    *(f32x8*)&raw_z[lrow][8 * l16] = sz_raw;
  };

  auto ln_split = [&](const f32x8& rawv, float eps, const f32x8& gw, const f32x8& gb, bool valid,
                      __bf16 (*planes)[kRows][kFinPlaneRow]) {
    const float pivot = row16_first(rawv[0]);
    const f32x8 sh = rawv - pivot;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += sh[e];
    const f32x8 d = sh - row16_sum(s) * (1.0f / kChannels);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) q += d[e] * d[e];
    const float rstd = __builtin_amdgcn_rsqf(row16_sum(q) * (1.0f / kChannels) + eps);
    f32x8 y = d * rstd * gw + gb;
    if (!valid) y = f32x8{};
    bf16x8 hi, lo;
    split_f16(y, hi, lo);
    *(bf16x8*)&planes[0][lrow][8 * l16] = hi;
    *(bf16x8*)&planes[1][lrow][8 * l16] = lo;
  };
  // Normalises the raw rows of the tile whose first pair row is j0 into
  // planes buf.  Rows past n (never stored) are zeroed.
  auto normalise = [&](int buf, int j0) {
    const bool valid = j0 + lrow < n;
    ln_split(*(const f32x8*)&raw_x[lrow][8 * l16], a.eps_out, lnw_out, lnb_out, valid, px[buf]);
    ln_split(*(const f32x8*)&raw_z[lrow][8 * l16], a.eps_in, lnw_in, lnb_in, valid, pz[buf]);
  };

  // acc[rb][0]: value, acc[rb][1]: gate, rows 16 rb + 4 g4 + r, channel ch.
  auto k_steps = [&](int buf, f32x4 (&acc)[2][2]) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) acc[rb][0] = acc[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    constexpr int kTerms[3][2] = {{0, 0}, {0, 1}, {1, 0}};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      bf16x8 ax[2][2], az[2][2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) {
          ax[rb][pl] = *(const bf16x8*)&px[buf][pl][16 * rb + l16][32 * t + 8 * g4];
          az[rb][pl] = *(const bf16x8*)&pz[buf][pl][16 * rb + l16][32 * t + 8 * g4];
        }
      }
#pragma unroll
      for (int tm = 0; tm < 3; ++tm) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          acc[rb][0] = mfma16_f16(ax[rb][kTerms[tm][0]], wz[kTerms[tm][1]][t], acc[rb][0]);
          acc[rb][1] = mfma16_f16(az[rb][kTerms[tm][0]], wg[kTerms[tm][1]][t], acc[rb][1]);
        }
      }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[rb][0][r] = __builtin_ldexpf(acc[rb][0][r], -(ex_out + ewz));
        acc[rb][1][r] = __builtin_ldexpf(acc[rb][1][r], -(ex_in + ewg));
      }
    }
  };

  // Residual values of a tile (accumulate), loaded an iteration ahead.
  f32x4 resid[2] = {};
  auto load_resid = [&](int tile) {
    if (!residual || tile >= ntiles) return;
    int i, jb;
    origin(tile, i, jb);
    const float* o = a.out + (int64_t)i * a.os_i + ch;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = min(jb * kRows + 16 * rb + 4 * g4 + r, n - 1);
        resid[rb][r] = o[(int64_t)j * a.os_j];
      }
    }
  };
  auto store = [&](int tile, const f32x4 (&acc)[2][2]) {
    int i, jb;
    origin(tile, i, jb);
    float* o = a.out + (int64_t)i * a.os_i + ch;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // native: value = sigmoid(g) * x, rounded; z + value when adding.
        // No fused multiply-add: the update is rounded before the sum, so
        // the in-place form equals z plus the separate update.
#pragma clang fp contract(off)
        const int j = jb * kRows + 16 * rb + 4 * g4 + r;
        const float v = sigmoidf_(acc[rb][1][r] + bg) * (acc[rb][0][r] + bz);
        if (j < n) o[(int64_t)j * a.os_j] = residual ? resid[rb][r] + v : v;
      }
    }
  };

  const bool lead = w < 4;
  const int stride = (int)gridDim.x;
  int tile = blockIdx.x;  // grid <= ntiles: every work-group has a tile
  int next = tile + stride;
  {
    int i0, jb0;
    origin(tile, i0, jb0);
    fetch(tile);
    copy_raw();
    normalise(0, jb0 * kRows);
  }
  fetch(next);
  copy_raw();
  fetch(next + stride);
  if (lead) load_resid(tile);
  __syncthreads();

  f32x4 res[2][2] = {};
  int done = -1;  // trail waves: the tile whose result `res` holds
  for (int buf = 0; tile < ntiles; buf ^= 1) {
    if (lead) k_steps(buf, res);
    if (next < ntiles) {
      int i1, jb1;
      origin(next, i1, jb1);
      normalise(buf ^ 1, jb1 * kRows);
    }
    __builtin_amdgcn_sched_barrier(0);
    copy_raw();
    fetch(next + 2 * stride);
    if (lead) {
      store(tile, res);
      load_resid(next);
    } else {
      if (done >= 0) store(done, res);
      load_resid(tile);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (!lead) {
      k_steps(buf, res);
      done = tile;
    }
    __syncthreads();
    tile = next;
    next += stride;
  }
  if (!lead && done >= 0) store(done, res);
}

int grid_for(int64_t ntiles, int per_cu) {
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  return (int)(ntiles < cap ? ntiles : cap);
}

}  // namespace

hipError_t launch_trimul(const TriMulArgs& a, hipStream_t stream) {
  if (a.n <= 0) return hipSuccess;
  if (a.np % kGemmTile || a.np < a.n) return hipErrorInvalidValue;
  const int64_t proj_tiles = (int64_t)a.n * (a.np / kRows);
  const int tiles = a.np / kGemmTile;
  const uint64_t gemm_total = (uint64_t)kChannels * tiles * tiles;
  const int tiles_j = (a.n + kRows - 1) / kRows;
  const int64_t fin_tiles = (int64_t)a.n * tiles_j;
  if (proj_tiles > 0x7fffffff || gemm_total > 0x7fffffffu || fin_tiles > 0x7fffffff)
    return hipErrorInvalidValue;
  hipError_t e;
  {
    GatedArgs g{};
    g.x = a.z;
    g.xs_r = a.outgoing ? a.zs_i : a.zs_j;
    g.xs_k = a.outgoing ? a.zs_j : a.zs_i;
    g.rows_r = a.n;
    g.rows_k = a.n;
    g.span_k = a.np;
    g.ln_w = a.ln_in_w;
    g.ln_b = a.ln_in_b;
    g.eps = a.eps_in;
    for (int side = 0; side < 2; ++side) {
      g.w_value[side] = a.w_ab[2 * side];
      g.w_gate[side] = a.w_ab[2 * side + 1];
      g.b_value[side] = a.b_ab[2 * side];
      g.b_gate[side] = a.b_ab[2 * side + 1];
    }
    g.mask = a.mask;
    g.ms_r = a.outgoing ? a.ms_i : a.ms_j;
    g.ms_k = a.outgoing ? a.ms_j : a.ms_i;
    g.out[0] = a.pa;
    g.out[1] = a.pb;
    g.np = a.np;
    g.rowmax = a.rowmax;
    if (a.rowmax == nullptr) return hipErrorInvalidValue;
    e = launch_gated_split<kGatedTriMul>(g, stream);
  }
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(trimul_contract_kernel, dim3((uint32_t)gemm_total), dim3(256), 0, stream,
                     a.pa, a.pb, a.rowmax, a.x, a.n, a.np, tiles, (uint32_t)gemm_total);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(trimul_finish_split_kernel, dim3(grid_for(fin_tiles, 1)), dim3(512), 0,
                     stream, a, tiles_j, (int)fin_tiles);
  return hipGetLastError();
}

}  // namespace fpx
