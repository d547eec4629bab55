// Pair-row projections on the CDNA4 FP32 matrix cores.
//
// A persistent work-group of NW wavefronts covers NW*32 output columns: wave w
// keeps the [128 x 32] weight fragment of its columns in 64 VGPRs for the whole
// launch (loaded once from the torch [out, in] weight), and the work-group
// streams row tiles of 32 pair rows through LDS.  Per tile every wave runs 64
// v_mfma_f32_32x32x2_f32 over the 128 input channels.
//
// kProjBlock fuses the pair LayerNorm into the prologue (one read of z, two
// register-level reductions per row on pivot-shifted values: mean, then the
// biased variance of the centred values) and the triangle-bias projection
// (4 wave reductions per row), and writes q (scaled by 1/sqrt(32)), k, v^T,
// sigmoid(g) and the bias (fragment order, bias_frag_index; once as is and once
// scaled by log2(e)) straight into the layouts the attention kernel reads.  The row addressing
// x + i*xs_i + j*xs_j makes the ending-node read of z^T free of copies.
#include "common.hpp"
#include "kernels.hpp"

namespace fpx {
namespace {

constexpr int kRows = 32;            // pair rows per tile
constexpr int kLdsStride = kChannels + 4;

template <int MODE>
struct ProjTraits;
template <>
struct ProjTraits<kProjBlock> {
  static constexpr int kWaves = 16;  // q, k, v, g: 4 x 128 columns
  static constexpr bool kLn = true;
};
template <>
struct ProjTraits<kProjQkv> {
  static constexpr int kWaves = 12;  // q, k, v
  static constexpr bool kLn = false;
};
template <>
struct ProjTraits<kProjOut> {
  static constexpr int kWaves = 4;   // 128 output channels
  static constexpr bool kLn = false;
};

template <int MODE>
__global__ __launch_bounds__(ProjTraits<MODE>::kWaves * 64) void projection_kernel(ProjArgs a,
                                                                                   int tiles_j,
                                                                                   int ntiles) {
  constexpr int NW = ProjTraits<MODE>::kWaves;
  constexpr int kThreads = NW * 64;
  constexpr int kRowsPerWave = kRows / NW;                 // LN mode only
  constexpr int kVecs = kRows * kChannels / 4;              // float4 per tile
  constexpr int kLoads = (kVecs + kThreads - 1) / kThreads; // non-LN mode
  __shared__ __attribute__((aligned(16))) float xs[kRows][kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;

  // Weight fragment: B[k][col] with col = 32*w + l32 and channel k = 64*half + s.
  float wf[64];
  {
    const float* src = a.w[w >> 2] + (int64_t)(32 * (w & 3) + l32) * kChannels + 64 * half;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const f32x4 v = *(const f32x4*)(src + 4 * t);
      wf[4 * t + 0] = v.x;
      wf[4 * t + 1] = v.y;
      wf[4 * t + 2] = v.z;
      wf[4 * t + 3] = v.w;
    }
  }

  // LN-mode per-lane constants: channels 2*lane, 2*lane+1.
  f32x2 lnw = {1.f, 1.f}, lnb = {0.f, 0.f};
  float wb[kHeads][2] = {};
  if (ProjTraits<MODE>::kLn) {
    if (a.ln_w) lnw = *(const f32x2*)(a.ln_w + 2 * lane);
    if (a.ln_b) lnb = *(const f32x2*)(a.ln_b + 2 * lane);
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
      const f32x2 v = *(const f32x2*)(a.w_bias + h * kChannels + 2 * lane);
      wb[h][0] = v.x;
      wb[h][1] = v.y;
    }
  }

  // Register stage for the next tile's raw rows.
  f32x2 stage_ln[ProjTraits<MODE>::kLn ? kRowsPerWave : 1];
  f32x4 stage_vec[ProjTraits<MODE>::kLn ? 1 : kLoads];

  auto fetch = [&](int tile) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows;
    if (ProjTraits<MODE>::kLn) {
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const int j = j0 + w * kRowsPerWave + rr;
        stage_ln[rr] = j < a.rows_j
                           ? *(const f32x2*)(a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j + 2 * lane)
                           : f32x2{0.f, 0.f};
      }
    } else {
#pragma unroll
      for (int t = 0; t < kLoads; ++t) {
        const int idx = tid + t * kThreads;
        const int row = idx >> 5;
        const int c4 = (idx & 31) * 4;
        const int j = j0 + row;
        stage_vec[t] = (idx < kVecs && j < a.rows_j)
                           ? *(const f32x4*)(a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j + c4)
                           : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };

  int tile = blockIdx.x;
  if (tile < ntiles) fetch(tile);
  for (; tile < ntiles; tile += gridDim.x) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows;

    // ---- stage the tile's rows (normalised in LN mode) into LDS
    if (ProjTraits<MODE>::kLn) {
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const int row = w * kRowsPerWave + rr;
        const int j = j0 + row;
        const bool valid = j < a.rows_j;
        const f32x2 xv = stage_ln[rr];
        float d0, d1, rstd;
        ln_stats_c128(xv.x, xv.y, a.eps, d0, d1, rstd);
        float y0 = d0 * rstd * lnw.x + lnb.x;
        float y1 = d1 * rstd * lnw.y + lnb.y;
        if (!valid) y0 = y1 = 0.f;
        *(f32x2*)&xs[row][2 * lane] = f32x2{y0, y1};
        if (MODE == kProjBlock) {
          float p[kHeads];
#pragma unroll
          for (int h = 0; h < kHeads; ++h) p[h] = wave_sum(y0 * wb[h][0] + y1 * wb[h][1]);
          if (lane < kHeads) {
            const float v = lane == 0 ? p[0] : lane == 1 ? p[1] : lane == 2 ? p[2] : p[3];
            const int64_t at = bias_frag_index(lane, i, j, a.np);
            a.tri_bias[at] = valid ? v : 0.f;
            a.tri_bias_l2[at] = valid ? v * kLog2e : 0.f;
          }
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < kLoads; ++t) {
        const int idx = tid + t * kThreads;
        if (idx < kVecs) *(f32x4*)&xs[idx >> 5][(idx & 31) * 4] = stage_vec[t];
      }
    }
    __syncthreads();
    if (tile + (int)gridDim.x < ntiles) fetch(tile + gridDim.x);

    // ---- 32 rows x 32 columns per wave: A[row][k] = xs[row][64*half + s]
    f32x16 acc = {};
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const f32x4 av = *(const f32x4*)&xs[l32][64 * half + 4 * t];
      acc = mfma32(av.x, wf[4 * t + 0], acc);
      acc = mfma32(av.y, wf[4 * t + 1], acc);
      acc = mfma32(av.z, wf[4 * t + 2], acc);
      acc = mfma32(av.w, wf[4 * t + 3], acc);
    }

    // ---- epilogue: lane holds rows mfma_row(r, half), column 32*w + l32
    const int group = w >> 2;   // 0 q, 1 k, 2 v, 3 g (kProjOut: always 0)
    const int hw = w & 3;       // head (q/k/v/g) or column block
    if (MODE == kProjBlock) {
      const int64_t bh = (int64_t)i * kHeads + hw;
      if (group == 0 || group == 1) {
        float* dst = (group == 0 ? a.qh : a.kh) + (bh * a.np + j0) * kHeadDim + l32;
        const float scale = group == 0 ? a.q_scale : 1.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(int64_t)mfma_row(r, half) * kHeadDim] = acc[r] * scale;
      } else if (group == 2) {
        float* dst = a.vt + (bh * kHeadDim + l32) * a.np + j0 + 4 * half;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          *(f32x4*)(dst + 8 * rr) =
              f32x4{acc[4 * rr + 0], acc[4 * rr + 1], acc[4 * rr + 2], acc[4 * rr + 3]};
      } else {
        const int col = 32 * hw + l32;
        const float bg = a.b_g ? a.b_g[col] : 0.f;
        float* dst = a.gs + ((int64_t)i * a.rows_j) * kHidden + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = j0 + mfma_row(r, half);
          if (j < a.rows_j) dst[(int64_t)j * kHidden] = sigmoidf_(acc[r] + bg);
        }
      }
    } else if (MODE == kProjQkv) {
      const int64_t rows = (int64_t)a.rows_i * a.rows_j;
      float* dst = a.out + ((int64_t)group * rows + (int64_t)i * a.rows_j) * kHidden + 32 * hw + l32;
      const float scale = group == 0 ? a.q_scale : 1.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = j0 + mfma_row(r, half);
        if (j < a.rows_j) dst[(int64_t)j * kHidden] = acc[r] * scale;
      }
    } else {
      const int col = 32 * w + l32;
      const float bo = a.b_g ? a.b_g[col] : 0.f;
      float* dst = a.out + (int64_t)i * a.os_i + col;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = j0 + mfma_row(r, half);
        if (j < a.rows_j) dst[(int64_t)j * a.os_j] = acc[r] + bo;
      }
    }
    __syncthreads();
  }
}

template <int MODE>
hipError_t launch_mode(const ProjArgs& a, hipStream_t stream, int wgs_per_cu) {
  const int tiles_j = (int)(round_up(a.span_j, kRows) / kRows);
  const int64_t ntiles = (int64_t)a.rows_i * tiles_j;
  if (ntiles == 0) return hipSuccess;
  if (ntiles > 0x7fffffffll) return hipErrorInvalidValue;
  const int64_t cap = (int64_t)device_cu_count() * wgs_per_cu;
  const int grid = (int)(ntiles < cap ? ntiles : cap);
  hipLaunchKernelGGL(projection_kernel<MODE>, dim3(grid), dim3(ProjTraits<MODE>::kWaves * 64), 0,
                     stream, a, tiles_j, (int)ntiles);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_projection(int mode, const ProjArgs& a, hipStream_t stream) {
  switch (mode) {
    case kProjBlock:
      return launch_mode<kProjBlock>(a, stream, 1);
    case kProjQkv:
      return launch_mode<kProjQkv>(a, stream, 1);
    case kProjOut:
      return launch_mode<kProjOut>(a, stream, 4);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace fpx
