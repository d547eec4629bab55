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
// (4 wave reductions per row, DPP and lane-swap steps with no LDS traffic),
// and writes q (scaled by 1/sqrt(32)), k, v^T,
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
  // Two row tiles: the MFMAs read one while the next is normalised into the
  // other, so a tile needs one barrier.
  __shared__ __attribute__((aligned(16))) float xs[2][kRows][kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
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

  // Per-lane bias of this wave's output column (gate bias in the block, b_o
  // in the output projection).
  const int col_w = MODE == kProjOut ? 32 * w + l32 : 32 * (w & 3) + l32;
  const float col_bias = (MODE != kProjQkv && a.b_g != nullptr) ? a.b_g[col_w] : 0.f;

  // LN-mode per-lane constants: channels 2*lane, 2*lane+1.
  f32x2 lnw = {1.f, 1.f}, lnb = {0.f, 0.f};
  float wb[kHeads][2] = {};
  if (ProjTraits<MODE>::kLn) {
    if (a.ln_w) lnw = *(const f32x2*)(a.ln_w + 2 * lane);
    if (a.ln_b) lnb = *(const f32x2*)(a.ln_b + 2 * lane);
    if (MODE == kProjBlock) {
#pragma unroll
      for (int h = 0; h < kHeads; ++h) {
        const f32x2 v = *(const f32x2*)(a.w_bias + h * kChannels + 2 * lane);
        wb[h][0] = v.x;
        wb[h][1] = v.y;
      }
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

  // The staged rows of `tile` into xs[buf]: normalised in LN mode (and, for
  // the block, the triangle bias of each row written out), copied otherwise.
  auto stage_rows = [&](int tile, int buf) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows;
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
        *(f32x2*)&xs[buf][row][2 * lane] = f32x2{y0, y1};
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
        if (idx < kVecs) *(f32x4*)&xs[buf][idx >> 5][(idx & 31) * 4] = stage_vec[t];
      }
    }
  };

  // 32 rows x 32 columns per wave: A[row][k] = xs[row][64*half + s].
  auto mfma_tile = [&](int buf) -> f32x16 {
    f32x16 acc = {};
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const f32x4 av = *(const f32x4*)&xs[buf][l32][64 * half + 4 * t];
      acc = mfma32(av.x, wf[4 * t + 0], acc);
      acc = mfma32(av.y, wf[4 * t + 1], acc);
      acc = mfma32(av.z, wf[4 * t + 2], acc);
      acc = mfma32(av.w, wf[4 * t + 3], acc);
    }
    return acc;
  };

  // Lane holds rows 4*half + 8*(r/4) + r%4 of the tile, column 32*w + l32.
  // Row offsets are compile-time constants once the lane's base includes
  // its 4*half rows.
  auto epilogue = [&](int tile, const f32x16& acc) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows + 4 * half;
    const int group = w >> 2;   // 0 q, 1 k, 2 v, 3 g (kProjOut: always 0)
    const int hw = w & 3;       // head (q/k/v/g) or column block
    if (MODE == kProjBlock) {
      const int64_t bh = (int64_t)i * kHeads + hw;
      if (group == 0 || group == 1) {
        float* dst = (group == 0 ? a.qh : a.kh) + (bh * a.np + j0) * kHeadDim + l32;
        if (group == 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[(8 * (r >> 2) + (r & 3)) * kHeadDim] = acc[r] * a.q_scale;
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[(8 * (r >> 2) + (r & 3)) * kHeadDim] = acc[r];
        }
      } else if (group == 2) {
        float* dst = a.vt + (bh * kHeadDim + l32) * a.np + j0;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          *(f32x4*)(dst + 8 * rr) =
              f32x4{acc[4 * rr + 0], acc[4 * rr + 1], acc[4 * rr + 2], acc[4 * rr + 3]};
      } else {
        // gate rows are padded to np: the tile is always stored whole
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
  };

  // Persistent loop: the tile after this one is fetched two tiles ahead and
  // normalised right after this tile's MFMAs are issued.
  // The weight fragment and bias must have landed before the loop: the
  // loop's waits then track only the row fetches and the output stores.
  __builtin_amdgcn_s_waitcnt(0);
  int tile = blockIdx.x;  // grid <= ntiles, so every work-group has a tile
  fetch(tile);
  stage_rows(tile, 0);
  int next = tile + (int)gridDim.x;
  if (next < ntiles) fetch(next);
  __syncthreads();
  for (int buf = 0; tile < ntiles; buf ^= 1) {
    const f32x16 acc = mfma_tile(buf);
    if (next < ntiles) {
      stage_rows(next, buf ^ 1);
      if (next + (int)gridDim.x < ntiles) fetch(next + gridDim.x);
    }
    epilogue(tile, acc);
    __syncthreads();
    tile = next;
    next += gridDim.x;
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
