// Pair transition (Protenix Transition, n = 4, c = 128) on the CDNA4 FP32
// matrix cores:
//
//   h   = silu(LN(x) W_a^T) * (LN(x) W_b^T)       [rows][512]
//   out = h W_o^T  (or out + h W_o^T, the residual)  [rows][128]
//
// transition_up_kernel: persistent; a work-group serves one quarter (128) of
//   the 512 hidden channels for its whole life, each of its 4 waves holding
//   the W_a and W_b fragments of 32 hidden channels in 128 VGPRs.  Per tile of
//   32 pair rows: LayerNorm of the raw rows (fetched a tile ahead) into a
//   second LDS buffer, 128 MFMAs per wave, and h stored row-major.
// transition_down_kernel: one 128-row tile of h W_o^T per work-group on the
//   shared gemm_nt_128 mainloop (K = 512), with the strided, optionally
//   accumulated store.
#include "common.hpp"
#include "gated_split.hpp"
#include "gemm.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace fpx {
namespace {

constexpr int kRows = 32;
constexpr int kLds = kChannels + 4;
constexpr int kHid = kTransitionHidden;
constexpr int kQuarters = kHid / kChannels;  // 4

__global__ __launch_bounds__(256, 2) void transition_up_kernel(TransitionArgs a, int tiles_j,
                                                               int ntiles, int slots) {
  __shared__ __attribute__((aligned(16))) float xs[2][kRows][kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int quarter = (int)(blockIdx.x % kQuarters);
  const int col = quarter * kChannels + 32 * w + l32;  // hidden channel of this lane

  float wa[64], wb[64];
  load_fragment(a.w_a, col, half, wa);
  load_fragment(a.w_b, col, half, wb);
  f32x2 lnw = {1.f, 1.f}, lnb = {0.f, 0.f};
  if (a.ln_w) lnw = *(const f32x2*)(a.ln_w + 2 * lane);
  if (a.ln_b) lnb = *(const f32x2*)(a.ln_b + 2 * lane);

  f32x2 st[kRows / 4];
  auto fetch = [&](int tile) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows;
#pragma unroll
    for (int rr = 0; rr < kRows / 4; ++rr) {
      const int j = j0 + 8 * w + rr;
      st[rr] = j < a.rows_j
                   ? *(const f32x2*)(a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j + 2 * lane)
                   : f32x2{0.f, 0.f};
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int rr = 0; rr < kRows / 4; ++rr) {
      float d0, d1, rstd;
      ln_stats_c128(st[rr].x, st[rr].y, a.eps, d0, d1, rstd);
      *(f32x2*)&xs[buf][8 * w + rr][2 * lane] =
          f32x2{d0 * rstd * lnw.x + lnb.x, d1 * rstd * lnw.y + lnb.y};
    }
  };

  __builtin_amdgcn_s_waitcnt(0);
  int tile = (int)(blockIdx.x / kQuarters);  // this work-group's slot; grid <= 4 * ntiles
  fetch(tile);
  stage(0);
  int next = tile + slots;
  if (next < ntiles) fetch(next);
  __syncthreads();
  for (int buf = 0; tile < ntiles; buf ^= 1) {
    f32x16 acc_a = {}, acc_b = {};
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const f32x4 av = *(const f32x4*)&xs[buf][l32][64 * half + 4 * t];
      acc_a = mfma32(av.x, wa[4 * t + 0], acc_a);
      acc_b = mfma32(av.x, wb[4 * t + 0], acc_b);
      acc_a = mfma32(av.y, wa[4 * t + 1], acc_a);
      acc_b = mfma32(av.y, wb[4 * t + 1], acc_b);
      acc_a = mfma32(av.z, wa[4 * t + 2], acc_a);
      acc_b = mfma32(av.z, wb[4 * t + 2], acc_b);
      acc_a = mfma32(av.w, wa[4 * t + 3], acc_a);
      acc_b = mfma32(av.w, wb[4 * t + 3], acc_b);
    }
    if (next < ntiles) {
      stage(buf ^ 1);
      if (next + slots < ntiles) fetch(next + slots);
    }
    // h row of pair (i, j) is i * rows_j + j; rows past rows_j are not stored.
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows;
    float* dst = a.h + ((int64_t)i * a.rows_j) * kHid + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = j0 + mfma_row(r, half);
      if (j < a.rows_j) {
        const float av = acc_a[r];
        dst[(int64_t)j * kHid] = av * sigmoidf_(av) * acc_b[r];  // silu(a) * b
      }
    }
    __syncthreads();
    tile = next;
    next += slots;
  }
}

// The fp16-plane path's maxima: max |W_o| of each output row, and the h max
// cleared for the up-projection's atomics.  One work-group of 256 threads.
__global__ __launch_bounds__(256) void transition_maxima_kernel(const float* __restrict__ w_o,
                                                                uint32_t* __restrict__ maxima) {
  const int t = threadIdx.x;
  if (t < kChannels) {
    const f32x4* row = reinterpret_cast<const f32x4*>(w_o + (int64_t)t * kHid);
    float m = 0.f;
    for (int i = 0; i < kHid / 4; ++i) {
      const f32x4 v = row[i];
      m = __builtin_elementwise_maximum(
          m, __builtin_elementwise_maximum(
                 __builtin_elementwise_maximum(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                 __builtin_elementwise_maximum(__builtin_fabsf(v.z), __builtin_fabsf(v.w))));
    }
    maxima[1 + t] = __builtin_bit_cast(uint32_t, m);
  } else if (t == kChannels) {
    maxima[0] = 0u;
  }
}

// kSplit: gemm_nt_128_f16 (16-bit matrix cores, scaled fp16 planes): every h
// row scaled by the launch's h exponent (the LN'd rows share one magnitude
// range), each W_o row by its own.
template <bool kSplit>
__global__ __launch_bounds__(256, 2) void transition_down_kernel(TransitionArgs a,
                                                                 int64_t rows) {
  using Stage = std::conditional_t<kSplit, F16Stage, GemmStage>;
  __shared__ __attribute__((aligned(16))) Stage As[2];
  __shared__ __attribute__((aligned(16))) Stage Bs[2];
  __shared__ int ea[kSplit ? kGemmTile : 1], eb[kSplit ? kGemmTile : 1];
  const int64_t r0 = (int64_t)blockIdx.x * kGemmTile;
  f32x16 acc[2][2] = {};
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int wi = (w >> 1) * 64;
  const int wj = (w & 1) * 64;
  // W_o is [128 out][512 in]: the B operand rows are output channels.
  if constexpr (kSplit) {
    const int t = threadIdx.x;
    const int ex = plane_exp(__builtin_bit_cast(float, a.maxima[0]));
    if (t < kGemmTile) ea[t] = ex;
    else eb[t - kGemmTile] = plane_exp(__builtin_bit_cast(float, a.maxima[1 + t - kGemmTile]));
    __syncthreads();
    gemm_nt_128_f16(a.h + r0 * kHid, kHid, a.w_o, kHid, 32, kHid / kSplitK, As, Bs, ea, eb,
                    acc);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int e = ex + eb[wj + 32 * cb + l32];
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[rb][cb][r] = __builtin_ldexpf(acc[rb][cb][r], -e);
      }
    }
  } else {
    gemm_nt_128(a.h + r0 * kHid, kHid, a.w_o, kHid, kHid / kKStage, As, Bs, acc);
  }

  const bool residual = a.accumulate != 0;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = r0 + wi + 32 * rb + mfma_row(r, half);
      if (row >= rows) continue;
      const int64_t i = row / a.rows_j;
      const int64_t j = row - i * a.rows_j;
      float* d = a.out + i * a.os_i + j * a.os_j + wj + l32;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const float v = acc[rb][cb][r];
        d[32 * cb] = residual ? d[32 * cb] + v : v;
      }
    }
  }
}

int grid_cap(int per_cu) { return device_cu_count() * per_cu; }

}  // namespace

hipError_t launch_transition(const TransitionArgs& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.rows_i * a.rows_j;
  if (rows == 0) return hipSuccess;
  const int tiles_j = (a.rows_j + kRows - 1) / kRows;
  const int64_t up_tiles = (int64_t)a.rows_i * tiles_j;
  const int64_t down_tiles = (rows + kGemmTile - 1) / kGemmTile;
  if (up_tiles > 0x7fffffff || down_tiles > 0x7fffffff) return hipErrorInvalidValue;
  // Persistent up-projection: slots per quarter, 2 work-groups per CU in all.
  int64_t slots = grid_cap(2) / kQuarters;
  if (slots > up_tiles) slots = up_tiles;
  if (slots < 1) slots = 1;
  hipError_t e;
  if (fp32_matrix_cores_selected()) {
    hipLaunchKernelGGL(transition_up_kernel, dim3((uint32_t)(slots * kQuarters)), dim3(256), 0,
                       stream, a, tiles_j, (int)up_tiles, (int)slots);
    e = hipGetLastError();
  } else {
    GatedArgs g{};
    g.x = a.x;
    g.xs_r = a.xs_i;
    g.xs_k = a.xs_j;
    g.rows_r = a.rows_i;
    g.rows_k = a.rows_j;
    g.span_k = tiles_j * kRows;
    g.ln_w = a.ln_w;
    g.ln_b = a.ln_b;
    g.eps = a.eps;
    // h = silu(x W_a^T) * (x W_b^T): W_a rows are the gates, W_b rows the values.
    for (int q = 0; q < kQuarters; ++q) {
      g.w_value[q] = a.w_b + (int64_t)q * kChannels * kChannels;
      g.w_gate[q] = a.w_a + (int64_t)q * kChannels * kChannels;
      g.out[q] = a.h + q * kChannels;
    }
    if (a.maxima == nullptr) return hipErrorInvalidValue;
    g.out_max = a.maxima;
    hipLaunchKernelGGL(transition_maxima_kernel, dim3(1), dim3(256), 0, stream, a.w_o, a.maxima);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = launch_gated_split<kGatedTransition>(g, stream);
  }
  if (e != hipSuccess) return e;
  if (fp32_matrix_cores_selected())
    hipLaunchKernelGGL(transition_down_kernel<false>, dim3((uint32_t)down_tiles), dim3(256), 0,
                       stream, a, rows);
  else
    hipLaunchKernelGGL(transition_down_kernel<true>, dim3((uint32_t)down_tiles), dim3(256), 0,
                       stream, a, rows);
  return hipGetLastError();
}

}  // namespace fpx
