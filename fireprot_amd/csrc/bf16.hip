// BF16-storage / FP32-accumulate variant of the triangle-attention block.
//
// Same dataflow as the FP32 block (projection.hip, attention.hip) with every
// stored tensor in bf16 -- z, weights, q, k, v^T, the sigmoid gate, the
// triangle bias, the gated output and dz -- and all accumulation, LayerNorm
// statistics and softmax arithmetic in FP32 on the gfx950 instruction
// v_mfma_f32_32x32x16_bf16.  The LayerNorm output is rounded to bf16 before
// it feeds the projections, which is where the native BF16 path rounds it.
//
// 32x32x16 bf16 operands: lane l holds 8 consecutive k values of row/column
// l % 32 for k-half l / 32; the result layout is that of the FP32 32x32
// instruction (lane l, register r -> D[8*(r/4) + 4*(l/32) + r%4][l % 32]).
// A and B agree on the (k-half, element) pairing, so any consistent channel
// order works for the projections and for S^T = K Q^T.  For O^T += V^T P^T the
// P operand is taken straight from the S^T registers: element e of MFMA m in
// lane half hb is register 8m + e, i.e. key 16m + 8(e/4) + 4hb + e%4 of the
// tile, and V^T is read with that same key order.
#include "common.hpp"
#include "kernels.hpp"

#include <cmath>

namespace fpx {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ----------------------------------------------------------------- projections

constexpr int kRows = 32;                  // pair rows per tile
constexpr int kXsStride = kChannels + 8;   // bf16 per LDS row (272 bytes)

template <int MODE>
struct Bf16ProjTraits;
template <>
struct Bf16ProjTraits<kProjBlock> {
  static constexpr int kWaves = 16;  // q, k, v, g
  static constexpr bool kLn = true;
};
template <>
struct Bf16ProjTraits<kProjOut> {
  static constexpr int kWaves = 4;
  static constexpr bool kLn = false;
};

template <int MODE>
__global__ __launch_bounds__(Bf16ProjTraits<MODE>::kWaves * 64) void projection_bf16_kernel(
    Bf16ProjArgs a, int tiles_j, int ntiles) {
  constexpr int NW = Bf16ProjTraits<MODE>::kWaves;
  constexpr bool kLn = Bf16ProjTraits<MODE>::kLn;
  constexpr int kThreads = NW * 64;
  constexpr int kRowsPerWave = kRows / NW;
  constexpr int kVecs = kRows * kChannels / 8;               // 16-byte vectors per tile
  constexpr int kLoads = (kVecs + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) __bf16 xs[kRows][kXsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;

  // B[k][col]: column 32*(w&3) + l32 of weight group w>>2, k = 16*m + 8*half + e.
  bf16x8 wf[8];
  {
    const __bf16* src = a.w[w >> 2] + (int64_t)(32 * (w & 3) + l32) * kChannels + 8 * half;
#pragma unroll
    for (int m = 0; m < 8; ++m) wf[m] = *(const bf16x8*)(src + 16 * m);
  }

  float lnw[2] = {1.f, 1.f}, lnb[2] = {0.f, 0.f};
  float wb[kHeads][2] = {};
  if (kLn) {
    if (a.ln_w) {
      const bf16x2 v = *(const bf16x2*)(a.ln_w + 2 * lane);
      lnw[0] = (float)v.x;
      lnw[1] = (float)v.y;
    }
    if (a.ln_b) {
      const bf16x2 v = *(const bf16x2*)(a.ln_b + 2 * lane);
      lnb[0] = (float)v.x;
      lnb[1] = (float)v.y;
    }
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
      const bf16x2 v = *(const bf16x2*)(a.w_bias + h * kChannels + 2 * lane);
      wb[h][0] = (float)v.x;
      wb[h][1] = (float)v.y;
    }
  }

  bf16x2 stage_ln[kLn ? kRowsPerWave : 1];
  bf16x8 stage_vec[kLn ? 1 : kLoads];
  const bf16x2 zero2 = {(__bf16)0.f, (__bf16)0.f};
  const bf16x8 zero8 = {(__bf16)0.f, (__bf16)0.f, (__bf16)0.f, (__bf16)0.f,
                        (__bf16)0.f, (__bf16)0.f, (__bf16)0.f, (__bf16)0.f};

  auto fetch = [&](int tile) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows;
    if (kLn) {
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const int j = j0 + w * kRowsPerWave + rr;
        stage_ln[rr] = j < a.rows_j
                           ? *(const bf16x2*)(a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j + 2 * lane)
                           : zero2;
      }
    } else {
#pragma unroll
      for (int t = 0; t < kLoads; ++t) {
        const int idx = tid + t * kThreads;
        const int row = idx >> 4;
        const int c8 = (idx & 15) * 8;
        const int j = j0 + row;
        stage_vec[t] = (idx < kVecs && j < a.rows_j)
                           ? *(const bf16x8*)(a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j + c8)
                           : zero8;
      }
    }
  };

  int tile = blockIdx.x;
  if (tile < ntiles) fetch(tile);
  for (; tile < ntiles; tile += gridDim.x) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows;
    if (kLn) {
#pragma unroll
      for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const int row = w * kRowsPerWave + rr;
        const int j = j0 + row;
        const bool valid = j < a.rows_j;
        float d0, d1, rstd;
        ln_stats_c128((float)stage_ln[rr].x, (float)stage_ln[rr].y, a.eps, d0, d1, rstd);
        float y0 = d0 * rstd * lnw[0] + lnb[0];
        float y1 = d1 * rstd * lnw[1] + lnb[1];
        if (!valid) y0 = y1 = 0.f;
        const bf16x2 yb = {(__bf16)y0, (__bf16)y1};
        *(bf16x2*)&xs[row][2 * lane] = yb;
        if (MODE == kProjBlock) {
          const float r0 = (float)yb.x;
          const float r1 = (float)yb.y;
          float p[kHeads];
#pragma unroll
          for (int h = 0; h < kHeads; ++h) p[h] = wave_sum(r0 * wb[h][0] + r1 * wb[h][1]);
          if (lane < kHeads) {
            const float v = lane == 0 ? p[0] : lane == 1 ? p[1] : lane == 2 ? p[2] : p[3];
            a.tri_bias[((int64_t)lane * a.np + i) * a.np + j] = (__bf16)(valid ? v : 0.f);
          }
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < kLoads; ++t) {
        const int idx = tid + t * kThreads;
        if (idx < kVecs) *(bf16x8*)&xs[idx >> 4][(idx & 15) * 8] = stage_vec[t];
      }
    }
    __syncthreads();
    if (tile + (int)gridDim.x < ntiles) fetch(tile + gridDim.x);

    f32x16 acc = {};
#pragma unroll
    for (int m = 0; m < 8; ++m) acc = mfma_bf16(*(const bf16x8*)&xs[l32][16 * m + 8 * half], wf[m], acc);

    const int group = w >> 2;
    const int hw = w & 3;
    if (MODE == kProjBlock) {
      const int64_t bh = (int64_t)i * kHeads + hw;
      if (group == 0 || group == 1) {
        __bf16* dst = (group == 0 ? a.qh : a.kh) + (bh * a.np + j0) * kHeadDim + l32;
        const float scale = group == 0 ? a.q_scale : 1.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(int64_t)mfma_row(r, half) * kHeadDim] = (__bf16)(acc[r] * scale);
      } else if (group == 2) {
        __bf16* dst = a.vt + (bh * kHeadDim + l32) * a.np + j0 + 4 * half;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          *(bf16x4*)(dst + 8 * rr) = bf16x4{(__bf16)acc[4 * rr + 0], (__bf16)acc[4 * rr + 1],
                                            (__bf16)acc[4 * rr + 2], (__bf16)acc[4 * rr + 3]};
      } else {
        const int col = 32 * hw + l32;
        const float bg = a.bias_vec ? (float)a.bias_vec[col] : 0.f;
        __bf16* dst = a.gs + ((int64_t)i * a.rows_j) * kHidden + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = j0 + mfma_row(r, half);
          if (j < a.rows_j) dst[(int64_t)j * kHidden] = (__bf16)sigmoidf_(acc[r] + bg);
        }
      }
    } else {
      const int col = 32 * w + l32;
      const float bo = a.bias_vec ? (float)a.bias_vec[col] : 0.f;
      __bf16* dst = a.out + (int64_t)i * a.os_i + col;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = j0 + mfma_row(r, half);
        if (j < a.rows_j) dst[(int64_t)j * a.os_j] = (__bf16)(acc[r] + bo);
      }
    }
    __syncthreads();
  }
}

template <int MODE>
hipError_t launch_proj_mode(const Bf16ProjArgs& a, hipStream_t stream, int wgs_per_cu) {
  const int tiles_j = (int)(round_up(a.span_j, kRows) / kRows);
  const int64_t ntiles = (int64_t)a.rows_i * tiles_j;
  if (ntiles == 0) return hipSuccess;
  if (ntiles > 0x7fffffffll) return hipErrorInvalidValue;
  const int64_t cap = (int64_t)device_cu_count() * wgs_per_cu;
  const int grid = (int)(ntiles < cap ? ntiles : cap);
  hipLaunchKernelGGL(projection_bf16_kernel<MODE>, dim3(grid),
                     dim3(Bf16ProjTraits<MODE>::kWaves * 64), 0, stream, a, tiles_j, (int)ntiles);
  return hipGetLastError();
}

// ------------------------------------------------------------------- attention

constexpr int kBq = 128;
constexpr int kBk = 32;
constexpr int kLdsPad = 8;        // bf16 elements: rows of 80 bytes
constexpr int kThreads = 256;
constexpr int kRowGroup = 8;

struct Bf16Tile {
  bf16x4 v;
  bf16x4 b[4];
  f32x4 m;
};

__device__ __forceinline__ bf16x4 load_k_bf16(const Bf16AttnArgs& a, int b, int h, int k0, int tid) {
  const int64_t bh = (int64_t)b * kHeads + h;
  return *(const bf16x4*)(a.k + (bh * a.np + k0 + (tid >> 3)) * kHeadDim + (tid & 7) * 4);
}

__device__ __forceinline__ void load_vbm_bf16(const Bf16AttnArgs& a, int b, int h, int j0, int k0,
                                              int tid, Bf16Tile& t) {
  const int row8 = tid >> 3;
  const int col4 = (tid & 7) * 4;
  const int64_t bh = (int64_t)b * kHeads + h;
  t.v = *(const bf16x4*)(a.v + (bh * kHeadDim + row8) * a.np + k0 + col4);
#pragma unroll
  for (int m = 0; m < 4; ++m)
    t.b[m] = *(const bf16x4*)(a.bias + ((int64_t)h * a.np + j0 + row8 + 32 * m) * a.np + k0 + col4);
  if (tid < 8) t.m = *(const f32x4*)(a.mbias + (int64_t)b * a.np + k0 + 4 * tid);
}

__device__ __forceinline__ float xor32_max_bf(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float xor32_sum_bf(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// One work-group = (outer row b, head h, 128 queries), four waves of 32
// queries, 32-key tiles; the order of work-groups and the online softmax
// (shared log2 reference, exp2(fma)) are those of the FP32 attention kernel.
__global__ __launch_bounds__(kThreads) void attention_bf16_kernel(Bf16AttnArgs a, int nqt, int nkt,
                                                                  uint32_t total) {
  __shared__ __attribute__((aligned(16))) __bf16 Ks[kBk][kHeadDim + kLdsPad];   // [key][channel]
  __shared__ __attribute__((aligned(16))) __bf16 Vs[kHeadDim][kBk + kLdsPad];   // [channel][key]
  __shared__ __attribute__((aligned(16))) __bf16 Bs[kBq][kBk + kLdsPad];        // [query][key]
  __shared__ __attribute__((aligned(16))) float Ms[kBk];

  const uint32_t logical = xcd_remap(blockIdx.x, total);
  const int groups = (a.batch + kRowGroup - 1) / kRowGroup;
  const int per_head = groups * kRowGroup * nqt;
  const int h = (int)(logical / per_head);
  const int rem = (int)(logical % per_head);
  const int grp = rem / (kRowGroup * nqt);
  const int in_grp = rem % (kRowGroup * nqt);
  const int qt = in_grp / kRowGroup;
  const int b = grp * kRowGroup + in_grp % kRowGroup;
  if (b >= a.batch) return;  // padding of the last row group; uniform per work-group
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int j0 = qt * kBq;
  const int jq = j0 + 32 * w + l32;

  // Q^T operand: lane holds Q[jq][16*m + 8*half + e].
  bf16x8 qf[2];
  {
    const __bf16* src = a.q + (((int64_t)b * kHeads + h) * a.np + jq) * kHeadDim + 8 * half;
    qf[0] = *(const bf16x8*)(src);
    qf[1] = *(const bf16x8*)(src + 16);
  }

  f32x16 o = {};
  float c_run = -INFINITY;
  float l_run = 0.f;
  const int row8 = tid >> 3;
  const int col4 = (tid & 7) * 4;
  Bf16Tile regs;

  auto qk = [&]() {
    f32x16 s = {};
    s = mfma_bf16(*(const bf16x8*)&Ks[l32][8 * half], qf[0], s);
    s = mfma_bf16(*(const bf16x8*)&Ks[l32][16 + 8 * half], qf[1], s);
    return s;
  };
  auto store_vbm = [&]() {
    *(bf16x4*)&Vs[row8][col4] = regs.v;
#pragma unroll
    for (int m = 0; m < 4; ++m) *(bf16x4*)&Bs[row8 + 32 * m][col4] = regs.b[m];
    if (tid < 8) *(f32x4*)&Ms[4 * tid] = regs.m;
  };
  auto softmax_pv = [&](f32x16 s) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x4 mb = *(const f32x4*)&Ms[8 * rr + 4 * half];
      const bf16x4 bb = *(const bf16x4*)&Bs[32 * w + l32][8 * rr + 4 * half];
      s[4 * rr + 0] = (s[4 * rr + 0] + mb.x) + (float)bb.x;
      s[4 * rr + 1] = (s[4 * rr + 1] + mb.y) + (float)bb.y;
      s[4 * rr + 2] = (s[4 * rr + 2] + mb.z) + (float)bb.z;
      s[4 * rr + 3] = (s[4 * rr + 3] + mb.w) + (float)bb.w;
    }
    float mt = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
    mt = xor32_max_bf(mt);
    const float c_new = mt == -INFINITY ? c_run : fmaxf(c_run, mt * kLog2e);
    const float c_use = c_new == -INFINITY ? 0.f : c_new;
    const float alpha = exp2_fast(c_run - c_use);
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[r] *= alpha;
    }
    l_run *= alpha;
    c_run = c_new;
    // P in bf16, summed as rounded so O / l is a proper weighted mean.
    bf16x8 pm[2];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const __bf16 pb = (__bf16)exp2_fast(__builtin_fmaf(s[r], kLog2e, -c_use));
      pm[r >> 3][r & 7] = pb;
      psum += (float)pb;
    }
    l_run += psum;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const bf16x4 lo = *(const bf16x4*)&Vs[l32][16 * m + 4 * half];
      const bf16x4 hi = *(const bf16x4*)&Vs[l32][16 * m + 8 + 4 * half];
      const bf16x8 va = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      o = mfma_bf16(va, pm[m], o);
    }
  };

  *(bf16x4*)&Ks[row8][col4] = load_k_bf16(a, b, h, 0, tid);
  __syncthreads();
  f32x16 s_cur = qk();
  bf16x4 kreg = {};
  if (nkt > 1) kreg = load_k_bf16(a, b, h, kBk, tid);
  load_vbm_bf16(a, b, h, j0, 0, tid, regs);
  for (int kt = 0; kt + 1 < nkt; ++kt) {
    __syncthreads();
    *(bf16x4*)&Ks[row8][col4] = kreg;
    store_vbm();
    __syncthreads();
    if (kt + 2 < nkt) kreg = load_k_bf16(a, b, h, (kt + 2) * kBk, tid);
    load_vbm_bf16(a, b, h, j0, (kt + 1) * kBk, tid, regs);
    const f32x16 s_next = qk();
    softmax_pv(s_cur);
    s_cur = s_next;
  }
  __syncthreads();
  store_vbm();
  __syncthreads();
  softmax_pv(s_cur);

  const float l_tot = xor32_sum_bf(l_run);
  if (jq < a.n) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int c = 8 * rr + 4 * half;
      const int64_t off = ((int64_t)b * a.n + jq) * kHidden + h * kHeadDim + c;
      const bf16x4 g = *(const bf16x4*)(a.gate + off);
      *(bf16x4*)(a.out + off) = bf16x4{(__bf16)(o[4 * rr + 0] / l_tot * (float)g.x),
                                       (__bf16)(o[4 * rr + 1] / l_tot * (float)g.y),
                                       (__bf16)(o[4 * rr + 2] / l_tot * (float)g.z),
                                       (__bf16)(o[4 * rr + 3] / l_tot * (float)g.w)};
    }
  }
}

}  // namespace

hipError_t launch_projection_bf16(int mode, const Bf16ProjArgs& a, hipStream_t stream) {
  switch (mode) {
    case kProjBlock:
      return launch_proj_mode<kProjBlock>(a, stream, 1);
    case kProjOut:
      return launch_proj_mode<kProjOut>(a, stream, 4);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_attention_bf16(const Bf16AttnArgs& a, hipStream_t stream) {
  const int nqt = a.np / kBq;
  const int nkt = a.np / kBk;
  const uint64_t groups = ((uint64_t)a.batch + kRowGroup - 1) / kRowGroup;
  const uint64_t total = groups * kRowGroup * kHeads * nqt;
  if (total == 0) return hipSuccess;
  if (total > 0x7fffffffull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_bf16_kernel, dim3((uint32_t)total), dim3(kThreads), 0, stream, a, nqt,
                     nkt, (uint32_t)total);
  return hipGetLastError();
}

}  // namespace fpx
