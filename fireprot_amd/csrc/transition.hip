// Pair transition (Protenix Transition, n = 4, c = 128) on the CDNA4 16-bit
// matrix cores, FP32-accurate:
//
//   h   = silu(LN(x) W_a^T) * (LN(x) W_b^T)       [rows][512]
//   out = h W_o^T  (or out + h W_o^T, the residual)  [rows][128]
//
// One fused kernel with h never leaving the registers
// (transition_fused_kernel below), after two small kernels that fold the
// LayerNorm affine into the weights and split them into scaled fp16 planes.
#include "attn_common.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "split.hpp"

#include <type_traits>

namespace fpx {
namespace {

constexpr int kHid = kTransitionHidden;

// ------------------------------------------------------- fused, fp16 cores
// out = x + silu(y Wa'^T + ba) * (y Wb'^T + bb) Wo^T with y = (x - mean)
// rstd, the LayerNorm affine folded into the weights (W' = W diag(ln_w),
// b = W ln_b), all three products on v_mfma_f32_32x32x16_f16 with
// power-of-two scaled fp16 (hi, lo) planes and three terms (FP32 accuracy).
// A wave owns 32 pair rows: its y^T planes (the B operand, 64 VGPRs) stay in
// registers while the 512 hidden channels pass in 16 chunks of 32; per chunk
//   value^T, gate^T [32 hidden][32 rows] = W' y^T      (48 MFMAs)
//   h = silu(gate) * value, as planes scaled by 2^e_h  (the A operand: a
//       lane holds its row's 16 hidden values, and W_o's columns are stored
//       in that order)
//   out [32 rows][128] += h W_o^T                       (24 MFMAs)
// so h never leaves the registers.  The chunks' weight planes (48 KB each,
// written once per call by transition_planes_kernel) go from L2 into a
// three-stage LDS ring by global_load_lds, shared by the 8 waves (256 rows)
// of a work-group, with one barrier per chunk.  Plane scales: y by 2^e_x
// (|y_c| <= sqrt(128)), each row of W' and of W_o by its own exponent, h by
// 2^e_h from the bound |h_c| <= max(|g_c|, 0.2785) |v_c| with |g_c| <=
// sqrt(128) |Wa'_c| + |ba_c| (likewise v), |silu(g)| <= max(|g|, 0.2785).
constexpr int kFusedWaves = 8;
constexpr int kFusedRows = 32 * kFusedWaves;               // rows per tile
constexpr int kChunkHid = 32;
constexpr int kChunks = kHid / kChunkHid;                  // 16
constexpr int kUpBlocks = 2 * 8 * 2;                       // [a, b][k step][hi, lo]
constexpr int kDownBlocks = 4 * 2 * 2;                     // [out block][k step][hi, lo]
constexpr int kPlaneBlock = 32 * 16;                       // fp16 values of a 1 KB block
constexpr int kChunkValues = (kUpBlocks + kDownBlocks) * kPlaneBlock;  // 24576 (48 KB)
constexpr int kChunkBytes = kChunkValues * 2;

// Plane exponents (TransitionArgs::exps): e_x of the y planes, e_h of h, one
// per W' row (a, then b) and one per W_o row; then the prep work-groups'
// largest h bounds (float bits), which transition_planes_kernel reduces to
// e_h.
constexpr int kExpX = 0;
constexpr int kExpH = 1;
constexpr int kExpW = 4;                 // [2][512]
constexpr int kExpO = kExpW + 2 * kHid;  // [128]
constexpr int kPrepGroups = 4;
constexpr int kExpPart = kExpO + kChannels;  // [kPrepGroups]

// kPrepGroups work-groups of 512 threads: the folded biases ([2][512]: ba,
// bb) and the exponents.  Work-group g: hidden channels 128 g .. + 127, four
// threads per channel (32 inputs each), and W_o rows 32 g .. + 31, sixteen
// threads per row.
__global__ __launch_bounds__(512) void transition_prep_kernel(TransitionArgs a) {
  __shared__ float red[8];
  __shared__ __attribute__((aligned(16))) float gb_lds[2][kChannels];
  const int tid = threadIdx.x;
  if (tid < kChannels) {
    gb_lds[0][tid] = a.ln_w ? a.ln_w[tid] : 1.f;
    gb_lds[1][tid] = a.ln_b ? a.ln_b[tid] : 0.f;
  }
  __syncthreads();
  const int c = (int)blockIdx.x * (kHid / kPrepGroups) + (tid >> 2);  // hidden channel
  const int i0 = (tid & 3) * (kChannels / 4);
  const float* wa = a.w_a + (int64_t)c * kChannels + i0;
  const float* wb = a.w_b + (int64_t)c * kChannels + i0;
  float sa2 = 0.f, sa1 = 0.f, sb2 = 0.f, sb1 = 0.f, ma = 0.f, mb = 0.f;
#pragma unroll
  for (int i = 0; i < kChannels / 4; i += 4) {
    const f32x4 va = *(const f32x4*)(wa + i), vb = *(const f32x4*)(wb + i);
    const f32x4 g = *(const f32x4*)&gb_lds[0][i0 + i], b = *(const f32x4*)&gb_lds[1][i0 + i];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float ga = g[e] * va[e], gbv = g[e] * vb[e];
      sa2 = __builtin_fmaf(ga, ga, sa2);
      sb2 = __builtin_fmaf(gbv, gbv, sb2);
      sa1 = __builtin_fmaf(b[e], va[e], sa1);
      sb1 = __builtin_fmaf(b[e], vb[e], sb1);
      ma = __builtin_elementwise_maximum(ma, __builtin_fabsf(ga));
      mb = __builtin_elementwise_maximum(mb, __builtin_fabsf(gbv));
    }
  }
  // the channel's four threads are lanes 4 q .. 4 q + 3
#pragma unroll
  for (int d = 1; d < 4; d <<= 1) {
    sa2 += __shfl_xor(sa2, d);
    sb2 += __shfl_xor(sb2, d);
    sa1 += __shfl_xor(sa1, d);
    sb1 += __shfl_xor(sb1, d);
    ma = __builtin_elementwise_maximum(ma, __shfl_xor(ma, d));
    mb = __builtin_elementwise_maximum(mb, __shfl_xor(mb, d));
  }
  float bh = 0.f;
  if ((tid & 3) == 0) {
    a.fbias[c] = sa1;
    a.fbias[kHid + c] = sb1;
    a.exps[kExpW + c] = plane_exp(ma);
    a.exps[kExpW + kHid + c] = plane_exp(mb);
    const float bg = __builtin_sqrtf(128.f * sa2) + __builtin_fabsf(sa1);
    const float bv = __builtin_sqrtf(128.f * sb2) + __builtin_fabsf(sb1);
    bh = __builtin_elementwise_maximum(bg, 0.2785f) * bv;
  }
  // max |W_o| of row 32 g + tid / 16, a sixteenth of it per thread
  {
    const int o = (int)blockIdx.x * (kChannels / kPrepGroups) + (tid >> 4);
    const float* wo = a.w_o + (int64_t)o * kHid + (tid & 15) * (kHid / 16);
    float mo = 0.f;
#pragma unroll
    for (int i = 0; i < kHid / 16; i += 4) {
      const f32x4 v = *(const f32x4*)(wo + i);
      mo = __builtin_elementwise_maximum(
          mo, __builtin_elementwise_maximum(
                  __builtin_elementwise_maximum(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                  __builtin_elementwise_maximum(__builtin_fabsf(v.z), __builtin_fabsf(v.w))));
    }
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) mo = __builtin_elementwise_maximum(mo, __shfl_xor(mo, d));
    if ((tid & 15) == 0) a.exps[kExpO + o] = plane_exp(mo);
  }
  bh = wave_max(bh);
  if ((tid & 63) == 0) red[tid >> 6] = bh;
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < 8; ++i) bh = __builtin_elementwise_maximum(bh, red[i]);
    a.exps[kExpPart + blockIdx.x] = __builtin_bit_cast(int, bh);
    if (blockIdx.x == 0) a.exps[kExpX] = plane_exp(11.3137085f * (1.0f + 0x1p-10f));
  }
}

// The chunks' weight planes, one value (hi and lo) per thread.  Chunk c:
//   up   [a, b][k step t][hi, lo][k / 8][hidden m][k % 8]: W'[32 c + m][16 t + k] 2^e_w
//   down [out block ob][k step s][hi, lo][k / 8][out o][k % 8]: W_o[32 ob + o][32 c +
//        16 s + 8 (k / 4 % 2) + 4 (k / 8) + k % 4] 2^e_o, the hidden order in
//        which a lane of the value^T / gate^T results holds its row's values.
// A 1 KB block's two halves are the k / 8 halves, so the 32 lanes of a half
// read 512 contiguous bytes (no LDS bank conflicts).
__global__ __launch_bounds__(256) void transition_planes_kernel(TransitionArgs a) {
  const int idx = (int)(blockIdx.x * 256 + threadIdx.x);
  if (idx == 0) {
    float bh = 0.f;
    for (int g = 0; g < kPrepGroups; ++g)
      bh = __builtin_elementwise_maximum(bh, __builtin_bit_cast(float, a.exps[kExpPart + g]));
    // the margin covers the roundings of the bound and of g, v and h
    a.exps[kExpH] = plane_exp(bh * (1.0f + 0x1p-8f));
  }
  constexpr int kPer = kChunkValues / 2;  // values (hi, lo pairs) per chunk
  if (idx >= kChunks * kPer) return;
  const int c = idx / kPer;
  int v = idx - c * kPer;
  __bf16* chunk = a.planes + (int64_t)c * kChunkValues;
  float x;
  int e;
  __bf16* dst;
  if (v < (kUpBlocks / 2) * kPlaneBlock) {
    const int ab = v / (8 * kPlaneBlock);
    const int t = (v / kPlaneBlock) % 8;
    const int m = (v / 16) % 32;
    const int k = v % 16;
    const int in = 16 * t + k;
    x = (a.ln_w ? a.ln_w[in] : 1.f) *
        (ab ? a.w_b : a.w_a)[(int64_t)(kChunkHid * c + m) * kChannels + in];
    e = a.exps[kExpW + ab * kHid + kChunkHid * c + m];
    dst = chunk + ((ab * 8 + t) * 2) * kPlaneBlock + (k >> 3) * 256 + m * 8 + (k & 7);
  } else {
    v -= (kUpBlocks / 2) * kPlaneBlock;
    const int ob = v / (2 * kPlaneBlock);
    const int st = (v / kPlaneBlock) % 2;
    const int o = (v / 16) % 32;
    const int k = v % 16;
    const int hid = kChunkHid * c + 16 * st + 8 * ((k >> 2) & 1) + 4 * (k >> 3) + (k & 3);
    x = a.w_o[(int64_t)(32 * ob + o) * kHid + hid];
    e = a.exps[kExpO + 32 * ob + o];
    dst = chunk + kUpBlocks * kPlaneBlock + ((ob * 2 + st) * 2) * kPlaneBlock + (k >> 3) * 256 +
          o * 8 + (k & 7);
  }
  const float y = __builtin_ldexpf(x, e);
  const _Float16 hi = (_Float16)y;
  const _Float16 lo = (_Float16)(y - (float)hi);
  dst[0] = __builtin_bit_cast(__bf16, hi);
  dst[kPlaneBlock] = __builtin_bit_cast(__bf16, lo);
}

// Persistent: work-group g serves row tiles g, g + grid, ... (kFusedRows
// rows each).  Chunk k of the work-group's sequence (chunk k % 16 of a tile)
// sits in LDS stage k % 3; it is copied in two chunks ahead (each wave
// copying 6 KB of it): at chunk k - 2, right after the barrier that shows
// every wave done with chunk k - 3, whose stage it takes.
__global__ __launch_bounds__(kFusedWaves * 64, 1) void transition_fused_kernel(TransitionArgs a,
                                                                              int64_t rows,
                                                                              int64_t ntiles) {
  __shared__ __attribute__((aligned(16))) uint8_t wbuf[3][kChunkBytes];
  __shared__ __attribute__((aligned(16))) float fb[2][kHid];
  __shared__ __attribute__((aligned(16))) int few[2][kHid];  // -(e_x + e_w) per W' row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int ex = a.exps[kExpX], eh = a.exps[kExpH];
  for (int i = tid; i < 2 * kHid; i += kFusedWaves * 64) {
    fb[i / kHid][i % kHid] = a.fbias[i];
    few[i / kHid][i % kHid] = -(ex + a.exps[kExpW + i]);
  }
  // -(e_h + e_o) of this lane's output channels 32 ob + l32
  int eout[4];
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) eout[ob] = -(eh + a.exps[kExpO + 32 * ob + l32]);

  const int64_t my_tiles = ntiles > blockIdx.x ? (ntiles - 1 - blockIdx.x) / gridDim.x + 1 : 0;
  const int64_t total = my_tiles * kChunks;  // chunks this work-group passes through
  constexpr int kWaveBytes = kChunkBytes / kFusedWaves;  // 6 KB
  const uint8_t* csrc = reinterpret_cast<const uint8_t*>(a.planes) + w * kWaveBytes + lane * 16;
  auto dma = [&](int64_t k) {
    const uint8_t* src = csrc + (k % kChunks) * kChunkBytes;
    uint8_t* dst = wbuf[k % 3] + w * kWaveBytes;
#pragma unroll
    for (int i = 0; i < kWaveBytes / 1024; ++i) lds_dma16(src + 1024 * i, dst + 1024 * i);
  };
  if (total > 0) dma(0);
  if (total > 1) dma(1);

  // Operand reads: lane (l32, half) reads row l32's 8 values of k half `half`.
  const uint32_t rd = (uint32_t)(half * 512 + l32 * 16);
  auto blk = [&](int buf, int b) -> bf16x8 {
    return *(const bf16x8*)(wbuf[buf] + b * 1024 + rd);
  };

  int64_t k = 0;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    // This lane's row and its channels 16 t + 8 half + e (the B operand of
    // the up products); rows past the end repeat the last row.
    const int64_t row0 = tile * kFusedRows + 32 * w;
    const int64_t rr = min(row0 + l32, rows - 1);
    const int64_t ri = rr / a.rows_j;
    const float* src = a.x + ri * a.xs_i + (rr - ri * a.rows_j) * a.xs_j + 8 * half;
    f32x8 xv[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const f32x4 u = *(const f32x4*)(src + 16 * t);
      const f32x4 v = *(const f32x4*)(src + 16 * t + 4);
      xv[t] = f32x8{u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
    }
    // LayerNorm over the row's 128 channels: this lane's 64 and lane l ^ 32's.
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s += xv[t][e];
    }
    const auto ts = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, s),
                                                     __builtin_bit_cast(unsigned, s), false, false);
    const float mean = (__builtin_bit_cast(float, (unsigned)ts[0]) +
                        __builtin_bit_cast(float, (unsigned)ts[1])) * (1.0f / kChannels);
    float q = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      xv[t] = xv[t] - mean;
#pragma unroll
      for (int e = 0; e < 8; ++e) q += xv[t][e] * xv[t][e];
    }
    const auto tq = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, q),
                                                     __builtin_bit_cast(unsigned, q), false, false);
    const float var = (__builtin_bit_cast(float, (unsigned)tq[0]) +
                       __builtin_bit_cast(float, (unsigned)tq[1])) * (1.0f / kChannels);
    const float sc = __builtin_ldexpf(__builtin_amdgcn_rsqf(var + a.eps), ex);
    bf16x8 yh[8], yl[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) split_f16(xv[t] * sc, yh[t], yl[t]);

    f32x16 o[4] = {};
    for (int c = 0; c < kChunks; ++c, ++k) {
      // chunk k landed: only chunk k + 1's six copies may still be pending
      if (k + 1 < total)
        wait_vmcnt<6>();
      else
        wait_vmcnt<0>();
      __syncthreads();  // chunk k landed for every wave; chunk k - 1's stage is free
      if (k + 2 < total) dma(k + 2);
      const int buf = (int)(k % 3);
      f32x16 gacc = {}, vacc = {};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const bf16x8 ah = blk(buf, (0 * 8 + t) * 2), al = blk(buf, (0 * 8 + t) * 2 + 1);
        const bf16x8 bh = blk(buf, (1 * 8 + t) * 2), bl = blk(buf, (1 * 8 + t) * 2 + 1);
        gacc = mfma_f16(ah, yh[t], gacc);
        vacc = mfma_f16(bh, yh[t], vacc);
        gacc = mfma_f16(ah, yl[t], gacc);
        vacc = mfma_f16(bh, yl[t], vacc);
        gacc = mfma_f16(al, yh[t], gacc);
        vacc = mfma_f16(bl, yh[t], vacc);
      }
      // h of this lane's row for hidden channels 32 c + mfma_row(r, half)
      f32x16 hv;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int m = kChunkHid * c + 8 * qd + 4 * half;
        const f32x4 ba = *(const f32x4*)&fb[0][m];
        const f32x4 bb = *(const f32x4*)&fb[1][m];
        typedef int i32x4 __attribute__((ext_vector_type(4)));
        const i32x4 sa = *(const i32x4*)&few[0][m];
        const i32x4 sb = *(const i32x4*)&few[1][m];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * qd + e;
          const float g = __builtin_ldexpf(gacc[r], sa[e]) + ba[e];
          const float v = __builtin_ldexpf(vacc[r], sb[e]) + bb[e];
          hv[r] = __builtin_ldexpf(g * sigmoidf_(g) * v, eh);  // silu(a) * b, scaled
        }
      }
      bf16x8 hh[2], hl[2];
#pragma unroll
      for (int st = 0; st < 2; ++st)
        split_f16(f32x8{hv[8 * st + 0], hv[8 * st + 1], hv[8 * st + 2], hv[8 * st + 3],
                        hv[8 * st + 4], hv[8 * st + 5], hv[8 * st + 6], hv[8 * st + 7]},
                  hh[st], hl[st]);
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int b0 = kUpBlocks + (ob * 2 + st) * 2;
          const bf16x8 wh = blk(buf, b0), wl = blk(buf, b0 + 1);
          o[ob] = mfma_f16(hh[st], wh, o[ob]);
          o[ob] = mfma_f16(hh[st], wl, o[ob]);
          o[ob] = mfma_f16(hl[st], wh, o[ob]);
        }
      }
    }

    // out[row][32 ob + l32]: rows 32 w + mfma_row(r, half) of the tile
    const bool residual = a.accumulate != 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = row0 + mfma_row(r, half);
      if (row >= rows) continue;
      const int64_t i = row / a.rows_j;
      float* d = a.out + i * a.os_i + (row - i * a.rows_j) * a.os_j + l32;
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
        const float val = __builtin_ldexpf(o[ob][r], eout[ob]);
        d[32 * ob] = residual ? d[32 * ob] + val : val;
      }
    }
  }
  wait_vmcnt<0>();  // no copy in flight when the work-group ends
}

}  // namespace

hipError_t launch_transition(const TransitionArgs& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.rows_i * a.rows_j;
  if (rows == 0) return hipSuccess;
  if (a.planes == nullptr || a.fbias == nullptr || a.exps == nullptr) return hipErrorInvalidValue;
  const int64_t tiles = (rows + kFusedRows - 1) / kFusedRows;
  if (tiles > 0x7fffffff) return hipErrorInvalidValue;
  const int64_t grid = tiles < device_cu_count() ? tiles : device_cu_count();
  hipError_t e;
  hipLaunchKernelGGL(transition_prep_kernel, dim3(kPrepGroups), dim3(512), 0, stream, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(transition_planes_kernel, dim3((kChunks * kChunkValues / 2 + 255) / 256),
                     dim3(256), 0, stream, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(transition_fused_kernel, dim3((uint32_t)grid), dim3(kFusedWaves * 64), 0,
                     stream, a, rows, tiles);
  return hipGetLastError();
}

}  // namespace fpx
