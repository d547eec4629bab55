// Flash-style triangle attention on the CDNA4 FP32 matrix cores.
//
// One work-group = (outer row b, head h, 128 queries); four wavefronts, each
// owning 32 queries.  Keys are streamed in tiles of 32: K and V^T tiles are
// staged once in LDS for the four waves, the [128 x 32] triangle-bias tile and
// the 32 mask-bias values beside them.  The N x N logits of a row and the
// N^3 score volume never reach HBM.
//
// Per key tile each wave computes S^T = K Q^T (16 x v_mfma_f32_32x32x2_f32)
// and O^T += V^T P^T (16 more).  Computing the transposed products puts one
// query per lane column (lane % 32) in both results, so the online-softmax
// row statistics, the P operand and the O rescale all live in the lane that
// needs them: the only cross-lane step is one xor-32 exchange of the tile max.
//
// Logits are formed in the native order fl(fl(s + mask_bias) + bias)
// (patches/protenix/0005-*.patch:36-45; kernels/amd/fireprot_softmax_fp32.cpp:
// 33-35), so fully masked padding rows reproduce the native tie structure of
// the -1e9-quantised logits.  exp is taken of (x - max) formed in the natural
// domain before scaling by log2(e), which keeps those ties exact.  A row whose
// logits are all -inf gives NaN, as torch.softmax does.
#include "common.hpp"
#include "kernels.hpp"

#include <cmath>

namespace fpx {
namespace {

constexpr int kBq = 128;   // queries per work-group
constexpr int kBk = 32;    // keys per tile
constexpr int kPad = 4;    // LDS row padding (floats): conflict-free b128 reads
constexpr int kThreads = 256;

struct TileRegs {
  f32x4 k;
  f32x4 v;
  f32x4 b[4];
  f32x4 m;
};

template <int LAYOUT>
__device__ __forceinline__ void load_tile(const AttnArgs& a, int b, int h, int j0, int k0, int tid,
                                          TileRegs& t) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const int row8 = tid >> 3;        // 0..31
  const int col4 = (tid & 7) * 4;   // 0..28
  if (LAYOUT == kAttnBlock) {
    const int64_t bh = (int64_t)b * kHeads + h;
    t.k = *(const f32x4*)(a.k + (bh * a.np + k0 + row8) * kHeadDim + col4);
    t.v = *(const f32x4*)(a.v + (bh * kHeadDim + row8) * a.np + k0 + col4);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int64_t row = j0 + row8 + 32 * m;
      t.b[m] = *(const f32x4*)(a.bias + ((int64_t)h * a.bias_rows + row) * a.bias_stride + k0 + col4);
    }
    if (tid < 8) t.m = *(const f32x4*)(a.mbias + (int64_t)b * a.mb_stride + k0 + 4 * tid);
  } else {
    const int key = k0 + row8;
    const bool kin = key < a.n;
    const int64_t kv = (((int64_t)b * a.n + key) * kHeads + h) * kHeadDim + col4;
    t.k = kin ? *(const f32x4*)(a.k + kv) : zero;
    t.v = kin ? *(const f32x4*)(a.v + kv) : zero;
    const bool cin = k0 + col4 < a.n;  // n % 4 == 0: a float4 is all-in or all-out
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int row = j0 + row8 + 32 * m;
      t.b[m] = (cin && row < a.n)
                   ? *(const f32x4*)(a.bias + ((int64_t)h * a.bias_rows + row) * a.bias_stride + k0 + col4)
                   : zero;
    }
    if (tid < 8) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = k0 + 4 * tid + e;
        t.m[e] = kk < a.n ? (a.mbias ? a.mbias[(int64_t)b * a.mb_stride + kk] : 0.f) : -INFINITY;
      }
    }
  }
}

template <int LAYOUT>
__global__ __launch_bounds__(kThreads) void attention_kernel(AttnArgs a, int nqt, int nkt,
                                                            uint32_t total) {
  __shared__ __attribute__((aligned(16))) float Ks[kBk][kHeadDim + kPad];
  __shared__ __attribute__((aligned(16))) float Vs[kHeadDim][kBk + kPad];
  __shared__ __attribute__((aligned(16))) float Bs[kBq][kBk + kPad];
  __shared__ __attribute__((aligned(16))) float Ms[kBk];

  const uint32_t logical = xcd_remap(blockIdx.x, total);
  const int qt = logical % nqt;
  const int h = (logical / nqt) % kHeads;
  const int b = logical / (nqt * kHeads);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int j0 = qt * kBq;
  const int jq = j0 + 32 * w + l32;

  // Q fragment (B operand of S^T = K Q^T): lane holds Q[jq][16*half + s].
  float qf[16];
  {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const float* src;
    bool ok = true;
    if (LAYOUT == kAttnBlock) {
      src = a.q + (((int64_t)b * kHeads + h) * a.np + jq) * kHeadDim + 16 * half;
    } else {
      ok = jq < a.n;
      src = a.q + (((int64_t)b * a.n + (ok ? jq : 0)) * kHeads + h) * kHeadDim + 16 * half;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f32x4 v = ok ? *(const f32x4*)(src + 4 * t) : zero;
      qf[4 * t + 0] = v.x;
      qf[4 * t + 1] = v.y;
      qf[4 * t + 2] = v.z;
      qf[4 * t + 3] = v.w;
    }
  }

  f32x16 o = {};
  float m_run = -INFINITY;
  float l_run = 0.f;

  TileRegs regs;
  load_tile<LAYOUT>(a, b, h, j0, 0, tid, regs);

  const int row8 = tid >> 3;
  const int col4 = (tid & 7) * 4;
  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();  // previous tile's LDS reads are complete
    *(f32x4*)&Ks[row8][col4] = regs.k;
    if (LAYOUT == kAttnBlock) {
      *(f32x4*)&Vs[row8][col4] = regs.v;
    } else {
      Vs[col4 + 0][row8] = regs.v.x;
      Vs[col4 + 1][row8] = regs.v.y;
      Vs[col4 + 2][row8] = regs.v.z;
      Vs[col4 + 3][row8] = regs.v.w;
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) *(f32x4*)&Bs[row8 + 32 * m][col4] = regs.b[m];
    if (tid < 8) *(f32x4*)&Ms[4 * tid] = regs.m;
    __syncthreads();
    if (kt + 1 < nkt) load_tile<LAYOUT>(a, b, h, j0, (kt + 1) * kBk, tid, regs);

    // S^T[key][q] = sum_c K[key][c] Q[q][c]; channel for step s, half hb is 16*hb + s.
    f32x16 s = {};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f32x4 kv = *(const f32x4*)&Ks[l32][16 * half + 4 * t];
      s = mfma32(kv.x, qf[4 * t + 0], s);
      s = mfma32(kv.y, qf[4 * t + 1], s);
      s = mfma32(kv.z, qf[4 * t + 2], s);
      s = mfma32(kv.w, qf[4 * t + 3], s);
    }

    // Register r of this lane is key 8*(r/4) + 4*half + r%4 of the tile.
    float x[16];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x4 mb = *(const f32x4*)&Ms[8 * rr + 4 * half];
      const f32x4 bb = *(const f32x4*)&Bs[32 * w + l32][8 * rr + 4 * half];
      x[4 * rr + 0] = (s[4 * rr + 0] + mb.x) + bb.x;
      x[4 * rr + 1] = (s[4 * rr + 1] + mb.y) + bb.y;
      x[4 * rr + 2] = (s[4 * rr + 2] + mb.z) + bb.z;
      x[4 * rr + 3] = (s[4 * rr + 3] + mb.w) + bb.w;
    }
    float mt = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, x[r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast((m_run - m_use) * kLog2e);
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x[r] = exp2_fast((x[r] - m_use) * kLog2e);
      psum += x[r];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] *= alpha;

    // O^T[c][q] += sum_key V^T[c][key] P^T[key][q]; MFMA r pairs keys of register r.
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x4 vv = *(const f32x4*)&Vs[l32][8 * rr + 4 * half];
      o = mfma32(vv.x, x[4 * rr + 0], o);
      o = mfma32(vv.y, x[4 * rr + 1], o);
      o = mfma32(vv.z, x[4 * rr + 2], o);
      o = mfma32(vv.w, x[4 * rr + 3], o);
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  if (jq < a.n) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int c = 8 * rr + 4 * half;  // channels c..c+3 of head h
      f32x4 ov = {o[4 * rr + 0] / l_tot, o[4 * rr + 1] / l_tot, o[4 * rr + 2] / l_tot,
                  o[4 * rr + 3] / l_tot};
      if (LAYOUT == kAttnBlock) {
        const int64_t off = ((int64_t)b * a.n + jq) * kHidden + h * kHeadDim + c;
        if (a.gate) ov = ov * *(const f32x4*)(a.gate + off);
        *(f32x4*)(a.out + off) = ov;
      } else {
        *(f32x4*)(a.out + (((int64_t)b * a.n + jq) * kHeads + h) * kHeadDim + c) = ov;
      }
    }
  }
}

}  // namespace

hipError_t launch_attention(int layout, const AttnArgs& a, hipStream_t stream) {
  const int nqt = (int)((layout == kAttnBlock ? a.np : round_up(a.n, kBq)) / kBq);
  const int nkt = (int)((layout == kAttnBlock ? a.np : round_up(a.n, kBk)) / kBk);
  const uint64_t total = (uint64_t)a.batch * kHeads * nqt;
  if (total == 0) return hipSuccess;
  if (total > 0x7fffffffull) return hipErrorInvalidValue;
  if (layout == kAttnBlock) {
    hipLaunchKernelGGL(attention_kernel<kAttnBlock>, dim3((uint32_t)total), dim3(kThreads), 0,
                       stream, a, nqt, nkt, (uint32_t)total);
  } else {
    hipLaunchKernelGGL(attention_kernel<kAttnHeadLast>, dim3((uint32_t)total), dim3(kThreads), 0,
                       stream, a, nqt, nkt, (uint32_t)total);
  }
  return hipGetLastError();
}

}  // namespace fpx
