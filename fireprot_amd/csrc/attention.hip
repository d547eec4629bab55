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
#ifndef FPX_ATTN_ROW_GROUP
#define FPX_ATTN_ROW_GROUP 8
#endif
constexpr int kRowGroup = FPX_ATTN_ROW_GROUP;  // outer rows that share a bias slice in L2

struct TileRegs {
  f32x4 v;
  f32x4 b[4];
  f32x4 m;
};

// K rows of tile k0 (thread: key row8, channels col4..col4+3).
template <int LAYOUT>
__device__ __forceinline__ f32x4 load_k(const AttnArgs& a, int b, int h, int k0, int tid) {
  const int row8 = tid >> 3;
  const int col4 = (tid & 7) * 4;
  if (LAYOUT == kAttnBlock) {
    const int64_t bh = (int64_t)b * kHeads + h;
    return *(const f32x4*)(a.k + (bh * a.np + k0 + row8) * kHeadDim + col4);
  }
  const int key = k0 + row8;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  return key < a.n ? *(const f32x4*)(a.k + (((int64_t)b * a.n + key) * kHeads + h) * kHeadDim + col4)
                   : zero;
}

// V^T, triangle-bias and mask-bias slices of tile k0.
template <int LAYOUT>
__device__ __forceinline__ void load_vbm(const AttnArgs& a, int b, int h, int j0, int k0, int tid,
                                         TileRegs& t) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const int row8 = tid >> 3;        // 0..31
  const int col4 = (tid & 7) * 4;   // 0..28
  if (LAYOUT == kAttnBlock) {
    const int64_t bh = (int64_t)b * kHeads + h;
    t.v = *(const f32x4*)(a.v + (bh * kHeadDim + row8) * a.np + k0 + col4);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int64_t row = j0 + row8 + 32 * m;
      t.b[m] = *(const f32x4*)(a.bias + ((int64_t)h * a.bias_rows + row) * a.bias_stride + k0 + col4);
    }
    if (tid < 8) t.m = *(const f32x4*)(a.mbias + (int64_t)b * a.mb_stride + k0 + 4 * tid);
  } else {
    const int key = k0 + row8;
    t.v = key < a.n ? *(const f32x4*)(a.v + (((int64_t)b * a.n + key) * kHeads + h) * kHeadDim + col4)
                    : zero;
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

// max / sum of v over the lane pair (l, l ^ 32) with v_permlane32_swap
// (no LDS round trip): after the swap one copy holds the low half in both
// halves and the other the high half.
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// S^T[key][q] = sum_c K[key][c] Q[q][c] for the 32 keys in Ks; the channel of
// step s in lane half hb is 16*hb + s.
__device__ __forceinline__ f32x16 qk_tile(const float (*Ks)[kHeadDim + kPad], const float* qf,
                                          int l32, int half) {
  f32x16 s = {};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const f32x4 kv = *(const f32x4*)&Ks[l32][16 * half + 4 * t];
    s = mfma32(kv.x, qf[4 * t + 0], s);
    s = mfma32(kv.y, qf[4 * t + 1], s);
    s = mfma32(kv.z, qf[4 * t + 2], s);
    s = mfma32(kv.w, qf[4 * t + 3], s);
  }
  return s;
}

template <int LAYOUT>
__global__ __launch_bounds__(kThreads) void attention_kernel(AttnArgs a, int nqt, int nkt,
                                                            uint32_t total) {
  __shared__ __attribute__((aligned(16))) float Ks[kBk][kHeadDim + kPad];
  __shared__ __attribute__((aligned(16))) float Vs[kHeadDim][kBk + kPad];
  __shared__ __attribute__((aligned(16))) float Bs[kBq][kBk + kPad];
  __shared__ __attribute__((aligned(16))) float Ms[kBk];

  // Logical order, slowest to fastest: head, block of kRowGroup outer rows,
  // query tile, outer row in the block.  The work-groups that run together
  // on one XCD then share each triangle-bias slice across kRowGroup outer rows
  // and each K/V slice across all query tiles, in that XCD's L2.
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

  // Online-softmax state per query (this lane's column): running max m_run,
  // its log2-scaled value c_run = fl(m_run * log2 e) (-inf until a finite max
  // appears) and the running sum l_run.  p = exp2(fma(x, log2 e, -c)) with the
  // same rounded c used for the rescale alpha = exp2(c_old - c_new), so every
  // weight carries one common factor that cancels in O / l: the ratios
  // e^(x - x') stay exact, -1e9-quantised masked logits included.
  f32x16 o = {};
  float m_run = -INFINITY;
  float c_run = -INFINITY;
  float l_run = 0.f;

  const int row8 = tid >> 3;
  const int col4 = (tid & 7) * 4;
  TileRegs regs;

  auto store_vbm = [&]() {
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
  };

  // Softmax of the current tile's logits (in s, lane register r = key
  // 8*(r/4) + 4*half + r%4) and O^T[c][q] += V^T[c][key] P^T[key][q].
  auto softmax_pv = [&](f32x16 s) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x4 mb = *(const f32x4*)&Ms[8 * rr + 4 * half];
      const f32x4 bb = *(const f32x4*)&Bs[32 * w + l32][8 * rr + 4 * half];
      s[4 * rr + 0] = (s[4 * rr + 0] + mb.x) + bb.x;
      s[4 * rr + 1] = (s[4 * rr + 1] + mb.y) + bb.y;
      s[4 * rr + 2] = (s[4 * rr + 2] + mb.z) + bb.z;
      s[4 * rr + 3] = (s[4 * rr + 3] + mb.w) + bb.w;
    }
    float mt = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
    mt = xor32_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const float c_new = m_new == -INFINITY ? -INFINITY : m_new * kLog2e;
    const float c_use = m_new == -INFINITY ? 0.f : c_new;
    const float alpha = exp2_fast(c_run - c_use);
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = exp2_fast(__builtin_fmaf(s[r], kLog2e, -c_use));
      psum += s[r];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    c_run = c_new;
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[r] *= alpha;
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x4 vv = *(const f32x4*)&Vs[l32][8 * rr + 4 * half];
      o = mfma32(vv.x, s[4 * rr + 0], o);
      o = mfma32(vv.y, s[4 * rr + 1], o);
      o = mfma32(vv.z, s[4 * rr + 2], o);
      o = mfma32(vv.w, s[4 * rr + 3], o);
    }
  };

  // Prologue: K of tile 0 into LDS, S^T of tile 0; stage K(1) and V/bias/mask(0).
  *(f32x4*)&Ks[row8][col4] = load_k<LAYOUT>(a, b, h, 0, tid);
  __syncthreads();
  f32x16 s_cur = qk_tile(Ks, qf, l32, half);
  f32x4 kreg = {0.f, 0.f, 0.f, 0.f};
  if (nkt > 1) kreg = load_k<LAYOUT>(a, b, h, kBk, tid);
  load_vbm<LAYOUT>(a, b, h, j0, 0, tid, regs);

  // Steady state: LDS holds K of tile kt+1 and V/bias/mask of tile kt, so
  // the 16 MFMAs of S^T(kt+1) are independent of the softmax of tile kt.
  for (int kt = 0; kt + 1 < nkt; ++kt) {
    __syncthreads();  // every wave is done with K(kt) and V/bias/mask(kt-1)
    *(f32x4*)&Ks[row8][col4] = kreg;
    store_vbm();
    __syncthreads();
    if (kt + 2 < nkt) kreg = load_k<LAYOUT>(a, b, h, (kt + 2) * kBk, tid);
    load_vbm<LAYOUT>(a, b, h, j0, (kt + 1) * kBk, tid, regs);
    const f32x16 s_next = qk_tile(Ks, qf, l32, half);
    softmax_pv(s_cur);
    s_cur = s_next;
  }
  __syncthreads();
  store_vbm();
  __syncthreads();
  softmax_pv(s_cur);

  const float l_tot = xor32_sum(l_run);
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
  const uint64_t groups = ((uint64_t)a.batch + kRowGroup - 1) / kRowGroup;
  const uint64_t total = groups * kRowGroup * kHeads * nqt;
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
