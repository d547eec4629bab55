// GEMM mainloops shared by the triangle-multiplication contraction and the
// pair transition's output projection: FP32 matrix cores (gemm_nt_128) and
// FP32-accurate fp16 planes (gemm_nt_128_f16).
//
// One work-group (256 threads, four waves) accumulates a 128 x 128 tile
//   C[i][j] = sum_k A[i][k] B[j][k]
// with both operands K-contiguous (row-major, row strides lda / ldb floats).
// Wave w owns the 64 x 64 quadrant (64 (w / 2), 64 (w % 2)) as 2 x 2 blocks
// of v_mfma_f32_32x32x2_f32.  Keys are consumed in 32-wide stages staged in
// LDS (rows padded to 36 floats: the b128 fragment reads of 16 lanes hit 64
// distinct banks), double-buffered so the next stage's global loads are in
// flight during this stage's 64 MFMAs per wave; one barrier per stage.  Per
// stage, lane half h feeds keys 16h .. 16h + 15 of the stage (the sum over
// keys is order-free), so both fragments are contiguous row segments.
#pragma once

#include "common.hpp"
#include "split.hpp"

namespace fpx {

constexpr int kGemmTile = 128;
constexpr int kKStage = 32;
constexpr int kKPad = kKStage + 4;

typedef float GemmStage[kGemmTile][kKPad];

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const float* base, int64_t bytes) {
  // dword 3 = 0x00020000: raw 32-bit buffer access on gfx9-family parts.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ f32x4 buffer_load_f4(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                uint32_t soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// acc[rb][cb] (lane l, register r) += C[64 (w / 2) + 32 rb + mfma_row(r, l / 32)]
//                                       [64 (w % 2) + 32 cb + l % 32]
// over keys 0 .. 32 nk - 1.  a and b point at row 0 of the two 128-row
// tiles; all 128 rows of both and all 32 nk keys must be readable (callers
// pad their buffers), and (127 ld + 32 nk) * 4 bytes must stay below 2 GiB.
// As and Bs are the caller's LDS stages; the routine ends with a barrier, so
// they may be reused at once.
__device__ __forceinline__ void gemm_nt_128(const float* a, int64_t lda, const float* b,
                                            int64_t ldb, int nk, GemmStage* As, GemmStage* Bs,
                                            f32x16 (&acc)[2][2]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int wi = (w >> 1) * 64;
  const int wj = (w & 1) * 64;

  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a, (127 * lda + kKStage * nk) * 4);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(b, (127 * ldb + kKStage * nk) * 4);
  // Thread (row = tid / 8 + 32 u, keys 4 (tid % 8) .. +3) of each stage.
  const int lrow = tid >> 3;
  const int lc4 = (tid & 7) * 4;
  const uint32_t va = (uint32_t)((lrow * lda + lc4) * 4);
  const uint32_t vb = (uint32_t)((lrow * ldb + lc4) * 4);
  const uint32_t pa = (uint32_t)(32 * lda * 4);  // 32 rows further down
  const uint32_t pb = (uint32_t)(32 * ldb * 4);

  f32x4 ga[4], gb[4];
  auto load = [&](int kt) {
    const uint32_t s = (uint32_t)kt * (kKStage * 4);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ga[u] = buffer_load_f4(ra, va + u * pa, s);
      gb[u] = buffer_load_f4(rb, vb + u * pb, s);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      *(f32x4*)&As[buf][lrow + 32 * u][lc4] = ga[u];
      *(f32x4*)&Bs[buf][lrow + 32 * u][lc4] = gb[u];
    }
  };

  load(0);
  store(0);
  if (nk > 1) load(1);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int kc = 16 * half + 4 * t;
      const f32x4 a0 = *(const f32x4*)&As[buf][wi + l32][kc];
      const f32x4 a1 = *(const f32x4*)&As[buf][wi + 32 + l32][kc];
      const f32x4 b0 = *(const f32x4*)&Bs[buf][wj + l32][kc];
      const f32x4 b1 = *(const f32x4*)&Bs[buf][wj + 32 + l32][kc];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[0][0] = mfma32(a0[e], b0[e], acc[0][0]);
        acc[0][1] = mfma32(a0[e], b1[e], acc[0][1]);
        acc[1][0] = mfma32(a1[e], b0[e], acc[1][0]);
        acc[1][1] = mfma32(a1[e], b1[e], acc[1][1]);
      }
    }
    if (kt + 1 < nk) {
      store(buf ^ 1);
      if (kt + 2 < nk) load(kt + 2);
    }
    __syncthreads();
  }
}

// ------------------------------------------------ FP32-accurate, fp16 cores
//
// Stages of 16 keys (one k step), double-buffered; rows padded to 24 16-bit
// values (48 B), conflict-free b128 reads.
constexpr int kSplitK = 16;
constexpr int kSplitRow = kSplitK + 8;

// The same product on v_mfma_f32_32x32x16_f16 with power-of-two scaled fp16
// (hi, lo) planes (split.hpp): row r of A is scaled by 2^ea[r] and row r of
// B by 2^eb[r] (ea, eb: 128 per-row exponents, plane_exp of each row's max
// |value| over all keys, in LDS), so acc[rb][cb] comes out scaled by
// 2^(ea[row] + eb[col]) for the caller to undo with ldexp.  Three terms (hi
// hi, hi lo, lo hi) per 16-key stage: 12 MFMAs per wave and stage.  A row's
// keys are runs of 32 contiguous values, kblock floats apart (32: the whole
// row contiguous); nk (16-key stages) is even when kblock != 32.
typedef __bf16 F16Stage[2][kGemmTile][kSplitRow];  // planes hi, lo (fp16 bits)

__device__ __forceinline__ void gemm_nt_128_f16(const float* a, int64_t lda, const float* b,
                                                int64_t ldb, int64_t kblock, int nk,
                                                F16Stage* As, F16Stage* Bs,
                                                const int* ea, const int* eb,
                                                f32x16 (&acc)[2][2]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int wi = (w >> 1) * 64;
  const int wj = (w & 1) * 64;

  // Thread (row = tid / 4 + 64 u, keys 4 (tid % 4) .. +3) of each stage.
  const int lrow = tid >> 2;
  const int lc4 = (tid & 3) * 4;
  const uint32_t va = (uint32_t)((lrow * lda + lc4) * 4);
  const uint32_t vb = (uint32_t)((lrow * ldb + lc4) * 4);
  const uint32_t pa = (uint32_t)(64 * lda * 4);  // 64 rows further down
  const uint32_t pb = (uint32_t)(64 * ldb * 4);
  const int xa[2] = {ea[lrow], ea[lrow + 64]};
  const int xb[2] = {eb[lrow], eb[lrow + 64]};

  f32x4 ga[2], gb[2];
  auto load = [&](int kt) {
    // one buffer resource per 32-key run: the 32-bit offsets span 128 rows
    const int64_t run = (int64_t)(kt >> 1) * kblock;
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a + run, (127 * lda + 2 * kSplitK) * 4);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(b + run, (127 * ldb + 2 * kSplitK) * 4);
    const uint32_t s = (uint32_t)((kt & 1) * kSplitK * 4);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      ga[u] = buffer_load_f4(ra, va + u * pa, s);
      gb[u] = buffer_load_f4(rb, vb + u * pb, s);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bf16x4 h, l;
      split_f16(ldexp4(ga[u], xa[u]), h, l);
      *(bf16x4*)&As[buf][0][lrow + 64 * u][lc4] = h;
      *(bf16x4*)&As[buf][1][lrow + 64 * u][lc4] = l;
      split_f16(ldexp4(gb[u], xb[u]), h, l);
      *(bf16x4*)&Bs[buf][0][lrow + 64 * u][lc4] = h;
      *(bf16x4*)&Bs[buf][1][lrow + 64 * u][lc4] = l;
    }
  };

  load(0);
  store(0);
  if (nk > 1) load(1);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    bf16x8 ap[2][2], bp[2][2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int pl = 0; pl < 2; ++pl) {
        ap[q][pl] = *(const bf16x8*)&As[buf][pl][wi + 32 * q + l32][8 * half];
        bp[q][pl] = *(const bf16x8*)&Bs[buf][pl][wj + 32 * q + l32][8 * half];
      }
    }
    constexpr int kTerms[3][2] = {{0, 0}, {0, 1}, {1, 0}};
#pragma unroll
    for (int t = 0; t < 3; ++t) {
#pragma unroll
      for (int rb2 = 0; rb2 < 2; ++rb2) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
          acc[rb2][cb] = mfma_f16(ap[rb2][kTerms[t][0]], bp[cb][kTerms[t][1]], acc[rb2][cb]);
      }
    }
    if (kt + 1 < nk) {
      store(buf ^ 1);
      if (kt + 2 < nk) load(kt + 2);
    }
    __syncthreads();
  }
}

}  // namespace fpx
