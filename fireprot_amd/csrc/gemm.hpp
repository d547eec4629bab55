// The GEMM mainloop of the triangle-multiplication contraction:
// FP32-accurate products on the 16-bit matrix cores (fp16 hi/lo planes).
//
// One work-group (256 threads, four waves) accumulates a 128 x 128 tile
//   C[i][j] = sum_k A[i][k] B[j][k]
// with both operands K-contiguous.  Wave w owns the 64 x 64 quadrant
// (64 (w / 2), 64 (w % 2)) as 2 x 2 blocks of 32 x 32 MFMA tiles.
#pragma once

#include "common.hpp"
#include "split.hpp"

namespace fpx {

constexpr int kGemmTile = 128;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const float* base, int64_t bytes) {
  // dword 3 = 0x00020000: raw 32-bit buffer access on gfx9-family parts.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ f32x4 buffer_load_f4(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                uint32_t soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Stages of 16 keys (one k step), double-buffered; rows padded to 24 16-bit
// values (48 B), conflict-free b128 reads.
constexpr int kSplitK = 16;
constexpr int kSplitRow = kSplitK + 8;

// The product on v_mfma_f32_32x32x16_f16 with power-of-two scaled fp16
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

  // Two register slots of staged rows: stage s sits in slot s % 2 from its
  // loads (issued two stages ahead) until its split into LDS.
  f32x4 ga[2][2], gb[2][2];
  auto load = [&](int kt, int slot) {
    // one buffer resource per 32-key run: the 32-bit offsets span 128 rows
    const int64_t run = (int64_t)(kt >> 1) * kblock;
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a + run, (127 * lda + 2 * kSplitK) * 4);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(b + run, (127 * ldb + 2 * kSplitK) * 4);
    const uint32_t s = (uint32_t)((kt & 1) * kSplitK * 4);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      ga[slot][u] = buffer_load_f4(ra, va + u * pa, s);
      gb[slot][u] = buffer_load_f4(rb, vb + u * pb, s);
    }
  };
  auto store = [&](int buf, int slot) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bf16x4 h, l;
      split_f16(ldexp4(ga[slot][u], xa[u]), h, l);
      *(bf16x4*)&As[buf][0][lrow + 64 * u][lc4] = h;
      *(bf16x4*)&As[buf][1][lrow + 64 * u][lc4] = l;
      split_f16(ldexp4(gb[slot][u], xb[u]), h, l);
      *(bf16x4*)&Bs[buf][0][lrow + 64 * u][lc4] = h;
      *(bf16x4*)&Bs[buf][1][lrow + 64 * u][lc4] = l;
    }
  };

  // Stage kt: its products from LDS buffer kt % 2; then stage kt + 1 goes
  // from its slot into the other buffer and stage kt + 3 is loaded into
  // that slot.  The slots and buffers are compile-time indices (two stages
  // per loop iteration).
  auto step = [&](int kt, int buf, int slot) {
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
      store(buf ^ 1, slot);
      if (kt + 3 < nk) load(kt + 3, slot);
    }
    __syncthreads();
  };

  load(0, 0);
  if (nk > 1) load(1, 1);
  store(0, 0);
  if (nk > 2) load(2, 0);  // after stage 0's split has read slot 0
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, 0, 1);
    if (kt + 1 < nk) step(kt + 1, 1, 0);
  }
}

}  // namespace fpx
