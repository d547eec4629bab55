// Helpers shared by the FP32-accurate attention kernels (attention.hip on the
// FP32 matrix cores, attention_split.hip on the 16-bit matrix cores, bf16.hip): buffer
// loads, the lane-pair exchanges of the transposed S^T / O^T layout, row
// reductions, and the softmax reference constants.
#pragma once

#include "common.hpp"

namespace fpx {

constexpr int kBq = 128;   // queries per work-group
constexpr int kBk = 32;    // keys per tile
constexpr int kRowGroup = 8;  // outer rows that share a bias slice in L2
// Exact path: rescale when a tile max exceeds the reference by 8 binary
// orders (in logit units).
constexpr float kRescaleNat = 8.0f * 0.69314718055994531f;
constexpr float kRescaleLog2 = 8.0f;  // the same in log2 units
// Fast path (log2 units): the reference snaps to 0 while the row max lies in
// [-kSnap, kSnap]; the running sum may grow to kSumLimit before a rescale; a
// rescale forced by the sum moves the reference up by at least kLift.
constexpr float kSnap = 56.0f;
constexpr float kSumLimit = 18446744073709551616.0f;  // 2^64
constexpr float kLift = 40.0f;

// Work item -> (outer row b, head h, query tile qt).  Items are dispatched
// round-robin over the XCDs (item % kXcds), each XCD with its own 4 MB L2.
// Item counts are rows8 * kHeads * nqt, rows8 = batch rounded up to
// kRowGroup.
//   pair groups (ppg > 0): the kHeads * nqt (head, query tile) pairs form
//     groups of ppg pairs; XCD x serves groups x, x + kXcds, ... one after
//     the other, each for every outer row, row-major (the ppg pairs of a row
//     are consecutive items, so they share the row's K/V slices in L2).  The
//     host picks ppg so that a group's bias slices (ppg x 128 queries x np
//     keys x 4 bytes) stay within about 2.5 MB of the L2.
//   row groups (ppg = 0): head, group of kRowGroup outer rows, query tile,
//     row in group, each XCD a contiguous range; logical row lr = u groups
//     + v runs outer row 8 v + u, so each XCD takes every 8th outer row and
//     rows that leave a launch early spread evenly over the XCDs.
__device__ __forceinline__ void attn_item(uint32_t item, uint32_t total, int batch, int nqt, int ppg,
                                          int& b, int& h, int& qt) {
  if (ppg > 0) {
    const int xcd = (int)(item % kXcds);
    const int slot = (int)(item / kXcds);
    const int rows8 = (int)(total / (uint32_t)(kHeads * nqt));
    const int pass = slot / (rows8 * ppg);
    const int within = slot - pass * rows8 * ppg;
    b = within / ppg;
    const int pair = (xcd + kXcds * pass) * ppg + within % ppg;
    h = pair / nqt;
    qt = pair % nqt;
    return;
  }
  const uint32_t logical = xcd_remap(item, total);
  const int groups = (batch + kRowGroup - 1) / kRowGroup;
  const int per_head = groups * kRowGroup * nqt;
  h = (int)(logical / per_head);
  const int rem = (int)(logical % per_head);
  const int grp = rem / (kRowGroup * nqt);
  const int in_grp = rem % (kRowGroup * nqt);
  qt = in_grp / kRowGroup;
  const int lr = grp * kRowGroup + in_grp % kRowGroup;
  b = kRowGroup * (lr % groups) + lr / groups;
}

// Pair groups of attn_item: the largest ppg dividing nqt / 2 (so the
// kHeads * nqt (head, query tile) pairs form a multiple of kXcds groups)
// whose bias slices (slice_bytes per pair) fit kGroupBiasBytes of an XCD's
// L2; 0 (the row-group order) when there is none, or when only ppg = 1
// fits (every K/V slice would then be fetched once per pair).
constexpr uint64_t kGroupBiasBytes = 2560ull << 10;
inline int pair_group_size(int nqt, uint64_t slice_bytes) {
  if (nqt % 2 != 0) return 0;
  for (int g = nqt / 2; g >= 2; --g)
    if ((nqt / 2) % g == 0 && (uint64_t)g * slice_bytes <= kGroupBiasBytes) return g;
  return 0;
}

// LDS rings of key tiles (attention_split.hip, bf16.hip): rows of 64 bytes.
// 16-byte chunk c of plane row r sits at chunk c ^ swz(r).  The operand
// reads (rows 0-31, one chunk per instruction and half-wave) then hit
// distinct banks in every group of 8 rows at 128 bytes per cycle and of 16
// rows at 256 bytes per cycle.
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }
// One global_load_lds_dwordx4: lane l copies 16 bytes from src into the LDS
// at dst + 16 l (dst uniform across the wave).  Written as inline assembly
// so the compiler does not see an LDS write it cannot tell apart from the
// stages being read, which would make it wait for every copy before the next
// LDS read; the kernel waits for the copies itself (wait_vmcnt).  Loads the
// compiler issues before or after stay correctly waited for, since vector
// memory loads retire in issue order.  M0 is clobbered: the kernel makes no
// other use of it (no LDS DMA, message or indexed-register instruction of
// the compiler's own).
__device__ __forceinline__ void lds_dma16(const void* src, const uint8_t* dst) {
  const uint32_t lds_addr =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)dst;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_addr)
               : "memory", "m0");
}

// The same copy addressed as a wave-uniform 64-bit base in SGPRs plus a
// per-lane 32-bit offset (global_load_lds_dwordx4's saddr form), so that
// advancing a copy by a tile costs scalar instructions only.  lds_addr: the
// LDS byte address of lane 0's 16 bytes (wave-uniform).  The instruction
// offset stays 0: it would move the LDS address as well as the global one.
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void* sbase, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds_addr)
               : "memory", "m0");
}
// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_address(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ f32x16 cat4(f32x4 a, f32x4 b, f32x4 c, f32x4 d) {
  f32x16 r;
  r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
  r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  r[8] = c.x; r[9] = c.y; r[10] = c.z; r[11] = c.w;
  r[12] = d.x; r[13] = d.y; r[14] = d.z; r[15] = d.w;
  return r;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const float* base, int64_t bytes) {
  // dword 3 = 0x00020000: raw 32-bit buffer access on gfx9-family parts.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ f32x4 buffer_f4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// max / sum of v over the lane pair (l, l ^ 32) with v_permlane32_swap
// (no LDS round trip): after the swap one copy holds the low half in both
// halves and the other the high half.
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_elementwise_maximum(__builtin_bit_cast(float, (unsigned)r[0]),
                                       __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// NaN-propagating max of 16 values (v_maximum3_f32): a NaN logit poisons its
// row, as in the native softmax.
__device__ __forceinline__ float max16(const f32x16& s) {
  auto mx = [](float x, float y) { return __builtin_elementwise_maximum(x, y); };
  float m0 = mx(mx(s[0], s[1]), s[2]);
  float m1 = mx(mx(s[3], s[4]), s[5]);
  float m2 = mx(mx(s[6], s[7]), s[8]);
  float m3 = mx(mx(s[9], s[10]), s[11]);
  float m4 = mx(mx(s[12], s[13]), s[14]);
  m0 = mx(mx(m0, m1), s[15]);
  m2 = mx(mx(m2, m3), m4);
  return mx(m0, m2);
}

__device__ __forceinline__ float sum16(const f32x16& p) {
  float a0 = p[0] + p[4], a1 = p[1] + p[5], a2 = p[2] + p[6], a3 = p[3] + p[7];
  a0 += p[8];
  a1 += p[9];
  a2 += p[10];
  a3 += p[11];
  a0 += p[12];
  a1 += p[13];
  a2 += p[14];
  a3 += p[15];
  return (a0 + a1) + (a2 + a3);
}

}  // namespace fpx
