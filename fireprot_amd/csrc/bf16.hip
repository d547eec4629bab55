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
#include "attn_common.hpp"
#include "common.hpp"
#include "kernels.hpp"

#include <cmath>
#include <type_traits>

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
  // Two row tiles: the MFMAs read one while the next is normalised into the
  // other, so a tile needs one barrier (the FP32 kernel's structure).
  __shared__ __attribute__((aligned(16))) __bf16 xs[2][kRows][kXsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  // B[k][col]: column 32*(w&3) + l32 of weight group w>>2, k = 16*m + 8*half + e.
  bf16x8 wf[8];
  {
    const __bf16* src = a.w[w >> 2] + (int64_t)(32 * (w & 3) + l32) * kChannels + 8 * half;
#pragma unroll
    for (int m = 0; m < 8; ++m) wf[m] = *(const bf16x8*)(src + 16 * m);
  }
  const int col_w = MODE == kProjOut ? 32 * w + l32 : 32 * (w & 3) + l32;
  const float col_bias = a.bias_vec != nullptr ? (float)a.bias_vec[col_w] : 0.f;

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
        const int64_t c = a.xs_h != 0 ? (c8 >> 5) * a.xs_h + (c8 & 31) : c8;
        stage_vec[t] = (idx < kVecs && j < a.rows_j)
                           ? *(const bf16x8*)(a.x + (int64_t)i * a.xs_i + (int64_t)j * a.xs_j + c)
                           : zero8;
      }
    }
  };

  auto stage_rows = [&](int tile, int buf) {
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
        *(bf16x2*)&xs[buf][row][2 * lane] = yb;
        if (MODE == kProjBlock) {
          const float r0 = (float)yb.x;
          const float r1 = (float)yb.y;
          float p[kHeads];
#pragma unroll
          for (int h = 0; h < kHeads; ++h) p[h] = wave_sum(r0 * wb[h][0] + r1 * wb[h][1]);
          if (lane < kHeads) {
            const float v = lane == 0 ? p[0] : lane == 1 ? p[1] : lane == 2 ? p[2] : p[3];
            a.tri_bias[bias_frag_index_bf16(lane, i, j, a.np)] = (__bf16)(valid ? v * kLog2e : 0.f);
          }
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < kLoads; ++t) {
        const int idx = tid + t * kThreads;
        if (idx < kVecs) *(bf16x8*)&xs[buf][idx >> 4][(idx & 15) * 8] = stage_vec[t];
      }
    }
  };

  auto mfma_tile = [&](int buf) -> f32x16 {
    f32x16 acc = {};
#pragma unroll
    for (int m = 0; m < 8; ++m)
      acc = mfma_bf16(*(const bf16x8*)&xs[buf][l32][16 * m + 8 * half], wf[m], acc);
    return acc;
  };

  // Stores rows r and r + 1 (r even) of a column-per-lane tile as 32-bit
  // words: lane pairs (l32, l32 ^ 1) exchange their bf16 pairs, so the even
  // lane stores columns l32, l32 + 1 of row r and the odd lane columns
  // l32 - 1, l32 of row r + 1.  dst addresses (row 0, column l32) of the
  // tile in a row-major bf16 array with `stride` elements per row.
  auto store_pairs = [&](__bf16* dst, int64_t stride, const f32x16& v) {
    const bool odd = l32 & 1;
    const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
    __bf16* base = dst + (odd ? stride - 1 : 0);
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const bf16x2 w2 = {(__bf16)v[r], (__bf16)v[r + 1]};
      const uint32_t mine = __builtin_bit_cast(uint32_t, w2);
      const uint32_t other = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mine, 0xB1, 0xF, 0xF, false);
      *(uint32_t*)(base + (int64_t)(8 * (r >> 2) + (r & 3)) * stride) =
          __builtin_amdgcn_perm(other, mine, sel);
    }
  };

  // Lane holds rows 4*half + 8*(r/4) + r%4 of the tile, column col_w.
  auto epilogue = [&](int tile, const f32x16& acc) {
    const int i = tile / tiles_j;
    const int j0 = (tile % tiles_j) * kRows + 4 * half;
    const int group = w >> 2;
    const int hw = w & 3;
    if (MODE == kProjBlock) {
      const int64_t bh = (int64_t)i * kHeads + hw;
      if (group == 0 || group == 1) {
        __bf16* dst = (group == 0 ? a.qh : a.kh) + (bh * a.np + j0) * kHeadDim + l32;
        const float scale = group == 0 ? a.q_scale : 1.0f;
        f32x16 v;
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = acc[r] * scale;
        store_pairs(dst, kHeadDim, v);
      } else if (group == 2) {
        // V^T tile-major, [np / 32 key tiles][32 channels][32 key positions]
        // per (i, head), so a tile's 2 KB are contiguous and its stores fill
        // whole cache lines.  Keys of a tile in the S^T accumulator's
        // register order (within each 16-key block: keys 0-3, 8-11, 4-7,
        // 12-15): this lane's 4-key group g = 2 rr + half (keys 4 g + e) goes
        // to position pos + e.
        __bf16* dst = a.vt + bh * a.np * kHeadDim + (int64_t)(tile % tiles_j) * (kRows * kHeadDim) +
                      l32 * kRows;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int g = 2 * rr + half;
          const int pos = (g >> 2) * 16 + ((g & 1) * 2 + ((g >> 1) & 1)) * 4;
          *(bf16x4*)(dst + pos) = bf16x4{(__bf16)acc[4 * rr + 0], (__bf16)acc[4 * rr + 1],
                                         (__bf16)acc[4 * rr + 2], (__bf16)acc[4 * rr + 3]};
        }
      } else {
        // gate rows are padded to np: the tile is always stored whole
        __bf16* dst = a.gs + ((int64_t)i * a.np + j0) * kHidden + col_w;
        f32x16 v;
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = sigmoidf_(acc[r] + col_bias);
        store_pairs(dst, kHidden, v);
      }
    } else {
      const bool full = (tile % tiles_j + 1) * kRows <= a.rows_j;
      __bf16* dst = a.out + (int64_t)i * a.os_i + (int64_t)j0 * a.os_j + col_w;
      // The residual update adds the bf16 update to the old value, rounding
      // where the native bf16 z += dz rounds.
      const bool residual = a.accumulate != 0;
      auto put = [&](__bf16* d, float v) {
        const __bf16 u = (__bf16)v;
        *d = residual ? (__bf16)((float)*d + (float)u) : u;
      };
      if (full) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          put(dst + (int64_t)(8 * (r >> 2) + (r & 3)) * a.os_j, acc[r] + col_bias);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dj = 8 * (r >> 2) + (r & 3);
          if (j0 + dj < a.rows_j) put(dst + (int64_t)dj * a.os_j, acc[r] + col_bias);
        }
      }
    }
  };

  // The weight fragment and bias must have landed before the loop: the
  // loop's waits then track only the row fetches and the output stores.
  __builtin_amdgcn_s_waitcnt(0);
  int tile = blockIdx.x;  // grid <= ntiles, so every work-group has a tile
  fetch(tile);
  stage_rows(tile, 0);
  int next = tile + (int)gridDim.x;
  if (next < ntiles) fetch(next);
  __syncthreads();
  // A tile's results are stored one iteration late, right after the next
  // tile's rows are staged: loads and stores share one counter, and the
  // wait for the staged rows' loads then finds the stores a full iteration
  // old instead of waiting for their completion.
  f32x16 acc_prev = {};
  int prev_tile = -1;
  for (int buf = 0; tile < ntiles; buf ^= 1) {
    const f32x16 acc = mfma_tile(buf);
    if (next < ntiles) stage_rows(next, buf ^ 1);
    if (prev_tile >= 0) epilogue(prev_tile, acc_prev);
    if (next < ntiles && next + (int)gridDim.x < ntiles) fetch(next + gridDim.x);
    acc_prev = acc;
    prev_tile = tile;
    __syncthreads();
    tile = next;
    next += gridDim.x;
  }
  if (prev_tile >= 0) epilogue(prev_tile, acc_prev);
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
//
// Same work-group shape, order and pipeline as the FP32-accurate split kernel
// (attention_split.hip): (outer row b, head h, 128 queries), four waves of 32
// queries, 32-key tiles, K staged one tile ahead of V^T in LDS (both
// double-buffered), the S^T MFMAs of tile t + 1 issued before the softmax of
// tile t, one barrier per tile.  Per tile a wave issues 4 MFMAs (S^T and O^T,
// two K-halves each) and about 60 VALU instructions.
//   - The triangle bias enters as the start value of the S^T accumulator:
//     its bf16 copy is held in the accumulator's lane and register order
//     (bias_frag_index_bf16), loaded two tiles ahead with two 1 KB reads and
//     widened to FP32 with one shift or mask per value (an FP32 copy doubles
//     the bytes per tile, and the kernel then waits on its loads).
//   - q and the bias copy are stored scaled by log2(e), so the logits leave
//     the matrix cores in log2 units.
//   - Rows with an unmasked key: p = exp2(x - c) with the FP32 kernels'
//     snapped reference c (0 while the row max lies within kSnap of it;
//     rescaled only when a running sum passes kSumLimit), so a tile needs no
//     max, no cross-lane exchange and no branch, and while every reference
//     of the wave is 0 no subtraction either: p = exp2(x).  The mask bias is
//     added (times log2(e)) on masked tiles only.  P is packed to bf16 with
//     v_cvt_pk_bf16_f32; the row sum l adds the FP32 weights (their bf16
//     roundings are unbiased, so O / l stays a weighted mean well within the
//     bf16 bar).
//   - Rows whose keys are all masked form fl(fl(s + mask_bias) + bias) in
//     FP32 in that order (log2 units), with a lazy running max (rescale when
//     a tile max exceeds it by 2^8) and the max itself as the reference, so
//     equal quantised logits get equal weights.

constexpr int kThreads = 256;
constexpr int kMaxKeysB = kTileFlagWords * 32 * kBk;
// LDS ring: stage s holds key tile t (t % kStagesB == s) as the K tile [32
// keys][32 channels] and the V^T tile [32 channels][32 key positions], 2 KB
// each, 16-byte chunks swizzled (swz); tile t is copied in two tiles ahead
// of its S^T.  The projection stores V^T with a tile's keys already in the
// order in which the S^T accumulator registers hold them (within each
// 16-key block, keys 0-3, 8-11, 4-7, 12-15).
constexpr int kStagesB = 4;
constexpr int kTileBytesB = 2048;
constexpr int kStageBytesB = 2 * kTileBytesB;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_b(const __bf16* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ bf16x4 buffer_b64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

__device__ __forceinline__ bf16x8 pack8(const f32x16& p, int m) {
  typedef float f32x8 __attribute__((ext_vector_type(8)));
  const f32x8 v = {p[8 * m + 0], p[8 * m + 1], p[8 * m + 2], p[8 * m + 3],
                   p[8 * m + 4], p[8 * m + 5], p[8 * m + 6], p[8 * m + 7]};
  return __builtin_convertvector(v, bf16x8);  // v_cvt_pk_bf16_f32, round to nearest even
}

__global__ __launch_bounds__(kThreads, 3) void attention_bf16_kernel(Bf16AttnArgs a, int nqt,
                                                                     int nkt, uint32_t total,
                                                                     int ppg) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kStagesB * kStageBytesB];
  __shared__ __attribute__((aligned(16))) float Ms[kMaxKeysB];

  int b, h, qt;
  attn_item(blockIdx.x, total, a.batch, nqt, ppg, b, h, qt);
  if (b >= a.batch) return;  // padding of the last row group; uniform per work-group
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int j0 = qt * kBq;
  const int jq = j0 + 32 * w + l32;
  const int qt32 = (j0 >> 5) + w;
  const int last = nkt - 1;

  // Per-work-group buffer descriptors: K [np][32], V^T [np / 32][32][32] of (b, h);
  // the wave's bias fragments (h, qt32, all key tiles), 2 KB each.
  const int64_t bh = (int64_t)b * kHeads + h;
  const int64_t slice = (int64_t)a.np * kHeadDim;
  const int64_t nt = a.np >> 5;
  const __amdgpu_buffer_rsrc_t rb = buffer_b(a.bias + ((int64_t)h * nt + qt32) * nt * 1024, nt * 2048);
  const uint32_t ob = (uint32_t)lane * 16;
  // Tile copies: wave w fills rows 16 (w % 2) .. + 15 of the K tile (w < 2)
  // or of the V^T tile; lane l writes chunk l % 4 of row l / 4 of them, read
  // from that row's chunk (l % 4) ^ swz(row) (swz(r + 16) == swz(r)).
  const int crow = 16 * (w & 1) + (lane >> 2);
  const int cchunk = (lane & 3) ^ swz(lane >> 2);
  // K rows and V^T tiles are both 2 KB blocks per 32-key tile, rows of 64 bytes.
  // The copy source is a wave-uniform base (scalar registers) plus a lane
  // offset; the tile loop's stage indices are constants (four tiles per
  // iteration), so ring addresses fold into instruction offsets.
  const __bf16* cbase = (w < 2 ? a.k : a.v) + bh * slice + 16 * (w & 1) * kHeadDim;
  const uint32_t cvoff = (uint32_t)(((crow - 16 * (w & 1)) * kHeadDim + 8 * cchunk) * 2);
  const uint32_t clds = lds_address(ring) + (uint32_t)((w >> 1) * kTileBytesB + (w & 1) * 1024);
  const int64_t ctile = kBk * kHeadDim;  // elements from tile t to t + 1
  auto dma = [&](int t, int stage) {
    lds_dma16_s(cvoff, cbase + t * ctile, clds + stage * kStageBytesB);
  };
  // Operand reads: lane (l32, half) reads chunks half and 2 + half of row l32.
  const uint32_t rd0 = l32 * 64 + 16 * (half ^ swz(l32));
  const uint32_t rd1 = l32 * 64 + 16 * ((2 + half) ^ swz(l32));
  auto tile_rd = [&](int stage, int which, int m) -> bf16x8 {
    return *(const bf16x8*)(ring + stage * kStageBytesB + which * kTileBytesB + (m ? rd1 : rd0));
  };
  // Registers 0-7 and 8-15 of the lane's bias fragment as packed bf16 pairs.
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  struct BiasWords {
    u32x4 lo, hi;
  };
  auto load_frag = [&](int t) -> BiasWords {
    const uint32_t so = (uint32_t)t * 2048;
    return BiasWords{__builtin_amdgcn_raw_buffer_load_b128(rb, ob, so, 0),
                     __builtin_amdgcn_raw_buffer_load_b128(rb, ob + 1024, so, 0)};
  };
  auto widen = [](const BiasWords& bw) -> f32x16 {
    f32x16 x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __builtin_bit_cast(float, bw.lo[i] << 16);
      x[2 * i + 1] = __builtin_bit_cast(float, bw.lo[i] & 0xffff0000u);
      x[8 + 2 * i] = __builtin_bit_cast(float, bw.hi[i] << 16);
      x[8 + 2 * i + 1] = __builtin_bit_cast(float, bw.hi[i] & 0xffff0000u);
    }
    return x;
  };

  // Row classification, as in the FP32 kernels.
  uint32_t mw[kTileFlagWords];
  uint32_t any = 0u, open = 0u;
  {
    const uint32_t* f = a.tile_flags + (int64_t)b * kTileFlagParts * kTileFlagWords;
#pragma unroll
    for (int i = 0; i < kTileFlagWords; ++i) {
      const int lo = 32 * i;
      const uint32_t valid = nkt >= lo + 32 ? 0xffffffffu : nkt > lo ? (1u << (nkt - lo)) - 1u : 0u;
      mw[i] = f[i];
      any |= mw[i] & valid;
      open |= ~f[kTileFlagWords + i] & valid;
    }
  }
  const bool has_unmasked = open != 0u;
  auto masked = [&](int t) -> bool {
    const uint32_t word = t < 32 ? mw[0] : t < 64 ? mw[1] : t < 96 ? mw[2] : mw[3];
    return (word >> (t & 31)) & 1u;
  };
  if (any != 0u) {
    const float* src = a.mbias + (int64_t)b * a.np;
    for (int k = 4 * tid; k < nkt * kBk; k += 4 * kThreads) *(f32x4*)&Ms[k] = *(const f32x4*)(src + k);
  }
  auto mask_vals = [&](int t) -> f32x16 {
    const float* m = &Ms[t * kBk + 4 * half];
    return cat4(*(const f32x4*)(m), *(const f32x4*)(m + 8), *(const f32x4*)(m + 16),
                *(const f32x4*)(m + 24));
  };

  // Q, the B operand of S^T: lane holds Q[jq][16m + 8half + e].
  bf16x8 qf[2];
  {
    const __bf16* src = a.q + (bh * a.np + jq) * kHeadDim + 8 * half;
    qf[0] = *(const bf16x8*)(src);
    qf[1] = *(const bf16x8*)(src + 16);
  }

  f32x16 o = {};
  float l_run = 0.f;

  auto run = [&](auto exact_tag) {
    constexpr bool kExact = decltype(exact_tag)::value;
    const f32x16 zero16 = {};
    // S^T of the tile in Ks[buf] added to x (the bias on the fast path).
    auto scores = [&](int buf, f32x16 x) -> f32x16 {
      const bf16x8 k0 = tile_rd(buf, 0, 0);
      const bf16x8 k1 = tile_rd(buf, 0, 1);
      x = mfma_bf16(k0, qf[0], x);
      return mfma_bf16(k1, qf[1], x);
    };
    // The rest of the logits of tile t (log2 units: q and the bias copy
    // carry log2(e)): the mask bias on masked tiles (fast), or
    // fl(fl(s + mask) + bias) (exact).
    auto finish = [&](f32x16& x, int t) {
      if (kExact) {
        const f32x16 mb = mask_vals(t);
        const f32x16 bias = widen(load_frag(t));
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = __builtin_fmaf(mb[r], kLog2e, x[r]) + bias[r];
      } else if (masked(t)) {
        const f32x16 mb = mask_vals(t);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = __builtin_fmaf(mb[r], kLog2e, x[r]);
      }
    };

    // Reference state of this lane's query (log2 units; see attention.hip).
    float m_ref = -INFINITY;
    float m_thr = -INFINITY;
    float c_ref = 0.f;
    bool has_ref = false;
    bool zero_ref = true;  // every query of the wave has c_ref == 0 (uniform)

    auto softmax = [&](const f32x16& x, bf16x8& p0, bf16x8& p1) {
      f32x16 p;
      if (kExact) {
        const float mt = xor32_max(max16(x));
        if (__any(mt > m_thr)) {
          const float m_new = __builtin_elementwise_maximum(m_ref, mt);
          const float c_new = m_new == -INFINITY ? 0.f : m_new;
          const float alpha = m_ref == -INFINITY ? 0.f : exp2_fast(c_ref - c_new);
#pragma unroll
          for (int r = 0; r < 16; ++r) o[r] *= alpha;
          l_run *= alpha;
          m_ref = m_new;
          c_ref = c_new;
          m_thr = m_new + kRescaleLog2;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r] - c_ref);
        l_run += sum16(p);
        p0 = pack8(p, 0);
        p1 = pack8(p, 1);
        return;
      }
      float ovf = 0.f;
      if (has_ref) {
        if (zero_ref) {
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r]);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r] - c_ref);
        }
        const float l_new = l_run + sum16(p);
        const bool over = !(l_new <= kSumLimit);  // NaN or inf count as overflow
        if (!__any(over)) {
          l_run = l_new;
          p0 = pack8(p, 0);
          p1 = pack8(p, 1);
          return;
        }
        ovf = over ? 1.f : 0.f;
      }
      // Rare path, taken by the whole wavefront (attention.hip), in log2 units.
      const float mt = xor32_max(max16(x));
      const bool fresh = m_ref == -INFINITY;
      const bool need = fresh || xor32_max(ovf) > 0.f || mt > c_ref + kSnap;
      m_ref = __builtin_elementwise_maximum(m_ref, mt);
      const float snapped =
          (m_ref == -INFINITY || (m_ref >= -kSnap && m_ref <= kSnap)) ? 0.f : m_ref;
      const float c_new = fresh ? snapped
                          : need ? __builtin_elementwise_maximum(snapped, c_ref + kLift)
                                 : c_ref;
      const float alpha = fresh ? 0.f : exp2_fast(c_ref - c_new);  // 1 when unchanged
#pragma unroll
      for (int r = 0; r < 16; ++r) o[r] *= alpha;
      l_run *= alpha;
      c_ref = c_new;
      zero_ref = __all(c_ref == 0.f);
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r] - c_ref);
      l_run += sum16(p);
      has_ref = __all(m_ref != -INFINITY);
      p0 = pack8(p, 0);
      p1 = pack8(p, 1);
    };

    // O^T += V^T P^T for the tile in Vs[buf]; P comes straight from the
    // S^T register order, which V^T's key positions follow.
    auto pv = [&](int buf, const bf16x8& p0, const bf16x8& p1) {
      const bf16x8 v0 = tile_rd(buf, 1, 0);
      const bf16x8 v1 = tile_rd(buf, 1, 1);
      o = mfma_bf16(v0, p0, o);
      o = mfma_bf16(v1, p1, o);
    };

    // Prologue: tiles 0-2 on their way into stages 0-2; S^T(0) once tiles 0
    // and 1 have landed.  The fast path's bias words of tile t are loaded at
    // iteration t - 3 (two slots alternate) and widened when S^T(t) starts.
    auto clamp = [&](int t) { return t < last ? t : last; };
    auto stage = [](int t) { return t & (kStagesB - 1); };
    BiasWords bw_e{}, bw_o{};
    if (!kExact) {
      bw_e = load_frag(0);
      bw_o = load_frag(clamp(1));
    }
    dma(0, 0);
    dma(clamp(1), 1);
    dma(clamp(2), 2);
    wait_vmcnt<1>();
    __syncthreads();
    f32x16 x_a = scores(0, kExact ? zero16 : widen(bw_e));
    if (!kExact) bw_e = load_frag(clamp(2));
    finish(x_a, 0);
    f32x16 x_b;

    // Iteration kt reads K(kt+1) and V(kt) and copies tile kt+3 into the
    // stage that held tile kt-1, which every wave left behind at the previous
    // barrier; cur = logits of tile kt; bw = bias words of tile kt+1,
    // refilled with tile kt+3.  Tiles past the last are clamped (in range,
    // never used).
    // Tile kt in ring stage s (s == kt % 4).
    auto body4 = [&](int kt, int s, f32x16& cur, f32x16& nxt, BiasWords& bw) {
      nxt = scores((s + 1) & 3, kExact ? zero16 : widen(bw));
      if (!kExact) bw = load_frag(clamp(kt + 3));
      bf16x8 p0, p1;
      softmax(cur, p0, p1);
      pv(s, p0, p1);
      finish(nxt, kt + 1);
      dma(clamp(kt + 3), (s + 3) & 3);
      // Tile kt+2 has landed once at most this iteration's copy and (fast
      // path) its two bias-word loads are outstanding: vector memory loads
      // retire in issue order.  When no later iteration reads the bias words
      // of tile kt+3, the compiler may drop their loads: then only the copy
      // counts.
      if (kExact || kt + 3 > last)
        wait_vmcnt<1>();
      else
        wait_vmcnt<3>();
      __syncthreads();
    };
    auto body = [&](int kt, f32x16& cur, f32x16& nxt, BiasWords& bw) {
      body4(kt, stage(kt), cur, nxt, bw);
    };
    auto tail = [&](const f32x16& cur, int kt) {
      bf16x8 p0, p1;
      softmax(cur, p0, p1);
      pv(stage(kt), p0, p1);
    };
    int kt = 0;
    // four tiles per iteration: kt % 4 == 0, so every stage is a constant
    for (; kt + 4 < nkt; kt += 4) {
      body4(kt, 0, x_a, x_b, bw_o);
      body4(kt + 1, 1, x_b, x_a, bw_e);
      body4(kt + 2, 2, x_a, x_b, bw_o);
      body4(kt + 3, 3, x_b, x_a, bw_e);
    }
    for (; kt + 2 < nkt; kt += 2) {
      body(kt, x_a, x_b, bw_o);
      body(kt + 1, x_b, x_a, bw_e);
    }
    if (kt + 1 < nkt) {
      body(kt, x_a, x_b, bw_o);
      tail(x_b, kt + 1);
    } else {
      tail(x_a, kt);
    }
    wait_vmcnt<0>();  // the clamped tail copies land before the LDS is released
  };
  if (has_unmasked) {
    run(std::false_type{});
  } else {
    run(std::true_type{});
  }

  const float l_tot = xor32_sum(l_run);
  if (jq < a.n) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int c = 8 * rr + 4 * half;
      const int64_t col = h * kHeadDim + c;
      const bf16x4 g = *(const bf16x4*)(a.gate + ((int64_t)b * a.np + jq) * kHidden + col);
      // head-major gated output [4][batch][n][32]: a work-group's 128 queries
      // of one head are 8 KB contiguous, so its stores fill whole cache lines
      *(bf16x4*)(a.out + (((int64_t)h * a.batch + b) * a.n + jq) * kHeadDim + c) = bf16x4{(__bf16)(o[4 * rr + 0] / l_tot * (float)g.x),
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
  const int nkt = (int)(round_up(a.n, kBk) / kBk);  // tiles wholly past n are not visited
  if (a.tile_flags == nullptr || nkt > kTileFlagWords * 32) return hipErrorInvalidValue;
  const uint64_t groups = ((uint64_t)a.batch + kRowGroup - 1) / kRowGroup;
  const uint64_t total = groups * kRowGroup * kHeads * nqt;
  if (total == 0) return hipSuccess;
  if (total > 0x7fffffffull) return hipErrorInvalidValue;
  const int ppg = pair_group_size(nqt, (uint64_t)kBq * (uint64_t)a.np * sizeof(__bf16));
  hipLaunchKernelGGL(attention_bf16_kernel, dim3((uint32_t)total), dim3(kThreads), 0, stream, a, nqt,
                     nkt, (uint32_t)total, ppg);
  return hipGetLastError();
}

}  // namespace fpx
