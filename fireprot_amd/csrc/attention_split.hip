// FP32-accurate triangle attention on the CDNA4 16-bit matrix cores.
//
// Every FP32 operand of the two products is held as power-of-two scaled fp16
// (hi, lo) planes: x 2^e = hi + lo with hi = fp16(x 2^e), lo = fp16(x 2^e -
// hi), 22 significant bits, e chosen per block of values (a head, from a
// bound on its values, or a 32 x 32 tile) so the block's max |value| 2^e stays
// below 2^15.  A product then takes three terms (hi hi, hi lo,
// lo hi) on v_mfma_f32_32x32x16_f16 with FP32 accumulation, an error per
// product of about 2^-22, at the level of an FP32 dot product.  That
// instruction does 8x the work of v_mfma_f32_32x32x2_f32 in half its cycles,
// and unlike the FP32 one it runs beside VALU work, so the softmax of one
// tile overlaps the matrix work of the next.
//
//   S^T = K Q^T: q and k arrive as scaled planes, one scale per head (the
//     block's prepare projection) or per 32 x 32 tile (stage_planes_kernel);
//     the logit is fma(acc, log2(e) 2^-(e_q + e_k), bias log2(e)) (exact
//     scaling, one rounding).  6 MFMAs per 32-key tile.
//   O^T += V^T P^T: v^T arrives as planes scaled per key tile t (2^e_t; the
//     block's one scale per head), its keys in the S^T accumulator's
//     register order; the weights P of tile t are split per tile into fp16
//     planes as P 2^(kVShift - (e_t - e_min)) (at most 2^15), so every
//     product carries the same 2^(e_min + kVShift), removed in the epilogue.
//     6 MFMAs per tile.
//
// Each key tile's four 2 KB planes (K hi, K lo, V^T hi, V^T lo) go straight
// from global memory into a ring of LDS stages (global_load_lds_dwordx4, no
// registers), two tiles ahead of use, with 16-byte chunks swizzled so the
// operand reads are free of bank conflicts.
//
// Softmax, two paths, each its own launch over the same grid (a work-group
// of the other path exits at once), so each gets its own register budget:
//   fast (rows with an unmasked key whose logits the magnitude record and
//     the row's largest mask bias bound below kFastBound): log2-domain
//     logits fma(acc, scale, bias log2(e)); an integer reference c per
//     query, moved up to the tile's max when a lane's weights of a tile
//     would pass 2^15;
//     P' = exp2(x - (c + g_t)) with the tile's exponent shift g_t folded into
//     the exact integer c + g_t.  The block's bias copy is stored relative
//     to each query's reference (bias_reference_kernel): the reference then
//     starts at 0, and while it and g_t stay 0 the weights are exp2(x);
//   exact (fully masked rows, and rows whose logits are not bounded):
//     fl(fl(s + mask) + bias) in natural units, as the native path rounds
//     them, with a lazy max and one rounded reference, so equal quantised
//     logits get equal weights (the -1e9 of a padding row has an FP32
//     spacing of 64).
// K is staged one tile ahead of V, and the S^T MFMAs of tile t + 1 are issued
// before the softmax of tile t.
//
// Rows whose keys all carry one mask bias m, small enough products given
// (constant_mask_row), have the same weights fl-softmax(m + bias) on every
// such row: attention_const_kernel runs only O^T for them, four rows per
// work item.  For the block, const_weights_kernel first forms those weights
// once for the m of the first such row, and lists the four-row chunks of
// that m and of any other m; the constant-mask launches walk those lists.
#include "attn_common.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "split.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace fpx {
namespace {

constexpr int kThreads = 256;

// Block layout ring: stage s holds one key tile as four 2 KB planes (K hi,
// K lo, V^T hi, V^T lo), each 32 rows of 64 bytes.  Tile t sits in stage
// t % kStages and is loaded two iterations before its S^T.
constexpr int kStages = 4;
constexpr int kPlaneBytes = 2048;
constexpr int kStageBytes = 4 * kPlaneBytes;
// Weights enter P.V as fp16 planes scaled by 2^(kVShift - d_t) (at most
// 2^15), d_t = e_t - e_min >= 0 the v^T tile's exponent above the row's
// smallest; kPlaneMax bounds a lane's 16 scaled weights of one tile.
constexpr int kVShift = 7;
// Relative bias: the largest product bound (log2 units) for which the
// reference may start at 0 (see attend_item).
constexpr float kRelBound = 4.0f;
constexpr float kPlaneMax = 32768.0f;
// Four waves per SIMD: four work-groups per CU (ring and mask row within
// 40 KB of LDS at N <= 1536).


typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// V^T keys are stored in the order in which the S^T accumulator registers
// hold them: within each 16-key block, keys 0-3, 8-11, 4-7, 12-15.  Position
// of the 4-key group g (keys 4g..4g+3) of a tile:
__device__ __forceinline__ int v_position(int g) {
  const int perm = (g & 1) * 2 + ((g >> 1) & 1);  // 0, 2, 1, 3
  return (g >> 2) * 16 + perm * 4;
}

// Rows whose mask bias is one finite nonzero value m on every key < n
// (padding rows: inf (mask - 1) = -1e9), when the products are bounded below
// half the float32 spacing next to m on either side: then fl(s + m) = m for
// every key (|s| <= 32 max|q| max|k|, with a margin for the native rounding
// of s), so the native logit fl(fl(s + m) + bias) is fl(m + bias), the same
// for every such row.  With |m| = f 2^e, f in [0.5, 1), the spacing above
// |m| is 2^(e - 24); toward zero it is the same unless |m| is a power of two
// (f = 0.5), where it halves.
__device__ __forceinline__ bool constant_mask_row(const AttnArgs& a, int b, float& m) {
  if (a.magnitudes == nullptr || a.magnitudes[4] != 1u) return false;
  const uint32_t* f3 =
      a.tile_flags + ((int64_t)b * kTileFlagParts + kTileFlagMaxPart) * kTileFlagWords;
  const float hi = __builtin_bit_cast(float, f3[0]);
  const float lo = __builtin_bit_cast(float, f3[1]);
  // false for NaN anywhere, for an infinite m and for m = 0
  if (!(hi == lo && __builtin_fabsf(hi) < INFINITY && hi != 0.f)) return false;
  const float mq = __builtin_bit_cast(float, a.magnitudes[0]);
  const float mk = __builtin_bit_cast(float, a.magnitudes[1]);
  const float s_bound = 32.0f * mq * mk * (1.0f + 0x1p-10f);
  const bool power_of_two = (__builtin_bit_cast(uint32_t, hi) & 0x7fffffu) == 0u;
  const float half_ulp =
      __builtin_ldexpf(1.0f, __builtin_amdgcn_frexp_expf(hi) - (power_of_two ? 26 : 25));
  m = hi;
  return s_bound < half_ulp;
}

// The constant-row kernel serves chunks of kConstRows consecutive outer
// rows: the rows of a chunk that satisfy constant_mask_row with the m of
// the chunk's first such row.  The exact launch leaves exactly those out.
__device__ __forceinline__ bool const_chunk_member(const AttnArgs& a, int b) {
  float m;
  if (!constant_mask_row(a, b, m)) return false;
  for (int r = b - b % kConstRows; r < b; ++r) {
    float mr;
    if (constant_mask_row(a, r, mr)) return mr == m;
  }
  return true;  // the chunk's first constant-mask row
}

// LDS of the attention work-group: the ring of key tiles, the per-tile
// scales, and the mask-bias row (dynamic, after the static arrays).
struct AttnLds {
  uint8_t* ring;  // kStages x kStageBytes
  float* Ms;      // mask-bias row of this outer row, nkt_all * kBk floats
  float* Sk;      // 2^-e_k of each key tile
  int* Ev;        // e_v of each key tile's v^T planes
  float* Wv;      // per wave: max 2^-e_v over its tiles
};

// Row classification from the tile flags and the magnitude record: returns
// whether row b takes the fast softmax path, with the key tiles it visits
// (nkt), the tile words of part 0 (mw: a tile holds a nonzero mask bias) and
// whether any visited tile does (any).
// On rows with an unmasked key, the trailing tiles whose every mask bias is
// <= -kSkipMask carry weights that are exactly 0 when the prepare
// projection's magnitude record bounds the logits (kernels.hpp), so they are
// left out; the result is bit-identical.  The fast softmax needs the same
// record to bound the logits below kFastBound, together with the row's
// largest mask bias when that is positive (its integer reference then stays
// exact when shifted by a tile's plane exponent); other rows take the exact
// path.
__device__ __forceinline__ bool row_is_fast(const AttnArgs& a, int b, int nkt_all, int& nkt,
                                            uint32_t (&mw)[kTileFlagWords], uint32_t& any) {
  uint32_t open = 0u;
  any = 0u;
  {
    const uint32_t* f = a.tile_flags + (int64_t)b * kTileFlagParts * kTileFlagWords;
#pragma unroll
    for (int i = 0; i < kTileFlagWords; ++i) {
      const int lo = 32 * i;
      const uint32_t valid =
          nkt_all >= lo + 32 ? 0xffffffffu : nkt_all > lo ? (1u << (nkt_all - lo)) - 1u : 0u;
      mw[i] = f[i];
      any |= mw[i] & valid;
      open |= ~f[kTileFlagWords + i] & valid;
    }
  }
  const bool has_unmasked = open != 0u;
  nkt = nkt_all;
  bool fast = false;
  if (has_unmasked && a.magnitudes != nullptr && a.magnitudes[4] == 1u) {
    const float mq = __builtin_bit_cast(float, a.magnitudes[0]);
    const float mk = __builtin_bit_cast(float, a.magnitudes[1]);
    const float mv = __builtin_bit_cast(float, a.magnitudes[2]);
    const float mb = __builtin_bit_cast(float, a.magnitudes[3]);
    const float mm = __builtin_bit_cast(
        float, a.tile_flags[((int64_t)b * kTileFlagParts + kTileFlagMaxPart) * kTileFlagWords]);
    const float bound = 32.0f * mq * mk + mb;
    const float lift = mm > 0.0f ? mm : 0.0f;
    // false for NaN anywhere (the comparison with mm rejects a NaN mask bias)
    fast = bound + lift < kFastBound && (mm <= 0.0f || mm < kFastBound) && mv < INFINITY;
    if (bound < kSkipBound && mv < INFINITY) {  // false for NaN
      const uint32_t* far =
          a.tile_flags + (int64_t)b * kTileFlagParts * kTileFlagWords + 2 * kTileFlagWords;
      while (nkt > 1) {
        const int t = nkt - 1;
        if (!((far[t >> 5] >> (t & 31)) & 1u)) break;
        nkt = t;
      }
    }
  }
  return fast;
}

// Rows served by the exact launch: neither fast nor taken by the
// constant-row kernel.
__device__ __forceinline__ bool row_is_exact(const AttnArgs& a, int b, int nkt_all) {
  int nkt;
  uint32_t mw[kTileFlagWords], any;
  return !row_is_fast(a, b, nkt_all, nkt, mw, any) && !const_chunk_member(a, b);
}

// Both layouts read q, k and v^T in the plane layout (ProjArgs::planes) with
// their per-tile scales, and the staged bias copies, mask rows and tile
// flags.  LAYOUT kAttnBlock: the block's workspace, gated head-last output;
// kAttnStaged: planes staged from a caller's strided q, k, v
// (launch_stage_planes), output through the caller's strides, no gate.
// One work item (b, h, qt) of the split attention.  Uniform per work-group;
// returns at once (before any LDS access) when the row belongs to the other
// softmax path or to the constant-row kernel.
template <int LAYOUT, bool EXACT>
__device__ __forceinline__ void attend_item(const AttnArgs& a, int nqt, int nkt_all, int b, int h,
                                            int qt, const AttnLds& L) {
  constexpr bool kBlock = LAYOUT == kAttnBlock;
  static_assert(LAYOUT == kAttnBlock || LAYOUT == kAttnStaged, "plane layouts only");
  uint8_t* const lds = L.ring;
  float* const Ms = L.Ms;
  float* const Sk = L.Sk;
  int* const Ev = L.Ev;
  float* const Wv = L.Wv;
  if (b >= a.batch) return;  // padding of the last row group; uniform per work-group
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int j0 = qt * kBq;
  const int jq = j0 + 32 * w + l32;
  const int qt32 = (j0 >> 5) + w;

  // Per-work-group buffer descriptors over the (b, h) slices and the wave's
  // bias fragments (h, qt32, all key tiles), as in the FP32 kernel.
  const int64_t bh = (int64_t)b * kHeads + h;
  const int64_t nt = a.np >> 5;
  const int64_t frag = ((int64_t)h * nt + qt32) * nt * 1024;
  const __amdgpu_buffer_rsrc_t rb = buffer(a.bias + frag, nt * 4096);
  const __amdgpu_buffer_rsrc_t rb2 = buffer(a.bias_l2 + frag, nt * 4096);
  const uint32_t ob = (uint32_t)lane * 16;

  // Per (b, h) a slice of np * 128 bytes, the hi plane and
  // then the lo plane of 16-bit values: q, k [np rows][32 channels], v^T
  // [np / 32 tiles][32 channels][32 key positions].  A tile's plane is 2 KB
  // contiguous.  Wave w fills plane w of a stage (K hi, K lo, V^T hi,
  // V^T lo): lane l writes chunk l % 4 of rows l / 4 and 16 + l / 4, read
  // from that row's chunk (l % 4) ^ swz(row).
  // The copy source is a wave-uniform base (scalar registers) plus a lane
  // offset; ring stages are compile-time indices (the tile loop is unrolled
  // over the four stages), so stage addresses fold into immediates.
  const int64_t slice_bytes = (int64_t)a.np * 128;
  const uint8_t* dma_base = reinterpret_cast<const uint8_t*>(w < 2 ? a.k : a.v) + bh * slice_bytes +
                            (w & 1) * (slice_bytes >> 1);
  const uint32_t dma_voff = (uint32_t)((lane >> 2) * 64 + 16 * ((lane & 3) ^ swz(lane >> 2)));
  const uint32_t dma_voff2 = dma_voff + 1024;
  const uint32_t dma_lds = lds_address(lds) + (uint32_t)w * kPlaneBytes;
  auto dma = [&](int t, int stage) {
    const uint8_t* src = dma_base + (int64_t)t * kPlaneBytes;
    lds_dma16_s(dma_voff, src, dma_lds + stage * kStageBytes);
    lds_dma16_s(dma_voff2, src, dma_lds + stage * kStageBytes + 1024);
  };
  // Operand reads: lane (l32, half) reads chunk 2m + half of row l32.
  const uint32_t rd0 = l32 * 64 + 16 * (half ^ swz(l32));
  const uint32_t rd1 = l32 * 64 + 16 * ((2 + half) ^ swz(l32));
  auto plane_rd = [&](int stage, int plane, int m) -> bf16x8 {
    return *(const bf16x8*)(lds + stage * kStageBytes + plane * kPlaneBytes + (m ? rd1 : rd0));
  };

  auto load_frag = [&](__amdgpu_buffer_rsrc_t r, int t) -> f32x16 {
    const uint32_t s = (uint32_t)t * 4096;
    return cat4(buffer_f4(r, ob, s), buffer_f4(r, ob + 1024, s), buffer_f4(r, ob + 2048, s),
                buffer_f4(r, ob + 3072, s));
  };
  uint32_t mw[kTileFlagWords];
  uint32_t any;
  int nkt;
  const bool fast = row_is_fast(a, b, nkt_all, nkt, mw, any);
  // Each row runs in the launch of its softmax path (uniform per work-group).
  if (fast == EXACT) return;
  // Exact rows that the constant-row kernel serves are left out; other
  // constant-mask rows (another m than their chunk's) still skip S^T here.
  if (EXACT && const_chunk_member(a, b)) return;
  // The block's fast launch reads the log2 bias relative to each query's
  // reference (launch_bias_reference): x' = x - C_q + kRelOffset.
  const bool rel = kBlock && !EXACT && a.magnitudes != nullptr &&
                   a.magnitudes[kRelativeBiasWord] == 1u;
  float m_row = 0.f;
  const bool constant_mask = EXACT && constant_mask_row(a, b, m_row);
  const int last = nkt - 1;
  const int full_tiles = a.n / kBk;  // key tiles wholly below n
  auto masked = [&](int t) -> bool {
    const uint32_t word = t < 32 ? mw[0] : t < 64 ? mw[1] : t < 96 ? mw[2] : mw[3];
    return (word >> (t & 31)) & 1u;
  };
  if (any != 0u) {
    const float* src = a.mbias + (int64_t)b * a.mb_stride;
    for (int k = 4 * tid; k < nkt * kBk; k += 4 * kThreads) *(f32x4*)&Ms[k] = *(const f32x4*)(src + k);
  }
  // The product scale 2^-(e_q + e_k) of this wave's queries and each key
  // tile, and each key tile's v^T exponent e_t with their maximum 2^-e_min
  // (read after the prologue's first barrier).  e_min runs over every key
  // tile, visited or not, so leaving out trailing tiles changes no bit.
  float sq = 1.0f;
  {
    const int64_t per = (int64_t)kHeads * nt;
    const float* sc = a.scales + (int64_t)b * per + (int64_t)h * nt;
    sq = sc[qt32];
    float vmax = 0.f;
    for (int t = tid; t < nkt_all; t += kThreads) {
      if (t < nkt) Sk[t] = sc[(int64_t)a.batch * per + t];
      const float sv = sc[2 * (int64_t)a.batch * per + t];
      Ev[t] = inv_scale_exp(sv);
      vmax = __builtin_elementwise_maximum(vmax, sv);
    }
    vmax = wave_max(vmax);
    if (lane == 0) Wv[w] = vmax;
  }
  auto mask_vals = [&](int t) -> f32x16 {
    const float* m = &Ms[t * kBk + 4 * half];
    return cat4(*(const f32x4*)(m), *(const f32x4*)(m + 8), *(const f32x4*)(m + 16),
                *(const f32x4*)(m + 24));
  };

  f32x16 o = {};
  float l_run = 0.f;
  int e_min = 0;  // smallest v^T plane exponent over the visited tiles
  // The block's prepare projection writes one plane exponent per head and
  // operand, so the product scale and the v^T tile shift are the same for
  // every key tile (set after the prologue's first barrier).
  float st_head = 1.0f;
  int g_head = 0;

  auto run = [&](auto exact_tag, auto constant_tag) {
    constexpr bool kExact = decltype(exact_tag)::value;
    // exact rows with a constant mask bias: logits fl(m_row + bias), V only
    constexpr bool kConst = decltype(constant_tag)::value;
    static_assert(kExact || !kConst, "the constant-mask shortcut serves exact rows");
    const f32x16 zero16 = {};
    // Tile copies into the ring; the constant-mask shortcut needs no K tiles
    // (waves 0 and 1 copy K hi and K lo).
    auto copy = [&](int t, int stage) {
      if (!kConst || w >= 2) dma(t, stage);
    };

    // Q planes, the B operand of S^T: lane holds Q[jq][16m + 8half + e], the
    // fp16 hi and lo planes (the log2(e) of the fast path enters with the
    // product scale).
    bf16x8 qh[2], ql[2];
    if (!kConst) {
      const uint8_t* src = reinterpret_cast<const uint8_t*>(a.q) + bh * slice_bytes + (int64_t)jq * 64;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        qh[m] = *(const bf16x8*)(src + 16 * (2 * m + half));
        ql[m] = *(const bf16x8*)(src + (slice_bytes >> 1) + 16 * (2 * m + half));
      }
    }

    // S^T of the tile in ring stage buf (scaled by 2^(e_q + e_k)); the
    // smallest terms first.
    auto scores = [&](int stage) -> f32x16 {
      f32x16 x = zero16;
      if (kConst) return x;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const bf16x8 kh = plane_rd(stage, 0, m);
        const bf16x8 kl = plane_rd(stage, 1, m);
        x = mfma_f16(kl, qh[m], x);
        x = mfma_f16(kh, ql[m], x);
        x = mfma_f16(kh, qh[m], x);
      }
      return x;
    };
    // The logits of tile t from its product acc (s = acc 2^-(e_q + e_k), an
    // exact scaling), x holding the tile's bias fragment: the bias in log2
    // units plus the mask bias on masked tiles (fast), or fl(fl(s + mask) +
    // bias) in natural units (exact).
    auto finish = [&](f32x16& x, const f32x16& acc, int t) {
      if (kConst) {
        if (t < full_tiles) {
#pragma unroll
          for (int r = 0; r < 16; ++r) x[r] = m_row + x[r];
        } else {
          // the tile holding key n - 1: -inf mask bias on the keys >= n
          const f32x16 mb = mask_vals(t);
#pragma unroll
          for (int r = 0; r < 16; ++r) x[r] = mb[r] + x[r];
        }
        return;
      }
      const float st = kBlock ? st_head : sq * Sk[t];
      if (kExact) {
        if (masked(t)) {
          const f32x16 mb = mask_vals(t);
#pragma unroll
          for (int r = 0; r < 16; ++r) x[r] = ((acc[r] * st) + mb[r]) + x[r];
        } else {
          // every mask bias of the tile is 0: fl(s + 0) = s
#pragma unroll
          for (int r = 0; r < 16; ++r) x[r] = (acc[r] * st) + x[r];
        }
        return;
      }
      {
        const float sl = st * kLog2e;
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = __builtin_fmaf(acc[r], sl, x[r]);
      }
      if (masked(t)) {
        const f32x16 mb = mask_vals(t);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = __builtin_fmaf(mb[r], kLog2e, x[r]);
      }
    };
    // A tile's bias fragment, loaded two tiles ahead of its logits: scaled
    // by log2(e) (fast) or as is (exact).
    auto init = [&](int t) -> f32x16 { return load_frag(kExact ? rb : rb2, t); };

    // Reference state of this lane's query: the weights are exp2(x - c_ref)
    // (x in log2 units on the fast path) or exp2(x log2(e) - c_ref) (natural
    // units on the exact path); m_ref is the running max (-inf: none yet).
    float m_ref = -INFINITY;
    float c_ref = 0.f;
    float w_ref = 1.f;  // exact path: 2^-(m_ref log2(e) - c_ref)
    bool has_ref = false;
    // Relative bias: the reference starts at 0 (C_q - kRelOffset in absolute
    // log2 units) when the products are bounded tightly enough.  With
    // |s_qk| <= |q|_2 |k|_2 <= |q|_2 sqrt(32) max|k| below kRelBound (log2
    // units) on every lane, a row's largest logit over the keys of the tiles
    // before T lies in [C_q - 1 - kRelBound, C_q + kRelBound]; its weight
    // P' = 2^(x' - g) then lies in [2^(kRelOffset - 1 - kRelBound),
    // 2^(kRelOffset + kRelBound)] (g = 0 with the block's one v^T exponent
    // per head), and a larger logit elsewhere moves the reference as usual.
    // ref_zero (uniform): c_ref = 0 on every lane.
    int ref_zero = 0;
    if constexpr (!kExact) {
      if (rel) {
        float s2 = 0.f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const f16x8 hv = __builtin_bit_cast(f16x8, qh[m]);
#pragma unroll
          for (int e = 0; e < 8; ++e) s2 = __builtin_fmaf((float)hv[e], (float)hv[e], s2);
        }
        // |q| <= |hi| (1 + 2^-11) per channel; the margin also covers the
        // square root and products
        const float qn = __builtin_sqrtf(xor32_sum(s2)) * sq * (1.0f + 0x1p-8f);
        const float mk = __builtin_bit_cast(float, a.magnitudes[1]);
        const float bound = qn * 5.65685425f * mk * kLog2e;
        if (__all(bound <= kRelBound)) {  // false for NaN
          has_ref = true;
          m_ref = 0.f;
          ref_zero = 1;
        }
      }
    }

    // Logits x of tile t -> the weights' fp16 hi and lo planes (P operand).
    // Tile t's v^T planes carry 2^e_t, so its weights P enter as
    // P' = P 2^-g, g = e_t - e_min - kVShift: every product then carries the
    // same 2^(e_min + kVShift), removed in the epilogue.  P <= 2^8 keeps
    // P' <= 2^15, within fp16; the largest weight of the row sits at or
    // above 2^(kVShift - 1) in the tiles of exponent e_min, far above the
    // fp16 planes' absolute resolution (2^-25).  The row sum adds the
    // unscaled P.
    auto softmax = [&](const f32x16& x, int t, bf16x8 (&ph)[2], bf16x8 (&pl)[2]) {
      // uniform; the relative bias holds the shift kVShift in kRelOffset
      const int g = kBlock ? g_head
                           : __builtin_amdgcn_readfirstlane(Ev[t]) - e_min - (rel ? 0 : kVShift);
      // The weights are formed, summed and split eight at a time (8 keys per
      // operand half m), so only half of them are live at once.
      auto sum8 = [](const f32x8& v) {
        return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
      };
      if (kExact) {
        // Lazy max: the reference moves when a tile's max exceeds the last
        // one by 8 binary orders; equal quantised logits get equal weights
        // (one rounded c_ref per reference).  c_ref = fl(m log2(e)) is off
        // by r0 = m log2(e) - c_ref (up to half its spacing: 64 at the
        // -1e9 of a padding row), so the weights p = exp2(x log2(e) - c_ref)
        // carry 2^r0: P = p w_r with w_r = 2^-r0 is at most 2^8, and the
        // sums hold P, in units of exp(x - m_ref).
        const float mt = xor32_max(max16(x));
        if (__any(mt > m_ref + kRescaleNat)) {
          const float m_new = __builtin_elementwise_maximum(m_ref, mt);
          const float c_new = m_new == -INFINITY ? 0.f : m_new * kLog2e;
          const float alpha = m_ref == -INFINITY ? 0.f : exp2_fast((m_ref - m_new) * kLog2e);
#pragma unroll
          for (int r = 0; r < 16; ++r) o[r] *= alpha;
          l_run *= alpha;
          m_ref = m_new;
          c_ref = c_new;
          w_ref = m_new == -INFINITY ? 1.f : exp2_fast(-__builtin_fmaf(m_new, kLog2e, -c_new));
        }
        const float f = w_ref * __builtin_ldexpf(1.0f, -g);  // exact: a power of two times w_ref
        float ps = 0.f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          f32x8 v;
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = exp2_fast(__builtin_fmaf(x[8 * m + e], kLog2e, -c_ref));
          ps += sum8(v);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] *= f;
          split_f16(v, ph[m], pl[m]);
        }
        l_run = __builtin_fmaf(ps, w_ref, l_run);
        return;
      }
      // Fast path: c_ref is an integer of magnitude below 2^22 once a tile
      // with an unmasked key has set it (kFastBound), so c_ref + g is exact
      // and P' = exp2(x - (c_ref + g)) costs no multiply.  A lane pair holds
      // one query's 32 keys and keeps one reference.
      const float gf = (float)g;
      f32x16 p;
      if (__builtin_amdgcn_readfirstlane(ref_zero) && g == 0) {
        // the reference and the tile's shift are 0: P' = exp2(x')
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r] - (c_ref + gf));
      }
      float ps = sum16(p);
      // ps <= 2^15 bounds every P' of the lane; NaN or inf counts as over.
      if (!has_ref || __any(!(ps <= kPlaneMax))) {
        // Rare, taken by the whole wavefront: the first tile, or a tile
        // whose weights would leave the fp16 range.  The reference moves up
        // to the tile's max rounded up to an integer, so every weight of the
        // tile is at most 1; the previous sums scale by the exact power of
        // two alpha.  A query whose logits are all -inf so far keeps no
        // reference (its weights are 0).
        const float mt = xor32_max(max16(x));
        const bool fresh = m_ref == -INFINITY;
        m_ref = __builtin_elementwise_maximum(m_ref, mt);
        const float top = __builtin_ceilf(mt);
        const float c_new = fresh ? (m_ref == -INFINITY ? 0.f : top)
                                  : __builtin_elementwise_maximum(c_ref, top);
        const float alpha = fresh ? 0.f : exp2_fast(c_ref - c_new);  // 1 when unchanged
#pragma unroll
        for (int r = 0; r < 16; ++r) o[r] *= alpha;
        l_run *= alpha;
        c_ref = c_new;
        has_ref = __all(m_ref != -INFINITY);
        ref_zero = __all(c_ref == 0.f);
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r] - (c_ref + gf));
        ps = sum16(p);
      }
      // P = P' 2^(g - kVShift) with the relative bias (P' 2^g otherwise)
      l_run = __builtin_fmaf(ps, __builtin_ldexpf(1.0f, rel ? g - kVShift : g), l_run);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const f32x8 v = {p[8 * m + 0], p[8 * m + 1], p[8 * m + 2], p[8 * m + 3],
                         p[8 * m + 4], p[8 * m + 5], p[8 * m + 6], p[8 * m + 7]};
        split_f16(v, ph[m], pl[m]);
      }
    };

    // O^T += V^T P^T for the tile in LDS buffer/stage buf.
    auto pv = [&](int stage, const bf16x8 (&ph)[2], const bf16x8 (&pl)[2]) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const bf16x8 vh = plane_rd(stage, 2, m);
        const bf16x8 vl = plane_rd(stage, 3, m);
        o = mfma_f16(vl, ph[m], o);
        o = mfma_f16(vh, pl[m], o);
        o = mfma_f16(vh, ph[m], o);
      }
    };

    auto clamp = [&](int t) { return t < last ? t : last; };
    int kt = 0;
    // Prologue: tiles 0-2 on their way into stages 0-2; S^T(0) once tiles
    // 0 and 1 have landed.  Iteration t reads K(t+1) and V(t) and starts
    // tile t+3 into the stage that held tile t-1, which every wave left
    // behind at the previous barrier.  The copy is issued after the
    // logits, whose bias-fragment loads the compiler waits for with a
    // count that also covers any later load.  Tiles past the last are
    // clamped (in range, never used).  Tile t sits in stage t % 4; the main
    // loop runs four tiles per iteration, so its stage indices are constants
    // and every ring address folds into an instruction offset.
    f32x16 x_a = init(0);
    f32x16 x_b = init(clamp(1));
    copy(0, 0);
    copy(clamp(1), 1);
    copy(clamp(2), 2);
    wait_vmcnt<2>();
    __syncthreads();
    e_min = __builtin_amdgcn_readfirstlane(
        inv_scale_exp(__builtin_elementwise_maximum(__builtin_elementwise_maximum(Wv[0], Wv[1]),
                                                    __builtin_elementwise_maximum(Wv[2], Wv[3]))));
    if constexpr (kBlock) {
      st_head = sq * Sk[0];
      g_head = __builtin_amdgcn_readfirstlane(Ev[0]) - e_min - (rel ? 0 : kVShift);
    }
    finish(x_a, scores(0), 0);
    // Tile t in ring stage s with its successor's S^T; t + 1 <= last.
    auto body = [&](int t, int s, f32x16& cur, f32x16& nxt) {
      const f32x16 acc = scores((s + 1) & 3);
      bf16x8 ph[2], pl[2];
      softmax(cur, t, ph, pl);
      cur = init(clamp(t + 2));
      pv(s, ph, pl);
      finish(nxt, acc, t + 1);
      copy(clamp(t + 3), (s + 3) & 3);
      // Tile t+2 has landed once at most this iteration's two tile loads
      // and four bias-fragment loads are outstanding: vector memory loads
      // retire in issue order.
      wait_vmcnt<6>();
      __syncthreads();
    };
    auto tail = [&](const f32x16& cur, int t) {
      bf16x8 ph[2], pl[2];
      softmax(cur, t, ph, pl);
      pv(t & 3, ph, pl);
    };
    for (; kt + 4 < nkt; kt += 4) {
      body(kt, 0, x_a, x_b);
      body(kt + 1, 1, x_b, x_a);
      body(kt + 2, 2, x_a, x_b);
      body(kt + 3, 3, x_b, x_a);
    }
    for (; kt + 2 < nkt; kt += 2) {
      body(kt, kt & 3, x_a, x_b);
      body(kt + 1, (kt + 1) & 3, x_b, x_a);
    }
    if (kt + 1 < nkt) {
      body(kt, kt & 3, x_a, x_b);
      tail(x_b, kt + 1);
    } else {
      tail(x_a, kt);
    }
    wait_vmcnt<0>();  // the clamped tail loads land before the LDS is released
  };
  if constexpr (EXACT) {
    if (constant_mask)
      run(std::true_type{}, std::true_type{});
    else
      run(std::true_type{}, std::false_type{});
  } else {
    run(std::false_type{}, std::false_type{});
  }

  const float l_tot = xor32_sum(l_run);
  if (jq < a.n) {
    // o carries 2^(e_min + kVShift) (exact powers of two)
    const int ue = -(e_min + kVShift);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int c = 8 * rr + 4 * half;  // channels c..c+3 of head h
      f32x4 ov4 = {__builtin_ldexpf(o[4 * rr + 0], ue) / l_tot,
                   __builtin_ldexpf(o[4 * rr + 1], ue) / l_tot,
                   __builtin_ldexpf(o[4 * rr + 2], ue) / l_tot,
                   __builtin_ldexpf(o[4 * rr + 3], ue) / l_tot};
      if constexpr (kBlock) {
        const int64_t col = h * kHeadDim + c;
        if (a.gate) ov4 = ov4 * *(const f32x4*)(a.gate + ((int64_t)b * a.np + jq) * kHidden + col);
        *(f32x4*)(a.out + ((int64_t)b * a.n + jq) * kHidden + col) = ov4;
      } else {
        *(f32x4*)(a.out + b * a.os[0] + h * a.os[1] + (int64_t)jq * a.os[2] + c) = ov4;
      }
    }
  }
}

// The fast launch runs one work item per work-group (total work-groups,
// attn_item order).  The exact launch is persistent: at most kExactGroups
// work-groups walk units u = blockIdx.x + k gridDim.x, unit u = pairs
// u % kExactChunks, u % kExactChunks + kExactChunks, ... of outer row
// u / kExactChunks; a row that is not exact costs one check, and an exact
// row's pairs spread over kExactChunks work-groups.  The barrier after an
// item releases the LDS for the next.  EXACT selects the softmax path the
// launch serves; the exact path holds a few more values and runs at three
// waves per SIMD.
constexpr int kExactGroups = 768;  // three work-groups of four waves per CU
constexpr int kExactChunks = 4;
template <int LAYOUT, bool EXACT>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(EXACT ? 3 : 4, EXACT ? 3 : 4)))
void attention_split_kernel(AttnArgs a, int nqt, int nkt_all, uint32_t total, int ppg) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kStages * kStageBytes];
  extern __shared__ __attribute__((aligned(16))) float Ms[];
  __shared__ float Sk[kTileFlagWords * 32];
  __shared__ int Ev[kTileFlagWords * 32];
  __shared__ float Wv[kThreads / 64];
  const AttnLds L{ring, Ms, Sk, Ev, Wv};
  if constexpr (!EXACT) {
    int b, h, qt;
    attn_item(blockIdx.x, total, a.batch, nqt, ppg, b, h, qt);
    attend_item<LAYOUT, EXACT>(a, nqt, nkt_all, b, h, qt, L);
  } else {
    const int npairs = kHeads * nqt;
    const uint32_t units = (uint32_t)a.batch * kExactChunks;
    for (uint32_t u = blockIdx.x; u < units; u += gridDim.x) {
      const int b = (int)(u / kExactChunks);
      if (!row_is_exact(a, b, nkt_all)) continue;  // uniform per work-group
      for (int pair = (int)(u % kExactChunks); pair < npairs; pair += kExactChunks) {
        attend_item<LAYOUT, EXACT>(a, nqt, nkt_all, b, pair / nqt, pair % nqt, L);
        __syncthreads();
      }
    }
  }
}

// Constant-mask rows (const_chunk_member): their logits fl(m + bias) and
// therefore their weights do not depend on the row, so a work-group forms
// the weights of its (head, 128 queries) once per key tile and applies them
// to the V of the up to kConstRows rows of its chunk.  No K tiles, no S^T;
// per row and tile 6 MFMAs (O^T += V^T P^T, three fp16 terms) and one fma
// per value.  The softmax is the exact path's (natural units, lazy max, one
// rounded reference), so equal quantised logits get equal weights.  The
// weights' planes P' = P 2^kVShift are shared by the rows; each row's v^T
// tile carries its own 2^e_t, so every tile's product starts from zero and
// is added to the row's O with the exact factor 2^-(e_t + kVShift).
// XCD x serves the (head, query tile) pairs [x H nqt / 8, (x + 1) H nqt / 8)
// of every chunk, chunk-major: a chunk's V slices meet in that XCD's L2
// across its query tiles, and every XCD holds the same share of the chunks
// that have work.
constexpr int kConstStages = 3;

// The per-row accumulators of the constant-row kernel as named members, and
// a loop over the rows with a compile-time index, so the rows' registers
// are never indexed at run time (which would move them to scratch memory).
struct ConstRowsO {
  f32x16 r0, r1, r2, r3;
};
static_assert(kConstRows == 4, "ConstRowsO holds four rows");
template <int R>
__device__ __forceinline__ f32x16& const_row(ConstRowsO& o) {
  if constexpr (R == 0) return o.r0;
  else if constexpr (R == 1) return o.r1;
  else if constexpr (R == 2) return o.r2;
  else return o.r3;
}
template <typename F>
__device__ __forceinline__ void for_const_rows(F&& f) {
  f(std::integral_constant<int, 0>{});
  f(std::integral_constant<int, 1>{});
  f(std::integral_constant<int, 2>{});
  f(std::integral_constant<int, 3>{});
}

// Stage s: V^T hi and lo planes of each chunk row, (row, plane) at
// (2 row + plane) kPlaneBytes.
constexpr int kStageBytesC = kConstRows * 2 * kPlaneBytes;
typedef float ConstScales[kTileFlagWords * 32];  // 2^-(e_t + kVShift) per tile of a row

// One work item of the constant-row kernel; uniform per work-group, returns
// at once (before any LDS access) when the item has no constant-mask rows.
// The rows of chunk `chunk` served by one item (bit r for row
// kConstRows chunk + r) and their m; uniform across the work-group.
__device__ __forceinline__ uint32_t const_chunk_rows(const AttnArgs& a, int chunk, float& m_row) {
  uint32_t live = 0u;
  m_row = 0.f;
  for (int r = 0; r < kConstRows; ++r) {
    const int b = chunk * kConstRows + r;
    float m = 0.f;
    if (b < a.batch && constant_mask_row(a, b, m) && (live == 0u || m == m_row)) {
      if (live == 0u) m_row = m;
      live |= 1u << r;
    }
  }
  return live;
}

// One work item: the chunk's constant-mask rows for (head, query tile) hq.
template <int LAYOUT, bool LOADED>
__device__ __forceinline__ void const_item(const AttnArgs& a, int nqt, int nkt, int chunk, int hq,
                                           uint8_t* ring, ConstScales* Sv) {
  constexpr bool kBlock = LAYOUT == kAttnBlock;
  static_assert(LAYOUT == kAttnBlock || LAYOUT == kAttnStaged, "plane layouts only");
  const int h = hq / nqt;
  const int qt = hq % nqt;

  float m_row = 0.f;
  const uint32_t live = __builtin_amdgcn_readfirstlane(const_chunk_rows(a, chunk, m_row));
  if (live == 0u) return;
  // Chunks whose m has the block's precomputed weights (const_weights_kernel,
  // formed once per (head, 32-query tile)) belong to the LOADED launch: its
  // tile loop loads those weights in place of the bias fragments and runs
  // no softmax.  The other launch serves every other chunk.
  const bool has_weights = kBlock && a.const_m != nullptr &&
                           __builtin_amdgcn_readfirstlane(a.const_m[0]) ==
                               __builtin_bit_cast(uint32_t, m_row);
  if (has_weights != LOADED) return;
  constexpr bool loaded = LOADED;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int j0 = qt * kBq;
  const int jq = j0 + 32 * w + l32;
  const int qt32 = (j0 >> 5) + w;
  const int64_t nt = a.np >> 5;
  const int64_t frag = ((int64_t)h * nt + qt32) * nt * 1024;
  // Per key tile 4 KB at the same lane offsets: the bias fragment (x), or
  // the loaded weights' planes (ph[0], ph[1], pl[0], pl[1] in x's four
  // 16-byte parts).
  const __amdgpu_buffer_rsrc_t rb =
      loaded ? buffer(reinterpret_cast<const float*>(
                          a.const_p + (((int64_t)h * nt + qt32) * nkt) * 4096),
                      (int64_t)nkt * 4096)
             : buffer(a.bias + frag, nt * 4096);
  const uint32_t ob = (uint32_t)lane * 16;
  const int64_t slice_bytes = (int64_t)a.np * 128;

  // Wave w copies the V^T planes of chunk row w (if live): lane l writes
  // chunk l % 4 of plane rows l / 4 and 16 + l / 4, as in the block kernel.
  const bool copies = (live >> w) & 1u;
  const uint8_t* vsrc = reinterpret_cast<const uint8_t*>(a.v) +
                        ((int64_t)(chunk * kConstRows + w) * kHeads + h) * slice_bytes +
                        (lane >> 2) * 64 + 16 * ((lane & 3) ^ swz(lane >> 2));
  auto copy = [&](int t, int stage) {
    if (!copies) return;
    const uint8_t* src = vsrc + (int64_t)t * kPlaneBytes;
    uint8_t* dst = ring + stage * kStageBytesC + 2 * w * kPlaneBytes;
    lds_dma16(src, dst);
    lds_dma16(src + 1024, dst + 1024);
    lds_dma16(src + (slice_bytes >> 1), dst + kPlaneBytes);
    lds_dma16(src + (slice_bytes >> 1) + 1024, dst + kPlaneBytes + 1024);
  };
  const uint32_t rd0 = l32 * 64 + 16 * (half ^ swz(l32));
  const uint32_t rd1 = l32 * 64 + 16 * ((2 + half) ^ swz(l32));
  auto plane_rd = [&](int stage, int r, int plane, int m) -> bf16x8 {
    return *(const bf16x8*)(ring + stage * kStageBytesC + (2 * r + plane) * kPlaneBytes + (m ? rd1 : rd0));
  };
  auto load_frag = [&](int t) -> f32x16 {
    const uint32_t so = (uint32_t)t * 4096;
    return cat4(buffer_f4(rb, ob, so), buffer_f4(rb, ob + 1024, so), buffer_f4(rb, ob + 2048, so),
                buffer_f4(rb, ob + 3072, so));
  };

  // Each live row's v^T tile factors 2^-(e_t + kVShift), exact powers of two.
  {
    const int64_t per = (int64_t)kHeads * nt;
    for (int i = tid; i < kConstRows * nkt; i += kThreads) {
      const int r = i / nkt, t = i % nkt;
      const int b = chunk * kConstRows + r;
      Sv[r][t] = b < a.batch
                     ? __builtin_ldexpf(a.scales[2 * (int64_t)a.batch * per + (int64_t)b * per +
                                                 (int64_t)h * nt + t],
                                        -kVShift)
                     : 0.f;
    }
  }

  // Logits of tile t from its bias fragment: fl(m + bias), -inf past key n.
  const int full_tiles = a.n / kBk;
  auto finish = [&](f32x16& x, int t) {
    if constexpr (loaded) return;
    if (t < full_tiles) {
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = m_row + x[r];
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = t * kBk + 8 * (r >> 2) + 4 * half + (r & 3);
        x[r] = key < a.n ? m_row + x[r] : -INFINITY;
      }
    }
  };

  ConstRowsO o = {};
  float l_run = 0.f;
  float m_ref = -INFINITY;
  float c_ref = 0.f;
  float w_ref = 1.f;
  const f32x16 zero16 = {};

  // The exact path's softmax of one tile, shared by the rows: weights
  // P = exp2(x log2(e) - c_ref) w_ref (at most 2^8 by the lazy max), into
  // fp16 planes as P 2^kVShift.
  auto softmax = [&](const f32x16& x, bf16x8 (&ph)[2], bf16x8 (&pl)[2]) {
    if constexpr (loaded) {
      ph[0] = __builtin_bit_cast(bf16x8, f32x4{x[0], x[1], x[2], x[3]});
      ph[1] = __builtin_bit_cast(bf16x8, f32x4{x[4], x[5], x[6], x[7]});
      pl[0] = __builtin_bit_cast(bf16x8, f32x4{x[8], x[9], x[10], x[11]});
      pl[1] = __builtin_bit_cast(bf16x8, f32x4{x[12], x[13], x[14], x[15]});
      return;
    }
    const float mt = xor32_max(max16(x));
    if (__any(mt > m_ref + kRescaleNat)) {
      const float m_new = __builtin_elementwise_maximum(m_ref, mt);
      const float c_new = m_new == -INFINITY ? 0.f : m_new * kLog2e;
      const float alpha = m_ref == -INFINITY ? 0.f : exp2_fast((m_ref - m_new) * kLog2e);
      for_const_rows([&](auto r) {
        f32x16& acc = const_row<decltype(r)::value>(o);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] *= alpha;
      });
      l_run *= alpha;
      m_ref = m_new;
      c_ref = c_new;
      w_ref = m_new == -INFINITY ? 1.f : exp2_fast(-__builtin_fmaf(m_new, kLog2e, -c_new));
    }
    const float f = w_ref * (float)(1 << kVShift);
    float ps = 0.f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      f32x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = exp2_fast(__builtin_fmaf(x[8 * m + e], kLog2e, -c_ref));
      ps += ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= f;
      split_f16(v, ph[m], pl[m]);
    }
    l_run = __builtin_fmaf(ps, w_ref, l_run);
  };
  // O_r += 2^-(e_t + kVShift) V'^T P'^T for every live row.  The block's
  // prepare projection gives every v^T tile of a head one plane exponent, the
  // same for every row, so there the products accumulate into O_r directly
  // and the factor is applied once in the epilogue.
  auto pv = [&](int stage, int t, const bf16x8 (&ph)[2], const bf16x8 (&pl)[2]) {
    if constexpr (kBlock && loaded) {
      // Every row's operands are read first and the 24 products issued row
      // by row within each term, so consecutive MFMAs are independent and no
      // LDS read waits on the MFMA before it.  Rows that are not live run on
      // whatever their stage holds (their copies are skipped) and are never
      // stored.
      bf16x8 vh[kConstRows][2], vl[kConstRows][2];
      for_const_rows([&](auto rc) {
        constexpr int r = decltype(rc)::value;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          vh[r][m] = plane_rd(stage, r, 0, m);
          vl[r][m] = plane_rd(stage, r, 1, m);
        }
      });
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        for_const_rows([&](auto rc) {
          constexpr int r = decltype(rc)::value;
          f32x16& orow = const_row<r>(o);
          orow = mfma_f16(vl[r][m], ph[m], orow);
        });
        for_const_rows([&](auto rc) {
          constexpr int r = decltype(rc)::value;
          f32x16& orow = const_row<r>(o);
          orow = mfma_f16(vh[r][m], pl[m], orow);
        });
        for_const_rows([&](auto rc) {
          constexpr int r = decltype(rc)::value;
          f32x16& orow = const_row<r>(o);
          orow = mfma_f16(vh[r][m], ph[m], orow);
        });
      }
      return;
    }
    for_const_rows([&](auto rc) {
      constexpr int r = decltype(rc)::value;
      if (!((live >> r) & 1u)) return;
      if constexpr (kBlock) {
        f32x16& orow = const_row<r>(o);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const bf16x8 vh = plane_rd(stage, r, 0, m);
          const bf16x8 vl = plane_rd(stage, r, 1, m);
          orow = mfma_f16(vl, ph[m], orow);
          orow = mfma_f16(vh, pl[m], orow);
          orow = mfma_f16(vh, ph[m], orow);
        }
        return;
      }
      f32x16 acc = zero16;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const bf16x8 vh = plane_rd(stage, r, 0, m);
        const bf16x8 vl = plane_rd(stage, r, 1, m);
        acc = mfma_f16(vl, ph[m], acc);
        acc = mfma_f16(vh, pl[m], acc);
        acc = mfma_f16(vh, ph[m], acc);
      }
      const float sc = Sv[r][t];
      f32x16& orow = const_row<r>(o);
#pragma unroll
      for (int e = 0; e < 16; ++e) orow[e] = __builtin_fmaf(acc[e], sc, orow[e]);
    });
  };

  const int last = nkt - 1;
  auto clamp = [&](int t) { return t < last ? t : last; };
  auto stage = [](int t) { return t % kConstStages; };
  // Prologue: tiles 0 and 1 on their way; tile t + 2 is copied at iteration
  // t into the stage that held tile t - 1, which every wave left behind at
  // the previous barrier.  Tiles past the last are clamped (in range, never
  // used).
  f32x16 x_a = load_frag(0);
  f32x16 x_b = load_frag(clamp(1));
  copy(0, 0);
  copy(clamp(1), 1);
  wait_vmcnt<4>();  // tile 0 and both bias fragments have landed
  __syncthreads();
  finish(x_a, 0);
  auto body = [&](int t, f32x16& cur, f32x16& nxt) {
    bf16x8 ph[2], pl[2];
    softmax(cur, ph, pl);
    cur = load_frag(clamp(t + 2));
    pv(stage(t), t, ph, pl);
    finish(nxt, t + 1);
    copy(clamp(t + 2), stage(t + 2));
    // Tile t + 1 has landed once at most this iteration's four bias-fragment
    // loads and four tile copies are outstanding (loads retire in order).
    // When tile t + 2 is past the last, nothing reads the loaded fragment
    // and the compiler may drop its loads: then only the four copies count.
    if (t + 2 <= last)
      wait_vmcnt<8>();
    else
      wait_vmcnt<4>();
    __syncthreads();
  };
  auto tail = [&](const f32x16& cur, int t) {
    bf16x8 ph[2], pl[2];
    softmax(cur, ph, pl);
    pv(stage(t), t, ph, pl);
  };
  int kt = 0;
  for (; kt + 2 < nkt; kt += 2) {
    body(kt, x_a, x_b);
    body(kt + 1, x_b, x_a);
  }
  if (kt + 1 < nkt) {
    body(kt, x_a, x_b);
    tail(x_b, kt + 1);
  } else {
    tail(x_a, kt);
  }
  wait_vmcnt<0>();  // the clamped tail loads land before the LDS is released

  const float l_tot = loaded ? a.const_l[h * a.np + jq] : xor32_sum(l_run);
  if (jq < a.n) {
    for_const_rows([&](auto rc) {
      constexpr int r = decltype(rc)::value;
      if (!((live >> r) & 1u)) return;
      const int b = chunk * kConstRows + r;
      const f32x16& orow = const_row<r>(o);
      // the block's products carry the head's v^T factor (exact powers of two)
      const float sc = kBlock ? Sv[r][0] : 1.0f;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int c = 8 * rr + 4 * half;  // channels c..c+3 of head h
        f32x4 ov4 = {orow[4 * rr + 0] * sc / l_tot, orow[4 * rr + 1] * sc / l_tot,
                     orow[4 * rr + 2] * sc / l_tot, orow[4 * rr + 3] * sc / l_tot};
        if constexpr (kBlock) {
          const int64_t col = h * kHeadDim + c;
          if (a.gate) ov4 = ov4 * *(const f32x4*)(a.gate + ((int64_t)b * a.np + jq) * kHidden + col);
          *(f32x4*)(a.out + ((int64_t)b * a.n + jq) * kHidden + col) = ov4;
        } else {
          *(f32x4*)(a.out + b * a.os[0] + h * a.os[1] + (int64_t)jq * a.os[2] + c) = ov4;
        }
      }
    });
  }
}

// The weights of the block's constant-mask rows, once for every such row
// (const_item's loaded path).  Every row whose keys all carry the mask bias
// m of the first constant-mask row has the logits x = fl(m + bias) for each
// (head, query, key), whatever its outer row.  One work-group per (head,
// 32-query tile), wave w on key tiles w, w + 4, ...: pass 1 each query's max
// m_q over all keys; pass 2 the exact softmax's weights with the reference
// at that max, P = exp2(x log2(e) - c) w, c = fl(m_q log2(e)),
// w = 2^-(m_q log2(e) - c) (equal quantised logits get equal weights), their
// sum l_q, and P 2^kVShift split into fp16 planes in the P.V operand order,
// stored as the four 16-byte parts of a bias fragment.  With no
// constant-mask row, const_m[0] becomes a NaN (no row's m matches it).
// Work-group 0 also writes the two chunk lists of the constant-mask launches
// (AttnArgs::const_m): the chunks whose rows have that m, and the others.
__global__ __launch_bounds__(kThreads) void const_weights_kernel(AttnArgs a, int nkt) {
  __shared__ int first;
  __shared__ int counts[2];
  __shared__ float red[kThreads / 64][32];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int nt = a.np >> 5;
  const int h = (int)blockIdx.x / nt;
  const int qt32 = (int)blockIdx.x % nt;
  if (tid == 0) first = a.batch;
  __syncthreads();
  for (int b = tid; b < a.batch; b += kThreads) {
    float m;
    if (constant_mask_row(a, b, m)) {
      atomicMin(&first, b);
      break;
    }
  }
  __syncthreads();
  const int b0 = first;
  float m_c = 0.f;
  const bool any = b0 < a.batch && constant_mask_row(a, b0, m_c);
  const uint32_t m_bits = any ? __builtin_bit_cast(uint32_t, m_c) : 0x7fc00000u;
  if (blockIdx.x == 0) {
    if (tid < 2) counts[tid] = 0;
    __syncthreads();
    const int nchunks = (a.batch + kConstRows - 1) / kConstRows;
    for (int c = tid; c < nchunks; c += kThreads) {
      float m_row;
      if (const_chunk_rows(a, c, m_row) == 0u) continue;
      const int list = __builtin_bit_cast(uint32_t, m_row) == m_bits ? 0 : 1;
      const int at = atomicAdd(&counts[list], 1);
      a.const_m[kConstListWord + list * nchunks + at] = (uint32_t)c;
    }
    __syncthreads();
    if (tid == 0) {
      a.const_m[0] = m_bits;
      a.const_m[1] = (uint32_t)counts[0];
      a.const_m[2] = (uint32_t)counts[1];
    }
  }
  if (!any) return;

  const __amdgpu_buffer_rsrc_t rb =
      buffer(a.bias + ((int64_t)h * nt + qt32) * nt * 1024, (int64_t)nt * 4096);
  const uint32_t ob = (uint32_t)lane * 16;
  const int full_tiles = a.n / kBk;
  auto logits = [&](int t) -> f32x16 {
    const uint32_t so = (uint32_t)t * 4096;
    f32x16 x = cat4(buffer_f4(rb, ob, so), buffer_f4(rb, ob + 1024, so),
                    buffer_f4(rb, ob + 2048, so), buffer_f4(rb, ob + 3072, so));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t * kBk + 8 * (r >> 2) + 4 * half + (r & 3);
      x[r] = (t < full_tiles || key < a.n) ? m_c + x[r] : -INFINITY;
    }
    return x;
  };
  float mx = -INFINITY;
  for (int t = w; t < nkt; t += kThreads / 64) mx = __builtin_elementwise_maximum(mx, max16(logits(t)));
  mx = xor32_max(mx);
  if (half == 0) red[w][l32] = mx;
  __syncthreads();
  const float m_q = __builtin_elementwise_maximum(
      __builtin_elementwise_maximum(red[0][l32], red[1][l32]),
      __builtin_elementwise_maximum(red[2][l32], red[3][l32]));
  __syncthreads();
  const float c = m_q * kLog2e;
  const float wr = exp2_fast(-__builtin_fmaf(m_q, kLog2e, -c));
  const float f = wr * (float)(1 << kVShift);
  uint8_t* const dst = a.const_p + (((int64_t)h * nt + qt32) * nkt) * 4096 + ob;
  float ps = 0.f;
  for (int t = w; t < nkt; t += kThreads / 64) {
    const f32x16 x = logits(t);
    bf16x8 ph[2], pl[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      f32x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = exp2_fast(__builtin_fmaf(x[8 * m + e], kLog2e, -c));
      ps += ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= f;
      split_f16(v, ph[m], pl[m]);
    }
    uint8_t* d = dst + (int64_t)t * 4096;
    *(bf16x8*)(d) = ph[0];
    *(bf16x8*)(d + 1024) = ph[1];
    *(bf16x8*)(d + 2048) = pl[0];
    *(bf16x8*)(d + 3072) = pl[1];
  }
  ps = xor32_sum(ps);
  if (half == 0) red[w][l32] = ps;
  __syncthreads();
  if (tid < 32)
    a.const_l[h * a.np + qt32 * 32 + tid] =
        ((red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid])) * wr;
}

// A work-group per item: the few items with work spread over the whole
// chip as the empty ones leave (a grid that walks the items would give some
// work-groups one item more than others).  The loop serves any grid.
// LOADED: the chunks with precomputed weights (no softmax registers, three
// work-groups per CU, as many as the LDS holds); the other launch keeps two.
template <int LAYOUT, bool LOADED>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(2, 2)))
void attention_const_kernel(AttnArgs a, int nqt, int nkt, int nchunks, uint32_t items) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kConstStages * kStageBytesC];
  __shared__ ConstScales Sv[kConstRows];
  // XCD x serves the (head, query tile) pairs [x H nqt / 8, (x + 1) H nqt / 8)
  // of every chunk, chunk-major.
  const int nhq = kHeads * nqt;
  const int xcd = (int)(blockIdx.x % kXcds);
  const int hq0 = xcd * nhq / kXcds;
  const int nh = (xcd + 1) * nhq / kXcds - hq0;
  if (nh == 0) return;
  if (LAYOUT == kAttnBlock && a.const_m != nullptr) {
    // The block's chunk lists (const_weights_kernel): a persistent grid, a
    // multiple of kXcds work-groups, walks this launch's list.
    const int count = (int)__builtin_amdgcn_readfirstlane(a.const_m[LOADED ? 1 : 2]);
    const uint32_t* list = a.const_m + kConstListWord + (LOADED ? 0 : nchunks);
    const int stride = (int)(gridDim.x / kXcds);
    for (int slot = (int)(blockIdx.x / kXcds); slot < nh * count; slot += stride) {
      const int chunk = (int)__builtin_amdgcn_readfirstlane(list[slot / nh]);
      const_item<LAYOUT, LOADED>(a, nqt, nkt, chunk, hq0 + slot % nh, ring, Sv);
      __syncthreads();
    }
    return;
  }
  // Every (chunk, pair) item, one work-group each (the items without
  // constant-mask rows leave at once).
  for (uint32_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int slot = (int)(item / kXcds);
    if (slot < nh * nchunks) {
      const_item<LAYOUT, LOADED>(a, nqt, nkt, slot / nh, hq0 + slot % nh, ring, Sv);
      __syncthreads();
    }
  }
}

// The relative log2 bias of the block (launch_bias_reference).  One
// work-group per (head, 32-query tile); every work-group first finds T, the
// first 32-key tile with a nonzero mask bias, minimised over the rows that
// have an unmasked key (so keys of tiles t < T are unmasked on every row the
// fast softmax serves); nkt when no row has a masked key.  Lane (half, l32)
// of a fragment holds 16 keys of query l32 (bias_frag_index), so a query's
// largest log2 bias over tiles t < T is a per-lane max, an xor-32 max and a
// max over the four waves (each takes every fourth tile).  C_q = ceil of it;
// every tile of the query is then rewritten as bias_l2 - (C_q - kRelOffset),
// one rounding.  With T = 0 nothing is rewritten and the flag stays 0.
__global__ __launch_bounds__(256) void bias_reference_kernel(const uint32_t* __restrict__ flags,
                                                             int batch, int n, int np,
                                                             float* __restrict__ bias_l2,
                                                             uint32_t* __restrict__ magnitudes) {
  __shared__ int wmin[4];
  __shared__ float qmax[4][32];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int nkt = (n + kBk - 1) / kBk;
  const int nt = np >> 5;
  int t_first = nkt;
  for (int b = tid; b < batch; b += 256) {
    const uint32_t* f = flags + (int64_t)b * kTileFlagParts * kTileFlagWords;
    uint32_t open = 0u;
    int first = nkt;
#pragma unroll
    for (int i = 0; i < kTileFlagWords; ++i) {
      const int lo = 32 * i;
      const uint32_t valid =
          nkt >= lo + 32 ? 0xffffffffu : nkt > lo ? (1u << (nkt - lo)) - 1u : 0u;
      open |= ~f[kTileFlagWords + i] & valid;
      const uint32_t m = f[i] & valid;
      if (first == nkt && m != 0u) first = lo + __builtin_ctz(m);
    }
    if (open != 0u) t_first = min(t_first, first);
  }
  // wave minimum, then the work-group's
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) t_first = min(t_first, __shfl_xor(t_first, d));
  if (lane == 0) wmin[w] = t_first;
  __syncthreads();
  const int T = min(min(wmin[0], wmin[1]), min(wmin[2], wmin[3]));
  if (T == 0) return;  // uniform
  const int h = (int)blockIdx.x / nt;
  const int qt = (int)blockIdx.x % nt;
  float* frag = bias_l2 + ((int64_t)h * nt + qt) * nt * 1024 + lane * 4;
  float m = -INFINITY;
  for (int t = w; t < T; t += 4) {
    const float* src = frag + (int64_t)t * 1024;
    const f32x16 x = cat4(*(const f32x4*)src, *(const f32x4*)(src + 256),
                          *(const f32x4*)(src + 512), *(const f32x4*)(src + 768));
    m = __builtin_elementwise_maximum(m, max16(x));
  }
  m = xor32_max(m);
  if (lane < 32) qmax[w][lane] = m;
  __syncthreads();
  const int q = lane & 31;
  const float mq = __builtin_elementwise_maximum(
      __builtin_elementwise_maximum(qmax[0][q], qmax[1][q]),
      __builtin_elementwise_maximum(qmax[2][q], qmax[3][q]));
  // |C_q| < 2^22 whenever the fast softmax runs (its logit bound); other
  // values are never read, and keep the copy as it is
  const float c = __builtin_ceilf(mq);
  const float shift = __builtin_fabsf(c) < 4194304.0f ? c - kRelOffset : 0.0f;
  for (int t = w; t < nt; t += 4) {
    float* dst = frag + (int64_t)t * 1024;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x4 v = *(const f32x4*)(dst + 256 * i);
      v = v - shift;
      *(f32x4*)(dst + 256 * i) = v;
    }
  }
  if (blockIdx.x == 0 && tid == 0) magnitudes[kRelativeBiasWord] = 1u;
}

}  // namespace

hipError_t launch_attention_split(int layout, const AttnArgs& a, hipStream_t stream) {
  const int nqt = (int)(a.np / kBq);
  const int nkt = (int)(round_up(a.n, kBk) / kBk);
  const uint64_t groups = ((uint64_t)a.batch + kRowGroup - 1) / kRowGroup;
  const uint64_t total = groups * kRowGroup * kHeads * nqt;
  if (total == 0) return hipSuccess;
  if (total > 0x7fffffffull) return hipErrorInvalidValue;
  if (a.tile_flags == nullptr || a.bias_l2 == nullptr || a.scales == nullptr ||
      nkt > kTileFlagWords * 32)
    return hipErrorInvalidValue;
  const size_t mask_row_bytes = (size_t)nkt * kBk * sizeof(float);
  const int ppg = pair_group_size(nqt, (uint64_t)kBq * (uint64_t)a.np * sizeof(float));
  // Three launches: rows on the fast softmax path (one work-group per work
  // item; the others leave after reading their row's flags), then the other
  // rows (fully masked rows, rows whose logits are not bounded) on a
  // persistent grid, then the constant-mask rows (padding rows), a chunk of
  // kConstRows at a time, one work-group per item.
  const uint32_t exact_grid =
      (uint32_t)std::min<uint64_t>((uint64_t)a.batch * kExactChunks, kExactGroups);
  const int nchunks = (a.batch + kConstRows - 1) / kConstRows;
  const uint64_t const_items =
      (uint64_t)kXcds * ((kHeads * nqt + kXcds - 1) / kXcds) * (uint64_t)nchunks;
  if (const_items > 0x7fffffffull) return hipErrorInvalidValue;
  const uint32_t const_grid = (uint32_t)const_items;
  if (layout == kAttnBlock) {
    hipLaunchKernelGGL((attention_split_kernel<kAttnBlock, false>), dim3((uint32_t)total),
                       dim3(kThreads), mask_row_bytes, stream, a, nqt, nkt, (uint32_t)total, ppg);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL((attention_split_kernel<kAttnBlock, true>), dim3(exact_grid),
                       dim3(kThreads), mask_row_bytes, stream, a, nqt, nkt, (uint32_t)total, ppg);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    if (a.const_m != nullptr) {
      // the shared weights and the chunk lists, then both constant-mask
      // launches on persistent grids (two work-groups per CU) over them
      if (a.const_l == nullptr || a.const_p == nullptr) return hipErrorInvalidValue;
      hipLaunchKernelGGL(const_weights_kernel, dim3((uint32_t)(kHeads * (a.np >> 5))),
                         dim3(kThreads), 0, stream, a, nkt);
      if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
      int cap = device_cu_count() * 2;
      cap -= cap % kXcds;
      const uint32_t grid = (uint32_t)std::max(cap, kXcds);
      hipLaunchKernelGGL((attention_const_kernel<kAttnBlock, true>), dim3(grid), dim3(kThreads), 0,
                         stream, a, nqt, nkt, nchunks, (uint32_t)const_items);
      if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
      hipLaunchKernelGGL((attention_const_kernel<kAttnBlock, false>), dim3(grid), dim3(kThreads), 0,
                         stream, a, nqt, nkt, nchunks, (uint32_t)const_items);
    } else {
      hipLaunchKernelGGL((attention_const_kernel<kAttnBlock, false>), dim3(const_grid),
                         dim3(kThreads), 0, stream, a, nqt, nkt, nchunks, (uint32_t)const_items);
    }
  } else if (layout == kAttnStaged) {
    hipLaunchKernelGGL((attention_split_kernel<kAttnStaged, false>), dim3((uint32_t)total),
                       dim3(kThreads), mask_row_bytes, stream, a, nqt, nkt, (uint32_t)total, ppg);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL((attention_split_kernel<kAttnStaged, true>), dim3(exact_grid),
                       dim3(kThreads), mask_row_bytes, stream, a, nqt, nkt, (uint32_t)total, ppg);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipLaunchKernelGGL((attention_const_kernel<kAttnStaged, false>), dim3(const_grid), dim3(kThreads), 0,
                       stream, a, nqt, nkt, nchunks, (uint32_t)const_items);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bias_reference(const uint32_t* flags, int batch, int n, int np, float* bias_l2,
                                 uint32_t* magnitudes, hipStream_t stream) {
  if (batch <= 0 || n <= 0) return hipSuccess;
  if (np % kBq || np < n || round_up(n, kBk) / kBk > kTileFlagWords * 32 || magnitudes == nullptr)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(bias_reference_kernel, dim3((uint32_t)(kHeads * (np >> 5))), dim3(256), 0,
                     stream, flags, batch, n, np, bias_l2, magnitudes);
  return hipGetLastError();
}

// ------------------------------------------------------------- staging
// A caller's strided q, k, v (element (b, h, j, c) at b s[0] + h s[1] +
// j s[2] + c) into the plane layout for kAttnStaged, one wave per (outer row
// b, head h, 32-row tile t, operand):
//   q, k: rows 32t .. 32t + 31 (zero past n) times 2^e, e chosen so that
//         the tile's max |value| 2^e lies in [2^14, 2^15) (|e| <=
//         kPlaneExpMax; 0 for a zero or non-finite tile), as fp16 hi and lo
//         planes [np][32] of the (b, h) slice, and 2^-e at
//         scales[((op batch + b) 4 + h) (np / 32) + t] (op 0: q, 1: k);
//   v:    the tile transposed to [32 channels][32 key positions] (a tile's
//         keys in v_position order) times 2^e (e = value_plane_exp of the
//         tile's max |value|) as fp16 hi and lo planes, and 2^-e at
//         scales[((2 batch + b) 4 + h) (np / 32) + t].
// partial (nullable): each work-group's NaN-propagating max |q|, |k|, |v| at
// partial[3 blockIdx.x + op] (0 for operands it did not stage), reduced by
// reduce_magnitudes_kernel.  Each wave transposes v through its own LDS
// tile.
__global__ __launch_bounds__(256) void stage_planes_kernel(AttnArgs a, uint8_t* qp, uint8_t* kp,
                                                           uint8_t* vp, float* scales,
                                                           float* partial, int64_t waves) {
  __shared__ float tv[4][32][33];
  __shared__ float wmax[4][3];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t gw = (int64_t)blockIdx.x * 4 + w;
  const int nt = a.np >> 5;
  float mq = 0.f, mk = 0.f, mv = 0.f;  // this wave's maxima (NaN-propagating)
  if (gw < waves) {  // whole waves
    const int op = (int)(gw % 3);
    const int64_t rest = gw / 3;
    const int t = (int)(rest % nt);
    const int64_t bh = rest / nt;
    const int h = (int)(bh & 3);
    const int64_t b = bh >> 2;
    const int r = lane >> 1;
    const int c0 = (lane & 1) * 16;
    const int j = 32 * t + r;
    const float* src = op == 0 ? a.q : op == 1 ? a.k : a.v;
    const int64_t* st = op == 0 ? a.qs : op == 1 ? a.ks : a.vs;
    f32x4 x[4] = {};
    if (j < a.n) {
      const float* row = src + b * st[0] + h * st[1] + (int64_t)j * st[2] + c0;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = *(const f32x4*)(row + 4 * i);
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      m = __builtin_elementwise_maximum(
          m, __builtin_elementwise_maximum(
                 __builtin_elementwise_maximum(__builtin_fabsf(x[i].x), __builtin_fabsf(x[i].y)),
                 __builtin_elementwise_maximum(__builtin_fabsf(x[i].z), __builtin_fabsf(x[i].w))));
    m = wave_max(m);
    const int64_t slice_bytes = (int64_t)a.np * 128;
    uint8_t* dst = (op == 0 ? qp : op == 1 ? kp : vp) + bh * slice_bytes;
    if (op < 2) {
      if (op == 0) mq = m;
      else mk = m;
      int e = plane_exp(m);
      e = e < -kPlaneExpMax ? -kPlaneExpMax : e > kPlaneExpMax ? kPlaneExpMax : e;
      const float f = __builtin_ldexpf(1.0f, e);
      bf16x8 hi[2], lo[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const f32x4 u = x[2 * i] * f, v = x[2 * i + 1] * f;
        split_f16(f32x8{u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w}, hi[i], lo[i]);
      }
      uint8_t* o = dst + (int64_t)j * 64 + c0 * 2;
      *(bf16x8*)o = hi[0];
      *(bf16x8*)(o + 16) = hi[1];
      *(bf16x8*)(o + (slice_bytes >> 1)) = lo[0];
      *(bf16x8*)(o + (slice_bytes >> 1) + 16) = lo[1];
      if (lane == 0)
        scales[(((int64_t)op * a.batch + b) * kHeads + h) * nt + t] = __builtin_ldexpf(1.0f, -e);
    } else {
      mv = m;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        tv[w][r][c0 + 4 * i + 0] = x[i].x;
        tv[w][r][c0 + 4 * i + 1] = x[i].y;
        tv[w][r][c0 + 4 * i + 2] = x[i].z;
        tv[w][r][c0 + 4 * i + 3] = x[i].w;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // lane: channel c = lane / 2, key positions p0 .. p0 + 15
      const int c = lane >> 1;
      const int p0 = (lane & 1) * 16;
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int p = p0 + i;
        const int g = 4 * (p >> 4) + v_position((p >> 2) & 3) / 4;  // (0, 2, 1, 3) is its own inverse
        v[i] = tv[w][4 * g + (p & 3)][c];
      }
      const int e = value_plane_exp(m);
      const float f = __builtin_ldexpf(1.0f, e);
      bf16x8 hi[2], lo[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        split_f16(f32x8{v[8 * i] * f, v[8 * i + 1] * f, v[8 * i + 2] * f, v[8 * i + 3] * f,
                        v[8 * i + 4] * f, v[8 * i + 5] * f, v[8 * i + 6] * f, v[8 * i + 7] * f},
                  hi[i], lo[i]);
      uint8_t* o = dst + (int64_t)t * kPlaneBytes + c * 64 + p0 * 2;
      *(bf16x8*)o = hi[0];
      *(bf16x8*)(o + 16) = hi[1];
      *(bf16x8*)(o + (slice_bytes >> 1)) = lo[0];
      *(bf16x8*)(o + (slice_bytes >> 1) + 16) = lo[1];
      if (lane == 0)
        scales[(((int64_t)2 * a.batch + b) * kHeads + h) * nt + t] = __builtin_ldexpf(1.0f, -e);
    }
  }
  if (partial != nullptr) {
    if (lane == 0) {
      wmax[w][0] = mq;
      wmax[w][1] = mk;
      wmax[w][2] = mv;
    }
    __syncthreads();
    if (threadIdx.x < 3) {
      const int op = threadIdx.x;
      partial[3 * (int64_t)blockIdx.x + op] = __builtin_elementwise_maximum(
          __builtin_elementwise_maximum(wmax[0][op], wmax[1][op]),
          __builtin_elementwise_maximum(wmax[2][op], wmax[3][op]));
    }
  }
}

// magnitudes[op] = max(magnitudes[op], partial[3 i + op]) over the count
// work-groups (op < 3; the record starts zeroed), one atomic per word and
// work-group; work-group 0 sets magnitudes[4] = 1.
__global__ __launch_bounds__(256) void reduce_magnitudes_kernel(const float* __restrict__ partial,
                                                                int64_t count,
                                                                uint32_t* __restrict__ magnitudes) {
  __shared__ float part[4][3];
  float m[3] = {0.f, 0.f, 0.f};
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
#pragma unroll
    for (int op = 0; op < 3; ++op) m[op] = __builtin_elementwise_maximum(m[op], partial[3 * i + op]);
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int op = 0; op < 3; ++op) {
    const float wm = wave_max(m[op]);
    if (lane == 0) part[w][op] = wm;
  }
  __syncthreads();
  if (threadIdx.x < 3) {
    const int op = threadIdx.x;
    const float r = __builtin_elementwise_maximum(__builtin_elementwise_maximum(part[0][op], part[1][op]),
                                                  __builtin_elementwise_maximum(part[2][op], part[3][op]));
    atomicMax(&magnitudes[op], __builtin_bit_cast(uint32_t, r));
    if (blockIdx.x == 0 && op == 0) magnitudes[4] = 1u;
  }
}

int64_t stage_planes_groups(const AttnArgs& a) {
  return (3 * (int64_t)a.batch * kHeads * (a.np / 32) + 3) / 4;
}

hipError_t launch_stage_planes(const AttnArgs& a, void* q_planes, void* k_planes, void* v_planes,
                               float* scales, float* partial, uint32_t* magnitudes,
                               hipStream_t stream) {
  const int64_t waves = 3 * (int64_t)a.batch * kHeads * (a.np / 32);
  if (waves == 0) return hipSuccess;
  const int64_t blocks = stage_planes_groups(a);
  if (blocks > 0x7fffffffll || a.np % kBq) return hipErrorInvalidValue;
  if ((partial == nullptr) != (magnitudes == nullptr)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(stage_planes_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, a,
                     static_cast<uint8_t*>(q_planes), static_cast<uint8_t*>(k_planes),
                     static_cast<uint8_t*>(v_planes), scales, partial, waves);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || magnitudes == nullptr) return e;
  const int64_t rgroups = (blocks + 255) / 256 < 256 ? (blocks + 255) / 256 : 256;
  hipLaunchKernelGGL(reduce_magnitudes_kernel, dim3((uint32_t)rgroups), dim3(256), 0, stream,
                     partial, blocks, magnitudes);
  return hipGetLastError();
}

}  // namespace fpx
