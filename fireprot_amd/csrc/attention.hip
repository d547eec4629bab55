// Flash-style triangle attention on the CDNA4 FP32 matrix cores, on the
// reference C-ABI layout (q, k, v, out [B][n][4][32], a shared [4][n][S]
// bias): the kernel behind ck_attention, ck_attention_exact1536,
// ck_attention_vector_bias1000, fpx_attn_core and fpx_attn_core_masked.
// The block and the strided (OpenFold3) entries run attention_split_kernel.
//
// One work-group = (outer row b, head h, 128 queries); four wavefronts, each
// owning 32 queries.  Keys are streamed in tiles of 32.  K and V^T tiles are
// staged once in LDS for the four waves, in double buffers, so there is one
// barrier per tile.  The N x N logits of a row and the N^3 score volume never
// reach HBM.
//
// Per key tile each wave computes S^T = K Q^T (16 x v_mfma_f32_32x32x2_f32)
// and O^T += V^T P^T (16 more).  With the transposed products, each lane
// column (lane % 32) holds one query in both results.  The online-softmax row
// statistics, the P operand and the O rescale therefore all live in the lane
// that needs them.  The only cross-lane step is an xor-32 exchange of a tile
// max.
//
// Cost model.  On gfx950 an FP32 MFMA and VALU work never overlap, whether
// they come from one wave or from several waves of a SIMD: a tile costs its
// 32 x 64 matrix cycles plus every VALU instruction around them, and a
// v_exp_f32 costs about as much as three other VALU instructions while the
// matrix cores are busy.  Software pipelining inside a wave buys nothing but
// load slack, so each tile runs S^T, softmax and O^T += V^T P^T in order, and
// the loop is built to issue as few VALU instructions as possible.
//
// Rows with at least one unmasked key (the fast path):
//   - S^T accumulates from zero and one fma per logit adds the triangle
//     bias pre-scaled by log2(e) (loaded from a fragment-major copy straight
//     into registers): fma(s, log2(e), bias log2(e)), logits in log2 units.
//     The dot product's partial sums thus round at its own magnitude; with
//     the bias as the accumulator's start value they rounded at the bias's
//     (|logit| ~ 60 in log2 units), about ten times the error of FP32
//     native attention.
//   - The mask bias is added only on tiles flagged as masked.  A masked key
//     of such a row gets weight exactly 0 whatever the rounding of its logit,
//     because its logit is about -1e9 below the row max.
//   - Weights are exp2(x - c) with one reference c per query, and c = 0
//     whenever the row max lies within 2^+-56.  Then a tile needs neither a
//     max nor a subtraction: 16 exp2 and the adds of the row sum.  A tile max
//     is formed only for the first tile and when the running sum passes
//     2^64; O and l are then rescaled to the new reference.
// Rows whose keys are all masked (the exact path):
//   - Every tile forms fl(fl(s + mask_bias) + bias) in natural units, the
//     native order (patches/protenix/0005-*.patch:36-45; kernels/amd/
//     fireprot_softmax_fp32.cpp:33-35), from the unscaled q and an unscaled
//     bias copy.  These logits are quantised to the FP32 spacing of -1e9 (64),
//     and this order reproduces which keys tie at the max.  Weights are
//     exp2(fma(x, log2 e, -c)) with c = fl(m log2 e) of a lazy running max m
//     (rescaled when a tile max exceeds it by 2^8), so equal logits get equal
//     weights.
// A row whose logits are all -inf gives NaN, as torch.softmax does.
#include "attn_common.hpp"
#include "common.hpp"
#include "kernels.hpp"

#include <cmath>
#include <type_traits>

namespace fpx {
namespace {

constexpr int kPad = 4;    // LDS row padding (floats): conflict-free b128 reads
constexpr int kThreads = 256;
// Occupancy the register budget is set for (waves per SIMD).
#ifndef FPX_ATTN_WAVES_PER_SIMD
#define FPX_ATTN_WAVES_PER_SIMD 3
#endif

typedef float KTile[kBk][kHeadDim + kPad];  // [key][channel]
typedef float VTile[kHeadDim][kBk + kPad];  // [channel][key]

// Tile sources of one work-group.  Every tile index passed in is in range.
template <int LAYOUT>
struct Tiles;

// The reference C-ABI layout (kernels/amd/fireprot_ck_attention.cpp:34-43):
// q, k, v, out [B][n][H][32]; bias [H][n][bias_stride]; mask bias nullable.
template <>
struct Tiles<kAttnHeadLast> {
  const AttnArgs& a;
  int b, h, row8, col4, half, jq;
  __device__ __forceinline__ Tiles(const AttnArgs& args, int b_, int h_, int /*qt32*/, int tid,
                                   int /*lane*/, int half_, int jq_)
      : a(args), b(b_), h(h_), row8(tid >> 3), col4((tid & 7) * 4), half(half_), jq(jq_) {}
  __device__ __forceinline__ f32x4 row(const float* base, int t) const {
    const int key = t * kBk + row8;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    return key < a.n
               ? *(const f32x4*)(base + (((int64_t)b * a.n + key) * kHeads + h) * kHeadDim + col4)
               : zero;
  }
  // thread (row8 = key, col4 = channel group) for both K and V
  __device__ __forceinline__ f32x4 k(int t) const { return row(a.k, t); }
  __device__ __forceinline__ f32x4 v(int t) const { return row(a.v, t); }
  static __device__ __forceinline__ void store_v(VTile& vs, f32x4 v, int row8, int col4) {
    vs[col4 + 0][row8] = v.x;
    vs[col4 + 1][row8] = v.y;
    vs[col4 + 2][row8] = v.z;
    vs[col4 + 3][row8] = v.w;
  }
  __device__ __forceinline__ f32x16 bias(int t) const {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 x[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int key = t * kBk + 8 * rr + 4 * half;  // n % 4 == 0: all-in or all-out
      x[rr] = (jq < a.n && key < a.n)
                  ? *(const f32x4*)(a.bias + ((int64_t)h * a.bias_rows + jq) * a.bias_stride + key)
                  : zero;
    }
    return cat4(x[0], x[1], x[2], x[3]);
  }
  __device__ __forceinline__ f32x16 bias_l2(int t) const {
    f32x16 r = bias(t);
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] *= kLog2e;
    return r;
  }
  __device__ __forceinline__ f32x16 mask(int t) const {
    f32x16 r;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = t * kBk + 8 * rr + 4 * half + e;
        r[4 * rr + e] = key < a.n ? (a.mbias ? a.mbias[(int64_t)b * a.mb_stride + key] : 0.f)
                                  : -INFINITY;
      }
    }
    return r;
  }
};

// S^T[key][q] = c + sum_ch K[key][ch] Q[q][ch] for the 32 keys of ks; lane
// half hb supplies channel 16*hb + s at step s.
__device__ __forceinline__ f32x16 qk_chain(const KTile& ks, const float* qf, int l32, int half,
                                           f32x16 c) {
  f32x16 s = c;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const f32x4 kv = *(const f32x4*)&ks[l32][16 * half + 4 * t];
    s = mfma32(kv.x, qf[4 * t + 0], s);
    s = mfma32(kv.y, qf[4 * t + 1], s);
    s = mfma32(kv.z, qf[4 * t + 2], s);
    s = mfma32(kv.w, qf[4 * t + 3], s);
  }
  return s;
}

template <int LAYOUT>
__global__ __launch_bounds__(kThreads, FPX_ATTN_WAVES_PER_SIMD) void attention_kernel(
    AttnArgs a, int nqt, int nkt, uint32_t total) {
  static_assert(LAYOUT == kAttnHeadLast, "the reference C-ABI layout only");
  __shared__ __attribute__((aligned(16))) KTile Ks[2];
  __shared__ __attribute__((aligned(16))) VTile Vs[2];

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
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;
  const int j0 = qt * kBq;
  const int jq = j0 + 32 * w + l32;
  const int qt32 = (j0 >> 5) + w;
  const int row8 = tid >> 3;
  const int col4 = (tid & 7) * 4;
  const int last = nkt - 1;
  const Tiles<LAYOUT> io(a, b, h, qt32, tid, lane, half, jq);

  // Row classification.  masked(t): some key of tile t has a nonzero mask
  // bias.  has_unmasked: some key k < n of the row has a zero mask bias.
  const bool any_masked = a.mbias != nullptr || a.n % kBk != 0;
  int found = a.mbias == nullptr;
  if (!found) {
    for (int k = tid; k < a.n; k += kThreads) found |= a.mbias[(int64_t)b * a.mb_stride + k] == 0.0f;
  }
  const bool has_unmasked = __syncthreads_or(found) != 0;
  auto masked = [&](int t) -> bool {
    return any_masked && (a.mbias != nullptr || (t + 1) * kBk > a.n);
  };
  auto mask_vals = [&](int t) -> f32x16 { return io.mask(t); };

  // Q fragment (B operand of S^T = K Q^T): lane holds Q[jq][16*half + s].
  float qf[16];
  {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    const bool ok = jq < a.n;
    const float* src = a.q + (((int64_t)b * a.n + (ok ? jq : 0)) * kHeads + h) * kHeadDim + 16 * half;
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
  float l_run = 0.f;

  // O^T[c][q] += V^T[c][key] P^T[key][q]; lane register r of p is key
  // 8*(r/4) + 4*half + r%4, as in the S^T accumulator.
  auto pv = [&](const VTile& vs, const f32x16& p) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x4 vv = *(const f32x4*)&vs[l32][8 * rr + 4 * half];
      o = mfma32(vv.x, p[4 * rr + 0], o);
      o = mfma32(vv.y, p[4 * rr + 1], o);
      o = mfma32(vv.z, p[4 * rr + 2], o);
      o = mfma32(vv.w, p[4 * rr + 3], o);
    }
  };

  // One pass over the key tiles.  Two register sets alternate between even
  // and odd tiles: a tile's bias is loaded into its set two tiles ahead, the
  // S^T chain of the tile accumulates there, and the weights go to p.
  auto run = [&](auto exact_tag) {
    constexpr bool kExact = decltype(exact_tag)::value;
    const f32x16 zero16 = {};
    f32x16 p;

    // Reference state of this lane's query.
    //   exact: m_ref = lazy running max (logit units), m_thr = the tile max
    //     that triggers a rescale, c_ref = fl(m_ref log2 e) (0 while m_ref is
    //     -inf, so all-(-inf) tiles give weight exp2(-inf) = 0).
    //   fast: m_ref = largest tile max seen on the rare path (log2 units;
    //     -inf while the query has no reference), c_ref = the reference;
    //     has_ref / c_zero are wave-uniform.
    float m_ref = -INFINITY;
    float m_thr = -INFINITY;
    float c_ref = 0.f;
    bool has_ref = false;
    bool c_zero = true;

    // x: this tile's logits (exact: logit units; fast: log2 units) -> p.
    auto softmax = [&](const f32x16& x) {
      if (kExact) {
        const float mt = xor32_max(max16(x));
        if (__any(mt > m_thr)) {
          const float m_new = __builtin_elementwise_maximum(m_ref, mt);
          const float c_new = m_new == -INFINITY ? 0.f : m_new * kLog2e;
          const float alpha = m_ref == -INFINITY ? 0.f : exp2_fast(c_ref - c_new);
#pragma unroll
          for (int r = 0; r < 16; ++r) o[r] *= alpha;
          l_run *= alpha;
          m_ref = m_new;
          c_ref = c_new;
          m_thr = m_new + kRescaleNat;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = exp2_fast(__builtin_fmaf(x[r], kLog2e, -c_ref));
        l_run += sum16(p);
        return;
      }
      float ovf = 0.f;
      if (has_ref) {
        if (c_zero) {
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
          return;
        }
        ovf = over ? 1.f : 0.f;
      }
      // Rare path, taken by the whole wavefront.  A lane moves its reference
      // only when it has none yet, when its own running sum overflowed, or
      // when this tile's max lies more than kSnap above the reference; the
      // decision is shared by the lane pair (l, l ^ 32) that holds the query.
      // After a sum overflow the true row max is at least c_ref + 52, so the
      // reference moves up by at least kLift and the weights stay below 2^24.
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
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = exp2_fast(x[r] - c_ref);
      l_run += sum16(p);
      has_ref = __all(m_ref != -INFINITY);
      c_zero = __all(c_ref == 0.f);
    };

    auto bias_of = [&](int t) -> f32x16 { return kExact ? io.bias(t) : io.bias_l2(t); };

    // Prologue: K(0), V(0) into LDS; K(1), V(1) and the biases of tiles 0
    // and 1 in flight.
    f32x16 set_a = bias_of(0);
    f32x16 set_b = bias_of(last < 1 ? last : 1);
    {
      const f32x4 k0 = io.k(0);
      const f32x4 v0 = io.v(0);
      *(f32x4*)&Ks[0][row8][col4] = k0;
      Tiles<LAYOUT>::store_v(Vs[0], v0, row8, col4);
    }
    f32x4 kreg = io.k(last < 1 ? last : 1);
    f32x4 vreg = io.v(last < 1 ? last : 1);
    __syncthreads();

    // Tile kt: Ks/Vs[kt&1] hold K(kt), V(kt); x holds bias(kt); kreg/vreg
    // hold K(kt+1), V(kt+1) (loads in flight).  Indices past the last tile
    // are clamped (in range, never used).
    auto body = [&](int kt, f32x16& x) {
      const int par = kt & 1;
      if (kExact) {
        p = qk_chain(Ks[par], qf, l32, half, zero16);
        const f32x16 mb = mask_vals(kt);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = (p[r] + mb[r]) + x[r];
      } else {
        // The dot product accumulates from zero (its partial sums round at
        // its own magnitude, not at the bias's), then one fma adds the
        // log2(e)-scaled bias: log2-domain logits at FP32 accuracy.
        p = qk_chain(Ks[par], qf, l32, half, zero16);
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = __builtin_fmaf(p[r], kLog2e, x[r]);
        if (masked(kt)) {
          const f32x16 mb = mask_vals(kt);
#pragma unroll
          for (int r = 0; r < 16; ++r) x[r] = __builtin_fmaf(mb[r], kLog2e, x[r]);
        }
      }
      softmax(x);
      x = bias_of(kt + 2 < last ? kt + 2 : last);
      pv(Vs[par], p);
      *(f32x4*)&Ks[par ^ 1][row8][col4] = kreg;
      Tiles<LAYOUT>::store_v(Vs[par ^ 1], vreg, row8, col4);
      kreg = io.k(kt + 2 < last ? kt + 2 : last);
      vreg = io.v(kt + 2 < last ? kt + 2 : last);
      __syncthreads();
    };

    int kt = 0;
    for (; kt + 1 < nkt; kt += 2) {
      body(kt, set_a);
      body(kt + 1, set_b);
    }
    if (kt < nkt) body(kt, set_a);
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
      const int c = 8 * rr + 4 * half;  // channels c..c+3 of head h
      f32x4 ov = {o[4 * rr + 0] / l_tot, o[4 * rr + 1] / l_tot, o[4 * rr + 2] / l_tot,
                  o[4 * rr + 3] / l_tot};
      *(f32x4*)(a.out + (((int64_t)b * a.n + jq) * kHeads + h) * kHeadDim + c) = ov;
    }
  }
}

}  // namespace

hipError_t launch_attention(int layout, const AttnArgs& a, hipStream_t stream) {
  if (layout != kAttnHeadLast) return hipErrorInvalidValue;
  const int nqt = (int)(round_up(a.n, kBq) / kBq);
  const int nkt = (int)(round_up(a.n, kBk) / kBk);
  const uint64_t groups = ((uint64_t)a.batch + kRowGroup - 1) / kRowGroup;
  const uint64_t total = groups * kRowGroup * kHeads * nqt;
  if (total == 0) return hipSuccess;
  if (total > 0x7fffffffull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_kernel<kAttnHeadLast>, dim3((uint32_t)total), dim3(kThreads), 0,
                     stream, a, nqt, nkt, (uint32_t)total);
  return hipGetLastError();
}

}  // namespace fpx
