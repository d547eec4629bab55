// Internal launch interface between the C-ABI layer (capi.hip) and the kernels.
// Nothing here is exported; the public surface is include/fireprot_amd.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fpx {

// ---------------------------------------------------------------- attention
// Row-wise triangle attention over B outer rows, H = 4 heads, d = 32.
//
// kAttnBlock:  the block's own workspace layout (all extents padded to np,
//              a multiple of 128; padded keys carry -inf in mbias):
//                q, k, v: the plane layout of ProjArgs (q pre-scaled by
//                        1/sqrt(32); v transposed per head), scales beside
//                mbias: [B][np]          (required)
//                tile_flags: [B][kTileFlagParts][kTileFlagWords] bit t of
//                        part 0 = some key of 32-key tile t has a nonzero
//                        mask bias; of part 1 = every key of tile t has one;
//                        of part 2 = every key of tile t has a mask bias at
//                        or below -kSkipMask; words 0 and 1 of part 3 =
//                        the row's largest mask bias and its smallest over
//                        the keys < n, as float bits (NaN-propagating)
//                magnitudes: nullable, kMagnitudeWords written by the
//                        prepare projection (see ProjArgs::magnitudes)
//                bias : [H][np][np] in fragment order (bias_frag_index)
//                bias_l2: the same scaled by log2(e)
//                gate : [B][np][128] sigmoid(g), multiplied in the epilogue
//                out  : [B][n][128]      (o * gate, head-last)
// kAttnHeadLast: the reference C-ABI layout (fireprot_ck_attention.cpp:34-43):
//                q, k, v, out : [B][n][H][32] (strides n*128, 32, 128, 1)
//                bias : [H][n][bias_stride]  (batch stride 0)
//                mbias: nullable, [B] rows of n values, row stride mb_stride
// kAttnStrided: any caller layout with channel stride 1 (the input of
//                launch_stage_planes):
//                q, k, v, out : element (b, h, j, c) at b*s[0] + h*s[1] + j*s[2] + c
//                               (qs, ks, vs, os), rows 16-byte aligned
//                mbias, tile_flags, bias, bias_l2 : staged as for kAttnBlock
//                               (launch_mask_rows, launch_stage_bias), np a
//                               multiple of 128
// kAttnStaged:  kAttnStrided's operands after launch_stage_planes: q, k, v
//                in the plane layout with their scales (as kAttnBlock
//                reads them), out through the os strides, no gate
enum AttnLayout { kAttnBlock = 0, kAttnHeadLast = 1, kAttnStrided = 2, kAttnStaged = 3 };

// Words of per-row tile flags: 32-key tiles of np <= 4096 keys.
constexpr int kTileFlagWords = 4;
constexpr int kTileFlagParts = 4;
constexpr int kTileFlagMaxPart = 3;

// Per-tile exponent range of the fp16 planes: |e| <= kPlaneExpMax, so the
// product scale 2^-(e_q + e_k) times log2(e) stays a normal float.
constexpr int kPlaneExpMax = 63;

// Trailing key tiles whose every mask bias is <= -kSkipMask are not visited
// on rows that have an unmasked key, when the logit magnitude bound
// B = 32 max|q| max|k| + max|bias| (q as stored, natural units) is below
// kSkipBound and max|v| is finite.  Their weights are then exactly 0: a
// skipped key's log2-domain logit lies at least (kSkipMask - 2 B) log2(e)
// > 5e8 below the row's softmax reference (which is at least the logit of
// the row's unmasked key), so exp2 underflows to 0 (bit-identical results).
constexpr float kSkipMask = 536870912.0f;  // 2^29
constexpr float kSkipBound = 67108864.0f;  // 2^26
// The FP32 block attention's fast softmax (attention_split.hip) runs on rows
// with an unmasked key when B plus the row's largest mask bias (if positive)
// is below kFastBound: every logit of an unmasked key then lies within 2^22
// of 0 in log2 units, so the integer softmax reference stays exact when a
// tile's plane exponent is added to it.
constexpr float kFastBound = 2097152.0f;  // 2^21
// Words of the magnitude record: max|q|, max|k|, max|v|, max|bias| as float
// bits (atomicMax on non-negative floats; a NaN sorts above inf, so any
// non-finite value disables the skip), then 1 once the projection wrote them.
// A skipped key with a non-finite v would have made the native row NaN
// (0 * inf), hence max|v| must be finite too.  Word kRelativeBiasWord is 1
// when launch_bias_reference rewrote the log2-scaled bias copy relative to
// each query's reference (zeroed with the rest of the record by the mask
// stage).
constexpr int kMagnitudeWords = 6;
constexpr int kRelativeBiasWord = 5;
// The relative log2 bias: bias log2(e) - C_q + kRelOffset, C_q = the ceiling
// of query q's largest log2 bias over the key tiles that precede every row's
// first masked tile (the keys unmasked on every row with an unmasked key).
constexpr float kRelOffset = 8.0f;

// The constant-mask attention serves chunks of kConstRows consecutive outer
// rows; kConstListWord: the first chunk-list word of AttnArgs::const_m.
constexpr int kConstRows = 4;
constexpr int kConstListWord = 64;

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* mbias;
  int64_t mb_stride;
  const float* bias;
  const float* bias_l2;  // kAttnBlock only
  int64_t bias_stride;
  int64_t bias_rows;
  const float* gate;
  float* out;
  const uint32_t* tile_flags;
  const uint32_t* magnitudes;  // kAttnBlock: nullable; enables the trailing-tile skip
  const float* scales;  // kAttnBlock, kAttnStaged: the planes' inverse scales
  // kAttnBlock, nullable: the constant-mask rows' shared weights and work
  // lists, written by the split launch itself (const_weights_kernel):
  // const_m[0] the mask bias m the weights serve (float bits; a NaN when no
  // row has a constant mask), const_m[1] and const_m[2] the numbers of
  // kConstRows-row chunks with constant-mask rows of that m and of another
  // m, their chunk indices from word kConstListWord (the first list) and
  // kConstListWord + ceil(batch / kConstRows) (the second);
  // const_l[4][np] each query's weight sum, const_p the weights' fp16 planes,
  // 4 KB per (head, 32-query tile, key tile).  Each may be null only with all.
  uint32_t* const_m;
  float* const_l;
  uint8_t* const_p;
  int64_t qs[3];  // kAttnStrided: (batch, head, row) element strides
  int64_t ks[3];
  int64_t vs[3];
  int64_t os[3];
  int batch;
  int n;
  int np;
};

// launch_attention: kAttnHeadLast (the reference C-ABI layout) on the FP32
// matrix cores (attention_kernel).  launch_attention_split runs
// attention_split_kernel (FP32-accurate products on the 16-bit matrix cores)
// for kAttnBlock or kAttnStaged.
hipError_t launch_attention(int layout, const AttnArgs& args, hipStream_t stream);
hipError_t launch_attention_split(int layout, const AttnArgs& args, hipStream_t stream);
// The FP32 block after its prepare stage: rewrite bias_l2 ([4][np][np],
// bias_frag_index order) as bias log2(e) - C_q + kRelOffset and set
// magnitudes[kRelativeBiasWord] = 1, unless no key tile precedes every row's
// first masked tile (then nothing changes).  flags: the rows' tile flags.
hipError_t launch_bias_reference(const uint32_t* flags, int batch, int n, int np, float* bias_l2,
                                 uint32_t* magnitudes, hipStream_t stream);
// kAttnStrided q, k, v of args -> the plane layout of kAttnStaged: q_planes,
// k_planes, v_planes each [batch][4] slices of np * 128 bytes, scales
// [3][batch][4][np / 32] floats.
// magnitudes (nullable, with partial of 3 stage_planes_groups floats):
// words 0-2 of the record (max |q|, |k|, |v|) and word 4.
int64_t stage_planes_groups(const AttnArgs& args);
hipError_t launch_stage_planes(const AttnArgs& args, void* q_planes, void* k_planes,
                               void* v_planes, float* scales, float* partial,
                               uint32_t* magnitudes, hipStream_t stream);

// --------------------------------------------------------------- projection
// Row tiles are 32 consecutive j of one outer row i; A rows are read at
// x + i*xs_i + j*xs_j (channel stride 1), which covers the ending-node
// transposed read without a copy.
enum ProjMode {
  kProjBlock = 0,  // LN -> q,k,v,g (+ triangle bias) into the block workspace
  kProjQkv = 1,    // q,k,v of already-normalised rows -> out[3][rows][128]
  kProjOut = 2,    // (o * gate) rows -> W_o (+ b_o) -> out + i*os_i + j*os_j
};

struct ProjArgs {
  const float* x;
  int64_t xs_i;
  int64_t xs_j;
  int rows_i;
  int rows_j;    // valid j extent
  int span_j;    // j extent covered by tiles (np for kProjBlock, else rows_j)
  const float* ln_w;
  const float* ln_b;
  float eps;
  const float* w[4];   // [128 out][128 in] torch layout, one per output group
  const float* b_g;    // kProjBlock: gate bias (nullable); kProjOut: b_o (nullable)
  const float* w_bias; // kProjBlock: [4][128] triangle-bias weights
  float q_scale;
  // kProjBlock outputs
  float* qh;
  float* kh;
  float* vt;
  float* gs;
  float* tri_bias;     // fragment order (bias_frag_index)
  float* tri_bias_l2;  // the same scaled by log2(e)
  uint32_t* magnitudes;  // nullable: max|q|, max|k|, max|v|, max|bias| (kMagnitudeWords)
  // Plane layout of q, k, v^T (kProjBlock): the (i, h) slice of np * 128
  // bytes holds a hi plane and then a lo plane of 16-bit values:
  //   q, k: [np rows j][32 channels] fp16 of the value times 2^e; hi =
  //         fp16(x 2^e) and lo = fp16(x 2^e - hi) carry 22 bits;
  //   v^T:  [np / 32 key tiles][32 channels][32 key positions] fp16 of the
  //         value times 2^e, hi and lo as for q, k; key 4g + e of a tile at
  //         position 16 (g / 4) + 4 (0, 2, 1, 3)[g % 4] + e (the S^T
  //         accumulator's register order);
  //   e: one per head and operand, from the bound sum_c |W_c| (sqrt(128)
  //         |ln_w_c| + |ln_b_c|) on the values of LayerNorm-normalised rows
  //         (times 1/sqrt(32) for q), so that the bound times 2^e lies in
  //         [2^14, 2^15) (v^T: value_plane_exp of the bound);
  //   scales[(t * rows_i + i) * 4 + h][j / 32] = 2^-e for t = 0 (q), 1 (k),
  //         2 (v^T): the same for every row i and tile of a head.
  float* scales;
  int np;
  // kProjQkv / kProjOut outputs
  float* out;
  int64_t os_i;
  int64_t os_j;
  int accumulate;  // kProjOut: out = out + (x W_o^T + b_o), the residual update
};

// projection_split_kernel: fp16 hi/lo planes on the 16-bit matrix cores.
hipError_t launch_projection(int mode, const ProjArgs& args, hipStream_t stream);

// -------------------------------------------------------------- elementwise
// mbias[i][k] = k < n ? inf * (mask_x[i][k] - 1) : -inf  (0 for k < n when
// mask is null), the per-row tile flags of the attention kernel, zero rows
// [n, np) of every head of the triangle bias: both float copies in fragment
// order (bias_frag_index, unscaled then log2(e)-scaled, contiguous), or the
// one bf16 copy (bias_frag_index_bf16) when bias_bf16, and zero the
// magnitude record (nullable) that the projection then fills.
hipError_t launch_mask_bias(const float* mask, int64_t ms_i, int64_t ms_j, int n, int np,
                            float inf, float* mbias, uint32_t* tile_flags, void* tri_bias,
                            bool bias_bf16, uint32_t* magnitudes, hipStream_t stream);

// Staging for kAttnStrided / kAttnStaged.  launch_mask_rows: mbias[i][k] =
// values[i*vs_i + k*vs_k] for k < n (0 when values is null), -inf for n <= k
// < np, and the tile flags, for rows i < rows; it zeroes the magnitude record
// (nullable).  launch_stage_bias: both fragment-order copies (as is, and
// scaled by log2(e)) of bias[h][q][k] read at h*sh + q*sq + k*sk, 0 for q or
// k >= n (and everywhere when bias is null); max |bias| into the record's
// word 3 (nullable).  launch_stage_planes fills words 0-2 and sets word 4.
hipError_t launch_mask_rows(const float* values, int64_t vs_i, int64_t vs_k, int rows, int n,
                            int np, float* mbias, uint32_t* tile_flags, uint32_t* magnitudes,
                            hipStream_t stream);
hipError_t launch_stage_bias(const float* bias, int64_t sh, int64_t sq, int64_t sk, int n, int np,
                             float* frag, float* frag_l2, uint32_t* magnitudes,
                             hipStream_t stream);

// LayerNorm over 128 channels of rows x[i][j] at x + i*xs_i + j*xs_j,
// written contiguously to y[(i*rows_j + j)*128 + c].
hipError_t launch_layer_norm(const float* x, int64_t rows_i, int64_t rows_j, int64_t xs_i,
                             int64_t xs_j, const float* w, const float* b, float eps, float* y,
                             hipStream_t stream);

// out = value * sigmoid(gate), float4 vectors.
hipError_t launch_sigmoid_mul(const float* gate, const float* value, float* out, int64_t count4,
                              hipStream_t stream);

// Exact bf16 plane split self-check (split.hpp) over count8 groups of 8 floats.
hipError_t launch_split_planes(const float* x, uint16_t* planes, int64_t count8,
                               hipStream_t stream);

// ------------------------------------------------------------ BF16 block
// BF16 storage / FP32 accumulation variant of the block (gfx950
// v_mfma_f32_32x32x16_bf16).  Same workspace roles and strides as the FP32
// block, with q, k, v^T, gate (rows padded to np), gated output and one
// triangle-bias copy (bias_frag_index_bf16) held as bf16; the mask bias and
// tile flags are shared with the FP32 layout.
struct Bf16ProjArgs {
  const __bf16* x;
  int64_t xs_i;
  int64_t xs_j;
  int64_t xs_h;  // finish: elements between the heads' 32-channel parts of a row (0: adjacent)
  int rows_i;
  int rows_j;
  int span_j;
  const __bf16* ln_w;
  const __bf16* ln_b;
  float eps;
  const __bf16* w[4];
  const __bf16* bias_vec;   // gate bias (prepare) or output bias (finish), nullable
  const __bf16* w_bias;
  float q_scale;      // log2(e) / sqrt(32): the attention's logits are in log2 units
  __bf16* qh;
  __bf16* kh;
  __bf16* vt;
  __bf16* gs;
  __bf16* tri_bias;  // fragment order (bias_frag_index_bf16), scaled by log2(e)
  int np;
  __bf16* out;
  int64_t os_i;
  int64_t os_j;
  int accumulate;  // finish: out = bf16(out + bf16(x W_o^T + b_o))
};

struct Bf16AttnArgs {
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  const float* mbias;
  const uint32_t* tile_flags;
  const __bf16* bias;  // fragment order (bias_frag_index_bf16), scaled by log2(e)
  const __bf16* gate;
  __bf16* out;
  int batch;
  int n;
  int np;
};

hipError_t launch_projection_bf16(int mode, const Bf16ProjArgs& args, hipStream_t stream);
hipError_t launch_attention_bf16(const Bf16AttnArgs& args, hipStream_t stream);

// -------------------------------------------------- triangle multiplication
// Outgoing / incoming triangle multiplicative update, c_z = c_hidden = 128
// (trimul.hip).  Workspace roles: a and b, 128 np^2 floats each (rows of the
// contraction frame; rows >= n unused, keys >= n zero): channel-blocked
// [8][np / 32][np][16][32]; x blocked [n][np / 32][128][32].  np is a
// multiple of 128.
struct TriMulArgs {
  const float* z;
  int64_t zs_i;
  int64_t zs_j;
  const float* mask;  // nullable {0,1} (or any) multiplier of a and b
  int64_t ms_i;
  int64_t ms_j;
  const float* ln_in_w;
  const float* ln_in_b;
  float eps_in;
  const float* w_ab[4];  // a_p, a_g, b_p, b_g: [128 out][128 in]
  const float* b_ab[4];  // nullable
  const float* ln_out_w;
  const float* ln_out_b;
  float eps_out;
  const float* w_z;
  const float* b_z;
  const float* w_g;
  const float* b_g;
  float* pa;
  float* pb;
  float* x;
  // fp16-plane path: [2 (a, b)][128 channels][np rows] running max |a|, |b|
  // over the keys of each (channel, row), as float bits (atomic max)
  uint32_t* rowmax;
  float* out;
  int64_t os_i;
  int64_t os_j;
  int n;
  int np;
  int outgoing;
  int accumulate;  // out = out + u (the in-place residual) instead of u
};

hipError_t launch_trimul(const TriMulArgs& args, hipStream_t stream);

// ---------------------------------------------------------- pair transition
// out = silu(LN(x) W_a^T) * (LN(x) W_b^T) W_o^T over rows x[i][j] at
// x + i*xs_i + j*xs_j (transition.hip).  h is the workspace's [rows padded to
// 128][512] intermediate.
constexpr int kTransitionHidden = 512;

struct TransitionArgs {
  const float* x;
  int64_t xs_i;
  int64_t xs_j;
  int rows_i;
  int rows_j;
  const float* ln_w;  // nullable
  const float* ln_b;  // nullable
  float eps;
  const float* w_a;   // [512][128]
  const float* w_b;   // [512][128]
  const float* w_o;   // [128][512]
  // the 16 chunks' weight planes (fp16 bits, 768 KB), the folded biases
  // [2][512] and the plane exponents (1156 ints, see transition.hip)
  __bf16* planes;
  float* fbias;
  int* exps;
  float* out;
  int64_t os_i;
  int64_t os_j;
  int accumulate;     // out = out + transition(x) instead of transition(x)
};

hipError_t launch_transition(const TransitionArgs& args, hipStream_t stream);

int device_cu_count();

}  // namespace fpx
