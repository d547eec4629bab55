// C-ABI entry points (declared in include/fireprot_amd.h).
//
// Every entry validates sizes and pointers on the host first (status 2 / 3 /
// 4, before any device pointer is touched), then enqueues on the caller's
// stream and returns the launch status.  Nothing here allocates or
// synchronises.
#include "fireprot_amd.h"

#include "common.hpp"
#include "kernels.hpp"

#include <cmath>
#include <mutex>

namespace {

using fpx::round_up;

bool aligned(const void* p, uintptr_t bytes) {
  return p != nullptr && reinterpret_cast<uintptr_t>(p) % bytes == 0;
}
bool aligned_or_null(const void* p, uintptr_t bytes) {
  return p == nullptr || reinterpret_cast<uintptr_t>(p) % bytes == 0;
}

constexpr int kMaxN = 4096;
constexpr int kQueryTile = 128;  // attention query tile: every block extent pads to it

size_t elem_bytes(int dtype) { return dtype == FPX_BF16 ? 2 : 4; }

// Workspace segments of the block, all 256-byte aligned, element size e
// (4 for FPX_F32, 2 for FPX_BF16; the mask bias is always float):
//   qh, kh [n][4][np][32]; vt [n][4][32][np] (BF16: [n][4][np / 32][32][32],
//   tile-major); gs [n][np][128]; og [n][n][128] (BF16: head-major [4][n][n][32]);
//   tri_bias [4][np][np] (FP32: fragment order, twice: as is and scaled by
//   log2(e); BF16: bias_frag_index_bf16, once); mbias [n][np] float;
//   tile flags [n][kTileFlagParts * kTileFlagWords] uint32, then the
//   kMagnitudeWords words of the magnitude record; scales [3][n][4][np / 32]
//   float (the plane layout's per-tile inverse scales of q, k and v^T); FP32
//   only: the constant-mask rows' weights and chunk lists (AttnArgs::const_m,
//   const_l, const_p: kConstListWord words and two lists of
//   ceil(n / kConstRows) chunk indices, l [4][np] float, the planes
//   [4][np / 32][ceil(n / 32)] x 4 KB).
// FP32 blocks hold q, k and v^T in the fp16 plane layout (ProjArgs), in the
// same bytes as FP32 values.
struct BlockWorkspace {
  size_t qh, kh, vt, gs, og, bias, mbias, flags, scales, cw_m, cw_l, cw_p, total;
};

BlockWorkspace block_workspace(int n, int dtype) {
  const size_t np = (size_t)round_up(n, kQueryTile);
  const size_t e = elem_bytes(dtype);
  auto seg = [](size_t bytes) { return (size_t)round_up((int64_t)bytes, 256); };
  const size_t qkv = seg((size_t)n * fpx::kHeads * np * fpx::kHeadDim * e);
  const size_t g = seg((size_t)n * n * fpx::kHidden * e);
  const size_t gate = seg((size_t)n * np * fpx::kHidden * e);
  const size_t bias = seg((size_t)fpx::kHeads * np * np * e * (dtype == FPX_F32 ? 2 : 1));
  const size_t mb = seg((size_t)n * np * sizeof(float));
  const size_t fl = seg(((size_t)n * fpx::kTileFlagParts * fpx::kTileFlagWords +
                        fpx::kMagnitudeWords) * sizeof(uint32_t));
  BlockWorkspace w{};
  w.qh = 0;
  w.kh = w.qh + qkv;
  w.vt = w.kh + qkv;
  w.gs = w.vt + qkv;
  w.og = w.gs + gate;
  w.bias = w.og + g;
  w.mbias = w.bias + bias;
  w.flags = w.mbias + mb;
  w.scales = w.flags + fl;
  const size_t cw_m = w.scales + seg((size_t)3 * n * fpx::kHeads * (np / 32) * sizeof(float));
  w.cw_m = cw_m;
  if (dtype == FPX_F32) {
    const size_t nkt = (size_t)(n + 31) / 32;
    const size_t chunks = (size_t)(n + fpx::kConstRows - 1) / fpx::kConstRows;
    w.cw_l = cw_m + seg((fpx::kConstListWord + 2 * chunks) * sizeof(uint32_t));
    w.cw_p = w.cw_l + seg((size_t)fpx::kHeads * np * sizeof(float));
    w.total = w.cw_p + (size_t)fpx::kHeads * (np / 32) * nkt * 4096;
  } else {
    w.cw_l = w.cw_p = w.total = cw_m;
  }
  return w;
}

bool block_dims_ok(int n, int c, int heads, int head_dim, int dtype) {
  return (dtype == FPX_F32 || dtype == FPX_BF16) && c == fpx::kChannels &&
         heads == fpx::kHeads && head_dim == fpx::kHeadDim && n >= 1 && n <= kMaxN;
}

int status(hipError_t e) { return e == hipSuccess ? FPX_OK : (int)e; }

struct BlockPointers {
  char *qh, *kh, *vt, *gs, *og, *tri;
  float* mbias;
  uint32_t* flags;
  uint32_t* magnitudes;
  float* scales;
  uint32_t* const_m;  // FP32 only (else null), as const_l and const_p
  float* const_l;
  uint8_t* const_p;
  int np;
};

BlockPointers block_pointers(void* workspace, int n, int dtype) {
  const BlockWorkspace ws = block_workspace(n, dtype);
  char* base = static_cast<char*>(workspace);
  BlockPointers p{};
  p.qh = base + ws.qh;
  p.kh = base + ws.kh;
  p.vt = base + ws.vt;
  p.gs = base + ws.gs;
  p.og = base + ws.og;
  p.tri = base + ws.bias;
  p.mbias = reinterpret_cast<float*>(base + ws.mbias);
  p.flags = reinterpret_cast<uint32_t*>(base + ws.flags);
  p.magnitudes = p.flags + (size_t)n * fpx::kTileFlagParts * fpx::kTileFlagWords;
  p.scales = reinterpret_cast<float*>(base + ws.scales);
  if (dtype == FPX_F32) {
    p.const_m = reinterpret_cast<uint32_t*>(base + ws.cw_m);
    p.const_l = reinterpret_cast<float*>(base + ws.cw_l);
    p.const_p = reinterpret_cast<uint8_t*>(base + ws.cw_p);
  }
  p.np = (int)round_up(n, kQueryTile);
  return p;
}

int check_workspace(int n, int dtype, const void* workspace, size_t workspace_bytes) {
  if (!aligned(workspace, 256)) return FPX_ERR_POINTER;
  if (workspace_bytes < block_workspace(n, dtype).total) return FPX_ERR_WORKSPACE;
  return FPX_OK;
}

template <typename T>
T* as(char* p) {
  return reinterpret_cast<T*>(p);
}

// Output projection into dz, or added to dz (accumulate), in z's frame.
int finish_stage(int dtype, const void* w_o, const void* b_o, int n, int ending, void* dz,
                 int64_t dz_stride0, int64_t dz_stride1, void* workspace, size_t workspace_bytes,
                 void* stream, int accumulate) {
  if (!block_dims_ok(n, fpx::kChannels, fpx::kHeads, fpx::kHeadDim, dtype)) return FPX_ERR_DIMS;
  if (ending != 0 && ending != 1) return FPX_ERR_DIMS;
  if (dz_stride0 < 0 || dz_stride1 < 0) return FPX_ERR_DIMS;
  if (!aligned(w_o, 16) || !aligned(dz, 16) || !aligned_or_null(b_o, 2)) return FPX_ERR_POINTER;
  if (dtype == FPX_F32 && !aligned_or_null(b_o, 4)) return FPX_ERR_POINTER;
  if (int rc = check_workspace(n, dtype, workspace, workspace_bytes)) return rc;
  const BlockPointers w = block_pointers(workspace, n, dtype);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t os_i = ending ? dz_stride1 : dz_stride0;
  const int64_t os_j = ending ? dz_stride0 : dz_stride1;
  if (dtype == FPX_BF16) {
    fpx::Bf16ProjArgs o{};
    o.x = as<__bf16>(w.og);  // head-major [4][n][n][32]
    o.xs_i = (int64_t)n * fpx::kHeadDim;
    o.xs_j = fpx::kHeadDim;
    o.xs_h = (int64_t)n * n * fpx::kHeadDim;
    o.rows_i = n;
    o.rows_j = n;
    o.span_j = n;
    o.w[0] = static_cast<const __bf16*>(w_o);
    o.bias_vec = static_cast<const __bf16*>(b_o);
    o.out = static_cast<__bf16*>(dz);
    o.os_i = os_i;
    o.os_j = os_j;
    o.accumulate = accumulate;
    return status(fpx::launch_projection_bf16(fpx::kProjOut, o, s));
  }
  fpx::ProjArgs o{};
  o.x = as<float>(w.og);
  o.xs_i = (int64_t)n * fpx::kHidden;
  o.xs_j = fpx::kHidden;
  o.rows_i = n;
  o.rows_j = n;
  o.span_j = n;
  o.w[0] = static_cast<const float*>(w_o);
  o.b_g = static_cast<const float*>(b_o);
  o.out = static_cast<float*>(dz);
  o.os_i = os_i;
  o.os_j = os_j;
  o.accumulate = accumulate;
  return status(fpx::launch_projection(fpx::kProjOut, o, s));
}

// The whole block: prepare, attend, then the output projection written to or
// (accumulate) added to dz.
int block_impl(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1, const float* mask,
               int64_t m_stride0, int64_t m_stride1, const void* ln_w, const void* ln_b,
               float eps, const void* w_qkvg, const void* b_g, const void* w_bias,
               const void* w_o, const void* b_o, float mask_inf, int n, int c, int heads,
               int head_dim, int ending, void* dz, int64_t dz_stride0, int64_t dz_stride1,
               void* workspace, size_t workspace_bytes, void* stream, int accumulate) {
  if (!block_dims_ok(n, c, heads, head_dim, dtype)) return FPX_ERR_DIMS;
  if (ending != 0 && ending != 1) return FPX_ERR_DIMS;
  if (dz_stride0 < 0 || dz_stride1 < 0) return FPX_ERR_DIMS;
  if (!aligned(w_o, 16) || !aligned(dz, 16) || !aligned_or_null(b_o, 2)) return FPX_ERR_POINTER;
  if (dtype == FPX_F32 && !aligned_or_null(b_o, 4)) return FPX_ERR_POINTER;
  int rc = fpx_tri_attn_prepare(dtype, z, z_stride0, z_stride1, mask, m_stride0, m_stride1, ln_w,
                                ln_b, eps, w_qkvg, b_g, w_bias, mask_inf, n, ending, workspace,
                                workspace_bytes, stream);
  if (rc) return rc;
  rc = fpx_tri_attn_attend(dtype, n, workspace, workspace_bytes, stream);
  if (rc) return rc;
  return finish_stage(dtype, w_o, b_o, n, ending, dz, dz_stride0, dz_stride1, workspace,
                      workspace_bytes, stream, accumulate);
}

// Workspace of fpx_attn_strided, 256-byte aligned segments:
//   bias [4][np][np] float in fragment order, twice (as is, scaled by log2(e));
//   mbias [batch][np] float; tile flags [batch][kTileFlagParts * kTileFlagWords] uint32;
//   q, k and v planes [batch][4] slices of np * 128 bytes each; their scales
//   [3][batch][4][np / 32] float; the magnitude record (kMagnitudeWords) and
//   the staging's per-work-group maxima (3 floats per group of 4 tiles).
struct StridedWorkspace {
  size_t bias, bias_l2, mbias, flags, qp, kp, vp, scales, magnitudes, partial, total;
};

StridedWorkspace strided_workspace(int batch, int n) {
  const size_t np = (size_t)round_up(n, kQueryTile);
  auto seg = [](size_t bytes) { return (size_t)round_up((int64_t)bytes, 256); };
  StridedWorkspace w{};
  w.bias = 0;
  w.bias_l2 = seg((size_t)fpx::kHeads * np * np * sizeof(float));
  w.mbias = 2 * w.bias_l2;
  w.flags = w.mbias + seg((size_t)batch * np * sizeof(float));
  w.qp = w.flags + seg((size_t)batch * fpx::kTileFlagParts * fpx::kTileFlagWords *
                        sizeof(uint32_t));
  const size_t planes = seg((size_t)batch * fpx::kHeads * np * 128);
  w.kp = w.qp + planes;
  w.vp = w.kp + planes;
  w.scales = w.vp + planes;
  w.magnitudes = w.scales + seg(3 * (size_t)batch * fpx::kHeads * (np / 32) * sizeof(float));
  w.partial = w.magnitudes + seg(fpx::kMagnitudeWords * sizeof(uint32_t));
  const size_t groups = (3 * (size_t)batch * fpx::kHeads * (np / 32) + 3) / 4;
  w.total = w.partial + seg(3 * groups * sizeof(float));
  return w;
}

// Workspace of fpx_tri_mul, 256-byte aligned segments: a and b, 128 np^2
// floats each (channel-blocked [8][np / 32][np][16][32]); x blocked
// [n][np / 32][128][32] float; the row maxima of a and b [2][128][np] uint32.
struct TriMulWorkspace {
  size_t pa, pb, x, rowmax, total;
};

TriMulWorkspace trimul_workspace(int n) {
  const size_t np = (size_t)round_up(n, kQueryTile);
  auto seg = [](size_t bytes) { return (size_t)round_up((int64_t)bytes, 256); };
  TriMulWorkspace w{};
  w.pa = 0;
  w.pb = seg((size_t)fpx::kChannels * np * np * sizeof(float));
  w.x = 2 * w.pb;
  w.rowmax = w.x + seg((size_t)n * np * fpx::kChannels * sizeof(float));
  w.total = w.rowmax + seg(2 * (size_t)fpx::kChannels * np * sizeof(uint32_t));
  return w;
}

// Workspace of fpx_transition: the fused kernel's weight planes (16 chunks
// of 48 KB), folded biases [2][512] float and its plane exponents (5 KB),
// whatever the number of rows.
constexpr size_t kTransitionPlanesBytes = 16 * 48 * 1024;
constexpr size_t kTransitionFusedBytes = kTransitionPlanesBytes + 2 * 512 * sizeof(float) + 5120;
size_t transition_workspace(int64_t /*rows*/) { return kTransitionFusedBytes; }

// A [batch][4][n][32] operand with channel stride 1 the strided attention
// kernel can read: non-negative strides that keep 16-byte rows aligned, and
// (for K and V) a (b, h) slice that a buffer descriptor covers.
bool strided_operand_ok(const int64_t s[3], int n, bool slice) {
  for (int d = 0; d < 3; ++d)
    if (s[d] < 0 || s[d] % 4 != 0) return false;
  return !slice || ((int64_t)(n - 1) * s[2] + fpx::kHeadDim) * 4 < 0x7fffffffll;
}

// Scratch of fpx_tri_attn_block_noalloc: the block workspace of N <= 128
// (block_workspace(128, FPX_F32).total = 42565888 bytes, every smaller N and
// the BF16 block need less), held by each GPU the library runs on until the
// process ends.  Host code never passes `scratch` itself (its host-side name
// is no device address): it uses the per-device address that
// hipGetSymbolAddress returns.
constexpr int kNoAllocMaxN = 128;
constexpr size_t kNoAllocScratchBytes = 41u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device with
// that device current; nullptr (and the HIP status in *err) on failure.
void* device_scratch(hipError_t* err) {
  int device = 0;
  *err = hipGetDevice(&device);
  if (*err != hipSuccess) return nullptr;
  if (device < 0 || device >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    scratch_ptr[device] = ptr;
  }
  return scratch_ptr[device];
}

}  // namespace

extern "C" {

int fpx_abi_version(void) { return FPX_ABI_VERSION; }

size_t fpx_tri_attn_workspace_bytes(int n, int c, int heads, int head_dim, int dtype) {
  if (!block_dims_ok(n, c, heads, head_dim, dtype)) return 0;
  return block_workspace(n, dtype).total;
}

int fpx_tri_attn_prepare(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                         const float* mask, int64_t m_stride0, int64_t m_stride1,
                         const void* ln_w, const void* ln_b, float eps, const void* w_qkvg,
                         const void* b_g, const void* w_bias, float mask_inf, int n, int ending,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (!block_dims_ok(n, fpx::kChannels, fpx::kHeads, fpx::kHeadDim, dtype)) return FPX_ERR_DIMS;
  if (ending != 0 && ending != 1) return FPX_ERR_DIMS;
  // rows must be 16-byte aligned: 4 floats or 8 bf16
  const int64_t row_align = dtype == FPX_BF16 ? 8 : 4;
  if (z_stride0 % row_align || z_stride1 % row_align || z_stride0 < 0 || z_stride1 < 0)
    return FPX_ERR_DIMS;
  if (m_stride0 < 0 || m_stride1 < 0) return FPX_ERR_DIMS;
  if (!(eps >= 0.0f) || !std::isfinite(mask_inf)) return FPX_ERR_DIMS;
  if (!aligned(z, 16) || !aligned(w_qkvg, 16) || !aligned(w_bias, 16)) return FPX_ERR_POINTER;
  if (!aligned_or_null(mask, 4) || !aligned_or_null(ln_w, 8) || !aligned_or_null(ln_b, 8) ||
      !aligned_or_null(b_g, 4))
    return FPX_ERR_POINTER;
  if (int rc = check_workspace(n, dtype, workspace, workspace_bytes)) return rc;

  const hipStream_t s = static_cast<hipStream_t>(stream);
  const BlockPointers w = block_pointers(workspace, n, dtype);
  // x-frame strides: the ending node reads x[i][j] = z[j][i] (and the mask alike).
  const int64_t xs_i = ending ? z_stride1 : z_stride0;
  const int64_t xs_j = ending ? z_stride0 : z_stride1;
  const int64_t ms_i = ending ? m_stride1 : m_stride0;
  const int64_t ms_j = ending ? m_stride0 : m_stride1;

  hipError_t e = fpx::launch_mask_bias(mask, ms_i, ms_j, n, w.np, mask_inf, w.mbias, w.flags,
                                       w.tri, dtype == FPX_BF16, w.magnitudes, s);
  if (e != hipSuccess) return status(e);

  const float q_scale = 1.0f / std::sqrt((float)fpx::kHeadDim);
  const int64_t wstride = (int64_t)fpx::kHidden * fpx::kChannels;
  if (dtype == FPX_BF16) {
    const __bf16* wq = static_cast<const __bf16*>(w_qkvg);
    fpx::Bf16ProjArgs p{};
    p.x = static_cast<const __bf16*>(z);
    p.xs_i = xs_i;
    p.xs_j = xs_j;
    p.rows_i = n;
    p.rows_j = n;
    p.span_j = w.np;
    p.ln_w = static_cast<const __bf16*>(ln_w);
    p.ln_b = static_cast<const __bf16*>(ln_b);
    p.eps = eps;
    for (int g = 0; g < 4; ++g) p.w[g] = wq + g * wstride;
    p.bias_vec = static_cast<const __bf16*>(b_g);
    p.w_bias = static_cast<const __bf16*>(w_bias);
    // BF16 attention logits come out of the matrix cores in log2 units: q
    // and the triangle bias are stored scaled by log2(e).
    p.q_scale = q_scale * fpx::kLog2e;
    p.qh = as<__bf16>(w.qh);
    p.kh = as<__bf16>(w.kh);
    p.vt = as<__bf16>(w.vt);
    p.gs = as<__bf16>(w.gs);
    p.tri_bias = as<__bf16>(w.tri);
    p.np = w.np;
    return status(fpx::launch_projection_bf16(fpx::kProjBlock, p, s));
  }
  const float* wq = static_cast<const float*>(w_qkvg);
  fpx::ProjArgs p{};
  p.x = static_cast<const float*>(z);
  p.xs_i = xs_i;
  p.xs_j = xs_j;
  p.rows_i = n;
  p.rows_j = n;
  p.span_j = w.np;
  p.ln_w = static_cast<const float*>(ln_w);
  p.ln_b = static_cast<const float*>(ln_b);
  p.eps = eps;
  for (int g = 0; g < 4; ++g) p.w[g] = wq + g * wstride;
  p.b_g = static_cast<const float*>(b_g);
  p.w_bias = static_cast<const float*>(w_bias);
  p.q_scale = q_scale;
  p.qh = as<float>(w.qh);
  p.kh = as<float>(w.kh);
  p.vt = as<float>(w.vt);
  p.gs = as<float>(w.gs);
  p.tri_bias = as<float>(w.tri);
  p.tri_bias_l2 = as<float>(w.tri) + (size_t)fpx::kHeads * w.np * w.np;
  p.magnitudes = w.magnitudes;
  p.scales = w.scales;
  p.np = w.np;
  e = fpx::launch_projection(fpx::kProjBlock, p, s);
  if (e != hipSuccess) return status(e);
  // the fast softmax reads the log2 bias relative to each query's reference
  return status(fpx::launch_bias_reference(w.flags, n, n, w.np, p.tri_bias_l2, w.magnitudes, s));
}

int fpx_tri_attn_attend(int dtype, int n, void* workspace, size_t workspace_bytes, void* stream) {
  if (!block_dims_ok(n, fpx::kChannels, fpx::kHeads, fpx::kHeadDim, dtype)) return FPX_ERR_DIMS;
  if (int rc = check_workspace(n, dtype, workspace, workspace_bytes)) return rc;
  const BlockPointers w = block_pointers(workspace, n, dtype);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == FPX_BF16) {
    fpx::Bf16AttnArgs a{};
    a.q = as<__bf16>(w.qh);
    a.k = as<__bf16>(w.kh);
    a.v = as<__bf16>(w.vt);
    a.mbias = w.mbias;
    a.tile_flags = w.flags;
    a.bias = as<__bf16>(w.tri);
    a.gate = as<__bf16>(w.gs);
    a.out = as<__bf16>(w.og);
    a.batch = n;
    a.n = n;
    a.np = w.np;
    return status(fpx::launch_attention_bf16(a, s));
  }
  fpx::AttnArgs a{};
  a.q = as<float>(w.qh);
  a.k = as<float>(w.kh);
  a.v = as<float>(w.vt);
  a.mbias = w.mbias;
  a.mb_stride = w.np;
  a.bias = as<float>(w.tri);
  a.bias_l2 = as<float>(w.tri) + (size_t)fpx::kHeads * w.np * w.np;
  a.bias_stride = w.np;
  a.bias_rows = w.np;
  a.gate = as<float>(w.gs);
  a.out = as<float>(w.og);
  a.tile_flags = w.flags;
  a.magnitudes = w.magnitudes;
  a.scales = w.scales;
  a.const_m = w.const_m;
  a.const_l = w.const_l;
  a.const_p = w.const_p;
  a.batch = n;
  a.n = n;
  a.np = w.np;
  return status(fpx::launch_attention_split(fpx::kAttnBlock, a, s));
}

int fpx_tri_attn_finish(int dtype, const void* w_o, const void* b_o, int n, int ending, void* dz,
                        int64_t dz_stride0, int64_t dz_stride1, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return finish_stage(dtype, w_o, b_o, n, ending, dz, dz_stride0, dz_stride1, workspace,
                      workspace_bytes, stream, 0);
}

int fpx_tri_attn_block(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                       const float* mask, int64_t m_stride0, int64_t m_stride1,
                       const void* ln_w, const void* ln_b, float eps, const void* w_qkvg,
                       const void* b_g, const void* w_bias, const void* w_o, const void* b_o,
                       float mask_inf, int n, int c, int heads, int head_dim, int ending,
                       void* dz, int64_t dz_stride0, int64_t dz_stride1, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return block_impl(dtype, z, z_stride0, z_stride1, mask, m_stride0, m_stride1, ln_w, ln_b, eps,
                    w_qkvg, b_g, w_bias, w_o, b_o, mask_inf, n, c, heads, head_dim, ending, dz,
                    dz_stride0, dz_stride1, workspace, workspace_bytes, stream, 0);
}

int fpx_tri_attn_block_noalloc(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                               const float* mask, int64_t m_stride0, int64_t m_stride1,
                               const void* ln_w, const void* ln_b, float eps, const void* w_qkvg,
                               const void* b_g, const void* w_bias, const void* w_o,
                               const void* b_o, float mask_inf, int n, int c, int heads,
                               int head_dim, int ending, void* dz, int64_t dz_stride0,
                               int64_t dz_stride1, void* stream) {
  if (!block_dims_ok(n, c, heads, head_dim, dtype) || n > kNoAllocMaxN) return FPX_ERR_DIMS;
  if (block_workspace(n, dtype).total > kNoAllocScratchBytes) return FPX_ERR_DIMS;
  hipError_t err = hipSuccess;
  void* ws = device_scratch(&err);
  if (ws == nullptr) return status(err);
  return block_impl(dtype, z, z_stride0, z_stride1, mask, m_stride0, m_stride1, ln_w, ln_b, eps,
                    w_qkvg, b_g, w_bias, w_o, b_o, mask_inf, n, c, heads, head_dim, ending, dz,
                    dz_stride0, dz_stride1, ws, kNoAllocScratchBytes, stream, 0);
}

int fpx_tri_attn_block_residual(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                                const float* mask, int64_t m_stride0, int64_t m_stride1,
                                const void* ln_w, const void* ln_b, float eps,
                                const void* w_qkvg, const void* b_g, const void* w_bias,
                                const void* w_o, const void* b_o, float mask_inf, int n, int c,
                                int heads, int head_dim, int ending, void* z_out,
                                int64_t out_stride0, int64_t out_stride1, void* workspace,
                                size_t workspace_bytes, void* stream) {
  if (z_out == z && (out_stride0 != z_stride0 || out_stride1 != z_stride1)) return FPX_ERR_DIMS;
  return block_impl(dtype, z, z_stride0, z_stride1, mask, m_stride0, m_stride1, ln_w, ln_b, eps,
                    w_qkvg, b_g, w_bias, w_o, b_o, mask_inf, n, c, heads, head_dim, ending, z_out,
                    out_stride0, out_stride1, workspace, workspace_bytes, stream, 1);
}

int fpx_attn_core_masked(const float* q, const float* k, const float* v, const float* mask_bias,
                         int64_t mask_bias_stride, const float* bias, int64_t bias_row_stride,
                         float* out, int batch, int n, void* stream) {
  if (batch < 1 || n < 1 || n % 4 != 0 || n > 65536) return FPX_ERR_DIMS;
  if (bias_row_stride < n || bias_row_stride % 4 != 0) return FPX_ERR_DIMS;
  if (mask_bias != nullptr && mask_bias_stride < 0) return FPX_ERR_DIMS;
  if ((int64_t)batch * fpx::kHeads * (round_up(n, kQueryTile) / kQueryTile) > 0x7fffffffll)
    return FPX_ERR_DIMS;
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(bias, 16) ||
      !aligned(out, 16))
    return FPX_ERR_POINTER;
  if (!aligned_or_null(mask_bias, 4)) return FPX_ERR_POINTER;
  fpx::AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.mbias = mask_bias;
  a.mb_stride = mask_bias_stride;
  a.bias = bias;
  a.bias_stride = bias_row_stride;
  a.bias_rows = n;
  a.gate = nullptr;
  a.out = out;
  a.batch = batch;
  a.n = n;
  a.np = n;
  return status(fpx::launch_attention(fpx::kAttnHeadLast, a, static_cast<hipStream_t>(stream)));
}

int fpx_attn_core(float* q, float* k, float* v, float* bias, float* out, int batch, int n,
                  void* stream) {
  return fpx_attn_core_masked(q, k, v, nullptr, 0, bias, n, out, batch, n, stream);
}

int ck_attention(float* q, float* k, float* v, float* bias, float* out, int batch, int n,
                 void* stream) {
  if (!((batch == 1000 && n == 1000) || (batch == 512 && n == 1536))) return FPX_ERR_DIMS;
  // the reference's physical bias row stride (fireprot_ck_attention.cpp:37)
  return fpx_attn_core_masked(q, k, v, nullptr, 0, bias, n == 1536 ? n + 16 : n, out, batch, n,
                              stream);
}

int ck_attention_exact1536(float* q, float* k, float* v, float* bias, float* out, int batch,
                           int n, void* stream) {
  if (batch != 512 || n != 1536) return FPX_ERR_DIMS;
  return fpx_attn_core_masked(q, k, v, nullptr, 0, bias, 1552, out, batch, n, stream);
}

int ck_attention_vector_bias1000(float* q, float* k, float* v, float* bias, float* out,
                                 int batch, int n, void* stream) {
  if (batch != 1000 || n != 1000) return FPX_ERR_DIMS;
  return fpx_attn_core_masked(q, k, v, nullptr, 0, bias, 1000, out, batch, n, stream);
}

size_t fpx_attn_strided_workspace_bytes(int batch, int n) {
  if (batch < 1 || n < 1 || n > kMaxN) return 0;
  return strided_workspace(batch, n).total;
}

int fpx_attn_strided(const float* q, int64_t q_sb, int64_t q_sh, int64_t q_sn, const float* k,
                     int64_t k_sb, int64_t k_sh, int64_t k_sn, const float* v, int64_t v_sb,
                     int64_t v_sh, int64_t v_sn, const float* mask_bias, int64_t m_sb,
                     int64_t m_sk, const float* bias, int64_t b_sh, int64_t b_sq, int64_t b_sk,
                     float* out, int64_t o_sb, int64_t o_sh, int64_t o_sn, int batch, int n,
                     void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 1 || n < 1 || n > kMaxN) return FPX_ERR_DIMS;
  const int np = (int)round_up(n, kQueryTile);
  if ((int64_t)batch * fpx::kHeads * (np / kQueryTile) > 0x7fffffffll) return FPX_ERR_DIMS;
  fpx::AttnArgs a{};
  const int64_t qs[3] = {q_sb, q_sh, q_sn}, ks[3] = {k_sb, k_sh, k_sn};
  const int64_t vs[3] = {v_sb, v_sh, v_sn}, os[3] = {o_sb, o_sh, o_sn};
  if (!strided_operand_ok(qs, n, false) || !strided_operand_ok(ks, n, true) ||
      !strided_operand_ok(vs, n, true) || !strided_operand_ok(os, n, false))
    return FPX_ERR_DIMS;
  if (m_sb < 0 || m_sk < 0 || b_sh < 0 || b_sq < 0 || b_sk < 0) return FPX_ERR_DIMS;
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16))
    return FPX_ERR_POINTER;
  if (!aligned_or_null(mask_bias, 4) || !aligned_or_null(bias, 4)) return FPX_ERR_POINTER;
  if (!aligned(workspace, 256)) return FPX_ERR_POINTER;
  const StridedWorkspace ws = strided_workspace(batch, n);
  if (workspace_bytes < ws.total) return FPX_ERR_WORKSPACE;
  char* base = static_cast<char*>(workspace);
  float* frag = as<float>(base + ws.bias);
  float* frag_l2 = as<float>(base + ws.bias_l2);
  float* mbias = as<float>(base + ws.mbias);
  uint32_t* flags = as<uint32_t>(base + ws.flags);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* mag = as<uint32_t>(base + ws.magnitudes);
  hipError_t e =
      fpx::launch_mask_rows(mask_bias, m_sb, m_sk, batch, n, np, mbias, flags, mag, st);
  if (e != hipSuccess) return status(e);
  e = fpx::launch_stage_bias(bias, b_sh, b_sq, b_sk, n, np, frag, frag_l2, mag, st);
  if (e != hipSuccess) return status(e);
  a.q = q;
  a.k = k;
  a.v = v;
  a.mbias = mbias;
  a.mb_stride = np;
  a.bias = frag;
  a.bias_l2 = frag_l2;
  a.out = out;
  a.tile_flags = flags;
  for (int d = 0; d < 3; ++d) {
    a.qs[d] = qs[d];
    a.ks[d] = ks[d];
    a.vs[d] = vs[d];
    a.os[d] = os[d];
  }
  a.batch = batch;
  a.n = n;
  a.np = np;
  // q, k, v into the plane layout, then the block attention's kernel on it;
  // the magnitude record enables its trailing masked-tile skip
  void* qp = base + ws.qp;
  void* kp = base + ws.kp;
  void* vp = base + ws.vp;
  float* scales = as<float>(base + ws.scales);
  e = fpx::launch_stage_planes(a, qp, kp, vp, scales, as<float>(base + ws.partial), mag, st);
  if (e != hipSuccess) return status(e);
  a.q = static_cast<const float*>(qp);
  a.k = static_cast<const float*>(kp);
  a.v = static_cast<const float*>(vp);
  a.scales = scales;
  a.magnitudes = mag;
  return status(fpx::launch_attention_split(fpx::kAttnStaged, a, st));
}

size_t fpx_tri_mul_workspace_bytes(int n, int c_z, int c_hidden) {
  if (n < 1 || n > kMaxN || c_z != fpx::kChannels || c_hidden != fpx::kHidden) return 0;
  return trimul_workspace(n).total;
}

int fpx_tri_mul(const float* z, int64_t z_stride0, int64_t z_stride1, const float* mask,
                int64_t m_stride0, int64_t m_stride1, const float* ln_in_w, const float* ln_in_b,
                float eps_in, const float* w_abpg, const float* b_abpg, const float* ln_out_w,
                const float* ln_out_b, float eps_out, const float* w_z, const float* b_z,
                const float* w_g, const float* b_g, int n, int c_z, int c_hidden, int outgoing,
                int accumulate, float* out, int64_t out_stride0, int64_t out_stride1,
                void* workspace, size_t workspace_bytes, void* stream) {
  if (n < 1 || n > kMaxN || c_z != fpx::kChannels || c_hidden != fpx::kHidden) return FPX_ERR_DIMS;
  if ((outgoing != 0 && outgoing != 1) || (accumulate != 0 && accumulate != 1)) return FPX_ERR_DIMS;
  if (z_stride0 < 0 || z_stride1 < 0 || z_stride0 % 4 || z_stride1 % 4) return FPX_ERR_DIMS;
  if (out_stride0 < 0 || out_stride1 < 0) return FPX_ERR_DIMS;
  if (mask != nullptr && (m_stride0 < 0 || m_stride1 < 0)) return FPX_ERR_DIMS;
  if (!(eps_in >= 0.0f) || !(eps_out >= 0.0f)) return FPX_ERR_DIMS;
  // out may be z itself (same strides: each pair row is read before it is
  // written, by the same tile); any other overlap is unsupported.
  if (out == z && (out_stride0 != z_stride0 || out_stride1 != z_stride1)) return FPX_ERR_DIMS;
  if (!aligned(z, 16) || !aligned(w_abpg, 16) || !aligned(w_z, 16) || !aligned(w_g, 16) ||
      !aligned(out, 4))
    return FPX_ERR_POINTER;
  if (!aligned_or_null(mask, 4) || !aligned_or_null(b_abpg, 4) || !aligned_or_null(ln_in_w, 8) ||
      !aligned_or_null(ln_in_b, 8) || !aligned_or_null(ln_out_w, 8) ||
      !aligned_or_null(ln_out_b, 8) || !aligned_or_null(b_z, 4) || !aligned_or_null(b_g, 4))
    return FPX_ERR_POINTER;
  if (!aligned(workspace, 256)) return FPX_ERR_POINTER;
  const TriMulWorkspace ws = trimul_workspace(n);
  if (workspace_bytes < ws.total) return FPX_ERR_WORKSPACE;
  char* base = static_cast<char*>(workspace);
  fpx::TriMulArgs a{};
  a.z = static_cast<const float*>(z);
  a.zs_i = z_stride0;
  a.zs_j = z_stride1;
  a.mask = mask;
  a.ms_i = m_stride0;
  a.ms_j = m_stride1;
  a.ln_in_w = ln_in_w;
  a.ln_in_b = ln_in_b;
  a.eps_in = eps_in;
  for (int g = 0; g < 4; ++g) {
    a.w_ab[g] = w_abpg + (int64_t)g * fpx::kHidden * fpx::kChannels;
    a.b_ab[g] = b_abpg ? b_abpg + (int64_t)g * fpx::kHidden : nullptr;
  }
  a.ln_out_w = ln_out_w;
  a.ln_out_b = ln_out_b;
  a.eps_out = eps_out;
  a.w_z = w_z;
  a.b_z = b_z;
  a.w_g = w_g;
  a.b_g = b_g;
  a.pa = as<float>(base + ws.pa);
  a.pb = as<float>(base + ws.pb);
  a.x = as<float>(base + ws.x);
  a.rowmax = as<uint32_t>(base + ws.rowmax);
  a.out = out;
  a.os_i = out_stride0;
  a.os_j = out_stride1;
  a.n = n;
  a.np = (int)round_up(n, kQueryTile);
  a.outgoing = outgoing;
  a.accumulate = accumulate;
  return status(fpx::launch_trimul(a, static_cast<hipStream_t>(stream)));
}

size_t fpx_transition_workspace_bytes(int64_t rows_i, int64_t rows_j, int c, int expansion) {
  if (rows_i < 0 || rows_j < 0 || rows_i > 0x7fffffff || rows_j > 0x7fffffff ||
      c != fpx::kChannels || expansion * c != fpx::kTransitionHidden)
    return 0;
  const int64_t rows = rows_i * rows_j;
  if (rows < 1 || (rows_j + 31) / 32 * rows_i > 0x7fffffffll) return 0;
  return transition_workspace(rows);
}

int fpx_transition(const float* x, int64_t rows_i, int64_t rows_j, int64_t x_stride_i,
                   int64_t x_stride_j, const float* ln_w, const float* ln_b, float eps,
                   const float* w_a, const float* w_b, const float* w_o, int c, int expansion,
                   int accumulate, float* out, int64_t out_stride_i, int64_t out_stride_j,
                   void* workspace, size_t workspace_bytes, void* stream) {
  const size_t need = fpx_transition_workspace_bytes(rows_i, rows_j, c, expansion);
  if (need == 0) return FPX_ERR_DIMS;
  if (accumulate != 0 && accumulate != 1) return FPX_ERR_DIMS;
  // x rows are read as 16-byte vectors: strides in multiples of 4 floats
  if (x_stride_i < 0 || x_stride_j < 0 || x_stride_i % 4 || x_stride_j % 4) return FPX_ERR_DIMS;
  if (out_stride_i < 0 || out_stride_j < 0) return FPX_ERR_DIMS;
  if (!(eps >= 0.0f)) return FPX_ERR_DIMS;
  if (out == x && (out_stride_i != x_stride_i || out_stride_j != x_stride_j)) return FPX_ERR_DIMS;
  if (!aligned(x, 16) || !aligned(w_a, 16) || !aligned(w_b, 16) || !aligned(w_o, 16) ||
      !aligned(out, 4) || !aligned_or_null(ln_w, 8) || !aligned_or_null(ln_b, 8))
    return FPX_ERR_POINTER;
  if (!aligned(workspace, 256)) return FPX_ERR_POINTER;
  if (workspace_bytes < need) return FPX_ERR_WORKSPACE;
  fpx::TransitionArgs a{};
  a.x = x;
  a.xs_i = x_stride_i;
  a.xs_j = x_stride_j;
  a.rows_i = (int)rows_i;
  a.rows_j = (int)rows_j;
  a.ln_w = ln_w;
  a.ln_b = ln_b;
  a.eps = eps;
  a.w_a = w_a;
  a.w_b = w_b;
  a.w_o = w_o;
  a.planes = static_cast<__bf16*>(workspace);
  a.fbias = as<float>(static_cast<char*>(workspace) + kTransitionPlanesBytes);
  a.exps = as<int>(static_cast<char*>(workspace) + kTransitionPlanesBytes + 2 * 512 * sizeof(float));
  a.out = out;
  a.os_i = out_stride_i;
  a.os_j = out_stride_j;
  a.accumulate = accumulate;
  return status(fpx::launch_transition(a, static_cast<hipStream_t>(stream)));
}

int fpx_layer_norm_c128(const float* x, int64_t rows_i, int64_t rows_j, int64_t stride_i,
                        int64_t stride_j, const float* w, const float* b, float eps, float* y,
                        void* stream) {
  if (rows_i < 0 || rows_j < 0 || stride_i < 0 || stride_j < 0) return FPX_ERR_DIMS;
  if (stride_i % 2 || stride_j % 2 || !(eps >= 0.0f)) return FPX_ERR_DIMS;
  if (!aligned(x, 8) || !aligned(y, 8) || !aligned_or_null(w, 8) || !aligned_or_null(b, 8))
    return FPX_ERR_POINTER;
  return status(fpx::launch_layer_norm(x, rows_i, rows_j, stride_i, stride_j, w, b, eps, y,
                                       static_cast<hipStream_t>(stream)));
}

int fpx_qkv_projection(const float* x, int64_t rows, const float* wq, const float* wk,
                       const float* wv, float* out, void* stream) {
  if (rows < 0 || rows > 0x7fffffffll) return FPX_ERR_DIMS;
  if (!aligned(x, 16) || !aligned(wq, 16) || !aligned(wk, 16) || !aligned(wv, 16) ||
      !aligned(out, 16))
    return FPX_ERR_POINTER;
  fpx::ProjArgs p{};
  p.x = x;
  p.xs_i = 0;
  p.xs_j = fpx::kChannels;
  p.rows_i = 1;
  p.rows_j = (int)rows;
  p.span_j = (int)rows;
  p.w[0] = wq;
  p.w[1] = wk;
  p.w[2] = wv;
  p.w[3] = wv;
  p.q_scale = 1.0f / std::sqrt((float)fpx::kHeadDim);
  p.out = out;
  return status(fpx::launch_projection(fpx::kProjQkv, p, static_cast<hipStream_t>(stream)));
}

int fpx_sigmoid_mul_out(const float* gate, const float* value, float* out, int64_t count,
                        void* stream) {
  if (count < 0 || count % 4 != 0) return FPX_ERR_DIMS;
  if (!aligned(gate, 16) || !aligned(value, 16) || !aligned(out, 16)) return FPX_ERR_POINTER;
  return status(fpx::launch_sigmoid_mul(gate, value, out, count / 4,
                                        static_cast<hipStream_t>(stream)));
}

int fpx_split_planes(const float* x, int64_t count, uint16_t* planes, void* stream) {
  if (count < 0 || count % 8 != 0) return FPX_ERR_DIMS;
  if (!aligned(x, 16) || !aligned(planes, 16)) return FPX_ERR_POINTER;
  return status(fpx::launch_split_planes(x, planes, count / 8, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
