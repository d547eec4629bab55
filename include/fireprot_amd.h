/*
 * fireprot_amd -- C ABI of the MI355X (gfx950) triangle-attention block.
 *
 * Plain pointers and sizes only: no torch or HIP types appear in the
 * signatures (streams are passed as void* hipStream_t).  Every entry point
 *   - validates its arguments on the host before any device pointer is
 *     dereferenced,
 *   - enqueues its kernels on the caller's stream for the caller's current
 *     device and returns without synchronising,
 *   - allocates nothing: outputs and workspace belong to the caller,
 *   - leaves its inputs unmodified,
 *   - is stateless and reentrant.
 *
 * Status codes follow the reference C ABI (kernels/amd/fireprot_ck_attention.cpp:
 * 35, 47, 106-108): 0 success; 2 unsupported sizes or layout; 3 a null or
 * misaligned pointer; 4 workspace too small; any other value is the
 * hipError_t of the failed launch.
 *
 * Paths in citations are relative to the reference checkout.
 */
#ifndef FIREPROT_AMD_H
#define FIREPROT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FPX_ABI_VERSION 1

#define FPX_OK 0
#define FPX_ERR_DIMS 2
#define FPX_ERR_POINTER 3
#define FPX_ERR_WORKSPACE 4

#define FPX_F32 0
#define FPX_BF16 1

/* ABI version of the loaded library (FPX_ABI_VERSION).
 * Replaces the reference bridge's ABI_VERSION probe
 * (crates/fireprot-bridge/src/lib.rs:151). */
int fpx_abi_version(void);

/* Bytes of device workspace fpx_tri_attn_block needs for an n x n pair
 * representation; 0 for unsupported sizes.  No reference counterpart: the
 * reference's native path allocates per call (docs/protenix-long1536.md:60-66). */
size_t fpx_tri_attn_workspace_bytes(int n, int c, int heads, int head_dim, int dtype);

/* The whole triangle-attention block (z[N,N,C], mask[N,N]) -> dz[N,N,C]:
 * pair LayerNorm, fused q/k/v/gate projection, triangle-bias projection,
 * row-wise attention with additive mask bias and pair bias, sigmoid gate and
 * output projection.  Replaces the Protenix module call
 * TriangleAttention.forward (patches/protenix/0005-*.patch:14-48, with
 * Attention.forward from patches/protenix/0002-*.patch:31-58) and AtlasFold's
 * triangle_attention(module, z, mask, ending) (python/fireprot/adapters/
 * atlasfold/runtime.py:32-71).  The residual z += dz stays with the caller
 * (patches/protenix/0006-*.patch:25).
 *
 *   z        [n][n][c] with element strides (z_stride0, z_stride1, 1)
 *   mask     nullable float {0,1} [n][n], strides (m_stride0, m_stride1);
 *            null omits the mask bias (patch 0005:18-19, 36-39)
 *   ln_w/b   nullable LayerNorm affine [c]; eps as in the module (1e-5)
 *   w_qkvg   [4*heads*head_dim][c]: W_q, W_k, W_v, W_g stacked, each torch
 *            nn.Linear [out, in]
 *   b_g      nullable gate bias [heads*head_dim]
 *   w_bias   [heads][c] triangle-bias projection (no bias term)
 *   w_o      [c][heads*head_dim]; b_o nullable [c]
 *   mask_inf the module's inf (1e9)
 *   ending   0: starting node; 1: ending node, dz = T(block(T(z), T(mask)))
 *            read and written through strides, with no transposed copies
 *   dz       [n][n][c] with strides (dz_stride0, dz_stride1, 1), z's frame
 *   workspace at least fpx_tri_attn_workspace_bytes(...) bytes, 256-aligned
 * Supported: dtype FPX_F32, c = 128, heads = 4, head_dim = 32, 1 <= n <= 4096.
 */
int fpx_tri_attn_block(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                       const float* mask, int64_t m_stride0, int64_t m_stride1,
                       const void* ln_w, const void* ln_b, float eps, const void* w_qkvg,
                       const void* b_g, const void* w_bias, const void* w_o, const void* b_o,
                       float mask_inf, int n, int c, int heads, int head_dim, int ending,
                       void* dz, int64_t dz_stride0, int64_t dz_stride1, void* workspace,
                       size_t workspace_bytes, void* stream);

/* The block as a residual update: z_out += dz, with dz the result
 * fpx_tri_attn_block would write, rounded first and then added (the native
 * z += dz).  z_out may be z itself (same pointer and strides: an in-place
 * update, safe because z is read in full before dz is added); any other
 * overlap is unsupported.  With ending = 1 the update lands in z's frame, so
 * the Pairformer pair step
 *     z += tri_att_start(z, mask)
 *     z = z^T; z += tri_att_end(z, mask^T); z = z^T
 * (patches/protenix/0006-*.patch:17-37, around PairformerBlock.forward) is two
 * calls with ending = 0 and ending = 1 on the same z, with no transposed
 * copies.  Same sizes, status codes and contract as fpx_tri_attn_block;
 * status 2 when z_out == z with different strides. */
int fpx_tri_attn_block_residual(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                                const float* mask, int64_t m_stride0, int64_t m_stride1,
                                const void* ln_w, const void* ln_b, float eps,
                                const void* w_qkvg, const void* b_g, const void* w_bias,
                                const void* w_o, const void* b_o, float mask_inf, int n, int c,
                                int heads, int head_dim, int ending, void* z_out,
                                int64_t out_stride0, int64_t out_stride1, void* workspace,
                                size_t workspace_bytes, void* stream);

/* fpx_tri_attn_block without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a fixed device array inside the library (41 MiB per GPU the
 * library runs on, held until the process ends), so it serves n <= 128 only
 * (status 2 above); everything else is as fpx_tri_attn_block, and the result
 * is bit-identical to it.  It allocates nothing and calls no allocating
 * library routine.  Every call on one GPU uses that GPU's one array: calls
 * that overlap on one GPU (two streams, or two host threads) race and must
 * be serialised by the caller. */
int fpx_tri_attn_block_noalloc(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                               const float* mask, int64_t m_stride0, int64_t m_stride1,
                               const void* ln_w, const void* ln_b, float eps, const void* w_qkvg,
                               const void* b_g, const void* w_bias, const void* w_o,
                               const void* b_o, float mask_inf, int n, int c, int heads,
                               int head_dim, int ending, void* dz, int64_t dz_stride0,
                               int64_t dz_stride1, void* stream);

/* The block's three stages, run in this order on one workspace;
 * fpx_tri_attn_block is exactly prepare + attend + finish.  Split so a caller
 * (or a profiler) can time or overlap the stages; the workspace carries the
 * intermediate q/k/v^T/gate/bias between them.  No reference counterpart as
 * separate calls: together they replace the same module call as
 * fpx_tri_attn_block.
 *   prepare: mask bias, pair LayerNorm, q/k/v/gate and triangle-bias
 *            projections (patch 0005:32-45; qkv_projection.py:54-66)
 *   attend:  flash attention with the gate multiplied in the epilogue
 *            (patch 0002:57; attention_gate.py:52-53)
 *   finish:  output projection into dz (attention_gate.py:54) */
int fpx_tri_attn_prepare(int dtype, const void* z, int64_t z_stride0, int64_t z_stride1,
                         const float* mask, int64_t m_stride0, int64_t m_stride1,
                         const void* ln_w, const void* ln_b, float eps, const void* w_qkvg,
                         const void* b_g, const void* w_bias, float mask_inf, int n, int ending,
                         void* workspace, size_t workspace_bytes, void* stream);
int fpx_tri_attn_attend(int dtype, int n, void* workspace, size_t workspace_bytes, void* stream);
int fpx_tri_attn_finish(int dtype, const void* w_o, const void* b_o, int n, int ending, void* dz,
                        int64_t dz_stride0, int64_t dz_stride1, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Attention core, argument-compatible with the reference's
 *   int ck_attention(float* q, float* k, float* v, float* bias, float* out,
 *                    int batch, int n, void* stream)
 * (kernels/amd/fireprot_ck_attention.cpp:34, 66, 102; ctypes binding at
 * python/fireprot/backends/amd/ck_attention.py:65-73), for any batch >= 1 and
 * n % 4 == 0 (the reference entries accept two shapes only).
 * q, k, v, out: [batch][heads=4][n][32] viewed with strides (n*128, 32, 128, 1),
 * i.e. memory [batch][n][4][32]; q already scaled by 1/sqrt(32).
 * bias: [1][4][n][n] contiguous, shared by every batch row (the reference's
 * padded N = 1536 rows of 1552 floats are ck_attention's and
 * ck_attention_exact1536's convention; fpx_attn_core_masked takes any row
 * stride).  Requires 16-byte aligned pointers (status 3 otherwise). */
int fpx_attn_core(float* q, float* k, float* v, float* bias, float* out, int batch, int n,
                  void* stream);

/* The reference's three exported entries, by name and behaviour, so that its
 * ctypes loader (python/fireprot/backends/amd/ck_attention.py:65-73) binds
 * this library unchanged and its attention() body (ck_attention.py:115-141)
 * runs as written.  Same arguments and layout as fpx_attn_core; each accepts
 * only the shapes of its reference counterpart and returns 2 for any other:
 *   ck_attention                 (batch, n) = (1000, 1000) or (512, 1536);
 *                                bias row stride 1552 at n = 1536
 *                                (fireprot_ck_attention.cpp:34-37)
 *   ck_attention_exact1536       (512, 1536), bias row stride 1552
 *                                (fireprot_ck_attention.cpp:66-72)
 *   ck_attention_vector_bias1000 (1000, 1000), bias row stride 1000
 *                                (fireprot_ck_attention.cpp:102-107)
 * A null or misaligned (16-byte) pointer returns 3 before any launch, as the
 * reference's vector_bias1000 entry does (fireprot_ck_attention.cpp:106-107);
 * the computation is FP32 on the FP32 matrix cores (v_mfma_f32_32x32x2_f32),
 * asynchronous on the caller's stream, with no allocation. */
int ck_attention(float* q, float* k, float* v, float* bias, float* out, int batch, int n,
                 void* stream);
int ck_attention_exact1536(float* q, float* k, float* v, float* bias, float* out, int batch,
                           int n, void* stream);
int ck_attention_vector_bias1000(float* q, float* k, float* v, float* bias, float* out,
                                 int batch, int n, void* stream);

/* Attention core with the additive mask bias of the two-bias form
 * biases = [mask_bias[batch,1,1,n], tri_bias[1,4,n,n]]
 * (python/fireprot/backends/amd/triangle_attention.py:199-256, native lambda of
 * patches/protenix/0002-*.patch:57).  mask_bias row b holds n values at
 * mask_bias + b*mask_bias_stride (nullable: no mask); bias rows are
 * bias_row_stride floats apart (>= n, multiple of 4), so padded rows such as
 * the reference's 1552-float N1536 rows (ck_attention.py:126-130) are accepted.
 * Logits are fl(fl(q.k + mask_bias) + bias) in that order. */
int fpx_attn_core_masked(const float* q, const float* k, const float* v, const float* mask_bias,
                         int64_t mask_bias_stride, const float* bias, int64_t bias_row_stride,
                         float* out, int batch, int n, void* stream);

/* Bytes of workspace fpx_attn_strided needs for (batch, n); 0 for unsupported
 * sizes. */
size_t fpx_attn_strided_workspace_bytes(int batch, int n);

/* OpenFold3's _attention(query, key, value, [mask_bias, tri_bias]) in one
 * call, for any strides: out = softmax(fl(fl(q.k^T + mask_bias) + tri_bias)) v
 * per (b, h), the order of `for b in biases: a += b`.  Replaces the scoped
 * dispatch of adapters/openfold3/attention.py:121-148 (whose fused path is a
 * QK einsum, the fireprot_softmax_f32 C ABI of backends/amd/softmax_fp32.py:
 * 57-84 and a PV einsum) with a single fused launch; the wire layouts are
 * those accepted by softmax_fp32.py:19-38 and attention.py:99-119.
 *   q, k, v, out  [batch][4][n][32]; element (b, h, j, c) at
 *                 b*s_b + h*s_h + j*s_n + c.  Strides >= 0 and multiples of 4,
 *                 pointers 16-byte aligned; q already scaled by 1/sqrt(32);
 *                 out must not overlap q, k, v or the workspace.
 *   mask_bias     nullable additive bias [batch or 1][1][1][n]: value (b, k) at
 *                 b*m_sb + k*m_sk (m_sb = 0 broadcasts one row, m_sk = n is the
 *                 transposed pair mask of the ending node)
 *   bias          nullable [1][4][n][n]: value (h, q, k) at h*b_sh + q*b_sq +
 *                 k*b_sk (head-first, head-last and transposed views alike)
 *   workspace     fpx_attn_strided_workspace_bytes(batch, n) bytes, 256-aligned;
 *                 the bias and mask are staged there in the kernel's order
 * Supported: 1 <= n <= 4096, batch >= 1.  Logits keep FP32 throughout, so
 * OpenFold3's use_high_precision flag needs no separate path. */
int fpx_attn_strided(const float* q, int64_t q_sb, int64_t q_sh, int64_t q_sn, const float* k,
                     int64_t k_sb, int64_t k_sh, int64_t k_sn, const float* v, int64_t v_sb,
                     int64_t v_sh, int64_t v_sn, const float* mask_bias, int64_t m_sb,
                     int64_t m_sk, const float* bias, int64_t b_sh, int64_t b_sq, int64_t b_sk,
                     float* out, int64_t o_sb, int64_t o_sh, int64_t o_sn, int batch, int n,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace fpx_tri_mul needs; 0 for unsupported sizes. */
size_t fpx_tri_mul_workspace_bytes(int n, int c_z, int c_hidden);

/* Triangle multiplicative update, outgoing or incoming, in one call:
 *   zn = LayerNorm_in(z); a = mask * sigmoid(zn W_a_g^T + b) * (zn W_a_p^T + b);
 *   b likewise; x[i,j] = sum_k a[i,k] * b[j,k] (outgoing) or
 *   sum_k a[k,i] * b[k,j] (incoming), per channel;
 *   u = sigmoid(zn W_g^T + b_g) * (LayerNorm_out(x) W_z^T + b_z);
 *   out = u (accumulate = 0) or out + u (accumulate = 1, the native z += u).
 * Replaces the Protenix module call TriangleMultiplicativeUpdate.forward(z,
 * mask, inplace_safe, _add_with_inplace) as dispatched by
 * patches/protenix/0001-*.patch:14-46 and python/fireprot/backends/amd/
 * triangle_multiplication.py:294-345 (LN once, gated projections packed
 * channel-first, BMM contraction, output LN, linear_z and the gated residual
 * kernel of kernels/amd/fireprot_amd_ops.cu:590-602), for any N and with an
 * explicit mask.
 *   z        [n][n][128], strides (z_stride0, z_stride1, 1), multiples of 4
 *   mask     nullable [n][n] multiplier of a and b (strides m_stride0/1)
 *   ln_*     nullable LayerNorm affine [128]; eps as in the module (1e-5)
 *   w_abpg   [4][128][128]: W_a_p, W_a_g, W_b_p, W_b_g stacked, torch [out, in]
 *   b_abpg   nullable [4][128] biases of those four projections
 *   w_z, w_g [128][128]; b_z, b_g nullable [128]
 *   out      [n][n][128], strides (out_stride0, out_stride1, 1); may be z
 *            itself with the same strides (the in-place update); any other
 *            overlap with z is unsupported (status 2 when out == z with
 *            different strides)
 *   workspace at least fpx_tri_mul_workspace_bytes(n, 128, 128), 256-aligned
 * Supported: c_z = c_hidden = 128, 1 <= n <= 4096. */
int fpx_tri_mul(const float* z, int64_t z_stride0, int64_t z_stride1, const float* mask,
                int64_t m_stride0, int64_t m_stride1, const float* ln_in_w, const float* ln_in_b,
                float eps_in, const float* w_abpg, const float* b_abpg, const float* ln_out_w,
                const float* ln_out_b, float eps_out, const float* w_z, const float* b_z,
                const float* w_g, const float* b_g, int n, int c_z, int c_hidden, int outgoing,
                int accumulate, float* out, int64_t out_stride0, int64_t out_stride1,
                void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace fpx_transition needs for rows_i x rows_j pair rows (the
 * fused kernel's weight planes, about 0.8 MB, whatever the row count); 0 for
 * unsupported sizes. */
size_t fpx_transition_workspace_bytes(int64_t rows_i, int64_t rows_j, int c, int expansion);

/* Pair transition: out = W_o (silu(W_a LN(x)) * (W_b LN(x))) per 128-channel
 * row, or out + that (accumulate = 1, the Pairformer's z += transition(z)).
 * Replaces the Protenix module call Transition.forward (n = 4, c_in = 128) as
 * hooked at python/fireprot/adapters/protenix/hooks.py:56-68 and dispatched
 * by python/fireprot/backends/amd/recycle.py:360-390 / :203-227 (LayerNorm,
 * transition_projection = silu(a) * b of kernels/amd/fireprot_amd_ops.cu:
 * 1111-1165, then linear_no_bias), for any row count.
 *   x        rows x[i][j] at x + i*x_stride_i + j*x_stride_j, 128 channels
 *            with stride 1 (strides multiples of 4, x 16-byte aligned); a flat
 *            [rows][128] tensor is rows_i = 1, x_stride_j = 128
 *   ln_w/b   nullable LayerNorm affine [128]; eps as in the module (1e-5)
 *   w_a, w_b [512][128]; w_o [128][512] (torch [out, in], no biases)
 *   out      same row addressing with out strides; may be x itself with the
 *            same strides (in place); other overlaps unsupported
 *   workspace fpx_transition_workspace_bytes(...) bytes, 256-aligned
 * Supported: c = 128, expansion = 4. */
int fpx_transition(const float* x, int64_t rows_i, int64_t rows_j, int64_t x_stride_i,
                   int64_t x_stride_j, const float* ln_w, const float* ln_b, float eps,
                   const float* w_a, const float* w_b, const float* w_o, int c, int expansion,
                   int accumulate, float* out, int64_t out_stride_i, int64_t out_stride_j,
                   void* workspace, size_t workspace_bytes, void* stream);

/* LayerNorm over 128 channels of rows x[i][j] read at x + i*stride_i + j*stride_j
 * (channel stride 1), written contiguously to y[rows_i][rows_j][128].  Covers
 * both the contiguous pair LN (kernels/amd/fireprot_amd_ops.cu:27-64,
 * layer_norm_f32_128*) and the transposed-view LN of the ending node
 * (fireprot_amd_ops.cu:957-1104, transposed_layer_norm; dispatch at
 * python/fireprot/backends/amd/recycle.py:293-357).  w, b nullable. */
int fpx_layer_norm_c128(const float* x, int64_t rows_i, int64_t rows_j, int64_t stride_i,
                        int64_t stride_j, const float* w, const float* b, float eps, float* y,
                        void* stream);

/* Fused q/k/v projection of already-normalised rows x[rows][128] with torch
 * [128,128] weights; out is [3][rows][128] (q, k, v), q scaled by 1/sqrt(32).
 * Replaces qkv_projection (kernels/amd/fireprot_amd_ops.cu:865-955; hook at
 * python/fireprot/backends/amd/qkv_projection.py:54-66). */
int fpx_qkv_projection(const float* x, int64_t rows, const float* wq, const float* wk,
                       const float* wv, float* out, void* stream);

/* out = value * sigmoid(gate) over count floats (count % 4 == 0), out of place.
 * Replaces sigmoid_mul_out_f32 (kernels/amd/fireprot_amd_ops.cu:536-565; hook at
 * python/fireprot/backends/amd/attention_gate.py:28-56). */
int fpx_sigmoid_mul_out(const float* gate, const float* value, float* out, int64_t count,
                        void* stream);

/* The fp16 (hi, lo) split behind every FP32-accurate product of this
 * library, exposed so its bits can be checked on a new driver or compiler:
 * count floats (count % 8 == 0), taken as given, into two [count] planes of
 * fp16 bit patterns, hi = fp16(x) and lo = fp16(x - hi) (round to nearest
 * even; x - hi is exact, so hi + lo holds 22 significant bits of x for
 * |x| in [2^-3, 65504]).  The kernels first scale each block of values by a
 * power of two so its max lies in [2^14, 2^15).  No counterpart in the
 * reference (its kernels compute in FP32 or round once); used by this
 * library's own parity tests. */
int fpx_split_planes(const float* x, int64_t count, uint16_t* planes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FIREPROT_AMD_H */
