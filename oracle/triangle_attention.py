"""CPU oracle for the triangle-attention block -- TEST INFRASTRUCTURE ONLY.

This module restates, in plain PyTorch on the CPU, the native arithmetic of the
Pairformer triangle-attention block that the reference accelerates.  It is the
checker for the HIP path: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and never as the code that
is measured or shipped.  The product path (``fireprot_amd``) must not import it.

Every function follows a reference call site (paths relative to the reference
checkout):

* block body and op order        -- patches/protenix/0005-*.patch:14-48
  (mask bias omitted when the mask is None; LN; ``inf * (mask - 1)`` mask bias;
  ``permute_final_dims(linear(x), (2, 0, 1)).unsqueeze(-4)`` triangle bias;
  ending node transposes x and mask on entry and the result on exit)
* scaling flag and native core   -- patches/protenix/0002-*.patch:31-58
  (``apply_scale`` divides q by sqrt(c_hidden); native core is
  ``_attention(q, k, v, biases).transpose(-2, -3)``)
* residual stays outside         -- patches/protenix/0006-*.patch:17-37
* complete block with gate/out   -- python/fireprot/adapters/atlasfold/runtime.py:32-71
* Q/K/V layout, 1/sqrt(32) on Q  -- python/fireprot/backends/amd/qkv_projection.py:54-66
* gate then output projection    -- python/fireprot/backends/amd/attention_gate.py:52-54
* closed-form core               -- tests/operators/test_direct_attention.py:36-49
* LN formula, eps 1e-5           -- python/fireprot/backends/amd/recycle.py:101-102
* mask-then-bias add order       -- kernels/amd/fireprot_softmax_fp32.cpp:23-36
* BF16 rounding points           -- kernels/amd/fireprot_pair_softmax.cu:10-41,
                                    kernels/amd/fireprot_mask_bias.cu:9-22

The upstream model code (Protenix ``_attention``, ``Attention``,
``TriangleAttention``) is not vendored in the reference and is not installed
here, so this restatement is pinned by the float64 brute-force in
``oracle/brute.py``, by the committed fixtures under ``tests/golden/`` that the
brute force wrote, and by closed forms and invariants in
``tests/test_oracle.py`` (see each function's docstring for what pins it).
"""
from __future__ import annotations

import dataclasses
import math
from collections.abc import Sequence

import torch

HEADS = 4
HEAD_DIM = 32
CHANNELS = 128
MASK_INF = 1e9
LN_EPS = 1e-5


@dataclasses.dataclass
class BlockParams:
    """Weights of one triangle-attention block in torch ``[out, in]`` layout.

    Names follow Protenix ``TriangleAttention``: ``layer_norm``, ``linear``
    (the triangle-bias projection, no bias term) and ``mha.linear_{q,k,v,g,o}``
    (patches/protenix/0005-*.patch:32-45; attention_gate.py:52-54).
    """

    ln_w: torch.Tensor | None          # [C]
    ln_b: torch.Tensor | None          # [C]
    w_q: torch.Tensor                  # [H*D, C]
    w_k: torch.Tensor                  # [H*D, C]
    w_v: torch.Tensor                  # [H*D, C]
    w_g: torch.Tensor                  # [H*D, C]
    b_g: torch.Tensor | None           # [H*D]
    w_bias: torch.Tensor               # [H, C]
    w_o: torch.Tensor                  # [C, H*D]
    b_o: torch.Tensor | None           # [C]
    inf: float = MASK_INF
    eps: float = LN_EPS

    def to(self, dtype: torch.dtype) -> "BlockParams":
        def cast(t):
            return None if t is None else t.to(dtype)
        return BlockParams(**{f.name: (cast(getattr(self, f.name))
                                       if isinstance(getattr(self, f.name), torch.Tensor)
                                       or getattr(self, f.name) is None
                                       else getattr(self, f.name))
                              for f in dataclasses.fields(self)})


def layer_norm(x: torch.Tensor, w: torch.Tensor | None, b: torch.Tensor | None,
               eps: float = LN_EPS) -> torch.Tensor:
    """``OpenFoldLayerNorm`` / ``torch.nn.LayerNorm`` over the last (128) axis.

    Biased variance, ``(x - mean) / sqrt(var + eps) * w + b``
    (kernels/amd/fireprot_amd_ops.cu:27-64; recycle.py:101-102, eps 1e-5).
    Pinned by oracle/brute.py (two-pass float64 loops) and by the closed form
    mean 0 / biased variance 1 for w=1, b=0.
    """
    return torch.nn.functional.layer_norm(x, (x.shape[-1],), w, b, eps)


def linear(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None = None) -> torch.Tensor:
    """``nn.Linear``: ``x @ w.T + b`` with torch ``[out, in]`` weights."""
    return torch.nn.functional.linear(x, w, b)


def permute_final_dims(t: torch.Tensor, inds: Sequence[int]) -> torch.Tensor:
    """OpenFold's ``permute_final_dims`` (used by patch 0005:42-45)."""
    zero_index = -1 * len(inds)
    first_inds = list(range(len(t.shape[:zero_index])))
    return t.permute(first_inds + [zero_index + i for i in inds])


def attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   biases: Sequence[torch.Tensor], *, logits_f32: bool = False) -> torch.Tensor:
    """Native ``_attention(q, k, v, biases)``: returns ``[*, H, Q, C]``.

    ``a = q @ k^T``; ``a += b`` for each bias in list order (mask bias first,
    then triangle bias: patch 0005:36-45, fireprot_softmax_fp32.cpp:33-35);
    softmax over keys with no upcast (a fully -inf row gives NaN, as
    ``torch.softmax`` does); ``a @ v``.  Closed form at
    tests/operators/test_direct_attention.py:44-47.  Pinned by brute-force
    loops and by closed forms (N=1 gives v; zero logits give mean_k v; a +80
    bias selects one key; an all -inf row gives NaN) in tests/test_oracle.py.

    ``logits_f32`` (float64 inputs): round the logits to float32 at the
    native add points, ``fl32(fl32(fl32(s) + fl32(mb)) + fl32(bias))``, and
    keep everything else in float64 -- the ``logits="f32"`` evaluation of
    oracle/brute.py.  It reproduces what the FP32 native path does to fully
    masked rows (-1e9 has a float32 spacing of 64, so their logits tie).
    """
    a = torch.matmul(q, permute_final_dims(k, (1, 0)))
    if logits_f32:
        def fl32(t):
            return t.to(torch.float32).to(a.dtype)
        a = fl32(a)
        for bias in biases:
            a = fl32(a + fl32(bias))
    else:
        for bias in biases:
            a += bias
    a = torch.softmax(a, dim=-1)
    return torch.matmul(a, v)


def prep_qkv(x: torch.Tensor, p: BlockParams, apply_scale: bool = True):
    """``Attention._prep_qkv``: q/k/v as ``[*, H, N, D]`` views, q /= sqrt(D).

    Layout ``[B, N, H, D].transpose(1, 2)`` with strides ``(N*H*D, D, H*D, 1)``
    (qkv_projection.py:62; tests/operators/test_qkv_projection.py:57).
    """
    heads = p.w_bias.shape[0]
    q = linear(x, p.w_q)
    k = linear(x, p.w_k)
    v = linear(x, p.w_v)
    q = q.view(q.shape[:-1] + (heads, -1)).transpose(-2, -3)
    k = k.view(k.shape[:-1] + (heads, -1)).transpose(-2, -3)
    v = v.view(v.shape[:-1] + (heads, -1)).transpose(-2, -3)
    if apply_scale:
        q = q / math.sqrt(q.shape[-1])
    return q, k, v


def wrap_up(o: torch.Tensor, x: torch.Tensor, p: BlockParams, *,
            abs_terms: bool = False) -> torch.Tensor:
    """``Attention._wrap_up``: ``linear_o(flatten(o * sigmoid(linear_g(x))))``.

    o is ``[*, N, H, D]`` (head-last).  attention_gate.py:52-54; the gate
    sigmoid(g) * o is checked against its closed form over linspace(-1000,
    1000) as in tests/operators/test_attention_gate.py:32-37.

    ``abs_terms``: return the magnitude of the output projection's terms,
    ``|o g| |W_o|^T + |b_o|`` (the componentwise condition scale of each
    output element: an error of u relative in every gated value moves an
    output by at most u times it).
    """
    heads = p.w_bias.shape[0]
    g = torch.sigmoid(linear(x, p.w_g, p.b_g))
    g = g.view(g.shape[:-1] + (heads, -1))
    o = o * g
    o = o.reshape(o.shape[:-2] + (-1,))
    if abs_terms:
        return linear(o.abs(), p.w_o.abs(), None if p.b_o is None else p.b_o.abs())
    return linear(o, p.w_o, p.b_o)


def mask_bias(mask: torch.Tensor, inf: float = MASK_INF) -> torch.Tensor:
    """``(inf * (mask - 1))[..., :, None, None, :]`` (patch 0005:36-39)."""
    return (inf * (mask - 1))[..., :, None, None, :]


def triangle_bias(x_ln: torch.Tensor, p: BlockParams) -> torch.Tensor:
    """``permute_final_dims(linear(x), (2, 0, 1)).unsqueeze(-4)`` -> [1, H, N, N]."""
    return permute_final_dims(linear(x_ln, p.w_bias), (2, 0, 1)).unsqueeze(-4)


def block(z: torch.Tensor, mask: torch.Tensor | None, p: BlockParams, *,
          ending: bool = False, outer_rows: torch.Tensor | None = None,
          chunk: int = 64, logits_f32: bool = False, abs_terms: bool = False) -> torch.Tensor:
    """Triangle-attention block ``(z[N,N,C], mask[N,N]) -> dz[N,N,C]``.

    Restates ``TriangleAttention.forward`` (patch 0005:14-48) with
    ``Attention.forward`` (patch 0002:31-58) and the AtlasFold full-block
    restatement (atlasfold/runtime.py:32-71).  The residual ``z += dz`` is the
    caller's (patch 0006:25).  The ending node is the starting node applied to
    the transposed pair representation and mask, transposed back.

    ``outer_rows`` (in the frame after the ending-node transpose) restricts the
    attention, gate and output projection to those outer rows; the LayerNorm
    and triangle bias are still computed for the whole pair representation.
    Rows are independent, so this equals the matching rows of the full result
    (chunk invariance: docs/protenix-long1536.md:889-901).  The result then has
    shape ``[len(outer_rows), N, C]`` in the (possibly transposed) x frame.
    ``chunk`` bounds the materialised score tensor to ``chunk * H * N * N``.
    ``logits_f32`` rounds the logits to float32 at the native add points
    (see ``attention_core``); meant for float64 inputs.  ``abs_terms`` returns
    the magnitude of each output's projection terms instead (``wrap_up``).
    """
    x = z
    if ending:
        x = x.transpose(-2, -3)
        if mask is not None:
            mask = mask.transpose(-1, -2)
    x = layer_norm(x, p.ln_w, p.ln_b, p.eps)
    tri = triangle_bias(x, p)
    n = x.shape[-2]
    rows = torch.arange(x.shape[-3]) if outer_rows is None else outer_rows
    out = []
    for start in range(0, len(rows), chunk):
        sel = rows[start:start + chunk]
        xs = x[sel]
        biases = []
        if mask is not None:
            biases.append(mask_bias(mask[sel], p.inf))
        biases.append(tri)
        q, k, v = prep_qkv(xs, p, apply_scale=True)
        o = attention_core(q, k, v, biases, logits_f32=logits_f32).transpose(-2, -3)
        out.append(wrap_up(o, xs, p, abs_terms=abs_terms))
    dz = torch.cat(out, dim=0) if out else x.new_empty((0, n, x.shape[-1]))
    if ending and outer_rows is None:
        dz = dz.transpose(-2, -3)
    return dz


def block_bf16(z: torch.Tensor, mask: torch.Tensor | None, p: BlockParams, *,
               ending: bool = False, outer_rows: torch.Tensor | None = None,
               chunk: int = 16) -> torch.Tensor:
    """BF16-storage block: the native path run on BF16 tensors.

    Every op is the native op on ``torch.bfloat16`` tensors, so each
    intermediate (LN output, projections, logits after the mask add and after
    the bias add, softmax output, attention output, gate) is rounded to BF16
    exactly where the native BF16 path rounds it (the reference reproduces the
    same points: fireprot_pair_softmax.cu:19-26, fireprot_mask_bias.cu:9-22).
    """
    pb = p.to(torch.bfloat16)
    return block(z.to(torch.bfloat16), None if mask is None else mask.to(torch.bfloat16),
                 pb, ending=ending, outer_rows=outer_rows, chunk=chunk)


def block_flops(n: int, c: int = CHANNELS, heads: int = HEADS, head_dim: int = HEAD_DIM) -> dict:
    """Algorithmic flop of one block direction (multiply-add = 2 flop)."""
    hd = heads * head_dim
    core = 4 * heads * head_dim * n ** 3                 # QK^T and PV
    proj = 2 * n * n * (c * 4 * hd + c * heads + hd * c)  # qkvg, bias, out
    return {"core": core, "projections": proj, "block": core + proj}
