"""Module-level drop-in: ``(z[N,N,128], mask[N,N]) -> dz[N,N,128]`` on gfx950.

One call runs the whole triangle-attention block through the C ABI entry
``fpx_tri_attn_block`` (include/fireprot_amd.h): pair LayerNorm, fused
q/k/v/gate and triangle-bias projection, flash attention with mask bias and
pair bias, sigmoid gate and output projection.  It stands in for the Protenix
``TriangleAttention.forward`` (patches/protenix/0005-*.patch:14-48) and for
AtlasFold's ``triangle_attention(module, z, mask, ending)``
(python/fireprot/adapters/atlasfold/runtime.py:32-71); the residual
``z += dz`` stays with the caller (patches/protenix/0006-*.patch:25).

Two storage types: float32 (FP32 throughout) and bfloat16 (BF16 storage of z,
weights, intermediates and dz with FP32 accumulation and softmax).  This
module has no CPU path: inputs must be tensors on a HIP device and the native
library must be loaded, otherwise it raises.  Capability-gated
fallback to the *caller's* native function lives in
``fireprot_amd.triangle_attention``.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Any

import torch

from . import _native

CHANNELS = 128
HEADS = 4
HEAD_DIM = 32
HIDDEN = HEADS * HEAD_DIM


@dataclasses.dataclass
class BlockWeights:
    """Device-resident weights of one block, torch ``[out, in]`` layout.

    ``w_qkvg`` stacks W_q, W_k, W_v, W_g (each ``[128, 128]``) into
    ``[512, 128]``.  ``ln_w``, ``ln_b``, ``b_g``, ``b_o`` may be None.
    """

    ln_w: torch.Tensor | None
    ln_b: torch.Tensor | None
    w_qkvg: torch.Tensor
    b_g: torch.Tensor | None
    w_bias: torch.Tensor
    w_o: torch.Tensor
    b_o: torch.Tensor | None
    inf: float = 1e9
    eps: float = 1e-5

    @classmethod
    def from_tensors(cls, *, ln_w, ln_b, w_q, w_k, w_v, w_g, b_g, w_bias, w_o, b_o,
                     inf: float = 1e9, eps: float = 1e-5,
                     dtype: torch.dtype = torch.float32) -> "BlockWeights":
        def prep(t):
            return None if t is None else t.detach().to(dtype).contiguous()
        w_qkvg = torch.cat([w.detach().to(dtype) for w in (w_q, w_k, w_v, w_g)], 0)
        return cls(prep(ln_w), prep(ln_b), w_qkvg.contiguous(), prep(b_g), prep(w_bias),
                   prep(w_o), prep(b_o), float(inf), float(eps))

    @property
    def dtype(self) -> torch.dtype:
        return self.w_qkvg.dtype

    @classmethod
    def from_protenix(cls, module: Any, dtype: torch.dtype | None = None) -> "BlockWeights":
        """Protenix/OpenFold ``TriangleAttention``: ``layer_norm``, ``linear``,
        ``mha.linear_{q,k,v,g,o}``, ``inf`` (patch 0005:32-45; 0002:31-58)."""
        mha = module.mha
        for linear in (mha.linear_q, mha.linear_k, mha.linear_v, module.linear):
            if getattr(linear, "bias", None) is not None:
                raise ValueError("q/k/v and triangle-bias projections must be bias-free")
        return cls.from_tensors(
            ln_w=module.layer_norm.weight, ln_b=module.layer_norm.bias,
            w_q=mha.linear_q.weight, w_k=mha.linear_k.weight, w_v=mha.linear_v.weight,
            w_g=mha.linear_g.weight, b_g=mha.linear_g.bias, w_bias=module.linear.weight,
            w_o=mha.linear_o.weight, b_o=mha.linear_o.bias,
            inf=float(getattr(module, "inf", 1e9)), eps=float(module.layer_norm.eps),
            dtype=dtype or mha.linear_q.weight.dtype)

    @classmethod
    def from_atlasfold(cls, module: Any, dtype: torch.dtype | None = None) -> "BlockWeights":
        """AtlasFold triangle node: ``layernorm``, fused ``linear_qkv``,
        ``linear_bias``, ``linear_g``, ``linear_out`` (atlasfold/runtime.py:38-70)."""
        w_q, w_k, w_v = module.linear_qkv.weight.chunk(3, dim=0)
        return cls.from_tensors(
            ln_w=module.layernorm.weight, ln_b=module.layernorm.bias,
            w_q=w_q, w_k=w_k, w_v=w_v, w_g=module.linear_g.weight,
            b_g=getattr(module.linear_g, "bias", None), w_bias=module.linear_bias.weight,
            w_o=module.linear_out.weight, b_o=getattr(module.linear_out, "bias", None),
            inf=float(module.inf), eps=float(getattr(module.layernorm, "eps", 1e-5)),
            dtype=dtype or module.linear_qkv.weight.dtype)

    def tensors(self) -> tuple[torch.Tensor | None, ...]:
        return (self.ln_w, self.ln_b, self.w_qkvg, self.b_g, self.w_bias, self.w_o, self.b_o)

    def to(self, device) -> "BlockWeights":
        def move(t):
            return None if t is None else t.to(device)
        return dataclasses.replace(self, **{f: move(getattr(self, f)) for f in
                                            ("ln_w", "ln_b", "w_qkvg", "b_g", "w_bias", "w_o", "b_o")})


DTYPES = {torch.float32: _native.FPX_F32, torch.bfloat16: _native.FPX_BF16}


def workspace_bytes(n: int, dtype: torch.dtype = torch.float32) -> int:
    """Device workspace for one block call at pair size n and storage dtype."""
    return int(_native.library().fpx_tri_attn_workspace_bytes(n, CHANNELS, HEADS, HEAD_DIM,
                                                              DTYPES[dtype]))


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def check_block_inputs(z: torch.Tensor, mask: torch.Tensor | None, weights: BlockWeights) -> None:
    """Raise ``ValueError`` unless the tensors fit the native block's contract."""
    if not z.is_cuda or z.dtype not in DTYPES:
        raise ValueError("z must be a float32 or bfloat16 tensor on a HIP device")
    if z.dim() != 3 or z.shape[0] != z.shape[1] or z.shape[2] != CHANNELS:
        raise ValueError(f"z must be [N, N, {CHANNELS}], got {tuple(z.shape)}")
    align = 16 // z.element_size()
    if z.stride(2) != 1 or z.stride(0) % align or z.stride(1) % align:
        raise ValueError("z needs unit channel stride and 16-byte aligned rows")
    if mask is not None and (mask.device != z.device or tuple(mask.shape) != tuple(z.shape[:2])):
        raise ValueError("mask must be [N, N] on z's device")
    shapes = {"w_qkvg": (4 * HIDDEN, CHANNELS), "w_bias": (HEADS, CHANNELS),
              "w_o": (CHANNELS, HIDDEN)}
    for name, shape in shapes.items():
        t = getattr(weights, name)
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must be {shape}, got {tuple(t.shape)}")
    for t in weights.tensors():
        if t is not None and (t.device != z.device or t.dtype != z.dtype
                              or not t.is_contiguous()):
            raise ValueError("weights must be contiguous tensors of z's dtype on z's device")


def triangle_attention_block(z: torch.Tensor, mask: torch.Tensor | None, weights: BlockWeights,
                             *, ending: bool = False, out: torch.Tensor | None = None,
                             workspace: torch.Tensor | None = None,
                             residual: bool = False) -> torch.Tensor:
    """Return dz for the starting (``ending=False``) or ending node.

    The ending node reads ``z`` and ``mask`` through swapped strides and writes
    ``dz`` transposed, so ``dz_end(z, m) == T(dz_start(T(z), T(m)))`` with no
    transposed copies.  With ``residual=True`` the update is added instead:
    ``out += dz`` (``out`` defaults to ``z`` itself, an in-place update), the
    Pairformer's ``z += tri_att_start(z)`` / ``z += tri_att_end(z)``
    (patches/protenix/0006-*.patch:17-37).  Runs asynchronously on the
    current stream.
    """
    lib = _native.library()
    check_block_inputs(z, mask, weights)
    n = z.shape[0]
    if mask is not None and mask.dtype != torch.float32:
        mask = mask.to(torch.float32)
    if out is None:
        out = z if residual else torch.empty((n, n, CHANNELS), device=z.device, dtype=z.dtype)
    elif (tuple(out.shape) != (n, n, CHANNELS) or out.dtype != z.dtype
          or out.device != z.device or out.stride(2) != 1):
        raise ValueError("out must be a [N, N, 128] tensor of z's dtype on z's device")
    align = 16 // z.element_size()
    if out.stride(0) % align or out.stride(1) % align:
        raise ValueError("out rows must be 16-byte aligned")
    if residual and out.data_ptr() == z.data_ptr() and out.stride() != z.stride():
        raise ValueError("an in-place update needs out and z with the same strides")
    with torch.cuda.device(z.device):
        need = workspace_bytes(n, z.dtype)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=z.device)
        elif workspace.numel() * workspace.element_size() < need:
            raise ValueError(f"workspace needs {need} bytes")
        stream = torch.cuda.current_stream(z.device).cuda_stream
        entry = lib.fpx_tri_attn_block_residual if residual else lib.fpx_tri_attn_block
        code = entry(
            DTYPES[z.dtype], z.data_ptr(), z.stride(0), z.stride(1),
            _ptr(mask), mask.stride(0) if mask is not None else 0,
            mask.stride(1) if mask is not None else 0,
            _ptr(weights.ln_w), _ptr(weights.ln_b), weights.eps,
            weights.w_qkvg.data_ptr(), _ptr(weights.b_g), weights.w_bias.data_ptr(),
            weights.w_o.data_ptr(), _ptr(weights.b_o), weights.inf,
            n, CHANNELS, HEADS, HEAD_DIM, int(bool(ending)),
            out.data_ptr(), out.stride(0), out.stride(1),
            workspace.data_ptr(), workspace.numel() * workspace.element_size(), stream)
    _native.check(code, "fpx_tri_attn_block_residual" if residual else "fpx_tri_attn_block")
    return out


def pair_step_triangle_attention(z: torch.Tensor, mask: torch.Tensor | None,
                                 start: BlockWeights, end: BlockWeights, *,
                                 workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The Pairformer's two triangle-attention updates on ``z`` in place:
    ``z += tri_att_start(z, mask)``, then the ending node on the updated ``z``
    (patches/protenix/0006-*.patch:17-37), with no transposed copies."""
    if workspace is None:
        workspace = torch.empty(workspace_bytes(z.shape[0], z.dtype), dtype=torch.uint8,
                                device=z.device)
    triangle_attention_block(z, mask, start, ending=False, workspace=workspace, residual=True)
    triangle_attention_block(z, mask, end, ending=True, workspace=workspace, residual=True)
    return z


def block_flops(n: int) -> dict[str, int]:
    """Algorithmic flop of one block direction (multiply-add counts 2)."""
    core = 4 * HEADS * HEAD_DIM * n ** 3
    proj = 2 * n * n * (CHANNELS * 4 * HIDDEN + CHANNELS * HEADS + HIDDEN * CHANNELS)
    return {"core": core, "projections": proj, "block": core + proj}


def q_scale() -> float:
    return 1.0 / math.sqrt(HEAD_DIM)
