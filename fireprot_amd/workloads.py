"""Seeded synthetic workloads for the triangle-attention block.

Five pair-representation configurations, c_z = 128, H = 4, d = 32:

  c1  N=124,  FP32, starting node, mask all ones (the CPU-runnable case)
  c2  N=512,  FP32, starting + ending, last 51 residues masked on both axes
  c3  N=1000, FP32, starting + ending, mask all ones
  c4  N=1536, FP32, starting + ending, z ~ 2*N(0,1), 12% tail masked
      (1352 valid), triangle-bias weights x8 so logits span about +/-40
  c5  N=2048, BF16 storage / FP32 accumulate, starting + ending, mask all ones

Everything is drawn on the CPU from ``torch.Generator`` seeds (z: 419 + N,
following benchmarks/protenix/benchmark_attention.py:145; weights: 719,
following benchmarks/protenix/benchmark_attention_surround.py:38) so the HIP
path and the oracle see identical bits.  Weights are N(0, 0.02) in torch
``[out, in]`` layout with no bias vectors; LN gamma = 1, beta = 0.  The
triangle-bias weight is N(0, 1/128) so the bias has std ~1 on unit-variance
LN output (scaled by 8 for c4).  A mask of all ones is omitted (``None``), as
the reference omits an implicit all-ones mask (patches/protenix/0005-*.patch:
18-19).
"""
from __future__ import annotations

import dataclasses
import math

import torch

Z_SEED_BASE = 419
WEIGHT_SEED = 719


@dataclasses.dataclass(frozen=True)
class Workload:
    key: str
    name: str
    n: int
    dtype: str                      # "f32" or "bf16" (storage)
    directions: tuple[str, ...]
    valid: int | None = None        # residues kept by the mask (None: no mask)
    z_scale: float = 1.0
    bias_scale: float = 1.0


CONFIGS: dict[str, Workload] = {
    "c1": Workload("c1", "n124-start-f32", 124, "f32", ("start",)),
    "c2": Workload("c2", "n512-tail51-f32", 512, "f32", ("start", "end"), valid=461),
    "c3": Workload("c3", "n1000-f32", 1000, "f32", ("start", "end")),
    "c4": Workload("c4", "n1536-tail184-bias8-f32", 1536, "f32", ("start", "end"),
                   valid=1536 - round(0.12 * 1536), z_scale=2.0, bias_scale=8.0),
    "c5": Workload("c5", "n2048-bf16", 2048, "bf16", ("start", "end")),
}


def make_weights(bias_scale: float = 1.0, channels: int = 128, heads: int = 4,
                 head_dim: int = 32) -> dict[str, torch.Tensor | None]:
    g = torch.Generator().manual_seed(WEIGHT_SEED)
    hidden = heads * head_dim

    def normal(*shape, std):
        return torch.randn(*shape, generator=g, dtype=torch.float32) * std

    weights: dict[str, torch.Tensor | None] = {
        "ln_w": torch.ones(channels),
        "ln_b": torch.zeros(channels),
        "w_q": normal(hidden, channels, std=0.02),
        "w_k": normal(hidden, channels, std=0.02),
        "w_v": normal(hidden, channels, std=0.02),
        "w_g": normal(hidden, channels, std=0.02),
        "b_g": None,
        "w_bias": normal(heads, channels, std=1.0 / math.sqrt(channels)) * bias_scale,
        "w_o": normal(channels, hidden, std=0.02),
        "b_o": None,
    }
    return weights


TRIMUL_WEIGHT_SEED = 4242


def make_trimul_weights(std: float = 0.1, *, biases: bool = False, affine: bool = False,
                        seed: int = TRIMUL_WEIGHT_SEED,
                        channels: int = 128) -> dict[str, torch.Tensor | None]:
    """Random-init weights of a triangle multiplicative update (c_z = c_hidden =
    128), every projection N(0, std^2) as the reference's operator tests draw
    them (tests/operators/test_packed_triangle.py:96-97).  ``biases`` adds
    N(0, std^2) biases to the six projections (OpenFold-style modules);
    ``affine`` draws non-trivial LayerNorm scales and shifts."""
    g = torch.Generator().manual_seed(seed)

    def normal(*shape, scale=std):
        return torch.randn(*shape, generator=g, dtype=torch.float32) * scale

    w: dict[str, torch.Tensor | None] = {
        "ln_in_w": torch.ones(channels), "ln_in_b": torch.zeros(channels),
        "ln_out_w": torch.ones(channels), "ln_out_b": torch.zeros(channels),
    }
    for name in ("w_a_p", "w_a_g", "w_b_p", "w_b_g", "w_z", "w_g"):
        w[name] = normal(channels, channels)
    for name in ("b_a_p", "b_a_g", "b_b_p", "b_b_g", "b_z", "b_g"):
        w[name] = normal(channels) if biases else None
    if affine:
        for side in ("in", "out"):
            w[f"ln_{side}_w"] = 1.0 + normal(channels, scale=0.1)
            w[f"ln_{side}_b"] = normal(channels, scale=0.1)
    return w


TRANSITION_WEIGHT_SEED = 4343


def make_transition_weights(std: float = 0.05, *, affine: bool = False,
                            seed: int = TRANSITION_WEIGHT_SEED,
                            channels: int = 128,
                            expansion: int = 4) -> dict[str, torch.Tensor | None]:
    """Random-init weights of a pair transition (Protenix ``Transition``,
    n = 4): ``W_a``, ``W_b`` ``[512, 128]`` and ``W_o`` ``[128, 512]``, all
    N(0, std^2); ``affine`` draws non-trivial LayerNorm scales and shifts."""
    g = torch.Generator().manual_seed(seed)
    hidden = expansion * channels

    def normal(*shape, scale=std):
        return torch.randn(*shape, generator=g, dtype=torch.float32) * scale

    w: dict[str, torch.Tensor | None] = {
        "ln_w": torch.ones(channels), "ln_b": torch.zeros(channels),
        "w_a": normal(hidden, channels), "w_b": normal(hidden, channels),
        "w_o": normal(channels, hidden),
    }
    if affine:
        w["ln_w"] = 1.0 + normal(channels, scale=0.1)
        w["ln_b"] = normal(channels, scale=0.1)
    return w


def make_pair(n: int, z_scale: float = 1.0, channels: int = 128) -> torch.Tensor:
    g = torch.Generator().manual_seed(Z_SEED_BASE + n)
    z = torch.randn(n, n, channels, generator=g, dtype=torch.float32)
    return z * z_scale if z_scale != 1.0 else z


def make_mask(n: int, valid: int | None) -> torch.Tensor | None:
    if valid is None:
        return None
    keep = torch.arange(n) < valid
    return (keep[:, None] & keep[None, :]).to(torch.float32)


def make_inputs(cfg: Workload | str):
    """Return ``(z, mask, weights)`` on the CPU for a configuration."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    return (make_pair(cfg.n, cfg.z_scale), make_mask(cfg.n, cfg.valid),
            make_weights(cfg.bias_scale))


def make_protenix_module(weights: dict[str, torch.Tensor | None], *, starting: bool = True,
                         device: str | torch.device = "cpu") -> torch.nn.Module:
    """A module with Protenix ``TriangleAttention``'s attributes
    (patches/protenix/0005-*.patch:32-45: ``layer_norm``, ``linear``,
    ``mha.linear_{q,k,v,g,o}``, ``mha.no_heads``, ``mha.c_hidden``, ``inf``,
    ``starting``) holding ``weights`` (``make_weights`` layout), in eval mode.
    It has no forward of its own: it is the ``module`` argument of the block
    dispatch, which reads its weights."""
    def linear(w, b=None):
        layer = torch.nn.Linear(w.shape[1], w.shape[0], bias=b is not None)
        with torch.no_grad():
            layer.weight.copy_(w)
            if b is not None:
                layer.bias.copy_(b)
        return layer

    module = torch.nn.Module()
    module.starting = starting
    module.layer_norm = torch.nn.LayerNorm(weights["ln_w"].shape[0])
    with torch.no_grad():
        module.layer_norm.weight.copy_(weights["ln_w"])
        module.layer_norm.bias.copy_(weights["ln_b"])
    module.linear = linear(weights["w_bias"])
    module.mha = torch.nn.Module()
    module.mha.linear_q = linear(weights["w_q"])
    module.mha.linear_k = linear(weights["w_k"])
    module.mha.linear_v = linear(weights["w_v"])
    module.mha.linear_g = linear(weights["w_g"], weights["b_g"])
    module.mha.linear_o = linear(weights["w_o"], weights["b_o"])
    module.mha.no_heads = weights["w_bias"].shape[0]
    module.mha.c_hidden = weights["w_q"].shape[0] // module.mha.no_heads
    module.inf = float(weights.get("inf", 1e9) or 1e9)
    return module.to(device).eval()
