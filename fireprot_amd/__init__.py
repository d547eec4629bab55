"""MI355X-native (gfx950) triangle-attention block for Pairformer pair stacks.

Public surface:

* ``fireprot_amd.block`` -- ``triangle_attention_block(z, mask, weights, ending)``,
  the whole block ``(z[N,N,128], mask[N,N]) -> dz`` in one C-ABI call;
* ``fireprot_amd.triangle_attention`` -- ``dispatch_triangle_attention`` (the
  operator-level core) and ``dispatch_triangle_attention_block`` (module level),
  both capability-gated with fallback to the caller's native function;
* ``fireprot_amd.registry`` -- ``OperationRegistry`` / ``OperationSignature``;
* ``fireprot_amd.layer_norm``, ``qkv_projection``, ``attention_gate``,
  ``pair_layout`` -- the per-stage hooks;
* ``fireprot_amd.workloads`` -- the seeded benchmark configurations.

The native library is ``fireprot_amd/_lib/libfireprot_amd.so`` (built by
``python -m fireprot_amd.build``); its C ABI is ``include/fireprot_amd.h``.
"""
__all__ = ["block", "registry", "triangle_attention", "workloads"]
