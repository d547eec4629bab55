"""The block call captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

A caller that captures its model step in a graph captures the block with it.
With the output and workspace passed in, a block call allocates nothing,
issues no memset and no synchronisation, and every kernel initialises the
workspace words it reads, so each replay must equal an eager call on the same
inputs bit for bit.  The replays run with new inputs copied into the captured
buffers, eager work and synchronisations between them.  The test also prints
the time per replayed call beside back-to-back eager calls.
"""
from __future__ import annotations

import time

import pytest
import torch

from fireprot_amd import block as hip_block
from fireprot_amd import workloads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,ending", [(torch.float32, False), (torch.float32, True),
                                          (torch.bfloat16, False)])
def test_block_replays_in_a_graph(dtype, ending):
    n, valid = 96, 80
    print(f"graph dtype={dtype} ending={ending} n={n}", flush=True)
    w = workloads.make_weights(bias_scale=8.0)
    weights = hip_block.BlockWeights.from_tensors(**w, dtype=dtype).to("cuda")
    mask = workloads.make_mask(n, valid).cuda()
    z = torch.empty(n, n, 128, device="cuda", dtype=dtype)
    out = torch.empty_like(z)
    ws = torch.empty(hip_block.workspace_bytes(n, dtype), dtype=torch.uint8, device="cuda")
    g = torch.Generator().manual_seed(31)

    def fill():
        z.copy_(torch.randn(n, n, 128, generator=g).to(dtype))

    fill()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.inference_mode(), torch.cuda.stream(side):
        hip_block.triangle_attention_block(z, mask, weights, ending=ending, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph):
        hip_block.triangle_attention_block(z, mask, weights, ending=ending, out=out, workspace=ws)
    torch.cuda.synchronize()

    eager_ws = torch.empty_like(ws)
    for rep in range(4):
        fill()
        graph.replay()
        torch.cuda.synchronize()
        with torch.inference_mode():
            want = hip_block.triangle_attention_block(z, mask, weights, ending=ending,
                                                      workspace=eager_ws)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
        assert torch.equal(out, want), f"replay {rep} differs from the eager call"

    # host time per call: graph replay against eager launches
    calls = 50
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        graph.replay()
    torch.cuda.synchronize()
    replay_ms = (time.perf_counter() - t0) / calls * 1e3
    t0 = time.perf_counter()
    with torch.inference_mode():
        for _ in range(calls):
            hip_block.triangle_attention_block(z, mask, weights, ending=ending, out=out,
                                               workspace=ws)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / calls * 1e3
    print(f"graph n={n} {dtype}: {replay_ms:.4f} ms per replayed call, "
          f"{eager_ms:.4f} ms per eager call (back to back)", flush=True)
