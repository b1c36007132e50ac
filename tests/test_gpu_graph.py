"""HIP graph capture of the drop-in calls.

Launch-bound callers (the skinny adapter linears take a few microseconds of
device time per call) replay a captured step instead of paying the host path
each time.  Every entry point only launches kernels on the caller's stream and
records no memset, so a captured call must reproduce the eager result bit for
bit on every replay, with fresh inputs copied into the captured buffers and
eager work run between the replays.
"""

import pytest
import torch

from vflash_amd.fp8_linear import RowFP8Execution
from vflash_amd.fused import fp8_ffn, fp8_linear_lora
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu


def capture(fn):
    """Warm up on a side stream (default priority), then capture fn() once."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def replay_matches_eager(graph, out, static_inputs, fresh_inputs, eager):
    for replay, inputs in enumerate(fresh_inputs):
        for dst, src in zip(static_inputs, inputs):
            dst.copy_(src)
        graph.replay()
        ref = eager(*inputs)  # eager launches between the replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {replay} differs from the eager call"


def test_skinny_lora_linear_replays_from_a_graph(dev):
    m, k, n, r = 512, 1536, 4608, 32
    g = torch.Generator().manual_seed(11)
    c, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    la = (torch.randn((r, k), generator=g) * 0.01).to(torch.bfloat16)
    lb = (torch.randn((n, r), generator=g) * 0.01).to(torch.bfloat16)
    c, s, b, la, lb = (t.to(dev) for t in (c, s, b, la, lb))
    xs = [torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev) for _ in range(4)]
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")

    def eager(x):
        return fp8_linear_lora(ex, x, c, s, b, la, lb, scaling=0.5, strength=1.375)

    static_x = xs[0].clone()
    graph, out = capture(lambda: eager(static_x))
    replay_matches_eager(graph, out, [static_x], [[x] for x in xs], eager)


@pytest.mark.parametrize("m,k,n", [(4096, 1024, 2048), (2100, 640, 2064)])
def test_w8a8_linear_replays_from_a_graph(dev, m, k, n):
    # 256 tiles of 256x128 and 187 tiles of 128x192 (partial last tiles).
    g = torch.Generator().manual_seed(m)
    c, s = quantize_weight_rows(torch.randn((n, k), generator=g) * 0.02)
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)
    c, s, b = c.to(dev), s.to(dev), b.to(dev)
    xs = [torch.randn((m, k), generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]
    ex = RowFP8Execution("w8a8", activation_quantizer="triton")

    def eager(x):
        return ex.linear(x, c, s, b)

    static_x = xs[0].clone()
    graph, out = capture(lambda: eager(static_x))
    replay_matches_eager(graph, out, [static_x], [[x] for x in xs], eager)


def test_gelu_ffn_replays_from_a_graph(dev):
    # Four launches: quantization, up GEMM with GELU and row maxima, requantization,
    # down GEMM with the gate-residual epilogue.
    m, h, f = 600, 512, 1024
    g = torch.Generator().manual_seed(5)
    cu, su = quantize_weight_rows(torch.randn((f, h), generator=g) * 0.02)
    bu = (torch.randn(f, generator=g) * 0.01).to(torch.bfloat16)
    cd, sd = quantize_weight_rows(torch.randn((h, f), generator=g) * 0.02)
    bd = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
    gate = torch.rand(h, generator=g).to(torch.bfloat16)
    cu, su, bu, cd, sd, bd, gate = (t.to(dev) for t in (cu, su, bu, cd, sd, bd, gate))
    pairs = [
        (torch.randn((m, h), generator=g).to(torch.bfloat16).to(dev),
         torch.randn((m, h), generator=g).to(torch.bfloat16).to(dev))
        for _ in range(3)
    ]
    ex = RowFP8Execution("w8a8", activation_quantizer="hip")

    def eager(x, res):
        return fp8_ffn(ex, x, cu, su, bu, cd, sd, bd, gate, res, activation="gelu_tanh")

    static_x, static_res = pairs[0][0].clone(), pairs[0][1].clone()
    graph, out = capture(lambda: eager(static_x, static_res))
    replay_matches_eager(graph, out, [static_x, static_res], [list(p) for p in pairs], eager)
