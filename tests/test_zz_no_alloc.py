"""The allocation-free SwiGLU projection + requantization against the two
allocating entries it fuses (vflash_fp8_linear_swiglu, vflash_requant_rows_e4m3),
called through the C-ABI twice in a row, the second call smaller, so the static
scratch holds the first call's maxima when the second starts."""

import pytest
import torch

from vflash_amd import _lib, kernels
from vflash_amd._lib import ptr, stream_of
from vflash_amd.prepare import quantize_weight_rows

pytestmark = pytest.mark.gpu


def operands(m, hidden, inner, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, hidden), generator=g).to(torch.bfloat16)
    w, s = quantize_weight_rows(torch.randn((2 * inner, hidden), generator=g) * 0.02)
    b = (torch.randn(2 * inner, generator=g) * 0.01).to(torch.bfloat16)
    a, sa = kernels.quantize_rows(x.to(dev))
    return a, sa, w.to(dev), s.to(dev), b.to(dev)


def test_noalloc_equals_the_allocating_entries_on_two_calls(dev):
    for m, hidden, inner, seed in ((3000, 1024, 2048, 1), (700, 512, 1024, 2)):
        a, sa, w, s, b = operands(m, hidden, inner, seed, dev)
        ref_h, part_max = kernels.fp8_gemm_swiglu(a, sa, w, s, m, b)
        ref_codes, ref_scales = kernels.requant_rows(ref_h, part_max)
        h = torch.full_like(ref_h, float("nan"))
        codes = torch.full_like(ref_codes.view(torch.uint8), 0x55).view(torch.float8_e4m3fn)
        scales = torch.full_like(ref_scales, -1.0)
        _lib.call("vflash_fp8_linear_swiglu_quantize_noalloc", ptr(a), ptr(sa), a.stride(0), ptr(w),
                  ptr(s), w.stride(0), m, w.shape[0], w.shape[1], ptr(b), ptr(h), h.stride(0),
                  ptr(codes), ptr(scales), codes.shape[0], stream_of(dev))
        torch.cuda.synchronize()
        assert torch.equal(h, ref_h)
        assert torch.equal(codes.view(torch.uint8), ref_codes.view(torch.uint8))
        assert torch.equal(scales, ref_scales)


def test_noalloc_refuses_calls_beyond_its_scratch(dev):
    # 16 MiB hold 2^22 partial maxima; 2^15 rows of a 2 x 16384 projection need
    # 2^15 * 128 = 2^22 of them (allowed), one more row is refused before any launch.
    parts = int(_lib.library().vflash_swiglu_parts(2 * 16384))
    assert parts * 32768 * 4 == _lib.NOALLOC_SCRATCH_BYTES
    p = torch.empty(16, dtype=torch.float32, device=dev)
    addr = ptr(p)
    status = _lib.library().vflash_fp8_linear_swiglu_quantize_noalloc(
        addr, addr, 1024, addr, addr, 1024, 32769, 2 * 16384, 1024, None, addr, 16384, addr, addr,
        32784, stream_of(dev))
    assert status == _lib.VFLASH_ESCRATCH


def test_noalloc_replays_from_a_graph(dev):
    # The entry for callers under graph capture: a captured call (both launches,
    # the scratch's device address as a kernel argument) replayed on fresh
    # activation codes copied into the captured buffers gives the allocating
    # entries' bits on every replay, with eager launches between the replays.
    m, hidden, inner = 1500, 1024, 1536
    _, _, w, s, b = operands(m, hidden, inner, 3, dev)
    fresh = [operands(m, hidden, inner, 10 + i, dev)[:2] for i in range(3)]
    a, sa = fresh[0][0].clone(), fresh[0][1].clone()
    h = torch.empty((m, inner), device=dev, dtype=torch.bfloat16)
    codes = torch.empty((kernels.padded_rows(m), inner), device=dev, dtype=torch.float8_e4m3fn)
    scales = torch.empty((kernels.padded_rows(m), 1), device=dev, dtype=torch.float32)

    def call():
        _lib.call("vflash_fp8_linear_swiglu_quantize_noalloc", ptr(a), ptr(sa), a.stride(0), ptr(w),
                  ptr(s), w.stride(0), m, w.shape[0], w.shape[1], ptr(b), ptr(h), h.stride(0),
                  ptr(codes), ptr(scales), codes.shape[0], stream_of(dev))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()  # eager warm-up on a default-priority side stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for replay, (fa, fsa) in enumerate(fresh * 2):
        a.copy_(fa)
        sa.copy_(fsa)
        graph.replay()
        ref_h, part_max = kernels.fp8_gemm_swiglu(fa, fsa, w, s, m, b)
        ref_codes, ref_scales = kernels.requant_rows(ref_h, part_max)
        torch.cuda.synchronize()
        assert torch.equal(h, ref_h), f"replay {replay}: h differs"
        assert torch.equal(codes.view(torch.uint8), ref_codes.view(torch.uint8)), f"replay {replay}"
        assert torch.equal(scales, ref_scales), f"replay {replay}: scales differ"
