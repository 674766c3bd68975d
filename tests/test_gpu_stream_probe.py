"""The streaming probes behind bench.py --ceiling move the bytes they claim:
copy, gather mix (each vector to `ways` streams) and combine mix (the bf16 sum
of `ways` streams, fp32 accumulation in stream order) checked against torch,
in both launch shapes, at a size that is not a multiple of the block.
Needs an MI355X."""
import pytest
import torch

import moe_route as M

pytestmark = pytest.mark.gpu

SHAPES = [0, 0x100]  # one pass, MOE_PROBE_GRID_STRIDE


@pytest.mark.parametrize("shape", SHAPES)
def test_probe_outputs(cuda, shape):
    L = M.lib()
    s = M._stream(torch.empty(1, device=cuda))
    n, ways = 1000 * 256 + 77, 3                       # 16-byte vectors
    g = torch.Generator(device=cuda).manual_seed(5)
    src = torch.randn(ways * n * 8, generator=g, device=cuda).bfloat16()
    dst = torch.zeros(ways * n * 8, dtype=torch.bfloat16, device=cuda)
    print("probe shape=%#x n=%d ways=%d" % (shape, n, ways), flush=True)
    M._check(L.moe_stream_probe(4 | shape, M._ptr(src), M._ptr(dst), n, 1, s))
    torch.cuda.synchronize()
    assert torch.equal(dst[:n * 8], src[:n * 8])
    dst.zero_()
    M._check(L.moe_stream_probe(2 | shape, M._ptr(src), M._ptr(dst), n, ways, s))
    torch.cuda.synchronize()
    assert torch.equal(dst.view(ways, n * 8), src[:n * 8].expand(ways, n * 8))
    out = torch.zeros(n * 8, dtype=torch.bfloat16, device=cuda)
    M._check(L.moe_stream_probe(3 | shape, M._ptr(src), M._ptr(out), n, ways, s))
    torch.cuda.synchronize()
    v = src.view(ways, n * 8).float()
    ref = torch.zeros(n * 8, device=cuda)
    for j in range(ways):
        ref += v[j]
    assert torch.equal(out, ref.bfloat16())
    # write and read run without error and the sink stays untouched
    sink = torch.zeros(8, dtype=torch.bfloat16, device=cuda)
    M._check(L.moe_stream_probe(1 | shape, None, M._ptr(dst), n, ways, s))
    M._check(L.moe_stream_probe(0 | shape, M._ptr(src), M._ptr(sink), n, ways, s))
    torch.cuda.synchronize()
    assert not bool(sink.any())
