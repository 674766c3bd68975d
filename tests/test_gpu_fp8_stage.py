"""The fp8 permute's two ways of writing its scales give the same bytes: with
moe_permute_fp8_workspace_bytes of workspace it stages them token-major and
copies whole destination rows afterwards; with only moe_permute_workspace_bytes
(or without offsets) it writes them into the k rows directly.  Ragged T, ids
outside [0, E) (fewer rows than pairs), both against the oracle.  Needs an
MI355X."""
import numpy as np
import pytest
import torch

import moe_route as M
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _permute_fp8(x, ids, E, ws_kind, with_offsets=True):
    L = M.lib()
    T, H = x.shape
    k = ids.shape[1]
    dev = x.device
    ns = T * k
    xg = torch.full((ns, H), 0xA5, dtype=torch.uint8, device=dev)
    sc = torch.full((ns, H // 128), -3.0, dtype=torch.float32, device=dev)
    rt = torch.empty(ns, dtype=torch.int32, device=dev)
    pr = torch.empty(ns, dtype=torch.int32, device=dev)
    offs = torch.empty(E + 1, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    n = (L.moe_permute_fp8_workspace_bytes(T, H, E, k) if ws_kind == "stage"
         else L.moe_permute_workspace_bytes(T, E, k))
    ws = torch.full((max(n, 256),), 0x5A, dtype=torch.uint8, device=dev)  # dirty
    P = M._ptr
    M._check(L.moe_permute(P(x), M.DTYPE_BF16, P(ids), T, H, E, k, M.DTYPE_FP8E4M3FN, P(xg), P(sc),
                           P(rt), P(pr), P(offs) if with_offsets else None, P(counts), P(ws), n,
                           M._stream(x)))
    torch.cuda.synchronize()
    return xg, sc, rt, offs


@pytest.mark.parametrize("T,H,E,k", [(1000, 7168, 256, 8), (77, 1024, 16, 2), (4097, 512, 64, 4),
                                     (33, 384, 8, 1)])
def test_staged_scales_match_direct_and_oracle(cuda, T, H, E, k):
    print("fp8 stage T=%d H=%d E=%d k=%d" % (T, H, E, k), flush=True)
    g = torch.Generator().manual_seed(T + H)
    x = (torch.randn(T, H, generator=g) * torch.rand(T, 1, generator=g) * 3).to(torch.bfloat16)
    ids = torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :k].int()
    if T > 5:
        ids[2, 0] = -1      # no row for this pair
        ids[5, k - 1] = E   # nor for this one
    x, ids = x.to(cuda), ids.to(cuda)
    a = _permute_fp8(x, ids, E, "stage")
    b = _permute_fp8(x, ids, E, "direct")
    c = _permute_fp8(x, ids, E, "stage", with_offsets=False)
    n = int(a[3][-1])
    assert n == int(((ids >= 0) & (ids < E)).sum())
    for o in (b, c):
        assert torch.equal(a[0][:n], o[0][:n]) and torch.equal(a[1][:n], o[1][:n])
    q, s = O.permute_fp8(x.cpu(), a[2][:n].cpu().numpy())
    assert torch.equal(a[0][:n].cpu(), q) and torch.equal(a[1][:n].cpu(), s)
    # rows past the last pair are left alone
    assert bool((a[1][n:] == -3.0).all())
