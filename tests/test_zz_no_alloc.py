"""moe_permute_noalloc (the allocation-free permute: fixed device scratch
instead of a caller workspace) against moe_permute, through the C ABI, on two
calls in a row -- the second smaller, so stale histograms left in the shared
scratch by the first would show.  bf16 and fp8 rows, C4-shaped routing.
Needs an MI355X."""
import ctypes

import pytest
import torch

import moe_route as M
from moe_route.configs import CONFIGS

pytestmark = pytest.mark.gpu


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _run(L, x, ids, E, fp8, noalloc):
    T, H = x.shape
    k = ids.shape[1]
    dev = x.device
    ns = T * k
    if fp8:
        xg = torch.full((ns, H), 0x7F, dtype=torch.uint8, device=dev)
        sc = torch.full((ns, H // 128), -1.0, dtype=torch.float32, device=dev)
    else:
        xg = torch.full((ns, H), -7.0, dtype=torch.bfloat16, device=dev)
        sc = None
    rt = torch.full((ns,), -5, dtype=torch.int32, device=dev)
    pr = torch.full((ns,), -5, dtype=torch.int32, device=dev)
    offs = torch.full((E + 1,), -5, dtype=torch.int32, device=dev)
    cnt = torch.full((E,), -5, dtype=torch.int32, device=dev)
    od = M.DTYPE_FP8E4M3FN if fp8 else M.DTYPE_BF16
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if noalloc:
        rc = L.moe_permute_noalloc(_p(x), M.DTYPE_BF16, _p(ids), T, H, E, k, od, _p(xg), _p(sc),
                                   _p(rt), _p(pr), _p(offs), _p(cnt), stream)
    else:
        nws = L.moe_permute_workspace_bytes(T, E, k)
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
        rc = L.moe_permute(_p(x), M.DTYPE_BF16, _p(ids), T, H, E, k, od, _p(xg), _p(sc), _p(rt),
                           _p(pr), _p(offs), _p(cnt), _p(ws), nws, stream)
    assert rc == 0, L.moe_last_error_string()
    torch.cuda.synchronize()
    return dict(xg=xg, sc=sc, rt=rt, pr=pr, offs=offs, cnt=cnt)


@pytest.mark.parametrize("fp8", [False, True])
def test_permute_noalloc_matches_permute(cuda, fp8):
    L = M.lib()
    c = CONFIGS["C4"]
    E, k = c.E, c.k
    # first call large (4096 tokens, 1024 histogram blocks' worth of pairs of E=256),
    # second smaller and with a skewed expert mix
    for T, seed, skew in [(4096, 0, False), (777, 1, True)]:
        x, w, bias, _ = M.make_inputs(c, T=T, seed=seed, device=cuda, with_y=False)
        _, ids, _, _ = M.route(x, w, bias, k, c.cfg)
        if skew:
            ids = torch.where(ids % 3 == 0, ids // 16, ids)
            ids = torch.sort(ids, dim=1).values.contiguous()  # still k ids per token
        ref = _run(L, x, ids, E, fp8, noalloc=False)
        got = _run(L, x, ids, E, fp8, noalloc=True)
        print("noalloc T=%d fp8=%s" % (T, fp8), flush=True)
        for n in ref:
            if ref[n] is not None:
                assert torch.equal(got[n], ref[n]), (T, n)
        assert int(got["offs"][-1]) == T * k
