"""moe_route_permute (route + stable permute in one call) against the two
calls it stands for, moe_route then moe_permute: every output bit-identical
(logits, ids, weights, gathered bf16 rows or fp8 bytes + scales, row_token,
pair_row, offsets, counts).

Where the route is the fused kernel and k divides 256 with 256 / k tokens
fitting its token tile (E = 256: k in {2, 4, 8}; E = 128: k in {4, 8}), the
fused kernel's epilogue writes the permute's block histograms; on the
two-kernel route (other shapes, fp32 weights) the scoring kernel writes them
when k divides 256; the small-E route kernel (E = 8 or 16, H % 256 == 0)
writes one histogram per 32 tokens, which the index kernel sums per block
when 256 / k is a multiple of 32 and E x columns <= 8192.  These cases check both handoffs: token counts that end
inside a block of 256 pairs and inside a route tile (1, 33, 129, 1000,
4133), k = 5, 3 and (fused) 1 (no handoff), unfused shapes from E = 8 to
E = 256, C2's split-K GEMM and fp32 weights (the hi/lo split route of the
reference's run() shape).  Needs an MI355X."""
import ctypes

import pytest
import torch

import moe_route as M
from moe_route.configs import RouteCfg, SCORING_SIGMOID_GROUP, SCORING_SOFTMAX

pytestmark = pytest.mark.gpu

BF16, FP8 = M.DTYPE_BF16, M.DTYPE_FP8E4M3FN


def cfg_for(E):
    if E == 256:
        return RouteCfg(SCORING_SIGMOID_GROUP, True, 8, 4, 2.5)
    return RouteCfg(SCORING_SOFTMAX, True)


def outputs(T, H, E, k, fp8, dev):
    ns = T * k
    return {
        "logits": torch.full((T, E), -7.0, dtype=torch.float32, device=dev),
        "ids": torch.full((T, k), -9, dtype=torch.int32, device=dev),
        "w": torch.full((T, k), -7.0, dtype=torch.float32, device=dev),
        "xg": torch.zeros(max(ns, 1), H, dtype=torch.uint8 if fp8 else torch.bfloat16, device=dev),
        "scales": torch.zeros(max(ns, 1), H // 128, dtype=torch.float32, device=dev),
        "row_token": torch.full((max(ns, 1),), -9, dtype=torch.int32, device=dev),
        "pair_row": torch.full((max(ns, 1),), -9, dtype=torch.int32, device=dev),
        "offsets": torch.full((E + 1,), -9, dtype=torch.int32, device=dev),
        "counts": torch.full((E,), -9, dtype=torch.int32, device=dev),
    }


def wcode(w):
    return M.DTYPE_FP32 if w.dtype == torch.float32 else BF16


def run_pair(x, w, bias, k, cfg, fp8, index_only):
    """moe_route then moe_permute (the reference sequence)."""
    L = M.lib()
    T, H = x.shape
    E = w.shape[0]
    o = outputs(T, H, E, k, fp8, x.device)
    c = M._ccfg(cfg)
    nr = L.moe_route_workspace_bytes(T, H, E, wcode(w))
    wr = torch.empty(max(nr, 256), dtype=torch.uint8, device=x.device)
    P = M._ptr
    M._check(L.moe_route(P(x), P(w), wcode(w), P(bias), T, H, E, k, ctypes.byref(c), P(o["logits"]),
                         P(o["ids"]), P(o["w"]), None, P(wr), nr, M._stream(x)))
    npm = L.moe_permute_workspace_bytes(T, E, k)
    wp = torch.empty(max(npm, 256), dtype=torch.uint8, device=x.device)
    M._check(L.moe_permute(P(x), BF16, P(o["ids"]), T, H, E, k, FP8 if fp8 else BF16,
                           None if index_only else P(o["xg"]), P(o["scales"]) if fp8 else None,
                           P(o["row_token"]), P(o["pair_row"]), P(o["offsets"]), P(o["counts"]),
                           P(wp), npm, M._stream(x)))
    return o


def run_one(x, w, bias, k, cfg, fp8, index_only, ws_bytes=None):
    L = M.lib()
    T, H = x.shape
    E = w.shape[0]
    o = outputs(T, H, E, k, fp8, x.device)
    c = M._ccfg(cfg)
    need = L.moe_route_permute_workspace_bytes(T, H, E, k, wcode(w))
    # the workspace starts dirty: every call writes all it reads
    ws = torch.full((max(need, 256),), 0x5A, dtype=torch.uint8, device=x.device)
    P = M._ptr
    rc = L.moe_route_permute(P(x), P(w), wcode(w), P(bias), T, H, E, k, ctypes.byref(c),
                             P(o["logits"]), P(o["ids"]), P(o["w"]), FP8 if fp8 else BF16,
                             None if index_only else P(o["xg"]), P(o["scales"]) if fp8 else None,
                             P(o["row_token"]), P(o["pair_row"]), P(o["offsets"]), P(o["counts"]),
                             P(ws), need if ws_bytes is None else ws_bytes, M._stream(x))
    return rc, o


def check_equal(a, b, T, k, fp8, index_only):
    ns = T * k
    for key in ("logits", "ids", "w", "offsets", "counts"):
        assert torch.equal(a[key], b[key]), key
    for key in ("row_token", "pair_row"):
        assert torch.equal(a[key][:ns], b[key][:ns]), key
    if not index_only:
        assert torch.equal(a["xg"][:ns], b["xg"][:ns]), "xg"
        if fp8:
            assert torch.equal(a["scales"][:ns], b["scales"][:ns]), "scales"


CASES = [
    # (E, H, k, T, fp8, index_only)
    (256, 7168, 8, 1, False, False),
    (256, 7168, 8, 33, False, False),
    (256, 7168, 8, 129, True, False),
    (256, 7168, 8, 1000, False, True),
    (256, 7168, 8, 4133, False, False),
    (256, 7168, 4, 77, False, False),      # 64-token blocks
    (256, 7168, 2, 300, True, False),      # 128-token blocks = one tile
    (256, 7168, 5, 333, False, False),     # no handoff: 256 % 5 != 0
    (256, 7168, 1, 129, False, False),     # no handoff: 256-token blocks > tile
    (128, 2048, 8, 1, False, False),
    (128, 2048, 8, 65, False, False),
    (128, 2048, 8, 4133, True, False),
    (128, 2048, 4, 1000, False, False),    # 64-token blocks = one tile
    (128, 2048, 2, 200, False, False),     # no handoff: 128-token blocks > tile
    (64, 1024, 8, 1000, False, False),     # unfused route: the scoring kernel's handoff
    (64, 8192, 8, 1571, False, True),      # fp32 weights (hi/lo split): the run() shape
    (8, 4096, 2, 8192, False, False),      # C2's shape: the small-E route, 4 columns per block
    (8, 3968, 2, 8192, False, False),      # H % 256 != 0: split-K GEMM + scoring kernel
    (8, 1024, 2, 1001, True, False),       # a last block of 18 pairs
    (16, 448, 1, 300, False, False),       # scoring kernel: 256-token blocks, 8 passes
    (32, 512, 4, 97, False, False),
    (128, 1024, 8, 333, False, False),     # unfused at E = 128
    (256, 1024, 8, 555, False, False),     # unfused at E = 256 (sigmoid groups, 16-token passes)
    (256, 1024, 2, 257, True, False),
    (64, 1024, 3, 400, False, False),      # no handoff: 256 % 3 != 0
    # the small-E route (E = 8 / 16, H % 256 == 0): 32-token histogram columns
    (16, 2048, 8, 333, False, False),      # one column per permute block
    (16, 1024, 4, 1000, True, False),      # two columns per block
    (8, 2048, 1, 777, False, False),       # eight columns per block
    (8, 4096, 3, 500, False, False),       # no handoff: 256 % 3 != 0
    (16, 2048, 2, 20000, False, True),     # no handoff: 16 x 625 columns > 8192
    (8, 1024, 2, 512, False, False),       # C1's shape (fp32 weights: the small-E hi/lo route)
]


@pytest.mark.parametrize("E,H,k,T,fp8,index_only", CASES)
def test_route_permute_matches_two_calls(cuda, E, H, k, T, fp8, index_only):
    print("route_permute E=%d H=%d k=%d T=%d fp8=%d index_only=%d" % (E, H, k, T, fp8, index_only),
          flush=True)
    g = torch.Generator().manual_seed(E + k * 7 + T)
    x = torch.randn(T, H, generator=g).bfloat16().to(cuda)
    w = torch.randn(E, H, generator=g) * 0.02
    w = (w if H == 8192 or (E, H, T) == (8, 1024, 512) else w.bfloat16()).to(cuda)
    bias = (torch.randn(E, generator=g) * 0.1).to(cuda)
    cfg = cfg_for(E)
    ref = run_pair(x, w, bias, k, cfg, fp8, index_only)
    rc, got = run_one(x, w, bias, k, cfg, fp8, index_only)
    assert rc == 0, M.lib().moe_last_error_string()
    torch.cuda.synchronize()
    check_equal(got, ref, T, k, fp8, index_only)
    if T > 0:
        assert int(got["counts"].sum()) == T * k
        assert torch.equal(got["counts"].long(),
                           torch.bincount(got["ids"].flatten().long(), minlength=E))


def test_route_permute_repeat_and_workspace(cuda):
    """Two calls in a row on one plan give the same bits, the second after
    the first's workspace contents; a short workspace is rejected before any
    launch (outputs untouched)."""
    T, H, E, k = 2048, 7168, 256, 8
    g = torch.Generator().manual_seed(3)
    x = torch.randn(T, H, generator=g).bfloat16().to(cuda)
    w = (torch.randn(E, H, generator=g) * 0.02).bfloat16().to(cuda)
    bias = (torch.randn(E, generator=g) * 0.1).to(cuda)
    cfg = cfg_for(E)
    plan = M.MoePlan(T, H, E, k, cfg, cuda)
    plan.route_permute(x, w, bias)
    first = [t.clone() for t in (plan.topk_ids, plan.pair_row, plan.row_token, plan.offsets,
                                 plan.counts, plan.xg)]
    plan.route_permute(x, w, bias)
    torch.cuda.synchronize()
    for a, b in zip(first, (plan.topk_ids, plan.pair_row, plan.row_token, plan.offsets,
                            plan.counts, plan.xg)):
        assert torch.equal(a, b)
    need = M.lib().moe_route_permute_workspace_bytes(T, H, E, k, BF16)
    rc, o = run_one(x, w, bias, k, cfg, False, False, ws_bytes=need - 256)
    assert rc == -4  # MOE_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert int((o["ids"] == -9).sum()) == T * k
