"""The fused router GEMM + scoring kernel (E = 256, H = 7168 with 128-token
tiles; E = 128, H = 2048 with 64-token tiles) against the
two-kernel path it replaces (moe_router_gemm, then moe_topk on the logits it
wrote) and against the oracle on the kernel's own logits.

The fused kernel accumulates K in the same order as the standalone GEMM, so
its logits are bit-identical to it, and selection on identical logits is
bit-identical (ids, weights, counts).  Cases: token counts that are not a
multiple of the 128-token tile (1, 77, 129, 1000, 4133), one full tile,
every scoring rule the fused path takes, k = 8 (compile-time) and k = 5
(runtime), bias present and absent.  Needs an MI355X."""
import ctypes

import numpy as np
import pytest
import torch

import moe_route as M
from moe_route.configs import RouteCfg, SCORING_SIGMOID_GROUP, SCORING_SOFTMAX, \
    SCORING_SOFTMAX_BIAS
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [(256, 7168), (128, 2048)]  # (E, H) the fused kernel takes

CFGS = {
    "sigmoid_group": RouteCfg(SCORING_SIGMOID_GROUP, True, 8, 4, 2.5),
    "softmax": RouteCfg(SCORING_SOFTMAX, True),
    "softmax_bias": RouteCfg(SCORING_SOFTMAX_BIAS, True, norm_min=1e-6),
}


def two_kernel_route(x, w, bias, k, cfg):
    L = M.lib()
    T, H = x.shape
    E = w.shape[0]
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    rc = L.moe_router_gemm(M._ptr(x), M._ptr(w), T, H, E, M._ptr(logits), M._stream(x))
    assert rc == 0, L.moe_last_error_string()
    ids, wts, counts = M.topk(logits, bias, k, cfg)
    return logits, ids, wts, counts


@pytest.mark.parametrize("T", [1, 77, 128, 129, 1000, 4133])
@pytest.mark.parametrize("rule", ["sigmoid_group", "softmax", "softmax_bias"])
@pytest.mark.parametrize("E,H", SHAPES)
def test_fused_route_matches_two_kernel_path(cuda, T, rule, E, H):
    cfg = CFGS[rule]
    if rule == "sigmoid_group" and E == 128:
        cfg = RouteCfg(SCORING_SIGMOID_GROUP, True, 4, 2, 2.5)  # 4 groups of 32
    k = 8 if T % 2 else 5
    g = torch.Generator().manual_seed(T * 7 + len(rule))
    x = torch.randn(T, H, generator=g).bfloat16().to(cuda)
    w = (torch.randn(E, H, generator=g) * 0.02).bfloat16().to(cuda)
    bias = None if T == 129 else (torch.randn(E, generator=g) * 0.1).to(cuda)
    L = M.lib()
    assert L.moe_route_workspace_bytes(T, H, E, 0) >= E * H * 2
    lf, idf, wf, cf = M.route(x, w, bias, k, cfg)
    lo, ido, wo, co = two_kernel_route(x, w, bias, k, cfg)
    torch.cuda.synchronize()
    print("fused E=%d H=%d T=%d rule=%s k=%d" % (E, H, T, rule, k), flush=True)
    assert torch.equal(lf, lo), "logits differ from the standalone GEMM"
    assert torch.equal(idf, ido)
    assert torch.equal(wf, wo)
    assert torch.equal(cf, co)
    assert torch.equal(cf.long(), torch.bincount(idf.flatten().long(), minlength=E))
    # the oracle's selection on the same logits
    ocfg = O.RouteCfg(cfg.scoring, cfg.renormalize, cfg.n_group, cfg.topk_group,
                      cfg.route_scale, cfg.norm_min)
    oi, ow = O.score_topk(lf.cpu().numpy(), None if bias is None else bias.cpu().numpy(), k,
                          ocfg)
    assert np.array_equal(idf.cpu().numpy(), oi)
    got = wf.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ow) <= 1e-5 * np.abs(ow) + 1e-30)


@pytest.mark.parametrize("E,H", SHAPES)
def test_fused_route_workspace_and_repeat(cuda, E, H):
    """Two calls in a row with the same workspace (rewritten by every call)
    give the same bits; the workspace is checked on the host."""
    T, k = 300, 8
    cfg = CFGS["sigmoid_group"] if E == 256 else CFGS["softmax"]
    g = torch.Generator().manual_seed(11)
    x = torch.randn(T, H, generator=g).bfloat16().to(cuda)
    w = (torch.randn(E, H, generator=g) * 0.02).bfloat16().to(cuda)
    w2 = (torch.randn(E, H, generator=g) * 0.02).bfloat16().to(cuda)
    bias = (torch.randn(E, generator=g) * 0.1).to(cuda)
    L = M.lib()
    nws = L.moe_route_workspace_bytes(T, H, E, 0)
    ws = torch.empty(nws, dtype=torch.uint8, device=cuda)
    c = M._ccfg(cfg)
    outs = []
    for ww in (w, w2, w):
        lg = torch.empty(T, E, dtype=torch.float32, device=cuda)
        ids = torch.empty(T, k, dtype=torch.int32, device=cuda)
        wts = torch.empty(T, k, dtype=torch.float32, device=cuda)
        rc = L.moe_route(M._ptr(x), M._ptr(ww), 0, M._ptr(bias), T, H, E, k, ctypes.byref(c),
                         M._ptr(lg), M._ptr(ids), M._ptr(wts), None, M._ptr(ws), nws,
                         M._stream(x))
        assert rc == 0, L.moe_last_error_string()
        outs.append((lg, ids, wts))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[2][0]) and torch.equal(outs[0][1], outs[2][1])
    assert not torch.equal(outs[0][0], outs[1][0])
    rc = L.moe_route(M._ptr(x), M._ptr(w), 0, M._ptr(bias), T, H, E, k, ctypes.byref(c),
                     M._ptr(outs[0][0]), M._ptr(outs[0][1]), M._ptr(outs[0][2]), None,
                     M._ptr(ws), nws - 256, M._stream(x))
    assert rc == -4  # MOE_ERR_WORKSPACE


@pytest.mark.parametrize("topk_group", [1, 2, 3, 4, 6, 8])
@pytest.mark.parametrize("k", [8, 6])
def test_fused_sigmoid_group_ties_and_kept_group_counts(cuda, topk_group, k):
    """E = 256 in 8 groups of 32 (one scoring lane per group, two tokens per
    lane group: with at most 4 kept groups the epilogue ranks only those,
    compacted into the lane group; with more it ranks all 8 lanes).  Router
    rows repeat every 37 experts and the bias every 37 entries, so many
    scores tie exactly, inside a group and across groups; ties go to the
    lower expert index.  The fused kernel must select what the one-token
    scoring kernel and the oracle select on the same logits, for 1 to 8
    kept groups."""
    E, H, T = 256, 7168, 300
    cfg = RouteCfg(SCORING_SIGMOID_GROUP, True, 8, topk_group, 2.5)
    g = torch.Generator().manual_seed(100 + 10 * topk_group + k)
    x = torch.randn(T, H, generator=g).bfloat16()
    base = (torch.randn(37, H, generator=g) * 0.02).bfloat16()
    w = base[torch.arange(E) % 37].contiguous()
    bias = (torch.randn(37, generator=g) * 0.1)[torch.arange(E) % 37].contiguous()
    x, w, bias = x.to(cuda), w.to(cuda), bias.to(cuda)
    lf, idf, wf, cf = M.route(x, w, bias, k, cfg)
    lo, ido, wo, co = two_kernel_route(x, w, bias, k, cfg)
    torch.cuda.synchronize()
    print("ties topk_group=%d k=%d" % (topk_group, k), flush=True)
    assert torch.equal(lf, lo)
    # exact ties are present: expert e and e + 37 have equal logits
    assert torch.equal(lf[:, 0], lf[:, 37])
    assert torch.equal(idf, ido)
    assert torch.equal(wf, wo)
    assert torch.equal(cf, co)
    ocfg = O.RouteCfg(cfg.scoring, cfg.renormalize, cfg.n_group, cfg.topk_group,
                      cfg.route_scale, cfg.norm_min)
    oi, ow = O.score_topk(lf.cpu().numpy(), bias.cpu().numpy(), k, ocfg)
    assert np.array_equal(idf.cpu().numpy(), oi)
    # every selected expert lies in one of the token's topk_group kept groups
    groups = idf.cpu().numpy() // 32
    assert all(len(set(r)) <= topk_group for r in groups)
