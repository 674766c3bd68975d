"""The small-E router GEMM + scoring kernel (E = 8 or 16, bf16 weights,
H % 256 == 0: the Mixtral shape C2 and C1-sized problems).

Its four waves each own a quarter of K and the partial tiles are added in
wave order, so its logits must equal, bit for bit, four standalone GEMMs over
the K quarters (moe_router_gemm, one K step after another, the same MFMA
and lane-to-k mapping) added ((p0 + p1) + p2) + p3 -- the two-kernel path's
result wherever it splits K in four, as at C2.  Selection on those logits must
equal the scoring kernel's (moe_topk) and the oracle's, bit for bit.  Cases:
token counts inside and at the edges of the 32-token tile (1, 31, 32, 33,
1000, 8192), H from 256 (one K step per quarter) to 8192,
every scoring rule (groups of 2 and 4 experts, and none), k = 2
(compile-time) and runtime k, bias present and absent.  Needs an MI355X."""
import numpy as np
import pytest
import torch

import moe_route as M
from moe_route.configs import RouteCfg, SCORING_SIGMOID_GROUP, SCORING_SOFTMAX, \
    SCORING_SOFTMAX_BIAS
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

CFGS = {
    "softmax": RouteCfg(SCORING_SOFTMAX, True),
    "softmax_norenorm": RouteCfg(SCORING_SOFTMAX, False),
    "softmax_bias": RouteCfg(SCORING_SOFTMAX_BIAS, True, norm_min=1e-6),
    "sigmoid_group4": RouteCfg(SCORING_SIGMOID_GROUP, True, 4, 2, 2.5),
    "sigmoid": RouteCfg(SCORING_SIGMOID_GROUP, True, 1, 1, 1.0),  # no groups
}


def quarter_sum_logits(x, w):
    """Four standalone GEMMs over the K quarters, added in quarter order."""
    L = M.lib()
    T, H = x.shape
    E = w.shape[0]
    kw = H // 4
    acc = None
    for q in range(4):
        xq = x[:, q * kw:(q + 1) * kw].contiguous()
        wq = w[:, q * kw:(q + 1) * kw].contiguous()
        p = torch.empty(T, E, dtype=torch.float32, device=x.device)
        rc = L.moe_router_gemm(M._ptr(xq), M._ptr(wq), T, kw, E, M._ptr(p), M._stream(x))
        assert rc == 0, L.moe_last_error_string()
        acc = p if acc is None else acc + p
    return acc


CASES = [
    # (E, H, T, rule, k)
    (8, 4096, 8192, "softmax", 2),        # C2
    (8, 4096, 1, "softmax", 2),
    (8, 4096, 33, "softmax_bias", 2),
    (8, 2048, 1000, "sigmoid_group4", 2),
    (8, 1024, 31, "softmax", 3),
    (8, 1024, 32, "softmax_norenorm", 1),
    (8, 1024, 4133, "sigmoid_pairs", 4),
    (8, 2048, 500, "sigmoid", 2),
    (16, 1024, 1000, "softmax", 8),
    (16, 2048, 33, "sigmoid_group4", 4),
    (16, 4096, 777, "sigmoid_pairs", 2),
    (16, 2048, 129, "softmax_bias", 5),
    (16, 8192, 64, "softmax", 2),
    (8, 256, 100, "softmax", 2),          # one K step per quarter
    (16, 512, 300, "softmax", 1),
]


@pytest.mark.parametrize("E,H,T,rule,k", CASES)
def test_route_small(cuda, E, H, T, rule, k):
    print("route_small E=%d H=%d T=%d rule=%s k=%d" % (E, H, T, rule, k), flush=True)
    if rule == "sigmoid_pairs":  # groups of two experts, the smallest the rule takes
        cfg = RouteCfg(SCORING_SIGMOID_GROUP, True, E // 2, E // 4, 1.0)
    else:
        cfg = CFGS[rule]
    L = M.lib()
    assert L.moe_route_workspace_bytes(T, H, E, 0) == 0
    g = torch.Generator().manual_seed(E * 1000 + T + k)
    x = torch.randn(T, H, generator=g).bfloat16().to(cuda)
    w = (torch.randn(E, H, generator=g) * 0.02).bfloat16().to(cuda)
    bias = None if T % 2 else (torch.randn(E, generator=g) * 0.1).to(cuda)
    lf, idf, wf, cf = M.route(x, w, bias, k, cfg)
    lq = quarter_sum_logits(x, w)
    ido, wo, co = M.topk(lf, bias, k, cfg)
    torch.cuda.synchronize()
    assert torch.equal(lf, lq), "logits differ from the K-quarter GEMMs added in order"
    assert torch.equal(idf, ido)
    assert torch.equal(wf, wo)
    assert torch.equal(cf, co)
    assert torch.equal(cf.long(), torch.bincount(idf.flatten().long(), minlength=E))
    ocfg = O.RouteCfg(cfg.scoring, cfg.renormalize, cfg.n_group, cfg.topk_group,
                      cfg.route_scale, cfg.norm_min)
    oi, ow = O.score_topk(lf.cpu().numpy(), None if bias is None else bias.cpu().numpy(), k,
                          ocfg)
    assert np.array_equal(idf.cpu().numpy(), oi)
    got = wf.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ow) <= 1e-5 * np.abs(ow) + 1e-30)
    # and the logits against the float64 product (fp32 summation bound)
    if T <= 1000:
        xd, wd = x.double().cpu(), w.double().cpu()
        ref = (xd @ wd.t()).numpy()
        bound = H * 2.0 ** -24 * (xd.abs() @ wd.abs().t()).numpy() + 1e-30
        assert np.all(np.abs(lf.cpu().numpy().astype(np.float64) - ref) <= bound)


def test_route_small_repeat(cuda):
    """Two calls in a row give the same bits (no state kept between calls)."""
    T, H, E, k = 2000, 4096, 8, 2
    g = torch.Generator().manual_seed(11)
    x = torch.randn(T, H, generator=g).bfloat16().to(cuda)
    w = (torch.randn(E, H, generator=g) * 0.02).bfloat16().to(cuda)
    cfg = CFGS["softmax"]
    a = M.route(x, w, None, k, cfg)
    b = M.route(x, w, None, k, cfg)
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.parametrize("H,T,k", [(1024, 512, 2), (1024, 1, 2), (4096, 1000, 3), (2048, 33, 1)])
def test_route_small_fp32_weights(cuda, H, T, k):
    """E = 8 with an fp32 weight (C1's toy route): the kernel loads the fp32
    rows and splits them hi = bf16(w), lo = bf16(w - hi) as its 16 fragment
    columns, and each logit is (sum of the four hi partials) + (sum of the
    four lo partials), each in K-quarter order (the reference's fold of the
    whole hi and lo products) -- equal, bit for bit, to the standalone GEMM
    over each quarter of each half (split here on the host side of the
    comparison) added that way; selection equals the scoring kernel's and the
    oracle's; no workspace."""
    print("route_small fp32 H=%d T=%d k=%d" % (H, T, k), flush=True)
    E = 8
    cfg = CFGS["softmax"]
    L = M.lib()
    assert L.moe_route_workspace_bytes(T, H, E, 1) == 0
    g = torch.Generator().manual_seed(H + T + k)
    x = torch.randn(T, H, generator=g).bfloat16().to(cuda)
    w = (torch.randn(E, H, generator=g) * 0.02).to(cuda)
    lf, idf, wf, cf = M.route(x, w, None, k, cfg)
    hi = w.bfloat16()
    lo = (w - hi.float()).bfloat16()
    kw = H // 4
    sums = []
    for half in (hi, lo):
        acc = None
        for q in range(4):
            xq = x[:, q * kw:(q + 1) * kw].contiguous()
            wq = half[:, q * kw:(q + 1) * kw].contiguous()
            p = torch.empty(T, E, dtype=torch.float32, device=cuda)
            rc = L.moe_router_gemm(M._ptr(xq), M._ptr(wq), T, kw, E, M._ptr(p), M._stream(x))
            assert rc == 0, L.moe_last_error_string()
            acc = p if acc is None else acc + p
        sums.append(acc)
    acc = sums[0] + sums[1]
    ido, wo, co = M.topk(lf, None, k, cfg)
    torch.cuda.synchronize()
    assert torch.equal(lf, acc), "logits differ from (sum of hi quarters) + (sum of lo quarters)"
    assert torch.equal(idf, ido) and torch.equal(wf, wo) and torch.equal(cf, co)
    ocfg = O.RouteCfg(cfg.scoring, cfg.renormalize, cfg.n_group, cfg.topk_group,
                      cfg.route_scale, cfg.norm_min)
    oi, _ = O.score_topk(lf.cpu().numpy(), None, k, ocfg)
    assert np.array_equal(idf.cpu().numpy(), oi)
    # the split reconstructs the fp32 weight to 2^-16 relative: the logits sit within
    # the fp32 summation bound plus that residual of the float64 product with w
    xd, wd = x.double().cpu(), w.double().cpu()
    ref = (xd @ wd.t()).numpy()
    mag = (xd.abs() @ wd.abs().t()).numpy()
    bound = 2 * H * 2.0 ** -24 * mag + 2.0 ** -16 * mag + 1e-30
    assert np.all(np.abs(lf.cpu().numpy().astype(np.float64) - ref) <= bound)
