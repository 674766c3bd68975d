"""Parity of the HIP path against the CPU oracle (needs an MI355X).

Bars (from the path's contract):
  * top-k ids, counts, offsets, permutation indices, gathered bf16 rows and
    fp8 bytes/scales: bit-exact;
  * gate weights: within 1e-5 relative (in practice bit-exact: the kernel
    evaluates the same fp32 operation sequence);
  * logits: within the fp32 summation bound H * 2^-24 * sum|x||w| of the
    float64 product (bf16 inputs are exact in fp32);
  * combine: within one bf16 ulp of the fp32-accumulated CPU result plus
    the fp32 accumulation-order error 2^-19 * sum_j |w_j y_j|.
Selection is compared on identical logits (the GPU's own, copied to the
host), which pins it exactly; against the oracle's own CPU logits the ids
may differ only at near-ties, which is checked separately.
"""
import os

import numpy as np
import pytest
import torch

import moe_route as M
from moe_route.configs import CONFIGS, RouteCfg
from oracle import moe_oracle as O
import helpers

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def ocfg(c):
    return O.RouteCfg(c.scoring, c.renormalize, c.n_group, c.topk_group, c.route_scale,
                      c.norm_min)


def gold(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def to_np(t):
    return t.detach().cpu().numpy()


def assert_weights(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-30), \
        np.abs(got - want).max()


def assert_logits(got, x, w):
    xd, wd = x.double().cpu(), w.double().cpu()
    ref = (xd @ wd.t()).numpy()
    bound = x.shape[1] * 2.0 ** -24 * (xd.abs() @ wd.abs().t()).numpy() + 1e-30
    err = np.abs(to_np(got).astype(np.float64) - ref)
    assert np.all(err <= bound), (err / bound).max()


def assert_bf16_close(got, want, mag=None):
    """|got - want| <= one bf16 ulp of want + fp32 accumulation error.

    Both sides accumulate in fp32 (in different orders / with FMA), then
    round once to bf16.  mag = shared + sum_j |w_j| |y_j| bounds the terms;
    the fp32 sums differ by at most 2 * (k+1) * 2^-24 * mag, which can move
    the rounding by one ulp -- or by more under cancellation, where |want| is
    far below mag."""
    g = got.float().cpu()
    wv = want.float().cpu()
    ulp = wv.abs() * 2.0 ** -7  # >= one bf16 spacing at |want|
    acc = 0.0 if mag is None else mag.float().cpu() * 2.0 ** -19
    tol = ulp + acc + 1e-30
    assert torch.all((g - wv).abs() <= tol), ((g - wv).abs() / tol).max()


def combine_mag(y, pair_row, w, shared=None):
    w = np.abs(np.asarray(w, dtype=np.float32))
    pr = np.asarray(pair_row).copy()
    return O.combine(y.float().abs(), pr, w, shared=None if shared is None else shared.float().abs(),
                     out_dtype=torch.float32)


# --------------------------------------------------------------------- stage 1
@pytest.mark.parametrize("E", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("T,H", [(64, 1024), (300, 2048)])
def test_router_gemm(cuda, E, T, H):
    g = torch.Generator().manual_seed(E + T)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    logits = M.router_gemm(x.to(cuda), w.to(cuda))
    torch.cuda.synchronize()
    assert_logits(logits, x, w)


def test_route_fp32_weights_split(cuda):
    """fp32 gate weight through the hi/lo split (K:1786-1824): logits match the
    fp32-weight product within the bound plus the split's 2^-16 residual."""
    g = torch.Generator().manual_seed(11)
    T, H, E = 128, 1024, 64
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.randn(E, H, generator=g) * 0.02
    b = torch.randn(E, generator=g)
    cfg = RouteCfg(M.SCORING_SOFTMAX_BIAS, True, 1, 1, 1.0, 1e-20)
    logits, ids, wts, counts = M.route(x.to(cuda), w.to(cuda), b.to(cuda), 8, cfg)
    torch.cuda.synchronize()
    ref = (x.double() @ w.double().t()).numpy()
    s = (x.double().abs() @ w.double().abs().t()).numpy()
    err = np.abs(to_np(logits) - ref)
    assert np.all(err <= (2 * H * 2.0 ** -24 + 2.0 ** -16) * s)
    oi, ow = O.score_topk(to_np(logits), b.numpy(), 8, ocfg(cfg))
    assert np.array_equal(to_np(ids), oi)
    assert_weights(to_np(wts), ow)


@pytest.mark.parametrize("T,E,k,scoring", [(1, 8, 1, 0), (333, 256, 8, 1), (4096, 32, 4, 2)])
def test_route_fp32_weights_shapes(cuda, T, E, k, scoring):
    """fp32 weights at other shapes: E=256 makes the split GEMM N=512 (two
    256-column blocks); T=1 and T not a multiple of any tile."""
    g = torch.Generator().manual_seed(T + E)
    H = 1024
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.randn(E, H, generator=g) * 0.02
    b = torch.randn(E, generator=g) * 0.1
    cfg = {0: RouteCfg(), 1: RouteCfg(M.SCORING_SIGMOID_GROUP, True, 8, 4, 2.5),
           2: RouteCfg(M.SCORING_SOFTMAX_BIAS, True, 1, 1, 1.0, 1e-20)}[scoring]
    logits, ids, wts, counts = M.route(x.to(cuda), w.to(cuda), b.to(cuda), k, cfg)
    torch.cuda.synchronize()
    ref = (x.double() @ w.double().t()).numpy()
    s = (x.double().abs() @ w.double().abs().t()).numpy()
    assert np.all(np.abs(to_np(logits) - ref) <= (2 * H * 2.0 ** -24 + 2.0 ** -16) * s)
    oi, ow = O.score_topk(to_np(logits), b.numpy(), k, ocfg(cfg))
    assert np.array_equal(to_np(ids), oi)
    assert_weights(to_np(wts), ow)
    assert np.array_equal(to_np(counts), np.bincount(oi.ravel(), minlength=E))


# --------------------------------------------------------------------- stage 2
TOPK_CASES = [
    ("C2-softmax-E8-k2", 8, 2, RouteCfg(), None),
    ("C3-softmax-zipf-E128-k8", 128, 8, RouteCfg(), "zipf"),
    ("C4-sigmoid-group-E256-k8", 256, 8, RouteCfg(M.SCORING_SIGMOID_GROUP, True, 8, 4, 2.5), "randn"),
    ("softmax-full-E64-k4", 64, 4, RouteCfg(M.SCORING_SOFTMAX, False), None),
    ("softmax-bias-ref-E64-k8", 64, 8, RouteCfg(M.SCORING_SOFTMAX_BIAS, True, 1, 1, 1.0, 1e-20), "randn"),
    ("sigmoid-nogroup-E32-k4", 32, 4, RouteCfg(M.SCORING_SIGMOID_GROUP, False, 1, 1, 1.0), "randn"),
    ("sigmoid-group-E16-k2", 16, 2, RouteCfg(M.SCORING_SIGMOID_GROUP, True, 4, 2, 1.0), None),
    ("sigmoid-group-E128-k6", 128, 6, RouteCfg(M.SCORING_SIGMOID_GROUP, True, 8, 3, 2.5), "randn"),
    ("softmax-scaled-E256-k1", 256, 1, RouteCfg(M.SCORING_SOFTMAX, True, 1, 1, 1.5), None),
    # small expert groups shrink the lanes' width: 32- and 64-lane token groups
    # whose top reduction levels are xor shuffles instead of DPP row moves
    ("sigmoid-group-E64-ng32-k3", 64, 3, RouteCfg(M.SCORING_SIGMOID_GROUP, True, 32, 5, 1.0), "randn"),
    ("sigmoid-group-E256-ng64-k8", 256, 8, RouteCfg(M.SCORING_SIGMOID_GROUP, True, 64, 6, 2.5), "randn"),
    ("sigmoid-group-E128-ng64-k2", 128, 2, RouteCfg(M.SCORING_SIGMOID_GROUP, False, 64, 2, 1.0), None),
]


@pytest.mark.parametrize("name,E,k,cfg,bias", TOPK_CASES, ids=[c[0] for c in TOPK_CASES])
def test_topk_on_identical_logits(cuda, name, E, k, cfg, bias):
    g = torch.Generator().manual_seed(E * 7 + k)
    T = 1000  # not a multiple of the 64-token block
    logits = torch.randn(T, E, generator=g) * 1.7
    if bias == "zipf":
        b = torch.tensor([2 * np.log(1.0 / (e + 1)) for e in range(E)], dtype=torch.float32)
    elif bias == "randn":
        b = torch.randn(E, generator=g) * 0.1
    else:
        b = None
    ids, wts, counts = M.topk(logits.to(cuda), None if b is None else b.to(cuda), k, cfg)
    torch.cuda.synchronize()
    oi, ow = O.score_topk(logits.numpy(), None if b is None else b.numpy(), k, ocfg(cfg))
    assert np.array_equal(to_np(ids), oi)
    assert_weights(to_np(wts), ow)
    assert np.array_equal(to_np(counts), np.bincount(oi.ravel(), minlength=E))


@pytest.mark.parametrize("name", ["tie_softmax_bias", "tie_sigmoid_group"])
def test_topk_tie_stress_fixture(cuda, name):
    d = gold(name)
    E = d["logits"].shape[1]
    cfg = (RouteCfg(M.SCORING_SOFTMAX_BIAS, True, 1, 1, 1.0, 1e-20) if "bias" in name
           else RouteCfg(M.SCORING_SIGMOID_GROUP, True, 8, 4, 2.5))
    ids, wts, _ = M.topk(torch.from_numpy(d["logits"]).to(cuda),
                         torch.from_numpy(d["bias"]).to(cuda), 8, cfg)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(ids), d["ids"])
    assert_weights(to_np(wts), d["weights"])


def test_sigmoid_weights_bit_exact_wide_sweep(cuda):
    """Sigmoid scoring without renormalisation at unit scale outputs the
    sigmoid itself, so every weight must equal the oracle's det_sigmoid of
    its expert's logit bit for bit.  8M logits: random fp32 bit patterns with
    |x| <= 90 (both clamps and the whole exp range), a dense ramp through
    [-20, 20], and the clamp edges."""
    g = np.random.default_rng(5)
    n = 1 << 23
    mag = g.integers(0, 0x42B40000, size=n, dtype=np.uint32)  # |x| <= 90
    vals = (mag | (g.integers(0, 2, size=n, dtype=np.uint32) << 31)).view(np.float32)
    vals[: 1 << 20] = np.linspace(-20, 20, 1 << 20, dtype=np.float32)
    edges = np.array([-90, -86.5, -86, -85.99999, 0, 85.99999, 86, 86.5, 90, -0.0, 1e-30, -1e-30],
                     dtype=np.float32)
    vals[1 << 20: (1 << 20) + edges.size] = edges
    logits = torch.from_numpy(vals.reshape(-1, 8).copy())
    cfg = RouteCfg(M.SCORING_SIGMOID_GROUP, False, 1, 1, 1.0)
    ids, wts, _ = M.topk(logits.to(cuda), None, 8, cfg)
    torch.cuda.synchronize()
    ids_np = to_np(ids)
    picked = np.take_along_axis(logits.numpy(), ids_np.astype(np.int64), axis=1)
    want = O.det_sigmoid(picked)
    assert np.array_equal(to_np(wts).view(np.uint32), want.view(np.uint32))
    # and the ranking itself on a sample of rows
    rows = slice(0, 4096)
    oi, _ = O.score_topk(logits.numpy()[rows], None, 8, ocfg(cfg))
    assert np.array_equal(ids_np[rows], oi)


# --------------------------------------------------------------------- stages 3-4
def check_permutation(p, ids_np, E):
    rt, pr = O.permutation(ids_np)
    c, o = O.counts_offsets(ids_np, E)
    assert np.array_equal(to_np(p["row_token"]), rt)
    assert np.array_equal(to_np(p["pair_row"]), pr)
    assert np.array_equal(to_np(p["offsets"]), o)
    assert np.array_equal(to_np(p["counts"]), c)
    return rt


@pytest.mark.parametrize("T,E,k,H", [(1, 8, 2, 64), (1000, 8, 2, 256), (777, 128, 8, 512),
                                     (4096, 256, 8, 128), (513, 1024, 3, 64)])
def test_permute_bf16(cuda, T, E, k, H):
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :k].int()
    p = M.permute(x.to(cuda), ids.to(cuda), E)
    torch.cuda.synchronize()
    rt = check_permutation(p, ids.numpy(), E)
    assert torch.equal(p["xg"].cpu(), x[torch.from_numpy(rt).long()])


def test_permute_fp32_rows(cuda):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(300, 1024, generator=g)
    ids = torch.argsort(torch.rand(300, 8, generator=g), dim=1)[:, :2].int()
    p = M.permute(x.to(cuda), ids.to(cuda), 8)
    torch.cuda.synchronize()
    rt = check_permutation(p, ids.numpy(), 8)
    assert torch.equal(p["xg"].cpu(), x[torch.from_numpy(rt).long()])


@pytest.mark.parametrize("T,H", [(64, 7168), (333, 1024)])
def test_permute_fp8(cuda, T, H):
    g = torch.Generator().manual_seed(T)
    x = (torch.randn(T, H, generator=g) * torch.rand(T, 1, generator=g) * 4).to(torch.bfloat16)
    x[0, :128] = 0  # an all-zero block
    ids = torch.argsort(torch.rand(T, 256, generator=g), dim=1)[:, :8].int()
    p = M.permute(x.to(cuda), ids.to(cuda), 256, fp8=True)
    torch.cuda.synchronize()
    rt = check_permutation(p, ids.numpy(), 256)
    q, s = O.permute_fp8(x, rt)
    assert torch.equal(p["xg"].cpu(), q)
    assert torch.equal(p["scales"].cpu(), s)


def test_permute_degenerate_fixture(cuda):
    d = gold("degenerate")
    ids = torch.from_numpy(d["ids"])
    x = torch.randn(ids.shape[0], 64).to(torch.bfloat16)
    p = M.permute(x.to(cuda), ids.to(cuda), 16)
    torch.cuda.synchronize()
    for key in ("row_token", "pair_row", "offsets", "counts"):
        assert np.array_equal(to_np(p[key]), d[key]), key
    assert (d["counts"][4:] == 0).all() and (d["counts"][:4] == 100).all()


def test_permute_invalid_ids_are_dropped(cuda):
    ids = torch.tensor([[0, 3], [-1, 2], [3, 8], [1, 0]], dtype=torch.int32)
    x = torch.arange(4 * 64, dtype=torch.float32).view(4, 64).to(torch.bfloat16)
    p = M.permute(x.to(cuda), ids.to(cuda), 8)
    torch.cuda.synchronize()
    pr = to_np(p["pair_row"])
    assert pr[2] == -1 and pr[5] == -1
    valid = ids.numpy().ravel()
    valid = valid[(valid >= 0) & (valid < 8)]
    assert np.array_equal(to_np(p["counts"]), np.bincount(valid, minlength=8))
    assert to_np(p["offsets"])[-1] == 6


@pytest.mark.parametrize("T,k,E,dist", [
    (8192, 2, 8, "uniform"),      # C2: 16384 pairs
    (8193, 2, 8, "uniform"),      # a last block of 2 pairs
    (8192, 8, 64, "collapsed"),   # every token on the same 8 experts (run()'s harness routing)
    (1571, 8, 64, "uniform"),
    (3000, 8, 65, "uniform"),
    (2000, 4, 1, "uniform"),      # one expert
    (7, 3, 5, "uniform"),
])
def test_dispatch_index_paths(cuda, T, k, E, dist):
    """The index kernels give the oracle's stable order on uniform, collapsed
    and single-expert routing, with partial last blocks."""
    g = torch.Generator().manual_seed(T * 131 + E)
    if dist == "collapsed":
        ids = torch.argsort(torch.rand(E, generator=g))[:k].int().repeat(T, 1)
    else:
        ids = torch.randint(0, E, (T, k), generator=g, dtype=torch.int32)
    x = torch.empty(T, 64, dtype=torch.bfloat16, device=cuda)
    print("dispatch index T=%d k=%d E=%d %s" % (T, k, E, dist), flush=True)
    p = M.permute(x, ids.to(cuda), E, index_only=True)
    torch.cuda.synchronize()
    check_permutation(p, ids.numpy(), E)


@pytest.mark.parametrize("T,E", [(5000, 8), (100000, 8), (3000, 64)])
def test_dispatch_index_drops_invalid_ids(cuda, T, E):
    """Out-of-range ids get pair_row -1 and no row; the valid pairs keep the
    stable order among themselves."""
    g = torch.Generator().manual_seed(T + E)
    k = 2
    ids = torch.randint(-2, E + 2, (T, k), generator=g, dtype=torch.int32)
    x = torch.empty(T, 64, dtype=torch.bfloat16, device=cuda)
    p = M.permute(x, ids.to(cuda), E, index_only=True)
    torch.cuda.synchronize()
    flat = ids.numpy().ravel()
    ok = (flat >= 0) & (flat < E)
    order = np.flatnonzero(ok)[np.argsort(flat[ok], kind="stable")]
    want_pr = np.full(flat.size, -1, dtype=np.int32)
    want_pr[order] = np.arange(order.size, dtype=np.int32)
    assert np.array_equal(to_np(p["pair_row"]), want_pr)
    assert np.array_equal(to_np(p["row_token"])[:order.size], (order // k).astype(np.int32))
    c = np.bincount(flat[ok], minlength=E)
    assert np.array_equal(to_np(p["counts"]), c)
    assert np.array_equal(to_np(p["offsets"]), np.concatenate([[0], np.cumsum(c)]))


def test_permute_empty(cuda):
    x = torch.empty(0, 64, dtype=torch.bfloat16, device=cuda)
    ids = torch.empty(0, 2, dtype=torch.int32, device=cuda)
    p = M.permute(x, ids, 8)
    torch.cuda.synchronize()
    assert to_np(p["offsets"]).tolist() == [0] * 9
    assert to_np(p["counts"]).tolist() == [0] * 8


def test_offsets_entry_point(cuda):
    c = torch.randint(0, 50, (200,), dtype=torch.int32)
    o = M.offsets(c.to(cuda))
    torch.cuda.synchronize()
    assert to_np(o).tolist() == [0] + np.cumsum(c.numpy()).tolist()


# --------------------------------------------------------------------- stage 5
@pytest.mark.parametrize("T,H,k", [(100, 256, 2), (64, 7168, 8), (33, 2048, 5), (1, 512, 1)])
def test_combine_bf16(cuda, T, H, k):
    g = torch.Generator().manual_seed(H + k)
    y = torch.randn(T * k, H, generator=g).to(torch.bfloat16)
    pr = torch.randperm(T * k, generator=g).int()
    w = torch.rand(T, k, generator=g)
    out = M.combine(y.to(cuda), pr.to(cuda), w.to(cuda))
    torch.cuda.synchronize()
    assert_bf16_close(out, O.combine(y, pr.numpy(), w.numpy()), combine_mag(y, pr.numpy(), w))


def test_combine_shared_and_missing_rows(cuda):
    g = torch.Generator().manual_seed(9)
    T, H, k = 50, 512, 4
    y = torch.randn(T * k, H, generator=g).to(torch.bfloat16)
    sh = torch.randn(T, H, generator=g).to(torch.bfloat16)
    pr = torch.randperm(T * k, generator=g).int()
    pr[::7] = -1
    w = torch.rand(T, k, generator=g)
    out = M.combine(y.to(cuda), pr.to(cuda), w.to(cuda), shared=sh.to(cuda))
    torch.cuda.synchronize()
    w_ref = w.clone().view(-1)
    w_ref[::7] = 0
    pr_ref = pr.clone()
    pr_ref[::7] = 0
    assert_bf16_close(out, O.combine(y, pr_ref.numpy(), w_ref.view(T, k).numpy(), shared=sh),
                      combine_mag(y, pr_ref.numpy(), w_ref.view(T, k).numpy(), shared=sh))


def test_c1_identity_experts_fixture(cuda):
    """C1 on the GPU path: identity experts, so combine(permute(x)) == x."""
    c = CONFIGS["C1"]
    d = gold("C1_full")
    x, w, _, _ = helpers.make_inputs(c, seed=0)
    assert helpers.sha(x) == str(d["sha_x"])
    ids, wts, counts = M.topk(torch.from_numpy(d["logits"]).to(cuda), None, c.k, c.cfg)
    p = M.permute(x.to(cuda), ids, c.E)
    out = M.combine(p["xg"], p["pair_row"], wts)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(ids), d["ids"])
    assert_weights(to_np(wts), d["weights"])
    for key in ("row_token", "pair_row", "offsets", "counts"):
        assert np.array_equal(to_np(p[key]), d[key]), key
    assert torch.allclose(out.cpu(), x, rtol=1e-6, atol=1e-6)


# --------------------------------------------------------------------- end to end
@pytest.mark.parametrize("name", ["C2", "C3", "C4", "C5"])
def test_end_to_end_cut_fixture(cuda, name):
    c = CONFIGS[name]
    d = gold(name + "_t64")
    x, w, bias, y = helpers.make_inputs(c, T=helpers.CUT_T, seed=0)
    assert helpers.sha(x) == str(d["sha_x"]) and helpers.sha(w) == str(d["sha_w"])
    r = M.route_dispatch_combine(x.to(cuda), w.to(cuda), None if bias is None else bias.to(cuda),
                                 y.to(cuda), c.k, c.cfg, fp8=c.fp8)
    torch.cuda.synchronize()
    assert_logits(r["logits"], x, w)
    # selection on the GPU's own logits is exact
    oi, ow = O.score_topk(to_np(r["logits"]), None if bias is None else bias.numpy(), c.k,
                          ocfg(c.cfg))
    assert np.array_equal(to_np(r["topk_ids"]), oi)
    assert_weights(to_np(r["topk_w"]), ow)
    # and agrees with the fixture (oracle's own CPU logits) -- no near-ties at T=64
    assert np.array_equal(to_np(r["topk_ids"]), d["ids"])
    for key in ("row_token", "pair_row", "offsets", "counts"):
        assert np.array_equal(to_np(r[key]), d[key]), key
    if c.fp8:
        assert helpers.sha(r["xg"]) == str(d["sha_xg_fp8"])
        assert np.array_equal(to_np(r["scales"]), d["scales"])
    else:
        assert helpers.sha(r["xg"]) == str(d["sha_xg"])
    assert_bf16_close(r["out"], O.combine(y, d["pair_row"], d["weights"]),
                      combine_mag(y, d["pair_row"], d["weights"]))


def test_deterministic_repeat(cuda):
    c = CONFIGS["C4"]
    x, w, bias, y = helpers.make_inputs(c, T=512, seed=1, device=cuda)
    a = M.route_dispatch_combine(x, w, bias, y, c.k, c.cfg)
    b = M.route_dispatch_combine(x, w, bias, y, c.k, c.cfg)
    torch.cuda.synchronize()
    for key in ("logits", "topk_ids", "topk_w", "row_token", "pair_row", "xg", "out"):
        assert torch.equal(a[key], b[key]), key
