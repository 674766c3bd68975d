"""Full-size top-k id parity against the oracle's OWN route: the oracle
computes the logits on the CPU (torch fp32 matmul of the same bf16 inputs)
and selects on them; the GPU computes its logits on MFMA and selects on
those.  The two logit sets differ by fp32 summation order only, so top-k ids
may differ only at near-ties.  For every token whose ids differ the test
shows that the CPU scores hold a decision gap no larger than the measured
score difference can bridge, and that the measured logit difference is
inside the a-priori fp32 summation bound H * 2^-24 * sum|x||w|.

The tie rule (ties -> lower expert index) is K:1886; the scoring rules
K:1857-1909 generalised to the benchmark configurations.

A second count compares the oracle's deterministic exp / sigmoid (det_exp /
det_sigmoid) with torch.sigmoid / torch.softmax on the same CPU logits: how
many tokens a PyTorch-eager evaluation of the same routing math would route
differently, and that each such token is a near-tie within a few ulp.

Counts are printed (run with -s to see them).  Needs an MI355X."""
import json
import os

import numpy as np
import pytest
import torch

import moe_route as M
from moe_route.configs import CONFIGS
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

f32 = np.float32


def ocfg(c):
    return O.RouteCfg(c.scoring, c.renormalize, c.n_group, c.topk_group, c.route_scale,
                      c.norm_min)


def sel_scores(l, bias, cfg, sigmoid=O.det_sigmoid):
    """Selection scores (what top-k ranks, before any group mask)."""
    b = np.zeros(l.shape[1], f32) if bias is None else bias.astype(f32)
    if cfg.scoring == O.SCORING_SIGMOID_GROUP:
        return (sigmoid(l) + b[None, :]).astype(f32)
    return (l + b[None, :]).astype(f32)


def decision_gap(s, cfg, k):
    """Smallest score gap that a perturbation must close to change the ordered
    top-k of each row: consecutive gaps of the k+1 best scores, and, for
    group-limited selection, half the consecutive gaps of the topk_group+1 best
    group scores (a group score is a sum of two scores, so it moves twice as
    far).  Returns (gap [T], group_gap [T] or None)."""
    T, E = s.shape
    if cfg.scoring == O.SCORING_SIGMOID_GROUP and cfg.n_group > 1:
        ng, tg = cfg.n_group, cfg.topk_group
        g = s.reshape(T, ng, E // ng)
        top2 = -np.sort(-g, axis=-1)[..., :2]
        gs = (top2[..., 0] + top2[..., 1]).astype(np.float64)
        gsort = -np.sort(-gs, axis=1)
        ggap = (gsort[:, :tg] - gsort[:, 1:tg + 1]).min(axis=1) / 2.0
        order = np.argsort(-gs, axis=1, kind="stable")[:, :tg]
        keep = np.zeros((T, ng), bool)
        np.put_along_axis(keep, order, True, axis=1)
        s = np.where(np.repeat(keep, E // ng, axis=1), s, -np.inf)
    else:
        ggap = None
    ss = -np.sort(-s.astype(np.float64), axis=1)[:, :k + 1]
    gap = (ss[:, :k] - ss[:, 1:]).min(axis=1)
    return gap if ggap is None else np.minimum(gap, ggap)


def torch_eager_ids(l, bias, k, cfg):
    """The same routing math written with torch.sigmoid / torch.softmax
    (fp32, CPU) and a stable sort for the lower-index tie rule."""
    lt = torch.from_numpy(l)
    T, E = lt.shape
    b = torch.zeros(E) if bias is None else torch.from_numpy(bias)
    if cfg.scoring == O.SCORING_SIGMOID_GROUP:
        s = torch.sigmoid(lt) + b
        if cfg.n_group > 1:
            g = s.view(T, cfg.n_group, -1)
            gs = g.topk(2, dim=-1).values.sum(-1)
            order = torch.sort(-gs, dim=1, stable=True).indices[:, :cfg.topk_group]
            keep = torch.zeros(T, cfg.n_group, dtype=torch.bool).scatter_(1, order, True)
            s = s.masked_fill(~keep.repeat_interleave(E // cfg.n_group, dim=1), float("-inf"))
    elif cfg.scoring == O.SCORING_SOFTMAX:
        # softmax is monotone: top-k of softmax(l + b) is top-k of l + b, but the
        # rounded softmax can collapse near-equal logits into a tie
        s = torch.softmax(lt + b, dim=1)
    else:
        s = torch.softmax(lt, dim=1) + b
    return torch.sort(-s, dim=1, stable=True).indices[:, :k].numpy().astype(np.int32)


@pytest.mark.parametrize("name,seed", [("C2", 0), ("C3", 0), ("C4", 0), ("C5", 1)])
def test_full_size_ids_vs_oracle_cpu_logits(cuda, name, seed):
    c = CONFIGS[name]
    T, E, k, H = c.T, c.E, c.k, c.H
    x, w, bias, _ = M.make_inputs(c, seed=seed, device="cpu", with_y=False)
    xd, wd = x.to(cuda), w.to(cuda)
    bd = None if bias is None else bias.to(cuda)
    lg, ids_g, wt_g, _ = M.route(xd, wd, bd, k, c.cfg)
    torch.cuda.synchronize()
    lg = lg.cpu().numpy()
    ids_g = ids_g.cpu().numpy()
    wt_g = wt_g.cpu().numpy()
    del xd, wd

    cfg = ocfg(c.cfg)
    bn = None if bias is None else bias.numpy()
    lc = O.router_logits(x, w)                       # the oracle's own CPU logits
    ids_c, wt_c = O.score_topk(lc, bn, k, cfg)

    # a-priori fp32 summation bound on both logit sets, per element
    absprod = (x.float().abs() @ w.float().abs().t()).numpy()
    bound = 2.0 * H * 2.0 ** -24 * absprod.astype(np.float64)
    dl = np.abs(lg.astype(np.float64) - lc.astype(np.float64))
    assert bool((dl <= bound).all()), "GPU vs CPU logits outside the fp32 summation bound"

    # score difference the logit difference can cause: sigmoid' <= 1/4 (+ a few
    # ulp of det_sigmoid on each side); softmax-rule selection ranks l + b
    sg = sel_scores(lg, bn, cfg).astype(np.float64)
    sc = sel_scores(lc, bn, cfg).astype(np.float64)
    ds = np.abs(sg - sc).max(axis=1)
    gap = decision_gap(sc, cfg, k)
    diff_tok = np.nonzero((ids_g != ids_c).any(axis=1))[0]
    n_slots = int((ids_g != ids_c).sum())
    # a token may route differently only if its decision gap is within reach
    # of twice the largest score movement of that token
    unexplained = [int(t) for t in diff_tok if not gap[t] <= 2.0 * ds[t]]
    assert not unexplained, "ids differ at tokens %s beyond the score difference" % unexplained[:8]

    # weights of tokens routed identically: relative difference within what the
    # logit difference moves a weight (|d ln w| <= 2 * max |dl| for both rules)
    same = np.setdiff1d(np.arange(T), diff_tok)
    dlt = dl.max(axis=1)[same][:, None]
    rel = np.abs(wt_g[same].astype(np.float64) - wt_c[same]) / np.abs(wt_c[same])
    assert bool((rel <= 2.0 * dlt + 1e-6).all()), "weights of identically routed tokens differ"

    # PyTorch-eager selection (torch.sigmoid / torch.softmax) on the CPU logits
    ids_t = torch_eager_ids(lc, bn, k, cfg)
    det_vs_torch = np.nonzero((ids_t != ids_c).any(axis=1))[0]
    if cfg.scoring == O.SCORING_SIGMOID_GROUP:
        st = (torch.sigmoid(torch.from_numpy(lc)).numpy() + (0 if bn is None else bn)).astype(
            np.float64)
        dst = np.abs(st - sc).max(axis=1)
        bad = [int(t) for t in det_vs_torch if not gap[t] <= 2.0 * dst[t]]
        assert not bad, "torch.sigmoid selection differs beyond a tie at %s" % bad[:8]
    else:
        # softmax rounding can only merge scores whose logits differ by a few ulp
        bad = [int(t) for t in det_vs_torch if not gap[t] <= 1e-5 * (1 + np.abs(sc[t]).max())]
        assert not bad, "torch.softmax selection differs beyond a tie at %s" % bad[:8]

    rep = {
        "config": name, "seed": seed, "T": T, "E": E, "k": k,
        "tokens_differing": int(len(diff_tok)), "slots_differing": n_slots,
        "slots_total": T * k,
        "min_decision_gap_all_tokens": float(gap.min()),
        "max_gap_of_differing_token": float(gap[diff_tok].max()) if len(diff_tok) else None,
        "max_abs_logit_diff": float(dl.max()),
        "max_logit_diff_over_bound": float((dl / bound).max()),
        "tokens_det_vs_torch_differing": int(len(det_vs_torch)),
        "max_weight_rel_diff_same_ids": float(rel.max()) if len(same) else None,
    }
    print("\nFULLSIZE-PARITY " + json.dumps(rep), flush=True)
    out = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gpurun_out")
    if os.path.isdir(out):
        with open(os.path.join(out, "fullsize_parity_%s.json" % name), "w") as f:
            json.dump(rep, f)
