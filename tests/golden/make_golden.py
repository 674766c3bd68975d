"""Write the committed golden fixtures tests/golden/*.npz from the CPU oracle.

The reference holds no golden vectors for this path, so these fixtures are
the oracle's outputs on seeded inputs, committed so that (a) the oracle
cannot drift silently (tests/test_golden.py recomputes them) and (b) the GPU
parity tests have expected outputs without re-running the oracle.  Inputs
are not stored: they are re-drawn from the seed and checked by sha256.

Cases: C1 in full (T=512); T=64 cuts of C2-C5 with their real E, k and
scoring; tie-stress logits (values on a 0.25 grid) for two scoring rules;
a degenerate routing (all tokens on k experts, the rest empty).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.join(REPO, "ernie-evolve-results_amd"), os.path.join(REPO, "tests")]

from oracle import moe_oracle as O  # noqa: E402
from moe_route.configs import CONFIGS  # noqa: E402
import helpers  # noqa: E402


def ocfg(c):
    return O.RouteCfg(c.scoring, c.renormalize, c.n_group, c.topk_group, c.route_scale,
                      c.norm_min)


def config_case(name, T):
    c = CONFIGS[name]
    x, w, bias, y = helpers.make_inputs(c, T=T, seed=0)
    r = O.route(x, w, None if bias is None else bias.numpy(), c.k, ocfg(c.cfg))
    rt, pr = O.permutation(r["ids"])
    d = dict(logits=r["logits"], ids=r["ids"], weights=r["weights"], counts=r["counts"],
             offsets=r["offsets"], row_token=rt, pair_row=pr,
             sha_x=helpers.sha(x), sha_w=helpers.sha(w))
    if c.fp8:
        q, s = O.permute_fp8(x, rt)
        d["sha_xg_fp8"] = helpers.sha(q)
        d["scales"] = s.numpy()
    else:
        d["sha_xg"] = helpers.sha(O.gather_rows(x, rt))
    yy = O.gather_rows(x, rt) if y is None else y
    out = O.combine(yy, pr, r["weights"])
    d["sha_out"] = helpers.sha(out)
    return d


def tie_case(scoring):
    if scoring == O.SCORING_SOFTMAX_BIAS:
        logits = helpers.tie_stress_inputs(T=96, E=64).numpy()
        bias = np.zeros(64, dtype=np.float32)
        cfg, k = O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=1e-20), 8
    else:
        logits = helpers.tie_stress_inputs(T=96, E=256).numpy()
        bias = np.zeros(256, dtype=np.float32)
        cfg, k = O.RouteCfg(O.SCORING_SIGMOID_GROUP, True, 8, 4, 2.5), 8
    ids, w = O.score_topk(logits, bias, k, cfg)
    return dict(logits=logits, bias=bias, ids=ids, weights=w)


def degenerate_case():
    ids = helpers.degenerate_ids(T=100, E=16, k=4).numpy()
    counts, offsets = O.counts_offsets(ids, 16)
    rt, pr = O.permutation(ids)
    return dict(ids=ids, counts=counts, offsets=offsets, row_token=rt, pair_row=pr)


def main():
    cases = {"C1_full": config_case("C1", 512)}
    for n in ("C2", "C3", "C4", "C5"):
        cases[n + "_t64"] = config_case(n, helpers.CUT_T)
    cases["tie_softmax_bias"] = tie_case(O.SCORING_SOFTMAX_BIAS)
    cases["tie_sigmoid_group"] = tie_case(O.SCORING_SIGMOID_GROUP)
    cases["degenerate"] = degenerate_case()
    for name, d in cases.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **{k: np.asarray(v) for k, v in d.items()})
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
