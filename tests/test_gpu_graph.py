"""The whole route -> permute -> combine step captured in a HIP graph and
replayed: every launch is stream-ordered and allocation-free, so capture
works; each replay is checked against the eager result, with eager work and
synchronisations between replays."""
import pytest
import torch

import moe_route as M
from moe_route.configs import CONFIGS

pytestmark = pytest.mark.gpu


def test_step_graph_capture_replays(cuda):
    c = CONFIGS["C4"]
    T = 4096
    x, w, bias, y = M.make_inputs(c, T=T, seed=3, device=cuda)
    plan = M.MoePlan(T, c.H, c.E, c.k, c.cfg, cuda)
    plan.step(x, w, bias, y)
    torch.cuda.synchronize()
    want = {n: getattr(plan, n).clone() for n in ("logits", "topk_ids", "topk_w", "row_token",
                                                   "pair_row", "offsets", "xg", "out")}
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.step(x, w, bias, y)          # warm up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        plan.step(x, w, bias, y)
    for rep in range(3):
        for n in want:                    # scribble over the outputs, eagerly
            getattr(plan, n).zero_()
        plan.permute(x, index_only=True)  # unrelated eager work on the same buffers
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n, v in want.items():
            assert torch.equal(getattr(plan, n), v), (rep, n)
