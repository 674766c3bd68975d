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


def test_two_streams_concurrently(cuda):
    """Two batches with their own plans (outputs and workspaces) on two
    default-priority streams at once give exactly the results of running them
    one after the other: the library keeps no shared device state."""
    c = CONFIGS["C3"]
    T = 2048
    ins = [M.make_inputs(c, T=T, seed=s, device=cuda) for s in (5, 6)]
    plans = [M.MoePlan(T, c.H, c.E, c.k, c.cfg, cuda) for _ in ins]
    for p, (x, w, bias, y) in zip(plans, ins):
        p.step(x, w, bias, y)
    torch.cuda.synchronize()
    names = ("logits", "topk_ids", "topk_w", "row_token", "pair_row", "offsets", "xg", "out")
    want = [{n: getattr(p, n).clone() for n in names} for p in plans]
    for p in plans:
        for n in names:
            getattr(p, n).zero_()
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(3):
        for s, p, (x, w, bias, y) in zip(streams, plans, ins):
            with torch.cuda.stream(s):
                p.step(x, w, bias, y)
    torch.cuda.synchronize()
    for p, wnt in zip(plans, want):
        for n, v in wnt.items():
            assert torch.equal(getattr(p, n), v), n


@pytest.mark.parametrize("experts", ["bf16", "int8"])
def test_run_graph_capture_replays(cuda, experts):
    """The whole reference entry point run() -- routing, index-only permute,
    expert and shared-expert GEMMs (bf16 or int8 with its quantisers),
    combine -- captured in one HIP graph: every stage is stream-ordered, with
    no host synchronisation and no memset.  Each replay equals the eager call
    bit for bit, with eager calls (which reuse the same kernels and scribble
    over device memory) between the replays."""
    from test_gpu_run import make
    args = [a.to(cuda) for a in make(seed=9)]
    norm_min = 1e-6
    out_e, logits_e = M.run(*args, norm_min, experts=experts)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        M.run(*args, norm_min, experts=experts)        # warm up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_g, logits_g = M.run(*args, norm_min, experts=experts)
    for rep in range(3):
        M.run(*args, norm_min, experts=experts)        # eager work in between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits_g, logits_e), rep
        assert torch.equal(out_g, out_e), rep
