"""The route-kernel probes behind bench.py --route-floor run the shipped K loop:
the whole-loop probe's raw tile equals moe_route's logits bit for bit (ragged
T, both x cache policies, since T spans more tiles than the temporal share),
and every variant launches and finishes.  Needs an MI355X."""
import pytest
import torch

import moe_route as M
from moe_route.configs import CONFIGS

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [300, 17000])
def test_loop_probe_computes_the_route_logits(cuda, T):
    c = CONFIGS["C4"]
    x, w, bias, _ = M.make_inputs(c, T=T, seed=9, device=cuda, with_y=False)
    print("route probe T=%d" % T, flush=True)
    logits = M.route(x, w, bias, c.k, c.cfg)[0]
    ws = torch.empty(c.E * c.H * 2, dtype=torch.uint8, device=cuda)
    got = torch.full((T, c.E), float("nan"), device=cuda)
    L = M.lib()
    s = M._stream(x)
    M._check(L.moe_route_probe(0, M._ptr(x), M._ptr(w), T, c.H, c.E, M._ptr(got), M._ptr(ws),
                               ws.numel(), s))
    torch.cuda.synchronize()
    assert torch.equal(got, logits)


def test_every_probe_variant_runs(cuda):
    c = CONFIGS["C4"]
    T = 1000
    x, w, _, _ = M.make_inputs(c, T=T, seed=10, device=cuda, with_y=False)
    ws = torch.empty(c.E * c.H * 2, dtype=torch.uint8, device=cuda)
    sink = torch.empty(T, c.E, device=cuda)
    L = M.lib()
    s = M._stream(x)
    for v in range(8):
        print("route probe variant %d" % v, flush=True)
        M._check(L.moe_route_probe(v, M._ptr(x), M._ptr(w), T, c.H, c.E,
                                   M._ptr(sink) if v % 2 else None, M._ptr(ws), ws.numel(), s))
        torch.cuda.synchronize()
