"""The reference entry point run() (K:4067-4077) on the GPU: same inputs and
outputs as the reference, checked against a torch fp32 CPU evaluation of the
same routing (oracle) + SwiGLU experts + shared expert + combine."""
import numpy as np
import pytest
import torch

import moe_route as M
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def make(B=2, S=96, H=512, E=64, Ni=128, SNi=256, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    hs = r(B, S, H).to(torch.bfloat16)
    gw = r(E, H) / H ** 0.5                      # fp32 gate weight (K:4068)
    bias = r(E)                                  # e_score_correction_bias, plain randn
    eg = (r(E, Ni, H) / H ** 0.5).to(torch.bfloat16)
    eu = (r(E, Ni, H) / H ** 0.5).to(torch.bfloat16)
    ed = (r(E, H, Ni) / Ni ** 0.5).to(torch.bfloat16)
    sg = (r(SNi, H) / H ** 0.5).to(torch.bfloat16)
    su = (r(SNi, H) / H ** 0.5).to(torch.bfloat16)
    sd = (r(H, SNi) / SNi ** 0.5).to(torch.bfloat16)
    return hs, gw, bias, eg, eu, ed, sg, su, sd


def test_run_matches_reference_semantics(cuda):
    args = make()
    norm_min = 1e-6
    hs, gw, bias, eg, eu, ed, sg, su, sd = args
    out, logits = M.run(*[a.to(cuda) for a in args], norm_min)
    torch.cuda.synchronize()
    B, S, H = hs.shape
    T = B * S
    assert out.shape == (B, S, H) and out.dtype == torch.bfloat16
    assert logits.shape == (T, 64) and logits.dtype == torch.float32
    x = hs.view(T, H)
    # router logits: fp32-accurate through the hi/lo split (K:1786-1824)
    ref_l = (x.double() @ gw.double().t()).numpy()
    s_abs = (x.double().abs() @ gw.double().abs().t()).numpy()
    assert np.all(np.abs(logits.cpu().numpy() - ref_l) <= (2 * H * 2.0 ** -24 + 2.0 ** -16) * s_abs)
    # routing on the GPU's logits with the reference's rule (K:1857-1909)
    cfg = O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=norm_min)
    ids, wts = O.score_topk(logits.cpu().numpy(), bias.numpy(), 8, cfg)
    # expert SwiGLU MLPs + shared expert in fp32 on CPU
    xf = x.float()
    acc = (torch.nn.functional.silu(xf @ sg.float().t()) * (xf @ su.float().t())) @ sd.float().t()
    for t in range(T):
        for j in range(8):
            e = int(ids[t, j])
            h = torch.nn.functional.silu(xf[t] @ eg[e].float().t()) * (xf[t] @ eu[e].float().t())
            acc[t] += float(wts[t, j]) * (h @ ed[e].float().t())
    got = out.view(T, H).float().cpu()
    # bf16 expert matmuls on the GPU: tolerance of bf16 products over K=512/128
    err = (got - acc).abs()
    assert float(err.max()) <= 0.05 * float(acc.abs().max())
    assert float((err <= 0.02 + 0.05 * acc.abs()).float().mean()) >= 0.99   # the harness gate, K:1640-1642


@pytest.mark.parametrize("S,atol,dispatch,need,experts", [
    (1571, 0.010, "bf16", 0.99, "bf16"),
    (4096, 0.014, "bf16", 0.99, "bf16"),
    (8192, 0.012, "bf16", 0.99, "bf16"),
    # int8 experts, the reference's own precision choice (kernel.cu:61-66)
    (1571, 0.010, "bf16", 0.99, "int8"),
    (4096, 0.014, "bf16", 0.99, "int8"),
    (8192, 0.012, "bf16", 0.99, "int8"),
    # the mix's other two token counts (K:431-437: atol 0.320 at T = 2048, where the
    # reference itself runs nvfp4 experts, and 0.012 at T = 4904)
    (2048, 0.320, "bf16", 0.99, "int8"),
    (4904, 0.012, "bf16", 0.99, "int8"),
    # fp8 dispatch (e4m3fn rows, per-128 scales) is a precision trade-off the
    # reference's gate does not admit at T = 1571: 97.9% of elements inside
    # atol + 5% (measured on MI355X) against the 99% required.  The case pins
    # that measured fraction; bf16 dispatch is the drop-in.
    (1571, 0.010, "fp8", 0.975, "bf16"),
])
def test_run_at_reference_workload_shape(cuda, S, atol, dispatch, need, experts):
    """run() at the reference's own workload shapes: T in {1571, 2048, 4096,
    4904, 8192} (B=1), H = 8192, NE = 64, Ni = 3584, shared SNi = 7168 (K:133-136,
    K:4081-4126), with the harness's input distribution (K:1292-1297) and its
    gate for each T: |x - y| <= atol + 0.05|y| on >= 99%, atol = 0.010 /
    0.320 / 0.014 / 0.012 / 0.012 (K:431-437, K:1640-1642).  The expected output is a GPU fp32
    evaluation of the same routing (the oracle on the returned logits) and
    SwiGLU experts."""
    B, H, E, Ni, SNi = 1, 8192, 64, 3584, 7168
    g = torch.Generator(device=cuda).manual_seed(7)
    r = lambda *s: torch.randn(*s, generator=g, device=cuda)
    hs = r(B, S, H).to(torch.bfloat16)
    gw = r(E, H) / H ** 0.5
    bias = r(E)
    eg = (r(E, Ni, H) / H ** 0.5).to(torch.bfloat16)
    eu = (r(E, Ni, H) / H ** 0.5).to(torch.bfloat16)
    ed = (r(E, H, Ni) / Ni ** 0.5).to(torch.bfloat16)
    sg = (r(SNi, H) / H ** 0.5).to(torch.bfloat16)
    su = (r(SNi, H) / H ** 0.5).to(torch.bfloat16)
    sd = (r(H, SNi) / SNi ** 0.5).to(torch.bfloat16)
    print("run T=%d dispatch=%s experts=%s" % (B * S, dispatch, experts), flush=True)
    out, logits = M.run(hs, gw, bias, eg, eu, ed, sg, su, sd, 1e-20, dispatch=dispatch,
                        experts=experts)
    torch.cuda.synchronize()
    T = B * S
    x = hs.view(T, H).float()
    ids, wts = O.score_topk(logits.cpu().numpy(), bias.cpu().numpy(), 8,
                            O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=1e-20))
    ids_t = torch.from_numpy(ids).to(cuda).long()
    w_t = torch.from_numpy(wts).to(cuda)
    silu = torch.nn.functional.silu
    ref = (silu(x @ sg.float().t()) * (x @ su.float().t())) @ sd.float().t()
    for e in range(E):
        tok, slot = (ids_t == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        xe = x[tok]
        h = silu(xe @ eg[e].float().t()) * (xe @ eu[e].float().t())
        ref.index_add_(0, tok, w_t[tok, slot][:, None] * (h @ ed[e].float().t()))
    ok = (out.view(T, H).float() - ref).abs() <= atol + 0.05 * ref.abs()
    frac = float(ok.float().mean())
    print("T=%d dispatch=%s experts=%s: %.5f of elements inside the gate"
          % (T, dispatch, experts, frac))
    assert frac >= need, frac


def test_run_fp8_dispatch_small_shape(cuda):
    """run(..., dispatch="fp8"): routed rows travel as e4m3fn + per-128 scales
    into the expert GEMM.  Checked against the same CPU fp32 evaluation as the
    bf16 path, with the harness's gate form (K:1640-1642) at atol 0.02, and
    against the bf16 path itself."""
    args = make(seed=4)
    norm_min = 1e-6
    dev_args = [a.to(cuda) for a in args]
    out8, logits8 = M.run(*dev_args, norm_min, dispatch="fp8")
    out16, logits16 = M.run(*dev_args, norm_min)
    torch.cuda.synchronize()
    assert torch.equal(logits8, logits16)
    hs, gw, bias, eg, eu, ed, sg, su, sd = args
    B, S, H = hs.shape
    T = B * S
    cfg = O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=norm_min)
    ids, wts = O.score_topk(logits8.cpu().numpy(), bias.numpy(), 8, cfg)
    x = hs.view(T, H)
    xf = x.float()
    acc = (torch.nn.functional.silu(xf @ sg.float().t()) * (xf @ su.float().t())) @ sd.float().t()
    for t in range(T):
        for j in range(8):
            e = int(ids[t, j])
            h = torch.nn.functional.silu(xf[t] @ eg[e].float().t()) * (xf[t] @ eu[e].float().t())
            acc[t] += float(wts[t, j]) * (h @ ed[e].float().t())
    got = out8.view(T, H).float().cpu()
    err = (got - acc).abs()
    assert float((err <= 0.02 + 0.05 * acc.abs()).float().mean()) >= 0.99   # K:1640-1642
    d = (out8.float() - out16.float()).abs()
    assert float(d.max()) <= 0.1 * float(out16.float().abs().max())


def test_run_int8_experts_small_shape(cuda):
    """run(..., experts="int8") at a small shape with tokens spread over many
    experts (not the harness's 8 hot experts): against the CPU fp32 evaluation
    with the harness gate form at atol 0.02, and close to the bf16 path."""
    args = make(seed=5)
    norm_min = 1e-6
    dev_args = [a.to(cuda) for a in args]
    out8, logits8 = M.run(*dev_args, norm_min, experts="int8")
    out16, logits16 = M.run(*dev_args, norm_min)
    torch.cuda.synchronize()
    assert torch.equal(logits8, logits16)
    hs, gw, bias, eg, eu, ed, sg, su, sd = args
    B, S, H = hs.shape
    T = B * S
    ids, wts = O.score_topk(logits8.cpu().numpy(), bias.numpy(), 8,
                            O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=norm_min))
    xf = hs.view(T, H).float()
    acc = (torch.nn.functional.silu(xf @ sg.float().t()) * (xf @ su.float().t())) @ sd.float().t()
    for t in range(T):
        for j in range(8):
            e = int(ids[t, j])
            h = torch.nn.functional.silu(xf[t] @ eg[e].float().t()) * (xf[t] @ eu[e].float().t())
            acc[t] += float(wts[t, j]) * (h @ ed[e].float().t())
    err = (out8.view(T, H).float().cpu() - acc).abs()
    assert float((err <= 0.02 + 0.05 * acc.abs()).float().mean()) >= 0.99   # K:1640-1642
    with pytest.raises(RuntimeError):
        M.run(*dev_args, norm_min, experts="int8", dispatch="fp8")


@pytest.mark.parametrize("B,S,zero_bias", [(1, 1, False), (2, 96, True), (1, 333, True)])
def test_run_int8_experts_spread_routing_and_tiny_batch(cuda, B, S, zero_bias):
    """run(..., experts="int8") where the routing does NOT collapse onto 8
    whole experts (zero bias: groups of uneven size, rows read through
    row_token) and at T = 1.  Against the CPU fp32 evaluation, harness gate
    form at atol 0.02 (K:1640-1642)."""
    hs, gw, bias, eg, eu, ed, sg, su, sd = make(B=B, S=S, seed=11)
    if zero_bias:
        bias = torch.zeros_like(bias)
    norm_min = 1e-6
    args = (hs, gw, bias, eg, eu, ed, sg, su, sd)
    print("run int8 B=%d S=%d zero_bias=%s" % (B, S, zero_bias), flush=True)
    out, logits = M.run(*[a.to(cuda) for a in args], norm_min, experts="int8")
    torch.cuda.synchronize()
    T, H = B * S, hs.shape[-1]
    ids, wts = O.score_topk(logits.cpu().numpy(), bias.numpy(), 8,
                            O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=norm_min))
    if zero_bias:
        assert len(np.unique(ids)) > 8        # the groups really are spread
    xf = hs.view(T, H).float()
    acc = (torch.nn.functional.silu(xf @ sg.float().t()) * (xf @ su.float().t())) @ sd.float().t()
    for t in range(T):
        for j in range(8):
            e = int(ids[t, j])
            h = torch.nn.functional.silu(xf[t] @ eg[e].float().t()) * (xf[t] @ eu[e].float().t())
            acc[t] += float(wts[t, j]) * (h @ ed[e].float().t())
    err = (out.view(T, H).float().cpu() - acc).abs()
    assert float((err <= 0.02 + 0.05 * acc.abs()).float().mean()) >= 0.99
