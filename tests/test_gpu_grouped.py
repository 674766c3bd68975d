"""Expert grouped GEMM (moe_grouped_gemm / moe_grouped_swiglu) against the
oracle's grouped_gemm / grouped_swiglu (needs an MI355X).

Bars, written per element with ref = the oracle's fp32 result:
  * plain:  |got - ref| <= 2^-8 |ref| + K * 2^-23 * sum_k |a_k w_k|
    (bf16 output rounding of the fp32 accumulator, plus the fp32 summation
    error of either summation order);
  * swiglu: the same accumulation bound carried through h = silu(g) * u
    (|silu'| <= 1.1), plus 2^-8 |ref| output rounding and 2^-20 |ref| for the
    fp32 exponential.
Rows outside every group must be left untouched.
"""
import numpy as np
import pytest
import torch

import moe_route as M
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def inclusive(sizes, dev):
    return torch.tensor(np.cumsum(sizes), dtype=torch.int32, device=dev)


def make(sizes, N, K, seed, extra_rows=0, dev="cpu"):
    g = torch.Generator().manual_seed(seed)
    G = len(sizes)
    Mr = int(sum(sizes)) + extra_rows
    a = torch.randn(Mr, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(G, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    return a, w


def acc_bound(a, w, offs):
    """K * 2^-23 * sum_k |a_k w_k| per element, from the oracle on |a|, |w|."""
    K = a.shape[1]
    return K * 2.0 ** -23 * O.grouped_gemm(a.float().abs().to(torch.bfloat16),
                                           w.float().abs().to(torch.bfloat16), offs).double()


def check_plain(got, a, w, offs_np, ident_a=None, ident_m=0):
    ref = O.grouped_gemm(a, w, offs_np, ident_a, ident_m).double()
    bnd = acc_bound(ident_a if ident_m else a, w, offs_np) if not ident_m else None
    got = got.double().cpu()
    Mg = int(offs_np[-1])
    err = (got[:Mg] - ref[:Mg]).abs()
    if bnd is None:  # identity case: recompute the bound per group below
        bnd = torch.zeros_like(ref)
        for gi, (lo, hi) in enumerate(O.group_bounds(offs_np, a.shape[0])):
            if hi > lo:
                src = ident_a[:ident_m] if hi - lo == ident_m else a[lo:hi]
                bnd[lo:hi] = a.shape[1] * 2.0 ** -23 * (src.double().abs() @
                                                         w[gi].double().abs().t())
    lim = 2.0 ** -8 * ref[:Mg].abs() + bnd[:Mg] + 1e-30
    assert bool((err <= lim).all()), float((err / lim).max())


@pytest.mark.parametrize("sizes,N,K", [
    ([300, 0, 1, 17, 0, 256, 511], 256, 128),     # empty, 1-row, tile-exact and multi-tile groups
    ([5, 7, 9], 200, 64),                         # N not a multiple of the 256-wide tile
    ([1000], 512, 256),                           # one dense group
    ([0, 0, 40, 0], 64, 192),                     # mostly empty
])
def test_grouped_gemm_ragged(cuda, sizes, N, K):
    a, w = make(sizes, N, K, seed=len(sizes) + N)
    offs = inclusive(sizes, cuda)
    got = M.grouped_gemm(a.to(cuda), w.to(cuda), offs)
    torch.cuda.synchronize()
    check_plain(got, a, w, np.cumsum(sizes))


@pytest.mark.parametrize("G", [64, 65, 200, 256, 257, 300])
def test_grouped_gemm_group_lookup_paths(cuda, G):
    """Each block finds its group by a wave scan of the group ends (up to 64
    groups in one pass, up to 256 in passes of 64) or, beyond 256 groups, from
    the plan kernel's tile starts: all three agree with the oracle on ragged
    groups with empty ones among them."""
    rng = np.random.default_rng(G)
    sizes = rng.integers(0, 40, size=G)
    sizes[rng.random(G) < 0.3] = 0
    sizes[-1] = 300  # a multi-tile last group
    N, K = 128, 64
    a, w = make(list(sizes), N, K, seed=G)
    print("group lookup G=%d M=%d" % (G, int(sizes.sum())), flush=True)
    got = M.grouped_gemm(a.to(cuda), w.to(cuda), inclusive(sizes, cuda))
    torch.cuda.synchronize()
    check_plain(got, a, w, np.cumsum(sizes))


@pytest.mark.parametrize("sizes,N,K", [
    ([700, 0, 900], 256, 64),      # large groups (pipelined K loop), a single K step
    ([700, 0, 900], 200, 192),     # three K steps (odd), partial column tile
    ([1200, 333], 512, 320),       # five K steps
])
def test_grouped_gemm_large_groups_odd_k_steps(cuda, sizes, N, K):
    """More than 320 rows per group selects the 256-row tiles with the
    software-pipelined K loop; its tail handles odd and single K-step
    counts."""
    a, w = make(sizes, N, K, seed=sum(sizes) + K)
    offs = inclusive(sizes, cuda)
    got = M.grouped_gemm(a.to(cuda), w.to(cuda), offs)
    torch.cuda.synchronize()
    check_plain(got, a, w, np.cumsum(sizes))


def test_grouped_swiglu_large_groups_odd_k_steps(cuda):
    sizes, N, K = [900, 500], 160, 192
    g = torch.Generator().manual_seed(77)
    a = torch.randn(sum(sizes), K, generator=g).to(torch.bfloat16)
    wg = (torch.randn(2, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    wu = (torch.randn(2, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    offs_np = np.cumsum(sizes)
    h = M.grouped_swiglu(a.to(cuda), wg.to(cuda), wu.to(cuda), inclusive(sizes, cuda))
    torch.cuda.synchronize()
    uu = O.grouped_gemm(a, wu, offs_np).double()
    gg = O.grouped_gemm(a, wg, offs_np).double()
    ref = O.grouped_swiglu(a, wg, wu, offs_np).double()
    dg, du = acc_bound(a, wg, offs_np), acc_bound(a, wu, offs_np)
    lim = 1.1 * dg * uu.abs() + torch.nn.functional.silu(gg).abs() * du + dg * du + \
        (2.0 ** -8 + 2.0 ** -20) * ref.abs()
    err = (h.double().cpu() - ref).abs()
    assert bool((err <= lim + 1e-30).all()), float((err / (lim + 1e-30)).max())


def test_grouped_gemm_leaves_rows_outside_groups(cuda):
    sizes = [33, 0, 70]
    a, w = make(sizes, 128, 128, seed=11, extra_rows=50)
    offs = inclusive(sizes, cuda)
    out = torch.full((a.shape[0], 128), 7.0, dtype=torch.bfloat16, device=cuda)
    M.grouped_gemm(a.to(cuda), w.to(cuda), offs, out=out)
    torch.cuda.synchronize()
    assert bool((out[103:] == 7.0).all())
    check_plain(out, a, w, np.cumsum(sizes))


def test_grouped_gemm_empty_and_clamped_offsets(cuda):
    a, w = make([64], 64, 64, seed=12)
    # all groups empty: nothing is written
    out = torch.full((64, 64), 3.0, dtype=torch.bfloat16, device=cuda)
    M.grouped_gemm(a.to(cuda), w[:1].to(cuda), torch.zeros(1, dtype=torch.int32, device=cuda),
                   out=out)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
    # an end past M is clamped to M (no out-of-range rows are read or written)
    got = M.grouped_gemm(a.to(cuda), w[:1].to(cuda),
                         torch.tensor([1 << 20], dtype=torch.int32, device=cuda))
    torch.cuda.synchronize()
    check_plain(got, a, w[:1], np.array([64]))


def test_grouped_gemm_identity_shortcut(cuda):
    sizes = [40, 64, 0, 3]
    K, N = 128, 256
    a, w = make(sizes, N, K, seed=13)
    g = torch.Generator().manual_seed(14)
    ident = torch.randn(64, K, generator=g).to(torch.bfloat16)
    got = M.grouped_gemm(a.to(cuda), w.to(cuda), inclusive(sizes, cuda), ident_a=ident.to(cuda),
                         ident_m=64)
    torch.cuda.synchronize()
    check_plain(got, a, w, np.cumsum(sizes), ident_a=ident, ident_m=64)
    # the 64-row group used ident_a, not its own rows of a
    ref_ident = ident.double() @ w[1].double().t()
    assert float((got[40:104].double().cpu() - ref_ident).abs().max()) < 0.05


@pytest.mark.parametrize("sizes,N,K", [
    ([300, 0, 1, 17, 256], 256, 128),
    ([9, 70], 96, 64),                            # N not a multiple of the 128 output columns
])
def test_grouped_swiglu(cuda, sizes, N, K):
    g = torch.Generator().manual_seed(21 + N)
    G = len(sizes)
    Mr = int(sum(sizes))
    a = torch.randn(Mr, K, generator=g).to(torch.bfloat16)
    wg = (torch.randn(G, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    wu = (torch.randn(G, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    offs_np = np.cumsum(sizes)
    h = M.grouped_swiglu(a.to(cuda), wg.to(cuda), wu.to(cuda), inclusive(sizes, cuda))
    torch.cuda.synchronize()
    gg = O.grouped_gemm(a, wg, offs_np).double()
    uu = O.grouped_gemm(a, wu, offs_np).double()
    ref = O.grouped_swiglu(a, wg, wu, offs_np).double()
    dg, du = acc_bound(a, wg, offs_np), acc_bound(a, wu, offs_np)
    silu = torch.nn.functional.silu(gg)
    lim = 1.1 * dg * uu.abs() + silu.abs() * du + dg * du + (2.0 ** -8 + 2.0 ** -20) * ref.abs()
    err = (h.double().cpu() - ref).abs()
    assert bool((err <= lim + 1e-30).all()), float((err / (lim + 1e-30)).max())


def test_grouped_at_reference_expert_shape(cuda):
    """The reference's expert shapes (NE=64, H=8192, Ni=3584, T=1571 routed
    top-8: kernel.cu:133-136, 4081-4126) on real routing counts; 96 sampled
    rows checked against a GPU fp64 evaluation."""
    E, H, Ni, T, k = 64, 8192, 3584, 1571, 8
    gen = torch.Generator(device=cuda).manual_seed(3)
    ids = torch.stack([torch.randperm(E, generator=gen, device=cuda)[:k] for _ in range(T)])
    counts = torch.bincount(ids.flatten().long(), minlength=E)
    offs = torch.cumsum(counts, 0).to(torch.int32)
    Mr = T * k
    a = torch.randn(Mr, H, generator=gen, device=cuda).to(torch.bfloat16)
    wg = (torch.randn(E, Ni, H, generator=gen, device=cuda) / H ** 0.5).to(torch.bfloat16)
    wu = (torch.randn(E, Ni, H, generator=gen, device=cuda) / H ** 0.5).to(torch.bfloat16)
    wd = (torch.randn(E, H, Ni, generator=gen, device=cuda) / Ni ** 0.5).to(torch.bfloat16)
    h = M.grouped_swiglu(a, wg, wu, offs)
    y = M.grouped_gemm(h, wd, offs)
    torch.cuda.synchronize()
    rows = torch.randperm(Mr, generator=gen, device=cuda)[:96]
    grp = torch.searchsorted(offs.long(), rows, right=True)
    for r, gi in zip(rows.tolist(), grp.tolist()):
        ar = a[r].double()
        gv = wg[gi].double() @ ar
        uv = wu[gi].double() @ ar
        href = torch.nn.functional.silu(gv) * uv
        herr = (h[r].double() - href).abs()
        hlim = 2.0 ** -7 * href.abs() + 1e-3 * (gv.abs().max() + uv.abs().max())
        assert bool((herr <= hlim).all()), (r, float((herr / hlim).max()))
        yref = wd[gi].double() @ h[r].double()
        yerr = (y[r].double() - yref).abs()
        ylim = 2.0 ** -8 * yref.abs() + Ni * 2.0 ** -23 * (wd[gi].double().abs() @
                                                            h[r].double().abs())
        assert bool((yerr <= ylim + 1e-30).all()), (r, float((yerr / ylim).max()))


# ---------------------------------------------------------------- fp8 A operand
@pytest.mark.parametrize("sizes,N,K", [
    ([300, 0, 1, 17, 256], 256, 256),
    ([9, 70, 0], 200, 128),
])
def test_grouped_fp8_equals_bf16_on_dequantised_rows(cuda, sizes, N, K):
    """The fp8 kernels dequantise A in registers as bf16(q * s) and then run
    the same MFMA sequence as the bf16 kernels, so they must equal the bf16
    kernels fed the oracle's dequantised rows bit for bit."""
    g = torch.Generator().manual_seed(31 + N)
    G, Mr = len(sizes), int(sum(sizes))
    x = (torch.randn(Mr, K, generator=g) * 3).to(torch.bfloat16)
    q, sc = O.fp8_quant_rows(x)
    a_deq = O.dequant_fp8_rows(q, sc)
    wg = (torch.randn(G, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    wu = (torch.randn(G, N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    offs = inclusive(sizes, cuda)
    qd, sd = q.view(torch.uint8).to(cuda), sc.to(cuda)
    y8 = M.grouped_gemm_fp8(qd, sd, wg.to(cuda), offs)
    y16 = M.grouped_gemm(a_deq.to(cuda), wg.to(cuda), offs)
    h8 = M.grouped_swiglu_fp8(qd, sd, wg.to(cuda), wu.to(cuda), offs)
    h16 = M.grouped_swiglu(a_deq.to(cuda), wg.to(cuda), wu.to(cuda), offs)
    torch.cuda.synchronize()
    assert torch.equal(y8, y16)
    assert torch.equal(h8, h16)
    check_plain(y8, a_deq, wg, np.cumsum(sizes))


def test_fp8_permute_feeds_grouped_gemm(cuda):
    """moe_permute(fp8) -> moe_grouped_swiglu_fp8 on real routing equals the
    bf16 kernel on the oracle's dequantisation of the permuted rows."""
    T, H, E, k, N = 300, 256, 16, 4, 128
    g = torch.Generator().manual_seed(41)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).to(torch.int32)
    wg = (torch.randn(E, N, H, generator=g) / H ** 0.5).to(torch.bfloat16)
    wu = (torch.randn(E, N, H, generator=g) / H ** 0.5).to(torch.bfloat16)
    p = M.permute(x.to(cuda), ids.to(cuda), E, fp8=True)
    ends = p["offsets"][1:]
    h8 = M.grouped_swiglu_fp8(p["xg"], p["scales"], wg.to(cuda), wu.to(cuda), ends)
    rt, _ = O.permutation(ids.numpy())
    q, sc = O.permute_fp8(x, rt)
    h16 = M.grouped_swiglu(O.dequant_fp8_rows(q, sc).to(cuda), wg.to(cuda), wu.to(cuda), ends)
    torch.cuda.synchronize()
    assert torch.equal(p["xg"].cpu().view(torch.uint8), q.view(torch.uint8))
    assert torch.equal(h8, h16)


@pytest.mark.parametrize("sizes,N,K", [
    ([30, 0, 200, 77], 256, 512),        # small groups: 128-row tiles
    ([700, 1, 900], 320, 384),           # large groups: pipelined, odd K steps
])
def test_grouped_rows_equal_gathered_rows(cuda, sizes, N, K):
    """moe_grouped_gemm_rows / moe_grouped_swiglu_rows read operand row r as
    a[a_rows[r]]: bit-identical to the plain kernels on the gathered rows
    a[a_rows] (same data, same MFMA order)."""
    g = torch.Generator().manual_seed(sum(sizes))
    T = 113
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).to(cuda)
    rows = torch.randint(0, T, (sum(sizes),), generator=g, dtype=torch.int32).to(cuda)
    w = (torch.randn(len(sizes), N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(cuda)
    wu = (torch.randn(len(sizes), N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(cuda)
    offs = inclusive(sizes, cuda)
    xg = x[rows.long()].contiguous()
    print("grouped rows sizes=%s N=%d K=%d" % (sizes, N, K), flush=True)
    got = M.grouped_gemm(x, w, offs, a_rows=rows)
    ref = M.grouped_gemm(xg, w, offs)
    hg = M.grouped_swiglu(x, w, wu, offs, a_rows=rows)
    hr = M.grouped_swiglu(xg, w, wu, offs)
    torch.cuda.synchronize()
    assert got.shape == (sum(sizes), N)
    assert torch.equal(got, ref)
    assert torch.equal(hg, hr)
