"""int8 expert path on the GPU (needs an MI355X): moe_quant_rows_i8,
moe_grouped_gemm_i8 and moe_grouped_swiglu_i8 against the oracle.

Bars:
  * quantisation: bit-exact bytes and scales (every step is one rounded fp32
    operation, the rotation's butterflies in a fixed order);
  * int8 grouped GEMM: bit-exact bf16 output (the int32 accumulation is
    exact; the dequantisation is two fp32 multiplies in a fixed order);
  * int8 SwiGLU: the gate and up values are exact as above, so the only
    difference is the fp32 exponential: |got - ref| <= 2^-8 |ref| (one bf16
    output rounding) + 2^-20 |ref|.
Rows outside every group, and rows of skipped groups, stay untouched.
"""
import numpy as np
import pytest
import torch

import moe_route as M
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def inclusive(sizes, dev):
    return torch.tensor(np.cumsum(sizes), dtype=torch.int32, device=dev)


@pytest.mark.parametrize("R,K,had,mul", [
    (5, 16, 0, 1.0), (33, 3584, 0, 1.0), (33, 3584, 128, 1.0), (17, 8192, 0, 1.0),
    (17, 8192, 128, 1.0 / 128), (3, 16384, 128, 0.5), (9, 4224, 128, 1.0),
    (33, 3584, 16, 1.0 / 16), (6, 8192, 16, 1.0), (5, 48, 16, 1.0), (7, 12304, 16, 1.0),
    # widths whose K / 16 leaves part of the 256-thread block idle
    (9, 512, 16, 1.0), (5, 1536, 0, 0.5), (70, 3584, 0, 1.0), (3, 7680, 16, 1.0 / 16),
])
def test_quant_rows_bit_exact(cuda, R, K, had, mul):
    g = torch.Generator().manual_seed(R * 7 + K)
    x = (torch.randn(R, K, generator=g) * torch.rand(R, 1, generator=g) * 4).to(torch.bfloat16)
    x[0] = 0  # zero row: q = 0, s = 0
    x[-1, 3] = 300.0  # one outlier
    print("quant R=%d K=%d had=%d" % (R, K, had), flush=True)
    q, s = M.quant_rows_i8(x.to(cuda), hadamard=had, scale_mul=mul)
    torch.cuda.synchronize()
    rq, rs = O.quant_rows_i8(x, hadamard=had, scale_mul=mul)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy(), rs)


@pytest.mark.parametrize("K,had", [(256, 128), (3584, 16)])
def test_quant_rows_group_gating(cuda, K, had):
    G, rows = 4, 6
    x = torch.randn(G * rows, K).to(torch.bfloat16)
    counts = torch.tensor([3, 0, 1, 0], dtype=torch.int32, device=cuda)
    q = torch.full((G * rows, K), 99, dtype=torch.int8, device=cuda)
    s = torch.full((G * rows,), -1.0, device=cuda)
    M.quant_rows_i8(x.to(cuda), hadamard=had, group_rows=rows, group_counts=counts, q=q, scales=s)
    torch.cuda.synchronize()
    rq, rs = O.quant_rows_i8(x, hadamard=had)
    for gi, c in enumerate([3, 0, 1, 0]):
        sl = slice(gi * rows, (gi + 1) * rows)
        if c:
            assert np.array_equal(q[sl].cpu().numpy(), rq[sl])
            assert np.array_equal(s[sl].cpu().numpy(), rs[sl])
        else:
            assert bool((q[sl] == 99).all()) and bool((s[sl] == -1.0).all())


def make_i8(sizes, N, K, seed, extra_rows=0, n_tok=None):
    rng = np.random.default_rng(seed)
    G = len(sizes)
    Mr = int(sum(sizes)) + extra_rows
    a = rng.integers(-127, 128, size=(Mr, K)).astype(np.int8)
    w = rng.integers(-127, 128, size=(G, N, K)).astype(np.int8)
    n_tok = n_tok or Mr
    rs = (rng.random(n_tok) * 0.02 + 0.001).astype(np.float32)
    idx = rng.integers(0, n_tok, size=Mr).astype(np.int32)
    ws = (rng.random((G, N)) * 0.02 + 0.001).astype(np.float32)
    return a, w, rs, idx, ws


def bf16(x):
    return torch.as_tensor(x).to(torch.bfloat16)


@pytest.mark.parametrize("sizes,N,K", [
    ([5, 0, 130, 17, 1], 320, 256),            # small groups: 128-row tiles
    ([0, 200, 64, 3], 256, 1152),             # small groups, odd K steps (9)
    ([700, 1, 513, 1300], 300, 384),          # large groups: pipelined, 3 K steps
    ([2048, 1100], 512, 1024),                # large groups, 8 K steps
])
def test_grouped_gemm_i8_bit_exact(cuda, sizes, N, K):
    a, w, rs, idx, ws = make_i8(sizes, N, K, seed=sum(sizes) + N, extra_rows=5, n_tok=97)
    offs = np.cumsum(sizes)
    print("grouped_gemm_i8 sizes=%s N=%d K=%d" % (sizes, N, K), flush=True)
    out = torch.full((a.shape[0], N), 7.0, dtype=torch.bfloat16, device=cuda)
    t = lambda v: torch.from_numpy(v).to(cuda)
    M.grouped_gemm_i8(t(a), t(rs), t(w), t(ws), inclusive(sizes, cuda), a_rows=t(idx),
                      out=out)
    torch.cuda.synchronize()
    ref = bf16(O.grouped_gemm_i8(a, rs, w, ws, offs, a_rows=idx))
    Mg = int(offs[-1])
    assert torch.equal(out[:Mg].cpu(), ref[:Mg])
    assert bool((out[Mg:] == 7.0).all())


def test_grouped_gemm_i8_reads_rows_through_index(cuda):
    """a is a 97-row token table; 1000 operand rows read it through a_rows
    (as run() does with moe_permute's row_token instead of a gather)."""
    rng = np.random.default_rng(21)
    sizes, N, K, n_tok = [300, 0, 450, 250], 256, 384, 97
    a = rng.integers(-127, 128, size=(n_tok, K)).astype(np.int8)
    rs = (rng.random(n_tok) * 0.02 + 0.001).astype(np.float32)
    rows = rng.integers(0, n_tok, size=sum(sizes)).astype(np.int32)
    w = rng.integers(-127, 128, size=(len(sizes), N, K)).astype(np.int8)
    ws = (rng.random((len(sizes), N)) * 0.02 + 0.001).astype(np.float32)
    t = lambda v: torch.from_numpy(v).to(cuda)
    out = M.grouped_gemm_i8(t(a), t(rs), t(w), t(ws), inclusive(sizes, cuda), a_rows=t(rows))
    torch.cuda.synchronize()
    assert out.shape == (sum(sizes), N)
    ref = bf16(O.grouped_gemm_i8(a, rs, w, ws, np.cumsum(sizes), a_rows=rows))
    assert torch.equal(out.cpu(), ref)


def test_grouped_gemm_i8_identity_groups(cuda):
    sizes, N, K, T = [40, 64, 64, 10], 256, 512, 64
    a, w, rs, idx, ws = make_i8(sizes, N, K, seed=3)
    rng = np.random.default_rng(9)
    ident = rng.integers(-127, 128, size=(T, K)).astype(np.int8)
    ids = (rng.random(T) * 0.01 + 0.001).astype(np.float32)
    t = lambda v: torch.from_numpy(v).to(cuda)
    out = M.grouped_gemm_i8(t(a), t(rs), t(w), t(ws), inclusive(sizes, cuda), ident_a=t(ident),
                            ident_scales=t(ids), ident_m=T)
    torch.cuda.synchronize()
    ref = bf16(O.grouped_gemm_i8(a, rs, w, ws, np.cumsum(sizes), ident_a=ident,
                                 ident_scales=ids, ident_m=T))
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("sizes,N,K", [([3, 150, 0, 77], 384, 512), ([900, 1200], 256, 640)])
def test_grouped_swiglu_i8(cuda, sizes, N, K):
    rng = np.random.default_rng(len(sizes) * 31 + K)
    a, wg, rs, idx, wgs = make_i8(sizes, N, K, seed=K, n_tok=50)
    wu = rng.integers(-127, 128, size=wg.shape).astype(np.int8)
    wus = (rng.random(wgs.shape) * 0.02 + 0.001).astype(np.float32)
    rs = (rs * 0.05).astype(np.float32)  # keep g, u in silu's interesting range
    t = lambda v: torch.from_numpy(v).to(cuda)
    print("grouped_swiglu_i8 sizes=%s N=%d K=%d" % (sizes, N, K), flush=True)
    h = M.grouped_swiglu_i8(t(a), t(rs), t(wg), t(wgs), t(wu), t(wus), inclusive(sizes, cuda),
                            a_rows=t(idx))
    torch.cuda.synchronize()
    ref = O.grouped_swiglu_i8(a, rs, wg, wgs, wu, wus, np.cumsum(sizes), a_rows=idx).double()
    Mg = int(np.sum(sizes))
    got = h[:Mg].double().cpu()
    err = (got - ref[:Mg]).abs()
    lim = (2.0 ** -8 + 2.0 ** -20) * ref[:Mg].abs() + 1e-30
    assert bool((err <= lim).all()), float((err / lim).max())


def test_int8_chain_matches_float_product(cuda):
    """quant -> int8 GEMM -> (rotated) quant -> int8 GEMM at an expert-like
    shape is within the int8 rounding of the bf16 product: a sanity bound on
    the composition run(experts='int8') uses (the per-stage bars above are
    exact)."""
    T, H, Ni = 256, 1024, 512
    g = torch.Generator(device=cuda).manual_seed(1)
    x = torch.randn(T, H, generator=g, device=cuda).to(torch.bfloat16)
    wd = (torch.randn(1, H, Ni, generator=g, device=cuda) / Ni ** 0.5).to(torch.bfloat16)
    h = torch.randn(T, Ni, generator=g, device=cuda).to(torch.bfloat16)
    hq, hs = M.quant_rows_i8(h, hadamard=16)
    wq, wsc = M.quant_rows_i8(wd, hadamard=16, scale_mul=1 / 16)
    ends = torch.tensor([T], dtype=torch.int32, device=cuda)
    y = M.grouped_gemm_i8(hq, hs, wq, wsc, ends).float()
    ref = h.float() @ wd[0].float().t()
    rel = float((y - ref).norm() / ref.norm())
    assert rel < 0.02, rel
