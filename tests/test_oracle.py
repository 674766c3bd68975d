"""Pinning the CPU oracle (oracle/moe_oracle.py) -- CPU only.

The reference ships no tests or golden vectors for this path (its
correctness gate is the external SOL-ExecBench harness), so each oracle
function is pinned here by something other than its own formula:

| oracle function       | pinned by                                                       |
|-----------------------|-----------------------------------------------------------------|
| det_exp / det_sigmoid | float64 math.exp within 2 / 3 ulp; exact special values          |
| tree_sum              | math.fsum bound + a known answer that only pairwise order gives  |
| _stable_topk          | brute-force Python sort on inputs full of ties                    |
| score_topk SOFTMAX    | torch.topk / torch.softmax (library), sum of weights = 1          |
| score_topk SIGMOID_GROUP | brute-force group-subset enumeration; invariants; torch.sigmoid |
| score_topk SOFTMAX_BIAS | torch.softmax + bias; norm_min closed form                     |
| counts_offsets        | torch.bincount / cumsum                                          |
| permutation           | brute-force sort of (expert, pair) keys; bijection; stability     |
| fp8_quant_rows        | hand e4m3fn decoder + brute-force nearest-even over all 256 codes |
| combine               | identity experts return x (C1 closed form); float64 loop          |
| router_logits         | float64 matmul with the fp32 summation error bound               |
| group_bounds          | brute-force row -> group lookup (searchsorted); clamping cases    |
| grouped_gemm          | float64 per-row loop over each row's own group; identity weights |
|                       | return a; identity shortcut reads ident_a                         |
| grouped_swiglu        | float64 math.exp closed form x / (1 + e^-x) * u                   |
| dequant_fp8_rows      | hand e4m3fn decoder x scale in numpy fp32, hand bf16 nearest-even |
| fwht_blocks           | scipy.linalg.hadamard (Sylvester) matrix product; H H = 128 I     |
| quant_rows_i8         | hand rows (half-even ties, zero row, clamp); error <= s/2;        |
|                       | rotated pair / 128 contracts to the unrotated product             |
| grouped_gemm_i8       | brute-force Python integer loop; row index / identity groups;    |
|                       | dequantised float64 product                                      |
"""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

f32 = np.float32


def ulp_err(got, ref64):
    got = np.asarray(got, dtype=np.float64)
    spacing = np.spacing(np.abs(ref64).astype(f32)).astype(np.float64)
    return np.abs(got - ref64) / spacing


# ---------------------------------------------------------------- exp / sigmoid
def test_det_exp_accuracy():
    x = np.linspace(-86.0, 88.0, 400001).astype(f32)
    ref = np.exp(x.astype(np.float64))
    assert ulp_err(O.det_exp(x), ref).max() <= 2.0


def test_det_exp_special_values():
    assert O.det_exp(f32(0.0)) == f32(1.0)
    assert O.det_exp(f32(-86.5)) == 0.0 and O.det_exp(f32(-np.inf)) == 0.0
    assert np.isinf(O.det_exp(f32(88.5)))
    assert O.det_exp(f32(1.0)) == f32(math.e) or abs(float(O.det_exp(f32(1.0))) - math.e) < 3e-7
    # every finite result is a normal float
    x = np.linspace(-86.0, -80.0, 1001).astype(f32)
    y = O.det_exp(x)
    assert (y >= np.finfo(f32).tiny).all()


def test_det_sigmoid_accuracy():
    x = np.linspace(-86.0, 86.0, 200001).astype(f32)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert ulp_err(O.det_sigmoid(x), ref).max() <= 3.0
    assert O.det_sigmoid(f32(0.0)) == f32(0.5)
    assert O.det_sigmoid(f32(100.0)) == f32(1.0)


# ---------------------------------------------------------------- tree sum
def test_tree_sum_known_answer_and_bound():
    # pairwise: (1e8 + 1) + (-1e8 + 1) = 1e8 - 1e8 = 0 in fp32;
    # left-to-right would give 1.  Only the adjacent-pair tree yields 0.
    a = np.array([1e8, 1.0, -1e8, 1.0], dtype=f32)
    assert O.tree_sum(a) == 0.0
    rng = np.random.default_rng(0)
    v = rng.standard_normal((50, 256)).astype(f32)
    got = O.tree_sum(v).astype(np.float64)
    ref = np.array([math.fsum(r.astype(np.float64)) for r in v])
    bound = 8 * 2.0 ** -24 * np.abs(v).astype(np.float64).sum(axis=1)  # log2(256) levels
    assert (np.abs(got - ref) <= bound).all()


# ---------------------------------------------------------------- selection
def test_stable_topk_brute_force_with_ties():
    rng = np.random.default_rng(1)
    s = rng.integers(-3, 4, size=(200, 16)).astype(f32)
    got = O._stable_topk(s, 5)
    for r in range(s.shape[0]):
        want = sorted(range(16), key=lambda e: (-s[r, e], e))[:5]
        assert got[r].tolist() == want


def test_softmax_renorm_vs_torch():
    rng = np.random.default_rng(2)
    l = rng.standard_normal((300, 8)).astype(f32)
    cfg = O.RouteCfg(O.SCORING_SOFTMAX, True)
    ids, w = O.score_topk(l, None, 2, cfg)
    tv, ti = torch.topk(torch.from_numpy(l), 2, dim=1)
    assert np.array_equal(ids, ti.numpy())
    tw = torch.softmax(tv.double(), dim=1).numpy()
    assert np.allclose(w, tw, rtol=1e-6, atol=1e-7)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)


def test_softmax_full_vs_torch_and_prebias():
    rng = np.random.default_rng(3)
    l = rng.standard_normal((200, 128)).astype(f32)
    b = np.array([2 * math.log(1.0 / (e + 1)) for e in range(128)], dtype=f32)
    cfg = O.RouteCfg(O.SCORING_SOFTMAX, False)
    ids, w = O.score_topk(l, b, 8, cfg)
    s = torch.from_numpy(l + b).double()
    p = torch.softmax(s, dim=1)
    tv, ti = torch.topk(s, 8, dim=1)
    assert np.array_equal(ids, ti.numpy())
    assert np.allclose(w, torch.gather(p, 1, ti).numpy(), rtol=2e-6, atol=1e-9)
    # skew: the Zipf bias sends most pairs to the first experts
    counts, _ = O.counts_offsets(ids, 128)
    assert counts[:8].sum() > counts[64:].sum()


def _dsv3_brute(s_row, b_row, ng, tg, k):
    """DeepSeek-V3 group-limited top-k by enumerating every subset of groups:
    the kept subset is the one whose summed group scores is largest (inputs
    are continuous, so there are no ties)."""
    E = len(s_row)
    gs = E // ng
    bb = s_row + b_row
    gscore = [sum(sorted(bb[g * gs:(g + 1) * gs], reverse=True)[:2]) for g in range(ng)]
    best = max(itertools.combinations(range(ng), tg), key=lambda c: sum(gscore[g] for g in c))
    allowed = [e for g in best for e in range(g * gs, (g + 1) * gs)]
    return sorted(allowed, key=lambda e: -bb[e])[:k]


def test_sigmoid_group_brute_force():
    rng = np.random.default_rng(4)
    E, ng, tg, k = 32, 8, 3, 4
    l = rng.standard_normal((150, E)).astype(f32)
    b = (rng.standard_normal(E) * 0.1).astype(f32)
    cfg = O.RouteCfg(O.SCORING_SIGMOID_GROUP, True, ng, tg, 2.5)
    ids, w = O.score_topk(l, b, k, cfg)
    s = O.det_sigmoid(l)
    for t in range(l.shape[0]):
        assert ids[t].tolist() == _dsv3_brute(s[t].astype(np.float64), b.astype(np.float64),
                                              ng, tg, k)
    sig = torch.sigmoid(torch.from_numpy(l).double())
    ws = torch.gather(sig, 1, torch.from_numpy(ids).long())
    ref = (ws / ws.sum(1, keepdim=True) * 2.5).numpy()
    assert np.allclose(w, ref, rtol=2e-6)
    assert np.allclose(w.sum(1), 2.5, rtol=1e-6)


def test_sigmoid_group_invariants_dsv3_shape():
    rng = np.random.default_rng(5)
    E, ng, tg, k = 256, 8, 4, 8
    l = (rng.standard_normal((64, E)) * 1.7).astype(f32)
    b = (rng.standard_normal(E) * 0.1).astype(f32)
    ids, w = O.score_topk(l, b, k, O.RouteCfg(O.SCORING_SIGMOID_GROUP, True, ng, tg, 2.5))
    bb = O.det_sigmoid(l) + b
    for t in range(64):
        groups = set(int(e) // 32 for e in ids[t])
        assert len(groups) <= tg
        assert len(set(ids[t].tolist())) == k
        sel = bb[t, ids[t]]
        assert (np.diff(sel) <= 0).all()  # slots in descending score
        assert np.allclose(w[t].sum(), 2.5, rtol=1e-6)


def test_softmax_bias_reference_rule():
    rng = np.random.default_rng(6)
    l = rng.standard_normal((100, 64)).astype(f32)
    b = rng.standard_normal(64).astype(f32)
    ids, w = O.score_topk(l, b, 8, O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=0.0))
    c = torch.softmax(torch.from_numpy(l).double(), 1) + torch.from_numpy(b).double()
    tv, ti = torch.topk(c, 8, dim=1)
    assert np.array_equal(ids, ti.numpy())
    tot = tv.sum(1, keepdim=True)
    assert np.allclose(w, (tv / tot).numpy(), rtol=1e-5, atol=1e-6)
    # norm_min floor: w = c / max(sum c, norm_min)
    ids2, w2 = O.score_topk(l, b, 8, O.RouteCfg(O.SCORING_SOFTMAX_BIAS, norm_min=1e6))
    assert np.allclose(w2, (tv / 1e6).numpy(), rtol=1e-5)


# ---------------------------------------------------------------- counts / permutation
def test_counts_offsets_vs_torch():
    rng = np.random.default_rng(7)
    ids = rng.integers(0, 16, size=(77, 4)).astype(np.int32)
    c, o = O.counts_offsets(ids, 16)
    assert np.array_equal(c, torch.bincount(torch.from_numpy(ids).long().flatten(), minlength=16).numpy())
    assert o[0] == 0 and o[-1] == 77 * 4 and np.array_equal(np.diff(o), c)


def test_permutation_brute_force_and_stability():
    rng = np.random.default_rng(8)
    T, k, E = 50, 3, 6
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    rt, pr = O.permutation(ids)
    keys = sorted(range(T * k), key=lambda p: (ids.flat[p], p))
    assert rt.tolist() == [p // k for p in keys]
    assert sorted(pr.tolist()) == list(range(T * k))
    for p in range(T * k):
        assert rt[pr[p]] == p // k
    _, offs = O.counts_offsets(ids, E)
    for e in range(E):
        seg = rt[offs[e]:offs[e + 1]]
        assert (np.diff(seg) > 0).all()


# ---------------------------------------------------------------- fp8
def e4m3fn_decode(code):
    code = int(code)
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 15 and m == 7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


_CODES = [(c, e4m3fn_decode(c)) for c in range(256) if not math.isnan(e4m3fn_decode(c))]


def nearest_even_code_value(v):
    best = min(abs(v - d) for _, d in _CODES)
    cands = [(c, d) for c, d in _CODES if abs(v - d) == best]
    even = [d for c, d in cands if c & 1 == 0]
    return even[0] if even else cands[0][1]


def test_fp8_conversion_is_round_nearest_even():
    rng = np.random.default_rng(9)
    x = torch.from_numpy((rng.standard_normal((4, 256)) * 3).astype(f32)).to(torch.bfloat16)
    q, s = O.fp8_quant_rows(x)
    xf = x.float().view(4, 2, 128)
    for r in range(4):
        for b in range(2):
            amax = float(xf[r, b].abs().max())
            assert float(s[r, b]) == float(np.float32(np.float32(amax) / np.float32(448.0)))
            scaled = (xf[r, b] / s[r, b]).numpy()
            for i in range(0, 128, 7):
                got = e4m3fn_decode(q[r, b * 128 + i])
                assert got == nearest_even_code_value(float(scaled[i])), (r, b, i)
            # the block's absmax element lands on (about) 448
            top = max(abs(e4m3fn_decode(c)) for c in q[r, b * 128:(b + 1) * 128].tolist())
            assert top == 448.0


def test_fp8_zero_block():
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    q, s = O.fp8_quant_rows(x)
    assert float(s[0, 0]) == float(np.float32(1e-10) / np.float32(448.0))
    assert (q == 0).all()


# ---------------------------------------------------------------- combine
def test_combine_identity_experts_returns_x():
    cfg = O.RouteCfg(O.SCORING_SOFTMAX, True)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(512, 1024, generator=g)
    w = torch.randn(8, 1024, generator=g) * 0.02
    r = O.route(x, w, None, 2, cfg)
    rt, pr = O.permutation(r["ids"])
    y = O.gather_rows(x, rt)          # identity experts: y = permuted x
    out = O.combine(y, pr, r["weights"])
    assert torch.allclose(out, x, rtol=1e-6, atol=1e-6)


def test_combine_vs_float64_loop():
    g = torch.Generator().manual_seed(1)
    T, k, H = 5, 3, 16
    y = torch.randn(T * k, H, generator=g)
    pr = torch.randperm(T * k, generator=g).int().numpy()
    w = torch.rand(T, k, generator=g).numpy().astype(f32)
    sh = torch.randn(T, H, generator=g)
    out = O.combine(y, pr, w, shared=sh)
    for t in range(T):
        ref = sh[t].double() + sum(float(w[t, j]) * y[pr[t * k + j]].double() for j in range(k))
        assert torch.allclose(out[t].double(), ref, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- router GEMM
def test_router_logits_error_bound():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(64, 2048, generator=g).to(torch.bfloat16)
    w = (torch.randn(16, 2048, generator=g) * 0.02).to(torch.bfloat16)
    got = O.router_logits(x, w).astype(np.float64)
    ref = (x.double() @ w.double().t()).numpy()
    bound = 2048 * 2.0 ** -24 * (x.double().abs() @ w.double().abs().t()).numpy()
    assert (np.abs(got - ref) <= bound).all()


def test_wsplit_hi_lo_reconstructs_fp32():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(8, 256, generator=g) * 0.02
    hi, lo = O.wsplit(w)
    rec = hi.double() + lo.double()
    # hi+lo carries 16 significant bits: relative error <= 2^-16
    assert ((rec - w.double()).abs() <= w.double().abs() * 2.0 ** -16).all()


# ---------------------------------------------------------------- grouped GEMM
def _ragged_offsets(sizes):
    return np.cumsum(np.asarray(sizes, dtype=np.int64)).astype(np.int32)


def test_group_bounds_brute_force_and_clamps():
    sizes = [3, 0, 5, 0, 0, 1, 7]
    offs = _ragged_offsets(sizes)
    M = int(offs[-1])
    b = O.group_bounds(offs, M)
    # row -> group by a lookup independent of the scan: first group whose end exceeds the row
    for r in range(M):
        g = int(np.searchsorted(offs, r, side="right"))
        assert b[g][0] <= r < b[g][1]
        assert sum(lo <= r < hi for lo, hi in b) == 1
    assert [hi - lo for lo, hi in b] == sizes
    # out-of-range ends are clamped into [0, M]; a group is never negative-sized;
    # each group starts at the previous raw end (clamped), as the device plan reads it
    assert O.group_bounds(np.array([5, 2, 40], np.int32), 10) == [(0, 5), (5, 5), (2, 10)]
    assert O.group_bounds(np.array([-3, 4], np.int32), 4) == [(0, 0), (0, 4)]


def test_grouped_gemm_vs_float64_per_row_loop():
    g = torch.Generator().manual_seed(5)
    sizes = [4, 0, 9, 1, 0, 6]
    offs = _ragged_offsets(sizes)
    M, N, K, G = int(offs[-1]), 7, 12, len(sizes)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(G, N, K, generator=g).to(torch.bfloat16)
    got = O.grouped_gemm(a, w, offs).double().numpy()
    A, W = a.double().numpy(), w.double().numpy()
    for r in range(M):
        gi = int(np.searchsorted(offs, r, side="right"))
        for n in range(N):
            ref = math.fsum(A[r, kk] * W[gi, n, kk] for kk in range(K))
            bound = K * 2.0 ** -24 * sum(abs(A[r, kk] * W[gi, n, kk]) for kk in range(K))
            assert abs(got[r, n] - ref) <= bound + 1e-30


def test_grouped_gemm_identity_weights_and_shortcut():
    g = torch.Generator().manual_seed(6)
    sizes = [3, 5, 2]
    offs = _ragged_offsets(sizes)
    M, K, G = int(offs[-1]), 8, 3
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    eye = torch.eye(K).repeat(G, 1, 1).to(torch.bfloat16)
    assert torch.equal(O.grouped_gemm(a, eye, offs), a.float())
    # identity shortcut: the 5-row group reads ident_a instead of a
    ident = torch.randn(5, K, generator=g).to(torch.bfloat16)
    got = O.grouped_gemm(a, eye, offs, ident_a=ident, ident_m=5)
    assert torch.equal(got[3:8], ident.float())
    assert torch.equal(got[:3], a[:3].float()) and torch.equal(got[8:], a[8:].float())


def test_grouped_swiglu_closed_form():
    g = torch.Generator().manual_seed(7)
    sizes = [2, 3]
    offs = _ragged_offsets(sizes)
    M, N, K = 5, 4, 8
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    eye = torch.eye(N, K).repeat(2, 1, 1).to(torch.bfloat16)        # picks the first N columns
    two = (2 * torch.eye(N, K)).repeat(2, 1, 1).to(torch.bfloat16)
    h = O.grouped_swiglu(a, eye, two, offs).double().numpy()
    A = a.double().numpy()
    for r in range(M):
        for n in range(N):
            x = A[r, n]
            assert abs(h[r, n] - x / (1.0 + math.exp(-x)) * 2 * x) <= 1e-6 * (1 + abs(h[r, n]))


def _bf16_rne_bits(v32):
    """fp32 -> bf16 bits by round to nearest even, in integer arithmetic."""
    u = np.asarray(v32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_dequant_fp8_rows_hand_decoder():
    rng = np.random.default_rng(12)
    x = torch.from_numpy((rng.standard_normal((3, 384)) * 5).astype(f32)).to(torch.bfloat16)
    q, s = O.fp8_quant_rows(x)
    got = O.dequant_fp8_rows(q, s).view(torch.int16).numpy().astype(np.uint16)
    codes = q.view(torch.uint8).numpy()
    sc = s.numpy()
    for r in range(3):
        for i in range(0, 384, 5):
            prod = np.float32(e4m3fn_decode(int(codes[r, i]))) * np.float32(sc[r, i // 128])
            assert got[r, i] == _bf16_rne_bits(np.float32(prod)), (r, i)
    # every one of the 256 codes (NaN codes excluded) at a scale that forces rounding
    allc = torch.arange(256, dtype=torch.uint8).view(2, 128)
    keep = [c for c in range(256) if (c & 0x7F) != 0x7F]
    sc2 = torch.full((2, 1), 1.0 / 3.0)
    got2 = O.dequant_fp8_rows(allc, sc2).view(torch.int16).numpy().astype(np.uint16).reshape(-1)
    for c in keep:
        prod = np.float32(e4m3fn_decode(c)) * np.float32(1.0 / 3.0)
        assert got2[c] == _bf16_rne_bits(np.float32(prod)), c


# ---------------------------------------------------------------------------
# int8 experts
# ---------------------------------------------------------------------------
def test_fwht_blocks_is_sylvester_hadamard():
    from scipy.linalg import hadamard
    rng = np.random.default_rng(11)
    v = rng.integers(-50, 50, size=(3, 256)).astype(f32)   # integer sums: exact in fp32
    Hm = hadamard(128).astype(np.float64)
    ref = np.concatenate([v[:, :128] @ Hm, v[:, 128:] @ Hm], axis=1)
    assert np.array_equal(O.fwht_blocks(v), ref.astype(f32))
    # involution up to the factor n: H H = 128 I
    assert np.array_equal(O.fwht_blocks(O.fwht_blocks(v)), (128 * v).astype(f32))
    H16 = hadamard(16).astype(np.float64)
    ref16 = (v.reshape(3, 16, 16).astype(np.float64) @ H16).reshape(3, 256)
    assert np.array_equal(O.fwht_blocks(v, 16), ref16.astype(f32))


def test_quant_rows_i8_hand_rows():
    # amax = 127 -> 127 / amax = 1: q = rint(v), ties to even
    row = np.zeros(16, dtype=f32)
    row[:8] = [127, 2.5, 3.5, -0.5, -1.5, 0.25, -127, 126.5]
    x = torch.tensor(np.stack([row, np.zeros(16, f32), row * 2]), dtype=torch.bfloat16)
    q, s = O.quant_rows_i8(x, scale_mul=0.5)
    assert q[0, :8].tolist() == [127, 2, 4, 0, -2, 0, -127, 126]
    assert q[1].tolist() == [0] * 16 and s[1] == 0.0
    assert s[0] == f32(0.5) and s[2] == f32(1.0)   # (amax / 127) * scale_mul
    assert q[2, :8].tolist() == [127, 2, 4, 0, -2, 0, -127, 126]


def test_quant_rows_i8_error_bound_and_rotation_fold():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 512, generator=g).to(torch.bfloat16)
    w = torch.randn(5, 512, generator=g).to(torch.bfloat16)
    q, s = O.quant_rows_i8(x)
    xf = x.double().numpy()
    assert np.all(np.abs(q * s[:, None].astype(np.float64) - xf) <= s[:, None] / 2 * (1 + 1e-6))
    assert np.abs(q).max() == 127
    # rotated on both sides, 1/128 folded into one scale: the same product
    ref = xf @ w.double().numpy().T
    for n in (16, 128):
        qx, sx = O.quant_rows_i8(x, hadamard=n)
        qw, sw = O.quant_rows_i8(w, hadamard=n, scale_mul=1 / n)
        got = (qx.astype(np.float64) @ qw.astype(np.float64).T) * sx[:, None] * sw[None, :]
        assert np.abs(got - ref).max() <= 0.02 * np.abs(ref).max()
    qx, sx = O.quant_rows_i8(x, hadamard=128)
    # the rotated operand is quantised to within half a step of the Hadamard
    # transform of its rows
    rot = O.fwht_blocks(x.float().numpy())
    assert np.all(np.abs(qx * sx[:, None].astype(np.float64) - rot) <= sx[:, None] / 2 * (1 + 1e-6))


def test_grouped_gemm_i8_brute_force():
    rng = np.random.default_rng(5)
    M, N, K, G = 11, 5, 8, 3
    a = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    w = rng.integers(-127, 128, size=(G, N, K)).astype(np.int8)
    rs = rng.random(7).astype(f32) + f32(0.5)
    idx = rng.integers(0, 7, size=M).astype(np.int32)
    ws = rng.random((G, N)).astype(f32)
    ident = rng.integers(-127, 128, size=(4, K)).astype(np.int8)
    ids = rng.random(4).astype(f32)
    offs = [3, 7, 9]                     # groups of 3, 4 (identity), 2 rows; rows 9-10 outside
    got = O.grouped_gemm_i8(a, rs, w, ws, offs, a_rows=idx, ident_a=ident,
                            ident_scales=ids, ident_m=4)
    bounds = [(0, 3), (3, 7), (7, 9)]
    for r in range(M):
        for n in range(N):
            gg = [g for g, (lo, hi) in enumerate(bounds) if lo <= r < hi]
            if not gg:
                assert got[r, n] == 0
                continue
            g = gg[0]
            if g == 1:
                arow, sa = ident[r - 3], ids[r - 3]
            else:
                arow, sa = a[idx[r]], rs[idx[r]]
            acc = sum(int(arow[k]) * int(w[g, n, k]) for k in range(K))
            assert got[r, n] == f32(acc) * (sa * ws[g, n])
    # against the dequantised float64 product
    deq = (a[idx].astype(np.float64) * rs[idx][:, None]) @ (w[0].astype(np.float64) * ws[0][:, None]).T
    assert np.allclose(got[:3], deq[:3], rtol=1e-6, atol=1e-6)
