"""CPU oracle for the MoE route -> dispatch -> combine path.

TEST INFRASTRUCTURE ONLY.  This module is the checker that the HIP kernels are
compared against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product library never
calls it and has no CPU fallback.

It restates, in numpy float32 arithmetic (every operation rounded to fp32,
no fused multiply-add) and torch fp32 matmul, the routing math of the
reference kernel ``sol-execbench/029_moe_sparse_routing_and_dispatch/kernel.cu``
(abbreviated K below), generalised to the scoring rules the benchmark
configurations name:

* router GEMM             K:4327-4339 (cublasGemmEx, fp32 accumulate)
* hi/lo weight split      K:1786-1824 (wsplit_kernel)
* softmax + bias + top-k  K:1857-1909 (topk_kernel: ties -> lower index K:1886,
                          w = c / max(sum c, norm_min) K:1909)
* histogram / offsets     K:1912-1919, K:2069-2086 (offsets_kernel scan)
* dispatch permutation    K:2109-2189 (dispatch_body: inv[s]=pos, tok[pos]=t)
* gather                  K:2216-2230 (gather_body)
* combine                 K:2365-2428 (combine_kernel: acc = shared, acc += w*y)
* fp8 A dequantisation   bf16(q * s) per 1x128 block, the inverse of the fp8 permute
* expert grouped GEMM     moe_gemm.h:66-95, moe_gemm.cu:616-650 (grouped_mm /
                          grouped_mm_pair over inclusive group ends offs; the
                          SwiGLU h = silu(g) * u of the expert MLP)
* int8 experts            per-row int8 quantisation with an optional block
                          Walsh-Hadamard rotation (the reference's xquant /
                          hquant / wquant, kernel.cu:61-66, kernel.cu:125-129,
                          moe_wq.h:150-188, here with per-row scales and
                          16- or 128-point blocks) and the int8 grouped GEMMs
                          (moe_int8.h:27-45): exact integer products, then
                          float(acc) * (row scale * column scale)

Two deliberate differences from the reference, shared by the HIP kernels:

1. The permutation is STABLE: inside an expert's segment, rows are ordered by
   ascending token (the reference orders them by atomic arrival, K:2155-2158).
   It equals ``argsort(ids.flatten(), stable=True)``.
2. exp and sigmoid are the deterministic fp32 routines ``det_exp`` /
   ``det_sigmoid`` below (Cody-Waite reduction + degree-7 Taylor polynomial),
   evaluated with exactly the same rounded operations on the GPU, so that
   selection on identical logits is bit-identical.

Pinning (which check fixes what) is listed in tests/test_oracle.py.  The
reference's own tests hold no golden vectors for this path, so the oracle is
pinned by closed forms, invariants, brute force and library routines.
"""
from __future__ import annotations

import numpy as np

try:  # torch is used only for fp32 matmul and the fp8 library conversion
    import torch
except Exception:  # pragma: no cover
    torch = None

f32 = np.float32

# ---------------------------------------------------------------------------
# deterministic exp / sigmoid (identical operation sequence in csrc/moe_math.h)
# ---------------------------------------------------------------------------
_h = float.fromhex
LOG2E = f32(_h("0x1.715476p+0"))
LN2_HI = f32(_h("0x1.62e4p-1"))          # 0x3F317200: 15 significant bits, k*LN2_HI exact
LN2_LO = f32(_h("0x1.7f7d1cp-20"))       # ln2 - LN2_HI, rounded to fp32
EXP_LO = f32(-86.0)                    # below: result 0 (keeps every result a normal float)
EXP_HI = f32(88.0)                     # above: +inf
SIG_CLAMP = f32(86.0)
# 1/n! for n = 7 .. 2, rounded to fp32
_TAYLOR = [f32(_h(c)) for c in ("0x1.a01a02p-13", "0x1.6c16c2p-10", "0x1.111112p-7",
                                  "0x1.555556p-5", "0x1.555556p-3", "0x1p-1")]


def det_exp(x):
    """exp(x) in fp32 from the published Cody-Waite method.

    k = rint(x*log2e); r = (x - k*ln2_hi) - k*ln2_lo;
    p = Horner(1/7!, ..., 1/2!, 1, 1)(r); exp = ldexp(p, k).
    Each step is one fp32-rounded mul or add (no FMA).  x < -86 -> 0,
    x > 88 -> +inf.  Mirrors ``moe_det_exp`` in csrc/moe_math.h.
    """
    x = np.asarray(x, dtype=f32)
    with np.errstate(over="ignore", invalid="ignore"):
        xc = np.clip(x, EXP_LO, EXP_HI).astype(f32)
        k = np.rint((xc * LOG2E).astype(f32)).astype(f32)
        r = (xc - (k * LN2_HI).astype(f32)).astype(f32)
        r = (r - (k * LN2_LO).astype(f32)).astype(f32)
        p = _TAYLOR[0]
        for c in _TAYLOR[1:]:
            p = ((p * r).astype(f32) + c).astype(f32)
        p = ((p * r).astype(f32) + f32(1.0)).astype(f32)
        p = ((p * r).astype(f32) + f32(1.0)).astype(f32)
        y = np.ldexp(p, k.astype(np.int32)).astype(f32)
    y = np.where(x < EXP_LO, f32(0.0), y)
    y = np.where(x > EXP_HI, f32(np.inf), y)
    return y.astype(f32)


def det_sigmoid(x):
    """1 / (1 + det_exp(-clamp(x, -86, 86))), fp32, correctly rounded divide."""
    x = np.asarray(x, dtype=f32)
    xc = np.clip(x, -SIG_CLAMP, SIG_CLAMP).astype(f32)
    e = det_exp(-xc)
    return (f32(1.0) / (f32(1.0) + e).astype(f32)).astype(f32)


def tree_sum(a):
    """Pairwise sum over the last axis (length a power of two): adjacent pairs
    first, i.e. ((a0+a1)+(a2+a3))+...; the order a 64-lane butterfly
    (xor 1, 2, 4, ...) over per-lane pairwise partials produces."""
    a = np.asarray(a, dtype=f32)
    n = a.shape[-1]
    assert n & (n - 1) == 0, "tree_sum needs a power-of-two length"
    while a.shape[-1] > 1:
        a = (a[..., 0::2] + a[..., 1::2]).astype(f32)
    return a[..., 0]


# ---------------------------------------------------------------------------
# scoring configuration
# ---------------------------------------------------------------------------
SCORING_SOFTMAX = 0        # Mixtral / Qwen3: top-k on (logit + bias), softmax weights
SCORING_SIGMOID_GROUP = 1  # DeepSeek-V3: sigmoid, +bias for selection, group-limited
SCORING_SOFTMAX_BIAS = 2   # reference run(): softmax, +bias after softmax, norm_min


class RouteCfg:
    """Mirror of ``moe_route_cfg`` in include/moe_route.h."""

    def __init__(self, scoring=SCORING_SOFTMAX, renormalize=True, n_group=1,
                 topk_group=1, route_scale=1.0, norm_min=0.0):
        self.scoring = int(scoring)
        self.renormalize = bool(renormalize)
        self.n_group = int(n_group)
        self.topk_group = int(topk_group)
        self.route_scale = float(route_scale)
        self.norm_min = float(norm_min)

    def __repr__(self):
        return ("RouteCfg(scoring=%d, renorm=%d, n_group=%d, topk_group=%d, "
                "scale=%g, norm_min=%g)" % (self.scoring, self.renormalize, self.n_group,
                                             self.topk_group, self.route_scale, self.norm_min))


def _stable_topk(score, k):
    """Indices of the k largest entries per row, descending; ties -> lower index
    (K:1886: ``ov > bv || (ov == bv && oi < bi)``)."""
    return np.argsort(-score, axis=-1, kind="stable")[:, :k].astype(np.int32)


# ---------------------------------------------------------------------------
# stage 1: router GEMM
# ---------------------------------------------------------------------------
def router_logits(x, w):
    """logits[T,E] = x[T,H] . w[E,H]^T in fp32 (K:4327-4339).

    x, w: torch tensors (bf16 or fp32) or numpy arrays; bf16 inputs are exact
    in fp32, so this is the fp32 GEMM of the rounded inputs.
    """
    xt = torch.as_tensor(x).float()
    wt = torch.as_tensor(w).float()
    return (xt @ wt.t()).numpy().astype(f32)


def wsplit(w):
    """fp32 w -> (hi, lo) bf16 with hi = bf16(w), lo = bf16(w - hi) (K:1815-1821)."""
    wt = torch.as_tensor(w).float()
    hi = wt.to(torch.bfloat16)
    lo = (wt - hi.float()).to(torch.bfloat16)
    return hi, lo


# ---------------------------------------------------------------------------
# stage 2: scoring + top-k
# ---------------------------------------------------------------------------
def score_topk(logits, bias, k, cfg):
    """Per-token scoring and top-k selection.

    Returns (topk_ids int32 [T,k], topk_w fp32 [T,k]); slot order is by
    descending selection score, ties -> lower expert index.

    SOFTMAX:        sel = logit (+ bias, added before the softmax);
                    renormalize: w_j = e_j / (e_0 + e_1 + ... ) over the k
                    selected, e_j = det_exp(sel_j - sel_0), summed in slot order;
                    else w_j = e_j / tree_sum(det_exp(sel - max)).
    SIGMOID_GROUP:  s = det_sigmoid(logit); b = s + bias; group score = sum of
                    the two largest b in the group; keep topk_group groups;
                    top-k of b over the kept groups; w_j = s_j / (sum_seq s + 1e-20)
                    (renormalize) then * route_scale.
    SOFTMAX_BIAS:   (reference run(), K:1857-1909) p = det_exp(l - max) *
                    (1 / tree_sum(det_exp(l - max))); c = p + bias; top-k of c;
                    w_j = c_j / max(sum_seq c, norm_min).
    """
    l = np.asarray(logits, dtype=f32)
    T, E = l.shape
    b = np.zeros(E, dtype=f32) if bias is None else np.asarray(bias, dtype=f32)
    if cfg.scoring == SCORING_SOFTMAX:
        sel = (l + b[None, :]).astype(f32)
        ids = _stable_topk(sel, k)
        ssel = np.take_along_axis(sel, ids, axis=1)
        e = det_exp((ssel - ssel[:, :1]).astype(f32))
        if cfg.renormalize:
            den = e[:, 0].copy()
            for j in range(1, k):
                den = (den + e[:, j]).astype(f32)
        else:
            den = tree_sum(det_exp((sel - ssel[:, :1]).astype(f32)))
        w = (e / den[:, None]).astype(f32)
        if cfg.route_scale != 1.0:
            w = (w * f32(cfg.route_scale)).astype(f32)
        return ids, w
    if cfg.scoring == SCORING_SIGMOID_GROUP:
        s = det_sigmoid(l)
        bb = (s + b[None, :]).astype(f32)
        ng, tg = cfg.n_group, cfg.topk_group
        gs = E // ng
        g = bb.reshape(T, ng, gs)
        top2 = -np.sort(-g, axis=-1, kind="stable")[..., :2]
        gscore = (top2[..., 0] + top2[..., 1]).astype(f32)
        gsel = _stable_topk(gscore, tg)
        keep = np.zeros((T, ng), dtype=bool)
        np.put_along_axis(keep, gsel, True, axis=1)
        masked = np.where(np.repeat(keep, gs, axis=1), bb, f32(-np.inf)).astype(f32)
        ids = _stable_topk(masked, k)
        ssel = np.take_along_axis(s, ids, axis=1)
        if cfg.renormalize:
            den = ssel[:, 0].copy()
            for j in range(1, k):
                den = (den + ssel[:, j]).astype(f32)
            den = (den + f32(1e-20)).astype(f32)
            w = (ssel / den[:, None]).astype(f32)
        else:
            w = ssel.copy()
        w = (w * f32(cfg.route_scale)).astype(f32)
        return ids, w
    if cfg.scoring == SCORING_SOFTMAX_BIAS:
        m = l.max(axis=1, keepdims=True)
        e = det_exp((l - m).astype(f32))
        rs = (f32(1.0) / tree_sum(e)).astype(f32)
        c = ((e * rs[:, None]).astype(f32) + b[None, :]).astype(f32)
        ids = _stable_topk(c, k)
        csel = np.take_along_axis(c, ids, axis=1)
        tot = csel[:, 0].copy()
        for j in range(1, k):
            tot = (tot + csel[:, j]).astype(f32)
        den = np.maximum(tot, f32(cfg.norm_min)).astype(f32)
        w = (csel / den[:, None]).astype(f32)
        return ids, w
    raise ValueError("unknown scoring %d" % cfg.scoring)


# ---------------------------------------------------------------------------
# stage 3: histogram, offsets, stable permutation
# ---------------------------------------------------------------------------
def counts_offsets(ids, E):
    """counts[E] = histogram of ids; offsets[E+1] exclusive (offsets[e+1] is the
    reference's inclusive group end ``offs[e]``, K:2084-2086)."""
    counts = np.bincount(np.asarray(ids).reshape(-1), minlength=E).astype(np.int32)
    offsets = np.zeros(E + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return counts, offsets


def permutation(ids):
    """(row_token [T*k], pair_row [T*k]) of the stable expert-major order.

    pair_row[t*k+j] = row of pair (t, j) (the reference's ``inv``, K:2178);
    row_token[row] = t (the reference's ``tok``, K:2179)."""
    ids = np.asarray(ids)
    T, k = ids.shape
    order = np.argsort(ids.reshape(-1), kind="stable")
    row_token = (order // k).astype(np.int32)
    pair_row = np.empty(T * k, dtype=np.int32)
    pair_row[order] = np.arange(T * k, dtype=np.int32)
    return row_token, pair_row


# ---------------------------------------------------------------------------
# stage 4: permute / gather (bf16 copy or fp8 e4m3fn + per-128 scales)
# ---------------------------------------------------------------------------
FP8_MAX = 448.0
FP8_EPS = 1e-10
FP8_BLOCK = 128


def gather_rows(x, row_token):
    """xg[row] = x[row_token[row]] (K:2216-2230)."""
    return torch.as_tensor(x)[torch.as_tensor(row_token, dtype=torch.long)]


def fp8_quant_rows(x):
    """Per-1x128-block fp8 e4m3fn quantisation of rows of x.

    scale = max(amax, 1e-10) / 448 (fp32 divide); q = e4m3fn(clamp(x / scale, +-448))
    using torch's own fp32 -> float8_e4m3fn conversion (round to nearest even).
    Returns (q uint8 [R,H] as raw bytes, scales fp32 [R, H/128])."""
    xf = torch.as_tensor(x).float()
    R, H = xf.shape
    blk = xf.view(R, H // FP8_BLOCK, FP8_BLOCK)
    amax = blk.abs().amax(dim=-1)
    scale = torch.clamp(amax, min=FP8_EPS) / FP8_MAX
    q = torch.clamp(blk / scale[..., None], -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(R, H).view(torch.uint8), scale


def permute_fp8(x, row_token):
    """Quantise each token row once, then place its copies (equal to quantising
    every gathered row)."""
    q, s = fp8_quant_rows(x)
    rt = torch.as_tensor(row_token, dtype=torch.long)
    return q[rt], s[rt]


# ---------------------------------------------------------------------------
# stage 5: combine
# ---------------------------------------------------------------------------
def combine(y, pair_row, topk_w, shared=None, out_dtype=None):
    """out[t] = cast(shared[t] + sum_j w[t,j] * y[pair_row[t,j]]), fp32 accumulate in
    slot order (K:2407-2424).  Returns a torch tensor of y's dtype."""
    yt = torch.as_tensor(y)
    pr = torch.as_tensor(pair_row, dtype=torch.long)
    w = torch.as_tensor(np.asarray(topk_w, dtype=f32))
    T, k = w.shape
    acc = torch.zeros(T, yt.shape[1], dtype=torch.float32) if shared is None \
        else torch.as_tensor(shared).float().clone()
    rows = pr.view(T, k)
    for j in range(k):
        acc = acc + w[:, j:j + 1] * yt[rows[:, j]].float()
    return acc.to(out_dtype or yt.dtype)


# ---------------------------------------------------------------------------
# expert grouped GEMM (the consumer of the offsets)
# ---------------------------------------------------------------------------
def group_bounds(offs_incl, M):
    """[(start, end)] row range of each group from inclusive ends offs
    (moe_gemm.h:66-69: group g owns rows [offs[g-1], offs[g]), offs[-1] = 0),
    clamped into [0, M] as the device plan does."""
    out, prev = [], 0
    for e in np.asarray(offs_incl, dtype=np.int64).tolist():
        lo = min(max(prev, 0), M)
        hi = min(max(e, 0), M)
        out.append((lo, max(lo, hi)))
        prev = e
    return out


def _group_a(a, lo, hi, ident_a, ident_m):
    """A rows of one group; the identity shortcut (moe_gemm.h:72-77) takes a
    group with exactly ident_m rows from ident_a instead."""
    if ident_m and hi - lo == ident_m:
        return torch.as_tensor(ident_a)[:ident_m].float()
    return torch.as_tensor(a)[lo:hi].float()


def grouped_gemm(a, w, offs_incl, ident_a=None, ident_m=0):
    """out[r] = a[r] . w[g]^T for the rows r of group g (grouped_mm,
    moe_gemm.h:66-85), fp32 accumulate, fp32 result.  Rows outside every group
    are left 0."""
    at = torch.as_tensor(a)
    wt = torch.as_tensor(w)
    M = at.shape[0]
    out = torch.zeros(M, wt.shape[1], dtype=torch.float32)
    for g, (lo, hi) in enumerate(group_bounds(offs_incl, M)):
        if hi > lo:
            out[lo:hi] = _group_a(at, lo, hi, ident_a, ident_m) @ wt[g].float().t()
    return out


def dequant_fp8_rows(q, scales):
    """bf16(float32(q) * s) per 1x128 block: the fp8 row permute's output
    turned back into the bf16 A operand of the expert GEMM (e4m3fn -> fp32 is
    exact; one fp32 multiply; round to nearest even).  q [M,K] e4m3fn (or its
    bytes), scales [M,K/128] fp32."""
    qt = torch.as_tensor(q)
    if qt.dtype == torch.uint8:
        qt = qt.view(torch.float8_e4m3fn)
    st = torch.as_tensor(scales).float()
    return (qt.float() * st.repeat_interleave(128, dim=1)).to(torch.bfloat16)


def silu(v):
    """silu(v) = v / (1 + exp(-v)) in fp32 (torch's fp32 silu)."""
    return torch.nn.functional.silu(torch.as_tensor(v).float())


def grouped_swiglu(a, wg, wu, offs_incl, ident_a=None, ident_m=0):
    """h[r] = silu(a[r] . wg[g]^T) * (a[r] . wu[g]^T): grouped_mm_pair
    (moe_gemm.h:87-95) followed by the expert MLP's silu*mul, fp32 result."""
    g = grouped_gemm(a, wg, offs_incl, ident_a, ident_m)
    u = grouped_gemm(a, wu, offs_incl, ident_a, ident_m)
    return silu(g) * u


# ---------------------------------------------------------------------------
# int8 experts
# ---------------------------------------------------------------------------
def fwht_blocks(v, n=128):
    """Unnormalised Walsh-Hadamard transform of each n-block of the last
    axis, in fp32, butterfly stages s = 1, 2, ..., n/2 (for k with bit s
    clear: v[k] = a + b, v[k^s] = a - b, a = v[k], b = v[k^s]) -- the order
    of moe_wq.h:178-188's wht16, over 128 points."""
    v = np.asarray(v, dtype=f32).copy()
    sh = v.shape
    s = 1
    while s < n:
        b = v.reshape(-1, n // (2 * s), 2, s)
        lo = b[:, :, 0, :].copy()
        hi = b[:, :, 1, :].copy()
        b[:, :, 0, :] = lo + hi
        b[:, :, 1, :] = lo - hi
        s *= 2
    return v.reshape(sh)


def quant_rows_i8(x, hadamard=0, scale_mul=1.0):
    """Per-row symmetric int8 of bf16 rows x [R, K] (optionally rotated):
    q = clamp(rint(v * (127 / amax)), -127, 127), s = (amax / 127) * scale_mul,
    all in fp32 (rint = round half to even); an all-zero row gives q = 0, s = 0.
    Returns (q int8 [R, K], s fp32 [R])."""
    v = torch.as_tensor(x).float().numpy().astype(f32)
    if hadamard:
        v = fwht_blocks(v, hadamard)
    amax = np.abs(v).max(axis=1).astype(f32)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, f32(127.0) / amax, f32(0.0)).astype(f32)
    q = np.clip(np.rint(v * inv[:, None]), -127, 127).astype(np.int8)
    s = ((amax / f32(127.0)).astype(f32) * f32(scale_mul)).astype(f32)
    return q, s


def grouped_gemm_i8(a, a_scales, w, w_scales, offs_incl, a_rows=None, ident_a=None,
                    ident_scales=None, ident_m=0):
    """out[r, n] = float32(sum_k A[r,k] w[g,n,k]) * (sa(r) * w_scales[g, n]),
    fp32 (bf16 rounding is the caller's), with operand row A[r] = a[a_rows[r]]
    and sa(r) = a_scales[a_rows[r]] (a_rows None: a[r], a_scales[r]).  The
    integer sums are formed in float64, which is exact (|sum| <= 127^2 K <
    2^53).  An identity group reads ident_a and ident_scales.  Rows outside
    every group stay 0."""
    a = np.asarray(a, dtype=np.int8)
    w = np.asarray(w, dtype=np.int8)
    ws = np.asarray(w_scales, dtype=f32)
    rs = np.asarray(a_scales, dtype=f32)
    if a_rows is not None:
        sel = np.asarray(a_rows, dtype=np.int64)
        a, rs = a[sel], rs[sel]
    M = a.shape[0]
    out = np.zeros((M, w.shape[1]), dtype=f32)
    for g, (lo, hi) in enumerate(group_bounds(offs_incl, M)):
        if hi <= lo:
            continue
        if ident_m and hi - lo == ident_m:
            ag = np.asarray(ident_a, dtype=np.int8)[:ident_m]
            sg = np.asarray(ident_scales, dtype=f32)[:ident_m]
        else:
            ag, sg = a[lo:hi], rs[lo:hi]
        acc = (ag.astype(np.float64) @ w[g].astype(np.float64).T).astype(f32)
        out[lo:hi] = acc * (sg[:, None] * ws[g][None, :]).astype(f32)
    return out


def grouped_swiglu_i8(a, a_scales, wg, wg_scales, wu, wu_scales, offs_incl, **kw):
    """h = silu(g) * u of the two dequantised int8 products (fp32)."""
    g = grouped_gemm_i8(a, a_scales, wg, wg_scales, offs_incl, **kw)
    u = grouped_gemm_i8(a, a_scales, wu, wu_scales, offs_incl, **kw)
    return silu(g) * torch.as_tensor(u)


# ---------------------------------------------------------------------------
# whole path
# ---------------------------------------------------------------------------
def route(x, w, bias, k, cfg):
    """Stages 1-3: returns dict(logits, ids, weights, counts, offsets)."""
    logits = router_logits(x, w)
    ids, wts = score_topk(logits, bias, k, cfg)
    counts, offsets = counts_offsets(ids, logits.shape[1])
    return dict(logits=logits, ids=ids, weights=wts, counts=counts, offsets=offsets)


def route_dispatch_combine(x, w, bias, y, k, cfg, fp8=False):
    """The full path on CPU: route, permute (bf16 or fp8), combine of y."""
    r = route(x, w, bias, k, cfg)
    row_token, pair_row = permutation(r["ids"])
    r["row_token"], r["pair_row"] = row_token, pair_row
    if fp8:
        r["xg"], r["scales"] = permute_fp8(x, row_token)
    else:
        r["xg"] = gather_rows(x, row_token)
    r["out"] = combine(y, pair_row, r["weights"])
    return r
