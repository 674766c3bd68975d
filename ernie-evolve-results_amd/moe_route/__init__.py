"""moe_route: MI355X-native MoE route -> dispatch -> combine.

Python host side of libmoe_route.so.  Mirrors the reference's operator
interface: the whole-layer entry point ``run`` keeps the signature of
``sol-execbench/029_moe_sparse_routing_and_dispatch/kernel.cu::run``
(K:4067-4077, bound at K:5729-5735), and the stage functions expose the five
stages it launches (K:4323-4431, K:5710-5718).

PyTorch only provides device memory and the current HIP stream; every stage
runs in the library's HIP kernels.  There is no CPU fallback: a missing
library or a CPU tensor raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

from .configs import (CONFIGS, SCORING_SIGMOID_GROUP, SCORING_SOFTMAX, SCORING_SOFTMAX_BIAS,
                      MoeConfig, RouteCfg, make_inputs)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoe_route.so")

DTYPE_BF16, DTYPE_FP32, DTYPE_FP8E4M3FN = 0, 1, 2
ERR_NAMES = {-1: "MOE_ERR_NULL_POINTER", -2: "MOE_ERR_INVALID_ARG", -3: "MOE_ERR_UNSUPPORTED",
             -4: "MOE_ERR_WORKSPACE", -5: "MOE_ERR_LAUNCH", -6: "MOE_ERR_ALIGNMENT"}

# Every extern "C" symbol of include/moe_route.h.
EXPORTS = ["moe_version", "moe_last_error_string", "moe_route_workspace_bytes",
           "moe_router_gemm", "moe_topk", "moe_route", "moe_offsets",
           "moe_permute_workspace_bytes", "moe_permute", "moe_combine",
           "moe_grouped_gemm_workspace_bytes", "moe_grouped_gemm", "moe_grouped_swiglu",
           "moe_grouped_gemm_fp8", "moe_grouped_swiglu_fp8", "moe_quant_rows_i8",
           "moe_grouped_gemm_i8", "moe_grouped_swiglu_i8", "moe_grouped_gemm_rows",
           "moe_grouped_swiglu_rows", "moe_permute_noalloc_max_scratch_bytes",
           "moe_permute_noalloc", "moe_route_permute_workspace_bytes",
           "moe_route_permute", "moe_permute_fp8_workspace_bytes"]


class MoeError(RuntimeError):
    """A libmoe_route entry point returned an error code (the reference raises
    RuntimeError from TORCH_CHECK, K:1771-1775)."""

    def __init__(self, code, msg):
        super().__init__("%s (%d): %s" % (ERR_NAMES.get(code, "MOE_ERR"), code, msg))
        self.code = code


class _Cfg(ctypes.Structure):
    _fields_ = [("scoring", ctypes.c_int), ("renormalize", ctypes.c_int),
                ("n_group", ctypes.c_int), ("topk_group", ctypes.c_int),
                ("route_scale", ctypes.c_float), ("norm_min", ctypes.c_float)]


_lib = None
_P, _I, _Z, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float


def lib():
    """Load libmoe_route.so (built by moe_route.build); raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libmoe_route.so is not built (%s); run "
                               "`python -m moe_route.build` or __graft_entry__.build()" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        L.moe_version.restype = _I
        L.moe_version.argtypes = []
        L.moe_last_error_string.restype = ctypes.c_char_p
        L.moe_last_error_string.argtypes = []
        L.moe_route_workspace_bytes.restype = _Z
        L.moe_route_workspace_bytes.argtypes = [_I, _I, _I, _I]
        L.moe_permute_workspace_bytes.restype = _Z
        L.moe_permute_workspace_bytes.argtypes = [_I, _I, _I]
        L.moe_permute_fp8_workspace_bytes.restype = _Z
        L.moe_permute_fp8_workspace_bytes.argtypes = [_I, _I, _I, _I]
        L.moe_router_gemm.restype = _I
        L.moe_router_gemm.argtypes = [_P, _P, _I, _I, _I, _P, _P]
        L.moe_topk.restype = _I
        L.moe_topk.argtypes = [_P, _P, _I, _I, _I, ctypes.POINTER(_Cfg), _P, _P, _P, _P]
        L.moe_route.restype = _I
        L.moe_route.argtypes = [_P, _P, _I, _P, _I, _I, _I, _I, ctypes.POINTER(_Cfg), _P, _P, _P,
                                _P, _P, _Z, _P]
        L.moe_offsets.restype = _I
        L.moe_offsets.argtypes = [_P, _I, _P, _P]
        L.moe_permute.restype = _I
        L.moe_permute.argtypes = [_P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _Z,
                                  _P]
        L.moe_permute_noalloc_max_scratch_bytes.restype = _Z
        L.moe_permute_noalloc_max_scratch_bytes.argtypes = []
        L.moe_permute_noalloc.restype = _I
        L.moe_permute_noalloc.argtypes = [_P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P,
                                          _P]
        L.moe_route_permute_workspace_bytes.restype = _Z
        L.moe_route_permute_workspace_bytes.argtypes = [_I, _I, _I, _I, _I]
        L.moe_route_permute.restype = _I
        L.moe_route_permute.argtypes = [_P, _P, _I, _P, _I, _I, _I, _I, ctypes.POINTER(_Cfg), _P,
                                        _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _Z, _P]
        L.moe_combine.restype = _I
        L.moe_combine.argtypes = [_P, _I, _P, _P, _P, _I, _I, _I, _P, _P]
        L.moe_grouped_gemm_workspace_bytes.restype = _Z
        L.moe_grouped_gemm_workspace_bytes.argtypes = [_I]
        L.moe_grouped_gemm.restype = _I
        L.moe_grouped_gemm.argtypes = [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P, _Z, _P]
        L.moe_grouped_swiglu.restype = _I
        L.moe_grouped_swiglu.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P, _Z, _P]
        L.moe_grouped_gemm_fp8.restype = _I
        L.moe_grouped_gemm_fp8.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _Z, _P]
        L.moe_grouped_swiglu_fp8.restype = _I
        L.moe_grouped_swiglu_fp8.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _Z, _P]
        L.moe_grouped_gemm_rows.restype = _I
        L.moe_grouped_gemm_rows.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _Z, _P]
        L.moe_grouped_swiglu_rows.restype = _I
        L.moe_grouped_swiglu_rows.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _Z, _P]
        L.moe_quant_rows_i8.restype = _I
        L.moe_quant_rows_i8.argtypes = [_P, ctypes.c_longlong, _I, _I, _F, _I, _P, _P, _P, _P]
        L.moe_grouped_gemm_i8.restype = _I
        L.moe_grouped_gemm_i8.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P,
                                          _P, _Z, _P]
        L.moe_grouped_swiglu_i8.restype = _I
        L.moe_grouped_swiglu_i8.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P,
                                            _I, _P, _P, _Z, _P]
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise MoeError(rc, lib().moe_last_error_string().decode())


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _dev(t, name):
    if not (isinstance(t, torch.Tensor) and t.is_cuda):
        raise RuntimeError("%s must be a CUDA (HIP) tensor; libmoe_route has no CPU path" % name)
    if not t.is_contiguous():
        raise RuntimeError("%s must be contiguous" % name)
    return t


def _want(t, name, dtypes, shape=None):
    """Check dtype and shape; the caller then checks the device of every
    argument with _devs.  The C ABI takes bare pointers: a wrong dtype or
    shape here would be read as another layout, or written past the end of a
    buffer."""
    if not isinstance(t, torch.Tensor):
        raise RuntimeError("%s must be a tensor" % name)
    if t.dtype not in dtypes:
        raise RuntimeError("%s must be %s, got %s" % (
            name, " or ".join(str(d).replace("torch.", "") for d in dtypes),
            str(t.dtype).replace("torch.", "")))
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise RuntimeError("%s must have shape %s, got %s" % (name, tuple(shape), tuple(t.shape)))
    return t


def _devs(**named):
    """_dev on every tensor argument that is not None."""
    for name, t in named.items():
        if t is not None:
            _dev(t, name)


_BF16, _F32, _I32 = (torch.bfloat16,), (torch.float32,), (torch.int32,)
_BF16_F32 = (torch.bfloat16, torch.float32)


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ccfg(cfg: RouteCfg):
    return _Cfg(int(cfg.scoring), int(bool(cfg.renormalize)), int(cfg.n_group),
                int(cfg.topk_group), float(cfg.route_scale), float(cfg.norm_min))


def _dtype_code(dt):
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_FP32
    raise RuntimeError("unsupported dtype %s" % dt)


# ---------------------------------------------------------------------------
# stage functions
# ---------------------------------------------------------------------------
def router_gemm(x, w):
    """logits[T,E] fp32 = x[T,H] bf16 . w[E,H]^T bf16 (K:4327-4339)."""
    _dev(x, "x"), _dev(w, "w")
    T, H = x.shape
    E = w.shape[0]
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise RuntimeError("router_gemm takes bf16 x and w")
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    _check(lib().moe_router_gemm(_ptr(x), _ptr(w), T, H, E, _ptr(logits), _stream(x)))
    return logits


def topk(logits, bias, k, cfg: RouteCfg):
    """Scoring + top-k + histogram on fp32 logits (K:1829-1920).
    Returns (topk_ids int32 [T,k], topk_w fp32 [T,k], counts int32 [E])."""
    _want(logits, "logits", _F32)
    T, E = logits.shape
    if bias is not None:
        _want(bias, "bias", _F32, (E,))
    _devs(logits=logits, bias=bias)
    ids = torch.empty(T, k, dtype=torch.int32, device=logits.device)
    wts = torch.empty(T, k, dtype=torch.float32, device=logits.device)
    counts = torch.empty(E, dtype=torch.int32, device=logits.device)
    c = _ccfg(cfg)
    _check(lib().moe_topk(_ptr(logits), _ptr(bias), T, E, k, ctypes.byref(c), _ptr(ids),
                          _ptr(wts), _ptr(counts), _stream(logits)))
    return ids, wts, counts


def route(x, w, bias, k, cfg: RouteCfg):
    """Router GEMM + scoring + top-k + histogram.  w bf16 [E,H], or fp32 [E,H]
    (hi/lo split on the device, K:1786-1824).
    Returns (logits fp32 [T,E], topk_ids, topk_w, counts)."""
    _want(x, "x", _BF16)  # the router reads bf16 hidden states (K:4327-4339)
    T, H = x.shape
    E = w.shape[0]
    _want(w, "w", _BF16_F32, (E, H))
    wd = _dtype_code(w.dtype)
    if bias is not None:
        _want(bias, "bias", _F32, (E,))
    _devs(x=x, w=w, bias=bias)
    dev = x.device
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    ids = torch.empty(T, k, dtype=torch.int32, device=dev)
    wts = torch.empty(T, k, dtype=torch.float32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    L = lib()
    nws = L.moe_route_workspace_bytes(T, H, E, wd)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
    c = _ccfg(cfg)
    _check(L.moe_route(_ptr(x), _ptr(w), wd, _ptr(bias), T, H, E, k, ctypes.byref(c),
                       _ptr(logits), _ptr(ids), _ptr(wts), _ptr(counts), _ptr(ws), nws,
                       _stream(x)))
    return logits, ids, wts, counts


def offsets(counts):
    """Exclusive offsets [E+1] of counts [E] (K:2069-2086)."""
    _dev(counts, "counts")
    E = counts.shape[0]
    out = torch.empty(E + 1, dtype=torch.int32, device=counts.device)
    _check(lib().moe_offsets(_ptr(counts), E, _ptr(out), _stream(counts)))
    return out


def permute(x, topk_ids, E, fp8=False, index_only=False):
    """Stable expert-major permutation + gather (K:1922-2238).

    Returns dict(xg, scales, row_token, pair_row, offsets, counts); xg is
    x.dtype rows (or uint8 e4m3fn bytes when fp8) in expert-contiguous order."""
    _want(x, "x", _BF16_F32)
    T, H = x.shape
    k = topk_ids.shape[1]
    _want(topk_ids, "topk_ids", _I32, (T, k))
    _devs(x=x, topk_ids=topk_ids)
    dev = x.device
    xd = _dtype_code(x.dtype)
    od = DTYPE_FP8E4M3FN if fp8 else xd
    ns = T * k
    xg = scales = None
    if not index_only:
        if fp8:
            xg = torch.empty(ns, H, dtype=torch.uint8, device=dev)
            scales = torch.empty(ns, H // 128, dtype=torch.float32, device=dev)
        else:
            xg = torch.empty(ns, H, dtype=x.dtype, device=dev)
    row_token = torch.empty(ns, dtype=torch.int32, device=dev)
    pair_row = torch.empty(ns, dtype=torch.int32, device=dev)
    offs = torch.empty(E + 1, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    L = lib()
    nws = (L.moe_permute_fp8_workspace_bytes(T, H, E, k) if fp8 and not index_only
           else L.moe_permute_workspace_bytes(T, E, k))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
    _check(L.moe_permute(_ptr(x), xd, _ptr(topk_ids), T, H, E, k, od, _ptr(xg), _ptr(scales),
                         _ptr(row_token), _ptr(pair_row), _ptr(offs), _ptr(counts), _ptr(ws),
                         nws, _stream(x)))
    return dict(xg=xg, scales=scales, row_token=row_token, pair_row=pair_row, offsets=offs,
                counts=counts)


def combine(y, pair_row, topk_w, shared=None, out=None):
    """out[t] = shared[t] + sum_j w[t,j] * y[pair_row[t,j]], fp32 accumulate
    (K:2365-2428)."""
    _want(y, "y", _BF16_F32)
    _want(topk_w, "topk_w", _F32)
    T, k = topk_w.shape
    H = y.shape[1]
    _want(pair_row, "pair_row", _I32)
    if pair_row.numel() != T * k:  # [T, k] or moe_permute's flat [T * k]
        raise RuntimeError("pair_row must hold T * k = %d entries, got %d" % (T * k,
                                                                            pair_row.numel()))
    if shared is not None:
        _want(shared, "shared", (y.dtype,), (T, H))
    if out is None:
        out = torch.empty(T, H, dtype=y.dtype, device=y.device)
    else:
        _want(out, "out", (y.dtype,), (T, H))
    _devs(y=y, topk_w=topk_w, pair_row=pair_row, shared=shared, out=out)
    _check(lib().moe_combine(_ptr(y), _dtype_code(y.dtype), _ptr(pair_row), _ptr(topk_w),
                             _ptr(shared), T, H, k, _ptr(out), _stream(y)))
    return out


def _grouped_args(a, offs, ident_a, ident_m, fp8=False):
    _dev(a, "a")
    _dev(offs, "offs")
    if offs.dtype != torch.int32:
        raise RuntimeError("offs must be int32 inclusive group ends")
    if fp8 and a.dtype not in (torch.uint8, torch.float8_e4m3fn):
        raise RuntimeError("fp8 a must be e4m3fn bytes (uint8 or float8_e4m3fn)")
    if not fp8 and a.dtype != torch.bfloat16:
        raise RuntimeError("a must be bf16")
    if ident_m and ident_a is None:
        raise RuntimeError("ident_m > 0 needs ident_a")
    ws = torch.empty(max(lib().moe_grouped_gemm_workspace_bytes(offs.numel()), 256),
                     dtype=torch.uint8, device=a.device)
    return ws


def _rows_arg(a_rows, ident_a):
    if a_rows is None:
        return None
    _dev(a_rows, "a_rows")
    if a_rows.dtype != torch.int32:
        raise RuntimeError("a_rows must be int32")
    if ident_a is not None:
        raise RuntimeError("a_rows and ident_a are exclusive")
    return a_rows


def grouped_gemm(a, w, offs, ident_a=None, ident_m=0, out=None, a_rows=None):
    """Expert grouped GEMM (the reference's grouped_mm, moe_gemm.h:66-85):
    out[r] = A[r] . w[g]^T for the rows r of group g = [offs[g-1], offs[g]).
    A[r] = a[r], or a[a_rows[r]] with a row map (moe_grouped_gemm_rows: the
    gather read through moe_permute's row_token).  a bf16 [rows, K], w
    [G,N,K] bf16, offs [G] int32 INCLUSIVE ends (moe_permute's offsets[1:]);
    returns out [M,N] bf16, M = len(a_rows) or a's rows.  Rows outside every
    group are not written."""
    ws = _grouped_args(a, offs, ident_a, ident_m)
    a_rows = _rows_arg(a_rows, ident_a)
    G, N, K = w.shape
    M = a_rows.numel() if a_rows is not None else a.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    if a_rows is not None:
        _check(lib().moe_grouped_gemm_rows(_ptr(a), _ptr(a_rows), _ptr(w), _ptr(offs), G, M, N,
                                           K, _ptr(out), _ptr(ws), ws.numel(), _stream(a)))
        return out
    _check(lib().moe_grouped_gemm(_ptr(a), _ptr(w), _ptr(offs), G, M, N, K, _ptr(ident_a),
                                  int(ident_m), _ptr(out), _ptr(ws), ws.numel(), _stream(a)))
    return out


def grouped_swiglu(a, wg, wu, offs, ident_a=None, ident_m=0, out=None, a_rows=None):
    """SwiGLU expert projection (grouped_mm_pair, moe_gemm.h:87-95, plus the
    silu*mul): h[r] = silu(A[r] . wg[g]^T) * (A[r] . wu[g]^T), bf16 [M,N];
    A[r] as in grouped_gemm."""
    ws = _grouped_args(a, offs, ident_a, ident_m)
    a_rows = _rows_arg(a_rows, ident_a)
    if wg.shape != wu.shape:
        raise RuntimeError("gate and up weights must have one shape")
    G, N, K = wg.shape
    M = a_rows.numel() if a_rows is not None else a.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    if a_rows is not None:
        _check(lib().moe_grouped_swiglu_rows(_ptr(a), _ptr(a_rows), _ptr(wg), _ptr(wu),
                                             _ptr(offs), G, M, N, K, _ptr(out), _ptr(ws),
                                             ws.numel(), _stream(a)))
        return out
    _check(lib().moe_grouped_swiglu(_ptr(a), _ptr(wg), _ptr(wu), _ptr(offs), G, M, N, K,
                                    _ptr(ident_a), int(ident_m), _ptr(out), _ptr(ws), ws.numel(),
                                    _stream(a)))
    return out


def grouped_gemm_fp8(a, a_scales, w, offs, out=None):
    """grouped_gemm with an fp8 A operand: a [M,K] e4m3fn bytes and a_scales
    [M,K/128] fp32 (moe_permute's fp8 output), dequantised in the GEMM's A
    load as bf16(q * s)."""
    ws = _grouped_args(a, offs, None, 0, fp8=True)
    _dev(a_scales, "a_scales")
    G, N, K = w.shape
    M = a.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    _check(lib().moe_grouped_gemm_fp8(_ptr(a), _ptr(a_scales), _ptr(w), _ptr(offs), G, M, N, K,
                                      _ptr(out), _ptr(ws), ws.numel(), _stream(a)))
    return out


def grouped_swiglu_fp8(a, a_scales, wg, wu, offs, out=None):
    """grouped_swiglu with an fp8 A operand (see grouped_gemm_fp8)."""
    ws = _grouped_args(a, offs, None, 0, fp8=True)
    _dev(a_scales, "a_scales")
    if wg.shape != wu.shape:
        raise RuntimeError("gate and up weights must have one shape")
    G, N, K = wg.shape
    M = a.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    _check(lib().moe_grouped_swiglu_fp8(_ptr(a), _ptr(a_scales), _ptr(wg), _ptr(wu), _ptr(offs),
                                        G, M, N, K, _ptr(out), _ptr(ws), ws.numel(), _stream(a)))
    return out


def quant_rows_i8(x, hadamard=0, scale_mul=1.0, group_rows=0, group_counts=None, q=None,
                  scales=None):
    """Per-row symmetric int8 of bf16 rows x [..., K] (the reference's
    xquant / hquant / wquant, moe_wq.h:150-188): optional 16- or 128-block
    Walsh-Hadamard rotation (hadamard = 0, 16, 128), q = clamp(rint(v * 127 / amax), +-127),
    scales = amax / 127 * scale_mul.  With group_counts, rows of groups with
    count 0 are skipped.  Returns (q int8, scales fp32 [rows])."""
    _dev(x, "x")
    if x.dtype != torch.bfloat16:
        raise RuntimeError("x must be bf16")
    K = x.shape[-1]
    R = x.numel() // K if K else 0
    if q is None:
        q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    if scales is None:
        scales = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    if group_counts is not None:
        _dev(group_counts, "group_counts")
    _check(lib().moe_quant_rows_i8(_ptr(x), R, K, int(hadamard), float(scale_mul),
                                   int(group_rows), _ptr(group_counts), _ptr(q), _ptr(scales),
                                   _stream(x)))
    return q, scales


def _i8_args(a, a_scales, offs, a_rows, ident_a, ident_scales, ident_m):
    for t, n in ((a, "a"), (a_scales, "a_scales"), (offs, "offs")):
        _dev(t, n)
    if a_rows is not None and (_dev(a_rows, "a_rows").dtype != torch.int32):
        raise RuntimeError("a_rows must be int32")
    if a.dtype != torch.int8:
        raise RuntimeError("a must be int8")
    if offs.dtype != torch.int32:
        raise RuntimeError("offs must be int32 inclusive group ends")
    if ident_m and (ident_a is None or ident_scales is None):
        raise RuntimeError("ident_m > 0 needs ident_a and ident_scales")
    return torch.empty(max(lib().moe_grouped_gemm_workspace_bytes(offs.numel()), 256),
                       dtype=torch.uint8, device=a.device)


def grouped_gemm_i8(a, a_scales, w, w_scales, offs, a_rows=None, ident_a=None,
                    ident_scales=None, ident_m=0, out=None):
    """int8 grouped GEMM (the reference's int8 grouped_mm, moe_int8.h:27-45):
    out[r, n] = bf16(float(A[r] . w[g, n]) * (sa(r) * w_scales[g, n])), exact
    int32 accumulation, where operand row r is A[r] = a[a_rows[r]] with scale
    sa(r) = a_scales[a_rows[r]] (a_rows None: a[r], a_scales[r]).  a int8
    [rows, K], w [G,N,K] int8, w_scales [G,N] fp32; returns bf16 [M,N] with
    M = len(a_rows) (or a's rows)."""
    ws = _i8_args(a, a_scales, offs, a_rows, ident_a, ident_scales, ident_m)
    G, N, K = w.shape
    M = a_rows.numel() if a_rows is not None else a.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    _check(lib().moe_grouped_gemm_i8(_ptr(a), _ptr(a_scales), _ptr(a_rows), _ptr(w),
                                     _ptr(w_scales), _ptr(offs), G, M, N, K, _ptr(ident_a),
                                     _ptr(ident_scales), int(ident_m), _ptr(out), _ptr(ws),
                                     ws.numel(), _stream(a)))
    return out


def grouped_swiglu_i8(a, a_scales, wg, wg_scales, wu, wu_scales, offs, a_rows=None,
                      ident_a=None, ident_scales=None, ident_m=0, out=None):
    """int8 SwiGLU grouped GEMM: h = bf16(silu(g) * u), g and u the dequantised
    int8 products of a with wg[g] and wu[g] (see grouped_gemm_i8)."""
    ws = _i8_args(a, a_scales, offs, a_rows, ident_a, ident_scales, ident_m)
    if wg.shape != wu.shape:
        raise RuntimeError("gate and up weights must have one shape")
    G, N, K = wg.shape
    M = a_rows.numel() if a_rows is not None else a.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    _check(lib().moe_grouped_swiglu_i8(_ptr(a), _ptr(a_scales), _ptr(a_rows), _ptr(wg),
                                       _ptr(wg_scales), _ptr(wu), _ptr(wu_scales), _ptr(offs), G,
                                       M, N, K, _ptr(ident_a), _ptr(ident_scales), int(ident_m),
                                       _ptr(out), _ptr(ws), ws.numel(), _stream(a)))
    return out


def route_dispatch_combine(x, w, bias, y, k, cfg: RouteCfg, fp8=False):
    """The whole path for one batch: route, permute (bf16 or fp8), combine y."""
    logits, ids, wts, counts = route(x, w, bias, k, cfg)
    p = permute(x, ids, w.shape[0], fp8=fp8)
    out = combine(y, p["pair_row"], wts) if y is not None else None
    p.update(logits=logits, topk_ids=ids, topk_w=wts, route_counts=counts, out=out)
    return p


# ---------------------------------------------------------------------------
# the reference entry point
# ---------------------------------------------------------------------------
REF_NE, REF_TOPK = 64, 8  # K:1582-1583
# Walsh-Hadamard block of the int8 down projection (h and the down weights):
# 16, the reference's HAD_N (moe_wq.h:174).  Measured on MI355X at T = 1571,
# 16 passes the harness gate on 99.71-99.75% of elements (128: 99.76-99.80%)
# and makes run() ~1.3% faster (no cross-lane butterflies).
INT8_HADAMARD = 16


def run(hidden_states, gate_weight, e_score_correction_bias, expert_gate_proj, expert_up_proj,
        expert_down_proj, shared_gate_proj, shared_up_proj, shared_down_proj, norm_min, *,
        dispatch="bf16", experts="bf16"):
    """Drop-in for the reference's run() (K:4067-4077): returns
    (out [B,S,H] bf16, router_logits [T,64] fp32).

    Every stage runs in libmoe_route, enqueued on the current stream with no
    host synchronisation:
      routing   fp32 gate_weight hi/lo split, softmax + post-softmax bias,
                top-8, w = c / max(sum c, norm_min)  (K:1786-1920);
      dispatch  stable expert-major permutation (K:1922-2238); the expert
                GEMM reads each routed row of x through row_token instead of
                a gathered copy (K:2216-2230's gather, fused);
      experts   h = silu(xg . Wg[e]^T) * (xg . Wu[e]^T), y = h . Wd[e]^T as two
                grouped GEMMs over the device offsets (the reference's CUTLASS
                grouped GEMMs, moe_gemm.h:66-95);
      shared    the same two kernels with one group of all T rows;
      combine   out = shared + sum_j w_j y[pair_row]  (K:2365-2428).
    dispatch="fp8" (keyword only, not in the reference signature) permutes the
    routed rows to e4m3fn with per-128 scales and dequantises them inside the
    expert gate+up GEMM's A load.

    experts="int8" (keyword only) runs the routed experts the way the
    reference's own run() does (int8 experts, kernel.cu:61-66): x quantised
    per token, each routed expert's weights per output row (only experts that
    received rows), the gate+up products dequantised in the GEMM epilogue
    before silu*mul, h rotated by 16-point Walsh-Hadamard blocks and
    quantised per row, the down weights rotated the same way (1/16 folded
    into their scales), and an int8 down GEMM.  The shared expert stays bf16."""
    if dispatch not in ("bf16", "fp8"):
        raise RuntimeError("dispatch must be 'bf16' or 'fp8'")
    if experts not in ("bf16", "int8"):
        raise RuntimeError("experts must be 'bf16' or 'int8'")
    if experts == "int8" and dispatch != "bf16":
        raise RuntimeError("experts='int8' dispatches int8 rows; dispatch must stay 'bf16'")
    B, S, H = hidden_states.shape
    T = B * S
    x = hidden_states.reshape(T, H)
    _dev(x, "hidden_states")
    E = gate_weight.shape[0]
    cfg = RouteCfg(SCORING_SOFTMAX_BIAS, True, 1, 1, 1.0, float(norm_min))
    logits, ids, wts, _ = route(x, gate_weight.float().contiguous(),
                                e_score_correction_bias.float().contiguous(), REF_TOPK, cfg)
    if experts == "int8":
        y, p = _experts_int8(x, ids, E, expert_gate_proj.contiguous(),
                             expert_up_proj.contiguous(), expert_down_proj.contiguous())
    else:
        y, p = _experts_bf16(x, ids, E, dispatch, expert_gate_proj.contiguous(),
                             expert_up_proj.contiguous(), expert_down_proj.contiguous())
    dense = torch.full((1,), T, dtype=torch.int32, device=x.device)
    sh_h = grouped_swiglu(x.contiguous(), shared_gate_proj.contiguous().unsqueeze(0),
                          shared_up_proj.contiguous().unsqueeze(0), dense)
    sh = grouped_gemm(sh_h, shared_down_proj.contiguous().unsqueeze(0), dense)
    out = combine(y, p["pair_row"], wts, shared=sh)
    return out.view(B, S, H), logits


def _experts_bf16(x, ids, E, dispatch, wg, wu, wd):
    if dispatch == "fp8":
        p = permute(x, ids, E, fp8=True)
        ends = p["offsets"][1:]  # inclusive group ends (moe_gemm.h:66-69)
        h = grouped_swiglu_fp8(p["xg"], p["scales"], wg, wu, ends)
    else:
        # index-only permute: the gate+up GEMM reads token rows through row_token
        p = permute(x, ids, E, index_only=True)
        ends = p["offsets"][1:]
        h = grouped_swiglu(x, wg, wu, ends, a_rows=p["row_token"])
    return grouped_gemm(h, wd, ends), p


def _experts_int8(x, ids, E, wg, wu, wd):
    """The routed experts in int8 (see run): returns (y [T*k, H] bf16, permute
    dict)."""
    T, H = x.shape
    Ni = wg.shape[1]
    xq, xs = quant_rows_i8(x)
    # no gather: the expert GEMM reads token rows of xq through row_token
    p = permute(x, ids, E, index_only=True)
    counts = p["counts"]
    ends = p["offsets"][1:]
    wgq, wgs = quant_rows_i8(wg, group_rows=Ni, group_counts=counts)
    wuq, wus = quant_rows_i8(wu, group_rows=Ni, group_counts=counts)
    wdq, wds = quant_rows_i8(wd, hadamard=INT8_HADAMARD, scale_mul=1.0 / INT8_HADAMARD,
                             group_rows=H, group_counts=counts)
    h = grouped_swiglu_i8(xq, xs, wgq, wgs, wuq, wus, ends, a_rows=p["row_token"],
                          ident_a=xq, ident_scales=xs, ident_m=T)
    hq, hs = quant_rows_i8(h, hadamard=INT8_HADAMARD)
    return grouped_gemm_i8(hq, hs, wdq, wds, ends), p


# ---------------------------------------------------------------------------
# preallocated plan: one batch shape, every buffer allocated once
# ---------------------------------------------------------------------------
class MoePlan:
    """All outputs and workspaces of one (T, H, E, k) batch shape, allocated
    once (the reference's per-call arena, K:4197-4268, hoisted out of the
    call).  ``route`` / ``permute`` / ``combine`` / ``step`` then only enqueue
    kernels on the current stream through the C ABI."""

    def __init__(self, T, H, E, k, cfg: RouteCfg, device, fp8=False, w_dtype=torch.bfloat16,
                 x_dtype=torch.bfloat16):
        self.T, self.H, self.E, self.k, self.fp8 = T, H, E, k, fp8
        self.cfg = _ccfg(cfg)
        self.wd = _dtype_code(w_dtype)
        self.xd = _dtype_code(x_dtype)
        dev = torch.device(device)
        ns = T * k
        L = lib()
        self.logits = torch.empty(T, E, dtype=torch.float32, device=dev)
        self.topk_ids = torch.empty(T, k, dtype=torch.int32, device=dev)
        self.topk_w = torch.empty(T, k, dtype=torch.float32, device=dev)
        self.route_counts = torch.empty(E, dtype=torch.int32, device=dev)
        self.row_token = torch.empty(ns, dtype=torch.int32, device=dev)
        self.pair_row = torch.empty(ns, dtype=torch.int32, device=dev)
        self.offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
        self.counts = torch.empty(E, dtype=torch.int32, device=dev)
        if fp8:
            self.xg = torch.empty(ns, H, dtype=torch.uint8, device=dev)
            self.scales = torch.empty(ns, H // 128, dtype=torch.float32, device=dev)
        else:
            self.xg = torch.empty(ns, H, dtype=x_dtype, device=dev)
            self.scales = None
        self.x_dtype, self.w_dtype = x_dtype, w_dtype
        self.out = torch.empty(T, H, dtype=x_dtype, device=dev)  # combine writes y's dtype
        self.nws_route = L.moe_route_workspace_bytes(T, H, E, self.wd)
        self.ws_route = torch.empty(max(self.nws_route, 256), dtype=torch.uint8, device=dev)
        self.nws_perm = (L.moe_permute_fp8_workspace_bytes(T, H, E, k) if fp8
                         else L.moe_permute_workspace_bytes(T, E, k))
        self.ws_perm = torch.empty(max(self.nws_perm, 256), dtype=torch.uint8, device=dev)
        # one call for route + permute (bf16 x): the route's and the permute's
        # workspaces back to back
        self.nws_rp = L.moe_route_permute_workspace_bytes(T, H, E, k, self.wd)
        self.ws_rp = (torch.empty(max(self.nws_rp, 256), dtype=torch.uint8, device=dev)
                      if x_dtype == torch.bfloat16 else None)

    def route(self, x, w, bias, counts=False):
        """Router GEMM + scoring + top-k.  The per-expert counts are also
        produced by ``permute``; ``counts=True`` additionally fills
        ``route_counts`` from the scoring kernel's histogram."""
        _want(x, "x", _BF16, (self.T, self.H))
        _want(w, "w", (self.w_dtype,), (self.E, self.H))
        if bias is not None:
            _want(bias, "bias", _F32, (self.E,))
        _devs(x=x, w=w, bias=bias)
        _check(lib().moe_route(_ptr(x), _ptr(w), self.wd, _ptr(bias), self.T, self.H, self.E,
                               self.k, ctypes.byref(self.cfg), _ptr(self.logits),
                               _ptr(self.topk_ids), _ptr(self.topk_w),
                               _ptr(self.route_counts) if counts else None,
                               _ptr(self.ws_route), self.nws_route, _stream(x)))

    def router_gemm(self, x, w):
        _want(x, "x", _BF16, (self.T, self.H))
        _want(w, "w", _BF16, (self.E, self.H))
        _devs(x=x, w=w)
        _check(lib().moe_router_gemm(_ptr(x), _ptr(w), self.T, self.H, self.E, _ptr(self.logits),
                                     _stream(x)))

    def topk_only(self, bias):
        """Scoring + top-k on the current ``logits`` (used to time the stage)."""
        _check(lib().moe_topk(_ptr(self.logits), _ptr(bias), self.T, self.E, self.k,
                              ctypes.byref(self.cfg), _ptr(self.topk_ids), _ptr(self.topk_w), None,
                              _stream(self.logits)))

    def permute(self, x, index_only=False):
        _devs(x=_want(x, "x", (self.x_dtype,), (self.T, self.H)))
        od = DTYPE_FP8E4M3FN if self.fp8 else self.xd
        _check(lib().moe_permute(_ptr(x), self.xd, _ptr(self.topk_ids), self.T, self.H, self.E,
                                 self.k, od, None if index_only else _ptr(self.xg),
                                 _ptr(self.scales),
                                 _ptr(self.row_token), _ptr(self.pair_row), _ptr(self.offsets),
                                 _ptr(self.counts), _ptr(self.ws_perm), self.nws_perm,
                                 _stream(x)))

    def route_permute(self, x, w, bias, index_only=False):
        """``route`` then ``permute`` in one C-ABI call (moe_route_permute):
        the same outputs; where the route is the fused kernel its epilogue
        also writes the permute's block histograms.  bf16 x only."""
        if self.ws_rp is None:
            raise RuntimeError("route_permute needs bf16 x")
        _want(x, "x", _BF16, (self.T, self.H))
        _want(w, "w", (self.w_dtype,), (self.E, self.H))
        if bias is not None:
            _want(bias, "bias", _F32, (self.E,))
        _devs(x=x, w=w, bias=bias)
        od = DTYPE_FP8E4M3FN if self.fp8 else self.xd
        _check(lib().moe_route_permute(
            _ptr(x), _ptr(w), self.wd, _ptr(bias), self.T, self.H, self.E, self.k,
            ctypes.byref(self.cfg), _ptr(self.logits), _ptr(self.topk_ids), _ptr(self.topk_w), od,
            None if index_only else _ptr(self.xg), _ptr(self.scales), _ptr(self.row_token),
            _ptr(self.pair_row), _ptr(self.offsets), _ptr(self.counts), _ptr(self.ws_rp),
            self.nws_rp, _stream(x)))

    def combine(self, y, shared=None):
        if y is None:  # identity experts: combine the gathered rows
            if self.fp8:
                raise RuntimeError("identity experts need the bf16 / fp32 permute (fp8 rows "
                                   "are not a combine input)")
            y = self.xg
        _want(y, "y", (self.out.dtype,), (self.T * self.k, self.H))
        if shared is not None:
            _want(shared, "shared", (self.out.dtype,), (self.T, self.H))
        _devs(y=y, shared=shared)
        _check(lib().moe_combine(_ptr(y), _dtype_code(y.dtype), _ptr(self.pair_row),
                                 _ptr(self.topk_w), _ptr(shared), self.T, self.H, self.k,
                                 _ptr(self.out), _stream(y)))

    def step(self, x, w, bias, y):
        """route -> permute -> combine for one batch.  y None: identity experts
        (the C1 configuration), i.e. the gathered rows are combined, which
        returns x when the weights sum to 1.  bf16 x: route and permute are
        one call (``route_permute``)."""
        if self.ws_rp is not None:
            self.route_permute(x, w, bias)
        else:
            self.route(x, w, bias)
            self.permute(x)
        self.combine(y)
        return self.out
