"""libmoe_route.so: loads, exports every declared symbol, and rejects bad
arguments with the documented error codes -- all without a GPU (validation
runs on the host before any launch)."""
import ctypes
import os
import re

import pytest
import torch

import moe_route as M

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: every call below fails validation


def header_functions():
    text = open(os.path.join(REPO, "include", "moe_route.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(moe_\w+)\s*\(", text, re.M)))


def test_library_exports_every_header_symbol():
    L = M.lib()
    names = header_functions()
    assert len(names) >= 10
    assert sorted(M.EXPORTS) == names
    for n in names:
        assert hasattr(L, n), n


def test_version_and_empty_error():
    assert M.lib().moe_version() == 1
    assert M.lib().moe_last_error_string() == b""


def cfg(**kw):
    c = M._Cfg(0, 1, 1, 1, 1.0, 0.0)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def err(rc, code, fragment=None):
    assert rc == code
    msg = M.lib().moe_last_error_string().decode()
    if fragment:
        assert fragment in msg, msg


def test_route_validation():
    L = M.lib()
    c = cfg()
    args = lambda T=16, H=128, E=8, k=2, wd=0, x=FAKE: (x, FAKE, wd, None, T, H, E, k,
                                                        ctypes.byref(c), FAKE, FAKE, FAKE, None,
                                                        None, 0, None)
    err(L.moe_route(*args(E=12)), -3, "E=12")
    err(L.moe_route(*args(k=0)), -2, "k=0")
    err(L.moe_route(*args(k=9, E=16)), -2)
    err(L.moe_route(*args(H=100)), -3, "multiple of 64")
    err(L.moe_route(*args(wd=2)), -3, "w_dtype")
    err(L.moe_route(*args(x=None)), -1)
    err(L.moe_route(*args(wd=1)), -4, "workspace")
    err(L.moe_route(*args(x=ctypes.c_void_p(0x10008))), -6)
    err(L.moe_route(*args(T=-1)), -2)


def test_group_cfg_validation():
    L = M.lib()
    def topk(c, E=256, k=8):
        return L.moe_topk(FAKE, None, 4, E, k, ctypes.byref(c), FAKE, FAKE, None, None)
    err(topk(cfg(scoring=7)), -2, "scoring")
    err(topk(cfg(scoring=1, n_group=6, topk_group=2)), -2, "power of two")
    err(topk(cfg(scoring=1, n_group=8, topk_group=9)), -2, "topk_group")
    err(topk(cfg(scoring=1, n_group=128, topk_group=4)), -3, "group size")
    err(topk(cfg(scoring=1, n_group=64, topk_group=1), E=64, k=2), -3, "group size")
    err(topk(cfg(scoring=1, n_group=32, topk_group=1), E=256, k=16), -2)
    err(L.moe_topk(FAKE, None, 4, 256, 8, None, FAKE, FAKE, None, None), -1)


def test_permute_and_combine_validation():
    L = M.lib()
    base = dict(x=FAKE, xd=0, ids=FAKE, T=8, H=256, E=16, k=2, od=0, xg=FAKE, sc=None,
                rt=FAKE, pr=FAKE, ws=FAKE, nws=1 << 20)
    def perm(**kw):
        a = dict(base, **kw)
        return L.moe_permute(a["x"], a["xd"], a["ids"], a["T"], a["H"], a["E"], a["k"], a["od"],
                             a["xg"], a["sc"], a["rt"], a["pr"], None, None, a["ws"], a["nws"],
                             None)
    err(perm(od=1), -3, "out_dtype")
    err(perm(od=2), -1, "scales")
    err(perm(od=2, sc=FAKE, H=192), -3, "128")
    err(perm(od=2, sc=FAKE, xd=1), -3)
    err(perm(H=4), -6)
    err(perm(E=0), -2)
    err(perm(k=9), -2)
    err(perm(nws=16), -4)
    err(perm(rt=None), -1)
    err(L.moe_combine(FAKE, 5, FAKE, FAKE, None, 4, 64, 2, FAKE, None), -3)
    err(L.moe_combine(FAKE, 0, FAKE, FAKE, None, 4, 4, 2, FAKE, None), -6)
    err(L.moe_combine(None, 0, FAKE, FAKE, None, 4, 64, 2, FAKE, None), -1)
    err(L.moe_combine(FAKE, 0, FAKE, FAKE, None, 4, 64, 0, FAKE, None), -2)
    assert L.moe_combine(None, 0, None, None, None, 0, 64, 2, None, None) == 0
    err(L.moe_offsets(FAKE, 2000, FAKE, None), -2)
    err(L.moe_router_gemm(FAKE, FAKE, 4, 96, 8, FAKE, None), -3)


def _router_ksplit(T, H, N):
    """K partitions of the router GEMM: the tile rule of router_gemm.hip
    (row x expert tiles 256x128 for N >= 256, 64xN for 32 <= N <= 128, 32x16
    below; K halves while blocks * ksplit stay under the fill target)."""
    bm, bn, target = (256, 128, 256) if N >= 256 else (64, N, 256) if N >= 32 else (32, 16, 1024)
    blocks = -(-T // bm) * -(-N // bn)
    ks = 1
    while blocks * ks < target and ks < 8 and H % (64 * ks * 2) == 0:
        ks *= 2
    return ks


def _route_small(H, E, fp32):
    """The small-E GEMM + scoring kernel: E = 8 or 16 with bf16 weights, E = 8 with
    fp32 weights (hi/lo split); H % 256 == 0."""
    return E in ((8,) if fp32 else (8, 16)) and H > 0 and H % 256 == 0


def _route_ws(T, H, E, fp32):
    r256 = lambda b: (b + 255) // 256 * 256
    if _route_small(H, E, fp32):
        # no K partitions (the four waves of a block split K and add in LDS), and
        # an fp32 weight is split hi/lo inside the kernel
        return 0
    N = 2 * E if fp32 else E
    parts = (N // E) * _router_ksplit(T, H, N)
    b = r256(2 * E * H * 2) if fp32 else 0
    b += r256(T * parts * E * 4) if parts > 1 else 0
    if not fp32 and (E, H) in ((256, 7168), (128, 2048)):  # fused GEMM + scoring: weight copy
        b = max(b, r256(E * H * 2))
    return b


def test_workspace_sizes():
    L = M.lib()
    # small N: 32-row tiles, 4 blocks at T=100 -> K split in 2 (H=128 allows no more)
    # -> [T, 2E] fp32 partial sums
    assert L.moe_route_workspace_bytes(100, 128, 8, 0) == 6400
    # fp32 weights: [2E,H] bf16 split (4096 B) + [T, 2 halves * 2 K parts * E] fp32
    assert L.moe_route_workspace_bytes(100, 128, 8, 1) == 4096 + 12800
    assert L.moe_route_workspace_bytes(100, 64, 8, 0) == 0        # H=64: one K step, no split
    # DeepSeek-V3 shape: the fused GEMM + scoring kernel keeps a fragment-major copy of the
    # [256, 7168] bf16 weight
    assert L.moe_route_workspace_bytes(32768, 7168, 256, 0) == 256 * 7168 * 2
    # ... but fp32 weights there still need the [2E,H] split and [T, 2E] hi/lo partial logits
    assert L.moe_route_workspace_bytes(32768, 7168, 256, 1) == 2 * 256 * 7168 * 2 + 32768 * 512 * 4
    assert L.moe_route_workspace_bytes(65536, 7168, 256, 0) == 256 * 7168 * 2
    assert L.moe_route_workspace_bytes(32768, 4096, 256, 0) == 0   # no fused kernel, no K split
    # C2 (Mixtral) shape: the small-E kernel, no workspace (with fp32 weights it splits them itself)
    assert L.moe_route_workspace_bytes(8192, 4096, 8, 0) == 0
    assert L.moe_route_workspace_bytes(8192, 4096, 8, 1) == 0
    for T, H, E in [(1, 64, 8), (100, 128, 8), (512, 1024, 8), (8192, 4096, 8), (16384, 2048, 128),
                    (300, 2048, 16), (300, 1536, 16), (512, 1024, 16), (100, 448, 8),
                    (1571, 8192, 64), (32768, 7168, 256), (300, 7168, 256), (4096, 8192, 64)]:
        for fp32 in (0, 1):
            assert L.moe_route_workspace_bytes(T, H, E, fp32) == _route_ws(T, H, E, fp32), (T, H, E, fp32)
    # T*k = 32768*8 pairs -> 1024 blocks of 256; [E, nblk] + [E] int32
    assert L.moe_permute_workspace_bytes(32768, 256, 8) == 256 * 1024 * 4 + 1024


def test_grouped_gemm_validation():
    L = M.lib()
    ws = ctypes.c_void_p(0x10000)
    args = lambda G=4, Mr=64, N=128, K=256, im=0, ia=None, wsb=4096, a=FAKE: (
        a, FAKE, FAKE, G, Mr, N, K, ia, im, FAKE, ws, wsb, None)
    err(L.moe_grouped_gemm(*args(G=0)), -2, "G=0")
    err(L.moe_grouped_gemm(*args(K=100)), -3, "multiple of 64")
    err(L.moe_grouped_gemm(*args(N=0)), -2)
    err(L.moe_grouped_gemm(*args(Mr=-1)), -2)
    err(L.moe_grouped_gemm(*args(im=-2)), -2, "ident_m")
    err(L.moe_grouped_gemm(*args(im=5)), -1, "ident_a")
    err(L.moe_grouped_gemm(*args(a=None)), -1)
    err(L.moe_grouped_gemm(*args(wsb=4)), -4, "workspace")
    err(L.moe_grouped_gemm(*args(a=ctypes.c_void_p(0x10008))), -6)
    err(L.moe_grouped_swiglu(FAKE, FAKE, None, FAKE, 4, 64, 128, 256, None, 0, FAKE, ws, 4096,
                             None), -1)
    err(L.moe_grouped_gemm_fp8(FAKE, None, FAKE, FAKE, 4, 64, 128, 256, FAKE, ws, 4096, None), -1,
        "a_scales")
    err(L.moe_grouped_gemm_fp8(FAKE, FAKE, FAKE, FAKE, 4, 64, 128, 192, FAKE, ws, 4096, None), -3,
        "128")
    err(L.moe_grouped_swiglu_fp8(FAKE, ctypes.c_void_p(0x10002), FAKE, FAKE, FAKE, 4, 64, 128, 256,
                                 FAKE, ws, 4096, None), -6)
    err(L.moe_grouped_gemm_fp8(FAKE, FAKE, FAKE, FAKE, 4, 1 << 24, 128, 1 << 14, FAKE, ws, 4096,
                               None), -3, "int32")
    # a, a_rows, w, offs, G, M, N, K, out, ws, ws_bytes, stream
    err(L.moe_grouped_gemm_rows(FAKE, None, FAKE, FAKE, 4, 64, 128, 256, FAKE, ws, 4096, None), -1,
        "a_rows")
    err(L.moe_grouped_swiglu_rows(FAKE, ctypes.c_void_p(0x10002), FAKE, FAKE, FAKE, 4, 64, 128,
                                  256, FAKE, ws, 4096, None), -6, "a_rows")
    err(L.moe_grouped_gemm_rows(FAKE, FAKE, FAKE, FAKE, 4, 64, 128, 100, FAKE, ws, 4096, None), -3)
    assert L.moe_grouped_gemm_workspace_bytes(64) == 512
    assert L.moe_grouped_gemm_workspace_bytes(0) == 256
    assert L.moe_grouped_gemm_workspace_bytes(-1) == 0


def test_int8_validation():
    L = M.lib()
    ws = ctypes.c_void_p(0x10000)
    # a, a_scales, a_rows, w, w_scales, offs, G, M, N, K, ident_a, ident_scales, ident_m,
    # out, ws, ws_bytes, stream
    args = lambda G=4, Mr=64, K=256, sc=FAKE, ia=None, isc=None, im=0, idx=None, wsb=4096: (
        FAKE, sc, idx, FAKE, FAKE, FAKE, G, Mr, 128, K, ia, isc, im, FAKE, ws, wsb, None)
    err(L.moe_grouped_gemm_i8(*args(K=192)), -3, "multiple of 128")
    err(L.moe_grouped_gemm_i8(*args(G=0)), -2, "G=0")
    err(L.moe_grouped_gemm_i8(*args(sc=None)), -1, "scales")
    err(L.moe_grouped_gemm_i8(*args(im=8, ia=FAKE)), -1, "ident_scales")
    err(L.moe_grouped_gemm_i8(*args(idx=ctypes.c_void_p(0x10002))), -6)
    err(L.moe_grouped_gemm_i8(*args(wsb=8)), -4, "workspace")
    err(L.moe_grouped_swiglu_i8(FAKE, FAKE, None, FAKE, FAKE, FAKE, None, FAKE, 4, 64, 128, 256,
                                None, None, 0, FAKE, ws, 4096, None), -1)
    # x, R, K, hadamard, scale_mul, group_rows, group_counts, q, scales, stream
    q = lambda R=4, K=256, had=0, mul=1.0, gr=0, gc=None, x=FAKE: (
        x, R, K, had, mul, gr, gc, FAKE, FAKE, None)
    err(L.moe_quant_rows_i8(*q(had=64)), -2, "hadamard")
    err(L.moe_quant_rows_i8(*q(K=200, had=128)), -3, "multiple of 128")
    err(L.moe_quant_rows_i8(*q(K=24)), -3, "multiple of 16")
    err(L.moe_quant_rows_i8(*q(K=40, had=16)), -3, "multiple of 16")
    err(L.moe_quant_rows_i8(*q(K=16384 + 128)), -3)
    err(L.moe_quant_rows_i8(*q(mul=0.0)), -2, "scale_mul")
    err(L.moe_quant_rows_i8(*q(mul=float("inf"))), -2, "scale_mul")
    err(L.moe_quant_rows_i8(*q(gc=FAKE)), -2, "group_rows")
    err(L.moe_quant_rows_i8(*q(R=6, gr=4, gc=FAKE)), -2, "divide")
    err(L.moe_quant_rows_i8(*q(R=5000, gr=1, gc=FAKE)), -3, "groups")
    err(L.moe_quant_rows_i8(*q(x=None)), -1)
    err(L.moe_quant_rows_i8(*q(x=ctypes.c_void_p(0x10008))), -6)
    err(L.moe_quant_rows_i8(*q(R=-1)), -2)
    assert L.moe_quant_rows_i8(*q(R=0, x=None)) == 0   # nothing to do: no pointer needed


def test_python_layer_refuses_cpu_tensors():
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        M.router_gemm(x, x)
    with pytest.raises(RuntimeError, match="no CPU path"):
        M.permute(x, torch.zeros(4, 2, dtype=torch.int32), 8)
    with pytest.raises(RuntimeError, match="no CPU path"):
        M.quant_rows_i8(x)


def test_python_layer_checks_dtype_and_shape_first():
    """A wrong dtype or shape is refused before the bare pointer reaches the C
    ABI (it would be read as another layout, or written past a buffer)."""
    xf = torch.zeros(4, 64)
    xb = xf.to(torch.bfloat16)
    w = torch.zeros(8, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="x must be bfloat16, got float32"):
        M.route(xf, w, None, 2, M.RouteCfg())
    with pytest.raises(RuntimeError, match=r"w must have shape \(8, 64\)"):
        M.route(xb, w[:, :32], None, 2, M.RouteCfg())
    with pytest.raises(RuntimeError, match="bias must be float32"):
        M.route(xb, w, torch.zeros(8, dtype=torch.bfloat16), 2, M.RouteCfg())
    with pytest.raises(RuntimeError, match="topk_ids must be int32"):
        M.permute(xb, torch.zeros(4, 2, dtype=torch.int64), 8)
    with pytest.raises(RuntimeError, match="pair_row must hold T"):
        M.combine(xb.repeat(2, 1), torch.zeros(7, dtype=torch.int32), torch.zeros(4, 2))
    with pytest.raises(RuntimeError, match="out must be bfloat16"):
        M.combine(xb.repeat(2, 1), torch.zeros(4, 2, dtype=torch.int32), torch.zeros(4, 2),
                  out=torch.zeros(4, 64))
    with pytest.raises(RuntimeError, match="logits must be float32"):
        M.topk(xb, None, 2, M.RouteCfg())


def test_plan_checks_inputs_against_its_shape():
    """MoePlan (buffers allocated for one shape) refuses inputs of another
    dtype or shape; its combine output takes the rows' dtype."""
    plan = M.MoePlan(4, 64, 8, 2, M.RouteCfg(), "cpu", x_dtype=torch.float32,
                     w_dtype=torch.float32)
    assert plan.out.dtype == torch.float32 and plan.xg.dtype == torch.float32
    xf = torch.zeros(4, 64)
    wf = torch.zeros(8, 64)
    with pytest.raises(RuntimeError, match="x must be bfloat16, got float32"):
        plan.route(xf, wf, None)  # the router reads bf16 hidden states
    with pytest.raises(RuntimeError, match="w must be float32"):
        plan.route(xf.to(torch.bfloat16), wf.to(torch.bfloat16), None)
    with pytest.raises(RuntimeError, match=r"x must have shape \(4, 64\)"):
        plan.permute(torch.zeros(5, 64))
    with pytest.raises(RuntimeError, match="y must be float32"):
        plan.combine(torch.zeros(8, 64, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="no CPU path"):
        plan.combine(None)  # identity experts: the plan's own rows pass the checks
    p8 = M.MoePlan(4, 128, 8, 2, M.RouteCfg(), "cpu", fp8=True)
    with pytest.raises(RuntimeError, match="identity experts"):
        p8.combine(None)


def test_run_rejects_bad_options():
    """run()'s keyword options are checked before any device work."""
    hs = torch.zeros(1, 4, 64, dtype=torch.bfloat16)
    args = (hs,) + (None,) * 8 + (1e-6,)
    with pytest.raises(RuntimeError, match="dispatch"):
        M.run(*args, dispatch="int4")
    with pytest.raises(RuntimeError, match="experts"):
        M.run(*args, experts="fp4")
    with pytest.raises(RuntimeError, match="dispatch must stay"):
        M.run(*args, experts="int8", dispatch="fp8")
    with pytest.raises(RuntimeError, match="no CPU path"):
        M.run(*args, experts="int8")


def test_missing_library_raises(monkeypatch):
    monkeypatch.setattr(M, "_lib", None)
    monkeypatch.setattr(M, "LIB_PATH", "/nonexistent/libmoe_route.so")
    with pytest.raises(RuntimeError, match="not built"):
        M.lib()


def test_error_string_is_thread_local():
    """moe_last_error_string() belongs to the calling thread: two threads that
    fail with different messages each read back their own."""
    import threading
    L = M.lib()
    barrier = threading.Barrier(2)
    got = {}

    def worker(name, E):
        rc = L.moe_router_gemm(FAKE, FAKE, 4, 128, E, FAKE, None)
        barrier.wait()   # both calls have failed before either reads its message
        got[name] = (rc, L.moe_last_error_string().decode())

    ts = [threading.Thread(target=worker, args=("a", 12)),
          threading.Thread(target=worker, args=("b", 24))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert got["a"][0] == -3 and "E=12" in got["a"][1]
    assert got["b"][0] == -3 and "E=24" in got["b"][1]


def test_permute_noalloc_validation():
    """The allocation-free permute shares moe_permute's checks and refuses
    sizes whose histograms exceed its fixed device scratch -- before any HIP
    call, so this runs without a GPU."""
    L = M.lib()
    cap = L.moe_permute_noalloc_max_scratch_bytes()
    assert cap == 4 << 20
    def perm(T=8, H=256, E=16, k=2, od=0, sc=None, x=FAKE, rt=FAKE):
        return L.moe_permute_noalloc(x, 0, FAKE, T, H, E, k, od, FAKE, sc, rt, FAKE, None, None,
                                     None)
    err(perm(od=1), -3, "out_dtype")
    err(perm(od=2), -1, "scales")
    err(perm(H=4), -6)
    err(perm(E=0), -2)
    err(perm(k=9), -2)
    err(perm(rt=None), -1)
    err(perm(x=None), -1)
    # largest T that fits at E=256, k=8: ceil(T*8/256) blocks x 256 experts x 4 B + 1 KiB
    T_max = ((cap - 1024) // (256 * 4)) * 32
    assert L.moe_permute_workspace_bytes(T_max, 256, 8) <= cap
    assert L.moe_permute_workspace_bytes(T_max + 1, 256, 8) > cap
    assert T_max == 131040
    err(perm(T=T_max + 1, H=7168, E=256, k=8), -3, "scratch")


def test_route_permute_workspace_and_validation():
    """moe_route_permute: workspace = the route's (rounded up to 256 bytes)
    then the permute's with its fp8 scale stage (T * H/128 fp32, rounded up
    to 256 bytes, when H % 128 == 0); every argument of both stages is
    checked before any launch."""
    L = M.lib()
    r256 = lambda n: (n + 255) // 256 * 256
    for (T, H, E, k) in [(32768, 7168, 256, 8), (16384, 2048, 128, 8), (100, 128, 8, 2),
                         (0, 7168, 256, 8), (4133, 7168, 256, 5), (100, 64, 8, 2),
                         (8192, 4096, 8, 2), (1001, 1024, 8, 2), (300, 2048, 16, 8),
                         (300, 2048, 16, 3), (70000, 4096, 8, 2), (5000, 4096, 16, 1)]:
        stage = r256(T * (H // 128) * 4) if T > 0 and H % 128 == 0 else 0
        # the small-E route's 32-token histograms [E, ceil(T/32)] for the permute, when
        # 256 / k tokens are whole 32-token columns and E * columns <= 8192
        ncol = -(-T // 32)
        sub = r256(E * ncol * 4) if (T > 0 and _route_small(H, E, 0) and 256 % k == 0
                                     and (256 // k) % 32 == 0 and E * ncol <= 8192) else 0
        assert L.moe_permute_fp8_workspace_bytes(T, H, E, k) == \
            L.moe_permute_workspace_bytes(T, E, k) + stage
        assert L.moe_route_permute_workspace_bytes(T, H, E, k, 0) == \
            r256(L.moe_route_workspace_bytes(T, H, E, 0)) + L.moe_permute_workspace_bytes(T, E, k) \
            + stage + sub, (T, H, E, k)
    # C2: 8 x 256 columns of 32 tokens
    assert L.moe_route_permute_workspace_bytes(8192, 4096, 8, 2, 0) == \
        L.moe_permute_fp8_workspace_bytes(8192, 4096, 8, 2) + 8 * 256 * 4
    assert L.moe_permute_fp8_workspace_bytes(32768, 7168, 256, 8) - \
        L.moe_permute_workspace_bytes(32768, 256, 8) == 32768 * 56 * 4
    assert L.moe_route_permute_workspace_bytes(-1, 7168, 256, 8, 0) == 0
    assert L.moe_permute_fp8_workspace_bytes(-1, 7168, 256, 8) == 0
    c = cfg()
    need = L.moe_route_permute_workspace_bytes(16, 128, 8, 2, 0)

    def args(T=16, H=128, E=8, k=2, x=FAKE, od=0, xg=FAKE, rt=FAKE, ws=FAKE, nws=None):
        n = L.moe_route_permute_workspace_bytes(T, H, E, k, 0) if nws is None else nws
        return (x, FAKE, 0, None, T, H, E, k, ctypes.byref(c), FAKE, FAKE, FAKE, od, xg, None,
                rt, FAKE, FAKE, FAKE, ws, n, None)

    err(L.moe_route_permute(*args(ws=None)), -4, "workspace")
    err(L.moe_route_permute(*args(nws=need - 1)), -4, "workspace")
    err(L.moe_route_permute(*args(ws=ctypes.c_void_p(0x10008))), -6, "aligned")
    err(L.moe_route_permute(*args(k=9, E=16)), -2)
    err(L.moe_route_permute(*args(E=12)), -3, "E=12")
    err(L.moe_route_permute(*args(x=None)), -1)
    err(L.moe_route_permute(*args(od=1)), -3, "out_dtype")
    err(L.moe_route_permute(*args(od=2, H=64)), -3, "H % 128")
    err(L.moe_route_permute(*args(rt=None)), -1, "row_token")
