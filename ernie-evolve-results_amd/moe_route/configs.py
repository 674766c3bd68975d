"""The benchmark configurations of the MoE route -> dispatch -> combine path
and their seeded synthetic inputs.

C1 toy (CPU-runnable), C2 Mixtral, C3 Qwen3 with Zipf-skewed bias, C4
DeepSeek-V3, C5 DeepSeek-V3 with an fp8 permute.  Inputs are drawn in the
order x, W, bias, y from one generator seeded with `seed`.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

SCORING_SOFTMAX = 0
SCORING_SIGMOID_GROUP = 1
SCORING_SOFTMAX_BIAS = 2


@dataclass
class RouteCfg:
    """Mirror of ``moe_route_cfg`` (include/moe_route.h)."""
    scoring: int = SCORING_SOFTMAX
    renormalize: bool = True
    n_group: int = 1
    topk_group: int = 1
    route_scale: float = 1.0
    norm_min: float = 0.0


@dataclass
class MoeConfig:
    name: str
    T: int
    H: int
    E: int
    k: int
    cfg: RouteCfg = field(default_factory=RouteCfg)
    x_dtype: torch.dtype = torch.bfloat16
    bias: str = "none"      # none | zipf | randn
    fp8: bool = False
    identity_experts: bool = False
    description: str = ""


CONFIGS = {
    "C1": MoeConfig("C1", 512, 1024, 8, 2, RouteCfg(), x_dtype=torch.float32,
                    identity_experts=True,
                    description="toy: T=512 H=1024 E=8 top-2 softmax renorm, fp32, identity experts"),
    "C2": MoeConfig("C2", 8192, 4096, 8, 2, RouteCfg(),
                    description="Mixtral: T=8192 H=4096 E=8 top-2 softmax renorm, bf16"),
    "C3": MoeConfig("C3", 16384, 2048, 128, 8, RouteCfg(), bias="zipf",
                    description="Qwen3 skewed: T=16384 H=2048 E=128 top-8 softmax renorm, "
                                "logit bias 2*ln(1/rank)"),
    "C4": MoeConfig("C4", 32768, 7168, 256, 8,
                    RouteCfg(SCORING_SIGMOID_GROUP, True, 8, 4, 2.5), bias="randn",
                    description="DeepSeek-V3: T=32768 H=7168 E=256 top-8 sigmoid+bias, "
                                "8 groups keep 4, x2.5"),
    "C5": MoeConfig("C5", 32768, 7168, 256, 8,
                    RouteCfg(SCORING_SIGMOID_GROUP, True, 8, 4, 2.5), bias="randn", fp8=True,
                    description="DeepSeek-V3 with fp8 e4m3fn permute + 1x128 scales"),
}


def make_inputs(cfg: MoeConfig, T: int | None = None, seed: int = 0, device="cpu",
                with_y: bool = True):
    """Seeded synthetic inputs (x, w, bias, y) of config `cfg` with T tokens.

    device="cpu" draws on the host generator (bit-identical everywhere, used
    for parity); a CUDA device draws on that device's generator (fast, used
    for the full-size benchmark)."""
    T = cfg.T if T is None else T
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(T, cfg.H, generator=g, device=dev).to(cfg.x_dtype)
    w = (torch.randn(cfg.E, cfg.H, generator=g, device=dev) * 0.02).to(cfg.x_dtype)
    if cfg.bias == "zipf":
        bias = torch.tensor([2.0 * math.log(1.0 / (e + 1)) for e in range(cfg.E)],
                            dtype=torch.float32, device=dev)
    elif cfg.bias == "randn":
        bias = torch.randn(cfg.E, generator=g, device=dev) * 0.1
    else:
        bias = None
    y = None
    if with_y and not cfg.identity_experts:
        y = torch.randn(T * cfg.k, cfg.H, generator=g, device=dev).to(cfg.x_dtype)
    return x, w, bias, y
