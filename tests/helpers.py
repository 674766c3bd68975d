"""Shared test helpers: the parity cases and input builders."""
from __future__ import annotations

import hashlib

import numpy as np
import torch

from moe_route.configs import CONFIGS, MoeConfig, RouteCfg, make_inputs  # noqa: F401

# Small cuts of every benchmark configuration (real E, k and scoring).
CUT_T = 64


def sha(t) -> str:
    """sha256 of a tensor's / array's raw bytes (bf16 viewed as int16)."""
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            t = t.view(torch.int16)
        elif t.dtype == torch.float8_e4m3fn:
            t = t.view(torch.uint8)
        t = t.numpy()
    return hashlib.sha256(np.ascontiguousarray(t).tobytes()).hexdigest()


def tie_stress_inputs(T=96, E=64, k=8, seed=3):
    """Logits with many exact ties (values on a 0.25 grid) fed straight to topk."""
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randint(-4, 5, (T, E), generator=g).float() * 0.25)
    return logits


def degenerate_ids(T=100, E=16, k=4):
    """Every token picks experts 0..k-1 (k experts full, E-k empty)."""
    return torch.arange(k, dtype=torch.int32).repeat(T, 1)


def case_cfg(name) -> MoeConfig:
    return CONFIGS[name]
