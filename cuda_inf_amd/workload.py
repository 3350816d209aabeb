"""Synthetic inputs of the attention path's workloads.

Values are N(0,1) drawn in float64 from a seeded torch generator and rounded
to fp16 (round-to-nearest-even).  K/V of the long-context workloads carry 1%
outliers multiplied by 20 to stress the group scales.  Q/K of the prefill
and short-decode workloads go through the reference's producers first:
per-head RMSNorm (eps 1e-5, unit weight; engine.cu:148-158) and rotate-half
RoPE at theta 5e6 (engine.cu:161-182), both in fp32 with fp16 results.
"""
from __future__ import annotations

import torch

from ._lib import D, NH, NKV

ROPE_THETA = 5.0e6
EPS = 1e-5


def generator(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def normal_f16(shape, g: torch.Generator, device) -> torch.Tensor:
    return torch.randn(shape, generator=g, dtype=torch.float64, device=device).to(torch.float16)


def with_outliers(x: torch.Tensor, g: torch.Generator, frac: float = 0.01,
                  mult: float = 20.0) -> torch.Tensor:
    """Multiply a Bernoulli(frac) subset of elements by mult (in fp32, back to fp16)."""
    mask = torch.rand(x.shape, generator=g, device=x.device) < frac
    y = x.float()
    y[mask] *= mult
    return y.to(torch.float16)


def rmsnorm_head(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """engine.cu:148-158 with unit weight: y = fp16(x * rsqrt(mean(x^2) + eps))."""
    xf = x.float()
    inv = torch.rsqrt((xf * xf).sum(-1, keepdim=True) / D + eps)
    return (xf * inv).to(torch.float16)


def rope(x: torch.Tensor, pos: torch.Tensor, theta: float = ROPE_THETA) -> torch.Tensor:
    """engine.cu:161-182: x [S, heads, 64] fp16, pos [S] int."""
    half = D // 2
    d = torch.arange(half, device=x.device, dtype=torch.float32)
    invf = torch.pow(torch.tensor(theta, dtype=torch.float32, device=x.device), -(2.0 * d) / D)
    ang = pos.to(torch.float32)[:, None] * invf[None, :]
    cs, sn = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    xf = x.float()
    x0, x1 = xf[..., :half], xf[..., half:]
    return torch.cat([(x0 * cs - x1 * sn), (x1 * cs + x0 * sn)], dim=-1).to(torch.float16)


def prep_qk(x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """QK-RMSNorm then RoPE (the reference's order, engine.cu:799-801)."""
    return rope(rmsnorm_head(x), pos)


def qkv(S: int, seed: int, device, *, past: int = 0, prep: bool = True,
        outliers: bool = False):
    """q [S,32,64], k, v [S,8,64] fp16 drawn in the order q, k, v."""
    g = generator(seed, device)
    q = normal_f16((S, NH, D), g, device)
    k = normal_f16((S, NKV, D), g, device)
    v = normal_f16((S, NKV, D), g, device)
    if outliers:
        k = with_outliers(k, g)
        v = with_outliers(v, g)
    if prep:
        pos = torch.arange(past, past + S, device=device)
        q = prep_qk(q, pos)
        k = prep_qk(k, pos)
    return q.contiguous(), k.contiguous(), v.contiguous()
