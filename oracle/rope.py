"""CPU restatement (float64) of the Strata stereographic RoPE — test infrastructure.

Reference: the attention of physicsnemo's Strata applies RoPE from the tile's
stereographic coordinates (helpers imported at screamcast/strata_wrappers.py:52
and docker/Dockerfile:164-168; mode chosen by _rope_mode at :153-162; length
scale from _resolve_rope_base :134-150 times the patch size :333-338, default
sqrt(pi*ph^2/(3*1024^2)) at screamcast/tile_geometry.py:157-170).  physicsnemo is
not installable here, so the formulas are the textbook ones:
  * stereographic projection of the unit sphere about (phi0, lam0) — Snyder,
    "Map Projections: A Working Manual", USGS PP 1395 (1987), eqs. 21-2..21-4;
  * rotary embedding — Su et al., "RoFormer" (2021): pair (a, b) rotated by
    theta = coord * base^(-j/(P/2)) per axis.
Conventions (pair split x | y, half pair layout, spherical-centroid centre,
tables broadcast over z) are the build's, recorded with the fixtures.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


def default_rope_length_scale(patch_size_horiz: int = 1) -> float:
    """screamcast/tile_geometry.py:157-170."""
    return math.sqrt(math.pi * patch_size_horiz**2 / (3.0 * 1024**2))


def unit_vectors(lat: Tensor, lon: Tensor) -> Tensor:
    lat, lon = lat.double(), lon.double()
    return torch.stack([torch.cos(lat) * torch.cos(lon), torch.cos(lat) * torch.sin(lon), torch.sin(lat)], dim=-1)


def spherical_centroid(lat: Tensor, lon: Tensor) -> tuple[Tensor, Tensor]:
    """Per batch entry: direction of the summed unit vectors of all points."""
    B = lat.shape[0]
    s = unit_vectors(lat, lon).reshape(B, -1, 3).sum(1)
    s = s / s.norm(dim=-1, keepdim=True)
    return torch.asin(s[:, 2]), torch.atan2(s[:, 1], s[:, 0])


def stereographic(lat: Tensor, lon: Tensor, lat0: Tensor, lon0: Tensor) -> tuple[Tensor, Tensor]:
    """Snyder eqs. 21-2..21-4 with R = 1 and scale factor k0 = 1 (k = 2/(1+cos c))."""
    lat, lon = lat.double(), lon.double()
    shape = [-1] + [1] * (lat.dim() - 1)
    p0, l0 = lat0.double().reshape(shape), lon0.double().reshape(shape)
    cosc = torch.sin(p0) * torch.sin(lat) + torch.cos(p0) * torch.cos(lat) * torch.cos(lon - l0)
    kk = 2.0 / (1.0 + cosc)
    x = kk * torch.cos(lat) * torch.sin(lon - l0)
    y = kk * (torch.cos(p0) * torch.sin(lat) - torch.sin(p0) * torch.cos(lat) * torch.cos(lon - l0))
    return x, y


def rope_angles(cx: Tensor, cy: Tensor, head_dim: int, base: float) -> Tensor:
    """Angles ``[..., D/2]``: pairs [0, P/2) rotate by cx, [P/2, P) by cy."""
    half = head_dim // 4
    j = torch.arange(half, dtype=torch.float64)
    omega = torch.pow(torch.tensor(float(base), dtype=torch.float64), -j / half)
    return torch.cat([cx.double()[..., None] * omega, cy.double()[..., None] * omega], dim=-1)


def tables(lat: Tensor, lon: Tensor, head_dim: int, base: float, length_scale: float) -> tuple[Tensor, Tensor]:
    """cos/sin ``[B, 1, Y, X, D/2]`` (float64) for token lat/lon ``[B, Y, X]``."""
    lat0, lon0 = spherical_centroid(lat, lon)
    x, y = stereographic(lat, lon, lat0, lon0)
    ang = rope_angles(x / length_scale, y / length_scale, head_dim, base)
    return torch.cos(ang).unsqueeze(1), torch.sin(ang).unsqueeze(1)


def apply_rope(t: Tensor, cos: Tensor, sin: Tensor, layout: str = "half") -> Tensor:
    """Rotate the channel pairs of heads-last ``t [B, Z, Y, X, H, D]``.

    cos/sin ``[B, Zt, Y, X, D/2]`` broadcast over z (Zt = 1) and heads."""
    c = cos.unsqueeze(-2).to(t.dtype)  # [B, Zt, Y, X, 1, P]
    s = sin.unsqueeze(-2).to(t.dtype)
    D = t.shape[-1]
    if layout == "half":
        a, b = t[..., : D // 2], t[..., D // 2 :]
        return torch.cat([a * c - b * s, a * s + b * c], dim=-1)
    if layout == "interleaved":
        a, b = t[..., 0::2], t[..., 1::2]
        return torch.stack([a * c - b * s, a * s + b * c], dim=-1).reshape(t.shape)
    raise ValueError(f"unknown rope layout {layout!r}")


def pooled_latlon(lat: Tensor, lon: Tensor, f: int = 2) -> tuple[Tensor, Tensor]:
    """Spherical centroid of each f x f block of pixels: ``[B, Y, X]`` -> ``[B, Y/f, X/f]``."""
    B, Y, X = lat.shape
    v = unit_vectors(lat, lon).view(B, Y // f, f, X // f, f, 3).sum(dim=(2, 4))
    v = v / v.norm(dim=-1, keepdim=True)
    return torch.asin(v[..., 2]), torch.atan2(v[..., 1], v[..., 0])
