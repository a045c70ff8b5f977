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

Level index in z: with ``level_pairs = L > 0`` the P = D/2
pairs split into three axis groups, x | y | level: pairs [0, n) rotate by x,
[n, 2n) by y and [2n, P) by the token's vertical level index z (0, 1, ...,
Z-1, in level units), n = (P - L)/2; inside each group of size m the angular
frequencies are base^(-j/m), j = 0..m-1.  configs[1] uses P = 32, L = 8
(12 | 12 | 8).  ``level_pairs = 0`` is the 2D table broadcast over z.
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


def _omega(m: int, base: float) -> Tensor:
    j = torch.arange(m, dtype=torch.float64)
    return torch.pow(torch.tensor(float(base), dtype=torch.float64), -j / m)


def rope_angles(cx: Tensor, cy: Tensor, head_dim: int, base: float, cz: Tensor | None = None,
                level_pairs: int = 0) -> Tensor:
    """Angles ``[..., D/2]``: pairs [0, n) rotate by cx, [n, 2n) by cy and, with
    ``level_pairs`` = L > 0, [2n, P) by cz (n = (P - L)/2; n = P/2 without levels)."""
    P = head_dim // 2
    n = (P - level_pairs) // 2
    if level_pairs < 0 or 2 * n + level_pairs != P or n < 1:
        raise ValueError(f"cannot split {P} pairs into x | y | {level_pairs} level pairs")
    om = _omega(n, base)
    parts = [cx.double()[..., None] * om, cy.double()[..., None] * om]
    if level_pairs:
        if cz is None:
            raise ValueError("level pairs need level coordinates cz")
        parts.append(cz.double()[..., None] * _omega(level_pairs, base))
    return torch.cat(parts, dim=-1)


def tables(lat: Tensor, lon: Tensor, head_dim: int, base: float, length_scale: float, levels: int = 0,
           level_pairs: int = 0) -> tuple[Tensor, Tensor]:
    """cos/sin (float64) for token lat/lon ``[B, Y, X]``: ``[B, 1, Y, X, D/2]``, or with
    ``levels`` = Z > 0 and ``level_pairs`` > 0 ``[B, Z, Y, X, D/2]`` (level index z)."""
    lat0, lon0 = spherical_centroid(lat, lon)
    x, y = stereographic(lat, lon, lat0, lon0)
    x, y = x / length_scale, y / length_scale
    if not level_pairs:
        ang = rope_angles(x, y, head_dim, base)
        return torch.cos(ang).unsqueeze(1), torch.sin(ang).unsqueeze(1)
    B, Y, X = lat.shape
    z = torch.arange(levels, dtype=torch.float64).view(1, levels, 1, 1).expand(B, levels, Y, X)
    ang = rope_angles(x.unsqueeze(1).expand(B, levels, Y, X), y.unsqueeze(1).expand(B, levels, Y, X), head_dim,
                      base, z, level_pairs)
    return torch.cos(ang), torch.sin(ang)


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
