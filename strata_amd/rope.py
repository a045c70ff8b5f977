"""Stereographic RoPE tables (host side of the RoPE + QKV-pack prologue).

Mirrors the helpers the reference imports from physicsnemo
(``spherical_centroid``, ``stereographic_projection``,
``build_axial_rope_cos_sin_2d_continuous``; screamcast/strata_wrappers.py:52,
docker/Dockerfile:164-168), which are not available here.  The conventions
this build fixes (the reference leaves them to physicsnemo):

* Centre: spherical centroid of the tile's token positions, i.e. the
  normalised mean of their unit vectors.
* Projection: textbook stereographic projection of the unit sphere about the
  centre (Snyder 1987, USGS PP 1395, eqs. 21-2..21-4).
* Coordinates are divided by the RoPE length scale (screamcast/tile_geometry.py:157-170,
  screamcast/strata_wrappers.py:134-150,333-338).
* Frequencies: P = D/2 pairs; the first P/2 pairs rotate by x, the last P/2 by
  y, with angular frequency ``base ** (-j / (P/2))`` for j in [0, P/2)
  (axial 2D RoPE; RoFormer frequency schedule per axis).
* Tables are ``[B, 1, Y, X, P]`` (one table per tile, broadcast over the
  vertical level index z), float32.  With ``level_pairs`` = L > 0 (BASELINE
  configs[1]'s level index in z) the pairs split x | y | level instead: [0, n)
  rotate by x, [n, 2n) by y, [2n, P) by the level index z = 0..Z-1, n = (P-L)/2,
  each group with frequencies base^(-j/m) over its own size m; the tables are
  then ``[B, Z, Y, X, P]``.
* Pair layout of the rotated vector: "half" (pair p = (p, p + D/2)).

Tables cost O(B*Y*X*P) and are built with torch ops on the tokens' device;
they are kernel inputs, not part of the timed hot path.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


def default_rope_length_scale(patch_size_horiz: int = 1) -> float:
    """sqrt(pi * ph^2 / (3 * 1024^2)) (screamcast/tile_geometry.py:157-170)."""
    return math.sqrt(math.pi * patch_size_horiz**2 / (3.0 * 1024**2))


def spherical_centroid(lat: Tensor, lon: Tensor) -> tuple[Tensor, Tensor]:
    """Centroid of points on the unit sphere; lat/lon ``[B, ...]`` radians -> ``[B]``."""
    B = lat.shape[0]
    cl = torch.cos(lat)
    vx = (cl * torch.cos(lon)).reshape(B, -1).sum(1)
    vy = (cl * torch.sin(lon)).reshape(B, -1).sum(1)
    vz = torch.sin(lat).reshape(B, -1).sum(1)
    n = torch.sqrt(vx * vx + vy * vy + vz * vz)
    return torch.asin(vz / n), torch.atan2(vy, vx)


def stereographic_projection(lat: Tensor, lon: Tensor, lat0: Tensor, lon0: Tensor) -> tuple[Tensor, Tensor]:
    """Stereographic (x, y) of lat/lon ``[B, Y, X]`` about centres ``[B]`` (unit sphere)."""
    lat0 = lat0.reshape(-1, *([1] * (lat.dim() - 1)))
    lon0 = lon0.reshape(-1, *([1] * (lat.dim() - 1)))
    dl = lon - lon0
    s0, c0 = torch.sin(lat0), torch.cos(lat0)
    s, c = torch.sin(lat), torch.cos(lat)
    kk = 2.0 / (1.0 + s0 * s + c0 * c * torch.cos(dl))
    return kk * c * torch.sin(dl), kk * (c0 * s - s0 * c * torch.cos(dl))


def axial_rope_cos_sin(cx: Tensor, cy: Tensor, head_dim: int, base: float, cz: Tensor | None = None,
                       level_pairs: int = 0) -> tuple[Tensor, Tensor]:
    """cos/sin ``[..., D/2]`` for per-token coordinates cx, cy (and level cz) ``[...]``."""
    P = head_dim // 2
    n, rem = divmod(P - level_pairs, 2)
    if head_dim % 2 or level_pairs < 0 or rem or n < 1:
        raise ValueError(f"cannot split {P} RoPE pairs into x | y | {level_pairs} level pairs")

    def freqs(m: int) -> Tensor:
        return base ** (-torch.arange(m, dtype=torch.float64, device=cx.device) / m)

    parts = [cx.double()[..., None] * freqs(n), cy.double()[..., None] * freqs(n)]
    if level_pairs:
        if cz is None:
            raise ValueError("level pairs need level coordinates")
        parts.append(cz.double()[..., None] * freqs(level_pairs))
    ang = torch.cat(parts, dim=-1)
    return torch.cos(ang).float(), torch.sin(ang).float()


def stereographic_rope_tables(
    lat: Tensor, lon: Tensor, head_dim: int, base: float, length_scale: float, levels: int = 0,
    level_pairs: int = 0,
) -> tuple[Tensor, Tensor]:
    """Tables ``[B, 1, Y, X, D/2]`` from token lat/lon ``[B, Y, X]`` (radians); with
    ``level_pairs`` > 0, ``[B, levels, Y, X, D/2]`` whose last ``level_pairs`` pairs
    rotate by the level index z."""
    lat64, lon64 = lat.double(), lon.double()
    lat0, lon0 = spherical_centroid(lat64, lon64)
    x, y = stereographic_projection(lat64, lon64, lat0, lon0)
    x, y = x / length_scale, y / length_scale
    if not level_pairs:
        cos, sin = axial_rope_cos_sin(x, y, head_dim, base)
        return cos.unsqueeze(1).contiguous(), sin.unsqueeze(1).contiguous()
    B, Y, X = lat.shape
    z = torch.arange(levels, dtype=torch.float64, device=lat.device).view(1, levels, 1, 1).expand(B, levels, Y, X)
    cos, sin = axial_rope_cos_sin(x.unsqueeze(1).expand(B, levels, Y, X), y.unsqueeze(1).expand(B, levels, Y, X),
                                  head_dim, base, z, level_pairs)
    return cos.contiguous(), sin.contiguous()


def synthetic_tile_latlon(
    batch: int, height: int, width: int, generator: torch.Generator, spacing: float | None = None
) -> tuple[Tensor, Tensor]:
    """Token lat/lon ``[B, Y, X]`` (radians) of synthetic tiles for benchmarks.

    Each tile is a ``height x width`` grid on the local tangent plane with
    ``spacing`` radians between tokens (default: one RoPE length-scale unit),
    centred at lat0 ~ U(-60, 60) deg, lon0 ~ U(0, 360) deg drawn from
    ``generator`` (CPU), one centre per batch entry.
    """
    spacing = default_rope_length_scale(1) if spacing is None else spacing
    lat0 = (torch.rand(batch, generator=generator, dtype=torch.float64) * 120.0 - 60.0) * math.pi / 180.0
    lon0 = torch.rand(batch, generator=generator, dtype=torch.float64) * 2.0 * math.pi
    v = (torch.arange(height, dtype=torch.float64) - (height - 1) / 2) * spacing
    u = (torch.arange(width, dtype=torch.float64) - (width - 1) / 2) * spacing
    lat = lat0[:, None, None] + v[None, :, None] + 0.0 * u[None, None, :]
    lon = lon0[:, None, None] + u[None, None, :] / torch.cos(lat0)[:, None, None] + 0.0 * v[None, :, None]
    return lat, lon
