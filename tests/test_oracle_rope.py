"""Pins of the CPU stereographic-RoPE oracle and of the product's table builder (no GPU)."""

import math

import torch

from oracle import rope as R
from strata_amd import rope as P


def test_length_scale_matches_reference_constant():
    # tests/test_dit_3d_pixel.py:335-343 of the reference pins these values
    assert R.default_rope_length_scale(4) == math.sqrt(math.pi * 4**2 / (3.0 * 1024**2))
    assert P.default_rope_length_scale(1) == math.sqrt(math.pi / (3.0 * 1024**2))


def test_stereographic_closed_forms():
    # centre maps to the origin
    lat0 = torch.tensor([0.3], dtype=torch.float64)
    lon0 = torch.tensor([1.1], dtype=torch.float64)
    x, y = R.stereographic(lat0.view(1, 1, 1), lon0.view(1, 1, 1), lat0, lon0)
    assert abs(x.item()) < 1e-15 and abs(y.item()) < 1e-15
    # equatorial aspect, point on the equator: x = 2 tan(dlon/2), y = 0
    lam = torch.tensor([[[0.4, -0.9, 1.3]]], dtype=torch.float64)
    x, y = R.stereographic(torch.zeros_like(lam), lam, torch.zeros(1, dtype=torch.float64), torch.zeros(1, dtype=torch.float64))
    assert torch.allclose(x, 2 * torch.tan(lam / 2)) and torch.allclose(y, torch.zeros_like(y))
    # equatorial aspect, point on the central meridian: y = 2 tan(lat/2)
    phi = torch.tensor([[[0.2, -0.7]]], dtype=torch.float64)
    x, y = R.stereographic(phi, torch.zeros_like(phi), torch.zeros(1, dtype=torch.float64), torch.zeros(1, dtype=torch.float64))
    assert torch.allclose(y, 2 * torch.tan(phi / 2)) and torch.allclose(x, torch.zeros_like(x), atol=1e-15)
    # polar aspect: radius 2 tan(pi/4 - lat/2)
    phi = torch.tensor([[[1.2, 0.9]]], dtype=torch.float64)
    lam = torch.tensor([[[0.3, 2.0]]], dtype=torch.float64)
    x, y = R.stereographic(phi, lam, torch.tensor([math.pi / 2], dtype=torch.float64), torch.zeros(1, dtype=torch.float64))
    assert torch.allclose(torch.sqrt(x * x + y * y), 2 * torch.tan(math.pi / 4 - phi / 2))


def test_centroid_of_symmetric_points():
    lat = torch.tensor([[[0.1, 0.1], [-0.1, -0.1]]], dtype=torch.float64)
    lon = torch.tensor([[[0.5, 0.7], [0.5, 0.7]]], dtype=torch.float64)
    la, lo = R.spherical_centroid(lat, lon)
    assert abs(la.item()) < 1e-15 and abs(lo.item() - 0.6) < 1e-12


def test_rotation_preserves_pair_norms_and_is_relative():
    g = torch.Generator().manual_seed(0)
    D = 16
    t = torch.randn(1, 1, 1, 3, 1, D, generator=g, dtype=torch.float64)
    cx = torch.tensor([[0.0, 1.5, -2.0]], dtype=torch.float64)
    cy = torch.tensor([[0.0, 0.5, 3.0]], dtype=torch.float64)
    ang = R.rope_angles(cx, cy, D, 100.0)  # [1, 3, P]
    cos, sin = torch.cos(ang)[:, None, None], torch.sin(ang)[:, None, None]  # [1,1,1,3,P]
    cos, sin = cos.reshape(1, 1, 1, 3, D // 2), sin.reshape(1, 1, 1, 3, D // 2)
    r = R.apply_rope(t, cos, sin)
    # zero angle is the identity
    assert torch.allclose(r[..., 0, :, :], t[..., 0, :, :])
    for layout in ("half", "interleaved"):
        rr = R.apply_rope(t, cos, sin, layout)
        if layout == "half":
            n0 = t[..., : D // 2] ** 2 + t[..., D // 2 :] ** 2
            n1 = rr[..., : D // 2] ** 2 + rr[..., D // 2 :] ** 2
        else:
            n0 = t[..., 0::2] ** 2 + t[..., 1::2] ** 2
            n1 = rr[..., 0::2] ** 2 + rr[..., 1::2] ** 2
        assert torch.allclose(n0, n1)
    # <R(a) q, R(b) k> depends only on a - b
    q = torch.randn(D, generator=g, dtype=torch.float64)
    k = torch.randn(D, generator=g, dtype=torch.float64)

    def rot(vec, ax, ay):
        a = R.rope_angles(torch.tensor([ax], dtype=torch.float64), torch.tensor([ay], dtype=torch.float64), D, 100.0)
        return R.apply_rope(vec.view(1, 1, 1, 1, 1, D), torch.cos(a).view(1, 1, 1, 1, -1), torch.sin(a).view(1, 1, 1, 1, -1)).view(D)

    d1 = rot(q, 2.0, -1.0) @ rot(k, 0.5, 0.25)
    d2 = rot(q, 1.5, -1.25) @ rot(k, 0.0, 0.0)
    assert abs(d1 - d2) < 1e-12


def test_product_tables_match_oracle():
    g = torch.Generator().manual_seed(0)
    lat, lon = P.synthetic_tile_latlon(2, 16, 24, g)
    ls = P.default_rope_length_scale(1)
    c1, s1 = P.stereographic_rope_tables(lat, lon, 64, 10000.0, ls)
    c2, s2 = R.tables(lat, lon, 64, 10000.0, ls)
    assert c1.shape == (2, 1, 16, 24, 32) and c1.dtype == torch.float32
    assert (c1.double() - c2).abs().max() < 1e-6 and (s1.double() - s2).abs().max() < 1e-6
    # neighbouring tokens are ~1 length-scale apart (equirectangular offsets distort a few %)
    x, y = R.stereographic(lat, lon, *R.spherical_centroid(lat, lon))
    dx = (x[:, :, 1:] - x[:, :, :-1]) / ls
    assert torch.allclose(dx, torch.ones_like(dx), atol=3e-2)


def test_level_index_convention_closed_forms():
    """configs[1]'s level index in z: pairs x | y | level = 12 | 12 | 8 for D = 64.
    Closed forms: the level pair j at level z has angle z * base^(-j/8) (pair 24:
    exactly z radians); level 0 is the identity on the level pairs; the x | y groups
    are the 2D table of a 48-wide head (12 frequencies per axis); the x | y part does
    not depend on z."""
    g = torch.Generator().manual_seed(0)
    lat, lon = P.synthetic_tile_latlon(2, 8, 8, g)
    ls = R.default_rope_length_scale(1)
    Z, base = 5, 10000.0
    c, s = R.tables(lat, lon, 64, base, ls, levels=Z, level_pairs=8)
    assert c.shape == (2, Z, 8, 8, 32)
    ang = torch.atan2(s, c)
    for z in range(Z):
        for j in range(8):
            want = z * base ** (-j / 8)
            got = ang[:, z, :, :, 24 + j]
            d = torch.remainder(got - want + math.pi, 2 * math.pi) - math.pi  # angle mod 2 pi
            assert d.abs().max() < 1e-12, (z, j)
    assert torch.equal(c[:, 0, ..., 24:], torch.ones_like(c[:, 0, ..., 24:]))
    assert torch.equal(s[:, 0, ..., 24:], torch.zeros_like(s[:, 0, ..., 24:]))
    c2, s2 = R.tables(lat, lon, 48, base, ls)  # 2D table of 24 pairs: 12 per axis
    for z in range(Z):
        assert torch.allclose(c[:, z, ..., :24], c2[:, 0], atol=1e-15)
        assert torch.allclose(s[:, z, ..., :24], s2[:, 0], atol=1e-15)


def test_level_rotation_is_relative_in_z():
    """<R(z1) q, R(z2) k> over the level pairs depends only on z1 - z2."""
    g = torch.Generator().manual_seed(1)
    lat, lon = P.synthetic_tile_latlon(1, 2, 2, g)
    c, s = R.tables(lat, lon, 64, 10000.0, R.default_rope_length_scale(1), levels=8, level_pairs=8)
    q = torch.zeros(1, 8, 2, 2, 1, 64, dtype=torch.float64)
    k = torch.zeros_like(q)
    qv = torch.randn(64, generator=g, dtype=torch.float64)
    kv = torch.randn(64, generator=g, dtype=torch.float64)
    lvl = [d for p in range(24, 32) for d in (p, p + 32)]  # half layout: pair p = (p, p + 32)
    q[..., lvl] = qv[lvl]
    k[..., lvl] = kv[lvl]
    rq, rk = R.apply_rope(q, c, s), R.apply_rope(k, c, s)
    dot = lambda z1, z2: (rq[0, z1, 0, 0, 0] * rk[0, z2, 0, 0, 0]).sum()  # noqa: E731
    assert abs(dot(5, 2) - dot(4, 1)) < 1e-12 and abs(dot(3, 3) - dot(0, 0)) < 1e-12
    assert abs(dot(5, 2) - dot(2, 5)) > 1e-6  # and it is not symmetric in the offset


def test_product_level_tables_match_oracle():
    g = torch.Generator().manual_seed(2)
    lat, lon = P.synthetic_tile_latlon(2, 16, 16, g)
    ls = P.default_rope_length_scale(1)
    cp, sp = P.stereographic_rope_tables(lat, lon, 64, 10000.0, ls, levels=8, level_pairs=8)
    co, so = R.tables(lat, lon, 64, 10000.0, ls, levels=8, level_pairs=8)
    assert cp.shape == (2, 8, 16, 16, 32) and cp.dtype == torch.float32
    assert (cp.double() - co).abs().max() < 1e-6 and (sp.double() - so).abs().max() < 1e-6
    import pytest

    with pytest.raises(ValueError):
        P.stereographic_rope_tables(lat, lon, 64, 10000.0, ls, levels=8, level_pairs=7)
