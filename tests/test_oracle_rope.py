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


# ---- spherical centroid and pooled positions ---------------------------------
# The stereographic RoPE centres each tile at the spherical centroid of its
# positions, not at the (mean lat, mean lon) centre used for wind rotation
# (screamcast/strata_wrappers.py:38-42 against screamcast/tile_geometry.py:141-155).
# The pins below tell the two apart: closed forms where they differ, a tile
# across lon 0 / 2 pi, the maximum of sum(u_i . c) over directions c, and
# equivariance under rotations of the sphere.

def _rad(deg):
    return math.radians(deg)


def test_centroid_closed_form_pole_and_two_equator_points():
    # unit vectors (0,0,1), (1,0,0), (0,1,0): centroid along (1,1,1), i.e. lat asin(1/sqrt 3), lon 45 deg;
    # the mean centre would give lat 30 deg
    lat = torch.tensor([[[_rad(90.0), 0.0, 0.0]]], dtype=torch.float64)
    lon = torch.tensor([[[_rad(45.0), 0.0, _rad(90.0)]]], dtype=torch.float64)
    for f in (R.spherical_centroid, P.spherical_centroid):
        la, lo = f(lat, lon)
        assert abs(la.item() - math.asin(1.0 / math.sqrt(3.0))) < 1e-12
        assert abs(lo.item() - _rad(45.0)) < 1e-12


def test_centroid_of_a_tile_across_lon_zero():
    # points at lon -0.1 (written 2 pi - 0.1) and +0.1 on the equator: centroid (0, 0), not lon pi
    lat = torch.zeros(1, 2, 2, dtype=torch.float64)
    lon = torch.tensor([[[2 * math.pi - 0.1, 0.1], [2 * math.pi - 0.1, 0.1]]], dtype=torch.float64)
    for f in (R.spherical_centroid, P.spherical_centroid):
        la, lo = f(lat, lon)
        assert abs(la.item()) < 1e-15
        assert abs(math.remainder(lo.item(), 2 * math.pi)) < 1e-12
    # and off the equator the centroid lies on the bisecting meridian, at a latitude above the
    # points' own (their great-circle midpoint bulges poleward)
    lat = torch.full((1, 1, 2), 0.8, dtype=torch.float64)
    lon = torch.tensor([[[-0.3, 0.3]]], dtype=torch.float64)
    la, lo = R.spherical_centroid(lat, lon)
    want = math.atan2(math.sin(0.8), math.cos(0.8) * math.cos(0.3))  # direction of u1 + u2
    assert abs(lo.item()) < 1e-15 and abs(la.item() - want) < 1e-12 and la.item() > 0.8


def _dirs(la, lo):
    return torch.stack([torch.cos(la) * torch.cos(lo), torch.cos(la) * torch.sin(lo), torch.sin(la)], -1)


def test_centroid_maximises_summed_cosine():
    """The centroid c maximises sum_i u_i . c over unit vectors c (the mean of the
    cosines of the angular distances); checked against a dense search around it."""
    g = torch.Generator().manual_seed(3)
    lat = (torch.rand(1, 5, 7, generator=g, dtype=torch.float64) - 0.5) * 1.2 + 0.4
    lon = (torch.rand(1, 5, 7, generator=g, dtype=torch.float64) - 0.5) * 1.5 + 5.9
    la, lo = R.spherical_centroid(lat, lon)
    u = _dirs(lat, lon).reshape(-1, 3)
    best = (u @ _dirs(la, lo).reshape(3)).sum()
    d = torch.linspace(-0.05, 0.05, 41, dtype=torch.float64)
    gl, go = torch.meshgrid(la + d, lo + d, indexing="ij")
    cand = (_dirs(gl, go).reshape(-1, 3) @ u.T).sum(1)
    assert cand.max() <= best + 1e-12
    # the mean centre is worse at this spread
    mean_c = _dirs(lat.mean(), torch.atan2(torch.sin(lon).mean(), torch.cos(lon).mean()))
    assert (u @ mean_c).sum() < best - 1e-6


def test_centroid_is_rotation_equivariant():
    g = torch.Generator().manual_seed(4)
    lat = (torch.rand(2, 4, 6, generator=g, dtype=torch.float64) - 0.5) * 2.0
    lon = torch.rand(2, 4, 6, generator=g, dtype=torch.float64) * 2 * math.pi
    a = torch.randn(3, 3, generator=g, dtype=torch.float64)
    rot, _ = torch.linalg.qr(a)
    if torch.det(rot) < 0:
        rot[:, 0] = -rot[:, 0]
    u = _dirs(lat, lon) @ rot.T
    lat2, lon2 = torch.asin(u[..., 2].clamp(-1, 1)), torch.atan2(u[..., 1], u[..., 0])
    la1, lo1 = R.spherical_centroid(lat, lon)
    la2, lo2 = R.spherical_centroid(lat2, lon2)
    assert torch.allclose(_dirs(la1, lo1) @ rot.T, _dirs(la2, lo2), atol=1e-12)


def test_pooled_latlon_is_the_centroid_of_each_block():
    g = torch.Generator().manual_seed(5)
    B, Y, X, f = 2, 6, 8, 2
    lat = (torch.rand(B, Y, X, generator=g, dtype=torch.float64) - 0.5) * 2.5
    lon = torch.rand(B, Y, X, generator=g, dtype=torch.float64) * 2 * math.pi
    pl, po = R.pooled_latlon(lat, lon, f)
    assert pl.shape == (B, Y // f, X // f)
    for b in range(B):
        for i in range(Y // f):
            for j in range(X // f):
                bl = lat[b:b + 1, f * i:f * i + f, f * j:f * j + f]
                bo = lon[b:b + 1, f * i:f * i + f, f * j:f * j + f]
                cl, co = R.spherical_centroid(bl, bo)
                assert abs(pl[b, i, j] - cl[0]) < 1e-12
                assert abs(math.remainder((po[b, i, j] - co[0]).item(), 2 * math.pi)) < 1e-12
    # a field constant over each block returns that block's point
    cl = (torch.rand(B, Y // f, X // f, generator=g, dtype=torch.float64) - 0.5) * 2.5
    co = (torch.rand(B, Y // f, X // f, generator=g, dtype=torch.float64) - 0.5) * 6.0
    up = lambda t: t.repeat_interleave(f, 1).repeat_interleave(f, 2)  # noqa: E731
    pl, po = R.pooled_latlon(up(cl), up(co), f)
    assert torch.allclose(pl, cl, atol=1e-12) and torch.allclose(po, co, atol=1e-12)
    # f = 1 is the identity (lon wrapped to (-pi, pi])
    pl, po = R.pooled_latlon(lat, lon, 1)
    assert torch.allclose(pl, lat, atol=1e-12)
    assert torch.allclose(torch.remainder(po - lon + math.pi, 2 * math.pi) - math.pi, torch.zeros_like(po), atol=1e-12)


def test_model_stage_tables_use_pooled_centroids():
    """The two-stage model's stage-2 tables: tokens at the spherical centroid of their
    2x2 pixels, patch-2 length scale (CPU torch ops, no kernel)."""
    from strata_amd.model import TwoStageStrata

    m = TwoStageStrata(in_channels=8, dim1=64, heads1=1, depth1=1, dim2=64, heads2=1, depth2=1)
    g = torch.Generator().manual_seed(6)
    lat, lon = P.synthetic_tile_latlon(2, 8, 12, g)
    (c1, s1), (c2, s2) = m.rope_tables(lat, lon)
    oc1, os1 = R.tables(lat, lon, 64, 10000.0, R.default_rope_length_scale(1))
    lat2, lon2 = R.pooled_latlon(lat, lon)
    oc2, os2 = R.tables(lat2, lon2, 64, 10000.0, R.default_rope_length_scale(2))
    assert (c1.double() - oc1).abs().max() < 1e-6 and (s1.double() - os1).abs().max() < 1e-6
    assert (c2.double() - oc2).abs().max() < 1e-6 and (s2.double() - os2).abs().max() < 1e-6


def test_planted_centre_mistakes_fail_the_pins():
    """Plausible mistakes planted in a copy of the oracle module each fail a pin above."""
    import types
    from pathlib import Path

    global R
    real = R
    src = Path(real.__file__).read_text()
    mean_centre = (
        "    s = unit_vectors(lat, lon).reshape(B, -1, 3).sum(1)\n"
        "    s = s / s.norm(dim=-1, keepdim=True)\n"
        "    return torch.asin(s[:, 2]), torch.atan2(s[:, 1], s[:, 0])")
    plants = {
        "mean (lat, lon) centre": (
            mean_centre,
            "    return lat.reshape(B, -1).double().mean(1), lon.reshape(B, -1).double().mean(1)"),
        "circular-mean lon, mean lat": (
            mean_centre,
            "    lo = torch.atan2(torch.sin(lon.double()).reshape(B, -1).mean(1), "
            "torch.cos(lon.double()).reshape(B, -1).mean(1))\n"
            "    return lat.reshape(B, -1).double().mean(1), lo"),
        "pooling blocks strided, not contiguous": (
            "view(B, Y // f, f, X // f, f, 3).sum(dim=(2, 4))", "view(B, f, Y // f, f, X // f, 3).sum(dim=(1, 3))"),
        "pooled mean of lat and lon": (
            "    v = unit_vectors(lat, lon).view(B, Y // f, f, X // f, f, 3).sum(dim=(2, 4))\n"
            "    v = v / v.norm(dim=-1, keepdim=True)\n"
            "    return torch.asin(v[..., 2]), torch.atan2(v[..., 1], v[..., 0])",
            "    return (lat.double().view(B, Y // f, f, X // f, f).mean(dim=(2, 4)),\n"
            "            lon.double().view(B, Y // f, f, X // f, f).mean(dim=(2, 4)))"),
    }
    pins = [test_centroid_closed_form_pole_and_two_equator_points, test_centroid_of_a_tile_across_lon_zero,
            test_centroid_maximises_summed_cosine, test_centroid_is_rotation_equivariant,
            test_pooled_latlon_is_the_centroid_of_each_block, test_model_stage_tables_use_pooled_centroids]
    try:
        for name, (a, b) in plants.items():
            assert src.count(a) == 1, name
            mod = types.ModuleType("oracle.rope")
            mod.__package__ = "oracle"
            exec(compile(src.replace(a, b), f"<planted: {name}>", "exec"), mod.__dict__)
            R = mod
            caught = 0
            for pin in pins:
                try:
                    pin()
                except AssertionError:
                    caught += 1
            assert caught > 0, f"planted mistake not caught: {name}"
    finally:
        R = real
