"""Pins for the cube-sphere halo-fill oracle (CPU).

The reference module imports earth2grid at load, which is not installed, so
its create_padded_faces_batched cannot run here; the restatement is pinned by
the reference test's shapes, constant fields, the seam geometry (every halo
is its neighbour's cells at the same depth, and the two faces of a seam see
each other the same way round), closed-form seams read off the reference's
quarter turns, and the corner rule's sides and diagonal.
"""

import pytest
import torch

from oracle import cube


def _ids(n):
    """data[f, x, y] = a unique integer id of the cell (exact in float64)."""
    return torch.arange(6 * n * n, dtype=torch.float64).view(6, n, n)


def _decode(v, n):
    v = int(v)
    return v // (n * n), (v // n) % n, v % n


def test_reference_test_shapes():
    # tests/test_cubesphere_transforms.py:35-44 at a CPU-sized face
    faces = torch.randn(1, 6, 64, 64)
    assert cube.pad_faces(faces, 16).shape == (1, 6, 96, 96)
    assert cube.pad_faces(faces, 0).shape == (1, 6, 64, 64)
    assert torch.equal(cube.pad_faces(faces, 0), faces)


def test_constant_field_and_crop_round_trip():
    d = torch.full((2, 6, 10, 10), 3.25)
    p = cube.pad_faces(d, 4)
    assert torch.equal(p, torch.full((2, 6, 18, 18), 3.25))
    r = torch.randn(3, 6, 10, 10)
    assert torch.equal(cube.crop(cube.pad_faces(r, 4), 4), r)


def _cell(side, n, d, t):
    """Cell at depth d from a face's side, position t along it."""
    return {"top": (n - 1 - d, t), "bottom": (d, t), "left": (t, d), "right": (t, n - 1 - d)}[side]


def _halo(side, n, p, d, t):
    """Padded position of the halo cell at depth d beyond a side, position t along it."""
    return {"top": (p + n + d, p + t), "bottom": (p - 1 - d, p + t), "left": (p + t, p - 1 - d),
            "right": (p + t, p + n + d)}[side]


@pytest.mark.parametrize("n,p", [(6, 3), (9, 4), (5, 5)])
def test_seams_are_consistent_from_both_sides(n, p):
    padded = cube.pad_faces(_ids(n), p)
    for f in range(6):
        for side, (g, edge) in cube.NEIGHBOURS[f].items():
            assert cube.NEIGHBOURS[g][edge] == (f, side)  # the table is symmetric
            for d in range(p):
                for t in range(n):
                    gg, x, y = _decode(padded[f][_halo(side, n, p, d, t)], n)
                    assert gg == g
                    # the neighbour cell sits at the same depth from the shared edge ...
                    tt = [u for u in range(n) if _cell(edge, n, d, u) == (x, y)]
                    assert len(tt) == 1, (f, side, d, t, x, y)
                    # ... and the neighbour's halo there shows this face's cell back
                    back = _decode(padded[g][_halo(edge, n, p, d, tt[0])], n)
                    assert back == (f, *_cell(side, n, d, t))


def test_closed_form_seams():
    """Two seams read off the reference's quarter turns: face 0's right halo is
    face 1's left columns unrotated (rot -1 then +1), and face 0's top halo is
    face 5's bottom rows unrotated (rot 0, 0)."""
    n, p = 8, 3
    data = torch.randn(6, n, n, dtype=torch.float64)
    padded = cube.pad_faces(data, p)
    assert torch.equal(padded[0, p : p + n, p + n :], data[1, :, :p])
    assert torch.equal(padded[0, p + n :, p : p + n], data[5, :p, :])
    # face 2's top halo is face 5's top rows turned twice (rot 2, then 0)
    assert torch.equal(padded[2, p + n :, p : p + n], torch.rot90(data[5, n - p :, :], 2, (0, 1)))


def test_corner_rule():
    """Bottom-left corner: the halo column beside it (column p) above the main
    diagonal, the halo row beside it (row p) below, their mean on it; the
    top-right corner the other way round."""
    n, p = 7, 4
    data = torch.randn(6, n, n, dtype=torch.float64)
    P = cube.pad_faces(data, p)
    for f in range(6):
        for i in range(p):
            for j in range(p):
                v, h = P[f, i, p], P[f, p, j]
                want = v if i < j else (h if i > j else (v + h) / 2)
                assert P[f, i, j] == want
                r, c = p + n + i, p + n + j
                v, h = P[f, r, p + n - 1], P[f, p + n - 1, c]
                want = v if i > j else (h if i < j else (v + h) / 2)
                assert P[f, r, c] == want
