"""CPU restatement of the single-GPU cube-sphere halo fill and crop — test infrastructure.

Follows ``create_padded_faces_batched`` (screamcast/cubesphere_transforms.py:369-445):
each of the 6 faces ``[..., 6, n, n]`` (dims (x, y), x = rows) is placed in the
middle of an ``S = n + 2p`` square; each side's halo is the neighbour's edge
strip (neighbour table :149-196), rotated to a canonical ``(p, n)`` strip
(:229-252) and then to the halo's orientation (:255-273); the four corners are
filled from the two adjacent halo lines, one per side of the corner diagonal
and their mean on it (:276-366, Appendix A2 of arXiv:2311.06253).  ``crop``
is ``TileTopology.crop`` (screamcast/distributed_halo.py:143-147).

Used only by tests and ``__graft_entry__.smoke()`` as the checker.
"""

from __future__ import annotations

import torch
from torch import Tensor

# neighbours[face][side] = (neighbour face, neighbour edge)   (:149-196)
NEIGHBOURS = {
    0: {"top": (5, "bottom"), "right": (1, "left"), "bottom": (4, "top"), "left": (3, "right")},
    1: {"top": (5, "right"), "right": (2, "left"), "bottom": (4, "right"), "left": (0, "right")},
    2: {"top": (5, "top"), "right": (3, "left"), "bottom": (4, "bottom"), "left": (1, "right")},
    3: {"top": (5, "left"), "right": (0, "left"), "bottom": (4, "left"), "left": (2, "right")},
    4: {"top": (0, "bottom"), "right": (1, "bottom"), "bottom": (2, "bottom"), "left": (3, "bottom")},
    5: {"top": (2, "top"), "right": (1, "top"), "bottom": (0, "top"), "left": (3, "top")},
}
# quarter turns (torch.rot90 k on the last two dims): edge -> canonical (:229-252),
# canonical -> halo side (:255-273)
K_TO_CANONICAL = {"bottom": 0, "left": -1, "right": 1, "top": 2}
K_TO_HALO = {"top": 0, "right": 1, "left": -1, "bottom": 2}


def edge_strip(face: Tensor, edge: str, p: int) -> Tensor:
    """The p rows/columns of a face next to one of its edges (:199-226)."""
    if edge == "top":
        return face[..., -p:, :]
    if edge == "bottom":
        return face[..., :p, :]
    if edge == "left":
        return face[..., :, :p]
    if edge == "right":
        return face[..., :, -p:]
    raise ValueError(edge)


def pad_faces(data: Tensor, p: int) -> Tensor:
    """``[..., 6, n, n]`` -> ``[..., 6, n + 2p, n + 2p]``."""
    if p == 0:
        return data
    *lead, f, n, n2 = data.shape
    if f != 6 or n != n2:
        raise ValueError("expected [..., 6, n, n]")
    S = n + 2 * p
    out = torch.full((*lead, 6, S, S), float("nan"), dtype=data.dtype)
    for face in range(6):
        out[..., face, p : p + n, p : p + n] = data[..., face, :, :]
        for side, (nbr, edge) in NEIGHBOURS[face].items():
            strip = edge_strip(data[..., nbr, :, :], edge, p)
            strip = torch.rot90(strip, K_TO_CANONICAL[edge], dims=(-2, -1))
            strip = torch.rot90(strip, K_TO_HALO[side], dims=(-2, -1))
            if side == "top":
                out[..., face, S - p :, p : p + n] = strip
            elif side == "bottom":
                out[..., face, :p, p : p + n] = strip
            elif side == "left":
                out[..., face, p : p + n, :p] = strip
            else:
                out[..., face, p : p + n, S - p :] = strip
    _fill_corners(out, p, n)
    return out


def _fill_corners(out: Tensor, p: int, n: int) -> None:
    """Each p x p corner from the halo column next to it (v, one value per row)
    and the halo row next to it (h, one value per column) (:276-366)."""
    S = n + 2 * p
    i = torch.arange(p).view(p, 1)
    j = torch.arange(p).view(1, p)
    lo, hi = slice(0, p), slice(p + n, S)
    # (rows, cols, v column, h row, diagonal, side of the diagonal that takes v)
    corners = [
        (lo, lo, p, p, "main", "above"),
        (lo, hi, p + n - 1, p, "anti", "above"),
        (hi, lo, p, p + n - 1, "anti", "below"),
        (hi, hi, p + n - 1, p + n - 1, "main", "below"),
    ]
    for rows, cols, vc, hr, diag, vside in corners:
        v = out[..., rows, vc : vc + 1].expand(*out.shape[:-2], p, p)
        h = out[..., hr : hr + 1, cols].expand(*out.shape[:-2], p, p)
        if diag == "main":
            above, below = i < j, i > j
        else:
            above, below = i + j < p - 1, i + j > p - 1
        vmask, hmask = (above, below) if vside == "above" else (below, above)
        out[..., rows, cols] = torch.where(vmask, v, torch.where(hmask, h, (v + h) / 2))


def crop(x: Tensor, h: int) -> Tensor:
    """``TileTopology.crop``: drop h cells on each side of the last two dims."""
    return x if h == 0 else x[..., h:-h, h:-h]
