"""CPU restatement of NATTEN 0.21.5 ``na3d`` (forward, non-causal) — test infrastructure.

The reference reaches NATTEN through the backend string ``na3d_backend``
(screamcast/config.py:99 -> train.py:143 -> screamcast/strata_wrappers.py:292,331,
439,490,582); NATTEN itself (pinned at docker/build_natten.sh:21, Makefile:11)
is not in the reference tree.  Semantics restated from NATTEN's published
definition (Hassani et al., "Neighborhood Attention Transformer", CVPR 2023,
and the NATTEN docs): on each axis of length L with odd kernel k and dilation
d, query i attends the k keys of its residue class g = i mod d nearest to it,
i.e. the window is shifted (never truncated) at the edges.  A kernel equal to
the whole undilated axis (even or odd) is every key of the axis: the depth-wise
attention of alternate blocks uses (Z, 1, 1), full attention over each column.  3D windows are the
Cartesian product of the per-axis windows; layout is heads-last
[B, Z, Y, X, H, D].

Three independent formulations are kept so that each pins the others:
  * ``na3d``            index tables from ``window_start`` (the closed form)
  * ``na3d_bruteforce`` pure-Python loops; the window is found by searching
                        all feasible runs for the one centred nearest the query
  * ``na3d_unfold``     keys gathered by ``torch.Tensor.unfold`` (dilation 1)
"""

from __future__ import annotations

import math
from typing import Sequence

import torch
from torch import Tensor


def window_start(i: int, length: int, kernel: int, dilation: int = 1) -> int:
    """Real coordinate of the first key of query ``i``'s window on one axis."""
    g = i % dilation
    ig = i // dilation
    lg = -(-(length - g) // dilation)  # ceil((length - g) / dilation)
    s = min(max(ig - kernel // 2, 0), lg - kernel)
    return g + dilation * s


def axis_keys(length: int, kernel: int, dilation: int = 1) -> Tensor:
    """LongTensor ``[length, kernel]``: key coordinates of every query on one axis."""
    if kernel < 1 or (kernel % 2 == 0 and not (kernel == length and dilation == 1)):
        raise ValueError(f"kernel size must be odd and positive (or the whole undilated axis), got {kernel}")
    if kernel * dilation > length:
        raise ValueError(f"kernel*dilation ({kernel}*{dilation}) exceeds axis length {length}")
    starts = torch.tensor([window_start(i, length, kernel, dilation) for i in range(length)], dtype=torch.long)
    return starts[:, None] + dilation * torch.arange(kernel, dtype=torch.long)[None, :]


def _triple(v) -> list[int]:
    return [v, v, v] if isinstance(v, int) else [int(x) for x in v]


def na3d(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kernel_size,
    dilation=1,
    scale: float | None = None,
    q_origin: Sequence[int] = (0, 0, 0),
    q_extent: Sequence[int] | None = None,
    compute_dtype: torch.dtype = torch.float32,
    max_chunk_bytes: int = 1 << 28,
    return_lse: bool = False,
):
    """NA3D forward on the CPU; returns ``[B, *q_extent, H, D]`` in ``compute_dtype``.

    Chunked over (batch, head, query z-slice, query y-rows) so the gathered
    window stays below ``max_chunk_bytes``.  ``return_lse``: also return each
    query's log2-sum-exp over its window of the log2-unit scores
    ``scale * log2(e) * q.k``, ``[B, *q_extent, H]`` (the statistic the HIP
    forward emits for the backward; NATTEN keeps the natural-log one).
    """
    B, Z, Y, X, H, D = q.shape
    kz, ky, kx = _triple(kernel_size)
    dz, dy, dx = _triple(dilation)
    oz, oy, ox = (int(a) for a in q_origin)
    ez, ey, ex = (Z - oz, Y - oy, X - ox) if q_extent is None else (int(a) for a in q_extent)
    scale = D**-0.5 if scale is None else scale
    iz = axis_keys(Z, kz, dz)[oz : oz + ez]
    iy = axis_keys(Y, ky, dy)[oy : oy + ey]
    ix = axis_keys(X, kx, dx)[ox : ox + ex]
    W = kz * ky * kx
    qc = q.to(compute_dtype)
    kc = k.to(compute_dtype)
    vc = v.to(compute_dtype)
    out = torch.empty((B, ez, ey, ex, H, D), dtype=compute_dtype)
    lse = torch.empty((B, ez, ey, ex, H), dtype=compute_dtype) if return_lse else None
    elem = torch.finfo(compute_dtype).bits // 8
    rows = max(1, min(ey, max_chunk_bytes // max(1, ex * W * D * elem)))
    for b in range(B):
        for h in range(H):
            kh = kc[b, :, :, :, h, :]
            vh = vc[b, :, :, :, h, :]
            for zi in range(ez):
                kzs = kh[iz[zi]]  # [kz, Y, X, D]
                vzs = vh[iz[zi]]
                for y0 in range(0, ey, rows):
                    yy = iy[y0 : y0 + rows]  # [r, ky]
                    r = yy.shape[0]
                    # [kz, r, ky, X, D] -> [kz, r, ky, ex, kx, D]
                    kw = kzs[:, yy][:, :, :, ix]
                    vw = vzs[:, yy][:, :, :, ix]
                    kw = kw.permute(1, 3, 0, 2, 4, 5).reshape(r, ex, W, D)
                    vw = vw.permute(1, 3, 0, 2, 4, 5).reshape(r, ex, W, D)
                    qq = qc[b, oz + zi, oy + y0 : oy + y0 + r, ox : ox + ex, h, :]  # [r, ex, D]
                    s = torch.einsum("yxd,yxwd->yxw", qq, kw) * scale
                    p = torch.softmax(s, dim=-1)
                    out[b, zi, y0 : y0 + r, :, h, :] = torch.einsum("yxw,yxwd->yxd", p, vw)
                    if return_lse:
                        lse[b, zi, y0 : y0 + r, :, h] = torch.logsumexp(s, dim=-1) / math.log(2.0)
    return (out, lse) if return_lse else out


def _window_by_search(i: int, length: int, kernel: int, dilation: int) -> list[int]:
    """Keys of query ``i``: among all runs of ``kernel`` consecutive members of
    i's residue class, the one whose centre is nearest ``i`` (unique for odd
    kernels)."""
    members = list(range(i % dilation, length, dilation))
    pos = members.index(i)
    best_s, best_d = None, None
    for s in range(0, len(members) - kernel + 1):
        dist = abs(s + kernel // 2 - pos)
        if best_d is None or dist < best_d:
            best_s, best_d = s, dist
    return members[best_s : best_s + kernel]


def na3d_bruteforce(q: Tensor, k: Tensor, v: Tensor, kernel_size, dilation=1, scale: float | None = None) -> Tensor:
    """Pure-Python loops (tiny grids only); float64 result ``[B, Z, Y, X, H, D]``."""
    B, Z, Y, X, H, D = q.shape
    kz, ky, kx = _triple(kernel_size)
    dz, dy, dx = _triple(dilation)
    scale = D**-0.5 if scale is None else scale
    qd, kd, vd = q.double(), k.double(), v.double()
    out = torch.empty((B, Z, Y, X, H, D), dtype=torch.float64)
    for z in range(Z):
        wz = _window_by_search(z, Z, kz, dz)
        for y in range(Y):
            wy = _window_by_search(y, Y, ky, dy)
            for x in range(X):
                wx = _window_by_search(x, X, kx, dx)
                keys = [(a, bb, c) for a in wz for bb in wy for c in wx]
                for b in range(B):
                    for h in range(H):
                        qv = qd[b, z, y, x, h]
                        logits = [float(qv @ kd[b, a, bb, c, h]) * scale for (a, bb, c) in keys]
                        m = max(logits)
                        w = [math.exp(t - m) for t in logits]
                        tot = sum(w)
                        acc = torch.zeros(D, dtype=torch.float64)
                        for wi, (a, bb, c) in zip(w, keys):
                            acc += (wi / tot) * vd[b, a, bb, c, h]
                        out[b, z, y, x, h] = acc
    return out


def na3d_unfold(q: Tensor, k: Tensor, v: Tensor, kernel_size, scale: float | None = None,
                compute_dtype: torch.dtype = torch.float32) -> Tensor:
    """Naive unfold + softmax attention (dilation 1), the configs[0] comparator.

    ``unfold`` enumerates every in-grid window; query i on an axis picks the
    window starting at clamp(i - k//2, 0, L - k)."""
    B, Z, Y, X, H, D = q.shape
    kz, ky, kx = _triple(kernel_size)
    scale = D**-0.5 if scale is None else scale
    kc, vc, qc = k.to(compute_dtype), v.to(compute_dtype), q.to(compute_dtype)
    # [B, Z', Y', X', H, D, kz, ky, kx]
    ku = kc.unfold(1, kz, 1).unfold(2, ky, 1).unfold(3, kx, 1)
    vu = vc.unfold(1, kz, 1).unfold(2, ky, 1).unfold(3, kx, 1)
    sz = torch.clamp(torch.arange(Z) - kz // 2, 0, Z - kz)
    sy = torch.clamp(torch.arange(Y) - ky // 2, 0, Y - ky)
    sx = torch.clamp(torch.arange(X) - kx // 2, 0, X - kx)
    kw = ku[:, sz][:, :, sy][:, :, :, sx]  # [B, Z, Y, X, H, D, kz, ky, kx]
    vw = vu[:, sz][:, :, sy][:, :, :, sx]
    kw = kw.reshape(B, Z, Y, X, H, D, -1)
    vw = vw.reshape(B, Z, Y, X, H, D, -1)
    s = torch.einsum("bzyxhd,bzyxhdw->bzyxhw", qc, kw) * scale
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bzyxhw,bzyxhdw->bzyxhd", p, vw)


def dense_attention(q: Tensor, k: Tensor, v: Tensor, scale: float | None = None) -> Tensor:
    """Global softmax attention over all tokens (kernel == grid special case)."""
    B, Z, Y, X, H, D = q.shape
    scale = D**-0.5 if scale is None else scale
    qf = q.double().reshape(B, -1, H, D).transpose(1, 2)
    kf = k.double().reshape(B, -1, H, D).transpose(1, 2)
    vf = v.double().reshape(B, -1, H, D).transpose(1, 2)
    o = torch.nn.functional.scaled_dot_product_attention(qf, kf, vf, scale=scale)
    return o.transpose(1, 2).reshape(B, Z, Y, X, H, D)


def na3d_flops(batch: int, heads: int, head_dim: int, n_queries: int, kernel_size) -> float:
    """Algorithmic FLOPs 4 * N_q * |W| * D per head (QK^T and PV, 2 flops per MAC)."""
    kz, ky, kx = _triple(kernel_size)
    return 4.0 * batch * heads * n_queries * kz * ky * kx * head_dim


def na3d_backward(q: Tensor, k: Tensor, v: Tensor, dout: Tensor, kernel_size, dilation=1, scale: float | None = None,
                  compute_dtype: torch.dtype = torch.float32) -> tuple[Tensor, Tensor, Tensor]:
    """``(dq, dk, dv)`` of ``na3d`` over the whole grid for the upstream gradient ``dout``:
    torch autograd through the restated forward (the gradient NATTEN's na3d autograd
    function returns, reached in training through train.py:1161)."""
    qc, kc, vc = (t.detach().to(compute_dtype).requires_grad_(True) for t in (q, k, v))
    with torch.enable_grad():
        out = na3d(qc, kc, vc, kernel_size, dilation, scale, compute_dtype=compute_dtype)
        dq, dk, dv = torch.autograd.grad(out, (qc, kc, vc), dout.to(compute_dtype))
    return dq, dk, dv
