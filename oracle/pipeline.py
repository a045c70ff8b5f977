"""CPU restatement of the rollout step around the network — test infrastructure.

Follows the pipeline of the reference:
  * input normalisation ``RunningNorm2d.forward`` (screamcast/normalization.py:109-123):
    ``(x - mean) / (sqrt(var) + eps)`` in fp32, non-finite inputs set to 0;
  * the patch embedding ``Conv3d(in, embed, kernel=patch, stride=patch)`` of
    ``PatchEmbed3D`` (the ``proj`` conv that ``DealiasedPatchEmbed3D``,
    screamcast/dealias.py:88-97, keeps state-dict compatible with), written as a
    patchify in the conv weight's (c, dz, dy, dx) order and a matmul;
  * ``DealiasedPatchEmbed3D.forward`` (screamcast/dealias.py:111-143) as the
    reference writes it: stride-1 conv, replicate pad, depthwise low-pass with
    stride = patch;
  * target denormalisation ``RunningNorm2d.denormalize`` (normalization.py:102-107):
    ``x * (sqrt(var) + eps) + mean`` in fp32, cast back to the prediction's dtype;
  * the prognostic update of ``MixedPredictionAsymmetric.step``
    (screamcast/model_pipelines.py:631-662, ``_process_mixed_statediff_predictions``
    :664-676): difference-predicted variables add the current state, state-predicted
    ones replace it; the qv floor ``clamp(min=1e-15)`` of :652-658.

Used only by tests and ``__graft_entry__.smoke()`` as the checker.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
import torch.nn.functional as F
from torch import Tensor


def norm_std(var: Tensor, eps: float) -> Tensor:
    """``sqrt(var) + eps`` in fp32, the divisor of normalization.py:117 and :106."""
    return var.float().sqrt() + eps


def normalize(x: Tensor, mean: Optional[Tensor], std: Optional[Tensor]) -> Tensor:
    """RunningNorm2d.forward on ``[B, C, ...]`` (normalization.py:109-123), fp32 out."""
    xf = x.float()
    if mean is None:
        y = xf.clone()
    else:
        shape = (1, -1) + (1,) * (x.dim() - 2)
        y = (xf - mean.float().view(shape)) / std.float().view(shape)
    return torch.where(torch.isfinite(xf), y, torch.zeros_like(y))


def patchify(x: Tensor, patch: Sequence[int]) -> Tensor:
    """``[B, C, Z, Y, X]`` -> ``[B, Z/pz, Y/py, X/px, C*pz*py*px]``, element order (c, dz, dy, dx)."""
    pz, py, px = patch
    B, C, Z, Y, X = x.shape
    t = x.reshape(B, C, Z // pz, pz, Y // py, py, X // px, px).permute(0, 2, 4, 6, 1, 3, 5, 7)
    return t.reshape(B, Z // pz, Y // py, X // px, C * pz * py * px)


def unpatchify(t: Tensor, channels: int, patch: Sequence[int], order: int) -> Tensor:
    """Inverse of ``patchify`` (order 0) or of the patch-major (dz, dy, dx, c) layout (order 1)."""
    pz, py, px = patch
    B, Tz, Ty, Tx, _ = t.shape
    if order == 0:
        u = t.reshape(B, Tz, Ty, Tx, channels, pz, py, px).permute(0, 4, 1, 5, 2, 6, 3, 7)
    else:
        u = t.reshape(B, Tz, Ty, Tx, pz, py, px, channels).permute(0, 7, 1, 4, 2, 5, 3, 6)
    return u.reshape(B, channels, Tz * pz, Ty * py, Tx * px)


def state_patchify(state: Tensor, mean: Optional[Tensor], std: Optional[Tensor], patch: Sequence[int]) -> Tensor:
    """Normalise then patchify, rounded to bf16 (the dtype the patch embedding runs in)."""
    return patchify(normalize(state, mean, std), patch).to(torch.bfloat16)


def patch_embed(state: Tensor, weight: Tensor, bias: Optional[Tensor], patch: Sequence[int]) -> Tensor:
    """Conv3d(kernel = stride = patch) as patchify + matmul, channels-last out (fp32)."""
    t = patchify(state.float(), patch)
    y = t @ weight.float().reshape(weight.shape[0], -1).T
    return y + bias.float() if bias is not None else y


def dealiased_patch_embed(
    x: Tensor, weight: Tensor, bias: Optional[Tensor], patch: Sequence[int], resample_filter: Sequence[float]
) -> Tensor:
    """``DealiasedPatchEmbed3D.forward`` (screamcast/dealias.py:111-143) in float64,
    channels-last out ``[B, Z/pz, Y/py, X/px, E]``: the stride-1 valid conv
    (:113), the per-axis filter (identity on axes with patch 1, :101-108)
    normalised by the product of the axis sums (:109), the replicate pad of
    ``(k-1)//2`` below and the rest above (:120-133), and the depthwise conv
    with stride = patch (:135-142)."""
    pz, py, px = patch
    E = weight.shape[0]
    s1 = F.conv3d(x.double(), weight.double(), None if bias is None else bias.double(), stride=1, padding=0)
    fa = torch.as_tensor(resample_filter, dtype=torch.float64)
    one = torch.ones(1, dtype=torch.float64)
    fd, fh, fw = (one if p == 1 else fa for p in (pz, py, px))
    f3d = fd[:, None, None] * fh[None, :, None] * fw[None, None, :]
    f3d = (f3d / (fd.sum() * fh.sum() * fw.sum()))[None, None]
    kd, kh, kw = f3d.shape[2:]
    pads = []
    for k in (kw, kh, kd):  # F.pad order: last axis first
        pads += [(k - 1) // 2, (k - 1) - (k - 1) // 2]
    if kd > 1 or kh > 1 or kw > 1:
        s1 = F.pad(s1, pads, mode="replicate")
    y = F.conv3d(s1, f3d.repeat(E, 1, 1, 1, 1), groups=E, stride=(pz, py, px), padding=0)
    return y.permute(0, 2, 3, 4, 1)


def state_update(
    pred: Tensor,
    state: Optional[Tensor],
    mean: Optional[Tensor],
    std: Optional[Tensor],
    src_channel: Optional[Sequence[int]],
    clamp_min: Optional[Tensor],
    grid: Sequence[int],
    patch: Sequence[int],
    order: int,
) -> Tensor:
    """Next fp32 state ``[B, C, Z, Y, X]`` from bf16 prediction tokens (model_pipelines.py:631-676)."""
    P = patch[0] * patch[1] * patch[2]
    C = pred.shape[-1] // P
    u = unpatchify(pred, C, patch, order)  # bf16 [B, C, Z, Y, X]
    d = u.float()
    if mean is not None:
        shape = (1, C, 1, 1, 1)
        d = d * std.float().view(shape) + mean.float().view(shape)
    d = d.to(pred.dtype).float()  # denormalize returns the prediction's dtype
    src = list(range(C)) if src_channel is None else [int(s) for s in src_channel]
    parts = []
    for c in range(C):
        s = src[c]
        part = d[:, c]
        if state is not None and 0 <= s < state.shape[1]:
            part = part + state[:, s].float()
        parts.append(part)
    out = torch.stack(parts, dim=1)
    if clamp_min is not None:
        for c in range(C):
            lo = float(clamp_min[c])
            if lo == lo:  # not NaN
                out[:, c] = out[:, c].clamp(min=lo)
    return out
