"""The rollout step around the network: patch embedding and state update.

``PatchEmbed3D`` is the Strata patch embedding, ``Conv3d(in_chans, embed_dim,
kernel_size=patch, stride=patch)`` under the state-dict keys ``proj.weight`` /
``proj.bias`` (the conv that ``DealiasedPatchEmbed3D`` keeps compatible with,
screamcast/dealias.py:88-97), run as the fused normalise + patchify kernel and
a GEMM, with channels-last tokens out.  ``DealiasedPatchEmbed3D`` is the
shift-invariant variant (screamcast/dealias.py:28-143): its low-pass runs as
one filter pass per decimated axis in front of the same patchify + GEMM.

``StepNorms`` carries what ``MixedPredictionAsymmetric.step``
(screamcast/model_pipelines.py:631-662) needs around the network: the input
and target ``RunningNorm2d`` statistics (screamcast/normalization.py:19-123),
which output channel adds which state channel (difference prediction,
``_process_mixed_statediff_predictions`` :664-676; -1 for state prediction),
and the qv floor (:652-658).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import _lib, ops


def running_norm_std(var: Tensor, eps: float) -> Tensor:
    """``sqrt(var) + eps`` in fp32 (normalization.py:106, :117), flattened to ``[C]``."""
    return (var.float().sqrt() + eps).reshape(-1)


@dataclass
class StepNorms:
    """Tables of one pipeline step; ``None`` entries mean identity / all-difference / no floor."""

    in_mean: Optional[Tensor] = None
    in_std: Optional[Tensor] = None
    tgt_mean: Optional[Tensor] = None
    tgt_std: Optional[Tensor] = None
    src_channel: Optional[Tensor] = None  # int [C_out]: state channel added, -1: state prediction
    clamp_min: Optional[Tensor] = None    # float [C_out], NaN: no floor

    @classmethod
    def from_running_norms(
        cls,
        in_mean: Tensor,
        in_var: Tensor,
        tgt_mean: Tensor,
        tgt_var: Tensor,
        eps: float = 1e-9,
        src_channel: Optional[Sequence[int]] = None,
        clamp_min: Optional[Sequence[float]] = None,
    ) -> "StepNorms":
        """From ``RunningNorm2d`` buffers (``mean``/``var`` of shape ``[C, 1, 1]``)."""
        return cls(
            in_mean=in_mean.float().reshape(-1),
            in_std=running_norm_std(in_var, eps),
            tgt_mean=tgt_mean.float().reshape(-1),
            tgt_std=running_norm_std(tgt_var, eps),
            src_channel=None if src_channel is None else torch.tensor(list(src_channel), dtype=torch.int32),
            clamp_min=None if clamp_min is None else torch.tensor(list(clamp_min), dtype=torch.float32),
        )

    def to(self, device) -> "StepNorms":
        return StepNorms(**{k: (v.to(device) if v is not None else None) for k, v in self.__dict__.items()})


class PatchEmbed3D(nn.Module):
    """``Conv3d(in_chans, embed_dim, kernel_size=patch, stride=patch)`` of the state,
    optionally normalised on the fly, to bf16 tokens ``[B, Z/pz, Y/py, X/px, embed_dim]``."""

    def __init__(self, patch_size: Sequence[int] | int, in_chans: int, embed_dim: int):
        super().__init__()
        p = (patch_size,) * 3 if isinstance(patch_size, int) else tuple(int(v) for v in patch_size)
        self.patch_size = p
        self.embed_dim = embed_dim
        self.proj = nn.Conv3d(in_chans, embed_dim, kernel_size=p, stride=p, bias=True)

    def forward(self, state: Tensor, mean: Optional[Tensor] = None, std: Optional[Tensor] = None) -> Tensor:
        tok = ops.state_patchify(state.float(), mean, std, self.patch_size)
        w = self.proj.weight.reshape(self.embed_dim, -1).to(torch.bfloat16)
        K = w.shape[1]
        if K % 8:  # the GEMM takes K in multiples of 8: zero columns change nothing
            pad = 8 - K % 8
            tok = F.pad(tok, (0, pad))
            w = F.pad(w, (0, pad))
        b = self.proj.bias.to(torch.bfloat16) if self.proj.bias is not None else None
        return ops.gemm_bias_act(tok, w.contiguous(), b, None, _lib.ACT_NONE)


class DealiasedPatchEmbed3D(PatchEmbed3D):
    """``DealiasedPatchEmbed3D`` (screamcast/dealias.py:28-143): a stride-1 valid
    ``Conv3d`` (kernel = patch) then, on each axis with patch > 1, the
    normalised ``resample_filter`` low-pass over the replicate-padded result
    (``(k-1)//2`` below, the rest above) decimated by the patch.  The same
    ``proj.weight`` / ``proj.bias`` keys as ``PatchEmbed3D``; the filter is the
    non-persistent buffer ``dealias_filter`` (their outer product, as in
    :101-110).

    Both stages are linear and each axis filter sums to 1, so the embedding is
    the plain patch embedding of the state filtered per decimated axis
    (``strata_hip::dealias_axis``, the input normalisation fused into the first
    pass): the GEMM does the plain embedding's FLOPs instead of a stride-1
    conv's ``pz*py*px`` times as many."""

    def __init__(self, depth: int, height: int, width: int, patch_size: Sequence[int] | int = 16, in_chans: int = 3,
                 embed_dim: int = 768, resample_filter: Sequence[float] = (1, 1)):
        super().__init__(patch_size, in_chans, embed_dim)
        for name, n, p in zip(("Depth", "Height", "Width"), (depth, height, width), self.patch_size):
            if n % p:
                raise ValueError(f"{name} ({n}) must be divisible by the patch size ({p})")
        self.depth, self.height, self.width = depth, height, width
        self.num_patches = (depth // self.patch_size[0]) * (height // self.patch_size[1]) * (width // self.patch_size[2])
        f = torch.as_tensor(resample_filter, dtype=torch.float64).reshape(-1)
        if not 1 <= f.numel() <= 16 or not bool(f.sum() != 0):
            raise ValueError("resample_filter: 1 to 16 taps with a nonzero sum")
        # per axis: the filter divided by its sum on decimated axes, identity elsewhere
        self.axis_taps = [[1.0] if p == 1 else (f / f.sum()).tolist() for p in self.patch_size]
        t = [torch.tensor(a, dtype=torch.float32) for a in self.axis_taps]
        f3d = t[0][:, None, None] * t[1][None, :, None] * t[2][None, None, :]
        self.register_buffer("dealias_filter", f3d[None, None], persistent=False)

    def forward(self, state: Tensor, mean: Optional[Tensor] = None, std: Optional[Tensor] = None) -> Tensor:
        x = state.float()
        for axis, (p, taps) in enumerate(zip(self.patch_size, self.axis_taps)):
            if len(taps) == 1:  # an identity pass (patch 1, or a one-tap filter)
                continue
            x = ops.dealias_axis(x, mean, std, axis, p, taps)
            mean = std = None  # normalised by the first pass
        return super().forward(x, mean, std)
