"""The rollout step around the network: patch embedding and state update.

``PatchEmbed3D`` is the Strata patch embedding, ``Conv3d(in_chans, embed_dim,
kernel_size=patch, stride=patch)`` under the state-dict keys ``proj.weight`` /
``proj.bias`` (the conv that ``DealiasedPatchEmbed3D`` keeps compatible with,
screamcast/dealias.py:88-97), run as the fused normalise + patchify kernel and
a GEMM, with channels-last tokens out.

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
