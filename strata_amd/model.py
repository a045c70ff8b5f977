"""Two-stage Strata-style model for the single-GPU rollout.

Structure (reference stack: ``Strata(**kw)`` built at screamcast/strata_wrappers.py:508
and stepped by the pipeline at screamcast/model_pipelines.py:631-662; the
stand-in below keeps the hot path — the blocks — identical to the drop-in
``StrataBlock`` and uses pointwise GEMMs for the stage transitions):

    x [B, Cin, Z, Y, X] -> tokens [B, Z, Y, X, Cin]
    embed   Linear(Cin -> dim1)                      per voxel
    stage 1 depth1 x StrataBlock(dim1, heads1, kernel1)   on (Z, Y, X)
    merge   2x2x2 space-to-depth + Linear(8*dim1 -> dim2) -> (Z/2, Y/2, X/2)
    stage 2 depth2 x StrataBlock(dim2, heads2, kernel2)
    head    LayerNorm + Linear(dim2 -> 8*Cin) + depth-to-space -> [B, Cin, Z, Y, X]

``step`` is one step of the pipeline (MixedPredictionAsymmetric.step,
screamcast/model_pipelines.py:631-662) on an fp32 state: the input
normalisation and the per-voxel patchify run as one HIP kernel
(``state_patchify``), the head's tokens go back through one HIP kernel that
un-patchifies (2x2x2, channels last), denormalises and adds the state
(``state_update``).  With no ``StepNorms`` the tables are identities and the
step is ``x <- x + bf16(model(x))``.  ``rollout`` repeats ``step``.  All
matmuls, LayerNorms, RoPE packs and NA3D calls run in the HIP library; the
2x2x2 merge permute is torch data movement.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn as nn
from torch import Tensor

from . import _lib, ops
from . import rope as R
from .modules import StrataBlock
from .pipeline import StepNorms


def space_to_depth(x: Tensor) -> Tensor:
    """[B, Z, Y, X, C] -> [B, Z/2, Y/2, X/2, 8C], channel order (dz, dy, dx, c)."""
    B, Z, Y, X, C = x.shape
    x = x.view(B, Z // 2, 2, Y // 2, 2, X // 2, 2, C).permute(0, 1, 3, 5, 2, 4, 6, 7)
    return x.reshape(B, Z // 2, Y // 2, X // 2, 8 * C)


def depth_to_space(x: Tensor, c_out: int) -> Tensor:
    """Inverse of space_to_depth: [B, Z, Y, X, 8C] -> [B, 2Z, 2Y, 2X, C]."""
    B, Z, Y, X, _ = x.shape
    x = x.view(B, Z, Y, X, 2, 2, 2, c_out).permute(0, 1, 4, 2, 5, 3, 6, 7)
    return x.reshape(B, 2 * Z, 2 * Y, 2 * X, c_out)


class TwoStageStrata(nn.Module):
    def __init__(
        self,
        in_channels: int = 80,
        dim1: int = 768,
        heads1: int = 12,
        depth1: int = 12,
        kernel1: Sequence[int] = (3, 7, 7),
        dim2: int = 1024,
        heads2: int = 16,
        depth2: int = 12,
        kernel2: Sequence[int] = (3, 9, 9),
        mlp_ratio: float = 4.0,
    ):
        super().__init__()
        self.in_channels = in_channels
        self.embed = nn.Linear(in_channels, dim1)
        self.stage1 = nn.ModuleList([StrataBlock(dim1, heads1, kernel1, mlp_ratio) for _ in range(depth1)])
        self.merge = nn.Linear(8 * dim1, dim2)
        self.stage2 = nn.ModuleList([StrataBlock(dim2, heads2, kernel2, mlp_ratio) for _ in range(depth2)])
        self.head = nn.Linear(dim2, 8 * in_channels)
        self.head_dims = (dim1 // heads1, dim2 // heads2)

    def rope_tables(self, lat: Tensor, lon: Tensor, base: float = 10000.0) -> tuple[tuple[Tensor, Tensor], tuple[Tensor, Tensor]]:
        """Stage tables from per-pixel lat/lon ``[B, Y, X]`` (radians).

        Stage 2 tokens sit at the spherical centroid of their 2x2 pixels and use
        a length scale for horizontal patch size 2.
        """
        t1 = R.stereographic_rope_tables(lat, lon, self.head_dims[0], base, R.default_rope_length_scale(1))
        B, Y, X = lat.shape
        v = torch.stack(
            [torch.cos(lat) * torch.cos(lon), torch.cos(lat) * torch.sin(lon), torch.sin(lat)], dim=-1
        ).view(B, Y // 2, 2, X // 2, 2, 3).sum(dim=(2, 4))
        v = v / v.norm(dim=-1, keepdim=True)
        lat2, lon2 = torch.asin(v[..., 2]), torch.atan2(v[..., 1], v[..., 0])
        t2 = R.stereographic_rope_tables(lat2, lon2, self.head_dims[1], base, R.default_rope_length_scale(2))
        return t1, t2

    def network(self, tokens: Tensor, rope1: tuple[Tensor, Tensor], rope2: tuple[Tensor, Tensor]) -> Tensor:
        """Input tokens ``[B, Z, Y, X, Cin]`` (bf16) -> head tokens ``[B, Z/2, Y/2, X/2, 8*Cin]``,
        each the 2x2x2 cell's outputs in (dz, dy, dx, c) order."""
        h = ops.gemm_bias_act(tokens, self.embed.weight, self.embed.bias, None, _lib.ACT_NONE)
        for blk in self.stage1:
            h = blk(h, rope1)
        h = space_to_depth(h).contiguous()
        h = ops.gemm_bias_act(h, self.merge.weight, self.merge.bias, None, _lib.ACT_NONE)
        for blk in self.stage2:
            h = blk(h, rope2)
        h = ops.layer_norm(h, 1e-6)
        return ops.gemm_bias_act(h, self.head.weight, self.head.bias, None, _lib.ACT_NONE)

    def forward(self, x: Tensor, rope1: tuple[Tensor, Tensor], rope2: tuple[Tensor, Tensor]) -> Tensor:
        """The tendency ``[B, Cin, Z, Y, X]`` of a bf16 input state."""
        h = self.network(x.permute(0, 2, 3, 4, 1).to(torch.bfloat16).contiguous(), rope1, rope2)
        return depth_to_space(h, self.in_channels).permute(0, 4, 1, 2, 3)

    @torch.no_grad()
    def step(self, state: Tensor, rope1, rope2, norms: Optional[StepNorms] = None) -> Tensor:
        """One pipeline step on an fp32 state ``[B, Cin, Z, Y, X]``: next fp32 state."""
        n = norms or StepNorms()
        tok = ops.state_patchify(state.float(), n.in_mean, n.in_std, (1, 1, 1))
        h = self.network(tok, rope1, rope2)
        return ops.state_update(h, state.float(), n.tgt_mean, n.tgt_std, n.src_channel, n.clamp_min,
                                tuple(state.shape[2:]), (2, 2, 2), 1)

    @torch.no_grad()
    def rollout(self, x: Tensor, steps: int, rope1, rope2, norms: Optional[StepNorms] = None) -> Tensor:
        """``steps`` pipeline steps from ``x``; the fp32 state after the last."""
        state = x.float()
        for _ in range(steps):
            state = self.step(state, rope1, rope2, norms)
        return state

    def step_flops(self, batch: int, grid: Sequence[int]) -> float:
        """Block FLOPs of one step (GEMMs 24*M*C^2 per block + NA3D 4*M*|W|*C)."""
        Z, Y, X = grid
        total = 0.0
        for stage, g in ((self.stage1, (Z, Y, X)), (self.stage2, (Z // 2, Y // 2, X // 2))):
            M = batch * g[0] * g[1] * g[2]
            for blk in stage:
                C = blk.attn.dim
                W = math.prod(blk.attn.kernel_size)
                total += 24.0 * M * C * C + 4.0 * M * W * C
        return total
