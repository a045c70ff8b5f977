"""CPU restatement of the Strata transformer block and the configs[4] two-stage
model — test infrastructure.

The block follows the pre-norm structure the reference's manifests and call
sites fix (parameter names/order tests/regression_data/sweep1_...param_order.txt:3-12;
Mlp layers 0/2 screamcast/checkpoint_compat.py:243-249; tanh GELU
screamcast/strata_wrappers.py:76-100; RoPE mode/base :153-162,:333-338):

    x = x + proj(na3d(rope(q), rope(k), v))      q, k, v = split(qkv(LN(x)))
    x = x + fc2(gelu_tanh(fc1(LN(x))))

LayerNorm is non-affine (no LN parameters in the manifests), eps 1e-6.
Optional production variants: gated attention ``a * sigmoid(gate_proj(h))``
(attn.gate_proj in the manifests) and qk RMSNorm over the head dim before
RoPE (screamcast/config.py:91-93; weights ``attn.q_norm.weight`` /
``attn.k_norm.weight`` when elementwise-affine).  Their exact placement inside
physicsnemo's block is not visible here: parity for those two is unpinned
beyond this restatement.
Composition of torch's own F.linear / F.layer_norm / F.gelu with the pinned
``oracle.na3d`` and ``oracle.rope``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from . import na3d as _na3d
from . import rope as _rope


def rms_norm(t: Tensor, eps: float, weight: Tensor | None = None) -> Tensor:
    """RMSNorm over the last dim: t * rsqrt(mean(t^2) + eps) * weight."""
    y = t * torch.rsqrt(t.pow(2).mean(dim=-1, keepdim=True) + eps)
    return y * weight if weight is not None else y


def block_forward(x: Tensor, params: dict, heads: int, kernel_size, cos: Tensor | None, sin: Tensor | None,
                  dilation=1, eps: float = 1e-6, layout: str = "half", gated: bool = False,
                  dtype: torch.dtype = torch.float32, qk_norm: bool = False, qk_norm_eps: float = 1e-6) -> Tensor:
    """x ``[B, Z, Y, X, C]``; params keyed like the block's state dict."""
    p = {k: v.to(dtype) for k, v in params.items()}
    x = x.to(dtype)
    B, Z, Y, X, C = x.shape
    D = C // heads
    h = F.layer_norm(x, (C,), eps=eps)
    qkv = F.linear(h, p["attn.qkv.weight"], p.get("attn.qkv.bias")).view(B, Z, Y, X, 3, heads, D)
    q, k, v = qkv.unbind(dim=4)
    if qk_norm:
        q = rms_norm(q, qk_norm_eps, p.get("attn.q_norm.weight"))
        k = rms_norm(k, qk_norm_eps, p.get("attn.k_norm.weight"))
    if cos is not None:
        q = _rope.apply_rope(q, cos, sin, layout)
        k = _rope.apply_rope(k, cos, sin, layout)
    a = _na3d.na3d(q, k, v, kernel_size, dilation, compute_dtype=dtype).reshape(B, Z, Y, X, C)
    if gated:
        a = a * torch.sigmoid(F.linear(h, p["attn.gate_proj.weight"], p["attn.gate_proj.bias"]))
    x = x + F.linear(a, p["attn.proj.weight"], p["attn.proj.bias"])
    h = F.layer_norm(x, (C,), eps=eps)
    f = F.gelu(F.linear(h, p["mlp.layers.0.weight"], p["mlp.layers.0.bias"]), approximate="tanh")
    return x + F.linear(f, p["mlp.layers.2.weight"], p["mlp.layers.2.bias"])


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


def two_stage_forward(x: Tensor, params: dict, cfg: dict, rope1, rope2, dtype=torch.float32) -> Tensor:
    """configs[4] model: embed -> stage-1 blocks -> 2x merge -> stage-2 blocks -> head.

    x ``[B, Cin, Z, Y, X]``; returns the same shape (the model's tendency)."""
    p = {k: v.to(dtype) for k, v in params.items()}
    h = x.to(dtype).permute(0, 2, 3, 4, 1)
    h = F.linear(h, p["embed.weight"], p["embed.bias"])
    for i in range(cfg["depth1"]):
        bp = {k[len(f"stage1.{i}.") :]: v for k, v in p.items() if k.startswith(f"stage1.{i}.")}
        h = block_forward(h, bp, cfg["heads1"], cfg["kernel1"], *rope1, dtype=dtype)
    h = F.linear(space_to_depth(h), p["merge.weight"], p["merge.bias"])
    for i in range(cfg["depth2"]):
        bp = {k[len(f"stage2.{i}.") :]: v for k, v in p.items() if k.startswith(f"stage2.{i}.")}
        h = block_forward(h, bp, cfg["heads2"], cfg["kernel2"], *rope2, dtype=dtype)
    h = F.layer_norm(h, (h.shape[-1],), eps=1e-6)
    h = F.linear(h, p["head.weight"], p["head.bias"])
    return depth_to_space(h, x.shape[1]).permute(0, 4, 1, 2, 3)
