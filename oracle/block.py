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


# ---------------------------------------------------------------------------
# Pixel-stage block (this build's convention; physicsnemo's StrataPixel3DBlock is
# absent here: the composition below is unpinned beyond its parts).  Parameters as
# tests/regression_data/pixeldit_...param_order.txt:245-256 (attn.qkv, attn.proj,
# mlp.layers.0 / .2, adaln_bilinear_dw_conv, adaln_bilinear_dw_proj), enabled by
# use_bilinear_dw_gelu_project_adaln_pixel (screamcast/strata_wrappers.py:443,471-477).
# ---------------------------------------------------------------------------
def bilinear_index(n_out: int, n_in: int, factor: int):
    """Per output coordinate: source indices (i0, i1) and the weight of i1 of a linear
    upsampling by ``factor`` with half-pixel centres (torch's align_corners=False):
    src = (o + 0.5) / factor - 0.5 clamped at 0, i0 = floor(src), i1 = min(i0 + 1, n_in - 1)."""
    o = torch.arange(n_out, dtype=torch.float64)
    src = ((o + 0.5) / factor - 0.5).clamp(min=0.0)
    i0 = src.floor().long().clamp(max=n_in - 1)
    i1 = torch.where(i0 < n_in - 1, i0 + 1, i0)
    return i0, i1, src - i0.double()


def upsample_dw_gelu(cond: Tensor, weight: Tensor, bias: Tensor | None, factor: int) -> Tensor:
    """GELU_tanh(dwconv3x3(bilinear_up(cond)) + bias) on ``[B, Z, Yc, Xc, C]`` tokens:
    bilinear upsampling by ``factor`` in y and x, then every channel's 3x3 taps
    (``weight`` ``[C, 1, 1, 3, 3]``) over the upsampled map with zero padding, in float64."""
    c = cond.double()
    B, Z, Yc, Xc, C = c.shape
    Y, X = Yc * factor, Xc * factor
    y0, y1, wy = bilinear_index(Y, Yc, factor)
    x0, x1, wx = bilinear_index(X, Xc, factor)
    rows = c[:, :, y0] * (1 - wy).view(1, 1, Y, 1, 1) + c[:, :, y1] * wy.view(1, 1, Y, 1, 1)
    up = rows[:, :, :, x0] * (1 - wx).view(1, 1, 1, X, 1) + rows[:, :, :, x1] * wx.view(1, 1, 1, X, 1)
    pad = torch.zeros(B, Z, Y + 2, X + 2, C, dtype=torch.float64)
    pad[:, :, 1:-1, 1:-1] = up
    w = weight.double().reshape(C, 3, 3)
    out = torch.zeros(B, Z, Y, X, C, dtype=torch.float64)
    for dy in range(3):
        for dx in range(3):
            out += w[:, dy, dx] * pad[:, :, dy:dy + Y, dx:dx + X]
    if bias is not None:
        out += bias.double()
    return F.gelu(out, approximate="tanh")


def pixel_block_forward(x: Tensor, cond: Tensor, params: dict, heads: int, kernel_size, factor: int,
                        dilation=1, eps: float = 1e-6, qk_norm: bool = False, qk_norm_eps: float = 1e-6,
                        cos: Tensor | None = None, sin: Tensor | None = None, layout: str = "half",
                        dtype: torch.dtype = torch.float64) -> Tensor:
    """Pixel block with a spatially varying adaLN from the semantic tokens ``cond``
    ``[B, Z, Y / factor, X / factor, Cs]``:

        mod = adaln_bilinear_dw_proj(upsample_dw_gelu(cond))  -> shift1, scale1, gate1, shift2, scale2, gate2
        x = x + gate1 * proj(attn(LN(x) * (1 + scale1) + shift1))
        x = x + gate2 * fc2(gelu_tanh(fc1(LN(x) * (1 + scale2) + shift2)))

    (DiT's adaLN-Zero order of the six modulations; attention as ``block_forward``'s)."""
    p = {k: v.to(dtype) for k, v in params.items()}
    x = x.to(dtype)
    B, Z, Y, X, C = x.shape
    D = C // heads
    c = upsample_dw_gelu(cond, p["adaln_bilinear_dw_conv.weight"], p.get("adaln_bilinear_dw_conv.bias"),
                         factor).to(dtype)
    mod = F.linear(c, p["adaln_bilinear_dw_proj.weight"], p["adaln_bilinear_dw_proj.bias"])
    sh1, sc1, g1, sh2, sc2, g2 = mod.split(C, dim=-1)
    h = F.layer_norm(x, (C,), eps=eps) * (1 + sc1) + sh1
    qkv = F.linear(h, p["attn.qkv.weight"], p.get("attn.qkv.bias")).unflatten(-1, (3, heads, D))
    q, k, v = qkv[..., 0, :, :], qkv[..., 1, :, :], qkv[..., 2, :, :]
    if qk_norm:
        q = rms_norm(q, qk_norm_eps, p.get("attn.q_norm.weight"))
        k = rms_norm(k, qk_norm_eps, p.get("attn.k_norm.weight"))
    if cos is not None:
        q = _rope.apply_rope(q, cos, sin, layout)
        k = _rope.apply_rope(k, cos, sin, layout)
    a = _na3d.na3d(q, k, v, kernel_size, dilation, compute_dtype=dtype).reshape(B, Z, Y, X, C)
    x = x + g1 * F.linear(a, p["attn.proj.weight"], p["attn.proj.bias"])
    h = F.layer_norm(x, (C,), eps=eps) * (1 + sc2) + sh2
    f = F.gelu(F.linear(h, p["mlp.layers.0.weight"], p["mlp.layers.0.bias"]), approximate="tanh")
    return x + g2 * F.linear(f, p["mlp.layers.2.weight"], p["mlp.layers.2.bias"])
