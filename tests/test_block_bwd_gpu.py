"""Backward of the block's remaining ops (LayerNorm, RoPE pack with and
without the qk RMSNorm) and of a whole StrataBlock (plain, gated, and gated
with affine qk-norm) on the GPU against torch autograd of the CPU oracle
(relative L2 <= 1e-2 on the same bf16 inputs and weights; 2e-2 for the block)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import block as OB
from oracle import rope as R
from strata_amd import _lib, ops
from strata_amd import rope as P
from strata_amd.modules import StrataBlock, init_xavier_

from .conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("C", [64, 768, 1024, 2048, 3840, 4096])
def test_layer_norm_backward(gpu, C):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(3, 37, C, generator=g) * 2 + 0.5).bfloat16()
    dy = torch.randn(3, 37, C, generator=g).bfloat16()
    xg = x.to(gpu).requires_grad_(True)
    ops.layer_norm(xg, 1e-6).backward(dy.to(gpu))
    xr = x.float().requires_grad_(True)
    F.layer_norm(xr, (C,), eps=1e-6).backward(dy.float())
    assert rel_l2(xg.grad.float().cpu(), xr.grad) <= 1e-2


@pytest.mark.parametrize("layout", [_lib.ROPE_HALF, _lib.ROPE_INTERLEAVED])
@pytest.mark.parametrize("zt", [1, 3])
def test_rope_pack_backward_is_the_inverse_rotation(gpu, layout, zt):
    B, Z, Y, X, H, D = 2, 3, 4, 5, 2, 64
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(B, Z, Y, X, 3 * H * D, generator=g).bfloat16().to(gpu).requires_grad_(True)
    ang = torch.rand(B, zt, Y, X, D // 2, generator=g) * 6.3
    cos, sin = torch.cos(ang).to(gpu), torch.sin(ang).to(gpu)
    grads = [torch.randn(B, Z, Y, X, H, D, generator=g).bfloat16().to(gpu) for _ in range(3)]
    q, k, v = ops.rope_qkv_pack(qkv, cos, sin, H, layout)
    torch.autograd.backward((q, k, v), grads)
    # reference: autograd of the same rotation written in fp32 torch
    qr = qkv.detach().float().cpu().requires_grad_(True)
    c, s = cos.cpu().expand(B, Z, Y, X, D // 2), sin.cpu().expand(B, Z, Y, X, D // 2)
    parts = qr.view(B, Z, Y, X, 3, H, D)
    outs = []
    for t in range(2):
        u = parts[..., t, :, :]
        if layout == _lib.ROPE_HALF:
            a, b = u[..., : D // 2], u[..., D // 2 :]
            cc, ss = c.unsqueeze(-2), s.unsqueeze(-2)
            outs.append(torch.cat([a * cc - b * ss, a * ss + b * cc], dim=-1))
        else:
            a, b = u[..., 0::2], u[..., 1::2]
            cc, ss = c.unsqueeze(-2), s.unsqueeze(-2)
            outs.append(torch.stack([a * cc - b * ss, a * ss + b * cc], dim=-1).flatten(-2))
    outs.append(parts[..., 2, :, :])
    torch.autograd.backward(outs, [gr.float().cpu() for gr in grads])
    assert rel_l2(qkv.grad.float().cpu(), qr.grad) <= 1e-2
    assert rel_l2(q.detach().float().cpu(), outs[0].detach()) <= 1e-2


def _rope_norm_reference(qkv, cos, sin, H, layout, eps, qw, kw):
    """q, k, v of the pack with qk RMSNorm, in torch autograd (dtype of qkv)."""
    B, Z, Y, X, _ = qkv.shape
    D = qkv.shape[-1] // (3 * H)
    t = qkv.view(B, Z, Y, X, 3, H, D)
    name = "half" if layout == _lib.ROPE_HALF else "interleaved"
    q = R.apply_rope(OB.rms_norm(t[..., 0, :, :], eps, qw), cos, sin, name)
    k = R.apply_rope(OB.rms_norm(t[..., 1, :, :], eps, kw), cos, sin, name)
    return q, k, t[..., 2, :, :]


@pytest.mark.parametrize("layout,D", [(_lib.ROPE_HALF, 64), (_lib.ROPE_HALF, 128), (_lib.ROPE_INTERLEAVED, 64),
                                      (_lib.ROPE_INTERLEAVED, 32)], ids=str)
@pytest.mark.parametrize("affine", [False, True])
def test_rope_pack_qk_norm_backward_vs_oracle(gpu, layout, D, affine):
    """RMSNorm backward fused with the inverse rotation: d(qkv) and the norm
    weights' gradients against float64 autograd of the oracle's RMSNorm + RoPE
    on the same bf16 inputs."""
    B, Z, Y, X, H = 2, 3, 5, 7, 3
    g = torch.Generator().manual_seed(5 + D + layout + 2 * affine)
    qkv = (torch.randn(B, Z, Y, X, 3 * H * D, generator=g) * 3).bfloat16()
    ang = torch.rand(B, 1, Y, X, D // 2, generator=g, dtype=torch.float64) * 20 - 10
    cos, sin = torch.cos(ang), torch.sin(ang)
    ws = [(1 + 0.3 * torch.randn(D, generator=g)).bfloat16() if affine else None for _ in range(2)]
    grads = [torch.randn(B, Z, Y, X, H, D, generator=g).bfloat16() for _ in range(3)]
    eps = 1e-6
    xg = qkv.to(gpu).requires_grad_(True)
    wg = [w.to(gpu).requires_grad_(True) if w is not None else None for w in ws]
    outs = ops.rope_qkv_pack(xg, cos.float().to(gpu), sin.float().to(gpu), H, layout, True, eps, *wg)
    torch.autograd.backward(outs, [gr.to(gpu) for gr in grads])
    xr = qkv.double().requires_grad_(True)
    wr = [w.double().requires_grad_(True) if w is not None else None for w in ws]
    ref = _rope_norm_reference(xr, cos, sin, H, layout, eps, *wr)
    torch.autograd.backward(ref, [gr.double() for gr in grads])
    assert rel_l2(xg.grad.float().cpu(), xr.grad.float()) <= 1e-2
    for a, b in zip(wg, wr):
        if a is not None:
            assert a.grad.dtype == torch.bfloat16
            assert rel_l2(a.grad.float().cpu(), b.grad.float()) <= 1e-2


def test_rope_pack_qk_norm_backward_grid_stride(gpu):
    """Enough (token, head) runs that each thread of the bounded grid walks
    several, with the weight gradients summed over all of them (fp32 torch
    autograd on the GPU as the reference)."""
    B, Z, Y, X, H, D = 1, 8, 64, 96, 4, 64
    g = torch.Generator(device=gpu).manual_seed(7)
    qkv = torch.randn(B, Z, Y, X, 3 * H * D, generator=g, device=gpu).bfloat16()
    ang = torch.rand(B, Z, Y, X, D // 2, generator=g, device=gpu) * 6.3
    cos, sin = torch.cos(ang), torch.sin(ang)
    ws = [(1 + 0.3 * torch.randn(D, generator=g, device=gpu)).bfloat16() for _ in range(2)]
    grads = [torch.randn(B, Z, Y, X, H, D, generator=g, device=gpu).bfloat16() for _ in range(3)]
    xg = qkv.clone().requires_grad_(True)
    wg = [w.clone().requires_grad_(True) for w in ws]
    outs = ops.rope_qkv_pack(xg, cos, sin, H, _lib.ROPE_HALF, True, 1e-6, *wg)
    torch.autograd.backward(outs, grads)
    xr = qkv.float().requires_grad_(True)
    wr = [w.float().requires_grad_(True) for w in ws]
    ref = _rope_norm_reference(xr, cos, sin, H, _lib.ROPE_HALF, 1e-6, *wr)
    torch.autograd.backward(ref, [gr.float() for gr in grads])
    assert rel_l2(xg.grad.float(), xr.grad) <= 1e-2
    for a, b in zip(wg, wr):
        assert rel_l2(a.grad.float(), b.grad) <= 1e-2


@pytest.mark.parametrize("variant", ["plain", "gated", "gated_qk_norm"])
def test_strata_block_backward_vs_oracle(gpu, variant):
    C, H, kernel = 128, 2, (3, 5, 5)
    gated, qk_norm = variant != "plain", variant == "gated_qk_norm"
    torch.manual_seed(0)
    blk = StrataBlock(C, H, kernel, gated=gated, qk_norm=qk_norm, qk_norm_affine=qk_norm)
    init_xavier_(blk, torch.Generator().manual_seed(1))
    with torch.no_grad():  # nonzero biases (and non-unit norm weights) so their gradients are checked too
        for m in blk.modules():
            if isinstance(m, torch.nn.Linear):
                m.bias.uniform_(-0.1, 0.1)
            if isinstance(m, torch.nn.RMSNorm):
                m.weight.uniform_(0.7, 1.3)
    params = {k: v.detach().bfloat16().float().requires_grad_(True) for k, v in blk.state_dict().items()}
    blk = blk.to(gpu).bfloat16()
    g = torch.Generator().manual_seed(2)
    B, Z, Y, X = 1, 4, 12, 12
    x = torch.randn(B, Z, Y, X, C, generator=g).bfloat16()
    dy = torch.randn(B, Z, Y, X, C, generator=g).bfloat16()
    lat, lon = P.synthetic_tile_latlon(B, Y, X, g)
    cos, sin = P.stereographic_rope_tables(lat, lon, C // H, 10000.0, P.default_rope_length_scale(1))
    rope = (cos.to(gpu), sin.to(gpu))
    c1, s1 = R.tables(lat, lon, C // H, 10000.0, R.default_rope_length_scale(1))
    xg = x.to(gpu).requires_grad_(True)
    blk(xg, rope).backward(dy.to(gpu))
    xr = x.float().requires_grad_(True)
    OB.block_forward(xr, params, H, kernel, c1.float(), s1.float(), gated=gated, qk_norm=qk_norm).backward(dy.float())
    assert rel_l2(xg.grad.float().cpu(), xr.grad) <= 2e-2
    for name, p in blk.named_parameters():
        assert rel_l2(p.grad.float().cpu(), params[name].grad) <= 2e-2, name
