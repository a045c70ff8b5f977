"""Backward of the block's remaining ops (LayerNorm, RoPE pack) and of a whole
StrataBlock on the GPU against torch autograd of the fp32 CPU oracle
(relative L2 <= 1e-2 on the same bf16 inputs and weights)."""

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


@pytest.mark.parametrize("C", [64, 768, 1024, 4096])
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


@pytest.mark.parametrize("gated", [False, True])
def test_strata_block_backward_vs_oracle(gpu, gated):
    C, H, kernel = 128, 2, (3, 5, 5)
    torch.manual_seed(0)
    blk = StrataBlock(C, H, kernel, gated=gated)
    init_xavier_(blk, torch.Generator().manual_seed(1))
    with torch.no_grad():  # nonzero biases so their gradients are checked too
        for m in blk.modules():
            if isinstance(m, torch.nn.Linear):
                m.bias.uniform_(-0.1, 0.1)
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
    OB.block_forward(xr, params, H, kernel, c1.float(), s1.float(), gated=gated).backward(dy.float())
    assert rel_l2(xg.grad.float().cpu(), xr.grad) <= 2e-2
    for name, p in blk.named_parameters():
        assert rel_l2(p.grad.float().cpu(), params[name].grad) <= 2e-2, name
