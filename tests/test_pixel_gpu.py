"""The pixel-stage block's kernels and the block itself through the C ABI vs the CPU oracle
(oracle.block.upsample_dw_gelu / pixel_block_forward, whose parts are pinned against
torch's interpolate, conv3d and layer_norm in tests/test_oracle_block.py).  The block's
composition is this build's convention (physicsnemo's StrataPixel3DBlock is absent)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import block as OB
from strata_amd import ops
from strata_amd.modules import StrataPixelBlock, init_xavier_

from .conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape, factor", [
    ((1, 24, 16, 16, 64), 4),      # the production pixel stage's semantic grid at a 64 x 64 tile (Cs reduced)
    ((2, 3, 5, 7, 32), 4),         # odd coarse sizes: the edge rows and columns repeat
    ((1, 2, 9, 6, 16), 2),
    ((1, 2, 6, 5, 8), 1),          # factor 1: the depth-wise convolution alone
    ((1, 2, 1, 2, 8), 4),          # coarse grids narrower than the 3 x 3 block a thread loads
    ((1, 1, 2, 1, 16), 3),
    ((1, 4, 8, 9, 256), 4),        # 16 channel groups, 16 columns per workgroup (the production layout)
    ((2, 3, 11, 17, 48), 3),       # 6 channel groups: 42 output columns per workgroup, ragged rows
    ((1, 2, 70, 3, 24), 1),        # 3 channel groups: 85 columns per workgroup, 256 % 3 threads idle
])
def test_upsample_dw_gelu_vs_oracle(gpu, shape, factor):
    g = torch.Generator().manual_seed(sum(shape) + factor)
    C = shape[-1]
    cond = torch.randn(shape, generator=g).bfloat16()
    w = (torch.randn(C, 1, 1, 3, 3, generator=g) * 0.5).bfloat16()
    b = torch.randn(C, generator=g).bfloat16()
    print(f"upsample_dw_gelu {shape} f{factor}", flush=True)
    out = ops.upsample_dw_gelu(cond.to(gpu), w.to(gpu), b.to(gpu), factor)
    ref = OB.upsample_dw_gelu(cond, w, b, factor)
    assert out.shape == ref.shape
    assert rel_l2(out.float(), ref) <= 5e-3
    # a strided view of the semantic tokens (every other channel block of a wider tensor) reads the same
    wide = torch.cat([cond, torch.zeros_like(cond)], dim=-1).to(gpu)
    out2 = ops.upsample_dw_gelu(wide[..., :C], w.to(gpu), b.to(gpu), factor)
    assert torch.equal(out2, out)


@pytest.mark.parametrize("M, C", [(1000, 128), (257, 64), (64, 1024), (33, 3072), (5, 8)])
def test_layer_norm_modulate_vs_torch(gpu, M, C):
    g = torch.Generator().manual_seed(M + C)
    x = torch.randn(M, C, generator=g).bfloat16()
    mod = torch.randn(M, 6 * C, generator=g).bfloat16()
    xs, ms = x.to(gpu), mod.to(gpu)
    out = ops.layer_norm_modulate(xs, ms[:, :C], ms[:, C:2 * C], 1e-6)  # shift, scale as column slices
    ref = F.layer_norm(x.double(), (C,), eps=1e-6) * (1 + mod[:, C:2 * C].double()) + mod[:, :C].double()
    assert rel_l2(out.float(), ref) <= 5e-3


def test_gated_add_within_one_rounding(gpu):
    g = torch.Generator().manual_seed(7)
    M, C = 777, 128
    r, y = (torch.randn(M, C, generator=g).bfloat16() for _ in range(2))
    mod = torch.randn(M, 6 * C, generator=g).bfloat16()
    out = ops.gated_add(r.to(gpu), mod.to(gpu)[:, 2 * C:3 * C], y.to(gpu)).cpu()
    ref = r.double() + mod[:, 2 * C:3 * C].double() * y.double()
    err = (out.double() - ref).abs()
    assert (err <= ref.abs() * 2**-8 + 1e-30).all()


def _pixel_case(gpu, B, Z, Y, X, C, H, Cs, factor, kernel, qk_norm=False, seed=0):
    g = torch.Generator().manual_seed(1)
    blk = StrataPixelBlock(C, H, kernel, cond_dim=Cs, factor=factor, qk_norm=qk_norm)
    init_xavier_(blk, g)
    with torch.no_grad():  # non-zero modulations (adaLN-Zero starts the projection at zero)
        blk.adaln_bilinear_dw_proj.weight.normal_(0.0, 0.3 / Cs**0.5, generator=g)
        blk.adaln_bilinear_dw_proj.bias.normal_(0.0, 0.5, generator=g)
        blk.adaln_bilinear_dw_conv.weight.normal_(0.0, 0.3, generator=g)
        blk.adaln_bilinear_dw_conv.bias.normal_(0.0, 0.3, generator=g)
    params = {k: v.detach().clone().bfloat16().float() for k, v in blk.state_dict().items()}
    blk = blk.to(gpu).bfloat16()
    gx = torch.Generator().manual_seed(seed)
    x = torch.randn(B, Z, Y, X, C, generator=gx).bfloat16()
    cond = torch.randn(B, Z, Y // factor, X // factor, Cs, generator=gx).bfloat16()
    with torch.no_grad():
        out = blk(x.to(gpu), cond.to(gpu))
    ref = OB.pixel_block_forward(x.float(), cond.float(), params, H, kernel, factor, qk_norm=qk_norm,
                                 dtype=torch.float32)
    return out, ref


def test_pixel_block_small(gpu):
    out, ref = _pixel_case(gpu, 1, 6, 16, 16, 128, 2, 64, 4, (3, 3, 3))
    assert rel_l2(out.float(), ref) <= 1e-2


def test_pixel_block_production_window_and_qk_norm(gpu):
    """The production pixel stage: 128 wide, 2 heads of 64, window 9 (read as (9, 9, 9) over
    24 levels; kz = 9 runs the general kernel), qk RMSNorm, semantic patch 4."""
    out, ref = _pixel_case(gpu, 1, 24, 20, 24, 128, 2, 64, 4, (9, 9, 9), qk_norm=True)
    assert rel_l2(out.float(), ref) <= 1e-2


def test_pixel_block_refuses_mismatched_cond(gpu):
    blk = StrataPixelBlock(64, 1, (3, 3, 3), cond_dim=16, factor=4).to(gpu).bfloat16()
    x = torch.zeros(1, 3, 8, 8, 64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="does not match"):
        blk(x, torch.zeros(1, 3, 3, 2, 16, dtype=torch.bfloat16, device=gpu))
