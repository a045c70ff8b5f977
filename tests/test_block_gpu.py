"""The Strata block through the drop-in modules (all HIP kernels) vs the fp32 CPU oracle."""

import pytest
import torch

from oracle import block as OB
from oracle import rope as R
from strata_amd import rope as P
from strata_amd.modules import StrataBlock, init_xavier_

from .conftest import rel_l2

pytestmark = pytest.mark.gpu


def _block_case(gpu, B, Z, Y, X, C, H, kernel, seed=0, gated=False, qk_norm=False, qk_norm_affine=False,
                base=10000.0, ls_patch=1, depthwise=False):
    g = torch.Generator().manual_seed(1)
    blk = StrataBlock(C, H, kernel, gated=gated, qk_norm=qk_norm, qk_norm_affine=qk_norm_affine, depthwise=depthwise)
    init_xavier_(blk, g)
    if gated:
        with torch.no_grad():
            blk.attn.gate_proj.bias.normal_(generator=g)
    if qk_norm_affine:
        with torch.no_grad():
            blk.attn.q_norm.weight.normal_(1.0, 0.3, generator=g)
            blk.attn.k_norm.weight.normal_(1.0, 0.3, generator=g)
    params = {k: v.detach().clone() for k, v in blk.state_dict().items()}
    blk = blk.to(gpu).bfloat16()
    gx = torch.Generator().manual_seed(seed)
    x = torch.randn(B, Z, Y, X, C, generator=gx).bfloat16()
    ls = P.default_rope_length_scale(ls_patch)
    lat, lon = P.synthetic_tile_latlon(B, Y, X, gx, spacing=ls)
    cos, sin = P.stereographic_rope_tables(lat, lon, C // H, base, ls)
    with torch.no_grad():
        out = blk(x.to(gpu), (cos.to(gpu), sin.to(gpu)))
    # fp32 oracle on the same bf16 inputs and bf16-rounded weights
    params = {k: v.bfloat16().float() for k, v in params.items()}
    c64, s64 = R.tables(lat, lon, C // H, base, ls)
    ref_kernel = (Z, 1, 1) if depthwise else kernel
    ref = OB.block_forward(x.float(), params, H, ref_kernel, c64.float(), s64.float(), gated=gated, qk_norm=qk_norm)
    return out, ref


def test_block_small(gpu):
    out, ref = _block_case(gpu, 1, 4, 16, 16, 256, 4, (3, 7, 7))
    assert rel_l2(out.float(), ref) <= 1e-2


def test_block_gated(gpu):
    out, ref = _block_case(gpu, 1, 4, 12, 20, 256, 4, (3, 5, 5), gated=True)
    assert rel_l2(out.float(), ref) <= 1e-2


def test_block_qk_norm(gpu):
    out, ref = _block_case(gpu, 1, 4, 12, 16, 256, 4, (3, 5, 5), qk_norm=True)
    assert rel_l2(out.float(), ref) <= 1e-2


def test_block_production_variant(gpu):
    """Gated attention + qk RMSNorm with elementwise weights, 1024 wide (16 x 64 heads)."""
    out, ref = _block_case(gpu, 1, 4, 12, 12, 1024, 16, (3, 7, 7), gated=True, qk_norm=True, qk_norm_affine=True)
    assert rel_l2(out.float(), ref) <= 1e-2


def test_block_production_window(gpu):
    """The production attention on a reduced grid: window (3,3,3), gated, qk RMSNorm without
    weights, RoPE base 100 at the patch-4 length scale, 1024 wide (16 x 64 heads)."""
    out, ref = _block_case(gpu, 1, 6, 24, 24, 1024, 16, (3, 3, 3), gated=True, qk_norm=True, base=100.0, ls_patch=4)
    assert rel_l2(out.float(), ref) <= 1e-2


@pytest.mark.parametrize("Z", [6, 7])
def test_block_depthwise(gpu, Z):
    """Depth-wise block (every token attends its whole z column: window (Z, 1, 1), even and
    odd Z) with the production flags: gated, qk RMSNorm, RoPE base 100, 1024 wide."""
    out, ref = _block_case(gpu, 1, Z, 12, 12, 1024, 16, (3, 3, 3), gated=True, qk_norm=True, base=100.0, ls_patch=4,
                           depthwise=True)
    assert rel_l2(out.float(), ref) <= 1e-2


def test_block_cfg3_width(gpu):
    """configs[3] block width (1024, 16 x 64, W=(3,7,7)) on a reduced grid the
    CPU oracle finishes in seconds."""
    out, ref = _block_case(gpu, 1, 4, 16, 16, 1024, 16, (3, 7, 7))
    assert rel_l2(out.float(), ref) <= 1e-2


def test_block_residual_identity_with_zero_output_weights(gpu):
    blk = StrataBlock(256, 4, (3, 5, 5)).to(gpu).bfloat16()
    with torch.no_grad():
        for lin in (blk.attn.proj, blk.mlp.layers[2]):
            lin.weight.zero_()
            lin.bias.zero_()
    x = torch.randn(1, 3, 8, 8, 256, device=gpu).bfloat16()
    with torch.no_grad():
        assert torch.equal(blk(x), x)
