"""Pins for the block oracle's qk RMSNorm (CPU, float64)."""

import torch
import torch.nn.functional as F

from oracle import block as OB


def test_rms_norm_matches_torch_and_closed_forms():
    g = torch.Generator().manual_seed(0)
    t = torch.randn(5, 7, 64, generator=g, dtype=torch.float64) * 3
    w = 1 + 0.2 * torch.randn(64, generator=g, dtype=torch.float64)
    # torch's own routine
    assert torch.allclose(OB.rms_norm(t, 1e-6, w), F.rms_norm(t, (64,), w, 1e-6), atol=1e-12)
    # unit RMS without weights (eps -> 0), scale invariance, constant vectors -> +-1
    y = OB.rms_norm(t, 0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(5, 7, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(OB.rms_norm(7.5 * t, 0.0), y, atol=1e-12)
    c = torch.full((3, 64), -2.5, dtype=torch.float64)
    assert torch.allclose(OB.rms_norm(c, 0.0), -torch.ones_like(c))


def test_rms_norm_is_the_first_step_of_the_qk_norm_block():
    """With qk_norm the oracle block differs from the plain block: a planted
    no-op normalisation (the flag ignored) would fail here."""
    g = torch.Generator().manual_seed(1)
    C, H = 32, 2
    params = {
        "attn.qkv.weight": torch.randn(3 * C, C, generator=g) * C**-0.5,
        "attn.qkv.bias": torch.zeros(3 * C),
        "attn.proj.weight": torch.randn(C, C, generator=g) * C**-0.5,
        "attn.proj.bias": torch.zeros(C),
        "mlp.layers.0.weight": torch.randn(4 * C, C, generator=g) * C**-0.5,
        "mlp.layers.0.bias": torch.zeros(4 * C),
        "mlp.layers.2.weight": torch.randn(C, 4 * C, generator=g) * (4 * C) ** -0.5,
        "mlp.layers.2.bias": torch.zeros(C),
    }
    x = torch.randn(1, 3, 5, 5, C, generator=g)
    a = OB.block_forward(x, params, H, (3, 3, 3), None, None)
    b = OB.block_forward(x, params, H, (3, 3, 3), None, None, qk_norm=True)
    assert (a - b).abs().max() > 1e-3
