"""Pins the CPU oracle of the rollout step (oracle/pipeline.py) against library
routines and closed forms (no GPU)."""

import torch

from oracle import pipeline as P
from strata_amd.model import depth_to_space


def _state(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g) * 3.0 + 1.0


def test_patch_embed_is_conv3d_with_stride_patch():
    """patchify + matmul must equal torch's Conv3d(kernel = stride = patch)."""
    for patch in [(1, 1, 1), (1, 4, 4), (2, 2, 2), (3, 2, 5)]:
        x = _state((2, 5, 6, 8, 10), 0)
        x = x[..., : (6 // patch[0]) * patch[0], : (8 // patch[1]) * patch[1], : (10 // patch[2]) * patch[2]]
        conv = torch.nn.Conv3d(5, 7, kernel_size=patch, stride=patch)
        ref = conv(x).permute(0, 2, 3, 4, 1)
        got = P.patch_embed(x, conv.weight.detach(), conv.bias.detach(), patch)
        assert torch.allclose(got, ref.detach(), atol=1e-5, rtol=1e-5), patch


def test_unpatchify_inverts_patchify_and_matches_depth_to_space():
    x = _state((2, 3, 4, 6, 8), 1)
    for patch in [(1, 1, 1), (2, 2, 2), (1, 3, 2)]:
        assert torch.equal(P.unpatchify(P.patchify(x, patch), 3, patch, 0), x)
    # order 1 is the model head's (dz, dy, dx, c) layout: depth_to_space's inverse map
    t = _state((2, 2, 3, 4, 8 * 3), 2)
    ref = depth_to_space(t, 3).permute(0, 4, 1, 2, 3)
    assert torch.equal(P.unpatchify(t, 3, (2, 2, 2), 1), ref)


def test_normalize_closed_forms():
    C = 4
    mean = torch.tensor([1.0, -2.0, 0.5, 100.0])
    std = P.norm_std(torch.tensor([4.0, 0.25, 1.0, 9.0]), 1e-9)
    z = _state((2, C, 3, 4, 5), 3)
    x = z * std.view(1, C, 1, 1, 1) + mean.view(1, C, 1, 1, 1)
    assert torch.allclose(P.normalize(x, mean, std), z, atol=1e-5)
    # non-finite inputs become exactly 0, finite neighbours are untouched
    x[0, 1, 0, 0, 0] = float("nan")
    x[1, 2, 2, 3, 4] = float("inf")
    x[0, 3, 1, 1, 1] = -float("inf")
    y = P.normalize(x, mean, std)
    assert y[0, 1, 0, 0, 0] == 0 and y[1, 2, 2, 3, 4] == 0 and y[0, 3, 1, 1, 1] == 0
    assert torch.isfinite(y).all()
    assert torch.equal(P.normalize(x, None, None)[torch.isfinite(x)], x[torch.isfinite(x)])


def test_state_update_difference_state_and_floor():
    B, C, grid, patch = 2, 3, (2, 4, 4), (1, 2, 2)
    g = torch.Generator().manual_seed(4)
    pred = torch.randn(B, 2, 2, 2, C * 4, generator=g).bfloat16()
    state = _state((B, 4, *grid), 5)
    mean = torch.tensor([0.5, -1.0, 2.0])
    std = torch.tensor([2.0, 0.5, 3.0])
    src = [2, -1, 0]  # channel 0 adds state channel 2, channel 1 is a state prediction
    floor = torch.tensor([float("nan"), float("nan"), 1.5])
    out = P.state_update(pred, state, mean, std, src, floor, grid, patch, 0)
    d = P.unpatchify(pred, C, patch, 0).float() * std.view(1, C, 1, 1, 1) + mean.view(1, C, 1, 1, 1)
    d = d.bfloat16().float()
    assert torch.equal(out[:, 0], d[:, 0] + state[:, 2])
    assert torch.equal(out[:, 1], d[:, 1])
    assert torch.equal(out[:, 2], torch.clamp(d[:, 2] + state[:, 0], min=1.5))
    assert (out[:, 2] >= 1.5).all()
    # identity tables: next = bf16(pred) + state, the plain x <- x + model(x) update
    out2 = P.state_update(pred, state[:, :C], None, None, None, None, grid, patch, 0)
    assert torch.equal(out2, P.unpatchify(pred, C, patch, 0).float() + state[:, :C])
