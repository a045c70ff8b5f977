"""The rollout step's HIP kernels (state normalise + patchify, state update)
and the patch embeddings (plain and dealiased) against the CPU oracle:
bit-exact for the data movement and the fp32/bf16 element math, through the C
ABI; relative L2 <= 1e-2 for the bf16 embedding GEMMs."""

import ctypes

import pytest
import torch

from oracle import pipeline as O
from strata_amd import _lib, ops
from strata_amd.pipeline import DealiasedPatchEmbed3D, PatchEmbed3D, StepNorms

from .conftest import rel_l2

pytestmark = pytest.mark.gpu

CASES = [  # (B, C, grid, patch)
    (2, 80, (4, 16, 16), (1, 1, 1)),
    (1, 5, (4, 8, 12), (1, 4, 4)),
    (2, 3, (4, 6, 8), (2, 2, 2)),
    (1, 3, (3, 4, 10), (3, 2, 5)),
    (1, 7, (2, 5, 130), (1, 1, 1)),  # odd C*P (2-byte path), x rows over several workgroups
]


def _state(shape, seed, gpu, nonfinite=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * 3.0 + 0.5
    if nonfinite:
        x.view(-1)[:: 97] = float("nan")
        x.view(-1)[5 :: 211] = float("inf")
    return x, x.to(gpu)


@pytest.mark.parametrize("case", CASES, ids=str)
@pytest.mark.parametrize("norm", [False, True])
def test_state_patchify_matches_oracle(gpu, case, norm):
    B, C, grid, patch = case
    x, xg = _state((B, C, *grid), 0, gpu)
    mean = std = None
    if norm:
        g = torch.Generator().manual_seed(1)
        mean = torch.randn(C, generator=g)
        std = O.norm_std(torch.rand(C, generator=g) * 4 + 0.1, 1e-9)
    got = ops.state_patchify(xg, mean.to(gpu) if norm else None, std.to(gpu) if norm else None, patch)
    ref = O.state_patchify(x, mean, std, patch)
    assert got.shape == ref.shape
    assert torch.equal(got.cpu(), ref)


@pytest.mark.parametrize("case", CASES, ids=str)
@pytest.mark.parametrize("order", [0, 1])
def test_state_update_matches_oracle(gpu, case, order):
    B, C, grid, patch = case
    P = patch[0] * patch[1] * patch[2]
    g = torch.Generator().manual_seed(2)
    T = tuple(n // p for n, p in zip(grid, patch))
    pred = (torch.randn(B, *T, C * P, generator=g) * 2).bfloat16()
    state, _ = _state((B, C + 2, *grid), 3, gpu, nonfinite=False)
    mean = torch.randn(C, generator=g)
    std = torch.rand(C, generator=g) * 3 + 0.2
    src = [(c + 2) % (C + 2) if c % 3 else -1 for c in range(C)]
    floor = torch.full((C,), float("nan"))
    floor[C // 2] = 0.25
    got = ops.state_update(pred.to(gpu), state.to(gpu), mean.to(gpu), std.to(gpu),
                           torch.tensor(src, dtype=torch.int32), floor.to(gpu), grid, patch, order)
    ref = O.state_update(pred, state, mean, std, src, floor, grid, patch, order)
    assert torch.equal(got.cpu(), ref)
    # identity tables: next = bf16(pred) + state
    got = ops.state_update(pred.to(gpu), state[:, :C].contiguous().to(gpu), None, None, None, None, grid, patch, order)
    assert torch.equal(got.cpu(), O.state_update(pred, state[:, :C], None, None, None, None, grid, patch, order))


def test_state_update_in_place_through_c_abi(gpu):
    """next may alias the state when every channel adds its own state channel."""
    B, C, grid, patch = 1, 6, (2, 8, 8), (1, 2, 2)
    g = torch.Generator().manual_seed(4)
    pred = (torch.randn(B, 2, 4, 4, C * 4, generator=g)).bfloat16().to(gpu)
    state = torch.randn(B, C, *grid, generator=g).to(gpu)
    ref = O.state_update(pred.cpu(), state.cpu(), None, None, None, None, grid, patch, 0)
    a = _lib.StateUpdateArgs()
    a.pred, a.state, a.next = pred.data_ptr(), state.data_ptr(), state.data_ptr()
    a.batch, a.channels, a.state_channels, a.order = B, C, C, 0
    a.grid[:] = list(grid)
    a.patch[:] = list(patch)
    _lib.call("strata_hip_state_update", a, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(state.cpu(), ref)


@pytest.mark.parametrize("patch,C", [((1, 1, 1), 80), ((1, 4, 4), 5), ((2, 2, 2), 9)])
def test_patch_embed_module_vs_conv3d(gpu, patch, C):
    torch.manual_seed(0)
    emb = PatchEmbed3D(patch, C, 64)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, C, 4, 8, 16, generator=g)
    mean, std = torch.randn(C, generator=g), torch.rand(C, generator=g) + 0.5
    xn = O.normalize(x, mean, std).bfloat16().float()
    w = emb.proj.weight.detach().bfloat16().float()
    b = emb.proj.bias.detach().bfloat16().float()
    ref = torch.nn.functional.conv3d(xn, w, b, stride=patch).permute(0, 2, 3, 4, 1)
    with torch.no_grad():
        got = emb.to(gpu)(x.to(gpu), mean.to(gpu), std.to(gpu))
    assert got.shape == ref.shape
    assert rel_l2(got.float().cpu(), ref) <= 1e-2


def test_step_norms_from_running_norm_buffers(gpu):
    C = 4
    g = torch.Generator().manual_seed(6)
    mean, var = torch.randn(C, 1, 1, generator=g), torch.rand(C, 1, 1, generator=g) + 0.1
    n = StepNorms.from_running_norms(mean, var, mean * 2, var * 3, 1e-9, [0, 1, -1, 3], [float("nan")] * 3 + [0.0])
    assert torch.equal(n.in_std, (var.sqrt() + 1e-9).reshape(-1))
    assert n.src_channel.dtype == torch.int32 and n.src_channel.tolist() == [0, 1, -1, 3]
    n2 = n.to(gpu)
    assert n2.tgt_std.is_cuda and torch.equal(n2.tgt_mean.cpu(), (mean * 2).reshape(-1))


DEALIAS_CASES = [  # (B, C, grid, patch, resample_filter)
    (2, 5, (4, 16, 12), (1, 2, 2), (1, 4, 6, 4, 1)),
    (1, 3, (4, 8, 8), (2, 2, 2), (1, 1)),
    (1, 4, (2, 16, 8), (1, 4, 2), (1, 3, 3, 1)),
    (2, 80, (2, 8, 8), (1, 2, 2), (1, 4, 6, 4, 1)),
]


@pytest.mark.parametrize("case", DEALIAS_CASES, ids=str)
@pytest.mark.parametrize("normed", [False, True])
def test_dealiased_patch_embed_vs_oracle(gpu, case, normed):
    """DealiasedPatchEmbed3D (filter passes + patchify + GEMM) against the
    reference's stride-1 conv -> replicate pad -> strided low-pass
    (screamcast/dealias.py:111-143) in float64, on the normalised state
    rounded as the GPU path rounds its weights (bf16)."""
    B, C, grid, patch, filt = case
    torch.manual_seed(0)
    emb = DealiasedPatchEmbed3D(*grid, patch_size=patch, in_chans=C, embed_dim=48, resample_filter=filt)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(B, C, *grid, generator=g) * 2 + 0.5
    mean, std = (torch.randn(C, generator=g), torch.rand(C, generator=g) + 0.5) if normed else (None, None)
    if normed:
        x[0, 0, 0, 0, 0] = float("nan")  # normalised to 0, as RunningNorm2d does
    w = emb.proj.weight.detach().bfloat16().double()
    b = emb.proj.bias.detach().bfloat16().double()
    ref = O.dealiased_patch_embed(O.normalize(x, mean, std), w, b, patch, filt)
    with torch.no_grad():
        got = emb.to(gpu)(x.to(gpu), None if mean is None else mean.to(gpu), None if std is None else std.to(gpu))
    assert got.shape == ref.shape
    assert torch.isfinite(got.float()).all()
    assert rel_l2(got.float().cpu(), ref.float()) <= 1e-2


def test_dealias_axis_pass_vs_fp64(gpu):
    """One filter pass per axis against the clamped-tap sum in float64."""
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, 3, 6, 10, 12, generator=g)
    taps = [0.0625, 0.25, 0.375, 0.25, 0.0625]
    for axis, p in ((0, 2), (1, 2), (2, 4), (2, 1)):
        got = ops.dealias_axis(x.to(gpu), None, None, axis, p, taps).cpu()
        S = x.shape[2 + axis]
        i = torch.arange(S)
        ref = torch.zeros_like(x, dtype=torch.float64)
        for t, f in enumerate(taps):
            src = (p * (i // p) - 2 + t).clamp(0, S - p) + i % p
            ref += f * x.double().index_select(2 + axis, src)
        assert (got.double() - ref).abs().max() <= 1e-6 * ref.abs().max(), (axis, p)


def test_dealiased_embed_is_state_dict_compatible(gpu):
    """The dealiased embedding loads a PatchEmbed3D checkpoint under strict=True
    (proj.weight / proj.bias; the filter buffer is not persistent), and a
    one-tap filter makes it the plain embedding."""
    plain = PatchEmbed3D((1, 2, 2), 4, 32)
    deal = DealiasedPatchEmbed3D(2, 8, 8, patch_size=(1, 2, 2), in_chans=4, embed_dim=32, resample_filter=(5.0,))
    deal.load_state_dict(plain.state_dict(), strict=True)
    assert "dealias_filter" not in deal.state_dict()
    x = torch.randn(1, 4, 2, 8, 8, generator=torch.Generator().manual_seed(13)).to(gpu)
    with torch.no_grad():
        assert torch.equal(deal.to(gpu)(x), plain.to(gpu)(x))
