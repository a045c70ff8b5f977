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


def _conv_embed64(x, w, b, patch):
    """Plain PatchEmbed3D (Conv3d, kernel = stride = patch) in float64, channels last."""
    return torch.nn.functional.conv3d(x.double(), w.double(), b.double(), stride=patch).permute(0, 2, 3, 4, 1)


def _dealias_brute(x, w, b, patch, filt):
    """DealiasedPatchEmbed3D from its definition, loop by loop (tiny inputs):
    out[j] = sum over taps t of F[t] * (b + sum_u w[u] x[clamp(p*j - lo + t) + u])."""
    B, C, Z, Y, X = x.shape
    E = w.shape[0]
    S, pt = (Z, Y, X), patch
    fa = [float(v) for v in filt]
    taps = [[1.0] if p == 1 else [v / sum(fa) for v in fa] for p in pt]
    T = [s // p for s, p in zip(S, pt)]
    out = torch.zeros(B, T[0], T[1], T[2], E, dtype=torch.float64)
    xd, wd = x.double(), w.double()
    for jz in range(T[0]):
        for jy in range(T[1]):
            for jx in range(T[2]):
                acc = torch.zeros(B, E, dtype=torch.float64)
                for tz, fz in enumerate(taps[0]):
                    sz = min(max(pt[0] * jz - (len(taps[0]) - 1) // 2 + tz, 0), S[0] - pt[0])
                    for ty, fy in enumerate(taps[1]):
                        sy = min(max(pt[1] * jy - (len(taps[1]) - 1) // 2 + ty, 0), S[1] - pt[1])
                        for tx, fx in enumerate(taps[2]):
                            sx = min(max(pt[2] * jx - (len(taps[2]) - 1) // 2 + tx, 0), S[2] - pt[2])
                            patch_x = xd[:, :, sz : sz + pt[0], sy : sy + pt[1], sx : sx + pt[2]].reshape(B, -1)
                            s1 = patch_x @ wd.reshape(E, -1).T + b.double()
                            acc += fz * fy * fx * s1
                out[:, jz, jy, jx] = acc
    return out


def test_dealiased_patch_embed_brute_force_and_special_cases():
    """The oracle of screamcast/dealias.py:111-143 against a loop-by-loop
    restatement of its definition on tiny inputs (odd and even filter lengths,
    identity axes), a one-tap filter reducing it to the plain strided conv,
    and a constant input passing through unchanged by the low-pass."""
    g = torch.Generator().manual_seed(9)
    for patch, filt in [((1, 2, 2), (1, 4, 6, 4, 1)), ((2, 2, 2), (1, 1)), ((2, 4, 2), (1, 3, 3, 1)), ((1, 1, 2), (2, 1))]:
        x = torch.randn(2, 3, 4, 8, 6, generator=g, dtype=torch.float64)
        w = torch.randn(5, 3, *patch, generator=g, dtype=torch.float64)
        b = torch.randn(5, generator=g, dtype=torch.float64)
        got = P.dealiased_patch_embed(x, w, b, patch, filt)
        assert torch.allclose(got, _dealias_brute(x, w, b, patch, filt), atol=1e-10), (patch, filt)
        plain = _conv_embed64(x, w, b, patch)
        one_tap = P.dealiased_patch_embed(x, w, b, patch, (3.0,))
        assert torch.allclose(one_tap, plain, atol=1e-10), patch
        c = torch.full_like(x, 0.7)
        assert torch.allclose(P.dealiased_patch_embed(c, w, b, patch, filt), _conv_embed64(c, w, b, patch), atol=1e-10)
        # a filter with more than one tap does change a non-constant input
        if patch != (1, 1, 1):
            assert not torch.allclose(got, plain, atol=1e-3)


def test_dealias_as_filter_then_patch_embed():
    """The factorisation the HIP path uses: per decimated axis, filter the state
    along the stride-1 grid (clamped taps), then the plain patch embedding."""
    g = torch.Generator().manual_seed(10)
    for patch, filt in [((1, 2, 2), (1, 4, 6, 4, 1)), ((2, 2, 4), (1, 1)), ((2, 1, 2), (1, 2, 1))]:
        x = torch.randn(1, 4, 6, 8, 8, generator=g, dtype=torch.float64)
        w = torch.randn(6, 4, *patch, generator=g, dtype=torch.float64)
        b = torch.randn(6, generator=g, dtype=torch.float64)
        f = torch.tensor(filt, dtype=torch.float64)
        f = f / f.sum()
        y = x
        for axis, p in enumerate(patch):
            if p == 1:
                continue
            S, lo = y.shape[2 + axis], (len(f) - 1) // 2
            i = torch.arange(S)
            acc = torch.zeros_like(y)
            for t in range(len(f)):
                src = (p * (i // p) - lo + t).clamp(0, S - p) + i % p
                acc += f[t] * y.index_select(2 + axis, src)
            y = acc
        assert torch.allclose(_conv_embed64(y, w, b, patch), P.dealiased_patch_embed(x, w, b, patch, filt),
                              atol=1e-10), (patch, filt)
