"""The region kernel (na3d_region_kernel; the host takes it for windows kz = 3, ky = 3,
kx <= 3, head_dim 64 — the production window (3,3,3)) through the C ABI against the CPU
oracle, and against the strips / general kernel that take the same windows when the path
is switched off (STRATA_HIP_NA3D_NO_REGIONS=1).

The cases walk the z schedule's edges (z sub-grids of 3, 4, 6, 7, 8, 16 and 24 slices,
query z-boxes that start and end inside the grid, z dilation), the y and x clamping the
kernel handles by masks (grids narrower than a region, ragged regions, y dilation, which
the strips do not take), a window narrower in x than in y, the lse output, the query
rotation inside the kernel, and the exact recompute of tiles whose sums leave the fast
path's range.
"""

import pytest
import torch

from oracle import na3d as O
from strata_amd import ops  # noqa: F401

from .conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def _run(q, k, v, kernel, dilation=(1, 1, 1), origin=(0, 0, 0), extent=None):
    extent = list(q.shape[1:4]) if extent is None else list(extent)
    return torch.ops.strata_hip.na3d_fwd(q, k, v, list(kernel), list(dilation), None, list(origin), extent)


def _rand(shape, seed, device):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(shape, generator=g).bfloat16().to(device) for _ in range(3)]


REGION_CASES = [
    # shape (B, Z, Y, X, H, D), kernel, dilation, origin, extent
    ((1, 8, 24, 40, 2, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),
    ((1, 3, 16, 16, 1, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),      # Lz = 3: every tile starts at 0
    ((1, 4, 20, 18, 2, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),      # Lz = 4: four live tiles twice
    ((2, 6, 17, 23, 1, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),
    ((1, 7, 9, 31, 2, 64), (3, 3, 1), (1, 1, 1), (0, 0, 0), None),       # kx < ky, a grid one region tall
    ((1, 9, 30, 20, 1, 64), (3, 3, 3), (1, 1, 1), (2, 3, 1), (5, 22, 17)),  # query box inside every axis
    ((1, 8, 26, 34, 2, 64), (3, 3, 3), (1, 1, 1), (3, 0, 0), (5, 26, 34)),  # z box to the top end
    ((1, 12, 22, 26, 1, 64), (3, 3, 3), (2, 1, 2), (0, 0, 0), None),     # z and x dilation (sub-grids of 6, 13)
    ((1, 8, 33, 20, 2, 64), (3, 3, 3), (1, 3, 1), (0, 0, 0), None),      # y dilation (not on the strips)
    ((1, 5, 33, 20, 2, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),      # Lz = 5: five overlap, not a region
    ((2, 6, 3, 3, 3, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),        # windows span the y / x grid
    ((1, 16, 8, 16, 1, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),      # one region per z walk
    ((1, 24, 40, 36, 1, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),     # the production depth
]


@pytest.mark.parametrize("case", REGION_CASES, ids=[f"{c[0]}-k{c[1]}-d{c[2]}-box{c[3]}" for c in REGION_CASES])
def test_region_kernel_vs_oracle(gpu, case):
    shape, kernel, dil, origin, extent = case
    extent = shape[1:4] if extent is None else extent
    print(f"region case {shape} k{kernel} d{dil} o{origin} e{extent}", flush=True)
    q, k, v = _rand(shape, 17, gpu)
    out = _run(q, k, v, kernel, dil, origin, extent)
    ref = O.na3d(q.cpu(), k.cpu(), v.cpu(), kernel, dil, q_origin=origin, q_extent=extent)
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= BF16_TOL


@pytest.mark.parametrize("kernel", [(3, 3, 3), (3, 3, 1)])
def test_region_kernel_matches_strip_path(gpu, monkeypatch, kernel):
    """The same launch through the region kernel and, with it switched off, through the
    small-window strips and the general kernel: both within bf16 rounding."""
    g = torch.Generator(device=gpu).manual_seed(5)
    q, k, v = (torch.randn((1, 24, 64, 64, 4, 64), generator=g, device=gpu).bfloat16() for _ in range(3))
    print(f"region vs strips {kernel}", flush=True)
    a = _run(q, k, v, kernel)
    monkeypatch.setenv("STRATA_HIP_NA3D_NO_REGIONS", "1")
    b = _run(q, k, v, kernel)
    assert rel_l2(a.float(), b.float()) <= 5e-3


@pytest.mark.parametrize("shape, kernel, dil", [
    ((1, 8, 24, 40, 2, 64), (3, 3, 3), (1, 1, 1)),
    ((1, 4, 19, 21, 1, 64), (3, 3, 3), (1, 1, 1)),
    ((1, 12, 20, 24, 2, 64), (3, 3, 1), (2, 2, 1)),
])
def test_region_kernel_lse(gpu, shape, kernel, dil):
    """The lse instance: each query's log2-sum-exp against the oracle, and the output
    bit-identical to the inference instance's."""
    q, k, v = _rand(shape, 23, gpu)
    print(f"region lse {shape} k{kernel} d{dil}", flush=True)
    out, lse = torch.ops.strata_hip.na3d_fwd_lse(q, k, v, list(kernel), list(dil), None)
    plain = _run(q, k, v, kernel, dil)
    assert torch.equal(out, plain)
    _, ref = O.na3d(q.cpu(), k.cpu(), v.cpu(), kernel, dil, compute_dtype=torch.float64, return_lse=True)
    assert (lse.double().cpu() - ref).abs().max().item() <= 3e-2


def test_region_kernel_exact_path(gpu):
    """Queries whose best scores lie far above (~160 log2 units) or whose scores all lie far
    below zero leave the fast path's range: their tiles are recomputed exactly; the rest of
    the launch is untouched."""
    B, Z, Y, X, H = 1, 6, 20, 24, 2
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(B, Z, Y, X, H, 64, generator=g) for _ in range(3))
    u = torch.zeros(64)
    u[:32] = 1.0 / 32**0.5
    q[0, 2, 9, 10, 0] = 30.0 * u
    k[0, 3, 10, 11, 0] = 30.0 * u   # one key far above the rest for that query
    q[0, 4, 12, 5, 1] = -30.0 * u
    k[0, 3:6, 11:14, 4:7, 1] = 0.1 * k[0, 3:6, 11:14, 4:7, 1] + 30.0 * u  # every key far below
    q, k, v = (t.bfloat16() for t in (q, k, v))
    out = _run(q.to(gpu), k.to(gpu), v.to(gpu), (3, 3, 3))
    ref = O.na3d(q, k, v, (3, 3, 3))
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= BF16_TOL
    for idx in ((0, 2, 9, 10, 0), (0, 4, 12, 5, 1)):
        assert rel_l2(out[idx].float().cpu(), ref[idx]) <= BF16_TOL, idx


def test_region_kernel_strided_v_and_lse_box(gpu):
    """q, k and v as strided views of one packed qkv buffer (v at three times a packed
    tensor's token stride), a halo-interior query box, lse over the box."""
    from strata_amd import _lib

    B, Z, Y, X, H = 1, 8, 40, 48, 2
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(B, Z, Y, X, 3, H, 64, generator=g).bfloat16()
    q, k, v = (qkv[..., i, :, :] for i in range(3))
    org, ext = (1, 6, 5), (6, 28, 36)
    qg = qkv.to(gpu)
    out = _run(qg[..., 0, :, :], qg[..., 1, :, :], qg[..., 2, :, :], (3, 3, 3), (1, 1, 1), org, ext)
    ref_o, ref_l = O.na3d(q, k, v, (3, 3, 3), q_origin=org, q_extent=ext, compute_dtype=torch.float64,
                          return_lse=True)
    assert rel_l2(out.float(), ref_o) <= BF16_TOL
    lse = torch.empty((B, *ext, H), dtype=torch.float32, device=gpu)
    out2 = torch.empty_like(out)
    views = [qg[..., i, :, :] for i in range(3)]
    a = _lib.Na3dArgs()
    a.q, a.k, a.v, a.out, a.lse = (*(t.data_ptr() for t in views), out2.data_ptr(), lse.data_ptr())
    a.dtype, a.batch, a.heads, a.head_dim, a.scale = _lib.BF16, B, H, 64, 64**-0.5
    a.grid[:], a.q_origin[:], a.q_extent[:] = (Z, Y, X), org, ext
    a.kernel[:], a.dilation[:] = (3, 3, 3), [1, 1, 1]
    a.q_stride[:], a.k_stride[:], a.v_stride[:] = ([views[0].stride(i) for i in range(5)],) * 3
    a.o_stride[:] = [out2.stride(i) for i in range(5)]
    _lib.call("strata_hip_na3d_fwd", a, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
    assert (lse.double().cpu() - ref_l).abs().max().item() <= 3e-2
