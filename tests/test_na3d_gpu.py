"""NA3D on the GPU through the C-ABI library vs the CPU oracle.

Bars: fp32 max-abs <= 1e-5; bf16 relative L2
<= 1e-2 against an fp32 oracle evaluated on the same (bf16-rounded) inputs.
"""

import pytest
import torch

from oracle import na3d as O
from strata_amd import ops  # noqa: F401
from strata_amd.natten import na3d as natten_na3d

from .conftest import rel_l2

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
F32_TOL = 1e-5


def _run(q, k, v, kernel, dilation=(1, 1, 1), origin=(0, 0, 0), extent=None, scale=None):
    extent = list(q.shape[1:4]) if extent is None else list(extent)
    return torch.ops.strata_hip.na3d_fwd(q, k, v, list(kernel), list(dilation), scale, list(origin), extent)


def _rand(shape, seed, dtype, device, scale=None):
    g = torch.Generator().manual_seed(seed)
    t = [torch.randn(shape, generator=g) for _ in range(3)]
    if scale is not None:
        t = [x * scale for x in t]
    return [x.to(dtype).to(device) for x in t]


def test_goldens_fp32(gpu, na3d_golden):
    for name, c in na3d_golden.items():
        q, k, v = (torch.from_numpy(c[t]).to(gpu) for t in "qkv")
        print(f"golden fp32 {name} {c['shape']} kernel {c['kernel']} dil {c['dilation']}", flush=True)
        out = _run(q, k, v, c["kernel"], c["dilation"])
        torch.cuda.synchronize()
        err = (out.cpu() - torch.from_numpy(c["out"])).abs().max().item()
        assert err <= F32_TOL, (name, err)


def test_goldens_bf16(gpu, na3d_golden):
    for name, c in na3d_golden.items():
        q, k, v = (torch.from_numpy(c[t]).bfloat16() for t in "qkv")
        print(f"golden bf16 {name} {c['shape']} kernel {c['kernel']} dil {c['dilation']}", flush=True)
        out = _run(q.to(gpu), k.to(gpu), v.to(gpu), c["kernel"], c["dilation"])
        ref = O.na3d(q, k, v, c["kernel"], c["dilation"], compute_dtype=torch.float64)
        assert rel_l2(out.float(), ref) <= BF16_TOL, name


def test_cfg0_fp32_vs_unfold(gpu):
    """fp32 [1,4,16,16,4,32], W=(3,5,5), seed 0, vs naive unfold."""
    g = torch.Generator().manual_seed(0)
    shape = (1, 4, 16, 16, 4, 32)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    print("cfg0 fp32", flush=True)
    out = _run(q.to(gpu), k.to(gpu), v.to(gpu), (3, 5, 5)).cpu()
    ref = O.na3d_unfold(q, k, v, (3, 5, 5), compute_dtype=torch.float64)
    assert (out.double() - ref).abs().max().item() <= F32_TOL


MFMA_CASES = [
    # shape (B, Z, Y, X, H, D), kernel, dilation, origin, extent
    ((1, 4, 16, 16, 2, 64), (3, 5, 5), (1, 1, 1), None, None),
    ((2, 5, 12, 20, 2, 64), (3, 7, 7), (1, 1, 1), None, None),
    ((1, 4, 20, 24, 2, 64), (3, 13, 13), (1, 1, 1), None, None),
    ((1, 3, 17, 19, 3, 64), (3, 9, 9), (1, 1, 1), None, None),
    ((1, 3, 16, 30, 1, 64), (1, 5, 15), (1, 1, 1), None, None),
    ((1, 2, 8, 16, 1, 64), (1, 1, 1), (1, 1, 1), None, None),
    ((1, 4, 12, 12, 2, 32), (3, 5, 5), (1, 1, 1), None, None),
    ((1, 4, 12, 12, 2, 128), (3, 5, 5), (1, 1, 1), None, None),
    ((1, 6, 14, 18, 2, 64), (3, 3, 5), (2, 2, 3), None, None),
    ((1, 4, 20, 20, 2, 64), (3, 7, 7), (1, 1, 1), (1, 3, 2), (2, 14, 15)),
    ((2, 4, 24, 24, 2, 64), (3, 13, 13), (1, 1, 1), (0, 4, 4), (4, 16, 16)),
    ((1, 3, 7, 9, 2, 64), (3, 7, 9), (1, 1, 1), None, None),  # window spans the y/x grid
    # strip walk (4-column tiles): clamped edges that split the walk into segments,
    # a window as tall as the grid, dilation, ragged y/x, deeper z windows, y chunks
    ((1, 3, 40, 20, 2, 64), (3, 11, 11), (1, 1, 1), None, None),
    ((1, 3, 13, 26, 1, 64), (3, 13, 13), (1, 1, 1), None, None),
    ((1, 4, 30, 27, 2, 64), (3, 11, 13), (1, 2, 2), None, None),
    ((2, 3, 37, 35, 1, 64), (3, 5, 11), (1, 1, 1), None, None),
    ((1, 6, 21, 18, 1, 64), (5, 13, 11), (1, 1, 1), (1, 2, 1), (4, 17, 15)),
    ((1, 3, 64, 16, 1, 64), (3, 1, 13), (1, 1, 1), None, None),
    ((1, 3, 150, 16, 1, 64), (3, 9, 13), (1, 1, 1), None, None),
]


@pytest.mark.parametrize("case", MFMA_CASES, ids=[f"{c[0]}-k{c[1]}-d{c[2]}-box{c[3]}" for c in MFMA_CASES])
def test_mfma_vs_oracle(gpu, case):
    shape, kernel, dil, origin, extent = case
    origin = (0, 0, 0) if origin is None else origin
    extent = shape[1:4] if extent is None else extent
    print(f"mfma case {shape} k{kernel} d{dil} o{origin} e{extent}", flush=True)
    q, k, v = _rand(shape, 11, torch.bfloat16, gpu)
    out = _run(q, k, v, kernel, dil, origin, extent)
    ref = O.na3d(q.cpu(), k.cpu(), v.cpu(), kernel, dil, q_origin=origin, q_extent=extent)
    err = rel_l2(out.float(), ref)
    assert err <= BF16_TOL, err
    assert torch.isfinite(out.float()).all()


def test_strided_views_of_packed_qkv(gpu):
    """q/k/v as views into one [B,Z,Y,X,3,H,D] buffer equal the contiguous result."""
    B, Z, Y, X, H, D = 1, 4, 12, 16, 4, 64
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(B, Z, Y, X, 3, H, D, generator=g).bfloat16().to(gpu)
    q, k, v = qkv[..., 0, :, :], qkv[..., 1, :, :], qkv[..., 2, :, :]
    out_view = _run(q, k, v, (3, 5, 5))
    out_cont = _run(q.contiguous(), k.contiguous(), v.contiguous(), (3, 5, 5))
    assert torch.equal(out_view, out_cont)


def test_natten_shim(gpu):
    q, k, v = _rand((1, 4, 10, 12, 2, 64), 5, torch.bfloat16, gpu)
    out = natten_na3d(q, k, v, kernel_size=(3, 5, 7))
    ref = O.na3d(q.cpu(), k.cpu(), v.cpu(), (3, 5, 7))
    assert rel_l2(out.float(), ref) <= BF16_TOL
    with pytest.raises(NotImplementedError):
        natten_na3d(q, k, v, kernel_size=3, is_causal=True)
    with pytest.raises(ValueError):
        natten_na3d(q, k, v, kernel_size=(5, 3, 3))


@pytest.mark.parametrize("dtype, tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
def test_natten_shim_return_lse(gpu, dtype, tol):
    """``return_lse=True`` (NATTEN's functional API): the output as without it, and the
    natural-log logsumexp of each query's window against the float64 oracle (whose lse is
    in log2 units), with dilation and clamped edges on every axis."""
    import math

    q, k, v = _rand((1, 5, 9, 11, 2, 32 if dtype == torch.float32 else 64), 8, dtype, gpu)
    out, lse = natten_na3d(q, k, v, kernel_size=(3, 5, 5), dilation=(1, 1, 2), return_lse=True)
    assert lse.dtype == torch.float32 and tuple(lse.shape) == tuple(q.shape[:5])
    assert torch.equal(out, natten_na3d(q, k, v, kernel_size=(3, 5, 5), dilation=(1, 1, 2)))
    _, ref = O.na3d(q.cpu(), k.cpu(), v.cpu(), (3, 5, 5), (1, 1, 2), compute_dtype=torch.float64, return_lse=True)
    assert (lse.double().cpu() / math.log(2.0) - ref).abs().max().item() <= tol


def test_cfg1_shape_subboxes(gpu):
    """configs[1] shape [2,8,64,64,8,64], W=(3,7,7): full launch, oracle on boxes
    at the grid corners and the middle (a few seconds of CPU)."""
    shape = (2, 8, 64, 64, 8, 64)
    g = torch.Generator(device=gpu).manual_seed(0)
    q, k, v = (torch.randn(shape, generator=g, device=gpu).bfloat16() for _ in range(3))
    print("cfg1 full launch", flush=True)
    out = _run(q, k, v, (3, 7, 7))
    torch.cuda.synchronize()
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    for b, h in ((0, 0), (1, 7)):
        for org in ((0, 0, 0), (6, 56, 56), (3, 28, 30)):
            ext = (2, 8, 8)
            sl = (slice(b, b + 1), slice(None), slice(None), slice(None), slice(h, h + 1))
            ref = O.na3d(qc[sl], kc[sl], vc[sl], (3, 7, 7), q_origin=org, q_extent=ext)
            got = out[b : b + 1, org[0] : org[0] + 2, org[1] : org[1] + 8, org[2] : org[2] + 8, h : h + 1]
            assert rel_l2(got.float(), ref) <= BF16_TOL, (b, h, org)


def test_cfg2_halo_interior_subboxes(gpu):
    """6 x padded (16,144,144) x 16 heads x 64, W=(3,13,13), per-head
    scale U(0.5,2), outputs for the interior y, x in [8,136)."""
    g = torch.Generator(device=gpu).manual_seed(0)
    s_h = torch.rand(16, generator=g, device=gpu) * 1.5 + 0.5
    shape = (6, 16, 144, 144, 16, 64)
    q, k, v = (
        (torch.randn(shape, generator=g, device=gpu) * s_h.view(1, 1, 1, 1, 16, 1)).bfloat16() for _ in range(3)
    )
    print("cfg2 full launch", flush=True)
    out = _run(q, k, v, (3, 13, 13), origin=(0, 8, 8), extent=(16, 128, 128))
    torch.cuda.synchronize()
    assert out.shape == (6, 16, 128, 128, 16, 64)
    for b, h in ((0, 0), (5, 15), (2, 9)):
        sl = (slice(b, b + 1), slice(None), slice(None), slice(None), slice(h, h + 1))
        qc, kc, vc = q[sl].cpu(), k[sl].cpu(), v[sl].cpu()
        for org in ((0, 8, 8), (14, 120, 120), (7, 60, 70)):
            ext = (2, 16, 16)
            ref = O.na3d(qc, kc, vc, (3, 13, 13), q_origin=org, q_extent=ext)
            o = (org[0], org[1] - 8, org[2] - 8)
            got = out[b : b + 1, o[0] : o[0] + 2, o[1] : o[1] + 16, o[2] : o[2] + 16, h : h + 1]
            assert rel_l2(got.float(), ref) <= BF16_TOL, (b, h, org)


# Regular strips: ky = 13 and every query's y window unclamped (a halo of at
# least 6 rows in each dilation residue class).  These take the fixed-reference
# strip kernel; the cases cover one to eight tiles per strip, a partial last
# tile, ragged x, deeper z windows, dilation, and y chunks of the walk.
REGULAR_CASES = [
    # shape (B, Z, Y, X, H, D), kernel, dilation, origin, extent
    ((1, 3, 16, 28, 2, 64), (3, 13, 13), (1, 1, 1), (0, 6, 6), (3, 4, 16)),
    ((1, 4, 25, 29, 1, 64), (3, 13, 11), (1, 1, 1), (0, 6, 5), (4, 13, 19)),
    ((2, 5, 44, 24, 2, 64), (5, 13, 13), (1, 1, 1), (0, 6, 6), (5, 32, 12)),
    ((1, 4, 40, 40, 1, 64), (3, 13, 13), (1, 2, 2), (0, 12, 12), (4, 16, 16)),
    ((1, 3, 24, 30, 3, 64), (3, 13, 11), (1, 1, 1), (0, 6, 7), (3, 10, 13)),
]


@pytest.mark.parametrize("case", REGULAR_CASES, ids=[f"{c[0]}-k{c[1]}-d{c[2]}-box{c[3]}" for c in REGULAR_CASES])
def test_regular_strip_vs_oracle(gpu, case):
    shape, kernel, dil, origin, extent = case
    print(f"regular strip {shape} k{kernel} d{dil} o{origin} e{extent}", flush=True)
    q, k, v = _rand(shape, 21, torch.bfloat16, gpu)
    out = _run(q, k, v, kernel, dil, origin, extent)
    ref = O.na3d(q.cpu(), k.cpu(), v.cpu(), kernel, dil, q_origin=origin, q_extent=extent)
    assert rel_l2(out.float(), ref) <= BF16_TOL
    assert torch.isfinite(out.float()).all()


def test_regular_strip_chunks(gpu):
    """Enough strips that the y range is walked in four chunks of four tiles;
    the oracle checks boxes on both sides of the chunk seams."""
    shape = (1, 4, 76, 44, 64, 64)
    g = torch.Generator(device=gpu).manual_seed(4)
    q, k, v = (torch.randn(shape, generator=g, device=gpu).bfloat16() for _ in range(3))
    print("regular strip chunks", flush=True)
    out = _run(q, k, v, (3, 13, 13), origin=(0, 6, 6), extent=(4, 64, 32))
    torch.cuda.synchronize()
    for h in (0, 37, 63):
        sl = (slice(0, 1), slice(None), slice(None), slice(None), slice(h, h + 1))
        qc, kc, vc = q[sl].cpu(), k[sl].cpu(), v[sl].cpu()
        for org in ((0, 6, 6), (1, 18, 20), (2, 34, 10), (2, 58, 30)):
            ext = (2, 12, 8)
            ref = O.na3d(qc, kc, vc, (3, 13, 13), q_origin=org, q_extent=ext)
            o = (org[0], org[1] - 6, org[2] - 6)
            got = out[0:1, o[0] : o[0] + 2, o[1] : o[1] + 12, o[2] : o[2] + 8, h : h + 1]
            assert rel_l2(got.float(), ref) <= BF16_TOL, (h, org)


def test_regular_strip_score_far_above_own_key(gpu):
    """A key scoring ~160 (log2 units) overflows the reference-free softmax of
    the fast strip kernel (2^s above fp32 range); that tile must be recomputed
    exactly (its output is then the dominant key's value)."""
    shape = (1, 3, 20, 28, 1, 64)
    q, k, v = (t.float() for t in _rand(shape, 8, torch.bfloat16, "cpu"))
    u = torch.zeros(64)
    u[:32] = 1.0 / 32**0.5
    w = torch.zeros(64)
    w[32:] = 1.0 / 32**0.5
    # query (1, 9, 10): large along u, its own key along w (score 0), one
    # neighbour key (2, 12, 14) large along u: 30 * 30 / 8 nats ~ 162 log2 units.
    q[0, 1, 9, 10, 0] = 30.0 * u
    k[0, 1, 9, 10, 0] = 2.0 * w
    k[0, 2, 12, 14, 0] = 30.0 * u
    q, k, v = (t.bfloat16() for t in (q, k, v))
    out = _run(q.to(gpu), k.to(gpu), v.to(gpu), (3, 13, 13), origin=(0, 6, 6), extent=(3, 8, 16))
    ref = O.na3d(q, k, v, (3, 13, 13), q_origin=(0, 6, 6), q_extent=(3, 8, 16))
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= BF16_TOL
    got = out[0, 1, 3, 4, 0].float().cpu()
    assert rel_l2(got, v[0, 2, 12, 14, 0].float()) <= BF16_TOL


def test_regular_strip_all_scores_far_below_zero(gpu):
    """Every key of one query scores ~-160 (log2 units): 2^s underflows, the row
    sum falls below the fast path's range and the tile is recomputed exactly
    (a near-uniform average over the window, as the fp32 oracle computes)."""
    shape = (1, 3, 20, 28, 1, 64)
    q, k, v = (t.float() for t in _rand(shape, 9, torch.bfloat16, "cpu"))
    u = torch.zeros(64)
    u[:32] = 1.0 / 32**0.5
    k = k * 0.1 + 30.0 * u  # every key along u (plus a little noise)
    q[0, 1, 9, 10, 0] = -30.0 * u
    q, k, v = (t.bfloat16() for t in (q, k, v))
    out = _run(q.to(gpu), k.to(gpu), v.to(gpu), (3, 13, 13), origin=(0, 6, 6), extent=(3, 8, 16))
    ref = O.na3d(q, k, v, (3, 13, 13), q_origin=(0, 6, 6), q_extent=(3, 8, 16))
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= BF16_TOL
    assert rel_l2(out[0, 1, 3, 4, 0].float().cpu(), ref[0, 1, 3, 4, 0]) <= BF16_TOL


def test_regular_strip_large_scores_in_range(gpu):
    """Scores of ~70 log2 units stay inside the fast path's range (2^70 and the
    sums are finite) and must come out exact without the fallback's help."""
    shape = (1, 3, 20, 28, 2, 64)
    q, k, v = (t.float() for t in _rand(shape, 10, torch.bfloat16, "cpu"))
    u = torch.zeros(64)
    u[:32] = 1.0 / 32**0.5
    q[0, 1, 9, 10, 1] = 20.0 * u
    k[0, 2, 12, 14, 1] = 20.0 * u  # 400 / 8 nats ~ 72 log2 units
    k[0, 1, 7, 8, 1] = 19.0 * u    # ~69 log2 units: a second, smaller weight
    q, k, v = (t.bfloat16() for t in (q, k, v))
    out = _run(q.to(gpu), k.to(gpu), v.to(gpu), (3, 13, 13), origin=(0, 6, 6), extent=(3, 8, 16))
    ref = O.na3d(q, k, v, (3, 13, 13), q_origin=(0, 6, 6), q_extent=(3, 8, 16))
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= BF16_TOL
    assert rel_l2(out[0, 1, 3, 4, 1].float().cpu(), ref[0, 1, 3, 4, 1]) <= BF16_TOL


# Small windows on regular strips (2 x 8 tiles, two rows per stage, ky in {5, 7, 9},
# kx <= 9): the rows with unclamped y windows take the strip kernel, the clamped
# edge rows the general kernel, one output.  Cases: whole grids with every edge,
# ragged x, a query box reaching into the clamped rows, dilation in z and x, an
# anisotropic window, a grid with fewer regular rows than a tile pair, batches of heads.
SMALL_CASES = [
    # shape (B, Z, Y, X, H, D), kernel, dilation, origin, extent
    ((1, 4, 20, 24, 2, 64), (3, 7, 7), (1, 1, 1), (0, 0, 0), None),
    ((1, 5, 30, 33, 1, 64), (3, 5, 5), (1, 1, 1), (0, 0, 0), None),
    ((2, 6, 27, 40, 2, 64), (3, 9, 9), (1, 1, 1), (1, 3, 5), (4, 20, 30)),
    ((1, 6, 24, 24, 1, 64), (3, 7, 7), (2, 1, 2), (0, 0, 0), None),
    ((1, 3, 16, 16, 2, 64), (3, 7, 9), (1, 1, 1), (0, 2, 0), (3, 12, 16)),
    ((1, 4, 9, 16, 1, 64), (3, 7, 7), (1, 1, 1), (0, 0, 0), None),
    ((1, 3, 40, 36, 3, 64), (3, 9, 7), (1, 1, 1), (0, 0, 0), None),
    # query box clear of both y edges: the launch holds strips only
    ((2, 4, 40, 32, 2, 64), (3, 7, 7), (1, 1, 1), (1, 5, 3), (3, 25, 20)),
    # only the bottom edge is clamped (two rows of the general body)
    ((1, 4, 30, 20, 2, 64), (3, 5, 5), (1, 1, 1), (0, 10, 0), (4, 20, 20)),
    # a single unclamped row: no regular strip, the general kernel alone
    ((1, 3, 7, 16, 1, 64), (3, 7, 7), (1, 1, 1), (0, 0, 0), None),
    # the production window (3,3,3): two tile slots, one clamped row at each y edge
    ((1, 5, 24, 20, 2, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),
    ((2, 4, 19, 37, 2, 64), (3, 3, 3), (1, 1, 1), (1, 2, 3), (3, 15, 30)),
    ((1, 6, 12, 16, 2, 64), (3, 3, 3), (2, 1, 2), (0, 0, 0), None),
    ((1, 3, 3, 16, 1, 64), (3, 3, 3), (1, 1, 1), (0, 0, 0), None),
]


@pytest.mark.parametrize("case", SMALL_CASES, ids=[f"{c[0]}-k{c[1]}-d{c[2]}-box{c[3]}" for c in SMALL_CASES])
def test_small_window_strips_vs_oracle(gpu, case):
    shape, kernel, dil, origin, extent = case
    print(f"small strip {shape} k{kernel} d{dil} o{origin} e{extent}", flush=True)
    q, k, v = _rand(shape, 31, torch.bfloat16, gpu)
    out = _run(q, k, v, kernel, dil, origin, extent)
    ref = O.na3d(q.cpu(), k.cpu(), v.cpu(), kernel, dil, q_origin=origin, q_extent=extent)
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= BF16_TOL


def test_small_window_strip_score_out_of_range(gpu):
    """A 7x7 query whose best key scores ~160 (log2 units) and one whose keys all
    score ~-160 leave the reference-free range of the small-window strip kernel:
    their 2 x 8 tiles are recomputed exactly."""
    shape = (1, 3, 20, 24, 1, 64)
    q, k, v = (t.float() for t in _rand(shape, 12, torch.bfloat16, "cpu"))
    u = torch.zeros(64)
    u[:32] = 1.0 / 32**0.5
    q[0, 1, 9, 10, 0] = 30.0 * u
    k[0, 2, 11, 12, 0] = 30.0 * u
    q[0, 1, 12, 5, 0] = -30.0 * u
    k[0, :, 9:16, 2:9, 0] = 0.1 * k[0, :, 9:16, 2:9, 0] + 30.0 * u
    q, k, v = (t.bfloat16() for t in (q, k, v))
    out = _run(q.to(gpu), k.to(gpu), v.to(gpu), (3, 7, 7))
    ref = O.na3d(q, k, v, (3, 7, 7))
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= BF16_TOL
    for idx in ((0, 1, 9, 10, 0), (0, 1, 12, 5, 0)):
        assert rel_l2(out[idx].float().cpu(), ref[idx]) <= BF16_TOL, idx


@pytest.mark.parametrize("kernel", [(3, 7, 7), (3, 3, 3)])
def test_small_window_strips_match_general_kernel(gpu, monkeypatch, kernel):
    """The same configs[3]-like launch through the strip path and, with it
    switched off, through the general kernel: both within bf16 rounding."""
    g = torch.Generator(device=gpu).manual_seed(5)
    q, k, v = (torch.randn((1, 8, 64, 64, 4, 64), generator=g, device=gpu).bfloat16() for _ in range(3))
    a = _run(q, k, v, kernel)
    monkeypatch.setenv("STRATA_HIP_NA3D_NO_SMALL_STRIPS", "1")
    b = _run(q, k, v, kernel)
    assert rel_l2(a.float(), b.float()) <= 5e-3


def _column_attention(q, k, v, scale=None):
    """Softmax attention of every token over its whole z column (float64): the textbook
    dense attention, independent of the NA3D oracle's window tables."""
    B, Z, Y, X, H, D = q.shape
    scale = D**-0.5 if scale is None else scale
    qc, kc, vc = (t.double().permute(0, 2, 3, 4, 1, 5) for t in (q, k, v))  # [B, Y, X, H, Z, D]
    p = torch.softmax(scale * qc @ kc.transpose(-1, -2), dim=-1)
    return (p @ vc).permute(0, 4, 1, 2, 3, 5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Z", [8, 24, 5, 32, 1, 40])
def test_depthwise_window_is_column_attention(gpu, dtype, Z):
    """Window (Z, 1, 1): every query attends its whole z column, for even Z (a kernel equal
    to the whole axis) and odd Z; the production depth of 24 among them.  bf16 Z <= 32 runs
    the column kernel (Z = 1 and 32 at its ends), Z = 40 the tile kernels."""
    q, k, v = _rand((1, Z, 6, 10, 4, 64), 3, dtype, gpu)
    print(f"depthwise {dtype} Z={Z}", flush=True)
    out = _run(q, k, v, (Z, 1, 1))
    ref = _column_attention(q.cpu(), k.cpu(), v.cpu())
    if dtype == torch.float32:
        assert (out.cpu().double() - ref).abs().max().item() <= F32_TOL
    else:
        assert rel_l2(out.float(), ref) <= BF16_TOL


def test_even_kernel_short_of_the_axis_is_refused(gpu):
    q, k, v = _rand((1, 8, 6, 6, 2, 64), 4, torch.bfloat16, gpu)
    with pytest.raises(ValueError, match="odd"):
        _run(q, k, v, (6, 1, 1))
    with pytest.raises(ValueError, match="odd"):
        _run(q, k, v, (8, 1, 1), dilation=(2, 1, 1))


def test_depthwise_lse_and_strided_views(gpu):
    """The column kernel with lse (the training forward) and q / v as strided views of a
    packed qkv buffer, against the oracle's log2-sum-exp and outputs."""
    B, Z, Y, X, H = 2, 24, 5, 6, 3
    g = torch.Generator().manual_seed(8)
    qkv = torch.randn(B, Z, Y, X, 3, H, 64, generator=g).bfloat16()
    q, k, v = qkv[..., 0, :, :], qkv[..., 1, :, :].contiguous(), qkv[..., 2, :, :]
    qg = qkv.to(gpu)
    out, lse = torch.ops.strata_hip.na3d_fwd_lse(qg[..., 0, :, :], k.to(gpu), qg[..., 2, :, :], [Z, 1, 1],
                                                 [1, 1, 1], None)
    ref, ref_lse = O.na3d(q, k, v, (Z, 1, 1), compute_dtype=torch.float64, return_lse=True)
    assert rel_l2(out.float(), ref) <= BF16_TOL
    assert (lse.double().cpu() - ref_lse).abs().max().item() <= 2e-2
