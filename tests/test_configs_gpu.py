"""BASELINE configs[1], [3] and [4] run as their full workloads on the GPU, and the
hand-written GEMM epilogues at production size, checked against the CPU oracle.

Where the float oracle over the whole workload would take minutes, the full
launch runs on the GPU and the oracle checks what the domain makes independent:
sub-boxes of the NA3D output (each query depends only on its window), one batch
entry of a block (batch entries never interact), sampled GEMM rows spanning every
256-row tile (each output row depends only on its input row).  Whole-output
properties cover the rest: finiteness, bit-exact equivariance under a permutation
of the cube-face tiles, and the identity step of a zero head.
Bars: bf16 rel-L2 <= 1e-2 against fp32/fp64 references.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import block as OB
from oracle import na3d as O
from oracle import rope as R
from strata_amd import _lib, ops  # noqa: F401
from strata_amd import rope as P
from strata_amd.model import TwoStageStrata
from strata_amd.modules import StrataBlock, init_xavier_

from .conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-2


# ---------------------------------------------------------------------------
# NA3D + stereographic RoPE with the level index in z
# ---------------------------------------------------------------------------
def test_cfg1_rope_level_pack_na3d_full(gpu):
    """bf16 [2,8,64,64,8,64], W=(3,7,7); q/k/v ~ N(0,1) (seed 0, drawn in that order);
    tables from a 64x64 tile at lat0 ~ U(-60,60), lon0 ~ U(0,360) deg, 32 pairs split
    x | y | level = 12 | 12 | 8, base 1e4; RoPE + pack kernel, then NA3D, full launch."""
    B, Z, Y, X, H, D = 2, 8, 64, 64, 8, 64
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, Z, Y, X, H, D, generator=g).bfloat16() for _ in range(3))
    lat, lon = P.synthetic_tile_latlon(B, Y, X, g)
    ls = P.default_rope_length_scale(1)
    cos, sin = P.stereographic_rope_tables(lat, lon, D, 10000.0, ls, levels=Z, level_pairs=8)
    assert cos.shape == (B, Z, Y, X, D // 2)
    qkv = torch.stack([q, k, v], dim=4).reshape(B, Z, Y, X, 3 * H * D).to(gpu)
    print("cfg1 rope pack + na3d full launch", flush=True)
    qr, kr, vr = torch.ops.strata_hip.rope_qkv_pack(qkv, cos.to(gpu), sin.to(gpu), H, _lib.ROPE_HALF, False, 1e-6,
                                                    None, None)
    out = torch.ops.strata_hip.na3d_fwd(qr, kr, vr, [3, 7, 7], [1, 1, 1], None, [0, 0, 0], [Z, Y, X])
    # the path bench.py times: the pack writes k only, NA3D rotates q (a strided view of qkv)
    # as it loads each tile and reads v from qkv
    print("cfg1 k-only pack + na3d_fwd_rope_q full launch", flush=True)
    _, kf, _ = torch.ops.strata_hip.rope_qkv_pack(qkv, cos.to(gpu), sin.to(gpu), H, _lib.ROPE_HALF, False, 1e-6,
                                                  None, None, False, False)
    q6 = qkv.view(B, Z, Y, X, 3, H, D)
    out_f = torch.ops.strata_hip.na3d_fwd_rope_q(q6[..., 0, :, :], kf, q6[..., 2, :, :], cos.to(gpu), sin.to(gpu),
                                                 [3, 7, 7], [1, 1, 1], None)
    torch.cuda.synchronize()
    assert torch.equal(kf, kr)
    print(f"  fused vs pack-then-NA3D: identical {torch.equal(out_f, out)}, rel-L2 {rel_l2(out_f, out):.2e}",
          flush=True)
    assert torch.equal(out_f, out)  # the same rotation arithmetic and tile math
    assert torch.equal(vr.cpu(), v)
    co, so = R.tables(lat, lon, D, 10000.0, ls, levels=Z, level_pairs=8)
    for b, h in ((0, 0), (1, 7), (0, 5)):
        sl = (slice(b, b + 1), slice(None), slice(None), slice(None), slice(h, h + 1))
        rq = R.apply_rope(q[sl].double(), co[b : b + 1], so[b : b + 1])
        rk = R.apply_rope(k[sl].double(), co[b : b + 1], so[b : b + 1])
        # the pack kernel's rotation: within one bf16 rounding of the float64 rotation
        for got, ref in ((qr[sl].cpu().double(), rq), (kr[sl].cpu().double(), rk)):
            assert ((got - ref).abs() <= ref.abs() * 2**-7 + 1e-5).all()
        for org in ((0, 0, 0), (6, 56, 56), (3, 28, 30), (7, 0, 60)):
            ext = (1, 8, 4)
            ref = O.na3d(rq, rk, v[sl].double(), (3, 7, 7), q_origin=org, q_extent=ext,
                         compute_dtype=torch.float64)
            box = (slice(b, b + 1), slice(org[0], org[0] + ext[0]), slice(org[1], org[1] + ext[1]),
                   slice(org[2], org[2] + ext[2]), slice(h, h + 1))
            assert rel_l2(out[box].float(), ref) <= TOL, (b, h, org)
            assert rel_l2(out_f[box].float(), ref) <= TOL, ("fused", b, h, org)


# ---------------------------------------------------------------------------
# the full Strata block
# ---------------------------------------------------------------------------
def _block(gpu, C, H, kernel, gated=False, qk_norm=False):
    blk = StrataBlock(C, H, kernel, gated=gated, qk_norm=qk_norm)
    init_xavier_(blk, torch.Generator().manual_seed(1))
    params = {k: v.detach().bfloat16().float() for k, v in blk.state_dict().items()}
    return blk.to(gpu).bfloat16(), params


def _block_vs_oracle(gpu, B, grid, C, H, kernel, base=10000.0, ls_patch=1, gated=False, qk_norm=False,
                     entries=(0,)):
    Z, Y, X = grid
    blk, params = _block(gpu, C, H, kernel, gated, qk_norm)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, Z, Y, X, C, generator=g).bfloat16()
    lat, lon = P.synthetic_tile_latlon(B, Y, X, g)
    ls = P.default_rope_length_scale(ls_patch)
    cos, sin = P.stereographic_rope_tables(lat, lon, C // H, base, ls)
    print(f"block [{B},{Z},{Y},{X},{C}] H={H} kernel={kernel} gated={gated} qk_norm={qk_norm}", flush=True)
    with torch.no_grad():
        out = blk(x.to(gpu), (cos.to(gpu), sin.to(gpu)))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    co, so = R.tables(lat, lon, C // H, base, ls)
    for b in entries:
        ref = OB.block_forward(x[b : b + 1].float(), params, H, kernel, co[b : b + 1].float(), so[b : b + 1].float(),
                               gated=gated, qk_norm=qk_norm)
        err = rel_l2(out[b : b + 1].float(), ref)
        print(f"  entry {b}: rel-L2 {err:.3e}", flush=True)
        assert err <= TOL, (b, err)


def test_cfg3_block_full(gpu):
    """[4,8,64,64,1024], 16x64 heads, W=(3,7,7), Xavier seed 1, x ~ N(0,1) seed 0;
    batch entries 0 and 3 against the fp32 oracle."""
    _block_vs_oracle(gpu, 4, (8, 64, 64), 1024, 16, (3, 7, 7), entries=(0, 3))


# ---------------------------------------------------------------------------
# the two-stage model at full size
# ---------------------------------------------------------------------------
def test_cfg4_stage_blocks_full_shape(gpu):
    """One stage-1 block (768, 12x64, W=(3,7,7)) on [6,16,64,64] and one stage-2
    block (1024, 16x64, W=(3,9,9)) on [6,8,32,32] (tables at patch 2), batch entry 0."""
    _block_vs_oracle(gpu, 6, (16, 64, 64), 768, 12, (3, 7, 7), entries=(0,))
    _block_vs_oracle(gpu, 6, (8, 32, 32), 1024, 16, (3, 9, 9), ls_patch=2, entries=(0, 5))


def test_cfg4_full_model_step_properties(gpu):
    """Full configs[4] model (12 + 12 blocks, batch 6 face tiles, 80 channels):
    finite step; the step repeats bit for bit; permuting the faces (with their
    tables) permutes the output bit for bit (every kernel, the GEMMs included,
    computes each tile in a fixed order that does not depend on its position in
    the batch); a zero head makes the step the identity; 2 steps of rollout stay
    finite."""
    torch.manual_seed(0)
    model = TwoStageStrata()
    init_xavier_(model, torch.Generator().manual_seed(1))
    model = model.to(gpu).bfloat16()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(6, 80, 16, 64, 64, generator=g)
    lat, lon = P.synthetic_tile_latlon(6, 64, 64, g)
    r1, r2 = model.rope_tables(lat.to(gpu), lon.to(gpu))
    xg = x.to(gpu)
    perm = torch.tensor([3, 0, 5, 1, 4, 2], device=gpu)
    pr1 = tuple(t[perm] for t in r1)
    pr2 = tuple(t[perm] for t in r2)
    print("cfg4 full step", flush=True)
    y = model.step(xg, r1, r2)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    assert (y - xg).abs().max() > 0
    assert torch.equal(model.step(xg, r1, r2), y)  # deterministic run to run
    print("cfg4 permuted faces", flush=True)
    yp = model.step(xg[perm], pr1, pr2)
    d = (yp - y[perm]).abs().max().item()
    assert torch.equal(yp, y[perm]), f"face permutation changed the output by {d}"
    print("cfg4 rollout 2 steps", flush=True)
    yr = model.rollout(xg, 2, r1, r2)
    assert torch.isfinite(yr).all()
    with torch.no_grad():
        model.head.weight.zero_()
        model.head.bias.zero_()
    print("cfg4 zero head", flush=True)
    assert torch.equal(model.step(xg, r1, r2), xg)


# ---------------------------------------------------------------------------
# Hand-written GEMM epilogues at production size (persistent tile walk: many
# tiles per workgroup) against float64 on sampled rows of every 256-row tile
# ---------------------------------------------------------------------------
def _rows(M):
    r = torch.cat([torch.arange(0, M, 128), torch.arange(255, M, 256), torch.tensor([M - 1])])
    return torch.unique(r)


GEMM_PROD = [
    # M, N, K, act, res_op, residual: fc1 + GELU at configs[3]; its backward epilogue (GELU' * dout);
    # the gate (a * sigmoid); a ragged M with more tiles than CUs at K = 256; ragged M and N with
    # more tiles than CUs at one and two K steps per tile (the ring runs on from tile to tile)
    (131072, 4096, 1024, _lib.ACT_GELU_TANH, _lib.RES_ADD, False),
    (131072, 4096, 1024, _lib.ACT_GELU_TANH_GRAD, _lib.RES_MUL, True),
    (131072, 1024, 1024, _lib.ACT_SIGMOID, _lib.RES_MUL, True),
    (16421, 4096, 256, _lib.ACT_GELU_TANH, _lib.RES_ADD, True),
    (8300, 2104, 64, _lib.ACT_GELU_TANH, _lib.RES_ADD, True),
    (4100, 4200, 128, _lib.ACT_SIGMOID, _lib.RES_MUL, False),
]


def _act64(z, act):
    if act == _lib.ACT_GELU_TANH:
        return F.gelu(z, approximate="tanh")
    if act == _lib.ACT_SIGMOID:
        return torch.sigmoid(z)
    if act == _lib.ACT_GELU_TANH_GRAD:
        zz = z.clone().requires_grad_(True)
        F.gelu(zz, approximate="tanh").sum().backward()
        return zz.grad
    raise ValueError(act)


@pytest.mark.parametrize("case", GEMM_PROD, ids=[f"{c[0]}x{c[1]}x{c[2]}-act{c[3]}" for c in GEMM_PROD])
def test_gemm_epilogues_production_size(gpu, case):
    M, N, K, act, res_op, has_r = case
    print(f"gemm prod {case}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(M + N + K + act)
    x = torch.randn(M, K, generator=g, device=gpu).bfloat16()
    w = (torch.randn(N, K, generator=g, device=gpu) * K**-0.5).bfloat16()
    b = (torch.randn(N, generator=g, device=gpu) * 0.5).bfloat16()
    r = torch.randn(M, N, generator=g, device=gpu).bfloat16() if has_r else None
    out = torch.ops.strata_hip.gemm_bias_act(x, w, b, r, act, res_op)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    rows = _rows(M)
    xs = x[rows.to(gpu)].cpu().double()
    z = xs @ w.cpu().double().T + b.cpu().double()
    ref = _act64(z, act)
    if r is not None:
        rs = r[rows.to(gpu)].cpu().double()
        ref = ref * rs if res_op == _lib.RES_MUL else ref + rs
    got = out[rows.to(gpu)].cpu().double()
    err = rel_l2(got, ref)
    print(f"  {len(rows)} rows, rel-L2 {err:.3e}", flush=True)
    assert err <= TOL


# ---------------------------------------------------------------------------
# The production block (screamcast train_configs.py:295-317): 1024 wide, 16 x 64
# heads, attn_kernel = 3 (taken as (3,3,3)), gated attention, non-affine qk
# RMSNorm, stereographic RoPE with base 100 and the length scale of horizontal
# patch 4 (strata_wrappers.py:333-338), on the rollout tile geometry: a 512-px
# tile + 32-px halo at patch 4 = (24,144,144) tokens (run_screamcast_nudged.py:156-165).
# ---------------------------------------------------------------------------
def _crop_checks(out, x, params, cos, sin, H, kernel, crops, grid):
    """The block is local: on a crop of the input (tables cropped, not rebuilt)
    the oracle reproduces the full-grid output wherever a query's clamped
    window is the same in the crop as in the grid."""
    for lo, hi in crops:
        sl = tuple(slice(a, b) for a, b in zip(lo, hi))
        xc = x[(slice(0, 1), *sl)].float()
        cc, sc = cos[(slice(0, 1), *sl)], sin[(slice(0, 1), *sl)]
        ref = OB.block_forward(xc, params, H, kernel, cc, sc, gated=True, qk_norm=True)
        keep = []
        for a, b, L, k in zip(lo, hi, grid, kernel):
            r = k // 2
            keep.append(slice(0 if a == 0 else r, (b - a) if b == L else (b - a) - r))
        got = out[(slice(0, 1), *sl)][(slice(None), *keep)].float()
        want = ref[(slice(None), *keep)]
        err = rel_l2(got, want)
        print(f"  crop {lo}-{hi}: rel-L2 {err:.3e}", flush=True)
        assert err <= TOL, (lo, hi, err)


def test_production_block_rollout_geometry(gpu):
    """The production block on one full rollout tile: 1024 wide, 16 x 64 heads, window
    (3,3,3), gated, non-affine qk RMSNorm, RoPE base 100 at the patch-4 length scale
    (scripts/ace/run_screamcast_nudged.py:156-165, train_configs.py:303-317), checked
    against the oracle on three crops (corner, interior, far corner).  Its one earlier
    run faulted the GPU with the plain GEMMs on hipBLASLt (operands over 2 GiB); every
    launch it now issues is hand-written and replayed in bounds on the CPU at this exact
    shape (tests/test_launch_bounds.py)."""
    Z, Y, X, C, H, kernel = 24, 144, 144, 1024, 16, (3, 3, 3)
    blk = StrataBlock(C, H, kernel, gated=True, qk_norm=True)
    init_xavier_(blk, torch.Generator().manual_seed(1))
    with torch.no_grad():
        blk.attn.gate_proj.bias.normal_(generator=torch.Generator().manual_seed(2))
    params = {k: v.detach().bfloat16().float() for k, v in blk.state_dict().items()}
    blk = blk.to(gpu).bfloat16()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, Z, Y, X, C, generator=g).bfloat16()
    ls = P.default_rope_length_scale(4)
    lat, lon = P.synthetic_tile_latlon(1, Y, X, g, spacing=ls)
    cos, sin = P.stereographic_rope_tables(lat, lon, C // H, 100.0, ls)
    print("production block (24,144,144) x 1024, gated, qk-norm, RoPE base 100", flush=True)
    with torch.no_grad():
        out = blk(x.to(gpu), (cos.to(gpu), sin.to(gpu)))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    co, so = R.tables(lat, lon, C // H, 100.0, ls)
    co = co.float().expand(1, Z, Y, X, C // H // 2)
    so = so.float().expand(1, Z, Y, X, C // H // 2)
    _crop_checks(out.cpu(), x, params, co, so, H, kernel,
                 [((0, 0, 0), (5, 12, 12)), ((10, 70, 100), (15, 82, 112)), ((19, 132, 132), (24, 144, 144))],
                 (Z, Y, X))
