"""NA3D with the queries' rotary embedding inside the kernel (na3d_fwd_rope_q)
against the unfused path (the pack rotates q and k, then na3d_fwd), which the
other GPU tests check against the oracle; the k-only pack against the full one."""
import pytest
import torch

from .conftest import rel_l2
from strata_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _tables(B, Zt, Y, X, g, dev):
    theta = torch.rand(B, Zt, Y, X, 32, generator=g) * 6.283
    return theta.cos().to(dev), theta.sin().to(dev)


def _qkv(B, Z, Y, X, H, g, dev, scale=1.0):
    return (torch.randn(B, Z, Y, X, 3 * H * 64, generator=g) * scale).bfloat16().to(dev)


@pytest.mark.parametrize("shape, kernel, zt, dil", [
    ((2, 8, 64, 64, 8), (3, 7, 7), 1, (1, 1, 1)),
    ((2, 8, 64, 64, 8), (3, 7, 7), 8, (1, 1, 1)),     # configs[1]: tables with the level index in z
    ((1, 8, 32, 32, 4), (3, 9, 9), 1, (1, 1, 1)),
    ((1, 6, 24, 40, 2), (3, 5, 5), 6, (1, 1, 1)),
    ((1, 4, 20, 24, 2), (3, 7, 7), 1, (1, 1, 1)),     # short strips, ragged columns
    ((1, 8, 32, 40, 2), (3, 7, 7), 8, (2, 1, 2)),     # z and x dilation: residue classes, level tables
    ((1, 6, 24, 30, 2), (3, 5, 5), 1, (2, 1, 3)),
    ((1, 6, 24, 40, 2), (3, 3, 3), 1, (1, 1, 1)),     # the production window
    ((1, 4, 16, 24, 2), (3, 3, 3), 4, (1, 1, 1)),
])
def test_rope_q_fused_matches_pack_then_na3d(gpu, shape, kernel, zt, dil):
    B, Z, Y, X, H = shape
    g = torch.Generator().manual_seed(sum(shape) + zt + sum(dil))
    qkv = _qkv(B, Z, Y, X, H, g, gpu)
    cos, sin = _tables(B, zt, Y, X, g, gpu)
    q6 = qkv.view(B, Z, Y, X, 3, H, 64)
    v = q6[..., 2, :, :]
    q_ref, k_ref, _ = ops.rope_qkv_pack(qkv, cos, sin, H, _lib.ROPE_HALF, pack_v=False)
    ref = ops.na3d_fwd(q_ref, k_ref, v, list(kernel), list(dil), None, [0, 0, 0], [Z, Y, X])
    _, k, _ = ops.rope_qkv_pack(qkv, cos, sin, H, _lib.ROPE_HALF, pack_v=False, pack_q=False)
    assert torch.equal(k, k_ref)
    kst = [Z * Y * X * H * 64, Y * X * H * 64, X * H * 64, H * 64, 64]
    assert ops.na3d_rope_q_supported(q6[..., 0, :, :], kst, v, cos, sin, kernel, list(dil))
    out = ops.na3d_fwd_rope_q(q6[..., 0, :, :], k, v, cos, sin, list(kernel), list(dil), None)
    torch.cuda.synchronize()
    # q' is rotated by the same fused multiply-adds (rope_rot_a / rope_rot_b) and rounded
    # to bf16 as the pack does, and the tile math is the same: equal bit for bit
    print(f"fused vs unfused: rel-L2 {rel_l2(out, ref):.2e}, identical {torch.equal(out, ref)}", flush=True)
    assert torch.equal(out, ref)


def test_rope_q_exact_path(gpu):
    """Scores far outside the fast path's range send tiles to the exact recompute,
    which rotates its queries from global memory."""
    B, Z, Y, X, H = 1, 4, 24, 24, 2
    g = torch.Generator().manual_seed(5)
    qkv = _qkv(B, Z, Y, X, H, g, gpu)
    qkv.view(B, Z, Y, X, 3, H, 64)[..., 0, :, :] *= 40  # scores of ~several hundred log2 units
    cos, sin = _tables(B, 1, Y, X, g, gpu)
    q6 = qkv.view(B, Z, Y, X, 3, H, 64)
    v = q6[..., 2, :, :]
    q_ref, k_ref, _ = ops.rope_qkv_pack(qkv, cos, sin, H, _lib.ROPE_HALF, pack_v=False)
    ref = ops.na3d_fwd(q_ref, k_ref, v, [3, 7, 7], [1, 1, 1], None, [0, 0, 0], [Z, Y, X])
    out = ops.na3d_fwd_rope_q(q6[..., 0, :, :], k_ref, v, cos, sin, [3, 7, 7], [1, 1, 1], None)
    assert torch.isfinite(out.float()).all()
    print(f"exact path: rel-L2 {rel_l2(out, ref):.2e}, identical {torch.equal(out, ref)}", flush=True)
    assert rel_l2(out, ref) <= 2e-3, rel_l2(out, ref)


def test_rope_q_unsupported_shapes_are_refused(gpu):
    """The wide-window strip kernels carry no query rotation: the query says no and
    the entry point raises instead of computing something else."""
    B, Z, Y, X, H = 1, 4, 32, 32, 2
    g = torch.Generator().manual_seed(6)
    qkv = _qkv(B, Z, Y, X, H, g, gpu)
    cos, sin = _tables(B, 1, Y, X, g, gpu)
    q6 = qkv.view(B, Z, Y, X, 3, H, 64)
    q, v = q6[..., 0, :, :], q6[..., 2, :, :]
    kst = [Z * Y * X * H * 64, Y * X * H * 64, X * H * 64, H * 64, 64]
    assert not ops.na3d_rope_q_supported(q, kst, v, cos, sin, (3, 13, 13), [1, 1, 1])
    assert not ops.na3d_rope_q_supported(q.float(), kst, v.float(), cos, sin, (3, 7, 7), [1, 1, 1])
    with pytest.raises(_lib.StrataHipError):
        ops.na3d_fwd_rope_q(q, q.contiguous(), v, cos, sin, [3, 13, 13], [1, 1, 1], None)
