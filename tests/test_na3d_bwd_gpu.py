"""NA3D backward on the GPU (dq, dk, dv through the C ABI) vs the CPU oracle's
autograd: fp32 inputs to within fp32 summation-order differences, bf16 inputs
to relative L2 <= 1e-2 against the fp32 oracle on the same bf16-rounded inputs."""

import pytest
import torch

from oracle import na3d as O
from strata_amd import ops  # noqa: F401
from strata_amd.natten import na3d as natten_na3d

from .conftest import rel_l2

pytestmark = pytest.mark.gpu

CASES = [  # shape [B, Z, Y, X, H, D], kernel, dilation
    ((1, 4, 9, 11, 2, 64), (3, 5, 5), (1, 1, 1)),
    ((2, 3, 8, 8, 1, 32), (3, 3, 7), (1, 1, 1)),
    ((1, 4, 12, 12, 2, 64), (3, 5, 3), (1, 2, 2)),
    ((1, 3, 14, 16, 1, 128), (3, 13, 13), (1, 1, 1)),
    ((1, 5, 7, 9, 2, 64), (5, 7, 9), (1, 1, 1)),
    ((1, 3, 21, 30, 2, 64), (3, 13, 13), (1, 1, 1)),  # MFMA dq: x union of 16 keys, ragged tiles
    ((2, 4, 6, 37, 1, 64), (3, 5, 11), (1, 1, 1)),
    # LDS dq / dk/dv: three workgroup columns (the last ragged), keys at both x edges
    # needing two 16-query blocks, clamped y windows, a multi-stage ring
    ((1, 4, 13, 45, 2, 64), (3, 9, 13), (1, 1, 1)),
    # dq on strips (the unclamped rows) plus the tile walk on the clamped edge rows:
    # two 32-column boxes (the second ragged), two batches; an odd strip row count
    # cut into one-tile chunks
    ((2, 4, 20, 40, 2, 64), (3, 7, 7), (1, 1, 1)),
    ((1, 3, 33, 16, 3, 64), (3, 5, 5), (1, 1, 1)),
    # the production window (3,3,3) at head_dim 64 (dq, dV and dK strips with their clamped
    # edges; a ragged 32-column box and two batches)
    ((1, 5, 24, 20, 2, 64), (3, 3, 3), (1, 1, 1)),
    ((2, 4, 21, 40, 2, 64), (3, 3, 3), (1, 1, 1)),
    # depth-wise attention: the whole z column, even (a kernel equal to the axis) and odd
    ((1, 8, 6, 7, 2, 64), (8, 1, 1), (1, 1, 1)),
    ((1, 24, 4, 5, 2, 64), (24, 1, 1), (1, 1, 1)),
    ((1, 7, 5, 6, 1, 32), (7, 1, 1), (1, 1, 1)),
]


def _inputs(shape, seed, dtype, gpu):
    g = torch.Generator().manual_seed(seed)
    q, k, v, dout = (torch.randn(shape, generator=g).to(dtype) for _ in range(4))
    return (q, k, v, dout), tuple(t.to(gpu) for t in (q, k, v, dout))


def _fwd(q, k, v, kernel, dilation):
    return torch.ops.strata_hip.na3d_fwd(q, k, v, list(kernel), list(dilation), None, [0, 0, 0], list(q.shape[1:4]))


@pytest.mark.parametrize("case", CASES, ids=str)
def test_bwd_fp32_vs_oracle(gpu, case):
    shape, kernel, dil = case
    (q, k, v, dout), (qg, kg, vg, dg) = _inputs(shape, 0, torch.float32, gpu)
    out = _fwd(qg, kg, vg, kernel, dil)
    dq, dk, dv = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out, dg, list(kernel), list(dil), None)
    ref = O.na3d_backward(q, k, v, dout, kernel, dil, compute_dtype=torch.float64)
    for name, got, want in (("dq", dq, ref[0]), ("dk", dk, ref[1]), ("dv", dv, ref[2])):
        err = (got.double().cpu() - want).abs().max().item()
        assert err <= 1e-4 * max(1.0, want.abs().max().item()), (name, err)


@pytest.mark.parametrize("case", CASES, ids=str)
def test_bwd_bf16_vs_oracle(gpu, case):
    shape, kernel, dil = case
    (q, k, v, dout), (qg, kg, vg, dg) = _inputs(shape, 1, torch.bfloat16, gpu)
    out = _fwd(qg, kg, vg, kernel, dil)
    dq, dk, dv = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out, dg, list(kernel), list(dil), None)
    ref = O.na3d_backward(q, k, v, dout, kernel, dil)
    for name, got, want in (("dq", dq, ref[0]), ("dk", dk, ref[1]), ("dv", dv, ref[2])):
        assert rel_l2(got.float().cpu(), want) <= 1e-2, name


def test_autograd_through_the_forward_op_and_natten_shim(gpu):
    shape, kernel = (1, 4, 10, 10, 2, 64), (3, 5, 5)
    (q, k, v, dout), (qg, kg, vg, dg) = _inputs(shape, 2, torch.bfloat16, gpu)
    leaves = [t.clone().requires_grad_(True) for t in (qg, kg, vg)]
    out = natten_na3d(*leaves, kernel_size=kernel)
    out.backward(dg)
    # with gradients wanted the shim runs na3d_fwd_lse: the backward gets its lse
    out2, lse = torch.ops.strata_hip.na3d_fwd_lse(qg, kg, vg, list(kernel), [1, 1, 1], None)
    assert torch.equal(out.detach(), out2)
    direct = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out2, dg, list(kernel), [1, 1, 1], None, lse)
    for leaf, d in zip(leaves, direct):
        assert torch.equal(leaf.grad, d)
    ref = O.na3d_backward(q, k, v, dout, kernel)
    assert rel_l2(leaves[0].grad.float().cpu(), ref[0]) <= 1e-2


def test_backward_of_a_query_box_raises(gpu):
    (_, _, _, _), (qg, kg, vg, dg) = _inputs((1, 3, 8, 8, 1, 32), 3, torch.float32, gpu)
    q = qg.clone().requires_grad_(True)
    out = torch.ops.strata_hip.na3d_fwd(q, kg, vg, [3, 3, 3], [1, 1, 1], None, [0, 2, 2], [3, 4, 4])
    with pytest.raises(RuntimeError, match="full-grid"):
        out.sum().backward()


@pytest.mark.parametrize("case", [c for c in CASES if c[0][-1] == 64 and c[2] == (1, 1, 1)], ids=str)
def test_bwd_mfma_matches_valu_path(gpu, case, monkeypatch):
    """bf16, head_dim 64, dilation 1 runs the MFMA kernels; the VALU kernels
    (STRATA_HIP_NA3D_BWD_VALU) must agree with them."""
    shape, kernel, dil = case
    _, (qg, kg, vg, dg) = _inputs(shape, 4, torch.bfloat16, gpu)
    out = _fwd(qg, kg, vg, kernel, dil)
    fast = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out, dg, list(kernel), list(dil), None)
    monkeypatch.setenv("STRATA_HIP_NA3D_BWD_VALU", "1")
    slow = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out, dg, list(kernel), list(dil), None)
    for a, b in zip(fast, slow):
        assert rel_l2(a.float(), b.float()) <= 1e-2


@pytest.mark.parametrize("case", CASES, ids=str)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_forward_lse_vs_oracle(gpu, case, dtype):
    """The forward's log2-sum-exp (scalar, general MFMA and strip kernels, the
    reference-free strips included: their row sum is 2^lse itself) against the
    oracle's, and the output unchanged by asking for it, bit for bit (the same
    kernels serve both requests)."""
    shape, kernel, dil = case
    (q, k, v, _), (qg, kg, vg, _) = _inputs(shape, 5, dtype, gpu)
    out, lse = torch.ops.strata_hip.na3d_fwd_lse(qg, kg, vg, list(kernel), list(dil), None)
    plain = _fwd(qg, kg, vg, kernel, dil)
    assert torch.equal(out, plain)
    _, ref = O.na3d(q, k, v, kernel, dil, compute_dtype=torch.float64, return_lse=True)
    # bf16: the kernels score bf16(scale*log2(e)*q) against k, a 2^-9 relative rounding of q
    tol = 1e-4 if dtype == torch.float32 else 3e-2
    assert (lse.double().cpu() - ref).abs().max().item() <= tol


def _box_lse(qg, kg, vg, kernel, org, ext):
    """The C ABI's forward over a query box with the lse output; (out, lse)."""
    from strata_amd import _lib

    H = qg.shape[4]
    out = torch.empty((1, *ext, H, 64), dtype=torch.bfloat16, device=qg.device)
    lse = torch.empty((1, *ext, H), dtype=torch.float32, device=qg.device)
    a = _lib.Na3dArgs()
    a.q, a.k, a.v, a.out, a.lse = qg.data_ptr(), kg.data_ptr(), vg.data_ptr(), out.data_ptr(), lse.data_ptr()
    a.dtype, a.batch, a.heads, a.head_dim, a.scale = _lib.BF16, 1, H, 64, 64**-0.5
    a.grid[:], a.q_origin[:], a.q_extent[:] = qg.shape[1:4], org, ext
    a.kernel[:], a.dilation[:] = kernel, [1, 1, 1]
    a.q_stride[:], a.k_stride[:], a.v_stride[:] = ([qg.stride(i) for i in range(5)],) * 3
    a.o_stride[:] = [out.stride(i) for i in range(5)]
    _lib.call("strata_hip_na3d_fwd", a, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out, lse


def test_forward_lse_exact_path_on_the_regular_strip(gpu):
    """A query with a key scoring ~162 log2 units overflows the reference-free strip
    softmax; the tile's exact recompute writes its lse (~162) as well as its output."""
    shape = (1, 3, 20, 28, 1, 64)
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    u = torch.zeros(64)
    u[:32] = 1.0 / 32**0.5
    w = torch.zeros(64)
    w[32:] = 1.0 / 32**0.5
    q[0, 1, 9, 10, 0] = 30.0 * u
    k[0, 1, 9, 10, 0] = 2.0 * w
    k[0, 2, 12, 14, 0] = 30.0 * u
    q, k, v = (t.bfloat16() for t in (q, k, v))
    org, ext = (0, 6, 6), (3, 8, 16)
    out, lse = _box_lse(q.to(gpu), k.to(gpu), v.to(gpu), (3, 13, 13), org, ext)
    ref_o, ref_l = O.na3d(q, k, v, (3, 13, 13), q_origin=org, q_extent=ext, compute_dtype=torch.float64,
                          return_lse=True)
    assert torch.isfinite(lse).all()
    assert rel_l2(out.float().cpu(), ref_o.float()) <= 1e-2
    assert (lse.double().cpu() - ref_l).abs().max().item() <= 3e-2
    assert lse[0, 1, 3, 4, 0].item() > 150


def test_forward_lse_of_a_query_box_on_the_regular_strip_shape(gpu):
    """A halo-interior box on the reference-free strip kernel, with the lse asked for."""
    from strata_amd import _lib

    shape, kernel, org, ext = (1, 3, 24, 30, 2, 64), (3, 13, 13), (0, 6, 7), (3, 10, 13)
    (q, k, v, _), (qg, kg, vg, _) = _inputs(shape, 6, torch.bfloat16, gpu)
    out = torch.empty((1, *ext, 2, 64), dtype=torch.bfloat16, device=gpu)
    lse = torch.empty((1, *ext, 2), dtype=torch.float32, device=gpu)
    a = _lib.Na3dArgs()
    a.q, a.k, a.v, a.out, a.lse = qg.data_ptr(), kg.data_ptr(), vg.data_ptr(), out.data_ptr(), lse.data_ptr()
    a.dtype, a.batch, a.heads, a.head_dim, a.scale = _lib.BF16, 1, 2, 64, 64**-0.5
    a.grid[:], a.q_origin[:], a.q_extent[:] = shape[1:4], org, ext
    a.kernel[:], a.dilation[:] = kernel, [1, 1, 1]
    a.q_stride[:], a.k_stride[:], a.v_stride[:] = ([qg.stride(i) for i in range(5)],) * 3
    a.o_stride[:] = [out.stride(i) for i in range(5)]
    _lib.call("strata_hip_na3d_fwd", a, torch.cuda.current_stream().cuda_stream)
    ref_o, ref_l = O.na3d(q, k, v, kernel, q_origin=org, q_extent=ext, compute_dtype=torch.float64, return_lse=True)
    assert rel_l2(out.float().cpu(), ref_o.float()) <= 1e-2
    assert (lse.double().cpu() - ref_l).abs().max().item() <= 3e-2


@pytest.mark.parametrize("case", CASES, ids=str)
def test_bwd_with_forward_lse_matches_recompute(gpu, case):
    """The backward given the forward's lse (prep reduced to rowsum(dO*O)) agrees
    with the backward that recomputes it, and with the oracle."""
    shape, kernel, dil = case
    (q, k, v, dout), (qg, kg, vg, dg) = _inputs(shape, 7, torch.bfloat16, gpu)
    out, lse = torch.ops.strata_hip.na3d_fwd_lse(qg, kg, vg, list(kernel), list(dil), None)
    given = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out, dg, list(kernel), list(dil), None, lse)
    recomputed = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out, dg, list(kernel), list(dil), None)
    ref = O.na3d_backward(q, k, v, dout, kernel, dil)
    # The two lse values differ in the last bits (the forward sums bf16 probabilities), and
    # every bf16 output rounds on its own: the paths agree to about the bf16 rounding noise
    # (measured 1.6e-3 to 2.2e-3, lower for wider windows) and each matches the oracle
    # (about 3e-3).
    for name, a, b, r in zip(("dq", "dk", "dv"), given, recomputed, ref):
        assert rel_l2(a.float().cpu(), r) <= 1e-2, name
        assert rel_l2(b.float().cpu(), r) <= 1e-2, name
        assert rel_l2(a.float(), b.float()) <= 4e-3, name
