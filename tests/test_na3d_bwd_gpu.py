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
    direct = torch.ops.strata_hip.na3d_bwd(qg, kg, vg, out.detach(), dg, list(kernel), [1, 1, 1], None)
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
