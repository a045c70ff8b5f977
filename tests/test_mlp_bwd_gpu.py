"""GEMM-GELU backward on the GPU: the fused gelu'(x @ w.T + b) * dout epilogue
and the autograd of strata_hip::gemm_bias_act / GemmGeluMlp, against torch's
own autograd of Linear + GELU(tanh) in fp32 on the same bf16 inputs
(relative L2 <= 1e-2)."""

import pytest
import torch
import torch.nn.functional as F

from strata_amd import _lib, ops
from strata_amd.modules import GemmGeluMlp

from .conftest import rel_l2

pytestmark = pytest.mark.gpu

SHAPES = [(300, 512, 256), (4096, 1024, 1024), (77, 200, 64)]  # (M, N, K)


def _bf(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).bfloat16()


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_gelu_grad_epilogue(gpu, shape):
    M, N, K = shape
    g = torch.Generator().manual_seed(0)
    x, w, b, dout = _bf((M, K), g), _bf((N, K), g, K**-0.5), _bf((N,), g), _bf((M, N), g)
    got = ops.gemm_bias_act(x.to(gpu), w.to(gpu), b.to(gpu), dout.to(gpu), _lib.ACT_GELU_TANH_GRAD, _lib.RES_MUL)
    a = (x.double() @ w.double().T + b.double()).requires_grad_(True)
    (ga,) = torch.autograd.grad(F.gelu(a, approximate="tanh"), a, dout.double())
    assert rel_l2(got.float().cpu(), ga.float()) <= 1e-2


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("act", [_lib.ACT_GELU_TANH, _lib.ACT_NONE])
def test_gemm_autograd_vs_torch(gpu, shape, act):
    M, N, K = shape
    g = torch.Generator().manual_seed(1)
    x, w, b, r, dout = _bf((M, K), g), _bf((N, K), g, K**-0.5), _bf((N,), g), _bf((M, N), g), _bf((M, N), g)
    res = act == _lib.ACT_NONE  # the fc2 + residual shape; GELU runs without one (fc1)
    leaves = [t.to(gpu).requires_grad_(True) for t in ((x, w, b, r) if res else (x, w, b))]
    out = ops.gemm_bias_act(leaves[0], leaves[1], leaves[2], leaves[3] if res else None, act)
    out.backward(dout.to(gpu))
    ref_leaves = [t.float().requires_grad_(True) for t in ((x, w, b, r) if res else (x, w, b))]
    y = F.linear(ref_leaves[0], ref_leaves[1], ref_leaves[2])
    y = F.gelu(y, approximate="tanh") if act == _lib.ACT_GELU_TANH else y + ref_leaves[3]
    y.backward(dout.float())
    for name, a, bref in zip("xwbr", leaves, ref_leaves):
        assert rel_l2(a.grad.float().cpu(), bref.grad) <= 1e-2, name


@pytest.mark.parametrize("shape", [(300, 512, 256), (4096, 1024, 1024), (1000, 4104, 128)], ids=str)
def test_gemm_gelu_train(gpu, shape):
    """fc1 for training: its GELU output equals the inference launch's bit for bit, the
    saved derivative is gelu'(x @ w.T + b) within bf16 rounding, and its autograd (the
    derivative times the upstream gradient, then plain GEMMs and the bias gradient)
    matches torch's Linear + GELU(tanh) backward."""
    M, N, K = shape
    g = torch.Generator().manual_seed(3)
    x, w, b, dout = _bf((M, K), g), _bf((N, K), g, K**-0.5), _bf((N,), g), _bf((M, N), g)
    xg, wg, bg = (t.to(gpu).requires_grad_(True) for t in (x, w, b))
    out, dact = ops.gemm_gelu_train(xg, wg, bg)
    plain = ops.gemm_bias_act(x.to(gpu), w.to(gpu), b.to(gpu), None, _lib.ACT_GELU_TANH)
    assert torch.equal(out.detach(), plain)
    a = (x.double() @ w.double().T + b.double()).requires_grad_(True)
    (ga,) = torch.autograd.grad(F.gelu(a, approximate="tanh"), a, torch.ones_like(a))
    assert rel_l2(dact.float().cpu(), ga.float()) <= 1e-2
    out.backward(dout.to(gpu))
    ref = [t.float().requires_grad_(True) for t in (x, w, b)]
    F.gelu(F.linear(*ref), approximate="tanh").backward(dout.float())
    for name, got, r in zip("xwb", (xg, wg, bg), ref):
        assert rel_l2(got.grad.float().cpu(), r.grad) <= 1e-2, name


def test_mlp_module_backward(gpu):
    torch.manual_seed(0)
    mlp = GemmGeluMlp(256, 1024)
    g = torch.Generator().manual_seed(2)
    x, r, dout = _bf((2, 8, 16, 256), g), _bf((2, 8, 16, 256), g), _bf((2, 8, 16, 256), g)
    ref = GemmGeluMlp(256, 1024)
    ref.load_state_dict(mlp.state_dict())
    ref = ref.float()
    mlp = mlp.to(gpu).bfloat16()
    xg = x.to(gpu).requires_grad_(True)
    mlp(xg, r.to(gpu)).backward(dout.to(gpu))
    xr = x.float().requires_grad_(True)
    (ref.layers(xr) + r.float()).backward(dout.float())
    assert rel_l2(xg.grad.float().cpu(), xr.grad) <= 1e-2
    for (n1, p1), (n2, p2) in zip(mlp.named_parameters(), ref.named_parameters()):
        assert n1 == n2
        assert rel_l2(p1.grad.float().cpu(), p2.grad.bfloat16().float()) <= 1e-2, n1


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_gate_autograd_vs_torch(gpu, shape):
    """The attention gate sigmoid(x @ w.T + b) * a: gradients of x, w, b and a."""
    M, N, K = shape
    g = torch.Generator().manual_seed(3)
    x, w, b, a, dout = _bf((M, K), g), _bf((N, K), g, K**-0.5), _bf((N,), g), _bf((M, N), g), _bf((M, N), g)
    leaves = [t.to(gpu).requires_grad_(True) for t in (x, w, b, a)]
    ops.gemm_bias_act(*leaves, _lib.ACT_SIGMOID, _lib.RES_MUL).backward(dout.to(gpu))
    ref = [t.float().requires_grad_(True) for t in (x, w, b, a)]
    (torch.sigmoid(F.linear(ref[0], ref[1], ref[2])) * ref[3]).backward(dout.float())
    for name, got, want in zip("xwba", leaves, ref):
        assert rel_l2(got.grad.float().cpu(), want.grad) <= 1e-2, name
