"""GEMM (+bias/GELU/residual), RoPE+QKV pack and LayerNorm on the GPU vs CPU references."""

import pytest
import torch
import torch.nn.functional as F

from oracle import rope as R
from strata_amd import _lib, ops  # noqa: F401
from strata_amd import rope as P

from .conftest import rel_l2

pytestmark = pytest.mark.gpu


def _randn(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).bfloat16()


GEMM_CASES = [
    # M, N, K, act, bias, residual
    (256, 256, 64, _lib.ACT_NONE, False, False),
    (300, 200, 72, _lib.ACT_NONE, True, False),
    (1000, 384, 1024, _lib.ACT_GELU_TANH, True, False),
    (513, 1024, 256, _lib.ACT_GELU_ERF, True, True),
    (128, 96, 80, _lib.ACT_NONE, True, True),
    (4096, 3072, 1024, _lib.ACT_NONE, True, False),
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=[str(c[:4]) for c in GEMM_CASES])
def test_gemm_vs_fp64(gpu, case):
    M, N, K, act, has_b, has_r = case
    print(f"gemm {case}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    x = _randn((M, K), g)
    w = _randn((N, K), g, K**-0.5)
    b = _randn((N,), g) if has_b else None
    r = _randn((M, N), g) if has_r else None
    out = torch.ops.strata_hip.gemm_bias_act(
        x.to(gpu), w.to(gpu), None if b is None else b.to(gpu), None if r is None else r.to(gpu), act
    )
    ref = x.double() @ w.double().T
    if b is not None:
        ref = ref + b.double()
    if act == _lib.ACT_GELU_TANH:
        ref = F.gelu(ref, approximate="tanh")
    elif act == _lib.ACT_GELU_ERF:
        ref = F.gelu(ref)
    if r is not None:
        ref = ref + r.double()
    assert out.shape == (M, N)
    assert rel_l2(out.float(), ref) <= 1e-2


@pytest.mark.parametrize("M,N,K", [(300, 256, 128), (4096, 1024, 1024), (77, 200, 64)])
def test_gemm_sigmoid_gate_vs_fp64(gpu, M, N, K):
    """Gate epilogue: a * sigmoid(x @ w.T + b) with a passed as the residual (res_op MUL)."""
    print(f"gemm gate {M}x{N}x{K}", flush=True)
    g = torch.Generator().manual_seed(M + N)
    x = _randn((M, K), g)
    w = _randn((N, K), g, 2 * K**-0.5)
    b = _randn((N,), g)
    a = _randn((M, N), g)
    out = torch.ops.strata_hip.gemm_bias_act(x.to(gpu), w.to(gpu), b.to(gpu), a.to(gpu), _lib.ACT_SIGMOID, _lib.RES_MUL)
    ref = a.double() * torch.sigmoid(x.double() @ w.double().T + b.double())
    assert rel_l2(out.float(), ref) <= 1e-2


def test_gemm_sigmoid_saturates(gpu):
    """Pre-activations of +-200 give exactly the residual and exactly zero."""
    M, N, K = 64, 64, 64
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    w = torch.zeros(N, K, dtype=torch.bfloat16)
    b = torch.tensor([200.0, -200.0] * (N // 2), dtype=torch.bfloat16)
    a = torch.randn(M, N).bfloat16()
    out = torch.ops.strata_hip.gemm_bias_act(x.to(gpu), w.to(gpu), b.to(gpu), a.to(gpu), _lib.ACT_SIGMOID,
                                             _lib.RES_MUL).cpu()
    assert torch.equal(out[:, 0::2], a[:, 0::2])
    assert torch.equal(out[:, 1::2], torch.zeros_like(a[:, 1::2]))


def test_gemm_batched_shape_and_aliasing(gpu):
    g = torch.Generator().manual_seed(1)
    x = _randn((2, 3, 5, 64), g).to(gpu)
    w = _randn((128, 64), g, 0.125).to(gpu)
    r = _randn((2, 3, 5, 128), g).to(gpu)
    out = torch.ops.strata_hip.gemm_bias_act(x, w, None, r, 0)
    ref = x.double() @ w.double().T + r.double()
    assert out.shape == (2, 3, 5, 128)
    assert rel_l2(out.float(), ref) <= 1e-2


PLAIN_GEMM_CASES = [
    # M, N, K, bias, residual: the block's plain projections (qkv, proj + residual, fc2 + residual)
    # at reduced M, and ragged shapes.
    (2048, 3072, 1024, True, False),
    (2048, 1024, 1024, True, True),
    (1000, 1024, 4096, True, True),
    (333, 136, 80, True, False),
    (64, 640, 1024, False, True),
]


@pytest.mark.parametrize("case", PLAIN_GEMM_CASES, ids=[str(c) for c in PLAIN_GEMM_CASES])
def test_plain_gemm(gpu, case):
    """Plain GEMMs (bias, added residual) agree with fp64 and repeat bit for bit."""
    M, N, K, has_b, has_r = case
    print(f"plain gemm {case}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = _randn((M, K), g)
    w = _randn((N, K), g, K**-0.5)
    b = _randn((N,), g) if has_b else None
    r = _randn((M, N), g) if has_r else None
    ref = x.double() @ w.double().T
    if b is not None:
        ref = ref + b.double()
    if r is not None:
        ref = ref + r.double()
    args = (x.to(gpu), w.to(gpu), None if b is None else b.to(gpu), None if r is None else r.to(gpu), _lib.ACT_NONE)
    out = torch.ops.strata_hip.gemm_bias_act(*args)
    assert rel_l2(out.float(), ref) <= 1e-2
    assert torch.equal(torch.ops.strata_hip.gemm_bias_act(*args), out)


@pytest.mark.parametrize("M, N, K", [(393216, 768, 80), (300, 136, 80), (257, 520, 16), (64, 640, 200),
                                     (1000, 96, 1032), (77, 256, 8)])
def test_gemm_ragged_k_masks_the_last_stage(gpu, M, N, K):
    """K not a multiple of 64 (the rollout's patch embedding: K = 80) on the large-tile
    kernel: the last K stage's chunks past K read as zero.  x and w are views into
    wider rows whose padding holds NaN, so a chunk read past K would reach the output;
    also x and w at row stride K (the tail of the last row is the allocation's end)."""
    print(f"ragged K gemm {(M, N, K)}", flush=True)
    g = torch.Generator().manual_seed(M + 3 * N + K)
    x, w, b = _randn((M, K), g), _randn((N, K), g, K**-0.5), _randn((N,), g)
    ref = x.double() @ w.double().T + b.double()
    pad = 48
    xp = torch.full((M, K + pad), float("nan"), dtype=torch.bfloat16, device=gpu)
    wp = torch.full((N, K + pad), float("nan"), dtype=torch.bfloat16, device=gpu)
    xp[:, :K], wp[:, :K] = x.to(gpu), w.to(gpu)
    out = torch.ops.strata_hip.gemm_bias_act(xp[:, :K], wp[:, :K], b.to(gpu), None, _lib.ACT_NONE)
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out.float(), ref) <= 1e-2
    tight = torch.ops.strata_hip.gemm_bias_act(x.to(gpu), w.to(gpu), b.to(gpu), None, _lib.ACT_NONE)
    assert torch.equal(tight, out)


def _act_ref(act, y):
    if act == _lib.ACT_GELU_TANH:
        return F.gelu(y, approximate="tanh")
    if act == _lib.ACT_GELU_ERF:
        return F.gelu(y)
    if act == _lib.ACT_SIGMOID:
        return torch.sigmoid(y)
    if act in (_lib.ACT_GELU_TANH_GRAD, _lib.ACT_SIGMOID_GRAD):
        yr = y.clone().requires_grad_(True)
        f = F.gelu(yr, approximate="tanh") if act == _lib.ACT_GELU_TANH_GRAD else torch.sigmoid(yr)
        f.sum().backward()
        return yr.grad
    return y


@pytest.mark.parametrize("act", [_lib.ACT_NONE, _lib.ACT_GELU_TANH, _lib.ACT_GELU_ERF, _lib.ACT_SIGMOID,
                                 _lib.ACT_GELU_TANH_GRAD, _lib.ACT_SIGMOID_GRAD])
@pytest.mark.parametrize("res", [None, _lib.RES_ADD, _lib.RES_MUL])
def test_gemm_ragged_k_every_epilogue(gpu, act, res):
    """Every activation x residual instance of the ragged-K kernel (K = 80: one full and one
    16-column stage; ragged M and N) against float64."""
    M, N, K = 300, 136, 80
    g = torch.Generator().manual_seed(act * 3 + (0 if res is None else res + 1))
    x, w, b = _randn((M, K), g), _randn((N, K), g, 2 * K**-0.5), _randn((N,), g)
    r = _randn((M, N), g) if res is not None else None
    args = [x.to(gpu), w.to(gpu), b.to(gpu), None if r is None else r.to(gpu), act]
    out = torch.ops.strata_hip.gemm_bias_act(*args, _lib.RES_ADD if res is None else res)
    ref = _act_ref(act, x.double() @ w.double().T + b.double())
    if res == _lib.RES_ADD:
        ref = ref + r.double()
    elif res == _lib.RES_MUL:
        ref = ref * r.double()
    assert rel_l2(out.float(), ref) <= 1e-2


@pytest.mark.parametrize("act, res, has_b", [
    (_lib.ACT_NONE, None, True),                # early bias, the epilogue split by tile kind
    (_lib.ACT_GELU_TANH, None, True),
    (_lib.ACT_NONE, _lib.RES_ADD, True),        # early bias, one epilogue for both tile kinds
    (_lib.ACT_GELU_TANH_GRAD, _lib.RES_MUL, True),  # the bias loaded at the tile's start
    (_lib.ACT_NONE, None, False),
])
def test_gemm_walk_with_ragged_column_panels(gpu, act, res, has_b):
    """More tiles than workgroups (M = 40000, N = 1000: 628 tiles, 232 columns in the last
    panel), so workgroups load a later tile's bias, ragged panels included, while they
    finish the tile before it; every column's bias is distinct.  Against float64."""
    M, N, K = 40000, 1000, 128
    print(f"gemm walk ragged N act {act} res {res} bias {has_b}", flush=True)
    g = torch.Generator().manual_seed(act * 5 + (0 if res is None else res + 1) + has_b)
    x, w = _randn((M, K), g), _randn((N, K), g, 2 * K**-0.5)
    b = _randn((N,), g) if has_b else None
    r = _randn((M, N), g) if res is not None else None
    out = torch.ops.strata_hip.gemm_bias_act(x.to(gpu), w.to(gpu), None if b is None else b.to(gpu),
                                             None if r is None else r.to(gpu), act,
                                             _lib.RES_ADD if res is None else res)
    pre = x.double() @ w.double().T
    if b is not None:
        pre = pre + b.double()
    ref = _act_ref(act, pre)
    if res == _lib.RES_ADD:
        ref = ref + r.double()
    elif res == _lib.RES_MUL:
        ref = ref * r.double()
    assert rel_l2(out.float(), ref) <= 1e-2
    cols = (out.float().cpu().double() - ref).norm(dim=0) / ref.norm(dim=0).clamp_min(1e-30)
    assert cols.max().item() <= 3e-2  # no column panel with a wrong bias hides in the total


@pytest.mark.parametrize("N", [100, 36, 7])
def test_gemm_odd_n_through_the_op(gpu, N):
    """N not a multiple of 8: the op pads the weight (and bias, residual) to whole 16-byte
    output rows for the C ABI and returns the first N columns; also the GELU-saving launch."""
    M, K = 333, 128
    g = torch.Generator().manual_seed(N)
    x, w, b, r = _randn((M, K), g), _randn((N, K), g, K**-0.5), _randn((N,), g), _randn((M, N), g)
    out = torch.ops.strata_hip.gemm_bias_act(x.to(gpu), w.to(gpu), b.to(gpu), r.to(gpu), _lib.ACT_GELU_TANH)
    pre = x.double() @ w.double().T + b.double()
    assert out.shape == (M, N) and out.is_contiguous()
    assert rel_l2(out.float(), F.gelu(pre, approximate="tanh") + r.double()) <= 1e-2
    h, dact = torch.ops.strata_hip.gemm_gelu_train(x.to(gpu), w.to(gpu), b.to(gpu))
    pr = pre.clone().requires_grad_(True)
    F.gelu(pr, approximate="tanh").sum().backward()
    assert h.shape == dact.shape == (M, N)
    assert rel_l2(h.float(), F.gelu(pre, approximate="tanh")) <= 1e-2
    assert rel_l2(dact.float(), pr.grad) <= 1e-2


@pytest.mark.parametrize("K", [80, 200])
def test_gemm_gelu_save_ragged_k(gpu, K):
    """The GELU-saving fc1 launch at K not a multiple of 64: both outputs against fp64."""
    M, N = 1000, 768
    g = torch.Generator().manual_seed(K)
    x, w, b = _randn((M, K), g), _randn((N, K), g, K**-0.5), _randn((N,), g)
    pre = x.double() @ w.double().T + b.double()
    out, dact = torch.ops.strata_hip.gemm_gelu_train(x.to(gpu), w.to(gpu), b.to(gpu))
    pr = pre.clone().requires_grad_(True)
    F.gelu(pr, approximate="tanh").sum().backward()
    assert rel_l2(out.float(), F.gelu(pre, approximate="tanh")) <= 1e-2
    assert rel_l2(dact.float(), pr.grad) <= 1e-2


def test_plain_gemm_residual_in_place(gpu):
    """out may alias the residual (the C ABI's contract): out = x @ w.T + b + out."""
    M, N, K = 512, 768, 256
    g = torch.Generator().manual_seed(5)
    x, w, b, r = _randn((M, K), g), _randn((N, K), g, K**-0.5), _randn((N,), g), _randn((M, N), g)
    ref = x.double() @ w.double().T + b.double() + r.double()
    xd, wd, bd, rd = x.to(gpu), w.to(gpu), b.to(gpu), r.to(gpu)
    a = _lib.GemmArgs()
    a.x, a.w, a.bias, a.residual, a.out = xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), rd.data_ptr(), rd.data_ptr()
    a.m, a.n, a.k, a.ldx, a.ldw, a.ldr, a.ldo = M, N, K, K, K, N, N
    a.act, a.res_op = _lib.ACT_NONE, _lib.RES_ADD
    _lib.call("strata_hip_gemm_bias_act", a, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rel_l2(rd.float(), ref) <= 1e-2


@pytest.mark.parametrize("layout", [_lib.ROPE_HALF, _lib.ROPE_INTERLEAVED])
@pytest.mark.parametrize("zt", [1, 4])
def test_rope_pack_vs_oracle(gpu, layout, zt):
    B, Z, Y, X, H, D = 2, 4, 8, 12, 3, 64
    g = torch.Generator().manual_seed(7 + layout + zt)
    qkv = _randn((B, Z, Y, X, 3 * H * D), g)
    ang = torch.rand(B, zt, Y, X, D // 2, generator=g, dtype=torch.float64) * 20 - 10
    cos, sin = torch.cos(ang), torch.sin(ang)
    q, k, v = torch.ops.strata_hip.rope_qkv_pack(qkv.to(gpu), cos.float().to(gpu), sin.float().to(gpu), H, layout)
    t = qkv.double().view(B, Z, Y, X, 3, H, D)
    name = "half" if layout == _lib.ROPE_HALF else "interleaved"
    rq = R.apply_rope(t[..., 0, :, :], cos, sin, name)
    rk = R.apply_rope(t[..., 1, :, :], cos, sin, name)
    # bf16 output of an fp32 rotation: within one bf16 rounding of the exact value
    for got, ref in ((q, rq), (k, rk)):
        d = (got.double().cpu() - ref).abs()
        assert (d <= ref.abs() * 2**-8 + 1e-6).all(), d.max()
    assert torch.equal(v.cpu(), qkv.view(B, Z, Y, X, 3, H, D)[..., 2, :, :])


@pytest.mark.parametrize("layout", [_lib.ROPE_HALF, _lib.ROPE_INTERLEAVED])
@pytest.mark.parametrize("affine", [False, True])
def test_rope_pack_qk_norm_vs_oracle(gpu, layout, affine):
    """qk RMSNorm over D (per token, head) fused before the rotation."""
    from oracle import block as OB
    B, Z, Y, X, H, D = 1, 3, 6, 10, 4, 64
    g = torch.Generator().manual_seed(11 + layout + 2 * affine)
    qkv = _randn((B, Z, Y, X, 3 * H * D), g, 3.0)
    ang = torch.rand(B, 1, Y, X, D // 2, generator=g, dtype=torch.float64) * 20 - 10
    cos, sin = torch.cos(ang), torch.sin(ang)
    qw = (1 + 0.3 * torch.randn(D, generator=g)).bfloat16() if affine else None
    kw = (1 + 0.3 * torch.randn(D, generator=g)).bfloat16() if affine else None
    eps = 1e-6
    q, k, v = torch.ops.strata_hip.rope_qkv_pack(
        qkv.to(gpu), cos.float().to(gpu), sin.float().to(gpu), H, layout, True, eps,
        None if qw is None else qw.to(gpu), None if kw is None else kw.to(gpu))
    t = qkv.double().view(B, Z, Y, X, 3, H, D)
    name = "half" if layout == _lib.ROPE_HALF else "interleaved"
    rq = R.apply_rope(OB.rms_norm(t[..., 0, :, :], eps, None if qw is None else qw.double()), cos, sin, name)
    rk = R.apply_rope(OB.rms_norm(t[..., 1, :, :], eps, None if kw is None else kw.double()), cos, sin, name)
    for got, ref in ((q, rq), (k, rk)):
        d = (got.double().cpu() - ref).abs()
        assert (d <= ref.abs() * 2**-7 + 1e-3).all(), d.max()
    assert torch.equal(v.cpu(), qkv.view(B, Z, Y, X, 3, H, D)[..., 2, :, :])
    # each normalised (unrotated) head has RMS 1: the rotation preserves it
    if not affine:
        rms = q.double().cpu().pow(2).mean(-1).sqrt()
        assert (rms - 1).abs().max() < 1e-2


@pytest.mark.parametrize("layout", [_lib.ROPE_HALF, _lib.ROPE_INTERLEAVED])
@pytest.mark.parametrize("qk_norm", [False, True])
def test_rope_pack_without_v(gpu, layout, qk_norm):
    """pack_v=False (the block's path: v read out of qkv as a strided view) writes the
    same q and k bit for bit, returns no v, and the gradient reaching qkv through the
    pack and the view equals the one through the full pack."""
    B, Z, Y, X, H, D = 1, 3, 6, 10, 4, 64
    g = torch.Generator().manual_seed(21 + layout + 2 * qk_norm)
    qkv = _randn((B, Z, Y, X, 3 * H * D), g).to(gpu)
    ang = torch.rand(B, 1, Y, X, D // 2, generator=g) * 20 - 10
    cos, sin = torch.cos(ang).to(gpu), torch.sin(ang).to(gpu)
    wq = (1 + 0.3 * torch.randn(D, generator=g)).bfloat16().to(gpu) if qk_norm else None
    args = (cos, sin, H, layout, qk_norm, 1e-6, wq, None)
    q, k, v = ops.rope_qkv_pack(qkv, *args)
    q2, k2, v2 = ops.rope_qkv_pack(qkv, *args, pack_v=False)
    assert torch.equal(q, q2) and torch.equal(k, k2) and v2.numel() == 0
    w = [torch.randn(q.shape, generator=g).to(gpu) for _ in range(3)]
    grads = []
    for pack_v in (True, False):
        x = qkv.detach().clone().requires_grad_()
        a, b, c = ops.rope_qkv_pack(x, *args, pack_v=pack_v)
        if not pack_v:
            c = x.view(B, Z, Y, X, 3, H, D)[..., 2, :, :]
        ((a.float() * w[0]).sum() + (b.float() * w[1]).sum() + (c.float() * w[2]).sum()).backward()
        grads.append(x.grad)
    assert torch.equal(grads[0], grads[1])


def test_rope_pack_stereographic_tables(gpu):
    """configs[1]-style tables (64x64 tile, 32 pairs, base 1e4) built by the
    product helper agree with the float64 oracle and drive the pack kernel
    (the level-index tables of configs[1] run in tests/test_configs_gpu.py)."""
    g = torch.Generator().manual_seed(0)
    lat, lon = P.synthetic_tile_latlon(2, 64, 64, g)
    ls = P.default_rope_length_scale(1)
    cos, sin = P.stereographic_rope_tables(lat.to(gpu), lon.to(gpu), 64, 10000.0, ls)
    c2, s2 = R.tables(lat, lon, 64, 10000.0, ls)
    assert (cos.double().cpu() - c2).abs().max() < 1e-5
    assert (sin.double().cpu() - s2).abs().max() < 1e-5
    # ... and drive the pack kernel: [2, 2, 64, 64] tokens x 4 heads (tables broadcast over z)
    B, Z, H, D = 2, 2, 4, 64
    qkv = _randn((B, Z, 64, 64, 3 * H * D), g)
    q, k, v = torch.ops.strata_hip.rope_qkv_pack(qkv.to(gpu), cos, sin, H, _lib.ROPE_HALF, False, 1e-6, None, None)
    t = qkv.double().view(B, Z, 64, 64, 3, H, D)
    for got, ref in ((q, R.apply_rope(t[..., 0, :, :], c2, s2)), (k, R.apply_rope(t[..., 1, :, :], c2, s2))):
        d = (got.double().cpu() - ref).abs()
        assert (d <= ref.abs() * 2**-7 + 1e-6).all(), d.max()
    assert torch.equal(v.cpu(), qkv.view(B, Z, 64, 64, 3, H, D)[..., 2, :, :])


@pytest.mark.parametrize("M, N, ld", [(131072, 1024, 1024), (1000, 3072, 3072), (5, 8, 8), (300, 512, 520),
                                        (0, 16, 16)])
def test_bias_grad_vs_fp64(gpu, M, N, ld):
    """Column sums (the GEMM backward's bias gradient) against float64, rows strided
    when ld > N, and bit for bit the same on a second call."""
    g = torch.Generator().manual_seed(M + N)
    full = (_randn((max(M, 1), ld), g) * 2 + 0.25).bfloat16()[:M]
    x = full.to(gpu)[:, :N]
    out = torch.ops.strata_hip.bias_grad(x)
    again = torch.ops.strata_hip.bias_grad(x)
    torch.cuda.synchronize()
    ref = full[:, :N].double().sum(0)
    assert out.shape == (N,) and out.dtype == torch.bfloat16
    assert torch.equal(out, again)
    if M == 0:
        assert (out == 0).all()
    else:
        assert ((out.double().cpu() - ref).abs() <= ref.abs() * 2**-8 + 1e-3 * M**0.5).all()


@pytest.mark.parametrize("C", [64, 256, 768, 1024, 3840, 4096])
def test_layer_norm(gpu, C):
    g = torch.Generator().manual_seed(C)
    x = (_randn((257, C), g) * 3 + 1).bfloat16()
    out = torch.ops.strata_hip.layer_norm(x.to(gpu), 1e-6)
    ref = F.layer_norm(x.double(), (C,), eps=1e-6)
    assert rel_l2(out.float(), ref) <= 1e-2
    assert (out.double().cpu() - ref).abs().max() < 0.05


def test_ops_reject_cpu_tensors(gpu):
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        torch.ops.strata_hip.layer_norm(x, 1e-6)
