"""Pins of the CPU NA3D oracle (no GPU).

The oracle is trusted only as far as these checks go: golden vectors from the
brute-force search formulation, the unfold formulation, closed forms (dense
attention when the window covers the grid, kernel 1 returns v, constant v),
symmetry, and a planted mistake that the goldens must catch.
"""

import math

import pytest
import torch

from oracle import na3d as O


def test_window_start_known_values():
    # L=7, k=3: windows shift (never truncate) at the edges
    assert [O.window_start(i, 7, 3) for i in range(7)] == [0, 0, 1, 2, 3, 4, 4]
    # k = L: every query sees the whole axis
    assert [O.window_start(i, 5, 5) for i in range(5)] == [0] * 5
    # dilation 2 on L=9: residue classes {0,2,4,6,8} and {1,3,5,7}
    assert [O.window_start(i, 9, 3, 2) for i in range(9)] == [0, 1, 0, 1, 2, 3, 4, 3, 4]


def test_window_by_search_matches_closed_form():
    for L in range(1, 14):
        for k in (1, 3, 5, 7):
            for d in (1, 2, 3):
                if k * d > L:
                    continue
                for i in range(L):
                    keys = O._window_by_search(i, L, k, d)
                    s = O.window_start(i, L, k, d)
                    assert keys == [s + d * j for j in range(k)], (L, k, d, i)
                    assert len(keys) == k and i in keys


def test_oracle_matches_bruteforce_goldens(na3d_golden):
    for name, c in na3d_golden.items():
        q, k, v = (torch.from_numpy(c[t]) for t in "qkv")
        out = O.na3d(q, k, v, c["kernel"], c["dilation"], compute_dtype=torch.float64)
        err = (out - torch.from_numpy(c["out"]).double()).abs().max().item()
        assert err < 2e-6, (name, err)


def test_planted_truncated_window_fails_goldens(na3d_golden):
    """A plausible mistake — truncating windows at the edges instead of
    shifting them — must disagree with the golden vectors."""
    c = na3d_golden["clamp_small"]
    q, k, v = (torch.from_numpy(c[t]).double() for t in "qkv")
    B, Z, Y, X, H, D = q.shape
    kz, ky, kx = c["kernel"]
    wrong = torch.empty_like(q)
    for z in range(Z):
        for y in range(Y):
            for x in range(X):
                zs = range(max(0, z - kz // 2), min(Z, z + kz // 2 + 1))
                ys = range(max(0, y - ky // 2), min(Y, y + ky // 2 + 1))
                xs = range(max(0, x - kx // 2), min(X, x + kx // 2 + 1))
                kk = torch.stack([k[:, a, b, cc] for a in zs for b in ys for cc in xs], dim=1)
                vv = torch.stack([v[:, a, b, cc] for a in zs for b in ys for cc in xs], dim=1)
                s = torch.einsum("bhd,bwhd->bhw", q[:, z, y, x], kk) * D**-0.5
                wrong[:, z, y, x] = torch.einsum("bhw,bwhd->bhd", s.softmax(-1), vv)
    err = (wrong - torch.from_numpy(c["out"]).double()).abs().max().item()
    assert err > 1e-2


def test_unfold_formulation_matches_cfg0():
    """fp32, [1,4,16,16,4,32], W=(3,5,5), q/k/v ~ N(0,1) seed 0."""
    g = torch.Generator().manual_seed(0)
    shape = (1, 4, 16, 16, 4, 32)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    a = O.na3d(q, k, v, (3, 5, 5))
    b = O.na3d_unfold(q, k, v, (3, 5, 5))
    assert (a - b).abs().max().item() <= 1e-5


def test_kernel_covering_grid_is_dense_attention():
    g = torch.Generator().manual_seed(7)
    shape = (2, 3, 5, 7, 2, 8)
    q, k, v = (torch.randn(shape, generator=g, dtype=torch.float64) for _ in range(3))
    out = O.na3d(q, k, v, (3, 5, 7), compute_dtype=torch.float64)
    ref = O.dense_attention(q, k, v)
    assert (out - ref).abs().max().item() < 1e-12


def test_kernel_one_returns_v_and_constant_v():
    g = torch.Generator().manual_seed(3)
    shape = (1, 4, 4, 4, 2, 8)
    q, k, v = (torch.randn(shape, generator=g, dtype=torch.float64) for _ in range(3))
    assert torch.allclose(O.na3d(q, k, v, 1, compute_dtype=torch.float64), v)
    vc = torch.ones_like(v) * 0.75
    assert torch.allclose(O.na3d(q, k, vc, 3, compute_dtype=torch.float64), vc)


def test_query_box_is_a_crop():
    g = torch.Generator().manual_seed(5)
    shape = (1, 6, 9, 10, 2, 8)
    q, k, v = (torch.randn(shape, generator=g, dtype=torch.float64) for _ in range(3))
    full = O.na3d(q, k, v, (3, 5, 5), compute_dtype=torch.float64)
    box = O.na3d(q, k, v, (3, 5, 5), q_origin=(1, 2, 3), q_extent=(4, 5, 6), compute_dtype=torch.float64)
    assert torch.equal(box, full[:, 1:5, 2:7, 3:9])


def test_heads_and_batch_permute():
    g = torch.Generator().manual_seed(9)
    shape = (2, 4, 6, 6, 3, 8)
    q, k, v = (torch.randn(shape, generator=g, dtype=torch.float64) for _ in range(3))
    out = O.na3d(q, k, v, 3, compute_dtype=torch.float64)
    perm_h = torch.tensor([2, 0, 1])
    out_h = O.na3d(q[..., perm_h, :], k[..., perm_h, :], v[..., perm_h, :], 3, compute_dtype=torch.float64)
    assert torch.allclose(out_h, out[..., perm_h, :])
    out_b = O.na3d(q.flip(0), k.flip(0), v.flip(0), 3, compute_dtype=torch.float64)
    assert torch.allclose(out_b, out.flip(0))


def test_rejects_even_or_oversized_kernel():
    q = torch.zeros(1, 4, 4, 4, 1, 8)
    with pytest.raises(ValueError):
        O.na3d(q, q, q, (2, 3, 3))
    with pytest.raises(ValueError):
        O.na3d(q, q, q, (5, 3, 3))
    with pytest.raises(ValueError):  # even and the whole axis, but dilated
        O.axis_keys(4, 4, 2)


def _column_softmax(q, k, v):
    """Dense softmax attention over the z axis only, written directly (float64)."""
    B, Z, Y, X, H, D = q.shape
    out = torch.empty_like(q)
    for b in range(B):
        for y in range(Y):
            for x in range(X):
                for h in range(H):
                    s = (q[b, :, y, x, h] @ k[b, :, y, x, h].T) * D**-0.5
                    out[b, :, y, x, h] = torch.softmax(s, dim=-1) @ v[b, :, y, x, h]
    return out


@pytest.mark.parametrize("Z", [4, 5, 6])
def test_depthwise_window_is_column_softmax(Z):
    """Window (Z, 1, 1), even Z included (a kernel equal to the whole axis): every query
    attends its whole z column and nothing else."""
    assert O.axis_keys(Z, Z).tolist() == [list(range(Z))] * Z
    g = torch.Generator().manual_seed(11)
    shape = (1, Z, 3, 4, 2, 8)
    q, k, v = (torch.randn(shape, generator=g, dtype=torch.float64) for _ in range(3))
    ref = _column_softmax(q, k, v)
    assert (O.na3d(q, k, v, (Z, 1, 1), compute_dtype=torch.float64) - ref).abs().max().item() < 1e-12
    assert (O.na3d_bruteforce(q, k, v, (Z, 1, 1)) - ref).abs().max().item() < 1e-12
    # a planted mistake: a window one key short of the column (odd kernel Z - 1 when Z is
    # even, the nearest NATTEN window) does not reproduce it
    if Z % 2 == 0:
        assert (O.na3d(q, k, v, (Z - 1, 1, 1), compute_dtype=torch.float64) - ref).abs().max().item() > 1e-3


def test_flop_count_cfg2():
    # 6 tiles x interior (16,128,128) x 16 heads x W=507 x D=64
    f = O.na3d_flops(6, 16, 64, 16 * 128 * 128, (3, 13, 13))
    assert math.isclose(f, 3.266e12, rel_tol=1e-3)


@pytest.mark.parametrize("kernel,dilation", [((3, 3, 5), (1, 1, 1)), ((1, 3, 3), (1, 2, 1)), ((3, 5, 3), (1, 1, 2))])
def test_backward_matches_finite_differences(kernel, dilation):
    """The oracle's backward against central finite differences (torch gradcheck, fp64),
    on grids small enough that the windows clamp at every edge."""
    g = torch.Generator().manual_seed(7)
    shape = (1, 3, 6, 7, 2, 4)
    q, k, v = (torch.randn(shape, generator=g, dtype=torch.float64, requires_grad=True) for _ in range(3))

    def f(q, k, v):
        return O.na3d(q, k, v, kernel, dilation, compute_dtype=torch.float64)

    assert torch.autograd.gradcheck(f, (q, k, v), eps=1e-6, atol=1e-6, rtol=1e-5, fast_mode=True)


def test_backward_full_window_is_dense_attention_backward():
    """Kernel covering the grid: the gradients are those of dense softmax attention."""
    g = torch.Generator().manual_seed(9)
    B, Z, Y, X, H, D = 1, 3, 3, 5, 2, 4
    q, k, v, dout = (torch.randn((B, Z, Y, X, H, D), generator=g, dtype=torch.float64) for _ in range(4))
    dq, dk, dv = O.na3d_backward(q, k, v, dout, (Z, Y, X), compute_dtype=torch.float64)
    qt, kt, vt = (t.clone().requires_grad_(True) for t in (q, k, v))

    def heads(t):  # [B, Z, Y, X, H, D] -> [B, H, N, D]
        return t.reshape(B, Z * Y * X, H, D).transpose(1, 2)

    o = torch.nn.functional.scaled_dot_product_attention(heads(qt), heads(kt), heads(vt))
    gq, gk, gv = torch.autograd.grad(o, (qt, kt, vt), heads(dout))
    for a, b in zip((dq, dk, dv), (gq, gk, gv)):
        assert torch.allclose(a, b, atol=1e-10, rtol=1e-9)


def test_backward_dv_is_transposed_attention():
    """dV = P^T dO: with dout = one-hot rows, dv sums the softmax weights each key receives."""
    g = torch.Generator().manual_seed(8)
    shape = (1, 2, 5, 5, 1, 3)
    q, k, v = (torch.randn(shape, generator=g, dtype=torch.float64) for _ in range(3))
    dout = torch.zeros(shape, dtype=torch.float64)
    dout[..., 0] = 1.0
    _, _, dv = O.na3d_backward(q, k, v, dout, (1, 3, 3), compute_dtype=torch.float64)
    # total weight is conserved: every query distributes exactly 1
    assert torch.allclose(dv[..., 0].sum(), torch.tensor(2 * 5 * 5, dtype=torch.float64))
    assert torch.all(dv[..., 1:] == 0)


def test_lse_is_the_dense_logsumexp_when_the_window_is_the_grid():
    """With the window the whole (odd) grid, each query's lse is the base-2
    logsumexp of its dense scores; on a real window it matches a per-query
    loop over the keys that the brute-force oracle visits."""
    import math

    g = torch.Generator().manual_seed(31)
    B, Z, Y, X, H, D = 1, 3, 5, 7, 2, 16
    q, k, v = (torch.randn(B, Z, Y, X, H, D, generator=g, dtype=torch.float64) for _ in range(3))
    scale = 0.3
    _, lse = O.na3d(q, k, v, (Z, Y, X), scale=scale, compute_dtype=torch.float64, return_lse=True)
    qf = q.reshape(B, -1, H, D)
    kf = k.reshape(B, -1, H, D)
    s = torch.einsum("bqhd,bkhd->bhqk", qf, kf) * scale
    ref = (torch.logsumexp(s, dim=-1) / math.log(2.0)).permute(0, 2, 1).reshape(B, Z, Y, X, H)
    assert torch.allclose(lse, ref, atol=1e-12)
    # a clamped 3x3x5 window, one query near a corner, from the window definition
    _, lse = O.na3d(q, k, v, (3, 3, 5), scale=scale, compute_dtype=torch.float64, return_lse=True)
    z, y, x, h = 0, 4, 1, 1
    keys = [(a, b_, c) for a in range(0, 3) for b_ in range(2, 5) for c in range(0, 5)]
    sc = torch.stack([(q[0, z, y, x, h] * k[0, a, b_, c, h]).sum() * scale for a, b_, c in keys])
    assert abs(lse[0, z, y, x, h].item() - (torch.logsumexp(sc, 0) / math.log(2.0)).item()) < 1e-12
