"""Every global byte the production block's hand-written launches touch lies inside
its tensor, checked on the CPU by replaying the kernels' address arithmetic
(tests/launch_model.py) at the exact arguments StrataBlock.forward issues.

The production rollout tile (24,144,144) x 1024 (16 x 64 heads, window (3,3,3),
gated, qk-norm; scripts/ace/run_screamcast_nudged.py:156-165, train_configs.py:
303-317) is the first shape at which this library issues operands over 2 GiB
(qkv output 3.06 GB, fc1 output 4.08 GB).  The same replay runs at reduced
shapes that pass on the GPU, and the GEMM model's tile walk is checked to cover
every output tile exactly once, so the model follows the kernels.  A planted
32-bit offset (an allocation-wide buffer descriptor with 32-bit lane offsets,
the scheme that breaks past 2^31 bytes) must be caught.
"""

import numpy as np
import pytest

from . import launch_model as LM


def _problems(launches):
    out = []
    for name, acc, sizes in launches:
        out += [f"{name}: {p}" for p in acc.check(sizes)]
    return out


@pytest.mark.parametrize("shape", [
    (1, 24, 144, 144, 1024, 16, (3, 3, 3)),   # production rollout tile, one tile per call
    (1, 4, 24, 40, 256, 4, (3, 3, 3)),        # the reduced production test (passes on the GPU)
    (2, 8, 32, 32, 1024, 16, (3, 3, 3)),
])
def test_block_launches_stay_inside_their_tensors(shape):
    B, Z, Y, X, C, H, kernel = shape
    launches = LM.production_block_launches(B, Z, Y, X, C, H, kernel)
    assert _problems(launches) == []
    # every access was modelled: each launch reads and writes something
    for name, acc, sizes in launches:
        assert acc.lo, name
        assert set(acc.lo) <= set(sizes), name


def test_production_depthwise_block_stays_inside_its_tensors():
    """The production tile's alternate block (depth-wise attention, window (24, 1, 1) on
    the column kernel, v strided through the 3.06 GB qkv buffer): every launch inside its
    tensors, the column kernel's reads and writes reaching the views' last bytes."""
    B, Z, Y, X, C, H = 1, 24, 144, 144, 1024, 16
    launches = LM.production_block_launches(B, Z, Y, X, C, H, (Z, 1, 1), depthwise=True)
    assert _problems(launches) == []
    acc, sizes = {n: (a, s) for n, a, s in launches}["na3d (column kernel)"]
    assert acc.lo["q"] == 0 and acc.hi["q"] == sizes["q"]
    assert acc.hi["v"] == sizes["v"] and acc.hi["out"] == sizes["out"]


def test_column_kernel_small_grid_touches_exactly_its_tensors():
    """A ragged grid (Z = 5 of the 32 rows a wave loads; items not a multiple of 4): the
    modelled accesses cover each tensor exactly."""
    B, L, H = 2, (5, 3, 7), 3
    st = LM.contiguous_strides([B, *L, H, 64])[:5]
    acc = LM.na3d_column_launch(B, L, H, st, st, st, st)
    n = 2 * B * L[0] * L[1] * L[2] * H * 64
    assert acc.check({"q": n, "k": n, "v": n, "out": n}) == []
    assert all(acc.lo[t] == 0 and acc.hi[t] == n for t in ("q", "k", "v", "out"))


def test_production_tile_reaches_past_2gib():
    """The replay does reach the large offsets: qkv's last row lies beyond 2^31 bytes,
    fc1's output beyond 4 * 10^9."""
    B, Z, Y, X, C, H, kernel = 1, 24, 144, 144, 1024, 16, (3, 3, 3)
    launches = {n: (a, s) for n, a, s in LM.production_block_launches(B, Z, Y, X, C, H, kernel)}
    acc, sizes = launches["qkv gemm"]
    assert acc.hi["out"] == sizes["out"] > 2**31
    acc, sizes = launches["fc1 gemm + gelu"]
    assert acc.hi["out"] == sizes["out"] > 4 * 10**9
    acc, sizes = launches["na3d (region kernel)"]
    assert acc.hi["v"] == sizes["v"] and acc.hi["out"] == sizes["out"]


@pytest.mark.parametrize("M, N", [(256, 256), (1000, 136), (131072, 3072), (497664, 4096), (2304, 1280)])
def test_gemm_tile_walk_covers_each_tile_once(M, N):
    m0, n0 = LM.gemm_tile_origins(M, N)
    mt, nt = LM.cdiv(M, 256), LM.cdiv(N, 256)
    key = (m0 // 256) * nt + n0 // 256
    assert m0.max() < mt * 256 and n0.max() < nt * 256
    assert np.array_equal(np.sort(key), np.arange(mt * nt))


@pytest.mark.parametrize("M, N, K", [(300, 136, 128), (1000, 1024, 4096), (64, 640, 1024)])
def test_gemm_ragged_shapes_touch_exactly_their_tensors(M, N, K):
    """Ragged M and N: the epilogue writes up to the last element and no further."""
    acc = LM.gemm_dma_launch(M, N, K, K, K, N, N, bias=True)
    sizes = LM.gemm_sizes(M, N, K, K, K, N, N, bias=True)
    assert acc.check(sizes) == []
    assert acc.lo["out"] == 0 and acc.hi["out"] == sizes["out"]
    assert acc.hi["x"] == sizes["x"] and acc.hi["w"] == sizes["w"] and acc.hi["bias"] == 2 * N


@pytest.mark.parametrize("M, N, K", [(300, 136, 80), (393216, 768, 80), (257, 520, 16), (64, 640, 200),
                                     (1000, 96, 1032)])
def test_gemm_ragged_k_touches_exactly_its_tensors(M, N, K):
    """K not a multiple of 64 (the rollout's patch embedding: K = 80): with row strides
    equal to K the masked last stage reads up to the last element of x and w and no
    further."""
    acc = LM.gemm_dma_launch(M, N, K, K, K, N, bias=True)
    sizes = LM.gemm_sizes(M, N, K, K, K, N, bias=True)
    assert acc.check(sizes) == []
    assert acc.hi["x"] == sizes["x"] and acc.hi["w"] == sizes["w"]


def test_planted_unmasked_k_tail_is_caught(monkeypatch):
    """The same launch with the last stage's K mask dropped reads past the end of x."""
    orig = LM._gemm_dma_offsets
    monkeypatch.setattr(LM, "_gemm_dma_offsets", lambda *a, **k: orig(*a[:6]))
    M, N, K = 300, 136, 80
    acc = LM.gemm_dma_launch(M, N, K, K, K, N, bias=True)
    assert acc.check(LM.gemm_sizes(M, N, K, K, K, N, bias=True)) != []


def test_planted_32bit_descriptor_is_caught():
    """A GEMM whose x stage used ONE descriptor for the whole matrix with the row
    offset folded into the 32-bit lane offset (the kernel instead moves the
    descriptor base to the tile's first row): at M = 497664, K = 4096 the lane
    offsets pass 2^32 and the check reports it."""
    M, K = 497664, 4096
    acc = LM.Access()
    m0, _ = LM.gemm_tile_origins(M, 1024)
    row = m0[:, None] + np.arange(256)[None, :]
    acc.lane_offsets("planted lane offset", row * K * 2)
    assert acc.bad32, "an allocation-wide 32-bit offset at this size must be flagged"
    ok = LM.Access()  # the kernel's scheme: per-tile base, lane offsets within 256 rows
    ok.lane_offsets("tile-relative lane offset", np.arange(256) * K * 2)
    assert not ok.bad32


def test_na3d_general_kernel_small_shapes_cover_their_outputs():
    """At a shape with clamped windows in every axis and ragged tiles, the modelled
    output stores reach the first and the last byte of the output and no further."""
    B, L, H, D = 1, (4, 20, 24), 2, 64
    tok = LM.contiguous_strides([B, *L, H, D])[:5]
    acc = LM.na3d_general_launch(B, L, H, (3, 5, 7), (1, 1, 1), tok, tok, tok, tok)
    n = 2 * B * L[0] * L[1] * L[2] * H * D
    assert acc.check({"q": n, "k": n, "v": n, "out": n}) == []
    assert acc.lo["out"] == 0 and acc.hi["out"] == n
    assert acc.hi["k"] == n and acc.hi["v"] == n


@pytest.mark.parametrize("Lz", list(range(1, 13)) + [16, 24, 25])
def test_region_z_walk_schedules_every_tile_once(Lz):
    """The region kernel's z walk (zlo / zhi closed forms, slot assignment, the interior
    mask and the extra pass) holds every live query z in a computed slot of its own, and
    each tile starts at its first slice and finishes at its last, for every query
    z-range the host admits; the host refuses exactly the sub-grids where five overlap."""
    if Lz < 3:
        return
    for z0 in range(Lz):
        for z1 in range(z0 + 1, Lz + 1):
            admitted = LM.region_fits_z(Lz, 1, z0, z1 - z0)
            probs = LM.region_z_walk(Lz, z0, z1)
            if admitted:
                assert probs == [], (Lz, z0, z1, probs)
    assert LM.region_fits_z(Lz, 1, 0, Lz) == (Lz != 5)


@pytest.mark.parametrize("case", [
    # B, L, H, ker, dil, org, ext, rope_zt, lse, v_in_qkv  (the host launches ky = 3; the
    # template's other windows are replayed too)
    (2, (8, 64, 64), 8, (3, 7, 7), (1, 1, 1), (0, 0, 0), None, 8, False, True),     # configs[1] (query RoPE)
    (4, (8, 64, 64), 16, (3, 7, 7), (1, 1, 1), (0, 0, 0), None, 1, False, True),    # configs[3] block
    (6, (16, 64, 64), 12, (3, 7, 7), (1, 1, 1), (0, 0, 0), None, None, True, True),  # configs[4] stage 1, lse
    (1, (24, 144, 144), 16, (3, 3, 3), (1, 1, 1), (0, 0, 0), None, 1, False, True),  # production tile
    (1, (7, 21, 27), 2, (3, 5, 5), (1, 1, 1), (0, 0, 0), None, None, True, False),   # ragged regions
    (2, (9, 30, 37), 3, (3, 7, 5), (2, 1, 2), (0, 0, 0), None, None, False, False),  # dilation
    (1, (8, 40, 48), 2, (3, 7, 7), (1, 1, 1), (2, 6, 5), (4, 21, 30), None, True, False),  # query box
    (1, (6, 17, 19), 1, (3, 3, 1), (1, 3, 1), (0, 0, 0), None, None, False, False),
])
def test_region_kernel_launches_stay_inside_their_tensors(case):
    B, L, H, ker, dil, org, ext, zt, lse, v_in_qkv = case
    D = 64
    C = H * D
    tok = LM.contiguous_strides([B, *L, H, D])[:5]
    vst = [L[0] * L[1] * L[2] * 3 * C, L[1] * L[2] * 3 * C, L[2] * 3 * C, 3 * C, D] if v_in_qkv else tok
    ext_ = tuple(L) if ext is None else ext
    ost = LM.contiguous_strides([B, *ext_, H, D])[:5]
    acc = LM.na3d_region_launch(B, L, H, ker, dil, tok, tok, vst, ost, org=org, ext=ext, rope_zt=zt, lse=lse)
    n = 2 * B * L[0] * L[1] * L[2] * C
    no = 2 * B * ext_[0] * ext_[1] * ext_[2] * C
    sizes = {"q": n, "k": n, "v": LM.span(n // (2 * C), 3 * C, 3 * C) - 4 * C if v_in_qkv else n, "out": no,
             "lse": 4 * B * ext_[0] * ext_[1] * ext_[2] * H}
    if zt is not None:
        sizes["cos"] = sizes["sin"] = 4 * B * zt * L[1] * L[2] * 32
    assert acc.check(sizes) == []
    assert acc.lo["out"] == 0 and acc.hi["out"] == no  # every output reached, nothing past it



@pytest.mark.parametrize("B, Z, Yc, Xc, C, f", [
    (6, 24, 16, 16, 1024, 4),   # the production pixel stage (cond at patch 4, upsampled x4)
    (1, 24, 16, 16, 64, 4),
    (2, 3, 5, 7, 32, 4),
    (1, 2, 9, 6, 16, 2),
    (1, 2, 6, 5, 8, 1),
    (1, 2, 1, 2, 8, 4),
    (1, 1, 2, 1, 16, 3),
    (1, 2, 70, 3, 24, 1),       # 3 channel groups: 85 columns per workgroup, rows wider than one
])
def test_upsample_dw_gelu_stays_inside_its_tensors(B, Z, Yc, Xc, C, f):
    """The upsampling kernel's staged coarse runs, LDS taps and stores, for the GPU test
    shapes, the production shape and a ragged channel count: every read inside the
    coarse tensor, every store covering exactly the output, every tap inside the stage."""
    cs = LM.contiguous_strides([B, Z, Yc, Xc, C])[:4]
    os_ = LM.contiguous_strides([B, Z, Yc * f, Xc * f, C])[:4]
    acc, lds = LM.upsample_dw_gelu_launch(B, Z, Yc, Xc, C, f, cs, os_)
    ncond, nout = 2 * B * Z * Yc * Xc * C, 2 * B * Z * Yc * f * Xc * f * C
    assert lds == []
    assert acc.check({"cond": ncond, "out": nout, "weight": 2 * 9 * C}) == []
    assert acc.lo["out"] == 0 and acc.hi["out"] == nout
