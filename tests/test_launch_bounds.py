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


def test_production_tile_reaches_past_2gib():
    """The replay does reach the large offsets: qkv's last row lies beyond 2^31 bytes,
    fc1's output beyond 4 * 10^9."""
    B, Z, Y, X, C, H, kernel = 1, 24, 144, 144, 1024, 16, (3, 3, 3)
    launches = {n: (a, s) for n, a, s in LM.production_block_launches(B, Z, Y, X, C, H, kernel)}
    acc, sizes = launches["qkv gemm"]
    assert acc.hi["out"] == sizes["out"] > 2**31
    acc, sizes = launches["fc1 gemm + gelu"]
    assert acc.hi["out"] == sizes["out"] > 4 * 10**9
    acc, sizes = launches["na3d (general kernel)"]
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
