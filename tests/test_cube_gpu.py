"""Cube-sphere halo fill and crop on the GPU vs the CPU oracle (bit-exact: a
gather, plus the corner means computed in the tensor's own dtype)."""

import pytest
import torch

from oracle import cube
from strata_amd import ops  # noqa: F401

pytestmark = pytest.mark.gpu

CASES = [
    # lead dims, n, p, dtype
    ((1,), 8, 3, torch.float32),
    ((2, 3), 9, 4, torch.float32),
    ((1,), 5, 5, torch.float32),     # pad = n: the whole neighbour face
    ((3,), 16, 1, torch.bfloat16),
    ((2,), 33, 7, torch.bfloat16),   # ragged size
    ((4,), 512, 32, torch.float32),  # rollout geometry: 512-px tile, 32-px halo
]


@pytest.mark.parametrize("lead,n,p,dtype", CASES, ids=[f"{c[0]}-{c[1]}-{c[2]}-{str(c[3])[6:]}" for c in CASES])
def test_pad_faces_matches_oracle(gpu, lead, n, p, dtype):
    print(f"cube pad {lead} n={n} p={p} {dtype}", flush=True)
    g = torch.Generator().manual_seed(n + p)
    data = torch.randn(*lead, 6, n, n, generator=g).to(dtype)
    got = torch.ops.strata_hip.cube_pad_faces(data.to(gpu), p).cpu()
    ref = cube.pad_faces(data, p)
    assert got.shape == ref.shape
    assert torch.equal(got, ref)
    back = torch.ops.strata_hip.cube_crop(got.to(gpu), p).cpu()
    assert torch.equal(back, data)


def test_crop_matches_oracle_on_tiles(gpu):
    """TileTopology.crop of padded tiles [B, tiles, S, S] with a halo narrower than the pad."""
    x = torch.randn(2, 7, 40, 40, dtype=torch.float32)
    for h in (0, 3, 19):
        got = torch.ops.strata_hip.cube_crop(x.to(gpu), h).cpu()
        assert torch.equal(got, cube.crop(x, h))


def test_pad_zero_is_identity(gpu):
    x = torch.randn(1, 6, 4, 4, dtype=torch.bfloat16).to(gpu)
    assert torch.equal(torch.ops.strata_hip.cube_pad_faces(x, 0), x)
