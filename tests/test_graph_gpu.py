"""The block forward captured as a HIP graph (torch.cuda.CUDAGraph): every replay, with eager
work and synchronisations between replays, reproduces the eager forward."""

import pytest
import torch

from strata_amd import rope as P
from strata_amd.modules import StrataBlock, init_xavier_

from .conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("gated,qk_norm,kernel", [(False, False, (3, 7, 7)), (True, True, (3, 3, 3))], ids=["plain", "gated-qknorm"])
def test_block_graph_replays_match_eager(gpu, gated, qk_norm, kernel):
    B, Z, Y, X, C, H = 1, 4, 16, 16, 1024, 16
    blk = StrataBlock(C, H, kernel, gated=gated, qk_norm=qk_norm)
    init_xavier_(blk, torch.Generator().manual_seed(1))
    blk = blk.to(gpu).bfloat16().eval()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, Z, Y, X, C, generator=g).bfloat16().to(gpu)
    lat, lon = P.synthetic_tile_latlon(B, Y, X, g)
    cos, sin = P.stereographic_rope_tables(lat, lon, C // H, 10000.0, P.default_rope_length_scale(1))
    rope = (cos.to(gpu), sin.to(gpu))
    with torch.no_grad():
        eager = blk(x, rope).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                blk(x, rope)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = blk(x, rope)
        for i in range(4):
            graph.replay()
            torch.cuda.synchronize()
            got = out.clone()
            assert torch.isfinite(got.float()).all(), i
            assert rel_l2(got.float(), eager.float()) <= 1e-3, i
            again = blk(x, rope)  # eager work between replays
            torch.cuda.synchronize()
            assert rel_l2(again.float(), eager.float()) <= 1e-3, i
