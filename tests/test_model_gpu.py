"""The two-stage model (configs[4] structure, reduced sizes) through the HIP
library vs the fp32 CPU oracle, one step and a 2-step rollout."""

import pytest
import torch

from oracle import block as OB
from oracle import rope as R
from strata_amd import rope as P
from strata_amd.model import TwoStageStrata
from strata_amd.modules import init_xavier_

from .conftest import rel_l2

pytestmark = pytest.mark.gpu

CFG = dict(in_channels=16, dim1=128, heads1=2, depth1=2, kernel1=(3, 5, 5), dim2=256, heads2=4, depth2=2,
           kernel2=(1, 5, 5))


def _setup(gpu):
    torch.manual_seed(0)
    model = TwoStageStrata(**CFG)
    init_xavier_(model, torch.Generator().manual_seed(1))
    params = {k: v.detach().bfloat16().float() for k, v in model.state_dict().items()}
    model = model.to(gpu).bfloat16()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 16, 4, 16, 16, generator=g).bfloat16()
    lat, lon = P.synthetic_tile_latlon(1, 16, 16, g)
    rope1, rope2 = model.rope_tables(lat.to(gpu), lon.to(gpu))
    c1, s1 = R.tables(lat, lon, 64, 10000.0, R.default_rope_length_scale(1))
    lat2, lon2 = R.pooled_latlon(lat, lon)
    c2, s2 = R.tables(lat2, lon2, 64, 10000.0, R.default_rope_length_scale(2))
    ocfg = dict(depth1=2, heads1=2, kernel1=(3, 5, 5), depth2=2, heads2=4, kernel2=(1, 5, 5))
    return model, params, x, (rope1, rope2), ((c1.float(), s1.float()), (c2.float(), s2.float())), ocfg


def test_stage_tables_match_oracle(gpu):
    model, params, x, (r1, r2), (o1, o2), _ = _setup(gpu)
    assert (r2[0].cpu().double() - o2[0].double()).abs().max() < 1e-5
    assert (r1[1].cpu().double() - o1[1].double()).abs().max() < 1e-5


def test_two_stage_step(gpu):
    model, params, x, (r1, r2), (o1, o2), ocfg = _setup(gpu)
    with torch.no_grad():
        out = model(x.to(gpu), r1, r2)
    ref = OB.two_stage_forward(x.float(), params, ocfg, o1, o2)
    assert out.shape == x.shape
    assert rel_l2(out.float(), ref) <= 1e-2


def test_two_stage_rollout(gpu):
    model, params, x, (r1, r2), (o1, o2), ocfg = _setup(gpu)
    y = model.rollout(x.to(gpu), 2, r1, r2)
    ref = x.float()
    for _ in range(2):
        ref = ref + OB.two_stage_forward(ref, params, ocfg, o1, o2)
    assert rel_l2(y.float(), ref) <= 1e-2
