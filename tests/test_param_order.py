"""State-dict keys and parameter registration order of the drop-in modules against
the reference's committed manifests (CPU, no GPU).

The manifests (tests/golden/param_order/, copied by
tests/golden/copy_param_order.py from the reference's
tests/regression_data/*.param_order.txt) are what the reference's own
tests/test_param_order.py:87-119 freezes: checkpoints (screamcast/checkpoint_compat.py)
and index-mapped optimizer states depend on exactly these names in exactly this
order.  Here:
  * a ``StrataBlock(gated=True)`` registers the manifest's per-block names, in
    order, for every one of the 32 production blocks;
  * a module tree built name by name from the manifest, with reference-shaped
    attention (qkv / proj / gate_proj Linears) and Mlp (layers = Linear, GELU,
    Linear) modules, keeps its full ``named_parameters()`` list unchanged through
    ``swap_attention`` + ``swap_mlps``, and every swapped module shares the
    original parameters.
"""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch
import torch.nn as nn

from strata_amd.modules import (FusedNA3DAttention, GemmGeluMlp, StrataBlock, StrataPixelBlock, swap_attention,
                                swap_mlps)

from .conftest import GOLDEN

MANIFESTS = GOLDEN / "param_order"
SWEEP1 = MANIFESTS / "sweep1_nodilation_gated_tile64_kernel3_lr1em4_dim1024_hpatch4_depth32_r3_cos.param_order.txt"
PIXELDIT = MANIFESTS / "pixeldit_sem1024d24l_pix128d4l_bilineardwgeluproject_unfreeze_3src_const1em5_t128.param_order.txt"


def _names(path: Path) -> list[str]:
    return path.read_text().splitlines()


def _block_names(names: list[str], prefix: str, i: int) -> list[str]:
    p = f"{prefix}.{i}."
    return [n[len(p):] for n in names if n.startswith(p)]


def test_manifests_are_the_production_shapes():
    s = _names(SWEEP1)
    assert len(s) == 324 and s[0] == "strata.patch_embed.proj.weight" and s[-1] == "strata.final_layer.linear.bias"
    blocks = {int(m.group(1)) for n in s if (m := re.match(r"strata\.blocks\.(\d+)\.", n))}
    assert blocks == set(range(32))


def test_strata_block_matches_every_production_block():
    blk = StrataBlock(64, 4, (3, 3, 3), gated=True)  # names do not depend on the width
    got = [n for n, _ in blk.named_parameters()]
    s = _names(SWEEP1)
    for i in range(32):
        assert got == _block_names(s, "strata.blocks", i), i
    # and the backbone blocks of the two-stage production model
    p = _names(PIXELDIT)
    ungated = [n for n, _ in StrataBlock(64, 4, (3, 3, 3)).named_parameters()]
    for i in range(24):
        want = _block_names(p, "strata.backbone.blocks", i)
        assert want in (got, ungated), (i, want)


def test_pixel_block_matches_every_production_pixel_block():
    """The pixel-stage block registers the manifest's per-block names in order (its
    two adaLN modules after the attention and the MLP) for the four production blocks."""
    blk = StrataPixelBlock(128, 2, (3, 9, 9), cond_dim=64, factor=4)
    got = [n for n, _ in blk.named_parameters()]
    p = _names(PIXELDIT)
    for i in range(4):
        assert got == _block_names(p, "strata.pixel_blocks", i), i
    shapes = dict((n, tuple(t.shape)) for n, t in blk.named_parameters())
    assert shapes["adaln_bilinear_dw_conv.weight"] == (64, 1, 1, 3, 3)
    assert shapes["adaln_bilinear_dw_proj.weight"] == (6 * 128, 64)


class _RefAttention(nn.Module):
    """Reference-shaped attention: qkv, proj, gate_proj Linears (manifest order)."""

    def __init__(self, dim: int, gated: bool):
        super().__init__()
        self.qkv = nn.Linear(dim, 3 * dim)
        self.proj = nn.Linear(dim, dim)
        if gated:
            self.gate_proj = nn.Linear(dim, dim)


class _RefMlp(nn.Module):
    def __init__(self, dim: int):
        super().__init__()
        self.layers = nn.Sequential(nn.Linear(dim, 4 * dim), nn.GELU(), nn.Linear(4 * dim, dim))


def _tree_from_manifest(names: list[str], dim: int = 16) -> nn.Module:
    """A module tree whose named_parameters() are the manifest's names, with the
    reference's attention and Mlp shapes under every ``*.attn`` / ``*.mlp``."""
    root = nn.Module()

    def node(path: list[str]) -> nn.Module:
        m = root
        for part in path:
            if not hasattr(m, part) or getattr(m, part) is None:
                m.add_module(part, nn.Module())
            m = getattr(m, part)
        return m

    seen = set()
    for n in names:
        parts = n.split(".")
        if "attn" in parts:
            k = parts.index("attn")
            key = ".".join(parts[: k + 1])
            if key not in seen:
                seen.add(key)
                gated = f"{key}.gate_proj.weight" in names
                node(parts[:k]).add_module("attn", _RefAttention(dim, gated))
        elif "mlp" in parts:
            k = parts.index("mlp")
            key = ".".join(parts[: k + 1])
            if key not in seen:
                seen.add(key)
                node(parts[:k]).add_module("mlp", _RefMlp(dim))
        else:
            owner = node(parts[:-2])
            leaf = parts[-2]
            if not hasattr(owner, leaf):
                owner.add_module(leaf, nn.Linear(dim, dim))
    return root


@pytest.mark.parametrize("path", [SWEEP1], ids=["sweep1"])
def test_swaps_keep_keys_and_order(path):
    names = _names(path)
    model = _tree_from_manifest(names)
    assert [n for n, _ in model.named_parameters()] == names  # the stand-in tree is faithful
    before = dict(model.named_parameters())
    n_att = swap_attention(model.strata, num_heads=4, kernel_size=3, qk_norm=True)
    n_mlp = swap_mlps(model.strata)
    assert n_att == 32 and n_mlp == 32
    after = list(model.named_parameters())
    assert [n for n, _ in after] == names
    assert all(p is before[n] for n, p in after)  # shared, not copied
    assert list(model.state_dict().keys()) == names
    for blk in model.strata.blocks.children():
        assert isinstance(blk.attn, FusedNA3DAttention) and blk.attn.gate_proj is not None
        assert blk.attn.qk_norm and blk.attn.q_norm is None  # non-affine qk-norm: no parameters
        assert isinstance(blk.mlp, GemmGeluMlp)


def test_swap_attention_per_block_schedule_and_errors():
    names = _names(SWEEP1)
    model = _tree_from_manifest(names)
    sched = [(1, 1, 1) if i % 2 == 0 else (1, 3, 3) for i in range(32)]
    swap_attention(model.strata, 4, (3, 3, 3), dilation=sched)
    assert [b.attn.dilation for b in model.strata.blocks.children()][:3] == [[1, 1, 1], [1, 3, 3], [1, 1, 1]]
    with pytest.raises(RuntimeError, match="no module"):
        swap_attention(model.strata, 4, 3)  # nothing left to swap
    with pytest.raises(ValueError, match="per-module"):
        swap_attention(_tree_from_manifest(names).strata, 4, 3, dilation=[(1, 1, 1)] * 3 + [(1, 2, 2)])

    class _Odd(_RefAttention):
        def __init__(self):
            super().__init__(16, False)
            self.rel_bias = nn.Linear(4, 4)  # a parameterised child of unknown role

    holder = nn.Module()
    holder.attn = _Odd()
    with pytest.raises(TypeError, match="rel_bias"):
        swap_attention(holder, 4, 3)


def test_swapped_attention_keeps_an_affine_qk_norm():
    class _Att(_RefAttention):
        def __init__(self):
            super().__init__(16, True)
            self.q_norm = nn.RMSNorm(4)
            self.k_norm = nn.RMSNorm(4)

    holder = nn.Module()
    holder.attn = _Att()
    names = [n for n, _ in holder.named_parameters()]
    swap_attention(holder, 4, 3, qk_norm=True)
    assert [n for n, _ in holder.named_parameters()] == names
    assert holder.attn.q_norm is not None and holder.attn.q_norm.weight.shape == (4,)
    assert holder.attn.head_dim == 4 and torch.equal(holder.attn.qkv.weight, holder.attn.qkv.weight)


def test_interleaved_dilation_schedule():
    from strata_amd.modules import interleaved_dilations

    assert interleaved_dilations(4, 3, 3, (24, 16, 16), interleaved=False) == [[1, 1, 1]] * 4
    s = interleaved_dilations(4, 3, (3, 5, 5), (8, 16, 16))
    assert s[0] == s[2] == [1, 1, 1] and s[1] == s[3] == [1, 3, 3]  # 3*3 > 8 keeps z undilated
    assert interleaved_dilations(3, 3, 3, (24, 144, 144))[1] == [3, 3, 3]


def test_alternating_depthwise_schedule_keeps_keys_and_order():
    """The production flags (gated, qk-norm, do_alt_depthwise_attn): odd blocks attend their
    z column (window (Z, 1, 1) of the input's Z), even blocks keep (3, 3, 3); the manifest's
    keys, order and parameter objects are unchanged."""
    from strata_amd.modules import alternating_depthwise

    assert alternating_depthwise(4) == [False, True, False, True]
    assert alternating_depthwise(3, alternate=False) == [False] * 3
    names = _names(SWEEP1)
    model = _tree_from_manifest(names)
    before = dict(model.named_parameters())
    swap_attention(model.strata, 4, 3, qk_norm=True, depthwise=alternating_depthwise(32))
    after = list(model.named_parameters())
    assert [n for n, _ in after] == names and all(p is before[n] for n, p in after)
    blocks = list(model.strata.blocks.children())
    assert [b.attn.depthwise for b in blocks[:4]] == [False, True, False, True]
    assert blocks[0].attn.window(24) == ([3, 3, 3], [1, 1, 1])
    assert blocks[1].attn.window(24) == ([24, 1, 1], [1, 1, 1])
