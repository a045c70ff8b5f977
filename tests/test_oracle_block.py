"""Pins for the block oracle's qk RMSNorm (CPU, float64)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import block as OB


def test_rms_norm_matches_torch_and_closed_forms():
    g = torch.Generator().manual_seed(0)
    t = torch.randn(5, 7, 64, generator=g, dtype=torch.float64) * 3
    w = 1 + 0.2 * torch.randn(64, generator=g, dtype=torch.float64)
    # torch's own routine
    assert torch.allclose(OB.rms_norm(t, 1e-6, w), F.rms_norm(t, (64,), w, 1e-6), atol=1e-12)
    # unit RMS without weights (eps -> 0), scale invariance, constant vectors -> +-1
    y = OB.rms_norm(t, 0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(5, 7, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(OB.rms_norm(7.5 * t, 0.0), y, atol=1e-12)
    c = torch.full((3, 64), -2.5, dtype=torch.float64)
    assert torch.allclose(OB.rms_norm(c, 0.0), -torch.ones_like(c))


def test_rms_norm_is_the_first_step_of_the_qk_norm_block():
    """With qk_norm the oracle block differs from the plain block: a planted
    no-op normalisation (the flag ignored) would fail here."""
    g = torch.Generator().manual_seed(1)
    C, H = 32, 2
    params = {
        "attn.qkv.weight": torch.randn(3 * C, C, generator=g) * C**-0.5,
        "attn.qkv.bias": torch.zeros(3 * C),
        "attn.proj.weight": torch.randn(C, C, generator=g) * C**-0.5,
        "attn.proj.bias": torch.zeros(C),
        "mlp.layers.0.weight": torch.randn(4 * C, C, generator=g) * C**-0.5,
        "mlp.layers.0.bias": torch.zeros(4 * C),
        "mlp.layers.2.weight": torch.randn(C, 4 * C, generator=g) * (4 * C) ** -0.5,
        "mlp.layers.2.bias": torch.zeros(C),
    }
    x = torch.randn(1, 3, 5, 5, C, generator=g)
    a = OB.block_forward(x, params, H, (3, 3, 3), None, None)
    b = OB.block_forward(x, params, H, (3, 3, 3), None, None, qk_norm=True)
    assert (a - b).abs().max() > 1e-3


# ---------------------------------------------------------------------------
# Composition pins: the block and the two-stage model against independent
# constructions from torch's own modules (nn.LayerNorm, nn.MultiheadAttention,
# nn.Conv3d, nn.ConvTranspose3d).  A mistake in the residual source, the LN
# placement, the qkv column order / head split, the merge or head channel order
# fails one of these.
# ---------------------------------------------------------------------------

def _block_params(C: int, g: torch.Generator, gated: bool = False, scale: float = 1.0) -> dict:
    def lin(o, i):
        return torch.randn(o, i, generator=g, dtype=torch.float64) * (scale * i**-0.5)

    def b(n):
        return torch.randn(n, generator=g, dtype=torch.float64) * 0.1

    p = {"attn.qkv.weight": lin(3 * C, C), "attn.qkv.bias": b(3 * C),
         "attn.proj.weight": lin(C, C), "attn.proj.bias": b(C)}
    if gated:
        p.update({"attn.gate_proj.weight": lin(C, C), "attn.gate_proj.bias": b(C)})
    p.update({"mlp.layers.0.weight": lin(4 * C, C), "mlp.layers.0.bias": b(4 * C),
              "mlp.layers.2.weight": lin(C, 4 * C), "mlp.layers.2.bias": b(C)})
    return p


class _TorchBlock(torch.nn.Module):
    """Pre-norm block from torch modules; attention over all tokens (dense)."""

    def __init__(self, p: dict, C: int, H: int, gated: bool = False, eps: float = 1e-6):
        super().__init__()
        nn = torch.nn
        self.ln1 = nn.LayerNorm(C, eps=eps, elementwise_affine=False, dtype=torch.float64)
        self.ln2 = nn.LayerNorm(C, eps=eps, elementwise_affine=False, dtype=torch.float64)
        self.mha = nn.MultiheadAttention(C, H, batch_first=True, dtype=torch.float64)
        self.mlp = nn.Sequential(nn.Linear(C, 4 * C, dtype=torch.float64), nn.GELU(approximate="tanh"),
                                 nn.Linear(4 * C, C, dtype=torch.float64))
        self.gate = nn.Linear(C, C, dtype=torch.float64) if gated else None
        with torch.no_grad():
            self.mha.in_proj_weight.copy_(p["attn.qkv.weight"])
            self.mha.in_proj_bias.copy_(p["attn.qkv.bias"])
            self.mha.out_proj.weight.copy_(p["attn.proj.weight"])
            self.mha.out_proj.bias.copy_(p["attn.proj.bias"])
            self.mlp[0].weight.copy_(p["mlp.layers.0.weight"])
            self.mlp[0].bias.copy_(p["mlp.layers.0.bias"])
            self.mlp[2].weight.copy_(p["mlp.layers.2.weight"])
            self.mlp[2].bias.copy_(p["mlp.layers.2.bias"])
            if gated:
                self.gate.weight.copy_(p["attn.gate_proj.weight"])
                self.gate.bias.copy_(p["attn.gate_proj.bias"])

    def forward(self, x):  # [B, Z, Y, X, C]
        B, Z, Y, X, C = x.shape
        t = x.reshape(B, Z * Y * X, C)
        h = self.ln1(t)
        if self.gate is None:
            a, _ = self.mha(h, h, h, need_weights=False)
        else:  # gate before the output projection: a * sigmoid(gate_proj(h)), then proj
            nn_f = torch.nn.functional
            q, k, v = nn_f.linear(h, self.mha.in_proj_weight, self.mha.in_proj_bias).chunk(3, dim=-1)
            Hh = self.mha.num_heads
            sh = lambda u: u.view(B, -1, Hh, C // Hh).transpose(1, 2)  # noqa: E731
            o = nn_f.scaled_dot_product_attention(sh(q), sh(k), sh(v)).transpose(1, 2).reshape(B, -1, C)
            a = self.mha.out_proj(o * torch.sigmoid(self.gate(h)))
        t = t + a
        t = t + self.mlp(self.ln2(t))
        return t.view(B, Z, Y, X, C)


def test_block_zero_output_weights_is_identity():
    g = torch.Generator().manual_seed(2)
    C, H = 32, 2
    p = _block_params(C, g, gated=True)
    for k in ("attn.proj.weight", "attn.proj.bias", "mlp.layers.2.weight", "mlp.layers.2.bias"):
        p[k] = torch.zeros_like(p[k])
    x = torch.randn(2, 3, 5, 6, C, generator=g, dtype=torch.float64)
    for gated in (False, True):
        y = OB.block_forward(x, p, H, (3, 3, 5), None, None, gated=gated, dtype=torch.float64)
        assert torch.equal(y, x)


def test_block_dense_window_equals_torch_modules():
    """kernel == grid: NA3D is full attention, so the oracle block must equal a
    block assembled from nn.LayerNorm + nn.MultiheadAttention (qkv in_proj in its
    (q, k, v) x (head, dim) column order, proj as out_proj) + the Mlp."""
    g = torch.Generator().manual_seed(3)
    C, H = 48, 3
    for gated in (False, True):
        p = _block_params(C, g, gated=gated, scale=2.0)
        x = torch.randn(2, 3, 5, 5, C, generator=g, dtype=torch.float64) * 2 + 0.5
        y = OB.block_forward(x, p, H, (3, 5, 5), None, None, gated=gated, dtype=torch.float64)
        ref = _TorchBlock(p, C, H, gated=gated)(x)
        assert (y - ref).abs().max() < 1e-10, gated


def test_block_unit_window_reduces_to_value_path():
    """kernel (1,1,1): each query sees only its own key, attention returns v, so the
    block is a per-token map; evaluated token by token with the torch modules'
    value projection (rows 2C:3C of the in_proj)."""
    g = torch.Generator().manual_seed(4)
    C, H = 32, 4
    p = _block_params(C, g)
    x = torch.randn(1, 2, 3, 4, C, generator=g, dtype=torch.float64)
    y = OB.block_forward(x, p, H, (1, 1, 1), None, None, dtype=torch.float64)
    tb = _TorchBlock(p, C, H)
    for idx in [(0, 0, 0, 0), (0, 1, 2, 3), (0, 1, 0, 2)]:
        t = x[idx]
        h = tb.ln1(t)
        v = h @ p["attn.qkv.weight"][2 * C:].T + p["attn.qkv.bias"][2 * C:]
        t = t + tb.mha.out_proj(v)
        t = t + tb.mlp(tb.ln2(t))
        assert (y[idx] - t).abs().max() < 1e-12, idx


def test_space_to_depth_channel_order_and_inverse():
    g = torch.Generator().manual_seed(5)
    B, Z, Y, X, C = 2, 4, 6, 8, 3
    x = torch.randn(B, Z, Y, X, C, generator=g, dtype=torch.float64)
    s = OB.space_to_depth(x)
    assert s.shape == (B, Z // 2, Y // 2, X // 2, 8 * C)
    for (b, z, y, xx) in [(0, 0, 0, 0), (1, 1, 2, 3), (0, 1, 1, 2)]:
        for dz in range(2):
            for dy in range(2):
                for dx in range(2):
                    ch = ((dz * 2 + dy) * 2 + dx) * C
                    assert torch.equal(s[b, z, y, xx, ch:ch + C], x[b, 2 * z + dz, 2 * y + dy, 2 * xx + dx])
    assert torch.equal(OB.depth_to_space(s, C), x)
    # the product model's helpers are the same maps
    from strata_amd import model as M

    assert torch.equal(M.space_to_depth(x), s)
    assert torch.equal(M.depth_to_space(s, C), x)


def _two_stage_params(g, cin, d1, d2, depth1, depth2):
    p = {"embed.weight": torch.randn(d1, cin, generator=g, dtype=torch.float64) * cin**-0.5,
         "embed.bias": torch.randn(d1, generator=g, dtype=torch.float64) * 0.1,
         "merge.weight": torch.randn(d2, 8 * d1, generator=g, dtype=torch.float64) * (8 * d1) ** -0.5,
         "merge.bias": torch.randn(d2, generator=g, dtype=torch.float64) * 0.1,
         "head.weight": torch.randn(8 * cin, d2, generator=g, dtype=torch.float64) * d2**-0.5,
         "head.bias": torch.randn(8 * cin, generator=g, dtype=torch.float64) * 0.1}
    for i in range(depth1):
        p.update({f"stage1.{i}.{k}": v for k, v in _block_params(d1, g).items()})
    for i in range(depth2):
        p.update({f"stage2.{i}.{k}": v for k, v in _block_params(d2, g).items()})
    return p


def test_two_stage_zero_head_gives_zero_tendency():
    g = torch.Generator().manual_seed(6)
    cin, d1, d2 = 4, 16, 32
    p = _two_stage_params(g, cin, d1, d2, 1, 1)
    p["head.weight"].zero_()
    p["head.bias"].zero_()
    cfg = dict(depth1=1, heads1=2, kernel1=(1, 3, 3), depth2=1, heads2=2, kernel2=(1, 1, 1))
    x = torch.randn(1, cin, 2, 6, 6, generator=g, dtype=torch.float64)
    y = OB.two_stage_forward(x, p, cfg, (None, None), (None, None), dtype=torch.float64)
    assert y.shape == x.shape and torch.equal(y, torch.zeros_like(x))


def test_two_stage_equals_conv_construction():
    """Embed = 1x1x1 Conv3d, merge = 2x2x2 stride-2 Conv3d over (dz, dy, dx, c)
    channels, head = LayerNorm + 2x2x2 stride-2 ConvTranspose3d plus the bias of
    each (dz, dy, dx, c) output.  Stage 1 uses kernel (1,1,1) (attention returns v:
    the torch-module block with its value path) and stage 2 a dense window (the
    torch-module block with nn.MultiheadAttention)."""
    g = torch.Generator().manual_seed(7)
    cin, d1, d2, h1, h2 = 3, 16, 24, 2, 3
    p = _two_stage_params(g, cin, d1, d2, 1, 1)
    cfg = dict(depth1=1, heads1=h1, kernel1=(1, 1, 1), depth2=1, heads2=h2, kernel2=(3, 5, 5))
    x = torch.randn(2, cin, 6, 10, 10, generator=g, dtype=torch.float64)  # stage 2 grid (3, 5, 5)
    y = OB.two_stage_forward(x, p, cfg, (None, None), (None, None), dtype=torch.float64)

    F_ = torch.nn.functional
    sub = lambda pre: {k[len(pre):]: v for k, v in p.items() if k.startswith(pre)}  # noqa: E731
    e = F_.conv3d(x, p["embed.weight"].view(d1, cin, 1, 1, 1), p["embed.bias"]).permute(0, 2, 3, 4, 1)
    p1 = sub("stage1.0.")
    tb1 = _TorchBlock(p1, d1, h1)
    t = e + tb1.mha.out_proj(tb1.ln1(e) @ p1["attn.qkv.weight"][2 * d1:].T + p1["attn.qkv.bias"][2 * d1:])
    t = t + tb1.mlp(tb1.ln2(t))
    wm = p["merge.weight"].view(d2, 2, 2, 2, d1).permute(0, 4, 1, 2, 3)
    m = F_.conv3d(t.permute(0, 4, 1, 2, 3), wm, p["merge.bias"], stride=2).permute(0, 2, 3, 4, 1)
    h = _TorchBlock(sub("stage2.0."), d2, h2)(m)
    hn = F_.layer_norm(h, (d2,), eps=1e-6).permute(0, 4, 1, 2, 3)
    wh = p["head.weight"].view(2, 2, 2, cin, d2).permute(4, 3, 0, 1, 2)
    ref = F_.conv_transpose3d(hn, wh, None, stride=2)
    bias = p["head.bias"].view(2, 2, 2, cin).permute(3, 0, 1, 2)  # [cin, dz, dy, dx]
    ref = ref + bias.repeat(1, x.shape[2] // 2, x.shape[3] // 2, x.shape[4] // 2)[None]
    assert (y - ref).abs().max() < 1e-10


def test_planted_composition_mistakes_fail_the_pins():
    """Each plausible composition mistake, planted in a copy of the oracle block
    module, fails at least one of the pins above (so they pin something)."""
    import types
    from pathlib import Path

    global OB
    real = OB
    src = Path(real.__file__).read_text()
    plants = {
        "residual from the normed input": (
            'x = x + F.linear(a, p["attn.proj.weight"], p["attn.proj.bias"])',
            'x = h + F.linear(a, p["attn.proj.weight"], p["attn.proj.bias"])'),
        "second LayerNorm skipped": ("    h = F.layer_norm(x, (C,), eps=eps)\n    f = F.gelu", "    f = F.gelu"),
        "qkv columns read as (H, D, 3)": (
            ".view(B, Z, Y, X, 3, heads, D)\n    q, k, v = qkv.unbind(dim=4)",
            ".view(B, Z, Y, X, heads, D, 3)\n    q, k, v = qkv.unbind(dim=6)"),
        "merge channels (dx, dy, dz, c)": (
            "permute(0, 1, 3, 5, 2, 4, 6, 7)", "permute(0, 1, 3, 5, 6, 4, 2, 7)"),
        "gate after the projection": (
            '    x = x + F.linear(a, p["attn.proj.weight"], p["attn.proj.bias"])',
            '    x = x + F.linear(a, p["attn.proj.weight"], p["attn.proj.bias"]) * (torch.sigmoid('
            'F.linear(h, p["attn.gate_proj.weight"], p["attn.gate_proj.bias"])) if gated else 1)'),
    }
    pins = [test_block_zero_output_weights_is_identity, test_block_dense_window_equals_torch_modules,
            test_block_unit_window_reduces_to_value_path, test_space_to_depth_channel_order_and_inverse,
            test_two_stage_equals_conv_construction]
    try:
        for name, (a, b) in plants.items():
            assert src.count(a) == 1, name
            mod = types.ModuleType("oracle.block")
            mod.__package__ = "oracle"
            exec(compile(src.replace(a, b), f"<planted: {name}>", "exec"), mod.__dict__)
            OB = mod
            caught = 0
            for pin in pins:
                try:
                    pin()
                except AssertionError:
                    caught += 1
            assert caught > 0, f"planted mistake not caught: {name}"
    finally:
        OB = real


# ---------------------------------------------------------------------------
# Pixel-stage block (this build's convention): its parts are pinned against torch's
# own interpolate / conv3d / layer_norm, its composition against the plain block.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape, factor", [((1, 2, 3, 5, 4), 4), ((2, 1, 4, 4, 8), 2), ((1, 3, 1, 2, 3), 3),
                                           ((1, 1, 5, 3, 2), 1)])
def test_upsample_dw_gelu_is_interpolate_then_depthwise_conv(shape, factor):
    g = torch.Generator().manual_seed(sum(shape) + factor)
    C = shape[-1]
    cond, w, b = torch.randn(shape, generator=g), torch.randn(C, 1, 1, 3, 3, generator=g), torch.randn(C, generator=g)
    out = OB.upsample_dw_gelu(cond, w, b, factor)
    c5 = cond.double().permute(0, 4, 1, 2, 3)
    up = F.interpolate(c5, scale_factor=(1, factor, factor), mode="trilinear", align_corners=False)
    ref = F.gelu(F.conv3d(up, w.double(), b.double(), padding=(0, 1, 1), groups=C), approximate="tanh")
    assert torch.allclose(out, ref.permute(0, 2, 3, 4, 1), atol=1e-12)


def test_bilinear_index_closed_forms():
    """Factor 2 over 3 inputs: outputs 0, 1 sit on input 0 (clamped) and at 0.25; the last
    output sits at 2.25 -> index pair (2, 2) (the edge repeats)."""
    i0, i1, w = OB.bilinear_index(6, 3, 2)
    assert i0.tolist() == [0, 0, 0, 1, 1, 2] and i1.tolist() == [1, 1, 1, 2, 2, 2]
    assert torch.allclose(w, torch.tensor([0.0, 0.25, 0.75, 0.25, 0.75, 0.25], dtype=torch.float64))


def _pixel_params(C, Cs, heads, g, zero_proj=False, gate_one=False):
    p = {
        "attn.qkv.weight": torch.randn(3 * C, C, generator=g) / C**0.5, "attn.qkv.bias": torch.randn(3 * C, generator=g),
        "attn.proj.weight": torch.randn(C, C, generator=g) / C**0.5, "attn.proj.bias": torch.randn(C, generator=g),
        "mlp.layers.0.weight": torch.randn(4 * C, C, generator=g) / C**0.5,
        "mlp.layers.0.bias": torch.randn(4 * C, generator=g),
        "mlp.layers.2.weight": torch.randn(C, 4 * C, generator=g) / (4 * C)**0.5,
        "mlp.layers.2.bias": torch.randn(C, generator=g),
        "adaln_bilinear_dw_conv.weight": torch.randn(Cs, 1, 1, 3, 3, generator=g),
        "adaln_bilinear_dw_conv.bias": torch.randn(Cs, generator=g),
        "adaln_bilinear_dw_proj.weight": torch.randn(6 * C, Cs, generator=g) / Cs**0.5,
        "adaln_bilinear_dw_proj.bias": torch.randn(6 * C, generator=g),
    }
    if zero_proj or gate_one:
        p["adaln_bilinear_dw_proj.weight"] = torch.zeros(6 * C, Cs)
        p["adaln_bilinear_dw_proj.bias"] = torch.zeros(6 * C)
    if gate_one:  # shift = scale = 0, gate = 1: the plain pre-norm block
        p["adaln_bilinear_dw_proj.bias"][2 * C:3 * C] = 1.0
        p["adaln_bilinear_dw_proj.bias"][5 * C:6 * C] = 1.0
    return p


def test_pixel_block_zero_modulation_is_identity():
    """adaLN-Zero: a zero projection gives zero gates, so the block returns x."""
    g = torch.Generator().manual_seed(1)
    C, Cs, heads = 16, 8, 2
    x, cond = torch.randn(1, 3, 8, 8, C, generator=g), torch.randn(1, 3, 2, 2, Cs, generator=g)
    out = OB.pixel_block_forward(x, cond, _pixel_params(C, Cs, heads, g, zero_proj=True), heads, (3, 3, 3), 4)
    assert torch.equal(out, x.double())


def test_pixel_block_unit_gates_are_the_plain_block():
    """shift = scale = 0 and gate = 1 everywhere: the pixel block is block_forward."""
    g = torch.Generator().manual_seed(2)
    C, Cs, heads = 16, 8, 2
    x, cond = torch.randn(1, 3, 8, 8, C, generator=g), torch.randn(1, 3, 2, 2, Cs, generator=g)
    p = _pixel_params(C, Cs, heads, g, gate_one=True)
    out = OB.pixel_block_forward(x, cond, p, heads, (3, 3, 3), 4)
    ref = OB.block_forward(x, p, heads, (3, 3, 3), None, None, dtype=torch.float64)
    assert torch.allclose(out, ref, atol=1e-10)


def test_pixel_block_planted_chunk_order_fails_the_unit_gate_pin():
    """A restatement that takes the gates from the shift chunks (a plausible misreading of
    the six-way split) leaves x unchanged under unit gates, failing the plain-block pin."""
    g = torch.Generator().manual_seed(3)
    C, Cs, heads = 16, 8, 2
    x, cond = torch.randn(1, 3, 8, 8, C, generator=g), torch.randn(1, 3, 2, 2, Cs, generator=g)
    p = _pixel_params(C, Cs, heads, g, gate_one=True)
    # planted: modulation order (gate1, scale1, shift1, ...) -> the bias puts 1 in the shifts
    q = dict(p)
    bias = p["adaln_bilinear_dw_proj.bias"].view(6, C)
    q["adaln_bilinear_dw_proj.bias"] = bias[[2, 1, 0, 5, 4, 3]].reshape(-1)
    out = OB.pixel_block_forward(x, cond, q, heads, (3, 3, 3), 4)
    ref = OB.block_forward(x, p, heads, (3, 3, 3), None, None, dtype=torch.float64)
    assert not torch.allclose(out, ref, atol=1e-3)
