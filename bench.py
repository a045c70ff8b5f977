"""Benchmark of the Strata hot path on one MI355X (driver contract: one JSON line).

Headline (``value``): NA3D forward TFLOP/s at BASELINE configs[2] — 6 halo-
padded cube-face tiles (16,144,144), outputs for the interior (16,128,128),
16 heads x 64, window (3,13,13), bf16, q/k/v ~ N(0,1) * per-head U(0.5,2).
One step = one NA3D launch over the whole batch; inputs are resident in HBM.
FLOPs = 4 * N_q(interior) * |W| * D per head.

Also reported: configs[1] (RoPE pack + NA3D (3,7,7)), the full Strata block
(configs[3]) tokens/s with a per-kernel breakdown and the RoPE+QKV-pack
prologue's HBM GB/s, the configs[4] two-stage 4-step rollout, the roofline of
the dominant kernel (HBM-bound: its algorithmic bytes need longer at 8 TB/s than
its FLOPs at the bf16 peak), and the CPU oracle on this host's cores for
configs[0]-[4] (bounded; ``--cpu-full`` times configs[3] in full, median of 5).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cfg1] [--no-block] [--no-rollout] [--no-halo]
                    [--no-backward] [--no-cpu] [--cpu-full]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 4096 bf16 FLOP/clk/CU x 2.4 GHz (vendor "2.5 PF" dense)
PEAK_HBM_GBPS = 8000.0
METRIC = "NA3D fwd TFLOP/s & % bf16 MFMA peak; Strata-block tokens/s, 1 MI355X"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cfg2_inputs(device):
    import torch

    g = torch.Generator(device=device).manual_seed(0)
    s_h = torch.rand(16, generator=g, device=device) * 1.5 + 0.5
    shape = (6, 16, 144, 144, 16, 64)
    return [
        (torch.randn(shape, generator=g, device=device) * s_h.view(1, 1, 1, 1, 16, 1)).bfloat16() for _ in range(3)
    ]


def time_na3d(q, k, v, steps, warmup):
    """Per-launch time of the NA3D kernel (HIP events on torch's current
    stream, which is the stream the op launches on)."""
    import torch

    op = torch.ops.strata_hip.na3d_fwd
    args = ([3, 13, 13], [1, 1, 1], None, [0, 8, 8], [16, 128, 128])
    for _ in range(warmup):
        out = op(q, k, v, *args)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        out = op(q, k, v, *args)
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(stop) / steps, wall / steps * 1e3, out


def bench_block(device, steps, warmup):
    """one Strata block forward on [4, 8, 64, 64, 1024] bf16."""
    import torch

    from strata_amd import ops
    from strata_amd import rope as P
    from strata_amd.modules import StrataBlock, init_xavier_

    B, Z, Y, X, C, H = 4, 8, 64, 64, 1024, 16
    blk = StrataBlock(C, H, (3, 7, 7))
    init_xavier_(blk, torch.Generator().manual_seed(1))
    blk = blk.to(device).bfloat16().eval()
    gx = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(B, Z, Y, X, C, generator=gx, device=device).bfloat16()
    lat, lon = P.synthetic_tile_latlon(B, Y, X, torch.Generator().manual_seed(0))
    cos, sin = P.stereographic_rope_tables(lat.to(device), lon.to(device), C // H, 10000.0, P.default_rope_length_scale(1))
    rope = (cos, sin)
    with torch.no_grad():
        for _ in range(warmup):
            y = blk(x, rope)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            y = blk(x, rope)
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    M = B * Z * Y * X

    # per-kernel breakdown: the block's launches one by one, each bracketed by events
    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            r = fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps, r

    attn, mlp = blk.attn, blk.mlp
    with torch.no_grad():
        t_ln, h = timed(lambda: ops.layer_norm(x, 1e-6))
        t_qkv, qkv = timed(lambda: ops.gemm_bias_act(h, attn.qkv.weight, attn.qkv.bias, None, 0))
        # as the block: the pack writes q and k, v is read out of qkv as a strided view
        # as the block at inference: the pack writes k only, NA3D rotates the queries itself
        t_rope, (_, k, _) = timed(lambda: ops.rope_qkv_pack(qkv, cos, sin, H, 0, pack_v=False, pack_q=False))
        q6 = qkv.view(B, Z, Y, X, 3, H, C // H)
        q, v = q6[..., 0, :, :], q6[..., 2, :, :]
        t_na, a = timed(lambda: ops.na3d_fwd_rope_q(q, k, v, cos, sin, [3, 7, 7], [1, 1, 1], None))
        a = a.view(B, Z, Y, X, C)
        t_proj, x1 = timed(lambda: ops.gemm_bias_act(a, attn.proj.weight, attn.proj.bias, x, 0))
        t_fc1, f = timed(lambda: ops.gemm_bias_act(h, mlp.layers[0].weight, mlp.layers[0].bias, None, 1))
        t_fc2, _ = timed(lambda: ops.gemm_bias_act(f, mlp.layers[2].weight, mlp.layers[2].bias, x1, 0))
    gemm_flops = {"qkv": 2 * M * C * 3 * C, "proj": 2 * M * C * C, "fc1": 2 * M * C * 4 * C, "fc2": 2 * M * 4 * C * C}
    na_flops = 4.0 * M * H * 147 * (C // H)
    rope_bytes = M * C * 2 * 2 + B * Y * X * (C // H // 2) * 4 * 2  # k columns read + k written + tables
    kernels = {
        "layer_norm_ms": t_ln,
        "qkv_gemm_ms": t_qkv,
        "rope_pack_ms": t_rope,
        "na3d_ms": t_na,
        "proj_gemm_ms": t_proj,
        "fc1_gelu_gemm_ms": t_fc1,
        "fc2_gemm_ms": t_fc2,
    }
    tflops = {
        "qkv_gemm": gemm_flops["qkv"] / t_qkv / 1e9,
        "proj_gemm": gemm_flops["proj"] / t_proj / 1e9,
        "fc1_gelu_gemm": gemm_flops["fc1"] / t_fc1 / 1e9,
        "fc2_gemm": gemm_flops["fc2"] / t_fc2 / 1e9,
        "na3d": na_flops / t_na / 1e9,
    }
    total_flops = sum(gemm_flops.values()) + na_flops
    return {
        "workload": "configs[3] Strata block fwd: x [4,8,64,64,1024] bf16, 16x64 heads, W=(3,7,7), "
        "stereographic RoPE, MLP 4096 GELU(tanh), Xavier seed 1",
        "tokens_per_s": M / (ms * 1e-3),
        "ms_per_step": ms,
        "block_tflops": total_flops / (ms * 1e-3) / 1e12,
        "pct_bf16_peak": 100.0 * total_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "kernel_ms": {k: round(v, 4) for k, v in kernels.items()},
        "kernel_tflops": {k: round(v, 1) for k, v in tflops.items()},
        "prologue_GBps": rope_bytes / (t_rope * 1e-3) / 1e9,
        "prologue_pct_hbm": 100.0 * rope_bytes / (t_rope * 1e-3) / 1e9 / PEAK_HBM_GBPS,
    }


def bench_production(device, steps, warmup):
    """The production block on one rollout tile: (24, 144, 144) tokens x 1024, 16 x 64
    heads, window (3, 3, 3), gated, non-affine qk RMSNorm, RoPE base 100 at the patch-4
    length scale (scripts/ace/run_screamcast_nudged.py:156-165 tile 512 + halo 32 at
    patch 4; train_configs.py:303-317 block flags).  The production config also sets
    do_alt_depthwise_attn (train_configs.py:316): every other block attends its whole
    z column instead (window (24, 1, 1)); that block is timed as well."""
    import torch

    from strata_amd import rope as P
    from strata_amd.modules import StrataBlock, init_xavier_

    B, Z, Y, X, C, H, kernel = 1, 24, 144, 144, 1024, 16, (3, 3, 3)
    x = torch.randn(B, Z, Y, X, C, generator=torch.Generator(device=device).manual_seed(0), device=device).bfloat16()
    ls = P.default_rope_length_scale(4)
    lat, lon = P.synthetic_tile_latlon(B, Y, X, torch.Generator().manual_seed(0), spacing=ls)
    rope = P.stereographic_rope_tables(lat.to(device), lon.to(device), C // H, 100.0, ls)

    def timed_block(depthwise):
        blk = StrataBlock(C, H, kernel, gated=True, qk_norm=True, depthwise=depthwise)
        init_xavier_(blk, torch.Generator().manual_seed(1))
        blk = blk.to(device).bfloat16().eval()
        with torch.no_grad():
            for _ in range(warmup):
                y = blk(x, rope)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                y = blk(x, rope)
            e1.record()
            torch.cuda.synchronize()
        assert torch.isfinite(y.float()).all(), "production block produced non-finite values"
        return e0.elapsed_time(e1) / steps

    ms = timed_block(False)
    ms_dw = timed_block(True)
    M = B * Z * Y * X
    gemm = 2.0 * M * C * C * (3 + 1 + 1 + 8)  # qkv, gate, proj, fc1+fc2
    flops = gemm + 4.0 * M * H * 27 * (C // H)
    flops_dw = gemm + 4.0 * M * H * Z * (C // H)
    return {
        "workload": "production block: (24,144,144) tokens x 1024, 16x64 heads, W=(3,3,3), gated, qk RMSNorm, "
        "RoPE base 100 (patch-4 length scale), MLP 4096 GELU(tanh), Xavier seed 1; the alternate "
        "depth-wise block: window (24,1,1)",
        "ms_per_step": round(ms, 3),
        "tokens_per_s": M / (ms * 1e-3),
        "block_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "pct_bf16_peak": round(100.0 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "depthwise_ms_per_step": round(ms_dw, 3),
        "depthwise_block_tflops": round(flops_dw / (ms_dw * 1e-3) / 1e12, 1),
        "pair_tokens_per_s": M / ((ms + ms_dw) * 1e-3),  # M tokens through one block of each kind
    }


def bench_pixel(device, steps, warmup):
    """One pixel-stage block of the production two-stage model (train_configs.py:459-485:
    pixel width 128, 2 heads x 64, attn_kernel 9 read as (9, 9, 9), qk RMSNorm; semantic
    width 1024 at horizontal patch 4) on six 64 x 64 tiles of 24 levels, conditioned on
    the semantic tokens [6, 24, 16, 16, 1024] by the bilinear / depth-wise / GELU /
    projection adaLN (this build's convention).  Timed whole, and its modulation path
    (upsample_dw_gelu + the 1024 -> 768 projection) alone."""
    import torch

    from strata_amd.modules import StrataPixelBlock, init_xavier_

    B, Z, Y, X, C, H, Cs, f, kernel = 6, 24, 64, 64, 128, 2, 1024, 4, (9, 9, 9)
    g = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(B, Z, Y, X, C, generator=g, device=device).bfloat16()
    cond = torch.randn(B, Z, Y // f, X // f, Cs, generator=g, device=device).bfloat16()
    blk = StrataPixelBlock(C, H, kernel, cond_dim=Cs, factor=f, qk_norm=True)
    init_xavier_(blk, torch.Generator().manual_seed(1))
    with torch.no_grad():
        blk.adaln_bilinear_dw_proj.bias.normal_(0.0, 0.5, generator=torch.Generator().manual_seed(2))
    blk = blk.to(device).bfloat16().eval()

    def timed(fn):
        with torch.no_grad():
            for _ in range(warmup):
                y = fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                y = fn()
            e1.record()
            torch.cuda.synchronize()
        assert torch.isfinite(y.float()).all(), "pixel block produced non-finite values"
        return e0.elapsed_time(e1) / steps

    ms = timed(lambda: blk(x, cond))
    ms_mod = timed(lambda: blk.modulation(cond))
    M = B * Z * Y * X
    flops = 2.0 * M * C * C * (3 + 1 + 8) + 2.0 * M * Cs * 6 * C + 4.0 * M * H * 9 * 9 * 9 * (C // H)
    up_bytes = 2.0 * (B * Z * (Y // f) * (X // f) * Cs + M * Cs)  # the upsampling kernel: cond read, c written
    return {
        "workload": "pixel-stage block (this build's adaLN convention): [6,24,64,64,128] bf16, 2x64 heads, "
        "W=(9,9,9), qk RMSNorm, MLP 512 GELU(tanh); cond [6,24,16,16,1024] upsampled x4 (bilinear, "
        "depth-wise 3x3, GELU) and projected 1024 -> 6x128; Xavier seed 1",
        "ms_per_step": round(ms, 3),
        "tokens_per_s": M / (ms * 1e-3),
        "block_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "pct_bf16_peak": round(100.0 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "modulation_ms": round(ms_mod, 3),
        "upsample_min_bytes_GB": round(up_bytes / 1e9, 3),
    }


def cfg1_inputs(device):
    """configs[1] inputs: q, k, v ~ N(0,1) [2,8,64,64,8,64] (seed 0, in that order), the
    stereographic tables of 64x64 tiles with the level index in z (pairs x | y | level =
    12 | 12 | 8, base 1e4), and the packed qkv [2,8,64,64,3*8*64] the pack kernel reads."""
    import torch

    from strata_amd import rope as P

    B, Z, Y, X, H, D = 2, 8, 64, 64, 8, 64
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, Z, Y, X, H, D, generator=g).bfloat16() for _ in range(3))
    lat, lon = P.synthetic_tile_latlon(B, Y, X, g)
    cos, sin = P.stereographic_rope_tables(lat, lon, D, 10000.0, P.default_rope_length_scale(1), levels=Z,
                                           level_pairs=8)
    qkv = torch.stack([q, k, v], dim=4).reshape(B, Z, Y, X, 3 * H * D)
    return q, k, v, qkv, cos, sin, lat, lon


def bench_cfg1(device, steps, warmup):
    """stereographic RoPE (+ QKV pack) then NA3D (3,7,7) on [2,8,64,64,8,64] bf16."""
    import torch

    B, Z, Y, X, H, D = 2, 8, 64, 64, 8, 64
    _, _, _, qkv, cos, sin, _, _ = cfg1_inputs(torch.device("cpu"))
    qkv, cos, sin = qkv.to(device), cos.to(device), sin.to(device)
    pack = torch.ops.strata_hip.rope_qkv_pack
    na = torch.ops.strata_hip.na3d_fwd_rope_q

    # As the block runs it at inference: the pack rotates and writes k only; NA3D reads
    # q (unrotated, rotated inside the kernel) and v straight out of qkv as strided views.
    def run_pack():
        return pack(qkv, cos, sin, H, 0, False, 1e-6, None, None, False, False)

    _, k, _ = run_pack()
    q = qkv.view(B, Z, Y, X, 3, H, D)[..., 0, :, :]
    v = qkv.view(B, Z, Y, X, 3, H, D)[..., 2, :, :]

    def run_na():
        return na(q, k, v, cos, sin, [3, 7, 7], [1, 1, 1], None)

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps

    t_pack, t_na = timed(run_pack), timed(run_na)
    M = B * Z * Y * X
    flops = 4.0 * M * H * 147 * D
    na_bytes = 4 * M * H * D * 2  # q, k, v read once, o written once (the RoPE tables: L2-resident)
    pack_bytes = M * H * D * 2 * 2 + cos.numel() * 4 * 2  # k columns read, k written, tables read
    return {
        "workload": "configs[1] stereographic RoPE (level index in z: pairs x|y|level = 12|12|8, base 1e4) + "
        "QKV pack (k only; q rotated inside the NA3D kernel, q and v read from qkv as strided views), NA3D W=(3,7,7) on [2,8,64,64,8,64] bf16, "
        "q/k/v ~ N(0,1) seed 0",
        "na3d_ms": round(t_na, 4),
        "na3d_tflops": round(flops / (t_na * 1e-3) / 1e12, 1),
        "na3d_pct_bf16_peak": round(100.0 * flops / (t_na * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
        "na3d_algorithmic_GBps": round(na_bytes / (t_na * 1e-3) / 1e9, 1),
        "na3d_pct_hbm": round(100.0 * na_bytes / (t_na * 1e-3) / 1e9 / PEAK_HBM_GBPS, 1),
        "rope_pack_ms": round(t_pack, 4),
        "rope_pack_GBps": round(pack_bytes / (t_pack * 1e-3) / 1e9, 1),
        "rope_pack_pct_hbm": round(100.0 * pack_bytes / (t_pack * 1e-3) / 1e9 / PEAK_HBM_GBPS, 1),
        "total_ms": round(t_pack + t_na, 4),
    }


def bench_rollout(device, reps, warmup):
    """two-stage model (12 blocks @768 on (16,64,64), 2x merge, 12 blocks
    @1024 on (8,32,32)), batch 6 face tiles, 80 channels, 4 autoregressive steps."""
    import torch

    from strata_amd import rope as P
    from strata_amd.model import TwoStageStrata
    from strata_amd.modules import init_xavier_

    model = TwoStageStrata()
    init_xavier_(model, torch.Generator().manual_seed(1))
    model = model.to(device).bfloat16().eval()
    g = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(6, 80, 16, 64, 64, generator=g, device=device).bfloat16()
    lat, lon = P.synthetic_tile_latlon(6, 64, 64, torch.Generator().manual_seed(0))
    rope1, rope2 = model.rope_tables(lat.to(device), lon.to(device))
    steps = 4
    for _ in range(warmup):
        model.rollout(x, steps, rope1, rope2)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        y = model.rollout(x, steps, rope1, rope2)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    flops = model.step_flops(6, (16, 64, 64)) * steps
    tokens = 6 * 16 * 64 * 64 * steps
    assert torch.isfinite(y.float()).all(), "rollout produced non-finite values"
    return {
        "workload": "configs[4] two-stage rollout: B=6 tiles, 80 ch, s1 12x(768, 12x64, W=(3,7,7)) on (16,64,64), "
        "2x merge, s2 12x(1024, 16x64, W=(3,9,9)) on (8,32,32), 4 steps, Xavier seed 1",
        "rollout_ms": round(ms, 2),
        "step_ms": round(ms / steps, 2),
        "tokens_per_s": tokens / (ms * 1e-3),
        "block_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "pct_bf16_peak": round(100.0 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
    }


def bench_halo(device, reps, warmup):
    """Cube-sphere halo fill + crop at the rollout tile geometry: 80 channels x
    6 faces of 512 x 512 fp32, 32-cell halo (create_padded_faces_batched and
    TileTopology.crop).  Algorithmic bytes = input read once + output written once."""
    import torch

    L, n, p = 80, 512, 32
    g = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(L, 6, n, n, generator=g, device=device)
    pad = lambda: torch.ops.strata_hip.cube_pad_faces(x, p)  # noqa: E731
    y = pad()
    crop = lambda: torch.ops.strata_hip.cube_crop(y, p)  # noqa: E731
    out = {"workload": f"cube-sphere halo fill: [{L}, 6, {n}, {n}] fp32, halo {p}; crop back"}
    for name, fn, nbytes in (("pad", pad, (x.numel() + y.numel()) * 4), ("crop", crop, (x.numel() + y.numel()) * 4)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[f"{name}_ms"] = round(ms, 4)
        out[f"{name}_GBps"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        out[f"{name}_pct_hbm"] = round(100.0 * nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 1)
    return out


def bench_step_io(device, reps, warmup):
    """The rollout step's kernels around the network at the configs[4] geometry:
    fp32 state [6, 80, 16, 64, 64] -> normalised bf16 tokens (patch 1), and head
    tokens [6, 8, 32, 32, 640] (2x2x2 cells, channels last) -> denormalised,
    state-updated fp32 state with a floor on one channel.  Algorithmic bytes =
    each input read once + the output written once (the 80-entry tables aside).
    ``dealias``: the two filter passes (y, x; the (1, 4, 6, 4, 1) low-pass with
    patch (1, 2, 2), normalisation fused) of a dealiased patch embedding of the
    same state, each pass reading and writing the fp32 state once."""
    import torch

    from strata_amd import ops

    B, C, grid = 6, 80, (16, 64, 64)
    g = torch.Generator(device=device).manual_seed(0)
    state = torch.randn(B, C, *grid, generator=g, device=device)
    pred = torch.randn(B, 8, 32, 32, 8 * C, generator=g, device=device).bfloat16()
    mean = torch.randn(C, generator=g, device=device)
    std = torch.rand(C, generator=g, device=device) + 0.5
    src = torch.arange(C, dtype=torch.int32, device=device)
    floor = torch.full((C,), float("nan"), device=device)
    floor[7] = 0.0
    n = state.numel()
    taps = [0.0625, 0.25, 0.375, 0.25, 0.0625]
    fns = (
        ("patchify", lambda: ops.state_patchify(state, mean, std, (1, 1, 1)), n * (4 + 2)),
        ("update", lambda: ops.state_update(pred, state, mean, std, src, floor, grid, (2, 2, 2), 1), n * (2 + 4 + 4)),
        ("dealias", lambda: ops.dealias_axis(ops.dealias_axis(state, mean, std, 1, 2, taps), None, None, 2, 2, taps),
         2 * n * (4 + 4)),
    )
    out = {"workload": f"rollout step I/O: state [{B}, {C}, 16, 64, 64] fp32 <-> bf16 tokens (patchify 1, update 2x2x2)"}
    for name, fn, nbytes in fns:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        out[f"{name}_ms"] = round(ms, 4)
        out[f"{name}_GBps"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        out[f"{name}_pct_hbm"] = round(100.0 * nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 1)
    return out


def bench_backward(device, reps, warmup):
    """Training kernels: the NA3D backward at the configs[1] shape ([2, 8, 64, 64] tokens,
    8 x 64 heads, W=(3,7,7), bf16; FLOPs = 2.5 x the forward's 4*N*|W|*D, the usual
    attention-backward count) as training runs it (given the forward's log-sum-exp,
    ``na3d_bwd``) and with the statistic recomputed (``na3d_bwd_recompute``), and the
    GEMM-GELU backward's fused epilogue GEMM (gelu'(x @ w.T + b) * dout) at the
    configs[3] fc1 shape."""
    import torch

    from strata_amd import _lib, ops

    g = torch.Generator(device=device).manual_seed(0)
    shape, ker = (2, 8, 64, 64, 8, 64), [3, 7, 7]
    q, k, v, do = (torch.randn(shape, generator=g, device=device).bfloat16() for _ in range(4))
    out, lse = torch.ops.strata_hip.na3d_fwd_lse(q, k, v, ker, [1, 1, 1], None)
    M, N, K = 131072, 4096, 1024
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (torch.randn(N, K, generator=g, device=device) * K**-0.5).bfloat16()
    b = torch.randn(N, generator=g, device=device).bfloat16()
    dy = torch.randn(M, N, generator=g, device=device).bfloat16()
    B, Z, Y, X, H, D = shape
    fns = (
        ("na3d_bwd", lambda: ops.na3d_bwd(q, k, v, out, do, ker, [1, 1, 1], None, lse),
         2.5 * 4.0 * B * Z * Y * X * H * 147 * D),
        ("na3d_bwd_recompute", lambda: ops.na3d_bwd(q, k, v, out, do, ker, [1, 1, 1], None),
         2.5 * 4.0 * B * Z * Y * X * H * 147 * D),
        ("gelu_grad_gemm", lambda: ops.gemm_bias_act(x, w, b, dy, _lib.ACT_GELU_TANH_GRAD, _lib.RES_MUL),
         2.0 * M * N * K),
    )
    res = {"workload": "NA3D bwd at configs[1] (bf16, W=(3,7,7)); fused GELU-derivative GEMM at configs[3] fc1 "
                       "(M=131072, N=4096, K=1024)"}
    for name, fn, flops in fns:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        res[f"{name}_ms"] = round(ms, 4)
        res[f"{name}_tflops"] = round(flops / (ms * 1e-3) / 1e12, 1)
    res.update(_block_train_step(device, reps, warmup))
    return res


def _block_train_step(device, reps, warmup):
    """One training step of the configs[3] block: forward with autograd, then backward of
    a random output gradient into the input and every parameter (bf16 weights, as the
    forward bench). FLOPs: 3x the block's GEMMs (forward, input and weight gradients) and
    NA3D at 1 + 2.5 times its forward count."""
    import torch

    from strata_amd import rope as P
    from strata_amd.modules import StrataBlock, init_xavier_

    B, Z, Y, X, C, H = 4, 8, 64, 64, 1024, 16
    blk = StrataBlock(C, H, (3, 7, 7))
    init_xavier_(blk, torch.Generator().manual_seed(1))
    blk = blk.to(device).bfloat16().train()
    gx = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(B, Z, Y, X, C, generator=gx, device=device).bfloat16().requires_grad_(True)
    dy = torch.randn(B, Z, Y, X, C, generator=gx, device=device).bfloat16()
    lat, lon = P.synthetic_tile_latlon(B, Y, X, torch.Generator().manual_seed(0))
    rope = P.stereographic_rope_tables(lat.to(device), lon.to(device), C // H, 10000.0, P.default_rope_length_scale(1))

    def step():
        blk.zero_grad(set_to_none=True)
        x.grad = None
        blk(x, rope).backward(dy)

    for _ in range(max(warmup, 1)):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    assert torch.isfinite(x.grad.float()).all(), "block backward produced non-finite input gradients"
    M = B * Z * Y * X
    flops = 3 * 24.0 * M * C * C + 3.5 * 4.0 * M * 147 * C
    return {
        "block_train_workload": "configs[3] block [4,8,64,64,1024] forward + backward (input and parameter "
                                "gradients), 16x64 heads, W=(3,7,7), Xavier seed 1",
        "block_train_ms": round(ms, 3),
        "block_train_tokens_per_s": M / (ms * 1e-3),
        "block_train_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
    }


def _cpu_affinity() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _cpu_threads() -> int:
    """Host threads for the CPU baseline: the process's share of the host, i.e. its
    CPU affinity mask, capped by OMP_NUM_THREADS where the host sets one (the GPU
    boxes set 16 per GPU)."""
    n = _cpu_affinity()
    env = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(env)) if env.isdigit() and int(env) > 0 else n


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, reps: int, warmup: int = 1, what: str = "") -> tuple[float, list[float]]:
    """Median wall time of reps calls after warmup calls; one progress line per call on
    stderr (a full-size CPU case runs for minutes)."""
    for _ in range(warmup):
        fn()
    times = []
    for i in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if what:
            print(f"bench: cpu {what} run {i + 1}/{reps}: {times[-1]:.2f} s", file=sys.stderr, flush=True)
    return statistics.median(times), times


def _cpu_block_case(B, grid, C, H, kernel, ls_patch=1):
    """Inputs of one oracle block run: x ~ N(0,1) seed 0, Xavier seed 1 weights, tables."""
    import torch

    from oracle import rope as R
    from strata_amd import rope as P
    from strata_amd.modules import StrataBlock, init_xavier_

    blk = StrataBlock(C, H, kernel)
    init_xavier_(blk, torch.Generator().manual_seed(1))
    params = {k: v.detach().float() for k, v in blk.state_dict().items()}
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, *grid, C, generator=g)
    lat, lon = P.synthetic_tile_latlon(B, grid[1], grid[2], g)
    c, s = R.tables(lat, lon, C // H, 10000.0, R.default_rope_length_scale(ls_patch))
    return x, params, c.float(), s.float()


def cpu_baselines(full: bool):
    """The torch-CPU oracle (fp32) on this host, all its threads, beside the GPU figures.

    Headline (``cpu_baseline``): a bounded sample of configs[2] (tile 0, head 0,
    z 0-3 of the interior: 4.25 GFLOP), warm-up + median of 5.  ``cpu_configs``:
    configs[0] and configs[1] in full (median of 5 each), configs[3] on batch entry
    0 (x4, labelled extrapolated; in full with ``full``), configs[2] from the
    sample (x FLOP ratio) and configs[4] from one block per stage at batch 1
    (x tokens x blocks x tiles x steps), both labelled extrapolated."""
    import torch

    from oracle import block as OB
    from oracle import na3d as O
    from oracle import rope as R

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    reps = 5 if full else 3
    out = {}
    # configs[2] sample (the headline cpu_baseline)
    g = torch.Generator().manual_seed(0)
    shape = (1, 16, 144, 144, 1, 64)
    q, k, v = (torch.randn(shape, generator=g) for _ in range(3))
    box_o, box_e = (0, 8, 8), (4, 128, 128)
    f_sample = O.na3d_flops(1, 1, 64, box_e[0] * box_e[1] * box_e[2], (3, 13, 13))
    t2, _ = _median_time(lambda: O.na3d(q, k, v, (3, 13, 13), q_origin=box_o, q_extent=box_e), 5, what="configs[2] sample")
    f2 = 4.0 * 6 * 16 * (16 * 128 * 128) * 507 * 64
    headline = {
        "value": f_sample / t2 / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": "configs[2] NA3D, tile 0, head 0, query box z 0-3 x interior 128x128 (4.25 GFLOP), fp32 "
        f"torch-CPU oracle, warm-up + median of 5 = {t2:.2f} s, {threads} threads",
        "host": {"os_cpu_count": os.cpu_count(), "affinity_cpus": _cpu_affinity(),
                 "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
                 "torch_threads": torch.get_num_threads(), "cpu_model": _cpu_model()},
    }
    out["configs[2]"] = {"seconds": round(t2 * f2 / f_sample, 1), "extrapolated": True,
                         "from": "the sample above x FLOP ratio (x768)"}
    # fp32 NA3D [1,4,16,16,4,32], W=(3,5,5), vs nothing (plumbing)
    g = torch.Generator().manual_seed(0)
    s0 = (1, 4, 16, 16, 4, 32)
    q0, k0, v0 = (torch.randn(s0, generator=g) for _ in range(3))
    t0, _ = _median_time(lambda: O.na3d(q0, k0, v0, (3, 5, 5)), 5, what="configs[0]")
    out["configs[0]"] = {"seconds": round(t0, 5), "gflops": round(O.na3d_flops(1, 4, 32, 4 * 16 * 16, (3, 5, 5)) / t0 / 1e9, 2)}
    # RoPE (level tables) + NA3D in full
    q1, k1, v1, _, c1, s1, _, _ = cfg1_inputs(torch.device("cpu"))
    q1, k1, v1, c1, s1 = q1.float(), k1.float(), v1.float(), c1.float(), s1.float()

    def run1():
        return O.na3d(R.apply_rope(q1, c1, s1), R.apply_rope(k1, c1, s1), v1, (3, 7, 7))

    t1, _ = _median_time(run1, 5, 1, what="configs[1]")  # one warm-up, then the median of 5
    out["configs[1]"] = {"seconds": round(t1, 3), "gflops": round(4.0 * 2 * 8 * 64 * 64 * 8 * 147 * 64 / t1 / 1e9, 2)}
    # the block
    B3 = 4 if full else 1
    x, prm, c, s = _cpu_block_case(4, (8, 64, 64), 1024, 16, (3, 7, 7))
    x, c, s = x[:B3], c[:B3], s[:B3]
    t3, _ = _median_time(lambda: OB.block_forward(x, prm, 16, (3, 7, 7), c, s), reps if full else 1, 1 if full else 0,
                         what="configs[3]")
    out["configs[3]"] = {"seconds": round(t3 * 4 / B3, 2), "extrapolated": not full,
                         "tokens_per_s": round(4 * 8 * 64 * 64 / (t3 * 4 / B3), 1),
                         "from": "in full" if full else "batch entry 0 (one run) x4"}
    # one block per stage at batch 1 (stage 1 on a quarter of its z range
    # unless full), scaled by tokens x 12 blocks x 6 tiles x 4 steps
    za = 16 if full else 4
    xa, pa, ca, sa = _cpu_block_case(1, (za, 64, 64), 768, 12, (3, 7, 7))
    xb, pb, cb, sb = _cpu_block_case(1, (8, 32, 32), 1024, 16, (3, 9, 9), ls_patch=2)
    ta, _ = _median_time(lambda: OB.block_forward(xa, pa, 12, (3, 7, 7), ca, sa), 1, 0, what="configs[4] stage-1 block")
    tb, _ = _median_time(lambda: OB.block_forward(xb, pb, 16, (3, 9, 9), cb, sb), 1, 0, what="configs[4] stage-2 block")
    ta *= 16 / za
    t4 = (ta * 12 + tb * 12) * 6 * 4
    out["configs[4]"] = {"seconds": round(t4, 1), "extrapolated": True,
                         "from": f"one stage-1 block ({ta:.2f} s, run on z 0-{za - 1} and scaled) and one stage-2 "
                                 f"block ({tb:.2f} s) at batch 1, x12 blocks x6 tiles x4 steps (embed/merge/head "
                                 "not included)"}
    return headline, out


def load_traffic():
    """HBM bytes per NA3D launch from the committed rocprofv3 --pmc summary, if any, and
    the kernel (with its source commit) that summary was measured on."""
    p = ROOT / "profiles" / "na3d_cfg2_traffic.json"
    if p.exists():
        try:
            d = json.loads(p.read_text())
            return d.get("traffic_bytes"), f"{d.get('kernel')} (na3d.hip at {d.get('kernel_source_commit')})"
        except (ValueError, OSError):
            return None, None
    return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-block", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-rollout", action="store_true")
    ap.add_argument("--no-halo", action="store_true")
    ap.add_argument("--no-backward", action="store_true")
    ap.add_argument("--no-cfg1", action="store_true")
    ap.add_argument("--no-production", action="store_true", help="skip the production-tile block (profiling passes)")
    ap.add_argument("--no-pixel", action="store_true", help="skip the pixel-stage block (profiling passes)")
    ap.add_argument("--cpu-full", action="store_true",
                    help="CPU baseline in full: configs[3] over its whole batch, warm-up + median of 5 everywhere")
    ap.add_argument(
        "--copy-calibration",
        action="store_true",
        help="only run a plain 1 GiB device-to-device copy (steps times); for scaling rocprofv3 byte counters",
    )
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the tiles are "
            "independent per GPU, so run it per GPU.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    import strata_amd  # noqa: F401
    from strata_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": src.numel() * 2, "copies": args.steps}), flush=True)
        return
    log("bench: generating configs[2] inputs")
    q, k, v = cfg2_inputs(dev)
    torch.cuda.synchronize()
    log("bench: timing NA3D configs[2]")
    ms, wall_ms, _ = time_na3d(q, k, v, args.steps, args.warmup)
    flops = 4.0 * 6 * 16 * (16 * 128 * 128) * 507 * 64
    tflops = flops / (ms * 1e-3) / 1e12
    alg_bytes = (6 * 16 * 128 * 128 * 16 * 64 * 2) * 2 + (6 * 16 * 144 * 144 * 16 * 64 * 2) * 2
    del q, k, v
    torch.cuda.empty_cache()

    result = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "configs[2] NA3D fwd: 6 halo-padded tiles (16,144,144) -> interior (16,128,128), "
            "16 heads x 64, W=(3,13,13), bf16, q/k/v ~ N(0,1)*U(0.5,2) per head, seed 0",
            "batch": 6,
            "grid": [16, 144, 144],
            "interior": [16, 128, 128],
            "heads": 16,
            "head_dim": 64,
            "kernel": [3, 13, 13],
        },
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "wall_ms_per_step": round(wall_ms, 4),
        # Binding roofline: the algorithmic bytes (14.60 GB) take 1.825 ms at 8 TB/s, the
        # algorithmic FLOPs (3.266 TF) 1.298 ms at 2516.6 TFLOP/s, so HBM bounds the kernel.
        "roofline": {
            "bound": "hbm",
            "achieved": round(alg_bytes / (ms * 1e-3) / 1e9, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(alg_bytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4),
            "traffic": load_traffic()[0],
            "traffic_kernel": load_traffic()[1],
            "algorithmic_bytes": alg_bytes,
            "mfma": {"achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4)},
        },
    }
    if not args.no_cfg1:
        log("bench: timing configs[1] (RoPE pack + NA3D)")
        result["cfg1"] = bench_cfg1(dev, args.steps, args.warmup)
    if not args.no_block:
        log("bench: timing the configs[3] block")
        result["block"] = bench_block(dev, max(3, args.steps // 2), 2)
    if not args.no_block and not args.no_production:
        log("bench: timing the production block (one (24,144,144) x 1024 rollout tile)")
        result["production"] = bench_production(dev, 3, 1)
    if not args.no_block and not args.no_pixel:
        log("bench: timing the pixel-stage block")
        result["pixel"] = bench_pixel(dev, 5, 2)
    if not args.no_rollout:
        log("bench: timing the configs[4] rollout")
        result["rollout"] = bench_rollout(dev, 2, 1)
    if not args.no_halo:
        log("bench: timing the cube-sphere halo fill")
        result["halo"] = bench_halo(dev, 10, 2)
        log("bench: timing the rollout step's state kernels")
        result["step_io"] = bench_step_io(dev, 10, 2)
    if not args.no_backward:
        log("bench: timing the backward kernels")
        result["backward"] = bench_backward(dev, 5, 1)
    if not args.no_cpu:
        log("bench: timing the CPU oracle (configs[0]-[4], bounded)" + (" in full" if args.cpu_full else ""))
        result["cpu_baseline"], result["cpu_configs"] = cpu_baselines(args.cpu_full)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
