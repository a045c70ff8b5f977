"""Host-side replay of the address arithmetic of the hand-written kernels (test
infrastructure, CPU only).

For a given launch, each function below recomputes, with the kernel's own index
formulas (the source lines are named in each docstring), every global byte range
the launch reads or writes, as [lo, hi) intervals relative to the base pointer
of the tensor's allocation, and the 32-bit quantities the kernel forms (buffer
lane offsets, record counts, grid sizes).  ``Access`` keeps, per tensor, the
smallest lo and the largest hi and flags any 32-bit value out of range, so a
test can assert that a launch at a given shape stays inside its allocations
without running it.

Where an address is a sum of a part that depends only on the workgroup (tile
origin, batch, head, K step) and a part that depends only on the lane, and no
bounds mask couples them, the extremes over their Cartesian product are the
sums of the parts' extremes: that is how full GEMM tiles, LayerNorm rows and
the batch / head axes of NA3D are covered, exactly.  Everything under a mask
(ragged GEMM tiles, clamped NA3D windows, partial stages) is replayed lane by
lane (numpy, int64).  Offsets are affine in the K step and in the stage index,
so those loops are evaluated at their first and last iteration.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

OOB = 0x7FFFFFF0  # common.h: out-of-range lane offset / record count


@dataclass
class Access:
    """Per-tensor extremes of the byte ranges a launch touches."""

    lo: dict = field(default_factory=dict)
    hi: dict = field(default_factory=dict)
    bad32: list = field(default_factory=list)

    def add(self, name: str, start: np.ndarray, nbytes: int | np.ndarray, mask: np.ndarray | None = None):
        start = np.asarray(start, dtype=np.int64)
        end = start + np.asarray(nbytes, dtype=np.int64)
        if mask is not None:
            shape = np.broadcast_shapes(start.shape, end.shape, np.shape(mask))
            m = np.broadcast_to(np.asarray(mask, dtype=bool), shape)
            if not m.any():
                return
            start, end = np.broadcast_to(start, shape)[m], np.broadcast_to(end, shape)[m]
        if start.size == 0:
            return
        lo, hi = int(start.min()), int(end.max())
        self.lo[name] = min(self.lo.get(name, lo), lo)
        self.hi[name] = max(self.hi.get(name, hi), hi)

    def add_sum(self, name: str, outer: np.ndarray, inner: np.ndarray, nbytes: int):
        """Accesses at outer[i] + inner[j] for every pair (i, j), nbytes each."""
        outer, inner = np.asarray(outer, dtype=np.int64), np.asarray(inner, dtype=np.int64)
        if outer.size == 0 or inner.size == 0:
            return
        self.add(name, np.array([outer.min() + inner.min()]), np.array([outer.max() + inner.max() + nbytes]) -
                 np.array([outer.min() + inner.min()]))

    def u32(self, what: str, values, limit: int = 1 << 32):
        v = np.asarray(values, dtype=np.int64)
        if v.size and (v.min() < 0 or v.max() >= limit):
            self.bad32.append(f"{what}: {int(v.min())}..{int(v.max())} outside [0, {limit})")

    def lane_offsets(self, what: str, voff, nbytes: int = 16):
        """Buffer lane offsets: every offset but the out-of-range sentinel must keep
        its nbytes below the descriptor's record count OOB (else the load reads zeros)."""
        v = np.asarray(voff, dtype=np.int64)
        v = v[v != OOB]
        if v.size and (v.min() < 0 or v.max() + nbytes > OOB):
            self.bad32.append(f"{what}: lane offsets {int(v.min())}..{int(v.max())} reach past {OOB:#x}")

    def check(self, sizes: dict) -> list:
        """Problems: ranges outside [0, sizes[name]) and 32-bit overflows."""
        out = list(self.bad32)
        for name in self.lo:
            if self.lo[name] < 0 or self.hi[name] > sizes[name]:
                out.append(f"{name}: touches [{self.lo[name]}, {self.hi[name]}) of a {sizes[name]}-byte allocation")
        return out


def span(rows: int, cols: int, ld: int, esize: int = 2) -> int:
    """Bytes of a [rows, cols] view with row stride ld (elements)."""
    return 0 if rows == 0 else esize * ((rows - 1) * ld + cols)


# ---------------------------------------------------------------------------
# GEMM: gemm_dma_body<256, 256, 2, 4, 64, 2, ...> (strata_amd/csrc/gemm.hip)
# ---------------------------------------------------------------------------
def _xcd_order(n: int, ids: np.ndarray) -> np.ndarray:
    """common.h xcd_tile_order / gemm.hip tile_origin's first step."""
    xcd, local = ids & 7, ids >> 3
    q, rem = n >> 3, n & 7
    return np.where(xcd < rem, xcd * (q + 1) + local, rem * (q + 1) + (xcd - rem) * q + local)


def gemm_tile_origins(M: int, N: int) -> tuple[np.ndarray, np.ndarray]:
    """(m0, n0) of every persistent-walk tile index t (gemm.hip tile_origin)."""
    mt, nt = -(-M // 256), -(-N // 256)
    ntiles = mt * nt
    wg = _xcd_order(ntiles, np.arange(ntiles, dtype=np.int64))
    GRP = 4
    gi, li = wg // (GRP * nt), wg % (GRP * nt)
    gmn = np.minimum(GRP, mt - gi * GRP)
    return (gi * GRP + li % gmn) * 256, (li // gmn) * 256


def _gswz8(chunk, row):
    return chunk ^ ((row & 7) ^ ((row >> 3) & 1))


def _gemm_dma_offsets(m0, n0, M, N, ldx, ldw, kt_cols=0):
    """Lane offsets voff[j] of a stage's x / w copies (gemm.hip dma_off), broadcast
    over [tile, wave, lane]; and whether each copy reads w.  kt_cols > 0: the
    ragged last K stage of issue_at, whose chunks at or past kt_cols columns take
    the out-of-range offset (tail_ok)."""
    wave = np.arange(8)[None, :, None]
    lane = np.arange(64)[None, None, :]
    out = []
    for j in range(8):  # LPW = 8 copies of 1 KiB per wave, c = j * NW + wave
        c = j * 8 + wave
        isw = c >= 32
        row = 8 * np.where(isw, c - 32, c) + lane // 8
        lc = _gswz8(lane % 8, row)
        ok = np.where(isw, n0 + row < N, m0 + row < M)
        if kt_cols:
            ok = ok & (lc * 8 < kt_cols)
        ld = np.where(isw, ldw, ldx)
        out.append((np.where(ok, row * ld * 2 + lc * 16, OOB), np.broadcast_to(isw, ok.shape)))
    return out


def _gemm_epilogue_lanes():
    """(row, column) offsets inside the tile of every 16-byte epilogue store
    (gemm.hip: wave (wm, wn) = (w / 4, w % 4), lane chunk c = lane % 8, rows
    RPI * it + lane / 8 of its 128-row half-tile pair), shape [wave, it, lane]."""
    wave = np.arange(8)[:, None, None]
    it = np.arange(16)[None, :, None]
    lane = np.arange(64)[None, None, :]
    rows = (wave // 4) * 128 + 8 * it + lane // 8
    cols = (wave % 4) * 64 + 8 * (lane % 8)
    return np.broadcast_to(rows, (8, 16, 64)), np.broadcast_to(cols, (8, 16, 64))


def gemm_dma_launch(M: int, N: int, K: int, ldx: int, ldw: int, ldo: int, ldr: int | None = None,
                    bias: bool = False, save: bool = False, cus: int = 256) -> Access:
    """Every global access of one gemm_dma_kernel launch (gemm.hip gemm_dma_body:
    dma_off / issue_at for the x and w stages, the bias loads into binit, the
    residual loads r4 and the output (and SAVE) stores of the epilogue).
    Full tiles (every row < M, every column < N: no mask anywhere) by the
    separable sum tile base + lane offset; the ragged tiles of the last row and
    column panels lane by lane."""
    acc = Access()
    assert K % 8 == 0 and 256 * ldx * 2 + 4096 < OOB and 256 * ldw * 2 + 4096 < OOB  # gemm_params, gemm_big
    mt, nt = -(-M // 256), -(-N // 256)
    acc.u32("tiles", [mt * nt], 1 << 31)
    m0, n0 = gemm_tile_origins(M, N)
    nk, kt_cols = -(-K // 64), K % 64
    # the first and last K stages bound every stage's addresses; the last one
    # masked past K when K is not a multiple of 64
    stages = [(kt, kt_cols if kt == nk - 1 else 0) for kt in sorted({0, nk - 1})]
    full = (m0 + 256 <= M) & (n0 + 256 <= N)
    outs = [("out", ldo)] + ([("res", ldr)] if ldr is not None else []) + ([("out2", ldo)] if save else [])
    # ---- full tiles: offsets inside a full tile do not depend on which tile it is
    if full.any():
        fm, fn = m0[full], n0[full]
        for kt, kc in stages:
            for voff, isw in _gemm_dma_offsets(np.int64(0), np.int64(0), 1 << 62, 1 << 62, ldx, ldw, kc):
                acc.lane_offsets("gemm dma", voff)
                live = voff + 16 <= OOB
                acc.add_sum("x", 2 * (fm * ldx + kt * 64), voff[~isw & live], 16)
                acc.add_sum("w", 2 * (fn * ldw + kt * 64), voff[isw & live], 16)
        rows, cols = _gemm_epilogue_lanes()
        for name, ld in outs:
            acc.add_sum(name, 2 * (fm * ld + fn), 2 * (rows * ld + cols), 16)
        if bias:
            acc.add_sum("bias", 2 * fn, 2 * np.arange(0, 256, 4), 8)
    # ---- ragged tiles, lane by lane
    rg = ~full
    if rg.any():
        m0r, n0r = m0[rg][:, None, None], n0[rg][:, None, None]
        for kt, kc in stages:
            for voff, isw in _gemm_dma_offsets(m0r, n0r, M, N, ldx, ldw, kc):
                acc.lane_offsets("gemm dma", voff)
                live = voff + 16 <= OOB
                base = np.where(isw, 2 * (n0r * ldw + kt * 64), 2 * (m0r * ldx + kt * 64))
                acc.add("x", base + voff, 16, live & ~isw)
                acc.add("w", base + voff, 16, live & isw)
        wave = np.arange(8)[None, :, None]
        lane = np.arange(64)[None, None, :]
        gm0, gn0 = m0r + (wave // 4) * 128, n0r + (wave % 4) * 64
        gn = gn0 + 8 * (lane % 8)
        for it in range(16):
            gm = gm0 + 8 * it + lane // 8
            whole = (gm < M) & (gn + 8 <= N)
            ragged = ~whole & (gm < M) & (gn < N)
            for name, ld in outs:
                acc.add(name, 2 * (gm * ld + gn), 16, whole)
                for e in range(8):
                    acc.add(name, 2 * (gm * ld + gn + e), 2, ragged & (gn + e < N))
        if bias:
            hi = lane // 32
            for i in range(2):
                for q in range(4):
                    g = gn0 + 32 * i + 8 * q + 4 * hi
                    acc.add("bias", 2 * g, 8, g + 4 <= N)
                    for e in range(4):
                        acc.add("bias", 2 * (g + e), 2, (g + 4 > N) & (g + e < N))
    return acc


def gemm_sizes(M, N, K, ldx, ldw, ldo, ldr=None, bias=False, save=False) -> dict:
    s = {"x": span(M, K, ldx), "w": span(N, K, ldw), "out": span(M, N, ldo)}
    if ldr is not None:
        s["res"] = span(M, N, ldr)
    if bias:
        s["bias"] = 2 * N
    if save:
        s["out2"] = span(M, N, ldo)
    return s


# ---------------------------------------------------------------------------
# LayerNorm (strata_amd/csrc/layernorm.hip layer_norm_kernel<LPR, NR>)
# ---------------------------------------------------------------------------
def layer_norm_launch(M: int, C: int, ldx: int, ldo: int) -> Access:
    acc = Access()
    LPR = 64 if (C // 8) % 64 == 0 or (C // 8) % 32 != 0 else 32
    rows_per_block = 256 // LPR
    blocks = -(-M // rows_per_block)
    acc.u32("layer_norm grid", [blocks], 1 << 31)
    row = np.arange(M, dtype=np.int64)  # rows >= M return before any access
    run = np.arange(C // 8, dtype=np.int64)  # every run some lane holds (lane + LPR * r < runs)
    acc.add_sum("x", 2 * row * ldx, 16 * run, 16)
    acc.add_sum("out", 2 * row * ldo, 16 * run, 16)
    return acc


# ---------------------------------------------------------------------------
# RoPE + QKV pack, half layout (strata_amd/csrc/rope_pack.hip rope_pack_half_kernel)
# ---------------------------------------------------------------------------
def rope_pack_half_launch(B, Z, Y, X, H, D, ld, Zt, pack_q=True, pack_v=False, chunk=1 << 22) -> Access:
    acc = Access()
    cph = D // 16
    C = H * D
    total = B * Z * Y * X * H * cph
    slice_ = -(-total // 2)
    slice_ = -(-slice_ // 64) * 64
    acc.u32("rope_pack grid", [-(-slice_ // 256)], 1 << 31)
    # Every address grows with the thread index except the table row, which repeats
    # per z-slice (Zt = 1) and is largest in the last batch entry: the first and the
    # last chunk of threads (each longer than a z-slice of tokens) hold the extremes.
    assert chunk >= Y * X * H * cph or total <= 2 * chunk
    starts = sorted({0, max(0, total - chunk)})
    for s0 in starts:
        idx = np.arange(s0, min(total, s0 + chunk), dtype=np.int64)
        c = idx % cph
        th = idx // cph
        h = th % H
        tok = th // H
        src = tok * ld + h * D + 8 * c
        x, r = tok % X, tok // X
        y, r = r % Y, r // Y
        z, b = r % Z, r // Z
        trow = ((b * Zt + (0 if Zt == 1 else z)) * Y + y) * X + x
        for t in (0, 1):
            if t == 0 and not pack_q:
                continue
            acc.add("qkv", 2 * (src + t * C), 16)
            acc.add("qkv", 2 * (src + t * C + D // 2), 16)
        if pack_v:
            acc.add("qkv", 2 * (src + 2 * C), 16)
            acc.add("qkv", 2 * (src + 2 * C + D // 2), 16)
        acc.add("tables", 4 * (trow * (D // 2) + 8 * c), 32)
        dst = tok * C + h * D + 8 * c
        for name in (["q"] if pack_q else []) + ["k"] + (["v"] if pack_v else []):
            acc.add(name, 2 * dst, 16)
            acc.add(name, 2 * (dst + D // 2), 16)
    return acc


# ---------------------------------------------------------------------------
# NA3D, general MFMA kernel (strata_amd/csrc/na3d.hip na3d_mfma_body, D = 64)
# ---------------------------------------------------------------------------
def _sub_len(L, g, d):
    return (L - g + d - 1) // d


def _win_start(i, L, k):
    return np.minimum(np.maximum(i - k // 2, 0), L - k)


def _sub_first(o, g, d):
    return 0 if o <= g else (o - g + d - 1) // d


def _sub_end(o, e, g, d):
    hi = o + e
    return 0 if hi <= g else (hi - g + d - 1) // d


def _blocked_tile(w, nz, ny, nx):
    BZ = BY = BX = 4
    zb = w // (BZ * ny * nx)
    r = w - zb * BZ * ny * nx
    bz = np.minimum(BZ, nz - zb * BZ)
    yb = r // (bz * BY * nx)
    r = r - yb * bz * BY * nx
    by = np.minimum(BY, ny - yb * BY)
    xb = r // (bz * by * BX)
    r = r - xb * bz * by * BX
    bx = np.minimum(BX, nx - xb * BX)
    x = xb * BX + r % bx
    r = r // bx
    return zb * BZ + r // by, yb * BY + r % by, x


def na3d_general_launch(B, L, H, ker, dil, qs, ks, vs, os_, org=(0, 0, 0), ext=None, D=64) -> Access:
    """Every global access of one na3d_mfma_kernel launch (na3d.hip: make_tiles,
    the tile decode, the Q and own-key loads, the K/V stage descriptors (issue)
    and lane offsets (voff), the output stores)."""
    assert D == 64
    ext = tuple(L) if ext is None else tuple(ext)
    kx = ker[2]
    TX = 16 if kx == 1 else 8 if kx <= 9 else 4 if kx <= 13 else 2
    NTY, NWX = 4, 4
    TY = 16 // TX
    WY, WQX = NTY * TY, NWX * TX
    LW = (NWX - 1) * TX + 16
    KPK = 512 // D
    LWP = -(-LW // KPK) * KPK
    RB = LWP * D * 2
    RKB = RB // 1024

    def stage_b(rps):
        return 2 * rps * RB

    RPS = 4 if TX <= 4 and 2 * stage_b(4) <= 81920 else 2
    LPT = 2 * RPS * RKB // NWX
    CPK = D // 8
    acc = Access()
    nq = [max(_sub_end(org[a], ext[a], g, dil[a]) - _sub_first(org[a], g, dil[a]) for g in range(dil[a]))
          for a in range(3)]
    nzt, nyt, nxt = nq[0], -(-nq[1] // WY), -(-nq[2] // WQX)
    nres = dil[0] * dil[1] * dil[2]
    total = nxt * nyt * nzt * nres * H * B
    acc.u32("na3d workgroups", [total], 1 << 31)
    wg = _xcd_order(total, np.arange(total, dtype=np.int64))
    per = nxt * nyt * nzt
    t = wg // per
    zt, yt, xt = _blocked_tile(wg - t * per, nzt, nyt, nxt)
    res = t % nres
    t = t // nres
    h, b = t % H, t // H
    dz, dy, dx = dil
    gx, gy, gz = res % dx, (res // dx) % dy, res // (dx * dy)
    Lz = np.array([_sub_len(L[0], g, dz) for g in range(dz)])[gz]
    Ly = np.array([_sub_len(L[1], g, dy) for g in range(dy)])[gy]
    Lx = np.array([_sub_len(L[2], g, dx) for g in range(dx)])[gx]
    f = lambda a, g, d: np.array([_sub_first(org[a], i, d) for i in range(d)])[g]  # noqa: E731
    e = lambda a, g, d: np.array([_sub_end(org[a], ext[a], i, d) for i in range(d)])[g]  # noqa: E731
    qz0, qz1 = f(0, gz, dz), e(0, gz, dz)
    qy0, qy1 = f(1, gy, dy), e(1, gy, dy)
    qx0, qx1 = f(2, gx, dx), e(2, gx, dx)
    iz, y0, x0 = qz0 + zt, qy0 + yt * WY, qx0 + xt * WQX
    live = (iz < qz1) & (y0 < qy1) & (x0 < qx1)  # the rest return before any access
    # Batch and head enter every address as b * stride[0] + h * stride[4] and no mask
    # depends on them: the first and last of each bound the rest exactly.
    live &= ((h == 0) | (h == H - 1)) & ((b == 0) | (b == B - 1))
    sel = lambda a: a[live]  # noqa: E731
    iz, y0, x0, h, b, gx, gy, gz, Lz, Ly, Lx, qy1, qx1 = map(sel, (iz, y0, x0, h, b, gx, gy, gz, Lz, Ly, Lx, qy1, qx1))
    kz, ky = ker[0], ker[1]
    sz = _win_start(iz, Lz, kz)
    Y0 = _win_start(y0, Ly, ky)
    NR = _win_start(np.minimum(y0 + WY - 1, qy1 - 1), Ly, ky) + ky - Y0
    NQ = -(-NR // RPS)
    X0 = _win_start(x0, Lx, kx)
    acc.u32("y-union rows (<= 64: 32-bit stage masks)", NR, 65)
    col = lambda a: a[:, None]  # noqa: E731  (workgroup axis, then lanes of the whole workgroup)
    wave = np.arange(256)[None, :] // 64
    lane = np.arange(256)[None, :] % 64
    n16, g = lane & 15, lane >> 4
    # ---- Q and own-key loads (per tile tt of the wave)
    xw0 = col(x0) + wave * TX
    qx = xw0 + n16 % TX
    qxc = np.minimum(qx, col(qx1) - 1)
    rqx = col(gx) + dx * qxc
    rz = gz + dz * iz
    for tt in range(NTY):
        qyl = col(y0) + tt * TY + n16 // TX
        rqy = col(gy) + dy * np.minimum(qyl, col(qy1) - 1)
        for name, st in (("q", qs), ("k", ks)):
            p = col(b) * st[0] + col(rz) * st[1] + rqy * st[2] + rqx * st[3] + col(h) * st[4]
            for kk in range(D // 32):
                acc.add(name, 2 * (p + 32 * kk + 8 * g), 16)
        # ---- output of tile tt: queries inside the box only
        ok = (qyl < col(qy1)) & (qx < col(qx1))
        oz, oy, ox = col(rz) - org[0], col(gy) + dy * qyl - org[1], col(gx) + dx * qx - org[2]
        op = col(b) * os_[0] + oz * os_[1] + oy * os_[2] + ox * os_[3] + col(h) * os_[4]
        for db in range(D // 16):
            acc.add("out", 2 * (op + 16 * db + 4 * g), 8, ok)
    # ---- K/V stages: descriptor at (z slice, row group cp), lane offsets voff[j]
    for tensor, name, st in ((0, "k", ks), (1, "v", vs)):
        rowb = 2 * dy * st[2]
        for j in range(LPT):
            gc = j * NWX + wave
            reg = gc // RKB
            ten, row = reg // RPS, reg % RPS
            key = (gc % RKB) * KPK + lane // CPK
            c = (lane % CPK) ^ (key & 7)  # swz<64>
            keyok = (key < LW) & (col(X0) + key < col(Lx))
            voff = np.where(keyok, row * rowb + (col(gx) + dx * (col(X0) + key)) * st[3] * 2 + 16 * c, OOB)
            acc.lane_offsets("na3d dma", np.where(ten == tensor, voff, OOB))
            for cp_sel in ("first", "last"):
                cp = np.zeros_like(NQ) if cp_sel == "first" else NQ - 1
                nrow = np.minimum(np.maximum(NR - RPS * cp, 0), RPS)
                nrec = nrow * rowb
                acc.u32("na3d record count", nrec)
                for cz in (0, kz - 1):
                    base = 2 * (b * st[0] + h * st[4] + (gz + dz * (sz + cz)) * st[1] + (gy + dy * (Y0 + RPS * cp)) * st[2])
                    inrec = (ten == tensor) & (voff + 16 <= col(nrec))
                    acc.add(name, col(base) + voff, 16, inrec)
    return acc


def region_geom(KY: int) -> dict:
    """na3d.hip RegionGeom<KY>: the region kernel's LDS layout (head_dim 64)."""
    NRY, LW = 7 + KY, 15 + KY
    NK = -(-(NRY * LW) // 8) * 8
    REG_B = NK * 128
    NBUF = 3 if 3 * 2 * REG_B <= 160 * 1024 else 2
    return dict(NRY=NRY, LW=LW, NK=NK, REG_B=REG_B, STAGE_B=2 * REG_B, NDMA=2 * NK // 8,
                DPW=-(-(2 * NK // 8) // 8), NBUF=NBUF, LDS_B=NBUF * 2 * REG_B)


def region_z_walk(Lz: int, qz0: int, qz1: int, kz: int = 3) -> list:
    """The z walk of na3d_region_kernel for one residue class (the kernel's own
    closed forms: zhi_of, zlo_of, slot_z, the interior mask 0xF & ~(1 << IDLE) and
    the extra pass on slot IDLE), replayed stage by stage.  Returns a list of
    problems: a live tile in no computed slot or sharing a slot, a tile that does
    not start exactly at its first slice or finish at its last, more than four live."""
    assert kz == 3
    ws = lambda z: int(_win_start(z, Lz, kz))  # noqa: E731
    S0, S1 = ws(qz0), ws(qz1 - 1) + kz
    zbase = S0 - 1
    zhi = lambda s: qz1 - 1 if s >= Lz - kz else min(qz1 - 1, s + 1)  # noqa: E731
    zlo = lambda s: qz0 if s - kz + 1 <= 0 else max(qz0, s - kz + 1 + 1)  # noqa: E731
    slot_z = lambda k, zl: zl + ((k + zbase - zl) & 3)  # noqa: E731
    probs, started, finished, seen = [], {}, {}, {}
    for s in range(S0, S1):
        truth = [z for z in range(qz0, qz1) if ws(z) <= s < ws(z) + kz]
        zl, zh = zlo(s), zhi(s)
        if truth != list(range(zl, zh + 1)):
            probs.append(f"s={s}: live {truth} != [{zl}, {zh}]")
        idle = ((s - S0) + 3) & 3
        comp = {k for k in range(4) if k != idle}
        if zl <= s - 2 or zh >= s + 2:
            comp.add(idle)
        held = {}
        for k in range(4):
            z = slot_z(k, zl)
            if z <= zh:
                held[z] = k
                if (z - zbase) & 3 != k:
                    probs.append(f"s={s}: zq {z} in slot {k}")
                if k not in comp:
                    probs.append(f"s={s}: zq {z} (slot {k}) not computed")
                if ws(z) == s:
                    started[z] = started.get(z, 0) + 1
                if ws(z) + kz - 1 == s:
                    finished[z] = finished.get(z, 0) + 1
                seen[z] = seen.get(z, 0) + 1
        if sorted(held) != truth:
            probs.append(f"s={s}: slots hold {sorted(held)}, live {truth}")
        if len(truth) > 4:
            probs.append(f"s={s}: {len(truth)} live")
    for z in range(qz0, qz1):
        if started.get(z) != 1 or finished.get(z) != 1 or seen.get(z) != kz:
            probs.append(f"zq {z}: started {started.get(z)} finished {finished.get(z)} stages {seen.get(z)}")
    return probs


def region_fits_z(L0: int, dz: int, org0: int, ext0: int) -> bool:
    """The host's z condition of region_fits (na3d.hip), restated."""
    for g in range(dz):
        Lz = _sub_len(L0, g, dz)
        z0, z1 = _sub_first(org0, g, dz), _sub_end(org0, ext0, g, dz)
        if z1 <= z0:
            continue
        for s in range(int(_win_start(z0, Lz, 3)), int(_win_start(z1 - 1, Lz, 3)) + 3):
            live = [z for z in range(z0, z1) if _win_start(z, Lz, 3) <= s < _win_start(z, Lz, 3) + 3]
            lo, hi = min(live, default=1 << 30), max(live, default=-1)
            if len(live) > 4 or hi - lo + 1 != len(live) or lo < s - 2 or hi > s + 2 or (lo == s - 2 and hi == s + 2):
                return False
    return True


def na3d_region_launch(B, L, H, ker, dil, qs, ks, vs, os_, org=(0, 0, 0), ext=None, rope_zt=None,
                       lse=False) -> Access:
    """Every global access of one na3d_region_kernel launch (na3d.hip: launch_region,
    the work decode, the tile geometry (by, bx, the lane's query), the stage copies
    (doff, issue), the query and RoPE-table loads (load_q, load_rope), the output
    and lse stores (finish / flush)), plus the LDS extent of every read and copy."""
    D = 64
    ext = tuple(L) if ext is None else tuple(ext)
    kz, KY, kx = ker
    assert kz == 3 and KY in (3, 5, 7) and kx <= KY
    G = region_geom(KY)
    NRY, LW, REG_B, STAGE_B, NDMA, DPW = G["NRY"], G["LW"], G["REG_B"], G["STAGE_B"], G["NDMA"], G["DPW"]
    RB = LW * 128
    acc = Access()
    nq = [max(_sub_end(org[a], ext[a], g, dil[a]) - _sub_first(org[a], g, dil[a]) for g in range(dil[a]))
          for a in range(3)]
    nrx, nry = -(-nq[2] // 16), -(-nq[1] // 8)
    nres = dil[0] * dil[1] * dil[2]
    total = nrx * nry * nres * H * B
    acc.u32("na3d region workgroups", [total], 1 << 31)
    t = _xcd_order(total, np.arange(total, dtype=np.int64))
    rx = t % nrx
    t = t // nrx
    ry = t % nry
    t = t // nry
    res = t % nres
    t = t // nres
    h, b = t % H, t // H
    dz, dy, dx = dil
    gx, gy, gz = res % dx, (res // dx) % dy, res // (dx * dy)
    Lz = np.array([_sub_len(L[0], g, dz) for g in range(dz)])[gz]
    Ly = np.array([_sub_len(L[1], g, dy) for g in range(dy)])[gy]
    Lx = np.array([_sub_len(L[2], g, dx) for g in range(dx)])[gx]
    f = lambda a, g, d: np.array([_sub_first(org[a], i, d) for i in range(d)])[g]  # noqa: E731
    e = lambda a, g, d: np.array([_sub_end(org[a], ext[a], i, d) for i in range(d)])[g]  # noqa: E731
    qz0, qz1 = f(0, gz, dz), e(0, gz, dz)
    qy0, qy1 = f(1, gy, dy), e(1, gy, dy)
    qx0, qx1 = f(2, gx, dx), e(2, gx, dx)
    y0, x0 = qy0 + 8 * ry, qx0 + 16 * rx
    live = (qz0 < qz1) & (y0 < qy1) & (x0 < qx1)
    live &= ((h == 0) | (h == H - 1)) & ((b == 0) | (b == B - 1))
    sel = lambda a: a[live]  # noqa: E731
    (y0, x0, h, b, gx, gy, gz, Lz, Ly, Lx, qz0, qz1, qy1, qx1) = map(
        sel, (y0, x0, h, b, gx, gy, gz, Lz, Ly, Lx, qz0, qz1, qy1, qx1))
    RY0, RX0 = _win_start(y0, Ly, KY), _win_start(x0, Lx, kx)
    S0, S1 = _win_start(qz0, Lz, kz), _win_start(qz1 - 1, Lz, kz) + kz
    col = lambda a: a[:, None]  # noqa: E731
    wave = np.arange(512)[None, :] // 64
    lane = np.arange(512)[None, :] % 64
    n16, g = lane & 15, lane >> 4
    # ---- tile geometry
    yt, xt = col(y0) + 2 * (wave >> 1), col(x0) + 8 * (wave & 1)
    by = _win_start(np.minimum(yt, col(qy1) - 1), col(Ly), KY) - col(RY0)
    bx = np.where(wave & 1, np.minimum(_win_start(np.minimum(xt, col(qx1) - 1), col(Lx), kx) - col(RX0), LW - 16), 0)
    acc.u32("region: tile union row", by, NRY - KY)  # by + KY <= NRY - 1
    acc.u32("region: tile key column", bx, LW - 15)  # bx + 15 <= LW - 1
    # LDS: the largest K and V read offsets (row KY of the union, chunk slot 7) and the copies
    kmax = (by + KY) * RB + (bx + 15) * 128 + 16 * 7 + 16
    vmax = REG_B + (by + KY) * RB + (bx + 15) * 128 + 16 * 7 + 8 + 8
    acc.u32("region: LDS read past the stage", np.maximum(kmax, vmax), STAGE_B + 1)
    tq = n16 >> 3
    qyc, qxc = np.minimum(yt + tq, col(qy1) - 1), np.minimum(xt + (n16 & 7), col(qx1) - 1)
    qvalid = (yt + tq < col(qy1)) & (xt + (n16 & 7) < col(qx1))
    # ---- stage copies: doff (lane offsets) on the slice base of stages S0 and S1 - 1
    for j in range(DPW):
        J = 8 * j + wave
        isv = J >= NDMA // 2
        fk = 8 * np.where(isv, J - NDMA // 2, J) + lane // 8
        row, kc = fk // LW, fk % LW
        ok = (J < NDMA) & (fk < NRY * LW) & (col(RY0) + row < col(Ly)) & (col(RX0) + kc < col(Lx))
        acc.u32("region: LDS copy destination", np.where(J < NDMA, np.where(isv, REG_B + 1024 * (J - NDMA // 2),
                                                                             1024 * J) + 1024, 0), STAGE_B + 1)
        for name, st in (("k", ks), ("v", vs)):
            is_v = name == "v"
            doff = row * 2 * dy * st[2] + (col(gx) + dx * (col(RX0) + kc)) * 2 * st[3] + 16 * ((lane & 7) ^ (kc & 7))
            doff = np.where(ok & (isv == is_v), doff, OOB)
            acc.lane_offsets("region dma", doff)
            for s in (S0, S1 - 1):
                base = 2 * (b * st[0] + h * st[4] + (gz + dz * s) * st[1] + (gy + dy * RY0) * st[2])
                acc.add(name, col(base) + doff, 16, doff != OOB)
    # ---- queries (and RoPE tables), outputs and lse at the first and last query z
    for zq in (qz0, qz1 - 1):
        rz, ry_, rx_ = col(gz + dz * zq), col(gy) + dy * qyc, col(gx) + dx * qxc
        qp = 2 * (col(b) * qs[0] + col(h) * qs[4] + rz * qs[1] + ry_ * qs[2] + rx_ * qs[3])
        acc.add("q", qp + 16 * g, 16)
        acc.add("q", qp + 64 + 16 * g, 16)
        if rope_zt is not None:
            r = ((col(b) * rope_zt + (0 if rope_zt == 1 else rz)) * L[1] + ry_) * L[2] + rx_
            for tname in ("cos", "sin"):
                acc.add(tname, 4 * (r * 32 + 8 * g), 32)
        op = 2 * (col(b) * os_[0] + col(h) * os_[4] + (rz - org[0]) * os_[1] + (ry_ - org[1]) * os_[2] +
                  (rx_ - org[2]) * os_[3]) + 8 * g
        for db in range(4):
            acc.add("out", op + 32 * db, 8, qvalid)
        if lse:
            li = ((((col(b) * ext[0] + rz - org[0]) * ext[1] + ry_ - org[1]) * ext[2] + rx_ - org[2]) * H + col(h))
            acc.add("lse", 4 * li, 4, qvalid & (g == 0))
    return acc


def na3d_column_launch(B, L, H, qs, ks, vs, os_) -> Access:
    """Every global access of one na3d_column_kernel launch (na3d.hip: window (Z, 1, 1),
    head_dim 64; launch_column's grid of four waves per workgroup, the item decode
    (h, x, y, b) of each wave, its loads of the column's Q, K and V rows (lane l: row
    l / 8 + 8 c for c < 4 when below Z, 16-byte chunk l % 8) and the output stores).
    Offsets are 64-bit element offsets from each view's base."""
    Z, Y, X = L
    acc = Access()
    items = B * Y * X * H
    wgs = -(-items // 4)
    acc.u32("column grid", [wgs], 1 << 31)
    item = np.arange(wgs * 4, dtype=np.int64)
    item = item[item < items]  # the wave returns before any access
    h = item % H
    t = item // H
    x = t % X
    t //= X
    y = t % Y
    b = t // Y
    lane = np.arange(64, dtype=np.int64)
    r = (lane // 8)[:, None] + 8 * np.arange(4, dtype=np.int64)[None, :]
    live = r < Z
    for name, st in (("q", qs), ("k", ks), ("v", vs), ("out", os_)):
        base = b * st[0] + y * st[2] + x * st[3] + h * st[4]
        inner = (r * st[1] + 8 * (lane % 8)[:, None])[live]
        acc.add_sum(name, 2 * base, 2 * inner, 16)
    return acc


def _bilinear_i0(o, inv_f, n):
    """pixel.hip bilinear_src: the first source index of output coordinate o (fp32 as the
    kernel: src = (o + 0.5) * (1 / f) - 0.5, clamped at 0, truncated, capped at n - 1)."""
    src = (np.asarray(o, dtype=np.float32) + np.float32(0.5)) * inv_f - np.float32(0.5)
    src = np.maximum(src, np.float32(0.0))
    return np.minimum(src.astype(np.int64), n - 1)


def upsample_dw_gelu_launch(B, Z, Yc, Xc, C, f, cs, os_) -> tuple[Access, list]:
    """Every global access of one upsample_dw_gelu_kernel launch (pixel.hip), and its LDS
    stage indices: the host's workgroup shape (cgw channel groups, np columns, nxb
    workgroups per row), each thread's decode (cgb, xb, y, b; ci, pi), the staged runs
    (3 rows x ncol columns x cgw groups, STG per thread, the index clamped to nrun - 1)
    and the 9 stage indices a live thread reads.  Offsets are element offsets from each
    view's base.  Returns (Access, problems with the LDS indices)."""
    cg = C // 8
    cgw = next(d for d in range(16, 0, -1) if cg % d == 0)
    npx = 256 // cgw
    Y, X = Yc * f, Xc * f
    nxb = -(-X // npx)
    nrun_max = 3 * ((npx - 1) // f + 4) * cgw
    stg = 2 if nrun_max <= 512 else 4
    lds = []
    if nrun_max > 1024:
        lds.append(f"nrun bound {nrun_max} > 1024")
    inv_f = np.float32(1.0) / np.float32(f)
    blocks = B * Y * nxb * (cg // cgw)
    acc = Access()
    acc.u32("upsample grid", [blocks], 1 << 31)
    blk = np.arange(blocks, dtype=np.int64)
    cgb = blk % (cg // cgw)
    t = blk // (cg // cgw)
    xb = t % nxb
    t //= nxb
    y = t % Y
    b = t // Y
    tid = np.arange(256, dtype=np.int64)
    ci, pi = tid % cgw, tid // cgw
    x0 = (xb * npx)[:, None]
    xl = np.minimum(x0 + npx, X) - 1
    live = (pi[None, :] < npx) & (x0 + pi[None, :] <= xl)
    x = np.where(live, x0 + pi[None, :], xl)
    c0_of = lambda xx: np.minimum(_bilinear_i0(np.maximum(xx - 1, 0), inv_f, Xc), max(Xc - 3, 0))
    r0 = np.minimum(_bilinear_i0(np.maximum(y - 1, 0), inv_f, Yc), max(Yc - 3, 0))[:, None]
    cfirst, c0 = c0_of(x0), c0_of(x)
    ncol = c0_of(xl) - cfirst + 3
    nrun = 3 * ncol * cgw
    if (nrun > stg * 256).any():
        lds.append(f"nrun {int(nrun.max())} > {stg} x 256")
    for u in range(stg):
        s = np.minimum(tid[None, :] + 256 * u, nrun - 1)
        i, rem = s // (ncol * cgw), s % (ncol * cgw)
        soff = (np.minimum(r0 + i, Yc - 1) * cs[2] + np.minimum(cfirst + rem // cgw, Xc - 1) * cs[3] +
                8 * (cgb[:, None] * cgw + rem % cgw))
        for z in (0, Z - 1):
            acc.add("cond", 2 * (b[:, None] * cs[0] + z * cs[1] + soff), 16)
    for i in range(3):
        for j in range(3):
            tix = (i * ncol + c0 - cfirst + j) * cgw + ci[None, :]
            if ((tix < 0) | (tix >= nrun))[live].any():
                lds.append(f"tap ({i}, {j}) outside the staged runs")
    ch = 8 * (cgb[:, None] * cgw + ci[None, :])
    acc.add("weight", 2 * (8 * C + ch), 16)
    acc.add("weight", 2 * ch, 16)
    for z in (0, Z - 1):
        acc.add("out", 2 * (b[:, None] * os_[0] + z * os_[1] + y[:, None] * os_[2] + x * os_[3] + ch), 16, live)
    return acc, lds


def tensor_bytes(shape, strides, esize=2) -> int:
    """Bytes from a view's first element to one past its last (non-negative strides)."""
    if any(s == 0 for s in shape):
        return 0
    return esize * (sum((n - 1) * s for n, s in zip(shape, strides)) + 1)


def contiguous_strides(shape):
    st, acc = [], 1
    for n in reversed(shape):
        st.append(acc)
        acc *= n
    return list(reversed(st))


def production_block_launches(B, Z, Y, X, C, H, kernel, mlp_ratio=4, gated=True, cus=256, depthwise=False):
    """(name, Access, sizes) of every hand-written launch of one StrataBlock forward
    at inference with qk-norm (strata_amd/modules.py StrataBlock.forward,
    FusedNA3DAttention.attention): LN, qkv GEMM, pack (q and k, v read from qkv),
    NA3D (the region or general kernel; with depthwise, the alternate block's
    column kernel over window (Z, 1, 1)), the gate GEMM, proj + residual, LN,
    fc1 + GELU, fc2 + residual."""
    D = C // H
    M = B * Z * Y * X
    F = int(C * mlp_ratio)
    out = []
    out.append(("layer_norm 1", layer_norm_launch(M, C, C, C), {"x": span(M, C, C), "out": span(M, C, C)}))
    out.append(("qkv gemm", gemm_dma_launch(M, 3 * C, C, C, C, 3 * C, bias=True, cus=cus),
                gemm_sizes(M, 3 * C, C, C, C, 3 * C, bias=True)))
    out.append(("rope pack (q, k; qk-norm)", rope_pack_half_launch(B, Z, Y, X, H, D, 3 * C, 1),
                {"qkv": span(M, 3 * C, 3 * C), "q": 2 * M * C, "k": 2 * M * C, "tables": 4 * B * Y * X * D // 2}))
    tok = [Z * Y * X * H * D, Y * X * H * D, X * H * D, H * D, D]
    vst = [Z * Y * X * 3 * C, Y * X * 3 * C, X * 3 * C, 3 * C, D]
    if depthwise:
        acc, kname = na3d_column_launch(B, (Z, Y, X), H, tok, tok, vst, tok), "na3d (column kernel)"
    elif kernel[0] == 3 and kernel[1] == 3 and kernel[2] <= 3 and region_fits_z(Z, 1, 0, Z):
        acc, kname = na3d_region_launch(B, (Z, Y, X), H, kernel, (1, 1, 1), tok, tok, vst, tok), "na3d (region kernel)"
    else:
        acc, kname = na3d_general_launch(B, (Z, Y, X), H, kernel, (1, 1, 1), tok, tok, vst, tok), "na3d (general kernel)"
    # v is the view qkv[..., 2, :, :]: its base is 2C elements into the qkv allocation
    vsz = span(M, 3 * C, 3 * C) - 2 * 2 * C
    out.append((kname, acc, {"q": 2 * M * C, "k": 2 * M * C, "v": vsz, "out": 2 * M * C}))
    if gated:
        out.append(("gate gemm (sigmoid, x residual)", gemm_dma_launch(M, C, C, C, C, C, C, bias=True, cus=cus),
                    gemm_sizes(M, C, C, C, C, C, C, bias=True)))
    out.append(("proj gemm + residual", gemm_dma_launch(M, C, C, C, C, C, C, bias=True, cus=cus),
                gemm_sizes(M, C, C, C, C, C, C, bias=True)))
    out.append(("layer_norm 2", layer_norm_launch(M, C, C, C), {"x": span(M, C, C), "out": span(M, C, C)}))
    out.append(("fc1 gemm + gelu", gemm_dma_launch(M, F, C, C, C, F, bias=True, cus=cus),
                gemm_sizes(M, F, C, C, C, F, bias=True)))
    out.append(("fc2 gemm + residual", gemm_dma_launch(M, C, F, F, F, C, C, bias=True, cus=cus),
                gemm_sizes(M, C, F, F, F, C, C, bias=True)))
    return out


def cdiv(a, b):
    return -(-a // b)


__all__ = ["Access", "OOB", "gemm_dma_launch", "gemm_sizes", "gemm_tile_origins", "layer_norm_launch",
           "rope_pack_half_launch", "na3d_general_launch", "na3d_column_launch", "production_block_launches", "span", "tensor_bytes",
           "contiguous_strides", "cdiv", "math"]
