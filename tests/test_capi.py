"""The C-ABI library: loads, exports what include/strata_hip.h declares, its
structs match the ctypes mirrors byte for byte, and argument validation
rejects bad calls before touching the GPU (no GPU needed)."""

import ctypes
import re
import shutil
import subprocess

import pytest

from strata_amd import _lib

from .conftest import ROOT

HEADER = ROOT / "include" / "strata_hip.h"
STRUCTS = {
    "strata_hip_na3d_args": _lib.Na3dArgs,
    "strata_hip_na3d_bwd_args": _lib.Na3dBwdArgs,
    "strata_hip_layer_norm_bwd_args": _lib.LayerNormBwdArgs,
    "strata_hip_rope_pack_bwd_args": _lib.RopePackBwdArgs,
    "strata_hip_rope_pack_args": _lib.RopePackArgs,
    "strata_hip_gemm_args": _lib.GemmArgs,
    "strata_hip_bias_grad_args": _lib.BiasGradArgs,
    "strata_hip_layer_norm_args": _lib.LayerNormArgs,
    "strata_hip_cube_pad_args": _lib.CubePadArgs,
    "strata_hip_cube_crop_args": _lib.CubeCropArgs,
    "strata_hip_state_patchify_args": _lib.StatePatchifyArgs,
    "strata_hip_state_update_args": _lib.StateUpdateArgs,
    "strata_hip_dealias_axis_args": _lib.DealiasAxisArgs,
}


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built; run __graft_entry__.build()")
    return _lib.load()


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(strata_hip_\w+)\s*\(", text, flags=re.M))


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert names == set(_lib.EXPORTS), names ^ set(_lib.EXPORTS)
    for n in names:
        assert hasattr(lib, n), n
    assert lib.strata_hip_abi_version() == _lib.ABI_VERSION


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layout_matches_header(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, cls in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {}
    for line in out:
        if line:
            s, f, v = line.split()
            got[(s, f)] = int(v)
    for cname, cls in STRUCTS.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


def _na3d_args(**over):
    a = _lib.Na3dArgs()
    a.q = a.k = a.v = a.out = 0x1000
    a.dtype = _lib.BF16
    a.batch, a.heads, a.head_dim = 1, 2, 64
    a.grid[:] = [4, 8, 8]
    a.q_origin[:] = [0, 0, 0]
    a.q_extent[:] = [4, 8, 8]
    a.kernel[:] = [3, 3, 3]
    a.dilation[:] = [1, 1, 1]
    a.scale = 0.125
    for k, v in over.items():
        if isinstance(v, list):
            getattr(a, k)[:] = v
        else:
            setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "over, msg",
    [
        (dict(kernel=[2, 3, 3]), "odd"),
        (dict(kernel=[5, 3, 3]), "exceeds"),
        (dict(dilation=[1, 3, 3]), "exceeds"),
        (dict(dilation=[0, 1, 1]), "dilation"),
        (dict(q_extent=[4, 9, 8]), "box"),
        (dict(dtype=7), "dtype"),
        (dict(q=0), "null"),
    ],
)
def test_na3d_validation_rejects_before_launch(lib, over, msg):
    a = _na3d_args(**over)
    rc = lib.strata_hip_na3d_fwd(ctypes.byref(a), None)
    assert rc == _lib.EINVAL
    assert msg in lib.strata_hip_last_error().decode()


def test_bias_grad_validation_and_workspace(lib):
    assert lib.strata_hip_bias_grad_workspace(1000, 3072) == 3072  # one 1024-row chunk
    assert lib.strata_hip_bias_grad_workspace(131072, 1024) == 128 * 1024
    assert lib.strata_hip_bias_grad_workspace(0, 16) == 0
    b = _lib.BiasGradArgs()
    b.g = b.out = b.workspace = 0x1000
    b.m, b.n, b.ldg = 64, 12, 12  # n not a multiple of 8
    assert lib.strata_hip_bias_grad(ctypes.byref(b), None) == _lib.EINVAL
    assert "multiples of 8" in lib.strata_hip_last_error().decode()
    b.n, b.ldg, b.workspace = 16, 16, None
    assert lib.strata_hip_bias_grad(ctypes.byref(b), None) == _lib.EINVAL


def test_gemm_and_layernorm_validation(lib):
    g = _lib.GemmArgs()
    g.x = g.w = g.out = 0x1000
    g.m, g.n, g.k = 16, 16, 12  # k not a multiple of 8
    g.ldx = g.ldw = 12
    g.ldo = 16
    assert lib.strata_hip_gemm_bias_act(ctypes.byref(g), None) == _lib.EINVAL
    assert "multiple of 8" in lib.strata_hip_last_error().decode()
    ln = _lib.LayerNormArgs()
    ln.x = ln.out = 0x1000
    ln.m, ln.c, ln.ldx, ln.ldo, ln.eps = 4, 8192, 8192, 8192, 1e-6
    assert lib.strata_hip_layer_norm(ctypes.byref(ln), None) == _lib.EUNSUPPORTED
    r = _lib.RopePackArgs()
    r.qkv = r.cos = r.sin = r.q = r.k = r.v = 0x1000
    r.batch, r.heads, r.head_dim, r.layout, r.table_z = 1, 2, 64, 0, 3
    r.grid[:] = [4, 8, 8]
    r.qkv_row_stride = 384
    assert lib.strata_hip_rope_qkv_pack(ctypes.byref(r), None) == _lib.EINVAL
    assert "table_z" in lib.strata_hip_last_error().decode()
    r.table_z, r.qk_norm = 1, 2
    assert lib.strata_hip_rope_qkv_pack(ctypes.byref(r), None) == _lib.EINVAL
    assert "qk_norm" in lib.strata_hip_last_error().decode()
    r.qk_norm, r.head_dim, r.qkv_row_stride = 1, 48, 288  # D/16 = 3 is not a power of two
    assert lib.strata_hip_rope_qkv_pack(ctypes.byref(r), None) == _lib.EINVAL
    assert "power of two" in lib.strata_hip_last_error().decode()
    r.v = None  # v may be NULL (only q and k written): validation goes on to the next check
    assert lib.strata_hip_rope_qkv_pack(ctypes.byref(r), None) == _lib.EINVAL
    assert "power of two" in lib.strata_hip_last_error().decode()
    r.q = None  # q may be NULL as well (k only, the queries rotated inside NA3D): on to the next check
    assert lib.strata_hip_rope_qkv_pack(ctypes.byref(r), None) == _lib.EINVAL
    assert "power of two" in lib.strata_hip_last_error().decode()
    saved_k, r.k = r.k, None  # k is always written
    assert lib.strata_hip_rope_qkv_pack(ctypes.byref(r), None) == _lib.EINVAL
    assert "null pointer" in lib.strata_hip_last_error().decode()
    r.k = saved_k
    g.k = g.ldx = g.ldw = 16
    g.res_op = 5
    assert lib.strata_hip_gemm_bias_act(ctypes.byref(g), None) == _lib.EINVAL
    assert "res_op" in lib.strata_hip_last_error().decode()
    g.res_op, g.act = 0, 6
    assert lib.strata_hip_gemm_bias_act(ctypes.byref(g), None) == _lib.EINVAL
    assert "act" in lib.strata_hip_last_error().decode()
    # output rows are written 16 bytes at a time: a row stride of 4 mod 8 elements, or an
    # output 8 but not 16-byte aligned, is refused before any launch
    g.act, g.ldo = 0, 20
    assert lib.strata_hip_gemm_bias_act(ctypes.byref(g), None) == _lib.EINVAL
    assert "multiples of 8" in lib.strata_hip_last_error().decode()
    g.ldo, g.out = 16, 0x1008
    assert lib.strata_hip_gemm_bias_act(ctypes.byref(g), None) == _lib.EINVAL
    assert "16-byte aligned" in lib.strata_hip_last_error().decode()


def test_empty_problem_is_a_no_op(lib):
    a = _na3d_args(batch=0)
    assert lib.strata_hip_na3d_fwd(ctypes.byref(a), None) == _lib.OK


def test_empty_problems_return_before_any_launch(lib):
    """Zero rows (or batch 0) is a valid call for every compute entry point: it returns OK
    without touching the device (this container has none, so a launch would fail)."""
    g = _lib.GemmArgs()
    g.k, g.ldx, g.ldw, g.ldo, g.n = 64, 64, 64, 128, 128  # m = 0
    assert lib.strata_hip_gemm_bias_act(ctypes.byref(g), None) == _lib.OK, lib.strata_hip_last_error()
    ln = _lib.LayerNormArgs()
    ln.x = ln.out = 0x1000
    ln.c, ln.ldx, ln.ldo, ln.eps = 1024, 1024, 1024, 1e-6  # m = 0
    assert lib.strata_hip_layer_norm(ctypes.byref(ln), None) == _lib.OK, lib.strata_hip_last_error()
    lm = _lib.LayerNormModulateArgs()
    lm.x = lm.out = lm.shift = lm.scale = 0x1000
    lm.c = lm.ldx = lm.ldo = lm.ld_shift = lm.ld_scale = 128
    lm.eps = 1e-6
    assert lib.strata_hip_layer_norm_modulate(ctypes.byref(lm), None) == _lib.OK, lib.strata_hip_last_error()
    ga = _lib.GatedAddArgs()
    ga.res = ga.gate = ga.y = ga.out = 0x1000
    ga.c = ga.ld_res = ga.ld_gate = ga.ld_y = ga.ld_out = 128
    assert lib.strata_hip_gated_add(ctypes.byref(ga), None) == _lib.OK, lib.strata_hip_last_error()
    up = _lib.UpsampleDwGeluArgs()
    up.cond = up.out = up.weight = 0x1000
    up.batch, up.depth, up.height, up.width, up.channels, up.factor = 0, 4, 4, 4, 64, 4
    up.cond_stride[:] = [4 * 4 * 4 * 64, 4 * 4 * 64, 4 * 64, 64]
    up.out_stride[:] = [4 * 16 * 16 * 64, 16 * 16 * 64, 16 * 64, 64]
    assert lib.strata_hip_upsample_dw_gelu(ctypes.byref(up), None) == _lib.OK, lib.strata_hip_last_error()
    b = _lib.Na3dBwdArgs()
    b.q = b.k = b.v = b.out = b.dout = b.dq = b.dk = b.dv = b.workspace = 0x1000
    b.dtype, b.batch, b.heads, b.head_dim, b.scale = _lib.BF16, 0, 2, 64, 0.125
    b.grid[:], b.kernel[:], b.dilation[:] = [4, 8, 8], [3, 3, 3], [1, 1, 1]
    assert lib.strata_hip_na3d_bwd(ctypes.byref(b), None) == _lib.OK, lib.strata_hip_last_error()
    r = _lib.RopePackArgs()
    r.qkv = r.cos = r.sin = r.q = r.k = r.v = 0x1000
    r.batch, r.table_z, r.heads, r.head_dim, r.layout, r.qkv_row_stride = 0, 1, 2, 64, _lib.ROPE_HALF, 384
    r.grid[:] = [4, 8, 8]
    assert lib.strata_hip_rope_qkv_pack(ctypes.byref(r), None) == _lib.OK, lib.strata_hip_last_error()


def test_cube_validation(lib):
    a = _lib.CubePadArgs()
    a.src, a.dst, a.dtype, a.face_size, a.pad, a.lead = 0x1000, 0x2000, _lib.F32, 8, 9, 1
    assert lib.strata_hip_cube_pad_faces(ctypes.byref(a), None) == _lib.EINVAL
    assert "pad wider" in lib.strata_hip_last_error().decode()
    a.pad, a.dst = 2, 0x1000
    assert lib.strata_hip_cube_pad_faces(ctypes.byref(a), None) == _lib.EINVAL
    assert "alias" in lib.strata_hip_last_error().decode()
    a.dtype = 7
    assert lib.strata_hip_cube_pad_faces(ctypes.byref(a), None) == _lib.EINVAL
    c = _lib.CubeCropArgs()
    c.src, c.dst, c.dtype, c.extent, c.halo, c.planes = 0x1000, 0x2000, _lib.BF16, 8, 4, 3
    assert lib.strata_hip_cube_crop(ctypes.byref(c), None) == _lib.EINVAL
    assert "2*halo" in lib.strata_hip_last_error().decode()
    c.planes, c.halo = 0, 1
    assert lib.strata_hip_cube_crop(ctypes.byref(c), None) == _lib.OK


def test_state_step_validation(lib):
    a = _lib.StatePatchifyArgs()
    a.state, a.tokens, a.batch, a.channels = 0x1000, 0x2000, 1, 4
    a.grid[:] = [4, 8, 8]
    a.patch[:] = [1, 3, 2]
    assert lib.strata_hip_state_patchify(ctypes.byref(a), None) == _lib.EINVAL
    assert "multiple of the patch" in lib.strata_hip_last_error().decode()
    a.patch[:] = [1, 2, 2]
    a.mean = 0x3000
    assert lib.strata_hip_state_patchify(ctypes.byref(a), None) == _lib.EINVAL
    assert "mean and std" in lib.strata_hip_last_error().decode()
    a.mean, a.channels = None, 20000
    assert lib.strata_hip_state_patchify(ctypes.byref(a), None) == _lib.EUNSUPPORTED
    a.channels, a.batch = 4, 0
    assert lib.strata_hip_state_patchify(ctypes.byref(a), None) == _lib.OK
    u = _lib.StateUpdateArgs()
    u.pred, u.next, u.batch, u.channels, u.order = 0x1000, 0x2000, 1, 4, 2
    u.grid[:] = [4, 8, 8]
    u.patch[:] = [1, 2, 2]
    u.state, u.state_channels = 0x3000, 4
    assert lib.strata_hip_state_update(ctypes.byref(u), None) == _lib.EINVAL
    assert "order" in lib.strata_hip_last_error().decode()
    u.order, u.state_channels = 1, 3
    assert lib.strata_hip_state_update(ctypes.byref(u), None) == _lib.EINVAL
    assert "fewer channels" in lib.strata_hip_last_error().decode()
    u.state_channels, u.state = 4, None
    assert lib.strata_hip_state_update(ctypes.byref(u), None) == _lib.EINVAL
    u.state, u.batch = 0x3000, 0
    assert lib.strata_hip_state_update(ctypes.byref(u), None) == _lib.OK


def test_na3d_bwd_validation(lib):
    a = _lib.Na3dBwdArgs()
    a.dtype, a.batch, a.heads, a.head_dim, a.scale = _lib.BF16, 1, 2, 64, 0.125
    a.grid[:] = [4, 8, 8]
    a.kernel[:] = [3, 5, 4]
    a.dilation[:] = [1, 1, 1]
    assert lib.strata_hip_na3d_bwd(ctypes.byref(a), None) == _lib.EINVAL
    assert "odd" in lib.strata_hip_last_error().decode()
    a.kernel[:] = [3, 5, 5]
    a.dilation[:] = [1, 2, 1]
    assert lib.strata_hip_na3d_bwd(ctypes.byref(a), None) == _lib.EINVAL
    assert "exceeds" in lib.strata_hip_last_error().decode()
    a.dilation[:] = [1, 1, 1]
    assert lib.strata_hip_na3d_bwd(ctypes.byref(a), None) == _lib.EINVAL
    assert "null" in lib.strata_hip_last_error().decode()
    for name in ("q", "k", "v", "out", "dout", "dq", "dk", "dv", "workspace"):
        setattr(a, name, 0x1000)
    a.head_dim = 48
    assert lib.strata_hip_na3d_bwd(ctypes.byref(a), None) == _lib.EUNSUPPORTED
    a.batch = 0
    assert lib.strata_hip_na3d_bwd(ctypes.byref(a), None) == _lib.OK


def test_rope_pack_bwd_qk_norm_validation(lib):
    a = _lib.RopePackBwdArgs()
    a.dq = a.dk = a.dv = a.cos = a.sin = a.dqkv = 0x1000
    a.batch, a.heads, a.head_dim, a.layout, a.table_z = 1, 2, 64, _lib.ROPE_HALF, 1
    a.grid[:] = [4, 8, 8]
    a.dqkv_row_stride = 384
    a.q_norm_weight = 0x2000  # a weight without qk_norm
    assert lib.strata_hip_rope_qkv_pack_bwd(ctypes.byref(a), None) == _lib.EINVAL
    assert "without qk_norm" in lib.strata_hip_last_error().decode()
    a.qk_norm = 1  # the forward's qkv is needed to recompute the norms
    assert lib.strata_hip_rope_qkv_pack_bwd(ctypes.byref(a), None) == _lib.EINVAL
    assert "forward's qkv" in lib.strata_hip_last_error().decode()
    a.qkv, a.qkv_row_stride = 0x3000, 384
    assert lib.strata_hip_rope_qkv_pack_bwd(ctypes.byref(a), None) == _lib.EINVAL
    assert "accumulator" in lib.strata_hip_last_error().decode()
    a.dq_norm_weight = 0x4000
    a.head_dim, a.dqkv_row_stride, a.qkv_row_stride = 48, 288, 288  # D/16 = 3
    assert lib.strata_hip_rope_qkv_pack_bwd(ctypes.byref(a), None) == _lib.EINVAL
    assert "power of two" in lib.strata_hip_last_error().decode()
    a.head_dim, a.dqkv_row_stride, a.qkv_row_stride, a.batch = 64, 384, 384, 0
    assert lib.strata_hip_rope_qkv_pack_bwd(ctypes.byref(a), None) == _lib.OK


def test_dealias_axis_validation(lib):
    a = _lib.DealiasAxisArgs()
    a.src, a.dst = 0x1000, 0x2000
    a.batch, a.channels, a.axis, a.patch, a.taps = 1, 3, 1, 3, 5
    a.grid[:] = [4, 8, 8]
    assert lib.strata_hip_dealias_axis(ctypes.byref(a), None) == _lib.EINVAL  # 3 does not divide 8
    assert "divide" in lib.strata_hip_last_error().decode()
    a.patch, a.taps = 2, 17
    assert lib.strata_hip_dealias_axis(ctypes.byref(a), None) == _lib.EINVAL
    assert "taps" in lib.strata_hip_last_error().decode()
    a.taps, a.axis = 5, 3
    assert lib.strata_hip_dealias_axis(ctypes.byref(a), None) == _lib.EINVAL
    assert "axis" in lib.strata_hip_last_error().decode()
    a.axis, a.dst = 1, 0x1000
    assert lib.strata_hip_dealias_axis(ctypes.byref(a), None) == _lib.EINVAL
    assert "alias" in lib.strata_hip_last_error().decode()
    a.dst, a.mean = 0x2000, 0x3000
    assert lib.strata_hip_dealias_axis(ctypes.byref(a), None) == _lib.EINVAL
    assert "both" in lib.strata_hip_last_error().decode()
    a.mean, a.batch = None, 0
    assert lib.strata_hip_dealias_axis(ctypes.byref(a), None) == _lib.OK


def test_na3d_rope_q_validation(lib):
    """The fused query-RoPE entry point checks its tables before launching (no GPU needed)."""
    a = _lib.Na3dArgs()
    a.q = a.k = a.v = a.out = 4096
    a.dtype, a.batch, a.heads, a.head_dim = _lib.BF16, 1, 2, 64
    a.grid[:] = [4, 16, 16]
    a.q_extent[:] = [4, 16, 16]
    a.kernel[:] = [3, 7, 7]
    a.dilation[:] = [1, 1, 1]
    a.scale = 0.125
    for st in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        st[:] = [4 * 16 * 16 * 128, 16 * 16 * 128, 16 * 128, 128, 64]
    assert lib.strata_hip_na3d_fwd_rope_q(ctypes.byref(a), None, None, 1, None) == _lib.EINVAL
    assert "null cos" in lib.strata_hip_last_error().decode()
    assert lib.strata_hip_na3d_fwd_rope_q(ctypes.byref(a), 4096, 4104, 1, None) == _lib.EINVAL
    assert "16-byte aligned" in lib.strata_hip_last_error().decode()
    assert lib.strata_hip_na3d_fwd_rope_q(ctypes.byref(a), 4096, 8192, 3, None) == _lib.EINVAL
    assert "table_z" in lib.strata_hip_last_error().decode()
    assert lib.strata_hip_na3d_fwd_rope_q_supported(ctypes.byref(a), 4096, 8192, 1) == 1
    a.kernel[:] = [3, 13, 13]  # the wide-window strip kernels carry no query rotation
    assert lib.strata_hip_na3d_fwd_rope_q_supported(ctypes.byref(a), 4096, 8192, 1) == 0
    assert lib.strata_hip_na3d_fwd_rope_q(ctypes.byref(a), 4096, 8192, 1, None) == _lib.EUNSUPPORTED
    a.kernel[:] = [3, 7, 7]
    a.dtype = _lib.F32
    assert lib.strata_hip_na3d_fwd_rope_q_supported(ctypes.byref(a), 4096, 8192, 1) == 0
