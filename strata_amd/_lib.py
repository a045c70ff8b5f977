"""ctypes binding of ``libstrata_hip.so`` (C ABI declared in ``include/strata_hip.h``).

The structures below mirror the header field for field.  The library is
loaded lazily, after ``torch`` so that it binds to the HIP runtime torch
already loaded (both carry the SONAME ``libamdhip64.so.7``).  There is no
fallback: if the library is missing every op raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libstrata_hip.so"

ABI_VERSION = 6

OK = 0
EINVAL = -1
EUNSUPPORTED = -2
ELAUNCH = -3

F32 = 0
BF16 = 1

ACT_NONE = 0
ACT_GELU_TANH = 1
ACT_GELU_ERF = 2
ACT_SIGMOID = 3
ACT_GELU_TANH_GRAD = 4
ACT_SIGMOID_GRAD = 5

RES_ADD = 0
RES_MUL = 1

ROPE_HALF = 0
ROPE_INTERLEAVED = 1

_i32x3 = ctypes.c_int32 * 3
_i64x5 = ctypes.c_int64 * 5


class Na3dArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("grid", _i32x3),
        ("q_origin", _i32x3),
        ("q_extent", _i32x3),
        ("kernel", _i32x3),
        ("dilation", _i32x3),
        ("reserved", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("reserved_f", ctypes.c_float),
        ("q_stride", _i64x5),
        ("k_stride", _i64x5),
        ("v_stride", _i64x5),
        ("o_stride", _i64x5),
        ("lse", ctypes.c_void_p),
    ]


class RopePackArgs(ctypes.Structure):
    _fields_ = [
        ("qkv", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("grid", _i32x3),
        ("table_z", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("qkv_row_stride", ctypes.c_int64),
        ("qk_norm", ctypes.c_int32),
        ("qk_norm_eps", ctypes.c_float),
        ("q_norm_weight", ctypes.c_void_p),
        ("k_norm_weight", ctypes.c_void_p),
    ]


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("residual", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("m", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("ldx", ctypes.c_int64),
        ("ldw", ctypes.c_int64),
        ("ldr", ctypes.c_int64),
        ("ldo", ctypes.c_int64),
        ("act", ctypes.c_int32),
        ("res_op", ctypes.c_int32),
    ]


class LayerNormArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("m", ctypes.c_int64),
        ("c", ctypes.c_int64),
        ("ldx", ctypes.c_int64),
        ("ldo", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class UpsampleDwGeluArgs(ctypes.Structure):
    _fields_ = [
        ("cond", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("factor", ctypes.c_int32),
        ("cond_stride", ctypes.c_int64 * 4),
        ("out_stride", ctypes.c_int64 * 4),
    ]


class LayerNormModulateArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("shift", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("m", ctypes.c_int64),
        ("c", ctypes.c_int64),
        ("ldx", ctypes.c_int64),
        ("ldo", ctypes.c_int64),
        ("ld_shift", ctypes.c_int64),
        ("ld_scale", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class GatedAddArgs(ctypes.Structure):
    _fields_ = [
        ("res", ctypes.c_void_p),
        ("gate", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("m", ctypes.c_int64),
        ("c", ctypes.c_int64),
        ("ld_res", ctypes.c_int64),
        ("ld_gate", ctypes.c_int64),
        ("ld_y", ctypes.c_int64),
        ("ld_out", ctypes.c_int64),
    ]


# Every function the header declares, with its ctypes signature.
class CubePadArgs(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p),
        ("dst", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("face_size", ctypes.c_int32),
        ("pad", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("lead", ctypes.c_int64),
    ]


class CubeCropArgs(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p),
        ("dst", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("extent", ctypes.c_int32),
        ("halo", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("planes", ctypes.c_int64),
    ]


class Na3dBwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("dout", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("grid", ctypes.c_int32 * 3),
        ("kernel", ctypes.c_int32 * 3),
        ("dilation", ctypes.c_int32 * 3),
        ("scale", ctypes.c_float),
        ("lse", ctypes.c_void_p),
    ]


class LayerNormBwdArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("dx", ctypes.c_void_p),
        ("m", ctypes.c_int64),
        ("c", ctypes.c_int64),
        ("ld", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class BiasGradArgs(ctypes.Structure):
    _fields_ = [
        ("g", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("m", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("ldg", ctypes.c_int64),
    ]


class RopePackBwdArgs(ctypes.Structure):
    _fields_ = [
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("dqkv", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("grid", ctypes.c_int32 * 3),
        ("table_z", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("dqkv_row_stride", ctypes.c_int64),
        ("qkv", ctypes.c_void_p),
        ("qkv_row_stride", ctypes.c_int64),
        ("q_norm_weight", ctypes.c_void_p),
        ("k_norm_weight", ctypes.c_void_p),
        ("dq_norm_weight", ctypes.c_void_p),
        ("dk_norm_weight", ctypes.c_void_p),
        ("qk_norm", ctypes.c_int32),
        ("qk_norm_eps", ctypes.c_float),
    ]


class DealiasAxisArgs(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_void_p),
        ("dst", ctypes.c_void_p),
        ("mean", ctypes.c_void_p),
        ("std", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("grid", ctypes.c_int32 * 3),
        ("axis", ctypes.c_int32),
        ("patch", ctypes.c_int32),
        ("taps", ctypes.c_int32),
        ("filter", ctypes.c_float * 16),
    ]


class StatePatchifyArgs(ctypes.Structure):
    _fields_ = [
        ("state", ctypes.c_void_p),
        ("tokens", ctypes.c_void_p),
        ("mean", ctypes.c_void_p),
        ("std", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("grid", ctypes.c_int32 * 3),
        ("patch", ctypes.c_int32 * 3),
    ]


class StateUpdateArgs(ctypes.Structure):
    _fields_ = [
        ("pred", ctypes.c_void_p),
        ("state", ctypes.c_void_p),
        ("next", ctypes.c_void_p),
        ("mean", ctypes.c_void_p),
        ("std", ctypes.c_void_p),
        ("src_channel", ctypes.c_void_p),
        ("clamp_min", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("state_channels", ctypes.c_int32),
        ("order", ctypes.c_int32),
        ("grid", ctypes.c_int32 * 3),
        ("patch", ctypes.c_int32 * 3),
    ]


EXPORTS = {
    "strata_hip_na3d_fwd": ([ctypes.POINTER(Na3dArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_na3d_fwd_rope_q": (
        [ctypes.POINTER(Na3dArgs), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p], ctypes.c_int),
    "strata_hip_na3d_fwd_rope_q_supported": (
        [ctypes.POINTER(Na3dArgs), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32], ctypes.c_int),
    "strata_hip_na3d_bwd": ([ctypes.POINTER(Na3dBwdArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_na3d_bwd_noalloc": ([ctypes.POINTER(Na3dBwdArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_rope_qkv_pack": ([ctypes.POINTER(RopePackArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_gemm_bias_act": ([ctypes.POINTER(GemmArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_gemm_gelu_save": ([ctypes.POINTER(GemmArgs), ctypes.c_void_p, ctypes.c_void_p], ctypes.c_int),
    "strata_hip_bias_grad": ([ctypes.POINTER(BiasGradArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_bias_grad_workspace": ([ctypes.c_int64, ctypes.c_int64], ctypes.c_int64),
    "strata_hip_layer_norm": ([ctypes.POINTER(LayerNormArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_layer_norm_bwd": ([ctypes.POINTER(LayerNormBwdArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_rope_qkv_pack_bwd": ([ctypes.POINTER(RopePackBwdArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_cube_pad_faces": ([ctypes.POINTER(CubePadArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_cube_crop": ([ctypes.POINTER(CubeCropArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_state_patchify": ([ctypes.POINTER(StatePatchifyArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_dealias_axis": ([ctypes.POINTER(DealiasAxisArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_state_update": ([ctypes.POINTER(StateUpdateArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_upsample_dw_gelu": ([ctypes.POINTER(UpsampleDwGeluArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_layer_norm_modulate": ([ctypes.POINTER(LayerNormModulateArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_gated_add": ([ctypes.POINTER(GatedAddArgs), ctypes.c_void_p], ctypes.c_int),
    "strata_hip_last_error": ([], ctypes.c_char_p),
    "strata_hip_abi_version": ([], ctypes.c_int),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class StrataHipError(RuntimeError):
    """Raised when the HIP library rejects a call or a launch fails."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def load() -> ctypes.CDLL:
    """Load the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (bind to torch's HIP runtime first)

        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python -m strata_amd._build`"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (argtypes, restype) in EXPORTS.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        ver = lib.strata_hip_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def call(name: str, args: ctypes.Structure, stream: int) -> None:
    lib = load()
    rc = getattr(lib, name)(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != OK:
        msg = lib.strata_hip_last_error().decode(errors="replace")
        if rc == EINVAL:
            raise ValueError(f"{name}: {msg}")
        raise StrataHipError(name, rc, msg)
