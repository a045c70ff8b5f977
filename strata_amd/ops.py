"""PyTorch-ROCm custom ops ``torch.ops.strata_hip.*`` over the C-ABI HIP library.

Each op validates its tensors, allocates the output through torch's caching
allocator, and enqueues the kernel on torch's current stream of the input's
device.  There is no CPU or eager fallback: CPU tensors are rejected and a
missing library raises.  Every op has a fake (meta) implementation so that
``torch.compile`` traces through it.  ``na3d_fwd`` (full-grid queries),
``gemm_bias_act`` (act none / GELU(tanh) with an added residual, and the
sigmoid gate), ``layer_norm`` and ``rope_qkv_pack`` (with or without qk_norm)
have backwards on HIP kernels; the other ops' autograd formulas raise.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import torch
from torch import Tensor

from . import _lib

__all__ = [
    "na3d_fwd",
    "na3d_bwd",
    "na3d_fwd_lse",
    "na3d",
    "rope_qkv_pack",
    "gemm_bias_act",
    "gemm_gelu_train",
    "bias_grad",
    "layer_norm",
    "cube_pad_faces",
    "cube_crop",
    "state_patchify",
    "dealias_axis",
    "state_update",
    "upsample_dw_gelu",
    "layer_norm_modulate",
    "gated_add",
]


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(name: str, *ts: Optional[Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{name}: expected GPU tensors, got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{name}: tensors on different devices ({dev} and {t.device})")
    return dev


def _dtype_code(name: str, t: Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    if t.dtype == torch.float32:
        return _lib.F32
    raise ValueError(f"{name}: dtype must be bfloat16 or float32, got {t.dtype}")


def _triple(name: str, v: Sequence[int] | int) -> list[int]:
    if isinstance(v, int):
        return [v, v, v]
    v = [int(x) for x in v]
    if len(v) != 3:
        raise ValueError(f"{name} must have 3 entries, got {v}")
    return v


def _token_strides(name: str, t: Tensor) -> list[int]:
    if t.dim() != 6:
        raise ValueError(f"{name}: expected a heads-last [B, Z, Y, X, H, D] tensor, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: the head_dim axis must be contiguous (stride 1)")
    return [t.stride(i) for i in range(5)]


def _no_backward(op_name: str):
    def backward(ctx, *grads):
        raise RuntimeError(f"{op_name} is forward-only (inference kernels); no backward is implemented")

    return backward


# ---------------------------------------------------------------------------
# NA3D
# ---------------------------------------------------------------------------
@torch.library.custom_op("strata_hip::na3d_fwd", mutates_args=())
def na3d_fwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kernel: Sequence[int],
    dilation: Sequence[int],
    scale: Optional[float],
    q_origin: Sequence[int],
    q_extent: Sequence[int],
) -> Tensor:
    """Neighbourhood attention over a clamped 3D window (NATTEN ``na3d`` semantics).

    q, k, v: heads-last ``[B, Z, Y, X, H, D]`` on one GPU, bf16 or fp32.
    Only queries in the box ``[q_origin, q_origin + q_extent)`` are computed;
    the result has shape ``[B, *q_extent, H, D]`` and equals
    ``natten.na3d(q, k, v, kernel, dilation=dilation, scale=scale)`` cropped to
    the box.  Replaces NATTEN 0.21.5 ``na3d`` (pins docker/build_natten.sh:21,
    Makefile:11; call routed by screamcast/config.py:99 -> train.py:143 ->
    screamcast/strata_wrappers.py:331,490,582).
    """
    return _na3d_launch("na3d_fwd", q, k, v, kernel, dilation, scale, q_origin, q_extent, None)


def _na3d_launch(name, q, k, v, kernel, dilation, scale, q_origin, q_extent, lse: Optional[Tensor]) -> Tensor:
    _require_gpu(name, q, k, v)
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"{name}: q, k, v must share one shape, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"{name}: q, k, v must share one dtype")
    dt = _dtype_code(name, q)
    qs, ks, vs = _token_strides(name, q), _token_strides(name, k), _token_strides(name, v)
    B, Z, Y, X, H, D = q.shape
    kernel, dilation = _triple("kernel", kernel), _triple("dilation", dilation)
    q_origin, q_extent = _triple("q_origin", q_origin), _triple("q_extent", q_extent)
    out = torch.empty((B, *q_extent, H, D), dtype=q.dtype, device=q.device)
    if out.numel() == 0:
        return out
    a = _na3d_args(q, k, v, out, dt, qs, ks, vs, kernel, dilation, scale, q_origin, q_extent)
    a.lse = lse.data_ptr() if lse is not None else None
    with torch.cuda.device(q.device):
        _lib.call("strata_hip_na3d_fwd", a, _stream(q))
    return out


def _na3d_args(q, k, v, out, dt, qs, ks, vs, kernel, dilation, scale, q_origin, q_extent) -> "_lib.Na3dArgs":
    B, Z, Y, X, H, D = q.shape
    a = _lib.Na3dArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.dtype = dt
    a.batch, a.heads, a.head_dim = B, H, D
    a.grid[:] = [Z, Y, X]
    a.q_origin[:] = q_origin
    a.q_extent[:] = q_extent
    a.kernel[:] = kernel
    a.dilation[:] = dilation
    a.scale = float(D**-0.5 if scale is None else scale)
    a.q_stride[:] = qs
    a.k_stride[:] = ks
    a.v_stride[:] = vs
    a.o_stride[:] = [out.stride(i) for i in range(5)]
    a.lse = None
    return a


def _rope_q_tables(name, q, cos, sin):
    B, Z, Y, X, H, D = q.shape
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise ValueError(f"{name}: cos/sin tables must be float32")
    if cos.shape != sin.shape or cos.dim() != 5 or tuple(cos.shape[2:]) != (Y, X, D // 2) or cos.shape[0] != B \
            or cos.shape[1] not in (1, Z):
        raise ValueError(f"{name}: cos/sin must be [B, 1|Z, Y, X, D/2] = [{B}, 1|{Z}, {Y}, {X}, {D // 2}], "
                         f"got {tuple(cos.shape)}")
    return cos.contiguous(), sin.contiguous(), int(cos.shape[1])


def na3d_rope_q_supported(q: Tensor, k_strides: Sequence[int], v: Tensor, cos: Tensor, sin: Tensor,
                          kernel: Sequence[int], dilation: Sequence[int], scale: Optional[float] = None) -> bool:
    """Whether ``na3d_fwd_rope_q`` takes these shapes, strides and window (the
    small-window kernels: bf16, head_dim 64, half-layout tables); k is described by
    its strides only (the k-only pack writes it contiguous)."""
    name = "na3d_rope_q_supported"
    if not (q.is_cuda and v.is_cuda and cos.is_cuda and sin.is_cuda) or q.dtype != torch.bfloat16 \
            or v.dtype != torch.bfloat16 or q.dim() != 6 or q.shape != v.shape:
        return False
    try:
        cos_c, sin_c, zt = _rope_q_tables(name, q, cos, sin)
        qs, vs = _token_strides(name, q), _token_strides(name, v)
    except ValueError:
        return False
    Z, Y, X = q.shape[1:4]
    kernel, dilation = _triple("kernel", kernel), _triple("dilation", dilation)
    # k's pointer is not dereferenced by the query; q's stands in for it (aligned alike)
    a = _na3d_args(q, q, v, q, _dtype_code(name, q), qs, list(k_strides), vs, kernel, dilation, scale, [0, 0, 0],
                   [Z, Y, X])
    a.o_stride[:] = list(k_strides)
    lib = _lib.load()
    return bool(lib.strata_hip_na3d_fwd_rope_q_supported(ctypes.byref(a), cos_c.data_ptr(), sin_c.data_ptr(), zt))


@torch.library.custom_op("strata_hip::na3d_fwd_rope_q", mutates_args=())
def na3d_fwd_rope_q(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor, kernel: Sequence[int],
                    dilation: Sequence[int], scale: Optional[float]) -> Tensor:
    """``na3d_fwd`` over the full grid with the queries' rotary embedding applied
    inside the kernel: q is unrotated (e.g. a strided view of the qkv output), k
    already rotated (``rope_qkv_pack(..., pack_q=False)``), cos/sin the half-layout
    tables ``[B, 1|Z, Y, X, D/2]`` fp32.  Equals ``na3d_fwd(rope(q), k, v)`` with
    rope(q) rounded to bf16 as the pack rounds it.  Inference only (no lse); raises
    for shapes ``na3d_rope_q_supported`` rejects.  Fuses the query half of the
    attention's RoPE (screamcast/strata_wrappers.py:331-338) into the NATTEN call."""
    name = "na3d_fwd_rope_q"
    _require_gpu(name, q, k, v, cos, sin)
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"{name}: q, k, v must share one shape")
    if not (q.dtype == k.dtype == v.dtype == torch.bfloat16):
        raise ValueError(f"{name}: q, k, v must be bfloat16")
    cos_c, sin_c, zt = _rope_q_tables(name, q, cos, sin)
    qs, ks, vs = _token_strides(name, q), _token_strides(name, k), _token_strides(name, v)
    B, Z, Y, X, H, D = q.shape
    kernel, dilation = _triple("kernel", kernel), _triple("dilation", dilation)
    out = torch.empty((B, Z, Y, X, H, D), dtype=q.dtype, device=q.device)
    if out.numel() == 0:
        return out
    a = _na3d_args(q, k, v, out, _dtype_code(name, q), qs, ks, vs, kernel, dilation, scale, [0, 0, 0], [Z, Y, X])
    lib = _lib.load()
    with torch.cuda.device(q.device):
        rc = lib.strata_hip_na3d_fwd_rope_q(ctypes.byref(a), cos_c.data_ptr(), sin_c.data_ptr(), zt,
                                            ctypes.c_void_p(_stream(q)))
    if rc != _lib.OK:
        msg = lib.strata_hip_last_error().decode(errors="replace")
        raise (ValueError if rc == _lib.EINVAL else _lib.StrataHipError)(
            *((f"{name}: {msg}",) if rc == _lib.EINVAL else ("strata_hip_na3d_fwd_rope_q", rc, msg)))
    return out


@na3d_fwd_rope_q.register_fake
def _(q, k, v, cos, sin, kernel, dilation, scale):
    return q.new_empty(q.shape)


@na3d_fwd.register_fake
def _(q, k, v, kernel, dilation, scale, q_origin, q_extent):
    B, H, D = q.shape[0], q.shape[4], q.shape[5]
    return q.new_empty((B, *[int(e) for e in q_extent], H, D))


@torch.library.custom_op("strata_hip::na3d_fwd_lse", mutates_args=())
def na3d_fwd_lse(
    q: Tensor, k: Tensor, v: Tensor, kernel: Sequence[int], dilation: Sequence[int], scale: Optional[float]
) -> tuple[Tensor, Tensor]:
    """``na3d_fwd`` over the whole grid that also returns each query's log2-sum-exp
    ``[B, Z, Y, X, H]`` fp32 (of the log2-unit scores ``scale*log2(e)*q.k``), the
    statistic the backward needs; its autograd passes it on so the backward does
    not recompute it.  ``na3d`` below picks this op when gradients are wanted."""
    B, Z, Y, X, H, D = q.shape
    lse = torch.empty((B, Z, Y, X, H), dtype=torch.float32, device=q.device)
    out = _na3d_launch("na3d_fwd_lse", q, k, v, kernel, dilation, scale, [0, 0, 0], [Z, Y, X], lse)
    return out, lse


@na3d_fwd_lse.register_fake
def _(q, k, v, kernel, dilation, scale):
    return q.new_empty(q.shape), q.new_empty(q.shape[:5], dtype=torch.float32)


@torch.library.custom_op("strata_hip::na3d_bwd", mutates_args=())
def na3d_bwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    out: Tensor,
    dout: Tensor,
    kernel: Sequence[int],
    dilation: Sequence[int],
    scale: Optional[float],
    lse: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """``(dq, dk, dv)`` of ``out = na3d(q, k, v)`` over the whole grid, given ``dout``
    (NATTEN 0.21.5's na3d backward, reached in training through train.py:1161).
    Heads-last ``[B, Z, Y, X, H, D]``, bf16 or fp32 (fp32 math), D in {32, 64, 128}.
    ``lse``: the forward's statistics from ``na3d_fwd_lse`` (else recomputed)."""
    name = "na3d_bwd"
    _require_gpu(name, q, k, v, out, dout)
    shape = q.shape
    for t, nm in ((k, "k"), (v, "v"), (out, "out"), (dout, "dout")):
        if t.shape != shape or t.dtype != q.dtype:
            raise ValueError(f"{name}: {nm} must match q ({tuple(shape)}, {q.dtype}), got {tuple(t.shape)}, {t.dtype}")
    dt = _dtype_code(name, q)
    if q.dim() != 6:
        raise ValueError(f"{name}: expected heads-last [B, Z, Y, X, H, D], got {tuple(shape)}")
    B, Z, Y, X, H, D = shape
    kernel, dilation = _triple("kernel", kernel), _triple("dilation", dilation)
    ins = [t.contiguous() for t in (q, k, v, out, dout)]
    dq, dk, dv = (torch.empty_like(ins[0]) for _ in range(3))
    if q.numel() == 0:
        return dq, dk, dv
    ws = torch.empty(2 * B * Z * Y * X * H, dtype=torch.float32, device=q.device)
    a = _lib.Na3dBwdArgs()
    a.q, a.k, a.v, a.out, a.dout = (t.data_ptr() for t in ins)
    a.dq, a.dk, a.dv, a.workspace = dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr()
    a.dtype = dt
    a.batch, a.heads, a.head_dim = B, H, D
    a.grid[:] = [Z, Y, X]
    a.kernel[:] = kernel
    a.dilation[:] = dilation
    a.scale = float(D**-0.5 if scale is None else scale)
    if lse is not None:
        if lse.shape != shape[:5] or lse.dtype != torch.float32 or lse.device != q.device:
            raise ValueError(f"{name}: lse must be float32 {tuple(shape[:5])} on {q.device}")
        lse = lse.contiguous()
        a.lse = lse.data_ptr()
    with torch.cuda.device(q.device):
        _lib.call("strata_hip_na3d_bwd", a, _stream(q))
    return dq, dk, dv


@na3d_bwd.register_fake
def _(q, k, v, out, dout, kernel, dilation, scale, lse=None):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


na3d_bwd.register_autograd(_no_backward("strata_hip::na3d_bwd"))


def _na3d_setup_context(ctx, inputs, output):
    q, k, v, kernel, dilation, scale, q_origin, q_extent = inputs
    ctx.full_grid = list(q_origin) == [0, 0, 0] and list(q_extent) == list(q.shape[1:4])
    ctx.kernel, ctx.dilation, ctx.scale = kernel, dilation, scale
    ctx.save_for_backward(q, k, v, output)


def _na3d_backward(ctx, dout):
    if not ctx.full_grid:
        raise RuntimeError("strata_hip::na3d_fwd: the backward covers full-grid queries only (no query box)")
    q, k, v, out = ctx.saved_tensors
    dq, dk, dv = na3d_bwd(q, k, v, out, dout.contiguous(), ctx.kernel, ctx.dilation, ctx.scale)
    return dq, dk, dv, None, None, None, None, None


na3d_fwd.register_autograd(_na3d_backward, setup_context=_na3d_setup_context)


def _na3d_lse_setup_context(ctx, inputs, output):
    q, k, v, kernel, dilation, scale = inputs
    out, lse = output
    ctx.kernel, ctx.dilation, ctx.scale = kernel, dilation, scale
    ctx.mark_non_differentiable(lse)
    ctx.save_for_backward(q, k, v, out, lse)


def _na3d_lse_backward(ctx, dout, dlse):
    q, k, v, out, lse = ctx.saved_tensors
    dq, dk, dv = na3d_bwd(q, k, v, out, dout.contiguous(), ctx.kernel, ctx.dilation, ctx.scale, lse)
    return dq, dk, dv, None, None, None


na3d_fwd_lse.register_autograd(_na3d_lse_backward, setup_context=_na3d_lse_setup_context)


def na3d(q: Tensor, k: Tensor, v: Tensor, kernel: Sequence[int], dilation: Sequence[int],
         scale: Optional[float] = None) -> Tensor:
    """Full-grid NA3D for modules: ``na3d_fwd_lse`` (forward statistics kept for
    the backward) when autograd will need them, else ``na3d_fwd``."""
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return na3d_fwd_lse(q, k, v, kernel, dilation, scale)[0]
    Z, Y, X = q.shape[1:4]
    return na3d_fwd(q, k, v, kernel, dilation, scale, [0, 0, 0], [Z, Y, X])


# ---------------------------------------------------------------------------
# RoPE + QKV pack
# ---------------------------------------------------------------------------
@torch.library.custom_op("strata_hip::rope_qkv_pack", mutates_args=())
def rope_qkv_pack(qkv: Tensor, cos: Tensor, sin: Tensor, heads: int, rope_layout: int, qk_norm: bool = False,
                  qk_norm_eps: float = 1e-6, q_norm_weight: Optional[Tensor] = None,
                  k_norm_weight: Optional[Tensor] = None, pack_v: bool = True,
                  pack_q: bool = True) -> tuple[Tensor, Tensor, Tensor]:
    """Split ``attn.qkv``'s output into heads-last q, k, v and rotate q, k.

    qkv: ``[B, Z, Y, X, 3*H*D]`` bf16 (column order (3, H, D), last dim
    contiguous, rows possibly strided).  cos, sin: fp32 ``[B, Zt, Y, X, D/2]``
    with Zt in {1, Z}.  rope_layout: 0 = half split (pair p = (p, p + D/2)),
    1 = interleaved (pair p = (2p, 2p+1)).  qk_norm: RMSNorm over D of each
    (token, head) of q and k before the rotation, ``x * rsqrt(mean(x^2) + eps)
    * weight`` (weights bf16 ``[D]`` or None; screamcast/config.py:91-93).
    Returns q, k, v ``[B, Z, Y, X, H, D]``.  pack_v=False leaves v out (an empty
    tensor is returned in its place): the caller reads v straight out of qkv as
    the strided view ``qkv.view(B, Z, Y, X, 3, H, D)[..., 2, :, :]``, which the
    NA3D op takes as it is, and the pack moves a third fewer bytes.
    pack_q=False leaves q out likewise, for ``na3d_fwd_rope_q``, which rotates the
    queries inside the attention kernel.
    """
    name = "rope_qkv_pack"
    _require_gpu(name, qkv, cos, sin)
    if qkv.dtype != torch.bfloat16:
        raise ValueError(f"{name}: qkv must be bfloat16")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32:
        raise ValueError(f"{name}: cos/sin tables must be float32")
    if qkv.dim() != 5:
        raise ValueError(f"{name}: qkv must be [B, Z, Y, X, 3C], got {tuple(qkv.shape)}")
    B, Z, Y, X, C3 = qkv.shape
    if C3 % (3 * heads):
        raise ValueError(f"{name}: last dim {C3} is not divisible by 3*heads")
    D = C3 // (3 * heads)
    if cos.shape != sin.shape or cos.dim() != 5 or tuple(cos.shape[2:]) != (Y, X, D // 2) or cos.shape[0] != B:
        raise ValueError(f"{name}: cos/sin must be [B, Zt, Y, X, D/2] = [{B}, 1|{Z}, {Y}, {X}, {D // 2}], got {tuple(cos.shape)}")
    # rows of qkv must be evenly strided over the flattened token index
    flat = qkv.reshape(B * Z * Y * X, C3) if not qkv.is_contiguous() else qkv.view(-1, C3)
    if flat.stride(1) != 1:
        raise ValueError(f"{name}: the last dim of qkv must be contiguous")
    cos_c, sin_c = cos.contiguous(), sin.contiguous()
    wts = []
    for t, nm in ((q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight")):
        if t is not None:
            if not qk_norm:
                raise ValueError(f"{name}: {nm} given without qk_norm")
            _require_gpu(name, t)
            if t.dtype != torch.bfloat16 or tuple(t.shape) != (D,):
                raise ValueError(f"{name}: {nm} must be bfloat16 [{D}]")
            t = t.contiguous()
        wts.append(t)
    shape = (B, Z, Y, X, heads, D)
    k = torch.empty(shape, dtype=qkv.dtype, device=qkv.device)
    q = torch.empty_like(k) if pack_q else k.new_empty(0)
    v = torch.empty_like(k) if pack_v else k.new_empty(0)
    if k.numel() == 0:
        return q, k, v
    a = _lib.RopePackArgs()
    a.qkv, a.cos, a.sin = flat.data_ptr(), cos_c.data_ptr(), sin_c.data_ptr()
    a.q, a.k, a.v = (q.data_ptr() if pack_q else None), k.data_ptr(), (v.data_ptr() if pack_v else None)
    a.batch = B
    a.grid[:] = [Z, Y, X]
    a.table_z = cos.shape[1]
    a.heads, a.head_dim, a.layout = heads, D, int(rope_layout)
    a.qkv_row_stride = flat.stride(0)
    a.qk_norm = 1 if qk_norm else 0
    a.qk_norm_eps = float(qk_norm_eps)
    a.q_norm_weight = wts[0].data_ptr() if wts[0] is not None else None
    a.k_norm_weight = wts[1].data_ptr() if wts[1] is not None else None
    with torch.cuda.device(qkv.device):
        _lib.call("strata_hip_rope_qkv_pack", a, _stream(qkv))
    return q, k, v


@rope_qkv_pack.register_fake
def _(qkv, cos, sin, heads, rope_layout, qk_norm=False, qk_norm_eps=1e-6, q_norm_weight=None, k_norm_weight=None,
      pack_v=True, pack_q=True):
    B, Z, Y, X, C3 = qkv.shape
    D = C3 // (3 * heads)
    shape = (B, Z, Y, X, heads, D)
    return (qkv.new_empty(shape if pack_q else (0,)), qkv.new_empty(shape),
            qkv.new_empty(shape if pack_v else (0,)))


def _rope_setup_context(ctx, inputs, output):
    qkv, cos, sin, heads, rope_layout, qk_norm, qk_norm_eps, q_norm_weight, k_norm_weight, pack_v, _pack_q = inputs
    ctx.qk_norm, ctx.heads, ctx.layout, ctx.pack_v = bool(qk_norm), int(heads), int(rope_layout), bool(pack_v)
    ctx.qk_norm_eps = float(qk_norm_eps)
    ctx.qkv_shape = tuple(qkv.shape)
    if ctx.qk_norm:  # the RMSNorm backward recomputes the norms from the input
        ctx.save_for_backward(cos, sin, qkv, q_norm_weight, k_norm_weight)
    else:
        ctx.save_for_backward(cos, sin)


def _rope_backward(ctx, dq, dk, dv):
    """d(qkv) = (R(-theta) dq, R(-theta) dk, dv) in qkv's (3, H, D) column layout;
    with qk_norm, q and k further through the RMSNorm backward (and the norm
    weights' gradients, summed over tokens and heads in fp32).  Without a dv
    (pack_v=False, or no gradient reached v) v's columns are zero: a v read as a
    view of qkv adds its own gradient there."""
    cos, sin = ctx.saved_tensors[:2]
    B, Z, Y, X, C3 = ctx.qkv_shape
    D = C3 // (3 * ctx.heads)
    grads = [g.contiguous() if (g is not None and g.numel()) else
             torch.zeros((B, Z, Y, X, ctx.heads, D), dtype=torch.bfloat16, device=cos.device) for g in (dq, dk)]
    dv = dv.contiguous() if (ctx.pack_v and dv is not None) else None
    dqkv = torch.empty(ctx.qkv_shape, dtype=torch.bfloat16, device=cos.device)
    a = _lib.RopePackBwdArgs()
    a.dq, a.dk = (g.data_ptr() for g in grads)
    a.dv = dv.data_ptr() if dv is not None else None
    cos_c, sin_c = cos.contiguous(), sin.contiguous()
    a.cos, a.sin, a.dqkv = cos_c.data_ptr(), sin_c.data_ptr(), dqkv.data_ptr()
    a.batch = B
    a.grid[:] = [Z, Y, X]
    a.table_z = cos.shape[1]
    a.heads, a.head_dim, a.layout = ctx.heads, D, ctx.layout
    a.dqkv_row_stride = C3
    dws = [None, None]
    if ctx.qk_norm:
        qkv, qw, kw = ctx.saved_tensors[2:]
        qkv = qkv.contiguous()
        a.qkv, a.qkv_row_stride = qkv.data_ptr(), C3
        a.qk_norm, a.qk_norm_eps = 1, ctx.qk_norm_eps
        for i, w in enumerate((qw, kw)):
            if w is not None:
                dws[i] = torch.zeros(D, dtype=torch.float32, device=cos.device)
        a.q_norm_weight = qw.data_ptr() if qw is not None else None
        a.k_norm_weight = kw.data_ptr() if kw is not None else None
        a.dq_norm_weight = dws[0].data_ptr() if dws[0] is not None else None
        a.dk_norm_weight = dws[1].data_ptr() if dws[1] is not None else None
    if dqkv.numel():
        with torch.cuda.device(cos.device):
            _lib.call("strata_hip_rope_qkv_pack_bwd", a, _stream(dqkv))
    if ctx.qk_norm:
        dws = [d.to(w.dtype) if d is not None else None for d, w in zip(dws, ctx.saved_tensors[3:])]
    return dqkv, None, None, None, None, None, None, dws[0], dws[1], None, None


rope_qkv_pack.register_autograd(_rope_backward, setup_context=_rope_setup_context)


# ---------------------------------------------------------------------------
# GEMM + bias + activation + residual
# ---------------------------------------------------------------------------
ACTS = {"none": _lib.ACT_NONE, "gelu_tanh": _lib.ACT_GELU_TANH, "gelu": _lib.ACT_GELU_ERF, "sigmoid": _lib.ACT_SIGMOID}


def _rows(name: str, t: Tensor, what: str) -> Tensor:
    """View t as a 2D [rows, cols] matrix with a contiguous last dim (copy if needed)."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) % 8) or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2


def _pad_n(w: Tensor, bias: Optional[Tensor], residual: Optional[Tensor]):
    """N not a multiple of 8: w (and bias, residual) padded with zeros to the next
    multiple, so that the output and residual rows are whole 16-byte chunks (the
    C ABI's contract); the caller keeps the first N columns of the result."""
    N = w.shape[0]
    n8 = -(-N // 8) * 8
    if n8 == N:
        return w, bias, residual, N
    w = torch.cat([w, w.new_zeros((n8 - N, w.shape[1]))])
    if bias is not None:
        bias = torch.cat([bias, bias.new_zeros(n8 - N)])
    if residual is not None:
        residual = torch.nn.functional.pad(residual, (0, n8 - N))
    return w, bias, residual, N


@torch.library.custom_op("strata_hip::gemm_bias_act", mutates_args=())
def gemm_bias_act(x: Tensor, w: Tensor, bias: Optional[Tensor], residual: Optional[Tensor], act: int,
                  res_op: int = 0) -> Tensor:
    """``act(x @ w.T + bias) + residual`` (res_op 0) or ``* residual`` (res_op 1),
    fp32 accumulation, bf16 in/out.

    x ``[..., K]``, w ``[N, K]`` (nn.Linear layout), bias ``[N]``, residual
    ``[..., N]``.  act: 0 none, 1 GELU(tanh), 2 GELU(erf), 3 sigmoid, 4 / 5 the
    derivatives of GELU(tanh) / sigmoid (the backward's epilogues).  K is any
    multiple of 8 (a K not a multiple of 64 runs on the large-tile kernel's
    ragged-K instances).  Replaces
    nn.Linear (+ nn.GELU) in the block's attn.qkv / attn.proj / Mlp
    (screamcast/checkpoint_compat.py:243-249, screamcast/strata_wrappers.py:76-100)
    and, with act 3 / res_op 1, the attention gate ``a * sigmoid(gate_proj(x))``.
    """
    name = "gemm_bias_act"
    _require_gpu(name, x, w, bias, residual)
    for t, nm in ((x, "x"), (w, "w"), (bias, "bias"), (residual, "residual")):
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError(f"{name}: {nm} must be bfloat16, got {t.dtype}")
    K = x.shape[-1]
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError(f"{name}: w must be [N, {K}], got {tuple(w.shape)}")
    N = w.shape[0]
    if bias is not None and tuple(bias.shape) != (N,):
        raise ValueError(f"{name}: bias must be [{N}]")
    out_shape = (*x.shape[:-1], N)
    if residual is not None and tuple(residual.shape) != out_shape:
        raise ValueError(f"{name}: residual must have shape {out_shape}, got {tuple(residual.shape)}")
    if N % 8:
        w, bias, residual, _ = _pad_n(w, bias, residual)
        return _gemm_launch(x, w, bias, residual, act, res_op)[..., :N].contiguous()
    return _gemm_launch(x, w, bias, residual, act, res_op)


def _gemm_launch(x: Tensor, w: Tensor, bias: Optional[Tensor], residual: Optional[Tensor], act: int,
                 res_op: int) -> Tensor:
    """strata_hip_gemm_bias_act on validated operands whose N is a multiple of 8."""
    name = "gemm_bias_act"
    K, N = x.shape[-1], w.shape[0]
    out_shape = (*x.shape[:-1], N)
    x2 = _rows(name, x, "x")
    w2 = _rows(name, w, "w")
    b2 = bias.contiguous() if bias is not None else None
    r2 = _rows(name, residual, "residual") if residual is not None else None
    out = torch.empty(out_shape, dtype=torch.bfloat16, device=x.device)
    M = x2.shape[0]
    if M == 0 or N == 0:
        return out
    a = _lib.GemmArgs()
    a.x, a.w = x2.data_ptr(), w2.data_ptr()
    a.bias = b2.data_ptr() if b2 is not None else None
    a.residual = r2.data_ptr() if r2 is not None else None
    a.out = out.data_ptr()
    a.m, a.n, a.k = M, N, K
    a.ldx, a.ldw = x2.stride(0) if M > 1 else K, w2.stride(0) if N > 1 else K
    a.ldr = (r2.stride(0) if M > 1 else N) if r2 is not None else 0
    a.ldo = N
    a.act = int(act)
    a.res_op = int(res_op)
    with torch.cuda.device(x.device):
        _lib.call("strata_hip_gemm_bias_act", a, _stream(x))
    return out


@gemm_bias_act.register_fake
def _(x, w, bias, residual, act, res_op=0):
    return x.new_empty((*x.shape[:-1], w.shape[0]))


def _gemm_setup_context(ctx, inputs, output):
    x, w, bias, residual, act, res_op = inputs
    ctx.act, ctx.res_op = int(act), int(res_op)
    ctx.has_bias, ctx.has_res = bias is not None, residual is not None
    gate = int(act) == _lib.ACT_SIGMOID and residual is not None and int(res_op) == _lib.RES_MUL
    ctx.save_for_backward(x, w, bias, residual if gate else None)


def _gemm_backward(ctx, dout):
    """Backward of ``act(x @ w.T + bias) + residual`` for act none / GELU(tanh), residual
    added (the MLP's fc1 -> GELU and fc2 + residual, attn.qkv and attn.proj + residual), and
    of the attention gate ``sigmoid(x @ w.T + bias) * residual``.
    The gradient at the pre-activation of a GELU layer, ``gelu'(x @ w.T + bias) * dout``,
    recomputes the GEMM with that epilogue fused (hand-written kernel); the input and
    weight gradients are plain GEMMs."""
    gate = ctx.act == _lib.ACT_SIGMOID and ctx.has_res and ctx.res_op == _lib.RES_MUL
    if not gate and (ctx.act not in (_lib.ACT_NONE, _lib.ACT_GELU_TANH) or (ctx.has_res and ctx.res_op != _lib.RES_ADD)):
        raise RuntimeError("strata_hip::gemm_bias_act: backward covers act none / GELU(tanh) with an added "
                           "residual and the sigmoid gate (multiplied residual)")
    x, w, bias, res = ctx.saved_tensors
    g = dout.contiguous()
    dres = None
    if gate:  # out = sigmoid(z) * res: d res = dout * sigmoid(z), d z = dout * res * sigmoid'(z)
        if ctx.needs_input_grad[3]:
            dres = gemm_bias_act(x, w, bias, g, _lib.ACT_SIGMOID, _lib.RES_MUL)
        g = gemm_bias_act(x, w, bias, (g * res).contiguous(), _lib.ACT_SIGMOID_GRAD, _lib.RES_MUL)
    elif ctx.act == _lib.ACT_GELU_TANH:
        g = gemm_bias_act(x, w, bias, g, _lib.ACT_GELU_TANH_GRAD, _lib.RES_MUL)
    g2 = g.reshape(-1, g.shape[-1])
    x2 = x.reshape(-1, x.shape[-1])
    dx = (g2 @ w).reshape(x.shape) if ctx.needs_input_grad[0] else None
    dw = (g2.t() @ x2) if ctx.needs_input_grad[1] else None
    db = None
    if ctx.has_bias and ctx.needs_input_grad[2]:
        db = bias_grad(g2) if g2.shape[-1] % 8 == 0 else g2.float().sum(0).to(bias.dtype)
    if not gate:
        dres = dout if ctx.has_res and ctx.needs_input_grad[3] else None
    return dx, dw, db, dres, None, None


gemm_bias_act.register_autograd(_gemm_backward, setup_context=_gemm_setup_context)


@torch.library.custom_op("strata_hip::gemm_gelu_train", mutates_args=())
def gemm_gelu_train(x: Tensor, w: Tensor, bias: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """``gelu_tanh(x @ w.T + bias)`` and, from the same launch, its derivative at the
    pre-activation ``gelu_tanh'(x @ w.T + bias)`` (bf16): the MLP's fc1 under autograd,
    whose backward then multiplies the upstream gradient by the saved derivative
    instead of recomputing the GEMM.  K must be a multiple of 8."""
    name = "gemm_gelu_train"
    _require_gpu(name, x, w, bias)
    for t, nm in ((x, "x"), (w, "w"), (bias, "bias")):
        if t is not None and t.dtype != torch.bfloat16:
            raise ValueError(f"{name}: {nm} must be bfloat16, got {t.dtype}")
    K = x.shape[-1]
    if w.dim() != 2 or w.shape[1] != K:
        raise ValueError(f"{name}: w must be [N, {K}], got {tuple(w.shape)}")
    N = w.shape[0]
    if bias is not None and tuple(bias.shape) != (N,):
        raise ValueError(f"{name}: bias must be [{N}]")
    if N % 8:
        wp, bp, _, _ = _pad_n(w, bias, None)
        out, dact = _gemm_gelu_train_launch(x, wp, bp)
        return out[..., :N].contiguous(), dact[..., :N].contiguous()
    return _gemm_gelu_train_launch(x, w, bias)


def _gemm_gelu_train_launch(x: Tensor, w: Tensor, bias: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """strata_hip_gemm_gelu_save on validated operands whose N is a multiple of 8."""
    name = "gemm_gelu_train"
    K, N = x.shape[-1], w.shape[0]
    x2, w2 = _rows(name, x, "x"), _rows(name, w, "w")
    b2 = bias.contiguous() if bias is not None else None
    out = torch.empty((*x.shape[:-1], N), dtype=torch.bfloat16, device=x.device)
    dact = torch.empty_like(out)
    M = x2.shape[0]
    if M == 0 or N == 0:
        return out, dact
    a = _lib.GemmArgs()
    a.x, a.w = x2.data_ptr(), w2.data_ptr()
    a.bias = b2.data_ptr() if b2 is not None else None
    a.residual = None
    a.out = out.data_ptr()
    a.m, a.n, a.k = M, N, K
    a.ldx, a.ldw = x2.stride(0) if M > 1 else K, w2.stride(0) if N > 1 else K
    a.ldr, a.ldo = 0, N
    a.act, a.res_op = _lib.ACT_GELU_TANH, _lib.RES_ADD
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.strata_hip_gemm_gelu_save(ctypes.byref(a), ctypes.c_void_p(dact.data_ptr()),
                                           ctypes.c_void_p(_stream(x)))
    if rc != _lib.OK:
        raise _lib.StrataHipError("strata_hip_gemm_gelu_save", rc, lib.strata_hip_last_error().decode())
    return out, dact


@gemm_gelu_train.register_fake
def _(x, w, bias):
    shape = (*x.shape[:-1], w.shape[0])
    return x.new_empty(shape), x.new_empty(shape)


def _gelu_train_setup_context(ctx, inputs, output):
    x, w, bias = inputs
    _, dact = output
    ctx.has_bias = bias is not None
    ctx.mark_non_differentiable(dact)
    ctx.save_for_backward(x, w, dact)


def _gelu_train_backward(ctx, dout, _ddact):
    x, w, dact = ctx.saved_tensors
    g2 = (dact * dout).reshape(-1, dact.shape[-1])  # the gradient at the pre-activation
    x2 = x.reshape(-1, x.shape[-1])
    dx = (g2 @ w).reshape(x.shape) if ctx.needs_input_grad[0] else None
    dw = (g2.t() @ x2) if ctx.needs_input_grad[1] else None
    db = None
    if ctx.has_bias and ctx.needs_input_grad[2]:
        db = bias_grad(g2) if g2.shape[-1] % 8 == 0 else g2.float().sum(0).to(torch.bfloat16)
    return dx, dw, db


gemm_gelu_train.register_autograd(_gelu_train_backward, setup_context=_gelu_train_setup_context)


@torch.library.custom_op("strata_hip::bias_grad", mutates_args=())
def bias_grad(g: Tensor) -> Tensor:
    """Column sums of ``g`` ``[..., N]`` bf16 (fp32 accumulation in an order fixed by
    the shape, rounded once to bf16): the bias gradient of a Linear whose output
    gradient is ``g``.  N must be a multiple of 8."""
    name = "bias_grad"
    _require_gpu(name, g)
    if g.dtype != torch.bfloat16:
        raise ValueError(f"{name}: g must be bfloat16")
    g2 = _rows(name, g, "g")
    M, N = g2.shape
    out = torch.empty(N, dtype=torch.bfloat16, device=g.device)
    if N == 0:
        return out
    lib = _lib.load()
    ws = torch.empty(max(int(lib.strata_hip_bias_grad_workspace(M, N)), 4), dtype=torch.float32, device=g.device)
    a = _lib.BiasGradArgs()
    a.g, a.out, a.workspace = g2.data_ptr(), out.data_ptr(), ws.data_ptr()
    a.m, a.n, a.ldg = M, N, (g2.stride(0) if M > 1 else N)
    with torch.cuda.device(g.device):
        _lib.call("strata_hip_bias_grad", a, _stream(g))
    return out


@bias_grad.register_fake
def _(g):
    return g.new_empty((g.shape[-1],))


bias_grad.register_autograd(_no_backward("strata_hip::bias_grad"))


# ---------------------------------------------------------------------------
# LayerNorm (non-affine)
# ---------------------------------------------------------------------------
@torch.library.custom_op("strata_hip::layer_norm", mutates_args=())
def layer_norm(x: Tensor, eps: float) -> Tensor:
    """Non-affine LayerNorm over the last dim, bf16 in/out, fp32 statistics."""
    name = "layer_norm"
    _require_gpu(name, x)
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name}: x must be bfloat16")
    x2 = _rows(name, x, "x")
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if x2.shape[0] == 0:
        return out
    a = _lib.LayerNormArgs()
    a.x, a.out = x2.data_ptr(), out.data_ptr()
    a.m, a.c = x2.shape[0], x2.shape[1]
    a.ldx = x2.stride(0) if x2.shape[0] > 1 else x2.shape[1]
    a.ldo = x2.shape[1]
    a.eps = float(eps)
    with torch.cuda.device(x.device):
        _lib.call("strata_hip_layer_norm", a, _stream(x))
    return out


@layer_norm.register_fake
def _(x, eps):
    return torch.empty_like(x)


def _ln_setup_context(ctx, inputs, output):
    x, eps = inputs
    ctx.eps = float(eps)
    ctx.save_for_backward(x)


def _ln_backward(ctx, dy):
    (x,) = ctx.saved_tensors
    x2 = x.contiguous().view(-1, x.shape[-1])
    g2 = dy.to(torch.bfloat16).contiguous().view(-1, x.shape[-1])
    dx = torch.empty_like(x2)
    if x2.shape[0]:
        a = _lib.LayerNormBwdArgs()
        a.x, a.dy, a.dx = x2.data_ptr(), g2.data_ptr(), dx.data_ptr()
        a.m, a.c, a.ld, a.eps = x2.shape[0], x2.shape[1], x2.shape[1], ctx.eps
        with torch.cuda.device(x.device):
            _lib.call("strata_hip_layer_norm_bwd", a, _stream(x))
    return dx.view(x.shape), None


layer_norm.register_autograd(_ln_backward, setup_context=_ln_setup_context)


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


# ---------------------------------------------------------------------------
# Cube-sphere halo fill and crop
# ---------------------------------------------------------------------------
_CUBE_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


@torch.library.custom_op("strata_hip::cube_pad_faces", mutates_args=())
def cube_pad_faces(data: Tensor, pad: int) -> Tensor:
    """``[..., 6, n, n]`` -> ``[..., 6, n + 2*pad, n + 2*pad]``: each face framed
    by its neighbours' edge strips and diagonal-filled corners
    (create_padded_faces_batched, screamcast/cubesphere_transforms.py:369-445).
    f32 or bf16."""
    name = "cube_pad_faces"
    _require_gpu(name, data)
    if data.dtype not in _CUBE_DTYPES:
        raise ValueError(f"{name}: dtype must be float32 or bfloat16")
    if data.dim() < 3 or data.shape[-3] != 6 or data.shape[-1] != data.shape[-2]:
        raise ValueError(f"{name}: expected [..., 6, n, n], got {tuple(data.shape)}")
    n = data.shape[-1]
    if pad < 0 or pad > n:
        raise ValueError(f"{name}: pad must be in [0, {n}]")
    if pad == 0:
        return data.clone()
    src = data.contiguous()
    out = torch.empty((*data.shape[:-2], n + 2 * pad, n + 2 * pad), dtype=data.dtype, device=data.device)
    a = _lib.CubePadArgs()
    a.src, a.dst = src.data_ptr(), out.data_ptr()
    a.dtype, a.face_size, a.pad = _CUBE_DTYPES[data.dtype], n, int(pad)
    a.lead = src.numel() // (6 * n * n)
    with torch.cuda.device(data.device):
        _lib.call("strata_hip_cube_pad_faces", a, _stream(data))
    return out


@cube_pad_faces.register_fake
def _(data, pad):
    n = data.shape[-1]
    return data.new_empty((*data.shape[:-2], n + 2 * pad, n + 2 * pad))


cube_pad_faces.register_autograd(_no_backward("strata_hip::cube_pad_faces"))


@torch.library.custom_op("strata_hip::cube_crop", mutates_args=())
def cube_crop(x: Tensor, halo: int) -> Tensor:
    """``[..., S, S]`` -> ``[..., S - 2*halo, S - 2*halo]`` (TileTopology.crop,
    screamcast/distributed_halo.py:143-147), as a contiguous tensor."""
    name = "cube_crop"
    _require_gpu(name, x)
    if x.dtype not in _CUBE_DTYPES:
        raise ValueError(f"{name}: dtype must be float32 or bfloat16")
    if x.dim() < 2 or x.shape[-1] != x.shape[-2]:
        raise ValueError(f"{name}: expected [..., S, S], got {tuple(x.shape)}")
    S = x.shape[-1]
    if halo < 0 or 2 * halo >= S:
        raise ValueError(f"{name}: need 0 <= 2*halo < {S}")
    src = x.contiguous()
    out = torch.empty((*x.shape[:-2], S - 2 * halo, S - 2 * halo), dtype=x.dtype, device=x.device)
    if out.numel() == 0:
        return out
    a = _lib.CubeCropArgs()
    a.src, a.dst = src.data_ptr(), out.data_ptr()
    a.dtype, a.extent, a.halo = _CUBE_DTYPES[x.dtype], S, int(halo)
    a.planes = src.numel() // (S * S)
    with torch.cuda.device(x.device):
        _lib.call("strata_hip_cube_crop", a, _stream(x))
    return out


@cube_crop.register_fake
def _(x, halo):
    S = x.shape[-1]
    return x.new_empty((*x.shape[:-2], S - 2 * halo, S - 2 * halo))


cube_crop.register_autograd(_no_backward("strata_hip::cube_crop"))


# ---------------------------------------------------------------------------
# Rollout step: state normalisation + patchify, and the state update
# ---------------------------------------------------------------------------
def _state_tables(name: str, dev: torch.device, C: int, **tabs: Optional[Tensor]) -> dict:
    out = {}
    for key, t in tabs.items():
        if t is None:
            out[key] = None
            continue
        want = torch.int32 if key == "src_channel" else torch.float32
        if t.dim() != 1 or t.shape[0] != C:
            raise ValueError(f"{name}: {key} must have shape [{C}], got {tuple(t.shape)}")
        out[key] = t.to(device=dev, dtype=want).contiguous()
    return out


@torch.library.custom_op("strata_hip::state_patchify", mutates_args=())
def state_patchify(
    state: Tensor, mean: Optional[Tensor], std: Optional[Tensor], patch: Sequence[int]
) -> Tensor:
    """fp32 state ``[B, C, Z, Y, X]`` -> bf16 tokens ``[B, Z/pz, Y/py, X/px, C*pz*py*px]``:
    ``(state - mean[c]) / std[c]`` with non-finite values set to 0
    (RunningNorm2d.forward, screamcast/normalization.py:109-123; ``std = sqrt(var) + eps``),
    patchified in Conv3d weight order (c, dz, dy, dx), so ``tokens @
    conv.weight.reshape(E, -1).T + conv.bias`` is ``Conv3d(kernel=stride=patch)``.
    ``mean``/``std`` None: no normalisation."""
    name = "state_patchify"
    dev = _require_gpu(name, state)
    if state.dtype != torch.float32 or state.dim() != 5:
        raise ValueError(f"{name}: state must be float32 [B, C, Z, Y, X], got {state.dtype} {tuple(state.shape)}")
    if (mean is None) != (std is None):
        raise ValueError(f"{name}: give both mean and std, or neither")
    pz, py, px = _triple("patch", patch)
    B, C, Z, Y, X = state.shape
    if min(pz, py, px) <= 0 or Z % pz or Y % py or X % px:
        raise ValueError(f"{name}: grid {(Z, Y, X)} is not a multiple of patch {(pz, py, px)}")
    tabs = _state_tables(name, dev, C, mean=mean, std=std)
    src = state.contiguous()
    out = torch.empty((B, Z // pz, Y // py, X // px, C * pz * py * px), dtype=torch.bfloat16, device=dev)
    if out.numel() == 0:
        return out
    a = _lib.StatePatchifyArgs()
    a.state, a.tokens = src.data_ptr(), out.data_ptr()
    a.mean = tabs["mean"].data_ptr() if tabs["mean"] is not None else None
    a.std = tabs["std"].data_ptr() if tabs["std"] is not None else None
    a.batch, a.channels = B, C
    a.grid[:] = [Z, Y, X]
    a.patch[:] = [pz, py, px]
    with torch.cuda.device(dev):
        _lib.call("strata_hip_state_patchify", a, _stream(state))
    return out


@state_patchify.register_fake
def _(state, mean, std, patch):
    pz, py, px = _triple("patch", patch)
    B, C, Z, Y, X = state.shape
    return state.new_empty((B, Z // pz, Y // py, X // px, C * pz * py * px), dtype=torch.bfloat16)


state_patchify.register_autograd(_no_backward("strata_hip::state_patchify"))


@torch.library.custom_op("strata_hip::dealias_axis", mutates_args=())
def dealias_axis(
    state: Tensor, mean: Optional[Tensor], std: Optional[Tensor], axis: int, patch: int, taps: Sequence[float]
) -> Tensor:
    """One axis of the dealiasing low-pass of ``DealiasedPatchEmbed3D``
    (screamcast/dealias.py:111-143) moved in front of the patch conv: along
    ``axis`` (0: Z, 1: Y, 2: X) of the fp32 state ``[B, C, Z, Y, X]``,
    ``out[.., i, ..] = sum_t taps[t] * n(state[.., clamp(p*(i//p) - lo + t, 0, S - p) + i % p, ..])``
    with ``lo = (len(taps) - 1) // 2`` (the replicate pad of the stride-1 conv's
    output) and ``n`` the input normalisation when ``mean``/``std`` are given.
    ``taps``: the axis filter divided by its sum (1 to 16 taps)."""
    name = "dealias_axis"
    dev = _require_gpu(name, state)
    if state.dtype != torch.float32 or state.dim() != 5:
        raise ValueError(f"{name}: state must be float32 [B, C, Z, Y, X], got {state.dtype} {tuple(state.shape)}")
    if (mean is None) != (std is None):
        raise ValueError(f"{name}: give both mean and std, or neither")
    taps = [float(t) for t in taps]
    if not 1 <= len(taps) <= 16:
        raise ValueError(f"{name}: 1 to 16 taps, got {len(taps)}")
    B, C, Z, Y, X = state.shape
    if axis not in (0, 1, 2) or patch <= 0 or (Z, Y, X)[axis] % patch:
        raise ValueError(f"{name}: patch {patch} does not divide axis {axis} of the grid {(Z, Y, X)}")
    tabs = _state_tables(name, dev, C, mean=mean, std=std)
    src = state.contiguous()
    out = torch.empty_like(src)
    if out.numel() == 0:
        return out
    a = _lib.DealiasAxisArgs()
    a.src, a.dst = src.data_ptr(), out.data_ptr()
    a.mean = tabs["mean"].data_ptr() if tabs["mean"] is not None else None
    a.std = tabs["std"].data_ptr() if tabs["std"] is not None else None
    a.batch, a.channels = B, C
    a.grid[:] = [Z, Y, X]
    a.axis, a.patch, a.taps = axis, patch, len(taps)
    a.filter[: len(taps)] = taps
    with torch.cuda.device(dev):
        _lib.call("strata_hip_dealias_axis", a, _stream(state))
    return out


@dealias_axis.register_fake
def _(state, mean, std, axis, patch, taps):
    return torch.empty_like(state.contiguous())


dealias_axis.register_autograd(_no_backward("strata_hip::dealias_axis"))


@torch.library.custom_op("strata_hip::state_update", mutates_args=())
def state_update(
    pred: Tensor,
    state: Optional[Tensor],
    mean: Optional[Tensor],
    std: Optional[Tensor],
    src_channel: Optional[Tensor],
    clamp_min: Optional[Tensor],
    grid: Sequence[int],
    patch: Sequence[int],
    order: int,
) -> Tensor:
    """bf16 prediction tokens ``[B, Z/pz, Y/py, X/px, C*pz*py*px]`` -> fp32 next state
    ``[B, C, Z, Y, X]``: ``d = bf16(pred * std[c] + mean[c])`` (RunningNorm2d.denormalize,
    screamcast/normalization.py:102-107), ``next = d + state[:, src_channel[c]]`` for
    difference-predicted channels (``src_channel[c] >= 0``) and ``d`` for state-predicted
    ones, then ``max(next, clamp_min[c])`` where ``clamp_min[c]`` is not NaN
    (MixedPredictionAsymmetric.step, screamcast/model_pipelines.py:631-676).
    ``order`` 0: token elements (c, dz, dy, dx); 1: (dz, dy, dx, c).  None tables:
    mean 0, std 1, ``src_channel[c] = c``, no clamp."""
    name = "state_update"
    dev = _require_gpu(name, pred, state)
    if pred.dtype != torch.bfloat16 or pred.dim() != 5:
        raise ValueError(f"{name}: pred must be bfloat16 [B, Tz, Ty, Tx, K], got {pred.dtype} {tuple(pred.shape)}")
    if (mean is None) != (std is None):
        raise ValueError(f"{name}: give both mean and std, or neither")
    if order not in (0, 1):
        raise ValueError(f"{name}: order must be 0 or 1")
    Z, Y, X = _triple("grid", grid)
    pz, py, px = _triple("patch", patch)
    if min(pz, py, px) <= 0 or Z % pz or Y % py or X % px:
        raise ValueError(f"{name}: grid {(Z, Y, X)} is not a multiple of patch {(pz, py, px)}")
    B = pred.shape[0]
    P = pz * py * px
    if tuple(pred.shape[1:4]) != (Z // pz, Y // py, X // px) or pred.shape[4] % P:
        raise ValueError(f"{name}: pred {tuple(pred.shape)} does not match grid {(Z, Y, X)} / patch {(pz, py, px)}")
    C = pred.shape[4] // P
    Cin = 0
    if state is not None:
        if state.dtype != torch.float32 or state.dim() != 5 or state.shape[0] != B or tuple(state.shape[2:]) != (Z, Y, X):
            raise ValueError(f"{name}: state must be float32 [{B}, Cin, {Z}, {Y}, {X}], got {tuple(state.shape)}")
        Cin = state.shape[1]
    tabs = _state_tables(name, dev, C, mean=mean, std=std, src_channel=src_channel, clamp_min=clamp_min)
    if tabs["src_channel"] is not None:
        # checked when the table lives on the host (a device table is not read
        # back: the kernel adds nothing for entries outside [0, Cin))
        if src_channel.device.type == "cpu" and bool((src_channel >= Cin).any()):
            raise ValueError(f"{name}: src_channel entries must be < {Cin} (negative: state prediction)")
    elif Cin < C:
        raise ValueError(f"{name}: without src_channel the state needs at least {C} channels")
    pr = pred.contiguous()
    st = state.contiguous() if state is not None else None
    out = torch.empty((B, C, Z, Y, X), dtype=torch.float32, device=dev)
    if out.numel() == 0:
        return out
    a = _lib.StateUpdateArgs()
    a.pred, a.next = pr.data_ptr(), out.data_ptr()
    a.state = st.data_ptr() if st is not None else None
    for key in ("mean", "std", "src_channel", "clamp_min"):
        setattr(a, key, tabs[key].data_ptr() if tabs[key] is not None else None)
    a.batch, a.channels, a.state_channels, a.order = B, C, Cin, int(order)
    a.grid[:] = [Z, Y, X]
    a.patch[:] = [pz, py, px]
    with torch.cuda.device(dev):
        _lib.call("strata_hip_state_update", a, _stream(pred))
    return out


@state_update.register_fake
def _(pred, state, mean, std, src_channel, clamp_min, grid, patch, order):
    Z, Y, X = _triple("grid", grid)
    P = math.prod(_triple("patch", patch))
    return pred.new_empty((pred.shape[0], pred.shape[4] // P, Z, Y, X), dtype=torch.float32)


state_update.register_autograd(_no_backward("strata_hip::state_update"))


# ---------------------------------------------------------------------------
# Pixel-stage block pieces (adaLN conditioning from the semantic tokens)
# ---------------------------------------------------------------------------
def _cols_view(name: str, t: Tensor, what: str) -> Tensor:
    """A [rows, C] view of t with unit column stride, 16-byte aligned rows (no copy when
    t already is one, e.g. a column slice of the modulation tensor)."""
    t2 = t.reshape(-1, t.shape[-1]) if t.dim() != 2 else t
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) % 8) or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2


@torch.library.custom_op("strata_hip::upsample_dw_gelu", mutates_args=())
def upsample_dw_gelu(cond: Tensor, weight: Tensor, bias: Optional[Tensor], factor: int) -> Tensor:
    """``GELU_tanh(dwconv3x3(bilinear_up(cond)) + bias)``: cond ``[B, Z, Yc, Xc, C]`` bf16
    tokens upsampled by ``factor`` in y and x (align_corners = false), the depth-wise 3x3
    taps ``weight`` (a Conv3d weight ``[C, 1, 1, 3, 3]``, or ``[C, 3, 3]``) with zero
    padding; returns ``[B, Z, Yc * factor, Xc * factor, C]`` bf16."""
    name = "upsample_dw_gelu"
    _require_gpu(name, cond, weight, bias)
    if cond.dtype != torch.bfloat16 or cond.dim() != 5:
        raise ValueError(f"{name}: cond must be a bfloat16 [B, Z, Y, X, C] tensor")
    B, Z, Yc, Xc, C = cond.shape
    w = weight.reshape(C, 9).t().to(torch.bfloat16).contiguous()  # tap-major [9, C]
    b = bias.to(torch.bfloat16).contiguous() if bias is not None else None
    c = cond if cond.stride(-1) == 1 and cond.data_ptr() % 16 == 0 else cond.contiguous()
    f = int(factor)
    out = torch.empty((B, Z, Yc * f, Xc * f, C), dtype=torch.bfloat16, device=cond.device)
    if out.numel() == 0:
        return out
    a = _lib.UpsampleDwGeluArgs()
    a.cond, a.out, a.weight = c.data_ptr(), out.data_ptr(), w.data_ptr()
    a.bias = b.data_ptr() if b is not None else None
    a.batch, a.depth, a.height, a.width, a.channels, a.factor = B, Z, Yc, Xc, C, f
    a.cond_stride[:] = [c.stride(i) for i in range(4)]
    a.out_stride[:] = [out.stride(i) for i in range(4)]
    with torch.cuda.device(cond.device):
        _lib.call("strata_hip_upsample_dw_gelu", a, _stream(cond))
    return out


@upsample_dw_gelu.register_fake
def _(cond, weight, bias, factor):
    B, Z, Yc, Xc, C = cond.shape
    return cond.new_empty((B, Z, Yc * factor, Xc * factor, C))


upsample_dw_gelu.register_autograd(_no_backward("strata_hip::upsample_dw_gelu"))


@torch.library.custom_op("strata_hip::layer_norm_modulate", mutates_args=())
def layer_norm_modulate(x: Tensor, shift: Tensor, scale: Tensor, eps: float) -> Tensor:
    """``LN(x) * (1 + scale) + shift`` over the last dim (non-affine LayerNorm, fp32
    statistics); shift and scale have x's shape and may be column slices of one tensor."""
    name = "layer_norm_modulate"
    _require_gpu(name, x, shift, scale)
    for t, w in ((x, "x"), (shift, "shift"), (scale, "scale")):
        if t.dtype != torch.bfloat16 or t.shape != x.shape:
            raise ValueError(f"{name}: {w} must be bfloat16 of x's shape")
    x2, sh, sc = (_cols_view(name, t, w) for t, w in ((x, "x"), (shift, "shift"), (scale, "scale")))
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if x2.shape[0] == 0:
        return out
    a = _lib.LayerNormModulateArgs()
    a.x, a.out, a.shift, a.scale = x2.data_ptr(), out.data_ptr(), sh.data_ptr(), sc.data_ptr()
    a.m, a.c = x2.shape
    ld = lambda t: t.stride(0) if t.shape[0] > 1 else t.shape[1]  # noqa: E731
    a.ldx, a.ldo, a.ld_shift, a.ld_scale = ld(x2), x2.shape[1], ld(sh), ld(sc)
    a.eps = float(eps)
    with torch.cuda.device(x.device):
        _lib.call("strata_hip_layer_norm_modulate", a, _stream(x))
    return out


@layer_norm_modulate.register_fake
def _(x, shift, scale, eps):
    return torch.empty_like(x)


layer_norm_modulate.register_autograd(_no_backward("strata_hip::layer_norm_modulate"))


@torch.library.custom_op("strata_hip::gated_add", mutates_args=())
def gated_add(res: Tensor, gate: Tensor, y: Tensor) -> Tensor:
    """``res + gate * y`` (bf16, one shape; gate may be a column slice of a wider tensor)."""
    name = "gated_add"
    _require_gpu(name, res, gate, y)
    for t, w in ((res, "res"), (gate, "gate"), (y, "y")):
        if t.dtype != torch.bfloat16 or t.shape != res.shape:
            raise ValueError(f"{name}: {w} must be bfloat16 of res's shape")
    r2, g2, y2 = (_cols_view(name, t, w) for t, w in ((res, "res"), (gate, "gate"), (y, "y")))
    out = torch.empty(res.shape, dtype=res.dtype, device=res.device)
    if r2.shape[0] == 0:
        return out
    a = _lib.GatedAddArgs()
    a.res, a.gate, a.y, a.out = r2.data_ptr(), g2.data_ptr(), y2.data_ptr(), out.data_ptr()
    a.m, a.c = r2.shape
    ld = lambda t: t.stride(0) if t.shape[0] > 1 else t.shape[1]  # noqa: E731
    a.ld_res, a.ld_gate, a.ld_y, a.ld_out = ld(r2), ld(g2), ld(y2), r2.shape[1]
    with torch.cuda.device(res.device):
        _lib.call("strata_hip_gated_add", a, _stream(res))
    return out


@gated_add.register_fake
def _(res, gate, y):
    return torch.empty_like(res)


gated_add.register_autograd(_no_backward("strata_hip::gated_add"))
