"""Drop-in for ``natten.na3d`` (NATTEN 0.21.5 functional API) backed by the HIP kernel.

The physicsnemo Strata attention calls ``natten.na3d(q, k, v, kernel_size,
dilation=..., backend=...)`` with heads-last ``[B, Z, Y, X, H, D]`` tensors
(backend string from screamcast/config.py:99 -> train.py:143 ->
screamcast/strata_wrappers.py:331,490,582).  Installing this module under the
name ``natten`` (see :func:`install_as_natten`) routes that call to
``torch.ops.strata_hip.na3d_fwd`` (``na3d_fwd_lse`` when gradients are wanted,
so that the backward reuses the forward's log-sum-exp) without touching the caller.

Supported: odd kernel sizes, any dilation with kernel*dilation <= size,
non-causal, stride 1, default or explicit scale, ``return_lse`` (the
logsumexp, natural log, fp32 ``[B, Z, Y, X, H]``; no gradient through it).
Everything else raises ``NotImplementedError``; invalid sizes raise
``ValueError`` as NATTEN does.
"""

from __future__ import annotations

import math
import sys
import types
from typing import Optional, Sequence

import torch
from torch import Tensor

from . import ops

__all__ = ["na3d", "install_as_natten"]


def _as_triple(name: str, v) -> tuple[int, int, int]:
    if isinstance(v, int):
        return (v, v, v)
    t = tuple(int(x) for x in v)
    if len(t) != 3:
        raise ValueError(f"{name} must be an int or a 3-tuple, got {v!r}")
    return t


def _check_flag(name: str, value, ok) -> None:
    if isinstance(value, bool) or isinstance(value, int):
        values = (value,) * 3
    else:
        values = tuple(value)
    if any(x != ok for x in values):
        raise NotImplementedError(f"na3d: {name}={value!r} is not supported by the HIP backend")


def na3d(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    kernel_size: int | Sequence[int],
    stride: int | Sequence[int] = 1,
    dilation: int | Sequence[int] = 1,
    is_causal: bool | Sequence[bool] = False,
    scale: Optional[float] = None,
    additional_keys: Optional[Tensor] = None,
    additional_values: Optional[Tensor] = None,
    attention_kwargs: Optional[dict] = None,
    backend: Optional[str] = None,
    return_lse: bool = False,
    **tile_kwargs,
) -> Tensor | tuple[Tensor, Tensor]:
    """3D neighbourhood attention, NATTEN ``na3d`` signature, heads-last tensors."""
    _check_flag("stride", stride, 1)
    _check_flag("is_causal", is_causal, False)
    if additional_keys is not None or additional_values is not None:
        raise NotImplementedError("na3d: additional_keys/values are not supported by the HIP backend")
    if query.dim() != 6:
        raise ValueError(f"na3d expects heads-last [B, Z, Y, X, H, D] tensors, got {tuple(query.shape)}")
    if query.shape != key.shape or query.shape != value.shape:
        raise ValueError("na3d: query, key and value must have the same shape")
    ks = _as_triple("kernel_size", kernel_size)
    dil = _as_triple("dilation", dilation)
    grid = tuple(query.shape[1:4])
    for ax, (k, d, L) in enumerate(zip(ks, dil, grid)):
        if k < 1 or k % 2 == 0:
            raise ValueError(f"na3d: kernel_size must be odd and positive, got {ks}")
        if d < 1:
            raise ValueError(f"na3d: dilation must be positive, got {dil}")
        if k * d > L:
            raise ValueError(
                f"na3d: kernel_size * dilation ({k}*{d}) exceeds the input size {L} along axis {ax}"
            )
    if return_lse:
        # NATTEN's logsumexp: natural log of the sum of exp(scale * q.k) over each query's
        # window, fp32 [B, Z, Y, X, H]; the kernels keep it in log2 units.  It carries no
        # gradient (the output does, through the backward that consumes it).
        out, lse2 = ops.na3d_fwd_lse(query, key, value, list(ks), list(dil), scale)
        return out, lse2 * math.log(2.0)
    # with gradients wanted, the forward keeps its log-sum-exp for the backward
    return ops.na3d(query, key, value, list(ks), list(dil), scale)


def install_as_natten() -> types.ModuleType:
    """Register a module named ``natten`` whose ``na3d`` is this HIP-backed one.

    For hosts where NATTEN is not installed (e.g. ROCm): after this call
    ``import natten; natten.na3d(...)`` reaches the HIP kernel.  An already
    imported real ``natten`` is left alone and returned unchanged.
    """
    if "natten" in sys.modules:
        return sys.modules["natten"]
    mod = types.ModuleType("natten")
    mod.na3d = na3d
    mod.__version__ = "0.21.5+strata_hip"
    sys.modules["natten"] = mod
    return mod


# keep the op module referenced so the custom ops are registered on import
_ = ops
