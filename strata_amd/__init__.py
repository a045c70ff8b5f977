"""MI355X-native kernels for the Strata transformer block's hot path.

``torch.ops.strata_hip.{na3d_fwd, rope_qkv_pack, gemm_bias_act, layer_norm}``
over the C-ABI HIP library ``libstrata_hip.so`` (``include/strata_hip.h``),
plus drop-ins for ``natten.na3d`` (:mod:`strata_amd.natten`) and the block
modules (:mod:`strata_amd.modules`).
"""

from . import ops  # noqa: F401  (registers the custom ops)

__all__ = ["ops"]
