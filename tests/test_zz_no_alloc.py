"""strata_hip_na3d_bwd_noalloc (the allocation-free NA3D backward) against
strata_hip_na3d_bwd with a caller workspace, both called through the C ABI.

Two calls in a row on one device, the second with a smaller input, each
compared bit for bit with the workspace entry point on the same inputs (the
same kernels run on the same data, so the gradients must be identical; the
second call also shows that nothing of the first call's scratch contents
leaks into it).  Both with the statistics recomputed and with the forward's
log-sum-exp handed over.
"""

import ctypes

import pytest
import torch

from strata_amd import _lib, ops  # noqa: F401  (registers the forward ops)

pytestmark = pytest.mark.gpu


def _args(q, k, v, o, do, dq, dk, dv, ws, kernel, lse=None):
    B, Z, Y, X, H, D = q.shape
    a = _lib.Na3dBwdArgs()
    a.q, a.k, a.v, a.out, a.dout = (t.data_ptr() for t in (q, k, v, o, do))
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.workspace = None if ws is None else ws.data_ptr()
    a.dtype = _lib.BF16 if q.dtype == torch.bfloat16 else _lib.F32
    a.batch, a.heads, a.head_dim = B, H, D
    a.grid[:] = [Z, Y, X]
    a.kernel[:] = list(kernel)
    a.dilation[:] = [1, 1, 1]
    a.scale = D**-0.5
    a.lse = None if lse is None else lse.data_ptr()
    return a


def _both(gpu, shape, kernel, seed, use_lse, dtype=torch.bfloat16):
    lib = _lib.load()
    g = torch.Generator(device=gpu).manual_seed(seed)
    q, k, v, do = (torch.randn(shape, generator=g, device=gpu).to(dtype) for _ in range(4))
    if use_lse:
        o, lse = torch.ops.strata_hip.na3d_fwd_lse(q, k, v, list(kernel), [1, 1, 1], None)
    else:
        o, lse = torch.ops.strata_hip.na3d_fwd(q, k, v, list(kernel), [1, 1, 1], None, [0, 0, 0],
                                               list(shape[1:4])), None
    B, Z, Y, X, H, D = shape
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = []
    for noalloc in (False, True):
        dq, dk, dv = (torch.full_like(q, float("nan")) for _ in range(3))
        ws = None if noalloc else torch.empty(2 * B * Z * Y * X * H, dtype=torch.float32, device=gpu)
        a = _args(q, k, v, o, do, dq, dk, dv, ws, kernel, lse)
        fn = lib.strata_hip_na3d_bwd_noalloc if noalloc else lib.strata_hip_na3d_bwd
        rc = fn(ctypes.byref(a), stream)
        assert rc == 0, lib.strata_hip_last_error().decode()
        torch.cuda.synchronize()
        res.append((dq, dk, dv))
    for x, y in zip(*res):
        assert torch.isfinite(x.float()).all()
        assert torch.equal(x, y)


@pytest.mark.parametrize("use_lse", [False, True])
def test_noalloc_matches_workspace_entry_point_twice(gpu, use_lse):
    print(f"noalloc bwd, lse given: {use_lse}", flush=True)
    _both(gpu, (2, 6, 32, 32, 8, 64), (3, 7, 7), 1, use_lse)  # 98304 pairs
    _both(gpu, (1, 4, 12, 20, 2, 64), (3, 5, 5), 2, use_lse)  # smaller, different kernel
    _both(gpu, (1, 3, 8, 8, 2, 32), (3, 3, 3), 3, use_lse, torch.float32)


def test_noalloc_at_the_scratch_maximum_and_beyond(gpu):
    """2^21 (query, head) pairs is accepted (the configs[3] NA3D shape); one more
    batch entry is rejected with the scratch limit in the message."""
    print("noalloc bwd at 2^21 pairs", flush=True)
    _both(gpu, (4, 8, 64, 64, 16, 64), (3, 7, 7), 4, True)
    lib = _lib.load()
    shape = (5, 8, 64, 64, 16, 64)
    # real tensors of the refused shape (8 x 335 MB): should the host check ever let the
    # call through, every access still lands inside its own allocation
    ts = [torch.zeros(shape, dtype=torch.bfloat16, device=gpu) for _ in range(8)]
    a = _args(*ts, None, (3, 7, 7))
    rc = lib.strata_hip_na3d_bwd_noalloc(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == _lib.EUNSUPPORTED
    assert "scratch maximum" in lib.strata_hip_last_error().decode()
    del ts
