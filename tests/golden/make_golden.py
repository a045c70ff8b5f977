"""Write the NA3D golden vectors in ``na3d_golden.npz``.

NATTEN is not installable offline, so the expected outputs come from
``oracle.na3d.na3d_bruteforce`` — pure-Python loops whose window is found by
searching every feasible run for the one centred nearest the query — in
float64.  That formulation shares no code with the vectorised oracle or the
HIP kernels, so the fixture pins both.  Cases cover clamping at every face and
corner, anisotropic kernels, dilation, a kernel that spans a whole axis, and
head dims the MFMA kernel takes (32) as well as tiny ones.

Run from the repo root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.na3d import na3d_bruteforce  # noqa: E402

CASES = [
    # name, (B, Z, Y, X, H, D), kernel, dilation, seed
    ("clamp_small", (1, 4, 5, 6, 2, 8), (3, 3, 5), (1, 1, 1), 1),
    ("dilated", (1, 5, 6, 7, 1, 8), (3, 3, 3), (1, 2, 2), 2),
    ("full_z", (2, 3, 4, 4, 1, 16), (3, 3, 3), (1, 1, 1), 3),
    ("mfma_d32", (1, 3, 6, 20, 2, 32), (3, 5, 13), (1, 1, 1), 4),
    ("mfma_d32_k7", (1, 4, 9, 10, 1, 32), (3, 7, 7), (1, 1, 1), 5),
    ("mfma_dil3", (1, 3, 7, 12, 1, 32), (1, 3, 3), (1, 2, 3), 6),
]


def main() -> None:
    arrays = {}
    meta = []
    for name, shape, kernel, dil, seed in CASES:
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(shape, generator=g, dtype=torch.float32)
        k = torch.randn(shape, generator=g, dtype=torch.float32)
        v = torch.randn(shape, generator=g, dtype=torch.float32)
        o = na3d_bruteforce(q, k, v, kernel, dil)
        arrays[f"{name}__q"] = q.numpy()
        arrays[f"{name}__k"] = k.numpy()
        arrays[f"{name}__v"] = v.numpy()
        arrays[f"{name}__out"] = o.float().numpy()
        meta.append({"name": name, "shape": list(shape), "kernel": list(kernel), "dilation": list(dil), "seed": seed})
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    out = Path(__file__).with_name("na3d_golden.npz")
    np.savez_compressed(out, **arrays)
    print(f"wrote {out} ({out.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
