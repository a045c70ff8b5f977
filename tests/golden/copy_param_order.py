"""Copy the reference's committed parameter-order manifests into this tree.

The manifests (``tests/regression_data/*.param_order.txt`` in the reference,
written by its ``tests/test_param_order.py:87-119``) are data: one parameter
name per line in ``named_parameters()`` order.  They are the reference's only
fixture that touches the block's module structure (state-dict keys and
registration order, which checkpoints and index-mapped optimizer states depend
on).  ``tests/test_param_order.py`` here checks the drop-in modules against
them.  The reference tree is not needed at test time.

Run from the repo root:  python tests/golden/copy_param_order.py [reference_root]
"""

from __future__ import annotations

import shutil
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent / "param_order"
NAMES = [
    "sweep1_nodilation_gated_tile64_kernel3_lr1em4_dim1024_hpatch4_depth32_r3_cos.param_order.txt",
    "pixeldit_sem1024d24l_pix128d4l_bilineardwgeluproject_unfreeze_3src_const1em5_t128.param_order.txt",
]


def main(ref_root: str = "/root/reference") -> None:
    src = Path(ref_root) / "tests" / "regression_data"
    HERE.mkdir(exist_ok=True)
    for n in NAMES:
        shutil.copyfile(src / n, HERE / n)
        print(f"copied {n}")


if __name__ == "__main__":
    main(*sys.argv[1:])
