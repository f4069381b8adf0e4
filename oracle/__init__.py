"""CPU oracle for the fused RoFormer layer kernels.

TEST INFRASTRUCTURE ONLY.  This package restates, in numpy, the arithmetic of
the reference's fused layer kernels (baicai-1145/pymsst,
``src/pymsst/training/cuda/fused_band_split.cu`` and the pure-torch pieces of
``src/pymsst/training/fused_roformer.py``).  It exists to CHECK the HIP
kernels in ``pymsst_amd/csrc``.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it; the product path
(``pymsst_amd``) never imports, calls or falls back to anything here.

Every function is pinned by an independent check in
``tests/test_oracle_pinning.py``: torch float64 autograd of the closed-form
module (``F.normalize``/``F.linear``/``F.glu``/``bmm``), complex
multiplication for rotary, invariants (norm preservation, scale invariance,
zero rows) and the reference tests' own seeded shapes
(``tests/test_training_smoke.py:433-615``).  Functions whose only check
would be a retyping of the formula are marked "parity unpinned" in their
docstring; there are none at present.
"""

from .kernels import *  # noqa: F401,F403
from .dtypes import round_to, to_f64, DTYPES  # noqa: F401
