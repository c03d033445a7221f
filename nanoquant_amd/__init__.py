"""MI355X (gfx950) runtime for NanoQuant's packed binary low-rank linear.

Public API lives in ``nanoquant_amd.runtime`` (a mirror of the reference's
``nanoquant.runtime`` backend/planner/module surface for this path). The compute
is in hand-written HIP kernels behind the C ABI of ``include/nqamd.h``.
"""

__all__ = ["runtime"]
