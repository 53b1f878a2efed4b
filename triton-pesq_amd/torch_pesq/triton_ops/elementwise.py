"""``torch_pesq.triton_ops.elementwise`` (``elementwise.py:37,272,389,655,835``).

The four differentiable stage functions, each the HIP implementation.
"""

from ..hip_ops.elementwise import align_scale, edge_ramp, peak_normalize, pesq_epilogue

__all__ = ["peak_normalize", "edge_ramp", "align_scale", "pesq_epilogue"]
