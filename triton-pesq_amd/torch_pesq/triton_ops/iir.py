"""``torch_pesq.triton_ops.iir`` (``iir.py:137-147,1266``): ``TritonIIR`` is :class:`HipIIR`.

``CHUNK_CANDIDATES`` and ``METHODS`` are the values the constructor
validates ``chunk_size="tune"`` and ``method`` against; the HIP scan has a
fixed chunk geometry, so they do not change results.
"""

from ..hip_ops.iir import HipIIR

TritonIIR = HipIIR
CHUNK_CANDIDATES = (64, 128, 256, 512)
METHODS = ("scan", "matmul")

__all__ = ["TritonIIR", "CHUNK_CANDIDATES", "METHODS"]
