"""The reference's operator import paths, served by the HIP operators.

Code written against ``torch_pesq.triton_ops`` (``torch_pesq/triton_ops/
__init__.py``, ``iir.py:1266``, ``resample.py:442``, ``spectral.py:584``,
``chain.py:1024``, ``elementwise.py:272,389,655,835``, ``loss.py:18``) imports
the same names from here and gets the gfx950 kernels of
:mod:`torch_pesq.hip_ops`.  Nothing here is Triton and nothing dispatches:
every name is the HIP class or function itself.

``HAS_TRITON`` keeps the reference's availability flag, meaning "the GPU
backend can run" (a ROCm device is visible); the operators raise a
descriptive ``RuntimeError`` when the HIP library is not built.
"""

from ..hip_ops import HAS_HIP

HAS_TRITON = HAS_HIP

__all__ = ["HAS_TRITON"]
