"""``torch_pesq.triton_ops.resample`` (``resample.py:74,442``): ``TritonResample`` is :class:`HipResample`."""

from ..hip_ops.resample import HipResample

TritonResample = HipResample

__all__ = ["TritonResample"]
