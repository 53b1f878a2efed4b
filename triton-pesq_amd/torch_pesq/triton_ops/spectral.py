"""``torch_pesq.triton_ops.spectral`` (``spectral.py:135-138,584``): ``TritonStftBark`` is :class:`HipStftBark`."""

from ..hip_ops.spectral import HipStftBark, bark_segments

TritonStftBark = HipStftBark

__all__ = ["TritonStftBark", "bark_segments"]
