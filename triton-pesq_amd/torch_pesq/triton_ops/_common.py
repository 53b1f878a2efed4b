"""``torch_pesq.triton_ops._common`` (``_common.py:16-60`` of the reference).

``check_input`` and ``require_triton`` are the HIP backend's input checks
(GPU, float32, made contiguous; the same exception types and messages
modulo the backend's name).
"""

from ..hip_ops._common import check_input, require_hip
from . import HAS_TRITON

require_triton = require_hip

__all__ = ["HAS_TRITON", "require_triton", "check_input"]
