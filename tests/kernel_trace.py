"""Names of the GPU kernels a piece of code launches, through ``torch.profiler``.

The kernel-set tests mirror the reference's "only the backend's kernels touch
the data" checks (``tests/test_triton_iir.py:528-554``): the code runs once
under the profiler and every kernel with device time is listed.  Names are
normalised to the library's own spelling (``pesq_pipeline_kernels``):
demangled, without the return type, the namespace and the argument list, and
with no spaces, e.g. ``iir_output_kernel<5,1,PipeFwdMode,true,2,false>``.
"""

import ctypes
import re

import torch

_DEMANGLE = None


def _demangle(name: str) -> str:
    global _DEMANGLE
    if not name.startswith("_Z"):
        return name
    if _DEMANGLE is None:
        fn = ctypes.CDLL("libstdc++.so.6").__cxa_demangle
        fn.restype = ctypes.c_void_p
        fn.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_void_p,
                       ctypes.POINTER(ctypes.c_int)]
        _DEMANGLE = fn
    status = ctypes.c_int(0)
    out = _DEMANGLE(name.encode(), None, None, ctypes.byref(status))
    if status.value != 0 or not out:
        return name
    text = ctypes.string_at(out).decode()
    ctypes.CDLL(None).free(ctypes.c_void_p(out))
    return text


def normalise(name: str) -> str:
    """``void pesq::k<5, 1, pesq::M, true>(args)`` -> ``k<5,1,M,true>``."""

    name = _demangle(name.strip())
    name = re.sub(r"^void\s+", "", name)
    depth = 0
    for i, ch in enumerate(name):  # cut the argument list after the template list
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            name = name[:i]
            break
    name = name.replace("pesq::", "")
    return re.sub(r"\s+", "", name)


def launched_kernels(fn):
    """Run ``fn()`` under the profiler; return ``(result, {kernel: launches})``."""

    torch.cuda.synchronize()
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        result = fn()
        torch.cuda.synchronize()
    counts = {}
    for event in prof.key_averages():
        if event.self_device_time_total > 0:
            key = normalise(event.key)
            counts[key] = counts.get(key, 0) + event.count
    return result, counts


def library_kernels(batch: int, length: int, grad_mask: int, backward: bool):
    """The library's own list for a pipeline pass, normalised like the trace."""

    from torch_pesq import _lib

    return [normalise(n) for n in _lib.pipeline_kernels(batch, length, grad_mask, backward)]
