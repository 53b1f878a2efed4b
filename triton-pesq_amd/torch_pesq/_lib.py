"""ctypes binding of the HIP library's C ABI (``include/pesq_hip.h``).

The shared object is ``torch_pesq/_lib/libpesq_hip.so``, built in-tree by
``triton-pesq_amd/build.py``.  There is no fallback: every GPU operator of the
package calls through this library and fails with a descriptive error when it
is missing.
"""

import ctypes
import os
from pathlib import Path

import torch

__all__ = [
    "IirSections",
    "ResamplePlanInfo",
    "ModelConstants",
    "library",
    "torch_ext",
    "check",
    "stream_handle",
    "pipeline_kernels",
    "MAX_SECTIONS",
    "GRAD_REF",
    "GRAD_DEG",
]

MAX_SECTIONS = 8
MAX_CASCADE = 32
NBARKS = 49
NFFT = 512
GRAD_REF = 1
GRAD_DEG = 2
ERR_ARGUMENT = 1  # PESQ_ERR_ARGUMENT
NOALLOC_SCRATCH_BYTES = 32 << 20  # PESQ_NOALLOC_SCRATCH_BYTES

LIB_PATH = Path(os.environ.get("PESQ_HIP_LIB", Path(__file__).with_name("_lib") / "libpesq_hip.so"))

c_double8 = ctypes.c_double * MAX_SECTIONS


class ResamplePlanInfo(ctypes.Structure):
    """``pesq_resample_plan_info``: geometry of a tiled resampler plan."""

    _fields_ = [
        ("orig_step", ctypes.c_int32),
        ("new_step", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("width_total", ctypes.c_int32),
        ("taps", ctypes.c_int32),
        ("off_min", ctypes.c_int32),
        ("off_max", ctypes.c_int32),
        ("phases", ctypes.c_int32),
        ("sweeps", ctypes.c_int32),
        ("columns", ctypes.c_int32),
        ("fwd_span", ctypes.c_int32),
        ("bwd_span", ctypes.c_int32),
        ("bytes", ctypes.c_int64),
        ("off_offs", ctypes.c_int64),
        ("off_cols", ctypes.c_int64),
        ("off_col_lo", ctypes.c_int64),
        ("off_taps64", ctypes.c_int64),
        ("off_row64", ctypes.c_int64),
        ("adj_taps", ctypes.c_int32),
        ("adj_off_min", ctypes.c_int32),
        ("adj_off_max", ctypes.c_int32),
        ("adj_span", ctypes.c_int32),
        ("off_adj_taps", ctypes.c_int64),
        ("off_adj_offs", ctypes.c_int64),
    ]


class IirSections(ctypes.Structure):
    """``pesq_iir_sections``: a filter in parallel biquad form."""

    _fields_ = [
        ("count", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("c0", ctypes.c_double),
        ("b0", c_double8),
        ("b1", c_double8),
        ("b2", c_double8),
        ("a1", c_double8),
        ("a2", c_double8),
    ]


class ModelConstants(ctypes.Structure):
    """``pesq_model_constants``: every constant of the PESQ model."""

    _fields_ = [
        ("power_filter", IirSections),
        ("pre_filter", IirSections),
        ("window", ctypes.c_float * NFFT),
        ("band_start", ctypes.c_int32 * NBARKS),
        ("band_end", ctypes.c_int32 * NBARKS),
        ("corr", ctypes.c_double * NBARKS),
        ("threshs", ctypes.c_double * NBARKS),
        ("exps", ctypes.c_double * NBARKS),
        ("width", ctypes.c_double * NBARKS),
        ("total_width", ctypes.c_double),
        ("sl", ctypes.c_double),
        ("nbarks", ctypes.c_int32),
        ("n_fft", ctypes.c_int32),
        ("hop", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_SIZE_P = ctypes.POINTER(ctypes.c_size_t)

#: name -> (restype, argtypes) of every exported entry point
SIGNATURES = {
    "pesq_abi_version": (_INT, []),
    "pesq_last_error": (ctypes.c_char_p, []),
    "pesq_iir_table_bytes": (ctypes.c_size_t, []),
    "pesq_iir_table_pack": (_INT, [ctypes.POINTER(IirSections), _P]),
    "pesq_iir_cascade_pack": (_INT, [_P, _INT, _P]),
    "pesq_model_table_bytes": (ctypes.c_size_t, []),
    "pesq_model_table_pack": (_INT, [ctypes.POINTER(ModelConstants), _P]),
    "pesq_pipeline_forward_workspace": (_INT, [_I64, _I64, _INT, _SIZE_P]),
    "pesq_pipeline_backward_workspace": (_INT, [_I64, _I64, _INT, _SIZE_P]),
    "pesq_pipeline_region": (_INT, [_I64, _I64, _INT, ctypes.c_char_p, _SIZE_P, _SIZE_P]),
    "pesq_pipeline_forward_noalloc": (
        _INT, [_P, _P, _I64, _I64, _P, ctypes.c_double, _P, _P, _P, _P, _P],
    ),
    "pesq_pipeline_kernels": (_INT, [_I64, _I64, _INT, _INT, ctypes.c_char_p, ctypes.c_size_t,
                                     _SIZE_P]),
    "pesq_pipeline_forward": (
        _INT,
        [_P, _P, _I64, _I64, _P, ctypes.c_double, _INT, _P, _P, _P, _P, _P, _P],
    ),
    "pesq_pipeline_backward": (
        _INT,
        [_P, _P, _P, _P, _I64, _I64, _P, ctypes.c_double, _INT, _P, _P, _P, _P, _P],
    ),
    "pesq_pipeline_forward_stages": (
        _INT,
        [_P, _P, _I64, _I64, _P, ctypes.c_double, _INT, _P, _P, _P, _P, _P, ctypes.c_uint, _P],
    ),
    "pesq_pipeline_backward_stages": (
        _INT,
        [_P, _P, _P, _P, _I64, _I64, _P, ctypes.c_double, _INT, _P, _P, _P, _P, ctypes.c_uint, _P],
    ),
    "pesq_iir_workspace": (_INT, [_I64, _I64, _SIZE_P]),
    "pesq_iir_apply": (_INT, [_P, _P, _I64, _I64, _P, _INT, _INT, _P, _P]),
    "pesq_iir_cascade_workspace": (_INT, [_I64, _I64, _INT, _SIZE_P]),
    "pesq_iir_cascade_apply": (_INT, [_P, _P, _I64, _I64, _P, _INT, _INT, _P, _P]),
    "pesq_stft_bark_forward": (_INT, [_P, _I64, _I64, _I64, _P, _P, _P]),
    "pesq_stft_bark_backward": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P, _P]),
    "pesq_stft_table_bytes": (ctypes.c_size_t, []),
    "pesq_stft_table_pack": (_INT, [_INT, _INT, _P, _INT, _P, _P, _P, _P]),
    "pesq_stft_workspace": (_INT, [_I64, _I64, _I64, _INT, _INT, _SIZE_P]),
    "pesq_stft_forward": (_INT, [_P, _I64, _I64, _I64, _P, _INT, _INT, _INT, _P, _P]),
    "pesq_stft_backward": (_INT, [_P, _P, _I64, _I64, _I64, _P, _INT, _INT, _INT, _P, _P, _P]),
    "pesq_chain_forward_workspace": (_INT, [_I64, _I64, _INT, _SIZE_P]),
    "pesq_chain_backward_workspace": (_INT, [_I64, _I64, _INT, _SIZE_P]),
    "pesq_chain_table_pack": (_INT, [_INT, _P, _P, _P, ctypes.c_double, ctypes.c_double, _P]),
    "pesq_chain_forward": (_INT, [_P, _P, _I64, _I64, _INT, _P, _P, _P, _P, _P]),
    "pesq_chain_backward": (_INT, [_P, _P, _P, _P, _I64, _I64, _INT, _P, _P, _P, _P, _P, _P]),
    "pesq_elementwise_workspace": (_INT, [_I64, _SIZE_P]),
    "pesq_peak_normalize_forward": (_INT, [_P, _P, _I64, _I64, _P, _P, _P, _P, _P]),
    "pesq_peak_normalize_backward": (_INT, [_P, _P, _P, _I64, _I64, _P, _P, _P]),
    "pesq_edge_ramp": (_INT, [_P, _P, _I64, _I64, _P]),
    "pesq_align_scale_forward": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "pesq_align_scale_backward": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "pesq_epilogue_forward": (_INT, [_P, _P, _I64, ctypes.c_double, _P, _P, _P]),
    "pesq_epilogue_backward": (_INT, [_P, _P, _P, _P, _I64, ctypes.c_double, _P, _P, _P]),
    "pesq_resample_forward": (
        _INT,
        [_P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    ),
    "pesq_resample_backward": (
        _INT,
        [_P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    ),
    "pesq_resample_plan": (
        _INT,
        [_P, _P, _P, _I64, _I64, _I64, _I64, ctypes.POINTER(ResamplePlanInfo), _P],
    ),
    "pesq_resample_plan_forward": (
        _INT,
        [_P, _P, _I64, _I64, _I64, ctypes.POINTER(ResamplePlanInfo), _P, _P],
    ),
    "pesq_resample_plan_backward": (
        _INT,
        [_P, _P, _I64, _I64, _I64, ctypes.POINTER(ResamplePlanInfo), _P, _P],
    ),
    "pesq_resample_plan_forward_pair": (
        _INT,
        [_P, _P, _P, _P, _I64, _I64, _I64, ctypes.POINTER(ResamplePlanInfo), _P, _P],
    ),
    "pesq_resample_plan_backward_pair": (
        _INT,
        [_P, _P, _P, _P, _I64, _I64, _I64, ctypes.POINTER(ResamplePlanInfo), _P, _P],
    ),
}

_LIB = None


def library():
    """The loaded library; raises ``RuntimeError`` when it is not built."""

    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"The PESQ HIP library is not built ({LIB_PATH} is missing). Run "
                "`python triton-pesq_amd/build.py` (or `__graft_entry__.build()`)."
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = lib
    return _LIB


_EXT = None


def torch_ext():
    """The PyTorch extension module ``_pesq_torch`` (autograd nodes in C++).

    It links ``libpesq_hip.so`` by its soname, so loading :func:`library`
    first makes both use the same copy of the library.
    """

    global _EXT
    if _EXT is None:
        library()
        path = LIB_PATH.with_name("_pesq_torch.so")
        if not path.exists():
            raise RuntimeError(
                f"The PESQ PyTorch extension is not built ({path} is missing). Run "
                "`python triton-pesq_amd/build.py` (or `__graft_entry__.build()`)."
            )
        import importlib.util

        spec = importlib.util.spec_from_file_location("torch_pesq._pesq_torch", path)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        _EXT = module
    return _EXT


def check(status: int, what: str = "") -> None:
    """Turn a non-zero status into a ``RuntimeError`` with the library's message."""

    if status == 0:
        return
    message = library().pesq_last_error().decode(errors="replace")
    prefix = f"{what}: " if what else ""
    raise RuntimeError(f"{prefix}{message} (status {status})")


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    """Raw ``hipStream_t`` of the current PyTorch stream on ``device``."""

    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(tensor) -> ctypes.c_void_p:
    """Device pointer of a tensor, or NULL for ``None``."""

    return ctypes.c_void_p(0 if tensor is None else tensor.data_ptr())


def pipeline_kernels(batch: int, length: int, grad_mask: int, backward: bool) -> list:
    """Kernels one pipeline pass launches for a shape, in launch order (host only)."""

    lib = library()
    needed = ctypes.c_size_t(0)
    check(lib.pesq_pipeline_kernels(batch, length, grad_mask, int(backward), None, 0,
                                    ctypes.byref(needed)), "pesq_pipeline_kernels")
    buf = ctypes.create_string_buffer(int(needed.value))
    check(lib.pesq_pipeline_kernels(batch, length, grad_mask, int(backward), buf, len(buf), None),
          "pesq_pipeline_kernels")
    return buf.value.decode().split(";")


def size_query(fn, *args) -> int:
    out = ctypes.c_size_t(0)
    check(fn(*args, ctypes.byref(out)), fn.__name__)
    return int(out.value)
