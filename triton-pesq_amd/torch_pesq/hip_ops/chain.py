"""HIP perceptual chain (``TritonPesqChain``, ``torch_pesq/triton_ops/chain.py:1024-1126``).

Silent frames, band and frame power equalisation, Zwicker loudness,
disturbance with its deadzone, both width weighted norms, the ``h`` weighting
and the overlapping sums, evaluated in float64 from float32 Bark spectra.
Forward: silent frames / band partials, per frame distances, overlapping sums
(3 kernels); backward: the adjoint of the per frame distances and the frame
equalisation, then the band ratio / mean band power scatter (2 kernels).
"""

import torch

from .. import _lib
from ._common import check_input

__all__ = ["HipPesqChain"]

#: bands of the stand-alone chain, one per lane of a wavefront
_MAX_BANDS = 128


def _pack_chain(threshs, exps, widths, total_width, sl) -> torch.Tensor:
    import ctypes

    import numpy as np

    lib = _lib.library()
    cols = [np.ascontiguousarray(v.detach().cpu().double().numpy()) for v in (threshs, exps, widths)]
    buf = (ctypes.c_ubyte * lib.pesq_model_table_bytes())()
    _lib.check(
        lib.pesq_chain_table_pack(cols[0].shape[0], *[c.ctypes.data_as(ctypes.c_void_p) for c in cols],
                                  float(total_width), float(sl), buf),
        "pesq_chain_table_pack",
    )
    return torch.frombuffer(bytearray(buf), dtype=torch.uint8).clone()


class _ChainFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ref, deg, module):
        batch, frames, nb = ref.shape
        lib = _lib.library()
        ws_bytes = _lib.size_query(lib.pesq_chain_forward_workspace, batch, frames, nb)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=ref.device)
        d_symm = torch.empty(batch, device=ref.device)
        d_asymm = torch.empty(batch, device=ref.device)
        with torch.cuda.device(ref.device):
            _lib.check(
                lib.pesq_chain_forward(_lib.ptr(ref), _lib.ptr(deg), batch, frames, nb,
                                       _lib.ptr(module.table), _lib.ptr(d_symm), _lib.ptr(d_asymm),
                                       _lib.ptr(ws), _lib.stream_handle(ref.device)),
                "pesq_chain_forward",
            )
        ctx.save_for_backward(ref, deg, ws)
        ctx.module = module
        ctx.set_materialize_grads(False)
        return d_symm, d_asymm

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, g_symm, g_asymm):
        ref, deg, ws = ctx.saved_tensors
        if g_symm is None and g_asymm is None:
            return None, None, None
        batch, frames, nb = ref.shape
        lib = _lib.library()
        bw_bytes = _lib.size_query(lib.pesq_chain_backward_workspace, batch, frames, nb)
        scratch = torch.empty(bw_bytes, dtype=torch.uint8, device=ref.device)
        g_ref, g_deg = torch.empty_like(ref), torch.empty_like(deg)
        g_symm = None if g_symm is None else g_symm.contiguous().float()
        g_asymm = None if g_asymm is None else g_asymm.contiguous().float()
        with torch.cuda.device(ref.device):
            _lib.check(
                lib.pesq_chain_backward(_lib.ptr(g_symm), _lib.ptr(g_asymm), _lib.ptr(ref),
                                        _lib.ptr(deg), batch, frames, nb, _lib.ptr(ctx.module.table),
                                        _lib.ptr(g_ref), _lib.ptr(g_deg), _lib.ptr(ws),
                                        _lib.ptr(scratch), _lib.stream_handle(ref.device)),
                "pesq_chain_backward",
            )
        return (
            g_ref if ctx.needs_input_grad[0] else None,
            g_deg if ctx.needs_input_grad[1] else None,
            None,
        )


class HipPesqChain(torch.nn.Module):
    """Symmetric and asymmetric PESQ distance of two Bark spectrograms.

    Same constructor as ``TritonPesqChain``: hearing thresholds, loudness
    exponents, band widths in Bark, their total (bands 1..) and ``sl``.
    """

    def __init__(self, threshs, exp, width_bark, total_width, sl=0.1866055):
        super().__init__()
        threshs = torch.as_tensor(threshs).reshape(-1).double()
        exps = torch.as_tensor(exp).reshape(-1).double()
        widths = torch.as_tensor(width_bark).reshape(-1).double()
        if not (threshs.shape == exps.shape == widths.shape):
            raise ValueError(
                "`threshs`, `exp` and `width_bark` need the same number of bands, got "
                f"{threshs.numel()}, {exps.numel()} and {widths.numel()}."
            )
        if torch.any(threshs <= 0):
            raise ValueError("Hearing thresholds have to be strictly positive.")
        if threshs.numel() > _MAX_BANDS:
            raise ValueError(
                f"The HIP chain takes at most {_MAX_BANDS} bands (two per lane of a "
                f"wavefront), got {threshs.numel()}."
            )
        self.total_width, self.sl = float(total_width), float(sl)
        self.register_buffer("threshs", threshs.float())
        self.register_buffer("exp", exps.float())
        self.register_buffer("width_bark", widths.float())
        # float32 buffers like the reference's (chain.py:1060-1076); the kernels
        # evaluate the chain in float64 from the float64 constants
        self.register_buffer("table", _pack_chain(threshs, exps, widths, self.total_width,
                                                  self.sl), persistent=False)

    def forward(self, ref_bark: torch.Tensor, deg_bark: torch.Tensor):
        """``(d_symm, d_asymm)``, both ``[batch]``."""

        ref = check_input(ref_bark, "ref_bark")
        deg = check_input(deg_bark, "deg_bark")
        if ref.dim() != 3 or deg.dim() != 3:
            raise ValueError(
                f"The PESQ chain expects `[batch, frame, bark]` inputs, got {tuple(ref.shape)} and {tuple(deg.shape)}."
            )
        if ref.shape != deg.shape:
            raise ValueError(
                f"`ref_bark` and `deg_bark` need the same shape, got {tuple(ref.shape)} and {tuple(deg.shape)}."
            )
        if ref.shape[2] != self.threshs.shape[0]:
            raise ValueError(f"Expected {self.threshs.shape[0]} Bark bands, got {ref.shape[2]}.")
        if ref.shape[1] < 20:
            raise ValueError(
                f"The PESQ chain needs at least 20 frames for the overlapping sums, got {ref.shape[1]}."
            )
        if self.table.device != ref.device:
            raise RuntimeError(f"The module lives on {self.table.device} but the spectra on {ref.device}.")
        return _ChainFunction.apply(ref, deg, self)
