"""The kernel variants chosen for large grids against those of small grids.

The pipeline picks its kernels by grid size (``pesq_pipeline_kernels``): a
batch of eighteen 30 s items runs the large-grid variants (the scans recompute
the lane states, the STFT forward takes its lean form, the chain kernels four
frames per wavefront, the STFT backward two frames per wavefront in eight
wavefronts instead of one in nine), while the
same items one at a time run the small-grid ones.  Batch items are scored
independently, so both must give the same losses and gradients up to
rounding.  Measured: the losses agree bitwise and so do the scans' outputs
and the stand-alone chain's results; the two STFT forward kernels round
differently in float32 (the compiler fuses different multiply-adds in the two
instantiations), which moves the Bark values of bands at the float32 FFT's
rounding floor by up to 1e-4 relative and the gradient by up to 2e-5 of its
peak.  The gradient bound is therefore the 1e-4 of the peak that
``test_full_configs_gpu.py`` holds each variant to against float64, while
the loss bound is 1e-6; a mistake confined to one variant's code (an index in
the lean STFT, a frame slot of the wide chain, the two-frame overlap-add)
would show far above either.
"""

import pytest
import torch

from bench import speech_like_pair
from torch_pesq import PesqLossTriton, _lib

pytestmark = pytest.mark.gpu

# 18 x 30 s: 2124 chain tiles, 16884 forward and 8442 backward scan wavefronts
ITEMS, SAMPLES = 18, 480000
LOSS_RTOL = 1e-6
GRAD_RTOL = 1e-4  # of the largest gradient of the item


def _step(model, ref, deg):
    deg = deg.detach().clone().requires_grad_(True)
    loss = model(ref, deg)
    (g,) = torch.autograd.grad(loss.sum(), deg)
    return loss.detach().double().cpu(), g.double().cpu()


def test_large_grid_variants_match_small_grid_ones():
    wide = _lib.pipeline_kernels(ITEMS, SAMPLES, _lib.GRAD_DEG, backward=False)
    narrow = _lib.pipeline_kernels(1, SAMPLES, _lib.GRAD_DEG, backward=False)
    wide_b = _lib.pipeline_kernels(ITEMS, SAMPLES, _lib.GRAD_DEG, backward=True)
    narrow_b = _lib.pipeline_kernels(1, SAMPLES, _lib.GRAD_DEG, backward=True)
    # the batch and the single items take different variants of every stage
    assert "stft_fwd_kernel<float, true, 8>" in wide and "stft_fwd_kernel<float, false, 8>" in narrow
    assert "chain_fwd_kernel<4, 1>" in wide and "chain_fwd_kernel<8, 1>" in narrow
    assert "iir_output_kernel<5, 1, PipeFwdMode, false, false>" in wide
    assert "iir_output_kernel<5, 1, PipeFwdMode, true, false>" in narrow
    assert "stft_bwd_kernel<float, 2, 8>" in wide_b and "stft_bwd_kernel<float, 1, 9>" in narrow_b
    assert "chain_bwd_kernel<4, 1>" in wide_b and "chain_bwd_kernel<16, 1>" in narrow_b
    assert "iir_output_kernel<5, 1, PipeBwdMode, false, false>" in wide_b
    assert "iir_output_kernel<5, 1, PipeBwdMode, true, false>" in narrow_b

    ref_np, deg_np = speech_like_pair(ITEMS, SAMPLES, seed=21, noise=0.15)
    ref = torch.from_numpy(ref_np).cuda()
    deg = torch.from_numpy(deg_np).cuda()
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    loss_b, grad_b = _step(model, ref, deg)
    worst_loss = worst_grad = 0.0
    for i in range(ITEMS):
        loss_1, grad_1 = _step(model, ref[i : i + 1], deg[i : i + 1])
        worst_loss = max(worst_loss, float(((loss_b[i] - loss_1[0]).abs() / loss_1[0].abs()).max()))
        scale = float(grad_1.abs().max())
        worst_grad = max(worst_grad, float((grad_b[i] - grad_1[0]).abs().max()) / scale)
    print(f"\nwide vs narrow variants: loss {worst_loss:.3g}, gradient {worst_grad:.3g}", flush=True)
    assert worst_loss <= LOSS_RTOL
    assert worst_grad <= GRAD_RTOL
