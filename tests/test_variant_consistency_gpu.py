"""The kernel variants chosen for large grids against those of small grids.

The pipeline picks its kernels by grid size (``pesq_pipeline_kernels``): a
batch of eighteen 30 s items runs the large-grid variants (the scans recompute
the lane states, the STFT forward takes its lean form, the chain kernels four
frames per wavefront, the STFT backward two frames per wavefront in eight
wavefronts instead of one in nine), while the same items one at a time run
the small-grid ones.  Batch items are scored independently; the reference
pins that bitwise for its chain (``tests/test_triton_chain.py:568-598``) and
to 1e-5 for its loss (``tests/test_triton_loss.py:340-349``).

Here the losses must be bitwise equal.  The transforms round as written (no
compiler-chosen contraction) and every sum of the chain and the STFT is taken
in an order that does not depend on the variant, so those stages give the
same bits for an item in any batch.  What remains are the scans: the variant
that stores the lane states runs the zero-state recursion and an in-wave
scan and takes its block start states from the two previous blocks'
aggregates, the one that recomputes them uses weighted sums of the chunk's
inputs and an LDS sum for the block end state, and a prefix kernel.  Both evaluate the same recursion in
float64 and differ by float64 rounding (the parallel form's sections are
larger than their sum, so that is about 1e-11 of a sample); rounded to the
float32 signals of the forward, a few samples land on the other side of a
rounding boundary (one unit in the last place), and the backward filters
spread such a one-ulp input difference over their impulse response.  So the
gradients agree to a few float32 units of the item's largest gradient, not
bitwise: the bound is 1e-6 of that peak (measured 4e-8, 0.04 % of the
samples differ; before the transforms were written out the STFT variants
alone moved gradients by 2e-5 of the peak).  Bitwise gradients would need
the same float64 operations in both scan variants (the recursion and the
in-wave scan in the large-grid passes, about 30 us more at c5).
"""

import pytest
import torch

from bench import speech_like_pair
from torch_pesq import PesqLossTriton, _lib

pytestmark = pytest.mark.gpu

# 18 x 30 s: 2124 chain tiles, 16884 forward and 8442 backward scan wavefronts
ITEMS, SAMPLES = 18, 480000
GRAD_RTOL = 1e-6  # of the item's largest gradient: a few float32 units


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
    assert "iir_output_kernel<5, 1, PipeFwdMode, false, 0, false>" in wide
    assert "iir_output_kernel<5, 1, PipeFwdMode, true, 2, false>" in narrow
    assert "stft_bwd_kernel<float, 2, 8>" in wide_b and "stft_bwd_kernel<float, 1, 9>" in narrow_b
    assert "chain_bwd_kernel<4, 1>" in wide_b and "chain_bwd_kernel<16, 1>" in narrow_b
    assert "iir_output_kernel<5, 1, PipeBwdMode, false, 0, false>" in wide_b
    assert "iir_output_kernel<5, 1, PipeBwdMode, true, 2, false>" in narrow_b

    ref_np, deg_np = speech_like_pair(ITEMS, SAMPLES, seed=21, noise=0.15)
    ref = torch.from_numpy(ref_np).cuda()
    deg = torch.from_numpy(deg_np).cuda()
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    loss_b, grad_b = _step(model, ref, deg)
    loss_diff = grad_diff = 0
    worst_grad = 0.0
    for i in range(ITEMS):
        loss_1, grad_1 = _step(model, ref[i : i + 1], deg[i : i + 1])
        loss_diff += int(loss_b[i] != loss_1[0])
        grad_diff += int((grad_b[i] != grad_1[0]).sum())
        scale = float(grad_1.abs().max())
        worst_grad = max(worst_grad, float((grad_b[i] - grad_1[0]).abs().max()) / scale)
    print(f"\nwide vs narrow variants: {loss_diff} of {ITEMS} losses differ; {grad_diff} of "
          f"{grad_b.numel()} gradient samples differ, by at most {worst_grad:.3g} of the "
          f"item's largest gradient", flush=True)
    assert loss_diff == 0
    assert worst_grad <= GRAD_RTOL
