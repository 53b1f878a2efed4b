"""GPU parity at the full BASELINE shapes c3, c4 and c5, forward and backward.

The pipeline chooses kernel variants by grid size (``pesq_pipeline_kernels``
names them): grids of more than 8192 scan wavefronts recompute the lane
states instead of storing them and launch the block prefix kernel (c5: 32256
forward, 16128 backward), smaller ones take their block starts from the two
previous blocks' aggregates (c4: 938 blocks per row, whose backward keeps
its aggregate launch for both filters), and grids of more than 512 frame tiles run four frames per
wavefront in the STFT and chain kernels (c4: 940 tiles, c5: 4096).  Those
variants only run at these shapes, so these tests run the whole batch of each
config, record the kernels the step launches (``torch.profiler``), check that
they are the variants the shape selects, and compare every item with the
float64 oracle on the CPU.  The reference's long-shape contract is
``tests/test_triton_loss.py:409-423`` (48 kHz x 12 s and 16 kHz x 30 s, with
gradients); the same kind of check, at the configs the bench times.

Tolerances:

* distances, MOS and loss: ``1e-5`` relative to float64 (the north star);
* the gradient w.r.t. the degraded signal: ``1e-4`` of the batch's largest
  float64 gradient, the bound of the c2 test in ``test_pipeline_gpu.py``
  (its signals have digital silence too).  The reference-signal gradient is
  not compared element-wise, for the reason given there.
"""

import pytest
import torch

from bench import speech_like_pair, synthetic_config
from kernel_trace import launched_kernels, library_kernels
from oracle import pesq_oracle as O
from torch_pesq import PesqLossTriton, _lib

pytestmark = pytest.mark.gpu

F64_RTOL = 1e-5
GRAD_RTOL = 1e-4


def _run_step(config):
    ref_np, deg_np, fs = synthetic_config(config)
    batch = ref_np.shape[0]
    model = PesqLossTriton(0.5, sample_rate=fs).cuda()
    ref = torch.from_numpy(ref_np).cuda()
    deg = torch.from_numpy(deg_np).cuda().requires_grad_(True)
    weights = torch.linspace(0.5, 1.5, batch, dtype=torch.float64)
    upstream = weights.float().cuda()

    def step():
        out = model._run(ref, deg)
        (g_deg,) = torch.autograd.grad(out[3], deg, grad_outputs=upstream)
        return out, g_deg

    step()  # first call: module buffers, allocator
    (outputs, g_deg), kernels = launched_kernels(step)
    outputs = [o.detach().double().cpu() for o in outputs]
    g_deg = g_deg.double().cpu()
    print(f"\nconfig {config}: {batch} x {ref_np.shape[1]} @ {fs} Hz, kernels {sorted(kernels)}",
          flush=True)
    return ref_np, deg_np, fs, weights, outputs, g_deg, kernels


def _compare_with_oracle(ref_np, deg_np, fs, weights, outputs, g_deg, items):
    worst = dict.fromkeys(("d_symm", "d_asymm", "mos", "loss"), 0.0)
    grad_num, grad_den = 0.0, 0.0
    saturated = 0
    for i in items:
        r = torch.from_numpy(ref_np[i : i + 1]).double()
        d = torch.from_numpy(deg_np[i : i + 1]).double().requires_grad_(True)
        ds, da = O.pipeline(r, d, sample_rate=fs)
        mos, loss = O.epilogue(ds, da, 0.5)
        (want_g,) = torch.autograd.grad(loss.sum() * float(weights[i]), d)
        for name, got, want in zip(worst, outputs, (ds, da, mos, loss)):
            want = want.detach()
            err = abs(float(got[i]) - float(want)) / abs(float(want))
            worst[name] = max(worst[name], err)
        grad_num = max(grad_num, float((g_deg[i] - want_g[0]).abs().max()))
        grad_den = max(grad_den, float(want_g.abs().max()))
        saturated += int(float(da) >= 45.0 - 1e-9)
    grad_err = grad_num / grad_den
    print(f"items {len(items)}: worst rel err {worst}, deg-grad err {grad_err:.2e}, "
          f"d_asymm at the 45 clamp in {saturated} items", flush=True)
    for name, err in worst.items():
        assert err < F64_RTOL, (name, err)
    assert grad_err < GRAD_RTOL, grad_err
    return saturated


def _assert_pipeline_variants(kernels, batch, length):
    for backward in (False, True):
        want = library_kernels(batch, length, _lib.GRAD_DEG, backward)
        missing = [k for k in want if k not in kernels]
        assert not missing, (backward, missing, sorted(kernels))
    ours = set(library_kernels(batch, length, _lib.GRAD_DEG, False))
    ours |= set(library_kernels(batch, length, _lib.GRAD_DEG, True))
    others = {k for k in kernels if k not in ours and not k.startswith("resample_")}
    # the step's only other launches: none (the upstream gradient is a
    # contiguous float32 tensor and no sum is taken)
    assert not others, sorted(others)


def test_config4_full_batch_forward_and_backward():
    """4 x 60 s: windowed block starts over rows of 938 blocks in both scan
    passes, four frames per wavefront."""

    ref_np, deg_np, fs, weights, outputs, g_deg, kernels = _run_step(4)
    batch, length = ref_np.shape
    _assert_pipeline_variants(kernels, batch, length)
    for name in ("iir_aggregate_split_kernel<5,1,3,PipeBwdMode>",
                 "iir_output_kernel<5,1,PipeBwdMode,true,2,false>",
                 "iir_output_kernel<5,1,PipeFwdMode,true,2,false>", "chain_bwd_kernel<4,1>",
                 "chain_fwd_kernel<4,1>"):
        assert name in kernels, name
    assert "iir_prefix_kernel<6>" not in kernels
    # the STFT variant for large grids (its arithmetic type is the library's choice)
    assert any(k.startswith("stft_fwd_kernel<") and k.endswith(",true,8>") for k in kernels)
    saturated = _compare_with_oracle(ref_np, deg_np, fs, weights, outputs, g_deg, range(batch))
    # 0 dB pink noise then clipping: the asymmetric distance sits at its clamp,
    # the symmetric one does not, so the comparison above still measures the chain
    assert all(float(v) < 44.0 for v in outputs[0]), outputs[0]
    assert saturated <= batch


def test_config5_full_batch_forward_and_backward():
    """256 x 4 s at 48 kHz: lane states recomputed in both scan passes (grids of
    32256 and 16128 wavefronts), the 3:1 window resampler and its adjoint."""

    ref_np, deg_np, fs, weights, outputs, g_deg, kernels = _run_step(5)
    batch = ref_np.shape[0]
    length = O.resample_length(ref_np.shape[1], fs, 16000)
    _assert_pipeline_variants(kernels, batch, length)
    for name in ("iir_aggregate_kernel<5,1,PipeFwdMode,false,0,6>", "iir_prefix_kernel<6>",
                 "iir_output_kernel<5,1,PipeFwdMode,false,0,false>",
                 "iir_aggregate_kernel<5,1,PipeBwdMode,false,0,6>",
                 "iir_output_kernel<5,1,PipeBwdMode,false,0,false>",
                 "chain_bwd_kernel<4,1>", "resample_fwd_window<3>", "resample_bwd_window<3>"):
        assert name in kernels, name
    _compare_with_oracle(ref_np, deg_np, fs, weights, outputs, g_deg, range(batch))


def test_config3_full_batch_forward_and_backward():
    """16 x 4 s at 44.1 kHz: the 441:160 phase-major resampler and its adjoint over
    the full batch (the 16 kHz pipeline grid is small, like c2)."""

    ref_np, deg_np, fs, weights, outputs, g_deg, kernels = _run_step(3)
    batch = ref_np.shape[0]
    length = O.resample_length(ref_np.shape[1], fs, 16000)
    _assert_pipeline_variants(kernels, batch, length)
    # the forward of both signals in one launch (34 taps per phase, the 36-tap
    # instantiation with float samples) and the adjoint (the transposed bank, a
    # resampler from 16 kHz to 44.1 kHz with 13 taps per phase: 16 taps, double
    # samples)
    resamplers = {k: v for k, v in kernels.items() if k.startswith("resample")}
    assert resamplers == {
        "resample_phase_major<36,float>": 1,
        "resample_phase_major<16,double>": 1,
    }, resamplers
    _compare_with_oracle(ref_np, deg_np, fs, weights, outputs, g_deg, range(batch))



def test_config4_length_unsaturated_items():
    """Three 60 s items of the speech-like pair at a moderate noise level: the
    c4 row length (windowed block starts in both scan passes, the band totals kernel)
    and the four-frame chain variants (705 chain tiles), with both distances
    inside their clamps, so the asymmetric path of 60 s rows (its fifth root
    asymmetry factor, the band totals feeding it) is compared with float64."""

    ref_np, deg_np = speech_like_pair(3, 960000, seed=44, noise=0.1)
    fs = 16000
    model = PesqLossTriton(0.5, sample_rate=fs).cuda()
    ref = torch.from_numpy(ref_np).cuda()
    deg = torch.from_numpy(deg_np).cuda().requires_grad_(True)
    weights = torch.linspace(0.5, 1.5, 3, dtype=torch.float64)
    upstream = weights.float().cuda()

    def step():
        out = model._run(ref, deg)
        (g_deg,) = torch.autograd.grad(out[3], deg, grad_outputs=upstream)
        return out, g_deg

    step()
    (outputs, g_deg), kernels = launched_kernels(step)
    _assert_pipeline_variants(kernels, 3, 960000)
    for name in ("iir_output_kernel<5,1,PipeFwdMode,true,2,false>", "chain_fwd_kernel<4,1>",
                 "chain_bwd_kernel<4,1>"):
        assert name in kernels, name
    assert any(k.startswith("band_totals_kernel<") for k in kernels)
    outputs = [o.detach().double().cpu() for o in outputs]
    saturated = _compare_with_oracle(ref_np, deg_np, fs, weights, outputs, g_deg.double().cpu(),
                                     range(3))
    assert saturated == 0, outputs[1]
    assert all(0.0 < float(v) < 44.0 for v in outputs[1]), outputs[1]
