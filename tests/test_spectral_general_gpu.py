"""GPU parity of the STFT / Bark operator beyond the PESQ geometry.

``HipStftBark`` with other FFT lengths, band counts, hops and short windows
runs the general kernels of ``csrc/stft_generic.hip``; the cases follow the
reference's ``tests/test_triton_spectral.py:294-312,340-420,638-700``.

Oracle: ``oracle.pesq_oracle.stft_bark_op`` (float64 ``torch.stft``, DC
dropped, band sums), pinned against a direct float64 DFT in
``test_oracle.py``; gradients by float64 autograd through it.

Tolerance, the reference's error model for a spectrogram
(``test_triton_spectral.py:1-45``): ``|got - want| <= RTOL |want| + ATOL *
local_scale`` with the local scale the peak of the frame (forward) or of the
gradient over the frames a sample belongs to (backward); ``RTOL = 1e-5``,
``ATOL = 5e-6`` forward and ``1e-5`` backward.  The float64 FFT leaves the
float32 rounding of the outputs (about 1e-7).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import pesq_oracle as O
from torch_pesq.bark import BarkScale
from torch_pesq.hip_ops.spectral import HipStftBark

pytestmark = pytest.mark.gpu

RTOL = 1e-5
ATOL_FWD = 5e-6
ATOL_BWD = 1e-5


def _module(n_fft=512, nbarks=49, hop=256, window=None):
    scale = BarkScale(n_fft // 2, nbarks)
    window = torch.hann_window(n_fft) if window is None else window
    mod = HipStftBark(window, scale.fbank, scale.pow_dens_correction, n_fft, hop).cuda()
    return mod, window, scale


def _oracle(signal, mod, window, scale, n_padded=None):
    return O.stft_bark_op(signal.double().cpu(), window, scale.fbank, scale.pow_dens_correction,
                          mod.n_fft, mod.hop_length, n_padded)


def _violation(got, want, atol, scale):
    delta = (got.double().cpu() - want).abs()
    return float((delta - (RTOL * want.abs() + atol * scale)).max())


def _frame_scale(want):
    return want.abs().amax(dim=2, keepdim=True)


def _sample_scale(grad, hop, novertaps):
    n = grad.shape[1]
    blocks = F.pad(grad.abs(), (0, (-n) % hop)).reshape(grad.shape[0], -1, hop).amax(dim=2)
    dilated = F.max_pool1d(blocks.unsqueeze(1), 2 * novertaps + 1, 1, novertaps).squeeze(1)
    return dilated.repeat_interleave(hop, dim=1)[:, :n]


def _both(mod, window, scale, signal, n_padded=None, seed=0):
    x = signal.clone().requires_grad_(True)
    got = mod(x, n_padded)
    gen = torch.Generator().manual_seed(seed)
    up = torch.randn(got.shape, generator=gen, dtype=torch.float64)
    (g_got,) = torch.autograd.grad(got, x, up.float().cuda())
    xd = signal.double().cpu().requires_grad_(True)
    want = O.stft_bark_op(xd, window, scale.fbank, scale.pow_dens_correction, mod.n_fft,
                          mod.hop_length, n_padded)
    (g_want,) = torch.autograd.grad(want, xd, up)
    return got, want.detach(), g_got, g_want


@pytest.mark.parametrize("n_fft,nbarks", [(512, 32), (256, 49), (256, 32), (1024, 49), (64, 17)])
@pytest.mark.parametrize("batch,nsamples", [(1, 4096), (3, 5003), (5, 1024)])
def test_forward_parity(n_fft, nbarks, batch, nsamples):
    mod, window, scale = _module(n_fft, nbarks)
    assert mod.general
    torch.manual_seed(nsamples + n_fft + nbarks)
    signal = torch.randn(batch, nsamples, device="cuda") * 3000.0
    got = mod(signal)
    want = _oracle(signal, mod, window, scale)
    assert got.shape == want.shape
    assert _violation(got, want, ATOL_FWD, _frame_scale(want)) <= 0.0


@pytest.mark.parametrize("n_fft,nbarks", [(512, 32), (256, 49)])
def test_backward_parity(n_fft, nbarks):
    mod, window, scale = _module(n_fft, nbarks)
    torch.manual_seed(n_fft + nbarks)
    signal = torch.randn(3, 5003, device="cuda") * 1000.0
    got, want, g_got, g_want = _both(mod, window, scale, signal, seed=3)
    assert _violation(got, want, ATOL_FWD, _frame_scale(want)) <= 0.0
    scale_s = _sample_scale(g_want, mod.hop_length, mod.novertaps)
    assert _violation(g_got, g_want, ATOL_BWD, scale_s) <= 0.0


@pytest.mark.parametrize("hop_length", [128, 600, 100, 37])
def test_hop_length_sweep(hop_length):
    mod, window, scale = _module(512, 49, hop_length)
    assert mod.general
    assert mod.novertaps == -(-512 // hop_length)
    torch.manual_seed(hop_length)
    signal = torch.randn(2, 4096, device="cuda") * 1000.0
    got, want, g_got, g_want = _both(mod, window, scale, signal, seed=hop_length)
    assert got.shape[1] == 1 + (4096 - 512) // hop_length
    assert _violation(got, want, ATOL_FWD, _frame_scale(want)) <= 0.0
    scale_s = _sample_scale(g_want, hop_length, mod.novertaps)
    assert _violation(g_got, g_want, ATOL_BWD, scale_s) <= 0.0


def test_gradient_is_zero_in_the_gaps_between_frames():
    mod, window, scale = _module(512, 49, 600)
    signal = (torch.randn(1, 3000, device="cuda") * 1000.0).requires_grad_(True)
    out = mod(signal)
    (g,) = torch.autograd.grad(out.sum(), signal)
    covered = torch.zeros(3000, dtype=torch.bool)
    for t in range(out.shape[1]):
        covered[600 * t : 600 * t + 512] = True
    assert torch.count_nonzero(g[0, ~covered.cuda()]) == 0
    assert torch.count_nonzero(g[0, covered.cuda()]) > 0


@pytest.mark.parametrize("win_length", [400, 401, 33])
def test_short_window_is_centred(win_length):
    window = torch.hann_window(win_length)
    mod, _, scale = _module(512, 49, 256, window)
    torch.manual_seed(23)
    signal = torch.randn(2, 4096, device="cuda") * 1000.0
    got, want, g_got, g_want = _both(mod, window, scale, signal, seed=win_length)
    assert _violation(got, want, ATOL_FWD, _frame_scale(want)) <= 0.0
    scale_s = _sample_scale(g_want, 256, mod.novertaps)
    assert _violation(g_got, g_want, ATOL_BWD, scale_s) <= 0.0


def test_padding_and_tail_samples():
    """Frames past the signal read zeros; samples after the last frame get no gradient."""

    mod, window, scale = _module(256, 32, 128)
    torch.manual_seed(5)
    signal = torch.randn(2, 3001, device="cuda") * 100.0
    got, want, g_got, g_want = _both(mod, window, scale, signal, n_padded=3200, seed=5)
    assert got.shape[1] == 1 + (3200 - 256) // 128
    assert _violation(got, want, ATOL_FWD, _frame_scale(want)) <= 0.0
    scale_s = _sample_scale(g_want, 128, mod.novertaps)
    assert _violation(g_got, g_want, ATOL_BWD, scale_s) <= 0.0


def test_general_path_is_deterministic_and_rows_independent():
    mod, _, _ = _module(256, 49, 100)
    signal = torch.randn(4, 6000, device="cuda").requires_grad_(True)
    a, b = mod(signal), mod(signal)
    assert torch.equal(a, b)
    assert torch.equal(mod(signal[2:3]), a[2:3])
    (g1,) = torch.autograd.grad(a.sum(), signal)
    (g2,) = torch.autograd.grad(mod(signal).sum(), signal)
    assert torch.equal(g1, g2)


def test_default_geometry_agrees_with_the_general_kernels():
    """The PESQ geometry through both kernel families (radix-4 vs radix-2)."""

    mod, window, scale = _module(512, 49, 256)
    assert not mod.general
    torch.manual_seed(9)
    signal = torch.randn(2, 8000, device="cuda") * 1000.0
    want = _oracle(signal, mod, window, scale)
    got = mod(signal)
    assert _violation(got, want, ATOL_FWD, _frame_scale(want)) <= 0.0
    mod.general = True  # route the same constants through the general kernels
    mod.table = _general_table_for(mod, window, scale)
    got2 = mod(signal)
    assert _violation(got2, want, ATOL_FWD, _frame_scale(want)) <= 0.0


def _general_table_for(mod, window, scale):
    from torch_pesq.hip_ops.spectral import _general_table

    return _general_table(mod.window, mod.starts, mod.ends, scale.pow_dens_correction,
                          mod.n_fft, mod.hop_length).cuda()


# ---------------------------------------------------------------------------
# the whole loss at other STFT geometries (PesqLossTriton(n_fft=..., ...))
# ---------------------------------------------------------------------------

GEOMETRIES = [(256, 256, 128), (512, 400, 256), (512, 512, 200), (1024, 1024, 512)]


def _oracle_constants(n_fft, win_length, hop):
    c = dict(O.constants())
    c.update(n_fft=n_fft, hop=hop, window=torch.hann_window(win_length).double(),
             fbank=O.bark_fbank(n_fft // 2, 49))
    return c


@pytest.mark.parametrize("n_fft,win_length,hop", GEOMETRIES)
def test_loss_at_other_geometries_matches_float64(n_fft, win_length, hop):
    from bench import speech_like_pair
    from torch_pesq import PesqLossTriton

    model = PesqLossTriton(0.5, sample_rate=16000, n_fft=n_fft, win_length=win_length,
                           hop_length=hop).cuda()
    assert model.general
    ref, deg = speech_like_pair(2, 24000, seed=n_fft + hop, noise=0.1)
    r = torch.from_numpy(ref).cuda().requires_grad_(True)
    d = torch.from_numpy(deg).cuda().requires_grad_(True)
    ds, da, mos, loss = model._run(r, d)
    weights = torch.tensor([0.7, -1.3], dtype=torch.float64)
    g_ref, g_deg = torch.autograd.grad(loss, [r, d], grad_outputs=weights.float().cuda())

    c = _oracle_constants(n_fft, win_length, hop)
    rd = torch.from_numpy(ref).double().requires_grad_(True)
    dd = torch.from_numpy(deg).double().requires_grad_(True)
    wds, wda = O.pipeline(rd, dd, c=c)
    wmos, wloss = O.epilogue(wds, wda, 0.5)
    (wloss * weights).sum().backward()

    for name, got, want in (("d_symm", ds, wds), ("d_asymm", da, wda), ("mos", mos, wmos),
                            ("loss", loss, wloss)):
        got, want = got.detach().double().cpu(), want.detach()
        assert float(((got - want).abs() / want.abs()).max()) < 1e-5, name
    for name, got, want in (("g_ref", g_ref, rd.grad), ("g_deg", g_deg, dd.grad)):
        err = float((got.double().cpu() - want).abs().max() / want.abs().max())
        assert err < 2e-5, (name, err)


def test_other_geometry_rejects_too_few_frames():
    from torch_pesq import PesqLossTriton

    model = PesqLossTriton(0.5, sample_rate=16000, n_fft=256, win_length=256, hop_length=512).cuda()
    x = torch.randn(1, 8000, device="cuda")
    with pytest.raises(ValueError, match="20 frames"):
        model(x, x)
