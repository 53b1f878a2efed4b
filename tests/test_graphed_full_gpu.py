"""The graph modes at the BASELINE shapes, bit for bit against eager.

The reference promises that ``PesqLossTriton.graphed`` is bit exact with the
eager loss (``triton_ops/loss.py:149-201``, tested at
``tests/test_triton_loss.py:426-442``).  The other graph tests run small
shapes; these run the shapes the bench times:

* c2 (8 x 128000 at 16 kHz, BASELINE ``configs[1]``, "hipGraph-replayed"):
  ``graphed()`` replays, gradient w.r.t. deg, bitwise against eager over
  several replays with eager work between them, on the batch's own buffers
  (the first call stages them into the static inputs, later calls read them
  in place from a graph captured for their addresses), and one replay against
  the float64 oracle (1e-5 on the loss, 1e-4 of the largest gradient);
* c5 (256 x 192000 at 48 kHz, ``configs[4]``, "hipGraph step"): the whole
  step as one graph (``graphed_step``) and ``graphed()``, both bitwise
  against the eager step; this shape runs the large-grid kernel variants and
  the 3:1 resampler inside the graphs.

Also: a graphed loss whose calls alternate between two streams over more
input buffer pairs than it keeps graphs for (a graph is released while the
other stream may still run it unless it waits for that graph's own launch).
"""

import pytest
import torch

from bench import speech_like_pair, synthetic_config
from oracle import pesq_oracle as O
from torch_pesq import PesqLossTriton

pytestmark = pytest.mark.gpu

F64_RTOL = 1e-5
GRAD_RTOL = 1e-4


def _eager(model, r, d):
    d = d.detach().requires_grad_(True)
    loss = model(r, d)
    (g,) = torch.autograd.grad(loss.sum(), d)
    return loss.detach().clone(), g.clone()


def test_graphed_c2_full_batch():
    ref_np, deg_np, fs = synthetic_config(2)
    model = PesqLossTriton(0.5, sample_rate=fs).cuda()
    r = torch.from_numpy(ref_np).cuda()
    d = torch.from_numpy(deg_np).cuda().requires_grad_(True)
    want_loss, want_g = _eager(model, r, d)
    graphed = model.graphed(r, d)
    first = None
    for step in range(4):
        loss = graphed(r, d)
        (g,) = torch.autograd.grad(loss.sum(), d)
        torch.cuda.synchronize()
        assert torch.equal(loss, want_loss), step
        assert torch.equal(g, want_g), step
        if first is None:
            first = (loss.double().cpu(), g.double().cpu())
        # eager work on other inputs between the replays
        model(r * 0.5, d.detach() + 0.01)
        torch.cuda.synchronize()
    print(f"\nc2 graphed: {want_loss.tolist()}", flush=True)

    loss, g = first
    rd = torch.from_numpy(ref_np).double()
    dd = torch.from_numpy(deg_np).double().requires_grad_(True)
    ds, da = O.pipeline(rd, dd)
    _, want = O.epilogue(ds, da, 0.5)
    (want_grad,) = torch.autograd.grad(want.sum(), dd)
    err = float(((loss - want.detach()) / want.detach()).abs().max())
    gerr = float((g - want_grad).abs().max() / want_grad.abs().max())
    print(f"c2 graphed vs float64: loss {err:.2e}, deg gradient {gerr:.2e}", flush=True)
    assert err < F64_RTOL
    assert gerr < GRAD_RTOL


@pytest.fixture(scope="module")
def c5():
    ref_np, deg_np, fs = synthetic_config(5)
    model = PesqLossTriton(0.5, sample_rate=fs).cuda()
    r = torch.from_numpy(ref_np).cuda()
    d = torch.from_numpy(deg_np).cuda()
    return model, r, d


def test_graphed_step_c5_full_batch(c5):
    model, r, d = c5
    want_loss, want_g = _eager(model, r, d)
    step = model.graphed_step(r, d.detach().requires_grad_(True))
    static_r, static_d = step.inputs()
    assert torch.equal(static_r, r) and torch.equal(static_d, d)
    for replay in range(3):
        step.replay()
        torch.cuda.synchronize()
        loss, g_ref, g_deg = step.outputs()
        assert g_ref is None
        assert torch.equal(loss, want_loss), replay
        assert torch.equal(g_deg, want_g), replay
        model(r * 0.5, d + 0.01)
        torch.cuda.synchronize()
    # new contents written into the static inputs
    with torch.no_grad():
        static_d.mul_(0.5).add_(0.01 * r)
    want_loss, want_g = _eager(model, r, static_d.clone())
    step.replay()
    torch.cuda.synchronize()
    loss, _, g_deg = step.outputs()
    assert torch.equal(loss, want_loss)
    assert torch.equal(g_deg, want_g)
    print(f"\nc5 graphed step: {r.shape[0]} items bitwise equal to eager", flush=True)


def test_graphed_c5_full_batch(c5):
    model, r, d = c5
    want_loss, want_g = _eager(model, r, d)
    d = d.clone().requires_grad_(True)
    graphed = model.graphed(r, d)
    for replay in range(3):
        loss = graphed(r, d)
        (g,) = torch.autograd.grad(loss.sum(), d)
        torch.cuda.synchronize()
        assert torch.equal(loss, want_loss), replay
        assert torch.equal(g, want_g), replay


def test_graphed_alternating_streams_over_many_buffer_pairs():
    """Calls alternate between two streams over six buffer pairs (the loss
    keeps forward graphs for four), each pair passed twice in a row; each
    stream waits for the other's previous call, so the replays never overlap,
    but the host runs ahead and drops graphs whose last replay may still be
    queued on the other stream."""

    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = speech_like_pair(2, 32000, seed=41, noise=0.1)
    r, d = torch.from_numpy(r).cuda(), torch.from_numpy(d).cuda()
    pairs = [(r * (1 + i), (d * (1 + i) + 0.01 * i * r).requires_grad_(True)) for i in range(6)]
    want = [_eager(model, rb, db) for rb, db in pairs]
    graphed = model.graphed(r, pairs[0][1])
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    results = []
    turn = 0
    for sweep in range(2):
        for i, (rb, db) in enumerate(pairs):
            for call in range(2):
                stream = streams[turn % 2]
                stream.wait_stream(streams[(turn + 1) % 2])
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):
                    loss = graphed(rb, db)
                    (g,) = torch.autograd.grad(loss.sum(), db)
                    # the results alias static buffers: copy them out on this stream
                    results.append((i, loss.clone(), g.clone()))
                turn += 1
    torch.cuda.synchronize()
    for i, loss, g in results:
        assert torch.equal(loss, want[i][0]), i
        assert torch.equal(g, want[i][1]), i
    del graphed
    torch.cuda.synchronize()
