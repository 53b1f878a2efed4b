"""The no-allocation forward entry point against the allocating one.

``pesq_pipeline_forward_noalloc`` runs ``pesq_pipeline_forward`` (grad_mask 0)
on the library's static device scratch instead of a caller workspace.  Two
calls in a row, the second on a smaller input, must each give bitwise the
outputs of the allocating entry point; a shape whose workspace exceeds the
scratch is rejected on the host before any GPU work.  The call captured in a
HIP graph (the callers it is for), with and without an eager call before the
capture, replays to the allocating entry point's bits, new input contents
included.
"""

import ctypes

import pytest
import torch

from bench import speech_like_pair
from torch_pesq import PesqLossTriton, _lib

pytestmark = pytest.mark.gpu


def _outputs(batch):
    return [torch.full((batch,), float("nan"), device="cuda") for _ in range(4)]


def _allocating(ref, deg, table, factor):
    lib = _lib.library()
    batch, length = ref.shape
    ws = torch.empty(_lib.size_query(lib.pesq_pipeline_forward_workspace, batch, length, 0),
                     dtype=torch.uint8, device="cuda")
    out = _outputs(batch)
    _lib.check(lib.pesq_pipeline_forward(
        _lib.ptr(ref), _lib.ptr(deg), batch, length, _lib.ptr(table), factor, 0,
        *[_lib.ptr(o) for o in out], _lib.ptr(ws), _lib.stream_handle(ref.device)),
        "pesq_pipeline_forward")
    return out


def _noalloc(ref, deg, table, factor):
    lib = _lib.library()
    batch, length = ref.shape
    out = _outputs(batch)
    _lib.check(lib.pesq_pipeline_forward_noalloc(
        _lib.ptr(ref), _lib.ptr(deg), batch, length, _lib.ptr(table), factor,
        *[_lib.ptr(o) for o in out], _lib.stream_handle(ref.device)),
        "pesq_pipeline_forward_noalloc")
    return out


def _capture_noalloc(ref, deg, table, factor):
    """One noalloc call captured in a HIP graph (torch.cuda.graph) on the
    capture stream; returns the graph and its output buffers."""

    lib = _lib.library()
    batch, length = ref.shape
    out = _outputs(batch)  # filled before the capture, not inside it
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.pesq_pipeline_forward_noalloc(
            _lib.ptr(ref), _lib.ptr(deg), batch, length, _lib.ptr(table), factor,
            *[_lib.ptr(o) for o in out], _lib.stream_handle(ref.device))
    _lib.check(status, "pesq_pipeline_forward_noalloc (captured)")
    return graph, out


def _check_graph_replays(warm_up):
    table = PesqLossTriton(0.5, sample_rate=16000).cuda().model_table
    ref_np, deg_np = speech_like_pair(4, 48000, seed=35, noise=0.1)
    ref, deg = torch.from_numpy(ref_np).cuda(), torch.from_numpy(deg_np).cuda()
    if warm_up:
        _noalloc(ref, deg, table, 0.5)
        torch.cuda.synchronize()
    graph, out = _capture_noalloc(ref, deg, table, 0.5)
    for scale in (1.0, 1.0, 0.5, 2.0):
        with torch.no_grad():
            deg.copy_(torch.from_numpy(deg_np).cuda() * scale + 0.01 * (scale - 1.0) * ref)
        want = _allocating(ref, deg, table, 0.5)
        graph.replay()
        torch.cuda.synchronize()
        for name, g, w in zip(("d_symm", "d_asymm", "mos", "loss"), out, want):
            assert torch.isfinite(g).all(), (scale, name)
            assert torch.equal(g, w), (scale, name)
        # eager work between the replays
        _allocating(ref * 0.5, deg, table, 0.5)
        torch.cuda.synchronize()


def test_noalloc_forward_captured_without_a_warm_up_call():
    """The first noalloc call of the process (its device's scratch address is
    looked up there) made under graph capture; no other test file calls the
    entry point, and this is the first test of this file."""

    _check_graph_replays(warm_up=False)


def test_noalloc_forward_captured_after_a_warm_up_call():
    _check_graph_replays(warm_up=True)


def test_noalloc_forward_matches_the_allocating_entry_point():
    table = PesqLossTriton(0.5, sample_rate=16000).cuda().model_table
    for batch, samples, seed in ((8, 128000, 31), (3, 40000, 32)):
        ref_np, deg_np = speech_like_pair(batch, samples, seed=seed, noise=0.1)
        ref, deg = torch.from_numpy(ref_np).cuda(), torch.from_numpy(deg_np).cuda()
        want = _allocating(ref, deg, table, 0.5)
        got = _noalloc(ref, deg, table, 0.5)
        torch.cuda.synchronize()
        for name, g, w in zip(("d_symm", "d_asymm", "mos", "loss"), got, want):
            assert torch.isfinite(g).all(), (batch, name)
            assert torch.equal(g, w), (batch, name)


def test_noalloc_forward_rejects_shapes_beyond_its_scratch():
    lib = _lib.library()
    batch, samples = 16, 128000
    need = _lib.size_query(lib.pesq_pipeline_forward_workspace, batch, samples, 0)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    # rejected before any pointer is touched: NULL pointers are fine here
    status = lib.pesq_pipeline_forward_noalloc(None, None, batch, samples, None, 1.0,
                                               None, None, None, None, None)
    assert status == _lib.ERR_ARGUMENT
    assert b"static scratch" in lib.pesq_last_error()
