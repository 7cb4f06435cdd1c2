"""The decode entry point that allocates nothing (ftmoe_experts_decode_noalloc,
its workspace a static device array) against the workspace entry point
ftmoe_experts_decode, both called through the C ABI: bit-identical outputs on
two calls in a row, the second with a smaller batch (the array keeps the first
call's contents), replays of a captured no-alloc call, and a clear refusal
beyond the array's size."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import synth
from freetoken_amd import _lib

from _helpers import bf16_dev, to_device_bank

pytestmark = pytest.mark.gpu


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _call_pair(dev, L, bank, shared, x, w, ids):
    """(y from ftmoe_experts_decode with a caller workspace, y from the no-alloc entry)."""
    M, k = ids.shape
    b = bank.cstruct()
    sb = shared.cstruct() if shared is not None else None
    bp, sp = ctypes.byref(b), (ctypes.byref(sb) if sb is not None else None)
    nbytes = L.ftmoe_experts_decode_workspace(M, k, bp, sp)
    assert 0 < nbytes <= L.ftmoe_experts_decode_noalloc_capacity()
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    y_ws = torch.empty_like(x)
    y_na = torch.full_like(x, float("nan"))
    _lib.check(L.ftmoe_experts_decode(x.data_ptr(), M, k, w.data_ptr(), ids.data_ptr(), bp, sp, 0, 0, y_ws.data_ptr(),
                                      ws.data_ptr(), nbytes, _stream(dev)), "experts_decode")
    _lib.check(L.ftmoe_experts_decode_noalloc(x.data_ptr(), M, k, w.data_ptr(), ids.data_ptr(), bp, sp, 0, 0,
                                              y_na.data_ptr(), _stream(dev)), "experts_decode_noalloc")
    torch.cuda.synchronize()
    return y_ws, y_na


@pytest.mark.parametrize("fmt,sfmt", [("fp8", "fp8"), ("mxfp4", "bf16")])
def test_noalloc_decode_matches_workspace_entry(dev, fmt, sfmt):
    rng = np.random.default_rng(7)
    E, H, I, k = 32, 1024, 512, 8
    bank = to_device_bank(synth.make_bank(fmt, E, H, I, rng), dev)
    shared = to_device_bank(synth.make_bank(sfmt, 1, H, I, rng), dev)
    L = _lib.lib()
    for M in (64, 5):  # a second, smaller call: the array holds the first call's contents
        x = bf16_dev(synth.activations(rng, M, H), dev)
        ids = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)).to(dev)
        w = torch.from_numpy(rng.random((M, k), dtype=np.float32)).to(dev)
        y_ws, y_na = _call_pair(dev, L, bank, shared, x, w, ids)
        assert torch.equal(y_ws, y_na), M


def test_noalloc_decode_refuses_beyond_capacity(dev):
    rng = np.random.default_rng(8)
    E, H, I, k = 4, 7168, 2048, 8
    bank = to_device_bank(synth.make_bank("bf16", E, 256, 128, rng), dev)
    b = bank.cstruct()
    b.hidden, b.inter = H, I  # shape only: the call must stop at the size check, before any launch
    L = _lib.lib()
    M = 4096  # ~0.5 GB of decode scratch at H 7168, I 2048
    assert L.ftmoe_experts_decode_workspace(M, k, ctypes.byref(b), None) > L.ftmoe_experts_decode_noalloc_capacity()
    rc = L.ftmoe_experts_decode_noalloc(None, M, k, None, None, ctypes.byref(b), None, 0, 0, None, _stream(dev))
    assert rc == _lib.FTMOE_ERR_WORKSPACE
    assert b"beyond the static" in L.ftmoe_last_error()


def test_noalloc_decode_graph_replays_equal_workspace_entry(dev):
    """A no-alloc call captured in a HIP graph (after one eager call on the
    device, which looks up the array's address) replays bit for bit like the
    workspace entry point on the inputs written into the captured buffers, with
    eager no-alloc calls of another batch between the replays."""
    rng = np.random.default_rng(9)
    E, H, I, k, M = 32, 1024, 512, 8, 4
    bank = to_device_bank(synth.make_bank("fp8", E, H, I, rng), dev)
    shared = to_device_bank(synth.make_bank("fp8", 1, H, I, rng), dev)
    L = _lib.lib()
    b, sb = bank.cstruct(), shared.cstruct()
    bp, sp = ctypes.byref(b), ctypes.byref(sb)

    def inputs(m):
        x = bf16_dev(synth.activations(rng, m, H), dev)
        ids = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(m)]).astype(np.int32)).to(dev)
        w = torch.from_numpy(rng.random((m, k), dtype=np.float32)).to(dev)
        return x, w, ids

    x_buf, w_buf, i_buf = inputs(M)
    y_buf = torch.empty_like(x_buf)

    def noalloc(x, w, ids, y, stream):
        return L.ftmoe_experts_decode_noalloc(x.data_ptr(), x.shape[0], k, w.data_ptr(), ids.data_ptr(), bp, sp, 0, 0,
                                              y.data_ptr(), stream)

    _lib.check(noalloc(x_buf, w_buf, i_buf, y_buf, _stream(dev)), "experts_decode_noalloc (eager)")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            rc = noalloc(x_buf, w_buf, i_buf, y_buf, stream.cuda_stream)
    assert rc == _lib.FTMOE_OK, L.ftmoe_last_error()
    torch.cuda.synchronize()
    for rep in range(3):
        x, w, ids = inputs(M)
        x_buf.copy_(x)
        w_buf.copy_(w)
        i_buf.copy_(ids)
        xo, wo, io = inputs(9)  # an eager no-alloc call of another batch overwrites the array between replays
        _lib.check(noalloc(xo, wo, io, torch.empty_like(xo), _stream(dev)), "experts_decode_noalloc (between)")
        graph.replay()
        torch.cuda.synchronize()
        y_ws, _ = _call_pair(dev, L, bank, shared, x, w, ids)
        assert torch.equal(y_buf, y_ws), rep
        assert bool(torch.isfinite(y_buf.float()).all())
    del graph
