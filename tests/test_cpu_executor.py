"""The host-side expert executor of the hybrid decode (ftmoe_cpu_experts,
freetoken_amd/csrc/cpu_experts.hip) against the oracle's decode layer
(oracle.experts.moe_layer, the reference's rounding points) on host banks of
every format: the routes the CPU takes in the reference's hybrid backend
(layers/moe.py:325-372, CPU pool of moe/cpu_executor.py).  No GPU needed:
the synchronous entry point touches no HIP call."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from freetoken_amd import _lib, ops

from _helpers import to_device_bank
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel


@pytest.fixture(scope="module")
def executor():
    ex = ops.CpuExecutor(threads=4)
    yield ex
    ex.close()


def _host(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype))


@pytest.mark.parametrize("fmt", ["bf16", "fp8", "mxfp4"])
@pytest.mark.parametrize("M,k,skip", [(1, 2, False), (3, 4, True), (5, 8, True)])
def test_cpu_experts_match_oracle(executor, fmt, M, k, skip):
    rng = np.random.default_rng(M * 10 + k)
    E, H, I = 8, 256, 384
    bank = synth.make_bank(fmt, E, H, I, rng)
    x = synth.activations(rng, M, H)
    logits = synth.normal(rng, (M, E))
    w, ids = oracle.routing.softmax_topk(logits, k, True)
    if skip:  # routes the GPU takes are passed as -1 and contribute nothing
        ids = ids.copy()
        ids[rng.random(ids.shape) < 0.4] = -1
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, None)
    hb = to_device_bank(bank, "cpu")
    y = executor.run(hb, _host(x, np.float32).to(torch.bfloat16), _host(w, np.float32), _host(ids, np.int32))
    g = y.float().numpy()
    assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (fmt, max_rel(g, y_ref))
    if skip:
        none = (ids < 0).all(axis=1)
        assert (g[none] == 0).all()  # a token with every route elsewhere gets exact zeros


def test_cpu_experts_activation_variants(executor):
    """gelu and gelu_tanh change only the activation of the gate rows."""
    rng = np.random.default_rng(3)
    E, H, I = 4, 128, 128
    bank = synth.make_bank("bf16", E, H, I, rng)
    hb = to_device_bank(bank, "cpu")
    x = synth.activations(rng, 2, H)
    w, ids = oracle.routing.softmax_topk(synth.normal(rng, (2, E)), 2, True)
    args = (_host(x, np.float32).to(torch.bfloat16), _host(w, np.float32), _host(ids, np.int32))
    ys = {a: executor.run(hb, *args, activation=a).float().numpy() for a in ("silu", "gelu", "gelu_tanh")}
    assert cosine(ys["gelu"], ys["gelu_tanh"]) > 0.999  # the tanh form approximates erf
    assert not np.array_equal(ys["silu"], ys["gelu"])
    for a, y in ys.items():  # each against the oracle's activation of that name
        y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, activation=a)
        assert max_rel(y, y_ref) <= MAX_REL_TOL and cosine(y, y_ref) >= COS_TOL, (a, max_rel(y, y_ref))


def test_cpu_experts_validation(executor):
    rng = np.random.default_rng(5)
    bank = synth.make_bank("fp8", 4, 256, 128, rng)
    hb = to_device_bank(bank, "cpu")
    x = torch.zeros(2, 256, dtype=torch.bfloat16)
    w = torch.ones(2, 2)
    with pytest.raises(ValueError):
        executor.run(hb, x, w, torch.zeros(2, 2, dtype=torch.int64))
    L = _lib.lib()
    b = hb.host_cstruct()
    b.hidden = 200  # not a multiple of 128
    rc = L.ftmoe_cpu_experts(executor._h, b, x.data_ptr(), w.data_ptr(), w.data_ptr(), 2, 2, 0, x.data_ptr())
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED
    assert L.ftmoe_cpu_experts(None, b, None, None, None, 2, 2, 0, None) == _lib.FTMOE_ERR_INVALID


def test_executor_reports_isa(executor):
    assert executor.isa in ("avx512bf16", "avx512f", "scalar")


def test_cpu_experts_hot_experts(executor):
    """More routes on one expert than one weight pass takes (split groups)."""
    rng = np.random.default_rng(9)
    E, H, I, M, k = 4, 256, 256, 11, 2
    bank = synth.make_bank("fp8", E, H, I, rng)
    x = synth.activations(rng, M, H)
    ids = np.tile(np.array([[1, 3]], dtype=np.int32), (M, 1))
    ids[4] = [3, 1]
    w = rng.uniform(0.1, 1.0, size=(M, k)).astype(np.float32)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, None)
    y = executor.run(to_device_bank(bank, "cpu"), _host(x, np.float32).to(torch.bfloat16), _host(w, np.float32),
                     _host(ids, np.int32))
    g = y.float().numpy()
    assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, max_rel(g, y_ref)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_cpu_experts_deterministic_across_pools(fmt):
    """A route's numbers do not depend on how the passes are split over the
    pool: 1, 3 and 8 threads, and many jobs back to back, give identical bytes."""
    rng = np.random.default_rng(17)
    E, H, I, M, k = 8, 256, 256, 6, 4
    bank = to_device_bank(synth.make_bank(fmt, E, H, I, rng), "cpu")
    x = _host(synth.activations(rng, M, H), np.float32).to(torch.bfloat16)
    w, ids = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
    w, ids = _host(w, np.float32), _host(ids, np.int32)
    outs = []
    for threads in (1, 3, 8):
        ex = ops.CpuExecutor(threads=threads)
        ys = [ex.run(bank, x, w, ids).clone() for _ in range(10)]
        ex.close()
        assert all(torch.equal(y, ys[0]) for y in ys)
        outs.append(ys[0])
    assert all(torch.equal(o, outs[0]) for o in outs)


def test_hybrid_fetch_fraction_rule():
    # tests/moe/test_hybrid_fetch.py:44-63: standalone pcie / cpu, overlapped pcie / (pcie + cpu)
    from freetoken_amd.moe.cpu_decode import hybrid_fetch_fraction

    assert hybrid_fetch_fraction(40.0, 100.0, overlapped=False) == pytest.approx(0.4)
    assert hybrid_fetch_fraction(30.0, 90.0) == pytest.approx(0.25)
    assert hybrid_fetch_fraction(50.0, 80.0, overlapped=False) == pytest.approx(0.625)
    assert hybrid_fetch_fraction(120.0, 100.0, overlapped=False) == 1.0
    assert hybrid_fetch_fraction(0.0, 100.0) is None


def _small_job(rng, fmt="bf16", M=2, k=2):
    E, H, I = 4, 128, 128
    bank = synth.make_bank(fmt, E, H, I, rng)
    x = synth.activations(rng, M, H)
    w, ids = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
    args = (to_device_bank(bank, "cpu"), _host(x, np.float32).to(torch.bfloat16), _host(w, np.float32),
            _host(ids, np.int32))
    return args, oracle.experts.moe_layer("decode", x, w, ids, bank, None)


def test_watchdog_fails_a_stalled_job_and_poisons_the_executor():
    """A pool that makes no progress (the driver held from the host) turns the
    wait into an error after the watchdog period instead of blocking for ever;
    the executor stays unhealthy and fails later jobs at once (the reference's
    flag watchdog, moe/cpu_executor.py:602-656)."""
    import time

    rng = np.random.default_rng(41)
    ex = ops.CpuExecutor(threads=2, watchdog_s=0.3)
    args, y_ref = _small_job(rng)
    y = ex.run(*args)
    assert max_rel(y.float().numpy(), y_ref) <= MAX_REL_TOL and ex.healthy
    ex.hold(True)
    t0 = time.monotonic()
    with pytest.raises(_lib.FtmoeError, match="watchdog"):
        ex.run(*args)
    assert 0.25 <= time.monotonic() - t0 < 5.0
    assert not ex.healthy
    with pytest.raises(RuntimeError, match="watchdog fired"):
        ex.raise_if_unhealthy()
    ex.hold(False)
    t0 = time.monotonic()
    with pytest.raises(_lib.FtmoeError, match="watchdog"):  # unhealthy for good: fails without waiting
        ex.run(*args)
    assert time.monotonic() - t0 < 0.25
    ex.close()


def test_watchdog_spares_a_working_pool():
    """With the watchdog armed, jobs of a working pool complete normally, many
    times in a row, and a job that waits behind others is not failed."""
    rng = np.random.default_rng(43)
    ex = ops.CpuExecutor(threads=2, watchdog_s=0.5)
    args, y_ref = _small_job(rng, "fp8", M=4, k=2)
    for _ in range(20):
        y = ex.run(*args)
        assert max_rel(y.float().numpy(), y_ref) <= MAX_REL_TOL
    assert ex.healthy
    ex.raise_if_unhealthy()
    ex.close()


def test_destroy_refused_while_captured_jobs_may_replay():
    """The C ABI refuses to free an executor that holds no captured jobs only
    when asked to keep them: with none captured, destroy succeeds at once."""
    L = _lib.lib()
    h = L.ftmoe_cpu_executor_create(1)
    assert h
    assert L.ftmoe_cpu_executor_healthy(h) == _lib.FTMOE_OK
    assert L.ftmoe_cpu_executor_destroy(h, 0) == _lib.FTMOE_OK
    assert L.ftmoe_cpu_executor_destroy(None, 0) == _lib.FTMOE_OK


def test_close_returns_when_the_pool_is_wedged():
    """A job stuck inside the pool (the driver stalls in it) is abandoned by the
    watchdog: ``close`` must not wait for the wedged threads (the executor is
    kept for the process instead), and when the stuck job moves again it writes
    nothing more to the caller's output."""
    import time

    rng = np.random.default_rng(47)
    ex = ops.CpuExecutor(threads=2, watchdog_s=0.3)
    args, _ = _small_job(rng)
    y = torch.full_like(args[1], 7.0)
    ex.stall(True)
    with pytest.raises(_lib.FtmoeError, match="watchdog"):
        ex.run(*args, y=y)
    assert not ex.healthy
    h = ex._h
    t0 = time.monotonic()
    ex.close()
    assert time.monotonic() - t0 < 2.0 and ex._h is None
    assert ops._KEPT_EXECUTORS and ops._KEPT_EXECUTORS[-1] == h
    L = _lib.lib()
    L.ftmoe_cpu_executor_hold(h, 0)  # the stuck job resumes and finds itself abandoned
    deadline = time.monotonic() + 10.0
    while L.ftmoe_cpu_executor_destroy(h, 0) != _lib.FTMOE_OK:  # refused while the pool is still inside the job
        assert time.monotonic() < deadline, "the abandoned job never left the pool"
        time.sleep(0.05)
    ops._KEPT_EXECUTORS.remove(h)
    assert (y == 7).all()  # the abandoned job wrote no row of y


@pytest.mark.parametrize("fmt", ["mxfp4", "fp8"])
@pytest.mark.parametrize("lim", [0.0, 7.0, 0.75])
def test_cpu_experts_swiglu_limit(executor, fmt, lim):
    """The clamped SwiGLU of the CPU pass (reference cpu_moe_ext.cpp:1769-1781)
    against the oracle: the bank's limit binds at 0.75 and hardly at 7."""
    rng = np.random.default_rng(91 + int(lim * 4))
    E, H, I, M, k = 6, 512, 256, 3, 4
    bank = synth.make_bank(fmt, E, H, I, rng)
    bank.swiglu_limit = lim
    x = synth.activations(rng, M, H)
    w, ids = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, None)
    y = executor.run(to_device_bank(bank, "cpu"), _host(x, np.float32).to(torch.bfloat16), _host(w, np.float32),
                     _host(ids, np.int32))
    g = y.float().numpy()
    assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (fmt, lim, max_rel(g, y_ref))
    with pytest.raises(ValueError, match="silu"):
        executor.run(to_device_bank(bank, "cpu") if lim > 0 else _limited(bank, "cpu"),
                     _host(x, np.float32).to(torch.bfloat16), _host(w, np.float32), _host(ids, np.int32),
                     activation="gelu")


def _limited(bank, dev):
    b = to_device_bank(bank, dev)
    b.swiglu_limit = 1.0
    return b
