"""bench.py's step planning (no GPU): the timed decode never runs past the
context, whatever --steps is, and the CPU baseline never asks the oracle for a
position at or beyond ctx, or for more steps than the GPU produced tokens."""
import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


@pytest.mark.parametrize("steps,want", [
    (1, [1]), (20, [20]), (255, [255]), (256, [256]), (257, [256, 1]), (600, [256, 256, 88])])
def test_decode_segments_stay_below_ctx(steps, want):
    segs = bench.decode_segments(steps)
    assert segs == want and sum(segs) == steps
    assert all(bench.N_PROMPT + s <= bench.CTX for s in segs)


@pytest.mark.parametrize("steps,warmup,want", [(20, 5, [20]), (256, 8, [248, 8]), (251, 5, [251])])
def test_decode_segments_after_warmup(steps, warmup, want):
    """Each timed run follows W untimed steps from the restored prompt state, so
    it starts at 3840 + W and still stays below ctx."""
    segs = bench.decode_segments(steps, start=bench.N_PROMPT + warmup)
    assert segs == want and sum(segs) == steps
    assert all(bench.N_PROMPT + warmup + s <= bench.CTX for s in segs)


def test_decode_segments_small_ctx():
    assert bench.decode_segments(10, start=60, ctx=64) == [4, 4, 2]
    with pytest.raises(ValueError):
        bench.decode_segments(0)
    with pytest.raises(ValueError):
        bench.decode_segments(5, start=64, ctx=64)


@pytest.mark.parametrize("max_steps,n_tok,start,ctx,want", [
    (128, 20, 3840, 4096, 20),     # the driver's --steps 20 run: bounded by the GPU tokens
    (128, 256, 3840, 4096, 128),   # bounded by max_steps
    (128, 256, 4076, 4096, 20),    # bounded by ctx (the failing case: prompt 4076)
    (128, 256, 4096, 4096, 0),
    (5, 3, 10, 12, 2)])
def test_cpu_decode_steps_bounds(max_steps, n_tok, start, ctx, want):
    n = bench.cpu_decode_steps(max_steps, n_tok, start, ctx)
    assert n == want
    assert start + n <= ctx  # the last oracle position is start + n - 1 < ctx


def test_workload_is_the_3840_plus_256_configuration():
    assert bench.N_PROMPT == 3840 and bench.DECODE_TOKENS == 256 and bench.CTX == 4096
    assert bench.N_PROMPT + bench.DECODE_TOKENS == bench.CTX


def test_affinity_cores_respects_omp(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "1")
    assert bench.affinity_cores() == 1
    monkeypatch.delenv("OMP_NUM_THREADS")
    assert bench.affinity_cores() == len(os.sched_getaffinity(0))


def test_oracle_refuses_position_at_ctx(oracle):
    """The oracle's own guard that the bench bound keeps clear of: a forward at
    position ctx is an error, never a silent result."""
    import lfm_hip
    from model_util import model_tensors, oracle_engine, small_hparams
    hp = small_hparams(kinds=("conv",), dense_lead=1)
    o = oracle_engine(oracle, hp, model_tensors(hp), ctx=8)
    o.forward([1], 7)
    with pytest.raises(ValueError):
        o.forward([1], 8)
    assert lfm_hip is not None
