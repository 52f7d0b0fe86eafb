"""lfm_argmax_noalloc (the entry point that allocates nothing: its state block
and partials live in a device array of the library's own code object) against
lfm_argmax (state and partials allocated per call), through the C ABI, on calls
in a row -- the second smaller than the first, so stale partials of the first
call sit in the shared scratch past the second call's range -- and against the
oracle's argmax (main.rs:112-141 semantics)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _vector(n, seed, ties=True):
    v = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
    v[::97] = np.nan
    if ties and n > 1000:
        m = np.float32(v[~np.isnan(v)].max() + 1.0)
        v[n // 3] = m
        v[2 * n // 3] = m  # tie: the lower index wins
    return v


def test_noalloc_argmax_matches_allocating_entry_point(gpu, oracle):
    cases = [(128003, 11), (4099, 12), (1, 13), (300000, 14), (65536, 15)]
    for n, seed in cases:
        v = _vector(n, seed)
        buf = gpu.DeviceBuffer.from_array(v)
        i_alloc, v_alloc = gpu.argmax_device(buf, n)
        i_none, v_none = gpu.argmax_device(buf, n, noalloc=True)
        print(f"n={n}: index {i_none} (allocating entry point {i_alloc})")
        assert i_none == i_alloc == oracle.argmax(v), (n, i_none, i_alloc)
        assert np.float32(v_none).view(np.uint32) == np.float32(v_alloc).view(np.uint32)
        # a second call on the same input gives the same answer from the shared scratch
        assert gpu.argmax_device(buf, n, noalloc=True) == (i_none, v_none)
        buf.free()


def test_noalloc_argmax_all_nan_and_errors(gpu):
    v = np.full(777, np.nan, dtype=np.float32)
    buf = gpu.DeviceBuffer.from_array(v)
    assert gpu.argmax_device(buf, 777, noalloc=True)[0] == gpu.argmax_device(buf, 777)[0] == 0
    with pytest.raises(gpu.LfmError) as e:
        gpu.argmax_device(buf, 0, noalloc=True)
    assert e.value.code == gpu.LFM_EINVAL
    buf.free()
