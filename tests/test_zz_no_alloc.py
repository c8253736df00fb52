"""The allocation-free split-K entry point (ta_matmul_split_k2_noalloc,
which has no reference counterpart) against ta_matmul_split_k2 through the
C ABI: the same kernels, so results must be bit-identical.  Two calls in a
row, the second on a smaller problem, so the fixed scratch still holds the
first call's planes when the second runs."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run_pair(ta, ex, oracle, m, n, k, splits, seed, alpha=1.0, batch=1):
    ha = oracle.fill_det(batch * m * k, seed)
    hb = oracle.fill_det(k * n, seed + 1)
    a_shape = [batch, m, k] if batch > 1 else [m, k]
    c_shape = [batch, m, n] if batch > 1 else [m, n]
    a, b = ex.tensor_from(ha, shape=a_shape), ex.tensor_from(hb, shape=[k, n])
    c_ref, c_fix = ex.tensor(c_shape), ex.tensor(c_shape)
    print(f"noalloc split-K B={batch} {m}x{n}x{k} splits={splits}", flush=True)
    st_ref = ex.run_matmuls_split_k2(a, b, c_ref, splits, alpha)
    st_fix = ex.run_matmuls_split_k2_noalloc(a, b, c_fix, splits, alpha)
    assert st_fix.total_flops == st_ref.total_flops == 2 * batch * m * n * k
    got, ref = ex.download(c_fix), ex.download(c_ref)
    np.testing.assert_array_equal(got, ref)
    return got, ha, hb


@pytest.mark.parametrize("first,second", [
    ((64, 256, 65536, 16), (32, 128, 131072, 8)),   # config 4, large then small planes
    ((101, 103, 4000, 7), (33, 65, 999, 5)),         # ragged tiles and windows
])
def test_noalloc_matches_split_k2_twice(ta, ex, oracle, first, second):
    m, n, k, s = first
    got, ha, hb = _run_pair(ta, ex, oracle, m, n, k, s, 71)
    ref = oracle.cpu_bmm(ha, hb, None, 1, m, n, k)
    err, _ = oracle.max_abs_err(got.reshape(-1), ref)
    assert err <= oracle.tolerance(k) * 2 + 1e-4
    m, n, k, s = second
    _run_pair(ta, ex, oracle, m, n, k, s, 73, alpha=0.5)


def test_noalloc_batched_and_default_splits(ta, ex, oracle):
    _run_pair(ta, ex, oracle, 48, 80, 3000, 0, 81, batch=3)   # splits 0 = default
    _run_pair(ta, ex, oracle, 40, 72, 2048, 4, 83, batch=2)


def test_noalloc_single_split_matches_split_k2(ta, ex, oracle):
    """splits == 1 takes the data-parallel route in both entry points, so
    the bits agree; also against the oracle."""
    m, n, k = 96, 160, 1024
    got, ha, hb = _run_pair(ta, ex, oracle, m, n, k, 1, 91)
    err, _ = oracle.max_abs_err(got.reshape(-1), oracle.cpu_bmm(ha, hb, None, 1, m, n, k))
    assert err <= oracle.tolerance(k) * 2 + 1e-4


def test_noalloc_first_call_allocates_nothing(ta, ctx, oracle):
    """On a fresh executor whose slots hold no scratch yet, the call makes
    no device or pinned allocation (the library counts every one), then
    agrees bit for bit with the allocating entry point."""
    fresh = ta.Executor(ctx, n_slots=1, max_calls_per_submit=8, tune=False)
    m, n, k, s = 64, 256, 65536, 32     # config 4a: the largest plane set that fits
    ha, hb = oracle.fill_det(m * k, 95), oracle.fill_det(k * n, 96)
    a, b = fresh.tensor_from(ha, shape=[m, k]), fresh.tensor_from(hb, shape=[k, n])
    c_fix, c_ref = fresh.tensor([m, n]), fresh.tensor([m, n])
    print(f"noalloc fresh executor {m}x{n}x{k} splits={s}", flush=True)
    before = ta.allocation_count()
    fresh.run_matmuls_split_k2_noalloc(a, b, c_fix, s)
    fresh.run_matmuls_split_k2_noalloc(a, b, c_fix, s)
    assert ta.allocation_count() == before
    fresh.run_matmuls_split_k2(a, b, c_ref, s)
    assert ta.allocation_count() > before    # the allocating form grows the slot scratch
    np.testing.assert_array_equal(fresh.download(c_fix), fresh.download(c_ref))


def test_noalloc_rejects_planes_beyond_capacity(ta, ex, oracle):
    m = n = 1024
    k = 8192
    a, b, c = ex.tensor([m, k]), ex.tensor([k, n]), ex.tensor([m, n])
    with pytest.raises(RuntimeError, match="fixed scratch"):
        ex.run_matmuls_split_k2_noalloc(a, b, c, 16)
    # the existing entry point still takes it (it allocates)
    ex.run_matmuls_split_k2(a, b, c, 16)
