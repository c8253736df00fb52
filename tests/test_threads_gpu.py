"""Several host threads submitting to one executor at once: the slot pool
(src/executor/mod.rs:1-23: a submission checks out a free slot, waits on a
condvar when none is free) gives every thread its own stream and scratch,
so each result equals the same submission made alone, bit for bit.  The
mix covers the fused GEMM, a split-K op with an epilogue and a packed
decode GEMV (each with its own scratch use)."""

import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _jobs(ta, ex, oracle, idx):
    """Three submissions of thread `idx`, on tensors of its own."""
    s = 300 + 10 * idx
    out = []
    m, n, k = 256, 256, 1024
    a, b = ex.tensor_from(oracle.fill_det(m * k, s), shape=[m, k]), ex.tensor_from(oracle.fill_det(k * n, s + 1), shape=[k, n])
    bias, c = ex.tensor_from(oracle.fill_det(n, s + 2), shape=[n]), ex.tensor([m, n])
    out.append(([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_GELU))], c))
    m2, n2, k2 = 64, 256, 16384
    a2 = ex.tensor_from(oracle.fill_det(m2 * k2, s + 3), shape=[m2, k2])
    b2 = ex.tensor_from(oracle.fill_det(k2 * n2, s + 4), shape=[k2, n2])
    bias2, c2 = ex.tensor_from(oracle.fill_det(n2, s + 5), shape=[n2]), ex.tensor([m2, n2])
    out.append(([ta.MatmulOp(a2, b2, c2, epilogue=ta.Epilogue(bias=bias2, activation=ta.ACTIVATION_RELU))], c2))
    kk, nn = 2048, 1024
    w = oracle.fill_normal(kk * nn, s + 6, 0.02)
    tw = ex.tensor_from(ta.pack_f16w_row_tiles(w, kk, nn, ta.f16w_row_tile_n(kk, nn)), shape=[kk, nn], f16=True)
    tx, ty = ex.tensor_from(oracle.fill_det(kk, s + 7), shape=[1, kk]), ex.tensor([1, nn])
    out.append(([ta.MatmulOp(tx, tw, ty, packed_b=True)], ty))
    return out


@pytest.mark.parametrize("slots,threads", [(2, 4), (4, 4)])
def test_threads_share_one_executor(ta, ctx, oracle, slots, threads):
    ex = ta.Executor(ctx, n_slots=slots, max_calls_per_submit=8, tune=False)
    jobs = [_jobs(ta, ex, oracle, i) for i in range(threads)]
    # each submission alone first
    alone = []
    for per in jobs:
        res = []
        for ops, c in per:
            ex.run_ops(ops)
            res.append(ex.download(c).copy())
        alone.append(res)
    errors = []

    def worker(i):
        try:
            for _ in range(5):
                for ops, _c in jobs[i]:
                    ex.run_ops(ops)
        except Exception as e:  # reported below
            errors.append(repr(e))

    print(f"threads {threads} on {slots} slots", flush=True)
    ts = [threading.Thread(target=worker, args=(i,)) for i in range(threads)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in ts), "a submitting thread did not finish"
    assert not errors, errors
    for per, res in zip(jobs, alone):
        for (ops, c), want in zip(per, res):
            np.testing.assert_array_equal(ex.download(c), want)
