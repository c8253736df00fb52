"""GPU parity of the deterministic split-K route for ops with a fused
epilogue (bias, activation, binary with D, accumulate).

Stage 1 writes alpha-scaled partial planes; the reduce sums them in a fixed
order and then applies the epilogue once, in the order of
shaders/matmul_epilogue_common.glsl:14-21.  The reference splits plain
calls only (src/executor/mod.rs:179-210); the reduce's plane order follows
shaders/matmul_f32_splitk2_reduce.comp:44-75.

Bar: the f32 tolerances of test_gemm_gpu against the oracle's cpu_bmm plus
the f64 epilogue on the same inputs, and bit-identical output over 10 runs
at S = 8 / 16 / 32.
"""

import functools
import os

import numpy as np
import pytest

from test_gemm_gpu import check_f32

pytestmark = pytest.mark.gpu

# (name, bias kind, activation, binary, beta, accumulate)
EPILOGUES = {
    "bias_gelu": ("n", 3, 0, 0.0, False),
    "silu_mul_d": (None, 2, 2, 0.0, False),
    "bias_bn_add_scaled_d": ("bn", 0, 1, 0.75, False),
    "bias_relu_accumulate": ("n", 1, 0, 0.0, True),
}


@functools.lru_cache(maxsize=None)
def _inputs(oracle, batch, m, n, k, seed):
    ha = oracle.fill_det(batch * m * k, seed)
    hb = oracle.fill_det(k * n, seed + 1)
    return ha, hb


@functools.lru_cache(maxsize=None)
def _raw_product(oracle, batch, m, n, k, seed, alpha):
    ha, hb = _inputs(oracle, batch, m, n, k, seed)
    return oracle.cpu_bmm(ha, hb, None, batch, m, n, k, alpha)


def _case(ta, ex, oracle, batch, m, n, k, name, alpha=1.0, seed=81):
    bias_kind, act, binary, beta, acc = EPILOGUES[name]
    ha, hb = _inputs(oracle, batch, m, n, k, seed)
    sa = [batch, m, k] if batch > 1 else [m, k]
    sc = [batch, m, n] if batch > 1 else [m, n]
    a, b, c = ex.tensor_from(ha, shape=sa), ex.tensor_from(hb, shape=[k, n]), ex.tensor(sc)
    hbias = bias = hd = d = hc0 = None
    stride = 0
    if bias_kind == "n":
        hbias = oracle.fill_det(n, seed + 2)
        bias = ex.tensor_from(hbias, shape=[n])
    elif bias_kind == "bn":
        hbias = oracle.fill_det(batch * n, seed + 2)
        bias = ex.tensor_from(hbias, shape=[batch, n])
        stride = n
    if binary:
        hd = oracle.fill_det(batch * m * n, seed + 3)
        d = ex.tensor_from(hd, shape=sc)
    if acc:
        hc0 = oracle.fill_det(batch * m * n, seed + 4)
    op = ta.MatmulOp(a, b, c, alpha=alpha, accumulate=acc,
                     epilogue=ta.Epilogue(bias=bias, activation=act, binary=binary, d=d, beta=beta))
    # cpu_bmm, then (+C_old) and the f64 epilogue: accumulate adds C_old
    # after alpha, before the bias (matmul_epilogue_common.glsl:14-21).
    raw = _raw_product(oracle, batch, m, n, k, seed, alpha)
    if acc:
        raw = (raw.astype(np.float64) + hc0.astype(np.float64)).astype(np.float32)
    ref = oracle.epilogue(raw, n, m * n, hbias, stride, act, binary, hd, beta)

    def reset():
        if acc:
            ex.upload(c, hc0)

    return op, c, ref, reset


@pytest.mark.parametrize("name", list(EPILOGUES))
@pytest.mark.parametrize("splits", [8, 16, 32])
def test_splitk_epilogue_deterministic(ta, ex, oracle, name, splits):
    """256x256x16384 (the deep-K skinny shape of the bench's run_ops
    section) through explicit split counts: within tolerance of the oracle
    and bit-identical over 10 runs."""
    m = n = 256
    k = 16384
    op, c, ref, reset = _case(ta, ex, oracle, 1, m, n, k, name)
    reset()
    st = ex.run_op_split_k2(op, splits)
    assert st.total_flops == 2 * m * n * k
    first = ex.download(c).copy()
    check_f32(first, ref, k, oracle)
    for _ in range(9):
        reset()
        ex.run_op_split_k2(op, splits)
        np.testing.assert_array_equal(ex.download(c), first)


@pytest.mark.parametrize("name", list(EPILOGUES))
def test_run_ops_routes_fused_deep_k_through_splitk(ta, ex, oracle, name):
    """run_ops takes the split-K route by itself for a fused deep-K op whose
    tiles leave most CUs idle, and gives the bits of run_op_split_k2 at the
    planner's split count."""
    m = n = 256
    k = 16384
    info = ex.dispatch_info_for(1, m, n, k)
    assert info["split_k2"] is not None and info["split_k2"] >= 2, info
    op, c, ref, reset = _case(ta, ex, oracle, 1, m, n, k, name)
    reset()
    ex.run_ops([op])
    got = ex.download(c).copy()
    check_f32(got, ref, k, oracle)
    reset()
    ex.run_op_split_k2(op, info["split_k2"])
    np.testing.assert_array_equal(ex.download(c), got)


@pytest.mark.parametrize("batch,m,n,k,splits,name,alpha", [
    (3, 33, 65, 4000, 5, "bias_bn_add_scaled_d", 0.25),   # ragged: the generic stage-1 kernel
    (2, 64, 256, 16384, 4, "bias_gelu", 0.5),             # 64x64 stage-1 tiles, batched
    (1, 101, 103, 999, 7, "silu_mul_d", 1.0),             # odd N: quads cross rows in the reduce
    (1, 64, 256, 65536, 16, "bias_relu_accumulate", 1.0),  # config 4a shape with an epilogue
])
def test_splitk_epilogue_shapes(ta, ex, oracle, batch, m, n, k, splits, name, alpha):
    op, c, ref, reset = _case(ta, ex, oracle, batch, m, n, k, name, alpha)
    reset()
    ex.run_op_split_k2(op, splits)
    check_f32(ex.download(c), ref, k, oracle)


def test_splitk_epilogue_single_split_is_data_parallel(ta, ex, oracle):
    """splits == 1 runs the data-parallel route with the epilogue in the
    GEMM kernel itself."""
    m, n, k = 128, 256, 4096
    op, c, ref, reset = _case(ta, ex, oracle, 1, m, n, k, "bias_gelu")
    ex.run_op_split_k2(op, 1)
    check_f32(ex.download(c), ref, k, oracle)


def test_run_op_split_k2_rejects_f16_and_fusions(ta, ex):
    a, c = ex.tensor([4, 64]), ex.tensor([4, 8])
    b16 = ex.tensor([64, 8], f16=True)
    with pytest.raises(ta.TensorAshError, match="f32 A and B only"):
        ex.run_op_split_k2(ta.MatmulOp(a, b16, c), 2)
    b = ex.tensor([64, 8])
    with pytest.raises(ta.TensorAshError, match="exceeds K=64"):
        ex.run_op_split_k2(ta.MatmulOp(a, b, c), 65)


def test_splitk_fused_ops_in_graph_and_lanes(ta, ex, oracle):
    """Fused deep-K ops on the split-K route inside one submission: two
    independent ops in run_ops (one stream lane each or in order) give the
    bits of the ops run alone, and in run_op_graph a later op reads the
    first op's finished (reduced, epilogued) output as its A."""
    m, n, k = 256, 256, 16384
    op1, c1, ref1, _ = _case(ta, ex, oracle, 1, m, n, k, "bias_gelu", seed=91)
    op2, c2, ref2, _ = _case(ta, ex, oracle, 1, m, n, k, "silu_mul_d", seed=93)
    ex.run_ops([op1])
    alone1 = ex.download(c1).copy()
    ex.run_ops([op2])
    alone2 = ex.download(c2).copy()
    check_f32(alone1, ref1, k, oracle)
    check_f32(alone2, ref2, k, oracle)
    for lanes in ("1", "2"):
        os.environ["TA_RUN_OPS_LANES"] = lanes
        try:
            ex.run_ops([op1, op2])
        finally:
            del os.environ["TA_RUN_OPS_LANES"]
        np.testing.assert_array_equal(ex.download(c1), alone1)
        np.testing.assert_array_equal(ex.download(c2), alone2)
    # dependent graph: C3 = C1 @ B3 (256 x 64 x 256), reading op1's output
    hb3 = oracle.fill_det(n * 64, 95)
    b3, c3 = ex.tensor_from(hb3, shape=[n, 64]), ex.tensor([m, 64])
    ex.run_op_graph([op1, ta.MatmulOp(c1, b3, c3)])
    np.testing.assert_array_equal(ex.download(c1), alone1)
    # A = C1 is not unit-scaled (|C1| up to ~70), so the bound scales with max|A|
    got3, ref3 = ex.download(c3).reshape(-1), oracle.cpu_bmm(alone1, hb3, None, 1, m, 64, n)
    err, idx = oracle.max_abs_err(got3, ref3)
    assert err <= oracle.tolerance(n) * float(np.max(np.abs(alone1))), f"abs err {err} at {idx}"


def _rand_cases():
    """Seeded mixed shapes: ragged and aligned tiles, batched A or B, every
    epilogue, explicit split counts (the generic and the pipelined stage-1
    kernels both appear)."""
    rng = np.random.default_rng(123)
    names = list(EPILOGUES)
    out = []
    for i in range(12):
        m = int(rng.choice([17, 32, 64, 96, 128, 192]))
        n = int(rng.choice([8, 33, 64, 128, 256]))
        k = int(rng.choice([512, 1000, 2048, 4096, 6144]))
        splits = int(rng.choice([2, 3, 4, 8, 16]))
        batch = int(rng.choice([1, 1, 2]))
        b_batched = batch > 1 and bool(rng.integers(0, 2))
        out.append((i, batch, b_batched, m, n, k, splits, names[i % len(names)]))
    return out


@pytest.mark.parametrize("i,batch,b_batched,m,n,k,splits,name", _rand_cases())
def test_splitk_epilogue_mixed_shapes(ta, ex, oracle, i, batch, b_batched, m, n, k, splits, name):
    bias_kind, act, binary, beta, acc = EPILOGUES[name]
    seed = 200 + 7 * i
    ha = oracle.fill_det(batch * m * k, seed)
    nb = batch if b_batched else 1
    hb = oracle.fill_det(nb * k * n, seed + 1)
    sa = [batch, m, k] if batch > 1 else [m, k]
    sb = [nb, k, n] if nb > 1 else [k, n]
    sc = [batch, m, n] if batch > 1 else [m, n]
    a, b, c = ex.tensor_from(ha, shape=sa), ex.tensor_from(hb, shape=sb), ex.tensor(sc)
    hbias = bias = hd = d = None
    stride = 0
    if bias_kind == "n":
        hbias = oracle.fill_det(n, seed + 2)
        bias = ex.tensor_from(hbias, shape=[n])
    elif bias_kind == "bn":
        hbias = oracle.fill_det(batch * n, seed + 2)
        bias = ex.tensor_from(hbias, shape=[batch, n] if batch > 1 else [n])
        stride = n if batch > 1 else 0
    if binary:
        hd = oracle.fill_det(batch * m * n, seed + 3)
        d = ex.tensor_from(hd, shape=sc)
    hc0 = oracle.fill_det(batch * m * n, seed + 4) if acc else None
    if acc:
        ex.upload(c, hc0)
    op = ta.MatmulOp(a, b, c, accumulate=acc,
                     epilogue=ta.Epilogue(bias=bias, activation=act, binary=binary, d=d, beta=beta))
    print(f"fused split-K case {i}: B={batch} (B batched {b_batched}) {m}x{n}x{k} S={splits} {name}",
          flush=True)
    ex.run_op_split_k2(op, min(splits, k))
    if b_batched:
        raw = np.concatenate([oracle.cpu_bmm(ha[j * m * k:(j + 1) * m * k], hb[j * k * n:(j + 1) * k * n],
                                             None, 1, m, n, k) for j in range(batch)])
    else:
        raw = oracle.cpu_bmm(ha, hb, None, batch, m, n, k)
    if acc:
        raw = (raw.astype(np.float64) + hc0.astype(np.float64)).astype(np.float32)
    ref = oracle.epilogue(raw, n, m * n, hbias, stride, act, binary, hd, beta)
    check_f32(ex.download(c), ref, k, oracle)
