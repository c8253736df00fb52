"""GPU parity of the FP32-MFMA fused-epilogue GEMM against the CPU oracle.

Mirrors the reference's tests/correctness/{epilogue,shapes,batch,property,
kernels,f16}.rs: same seeds style (fill_det), same tolerance family.

Tolerances (written here, checked on every case):
  * abs:  max |gpu - ref| <= 2 * tolerance(K) + 1e-4, tolerance(K) = 8*K*eps
          (tests/correctness/epilogue.rs:49-54; plain GEMMs use tolerance(K))
  * rel:  max |gpu - ref| / max |ref| <= 1e-5 * sqrt(K)   (BASELINE north star)
"""

import math

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def check_f32(got, ref, k, oracle, epi=True):
    got = np.asarray(got, dtype=np.float32).reshape(-1)
    ref = np.asarray(ref, dtype=np.float32).reshape(-1)
    err, idx = oracle.max_abs_err(got, ref)
    tol = 2 * oracle.tolerance(k) + 1e-4 if epi else oracle.tolerance(k)
    assert err <= tol, f"abs err {err} at {idx} (gpu {got[idx]} ref {ref[idx]}) > {tol}"
    r = rel_err(got, ref)
    assert r <= 1e-5 * math.sqrt(k), f"rel err {r} > {1e-5 * math.sqrt(k)}"


def run_case(ta, ex, oracle, m, n, k, batch_a=1, batch_b=1, batch_c=1, alpha=1.0, accumulate=False,
             bias=None, act=0, binary=0, beta=0.0, seed=71, kernel_ex=None):
    e = kernel_ex or ex
    sa = [m, k] if batch_a == 1 and batch_c == 1 else [batch_a, m, k]
    sb = [k, n] if batch_b == 1 and batch_c == 1 else [batch_b, k, n]
    sc = [m, n] if batch_c == 1 else [batch_c, m, n]
    ha = oracle.fill_det(int(np.prod(sa)), seed)
    hb = oracle.fill_det(int(np.prod(sb)), seed + 1)
    a, b = e.tensor_from(ha, shape=sa), e.tensor_from(hb, shape=sb)
    c = e.tensor(sc)
    hc0 = None
    if accumulate:
        hc0 = oracle.fill_det(int(np.prod(sc)), seed + 2)
        e.upload(c, hc0)
    epi = ta.Epilogue(activation=act, binary=binary, beta=beta)
    hbias = None
    bias_stride = 0
    if bias is not None:
        hbias = oracle.fill_det(int(np.prod(bias)), seed + 3)
        epi.bias = e.tensor_from(hbias, shape=bias)
        bias_stride = n if len(bias) == 2 else 0
    hd = None
    if binary:
        hd = oracle.fill_det(int(np.prod(sc)), seed + 4)
        epi.d = e.tensor_from(hd, shape=sc)
    st = e.run_ops([ta.MatmulOp(a, b, c, alpha, accumulate, epi)])
    assert st.n_calls == 1 and st.total_flops == 2 * batch_c * m * n * k
    got = e.download(c)
    ref = oracle.reference_gemm(ha, hb, batch_c, m, n, k, alpha, hc0, accumulate, hbias,
                                bias_stride, act, binary, hd, beta)
    check_f32(got, ref, k, oracle)
    return st


def test_c_smoke_values(ta, ex):
    """examples/c_smoke.c:60-104: [58,64,139,154], then bias -58.5 + SiLU."""
    a = ex.tensor_from(np.array([1, 2, 3, 4, 5, 6], np.float32), shape=[2, 3])
    b = ex.tensor_from(np.array([7, 8, 9, 10, 11, 12], np.float32), shape=[3, 2])
    c = ex.tensor([2, 2])
    st = ex.matmul(a, b, c)
    np.testing.assert_allclose(ex.download(c).reshape(-1), [58, 64, 139, 154], atol=1e-4)
    assert st.has_gpu_time == 1 and st.total_flops == 24
    bias = ex.tensor_from(np.array([-58.5, 0.0], np.float32), shape=[2])
    ex.run_ops([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_SILU))])
    out = ex.download(c).reshape(-1)
    x = -0.5
    assert abs(out[0] - x / (1 + math.exp(-x))) < 1e-3
    assert abs(out[1] - 64 * (1 / (1 + math.exp(-64)))) < 1e-2


def test_config1_512_bias_relu(ta, ex, oracle):
    """512^3, bias[N] + ReLU, fill_det seeds 1, 2, 3."""
    m = n = k = 512
    ha, hb, hbias = oracle.fill_det(m * k, 1), oracle.fill_det(k * n, 2), oracle.fill_det(n, 3)
    a, b = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n])
    bias, c = ex.tensor_from(hbias, shape=[n]), ex.tensor([m, n])
    ex.run_ops([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_RELU))])
    ref = oracle.reference_gemm(ha, hb, 1, m, n, k, bias=hbias, act=1)
    check_f32(ex.download(c), ref, k, oracle)


@pytest.mark.parametrize("shape", [(512, 512, 512), (67, 45, 33), (130, 257, 129), (300, 520, 1000)])
@pytest.mark.parametrize("epi", [
    dict(bias=True), dict(act=1), dict(act=2, bias=True), dict(act=3, binary=1, beta=0.5),
    dict(binary=2), dict(alpha=0.25, accumulate=True, act=3), dict(bias=True, act=2, binary=2),
])
def test_epilogues(ta, ex, oracle, shape, epi):
    m, n, k = shape
    epi = dict(epi)
    bias = [n] if epi.pop("bias", False) else None
    run_case(ta, ex, oracle, m, n, k, bias=bias, **epi)


@pytest.mark.parametrize("ba,bb,bc", [(3, 1, 3), (1, 3, 3), (1, 1, 3), (3, 3, 3)])
def test_batch_broadcast(ta, ex, oracle, ba, bb, bc):
    run_case(ta, ex, oracle, 70, 90, 50, batch_a=ba, batch_b=bb, batch_c=bc, bias=[bc, 90], act=1)


@pytest.mark.parametrize("shape", [(1, 1, 1), (1, 7, 3), (5, 1, 9), (3, 4, 1), (17, 19, 23),
                                   (64, 64, 64), (65, 63, 17), (255, 257, 31), (256, 256, 16)])
def test_ragged_shapes(ta, ex, oracle, shape):
    run_case(ta, ex, oracle, *shape)


def test_property_random_shapes(ta, ex, oracle):
    """tests/correctness/property.rs:5-63: 32 random shapes from LcgRng(0xC0FFEE)."""
    dims = oracle.lcg_range(0xC0FFEE, 1, 300, 32 * 3).reshape(32, 3)
    for m, n, k in dims:
        run_case(ta, ex, oracle, int(m), int(n), int(k), seed=int(m) + 7)


def gemm_kernels(ta):
    return [n for n in ta.kernel_names() if n.startswith("f32_m")]


@pytest.mark.parametrize("shape", [(300, 200, 77), (512, 256, 128), (37, 41, 1088)])
def test_every_f32_kernel(ta, ctx, oracle, shape):
    """tests/correctness/kernels.rs:7-76: every registry GEMM agrees with the oracle."""
    for name in gemm_kernels(ta):
        kex = ta.Executor(ctx, kernel_selection=name, tune=False)
        run_case(ta, kex, oracle, *shape, bias=[shape[1]], act=3, kernel_ex=kex)
        kex.close()


@pytest.mark.parametrize("shape", [(32, 384, 256), (40, 130, 70)])
def test_f16w_gemm(ta, ctx, ex, oracle, shape):
    """f16 B widened exactly: parity against cpu_bmm on the f16-rounded B (f16.rs:65-122)."""
    m, n, k = shape
    ha, hb = oracle.fill_det(m * k, 81), oracle.fill_det(k * n, 82)
    hbr = oracle.round_via_f16(hb)
    import re
    for name in [None] + [n_ for n_ in ta.kernel_names() if re.match(r"f16w_m\d", n_)]:
        kex = ex if name is None else ta.Executor(ctx, kernel_selection=name, tune=False)
        a = kex.tensor_from(ha, shape=[m, k])
        b = kex.tensor_from(hb, shape=[k, n], f16=True)
        c = kex.tensor([m, n])
        kex.matmul(a, b, c)
        check_f32(kex.download(c), oracle.cpu_bmm(ha, hbr, None, 1, m, n, k), k, oracle)


def test_4096_cube_full(ta, ex, oracle):
    """Headline 4096^3 bias + ReLU checked on every output element against
    the oracle's multi-threaded cpu_bmm (rows split over the host's cores,
    bit-identical to the serial oracle) and its f64 epilogue."""
    m = n = k = 4096
    ha, hb, hbias = oracle.fill_det(m * k, 31), oracle.fill_det(k * n, 32), oracle.fill_det(n, 33)
    a, b = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n])
    bias, c = ex.tensor_from(hbias, shape=[n]), ex.tensor([m, n])
    print("4096^3 full-output parity: GPU run, then the oracle on all rows", flush=True)
    ex.run_ops([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_RELU))])
    got = ex.download(c).reshape(-1)
    raw = np.empty(m * n, np.float32)
    oracle.cpu_bmm_rows(ha, hb, 1, m, n, k, 1.0, raw, 0, m, min(16, oracle.max_threads()))
    check_f32(got, oracle.epilogue(raw, n, m * n, hbias, 0, 1), k, oracle)


def test_config2_batched_gelu_full(ta, ex, oracle):
    """BASELINE config 2a on every output element (B=8, 2048^3, bias[8,N],
    GELU; A ~ N(0,1), B ~ N(0, 1/sqrt(K)))."""
    bt, m, n, k = 8, 2048, 2048, 2048
    ha = oracle.fill_normal(bt * m * k, 21, 1.0)
    hb = oracle.fill_normal(k * n, 22, 1.0 / math.sqrt(k))
    hbias = oracle.fill_det(bt * n, 23)
    a, b = ex.tensor_from(ha, shape=[bt, m, k]), ex.tensor_from(hb, shape=[k, n])
    bias, c = ex.tensor_from(hbias, shape=[bt, n]), ex.tensor([bt, m, n])
    print("8x2048^3 full-output parity", flush=True)
    ex.run_ops([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_GELU))])
    got = ex.download(c).reshape(-1)
    raw = np.empty(bt * m * n, np.float32)
    oracle.cpu_bmm_rows(ha, hb, bt, m, n, k, 1.0, raw, 0, bt * m, min(16, oracle.max_threads()))
    check_f32(got, oracle.epilogue(raw, n, m * n, hbias, n, 3), k, oracle)


def f16_mfma_refs(ha, hb, batch, m, n, k, oracle, alpha=1.0, c0=None, acc=False, **epi):
    """f16-MFMA route: A is rounded to f16 at staging (like the reference's
    coopmat route, tests/correctness/f16.rs:776-817), so the oracle on the
    dual-rounded inputs is exact up to accumulation order (f32 tolerance),
    and the oracle on the unrounded A is within 2e-3."""
    har, hbr = oracle.round_via_f16(ha), oracle.round_via_f16(hb)
    return (oracle.reference_gemm(har, hbr, batch, m, n, k, alpha, c0, acc, **epi),
            oracle.reference_gemm(ha, hbr, batch, m, n, k, alpha, c0, acc, **epi))


def check_f16_mfma(got, refs, k, oracle):
    check_f32(got, refs[0], k, oracle)
    assert rel_err(got, refs[1]) <= 2e-3


@pytest.mark.parametrize("shape", [(512, 2560, 2048), (512, 2048, 5632), (128, 128, 64), (200, 300, 100),
                                   (65, 70, 33)])
def test_f16_mfma_gemm(ta, ctx, ex, oracle, shape):
    m, n, k = shape
    ha, hb = oracle.fill_det(m * k, 91), oracle.fill_normal(k * n, 92, 0.02)
    hbias = oracle.fill_det(n, 93)
    refs = f16_mfma_refs(ha, hb, 1, m, n, k, oracle, bias=hbias, act=2)
    names = [n_ for n_ in ta.kernel_names() if n_.startswith("f16w_mfma")] if m * n * k <= 1 << 24 else []
    if k % 64 or n % 8:  # the 256x256 tile exists only as a pipelined kernel
        names = [n_ for n_ in names if "m256n256" not in n_]
    for name in [None] + names:
        kex = ex if name is None else ta.Executor(ctx, kernel_selection=name, tune=False)
        if name is None:
            routed = kex.dispatch_info_for(1, m, n, k, True)["kernel"]
            assert "mfma" in routed or "_sk_" in routed, routed
        a = kex.tensor_from(ha, shape=[m, k])
        b = kex.tensor_from(hb, shape=[k, n], f16=True)
        bias, c = kex.tensor_from(hbias, shape=[n]), kex.tensor([m, n])
        kex.run_ops([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_SILU))])
        check_f16_mfma(kex.download(c), refs, k, oracle)


@pytest.mark.parametrize("name", ["f16w_mfma_m64n64", "f16w_mfma_m128n64", "f16w_mfma_m64n128",
                                  "f16w_mfma_m128n128", "f16w_mfma_m256n256"])
@pytest.mark.parametrize("epi", ["bias_bn_gelu", "add_scaled", "mul", "broadcast_a"])
def test_f16_mfma_pipelined_epilogues(ta, ctx, oracle, name, epi):
    """Pipelined f16-MFMA kernels (K % 64 == 0, N % 8 == 0): ragged M and N
    tiles, batched [B, N] bias, both binaries and a broadcast A plane (its
    f16 copy is one plane)."""
    kex = ta.Executor(ctx, kernel_selection=name, tune=False)
    bt, m, n, k = 2, 300, 264, 192
    ha = oracle.fill_det((1 if epi == "broadcast_a" else bt) * m * k, 7100)
    hb = oracle.fill_normal(bt * k * n, 7101, 0.05)
    hbias, hd = oracle.fill_det(bt * n, 7102), oracle.fill_det(bt * m * n, 7103)
    a = kex.tensor_from(ha, shape=[m, k] if epi == "broadcast_a" else [bt, m, k])
    b = kex.tensor_from(hb, shape=[bt, k, n], f16=True)
    c = kex.tensor([bt, m, n])
    d = kex.tensor_from(hd, shape=[bt, m, n])
    if epi == "bias_bn_gelu":
        e, kw = ta.Epilogue(bias=kex.tensor_from(hbias, shape=[bt, n]), activation=ta.ACTIVATION_GELU), \
            dict(bias=hbias, bias_batch_stride=n, act=3)
    elif epi == "add_scaled":
        e, kw = ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=d, beta=-0.5), dict(binary=1, d=hd, beta=-0.5)
    else:
        e, kw = ta.Epilogue(binary=ta.BINARY_MUL, d=d), dict(binary=2, d=hd)
    kex.run_ops([ta.MatmulOp(a, b, c, epilogue=e, alpha=1.25)])
    ha_full = np.tile(ha, bt) if epi == "broadcast_a" else ha
    refs = f16_mfma_refs(ha_full, hb, bt, m, n, k, oracle, alpha=1.25, **kw)
    check_f16_mfma(kex.download(c), refs, k, oracle)


@pytest.mark.parametrize("name", [None, "f16w_mfma_m128n128", "f16w_mfma_m128n64", "f16w_mfma_m64n128",
                                  "f16w_mfma_m64n64"])
@pytest.mark.parametrize("bt,m,n,k", [(1, 300, 264, 192), (2, 128, 256, 128), (1, 512, 5632, 2048)])
def test_f16w_dual_swiglu_pair(ta, ctx, ex, oracle, monkeypatch, name, bt, m, n, k):
    """A SwiGLU pair in an op graph, up = alpha * x @ Wu then
    h = SiLU(alpha * x @ Wg + bias) * up, runs as one dual launch on the
    pipelined f16w route (ta_gemm_h16dual_*: x read once for both weight
    matrices), which also leaves an f16 copy of h for the down-projection
    that follows.  All outputs must equal the unfused ops' bits (same K
    order per element, same rounding of h), and match the oracle (h on the
    GPU's own up)."""
    if name is not None and m * n * k > 1 << 26:
        pytest.skip("forced tiles on the small shapes only")
    kex = ex if name is None else ta.Executor(ctx, kernel_selection=name, tune=False)
    hx = oracle.fill_det(bt * m * k, 7400)
    hwu, hwg = oracle.fill_normal(k * n, 7401, 0.05), oracle.fill_normal(k * n, 7402, 0.05)
    hbias = oracle.fill_det(n, 7403)
    x = kex.tensor_from(hx, shape=[bt, m, k])
    wu, wg = kex.tensor_from(hwu, shape=[k, n], f16=True), kex.tensor_from(hwg, shape=[k, n], f16=True)
    bias = kex.tensor_from(hbias, shape=[n])
    up, h, up2, h2 = (kex.tensor([bt, m, n]) for _ in range(4))
    # down-projection reading h as A: takes the dual launch's f16 copy of h
    # instead of converting h (same RNE rounding of the same values)
    k2 = 2048 if n == 5632 else 128
    wd = kex.tensor_from(oracle.fill_normal(n * k2, 7404, 0.05), shape=[n, k2], f16=True)
    res = kex.tensor_from(oracle.fill_det(bt * m * k2, 7405), shape=[bt, m, k2])
    y, y2 = kex.tensor([bt, m, k2]), kex.tensor([bt, m, k2])
    pair = lambda u, g, yy: [ta.MatmulOp(x, wu, u, alpha=1.25),
                             ta.MatmulOp(x, wg, g, alpha=1.25, epilogue=ta.Epilogue(
                                 bias=bias, activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=u)),
                             ta.MatmulOp(g, wd, yy, epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=res,
                                                                         beta=1.0))]
    kex.run_op_graph(pair(up, h, y))
    monkeypatch.setenv("TA_NO_FUSE", "1")
    kex.run_op_graph(pair(up2, h2, y2))
    monkeypatch.delenv("TA_NO_FUSE")
    got_up, got_h = kex.download(up), kex.download(h)
    np.testing.assert_array_equal(got_up, kex.download(up2))
    np.testing.assert_array_equal(got_h, kex.download(h2))
    np.testing.assert_array_equal(kex.download(y), kex.download(y2))
    if m * n * k <= 1 << 26:  # the full config-5 shape: bits against the unfused ops only
        _dual_oracle_check(oracle, hx, hwu, hwg, hbias, got_up, got_h, bt, m, n, k)
    # the fused launch repeats its bits
    got_y = kex.download(y)
    kex.run_op_graph(pair(up, h, y))
    np.testing.assert_array_equal(kex.download(h), got_h)
    np.testing.assert_array_equal(kex.download(y), got_y)


def test_f16w_dual_swiglu_prepared_graph_replays(ta, ex, oracle):
    """The prefill SwiGLU triple (dual up/gate launch leaving h's f16 copy,
    down reading it) captured as one hipGraph and replayed five times, with
    the outputs cleared and eager work between replays: every replay equals
    the eager run."""
    m, hid, ffn = 512, 512, 1408
    x = ex.tensor_from(oracle.fill_det(m * hid, 7501), shape=[m, hid])
    wu = ex.tensor_from(oracle.fill_normal(hid * ffn, 7502, 0.05), shape=[hid, ffn], f16=True)
    wg = ex.tensor_from(oracle.fill_normal(hid * ffn, 7503, 0.05), shape=[hid, ffn], f16=True)
    wd = ex.tensor_from(oracle.fill_normal(ffn * hid, 7504, 0.05), shape=[ffn, hid], f16=True)
    res = ex.tensor_from(oracle.fill_det(m * hid, 7505), shape=[m, hid])
    up, h, y = ex.tensor([m, ffn]), ex.tensor([m, ffn]), ex.tensor([m, hid])
    ops = [ta.MatmulOp(x, wu, up),
           ta.MatmulOp(x, wg, h, epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up)),
           ta.MatmulOp(h, wd, y, epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=res, beta=1.0))]
    ex.run_op_graph(ops)
    eager = [ex.download(t).copy() for t in (up, h, y)]
    p = ex.prepare_op_graph(ops)
    other_a = ex.tensor_from(oracle.fill_det(m * hid, 7506), shape=[m, hid])
    other_c = ex.tensor([m, ffn])
    for _ in range(5):
        for t, e in zip((up, h, y), eager):
            ex.upload(t, np.zeros(e.size, np.float32))
        p.run()
        for t, e in zip((up, h, y), eager):
            np.testing.assert_array_equal(ex.download(t), e)
        ex.run_ops([ta.MatmulOp(other_a, wu, other_c)])  # eager work on the same executor between replays
    p.close()


def _dual_oracle_check(oracle, hx, hwu, hwg, hbias, got_up, got_h, bt, m, n, k):
    hwb = np.tile(hwu, bt)
    check_f16_mfma(got_up, f16_mfma_refs(hx, hwb, bt, m, n, k, oracle, alpha=1.25), k, oracle)
    refs_h = f16_mfma_refs(hx, np.tile(hwg, bt), bt, m, n, k, oracle, alpha=1.25, bias=hbias, act=2,
                           binary=2, d=got_up.reshape(-1))
    check_f16_mfma(got_h, refs_h, k, oracle)


def test_f16_mfma_batched_alpha_accumulate(ta, ex, oracle):
    """f16.rs:791-817: batched + alpha + accumulate."""
    bt, m, n, k = 2, 256, 384, 256
    ha, hb, hc = oracle.fill_det(bt * m * k, 9700), oracle.fill_det(bt * k * n, 9701), oracle.fill_det(bt * m * n, 9702)
    a = ex.tensor_from(ha, shape=[bt, m, k])
    b = ex.tensor_from(hb, shape=[bt, k, n], f16=True)
    c = ex.tensor_from(hc, shape=[bt, m, n])
    ex.run_ops([ta.MatmulOp(a, b, c, alpha=0.75, accumulate=True)])
    refs = f16_mfma_refs(ha, hb, bt, m, n, k, oracle, alpha=0.75, c0=hc, acc=True)
    check_f16_mfma(ex.download(c), refs, k, oracle)


@pytest.mark.parametrize("bt,m,n,k", [(1, 256, 384, 256), (1, 128, 128, 64), (1, 512, 256, 2048), (3, 64, 128, 96)])
def test_a16_activations(ta, ex, oracle, bt, m, n, k):
    """f16.rs:316-360: f16 A/B/C; tolerance(K) + half an f16 ulp of max|ref|
    (a16_tolerance, f16.rs:311-314)."""
    sa, sb, sc = ([m, k], [k, n], [m, n]) if bt == 1 else ([bt, m, k], [bt, k, n], [bt, m, n])
    ha = oracle.round_via_f16(oracle.fill_det(bt * m * k, 31))
    hb = oracle.round_via_f16(oracle.fill_det(bt * k * n, 32))
    a, b, c = ex.tensor_from(ha, f16=True, shape=sa), ex.tensor_from(hb, f16=True, shape=sb), ex.tensor(sc, f16=True)
    ex.matmul(a, b, c)
    ref = oracle.cpu_bmm(ha, hb, None, bt, m, n, k)
    got = ex.download(c).reshape(-1)
    tol = oracle.tolerance(k) + float(np.max(np.abs(ref))) * (0.5 / 1024.0)
    err, idx = oracle.max_abs_err(got, ref)
    assert err <= tol, f"a16 abs err {err} > {tol} at {idx}"


def test_a16_rejects_epilogue(ta, ex):
    a, b, c = ex.tensor([64, 64], f16=True), ex.tensor([64, 64], f16=True), ex.tensor([64, 64], f16=True)
    bias = ex.tensor([64])
    with pytest.raises(ta.TensorAshError, match="cannot fuse"):
        ex.run_ops([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=bias))])


def test_leaves_no_pending_hip_error(ta, ctx, oracle):
    """Kernel lookups probe every code object; a miss must not leave HIP's
    thread-local last error set for the host application (torch and other
    HIP users check it after their own calls)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipGetLastError.restype = ctypes.c_int
    hip.hipGetLastError()
    kex = ta.Executor(ctx, tune=False)
    a, b, c = kex.tensor_from(oracle.fill_det(64 * 64, 1), shape=[64, 64]), \
        kex.tensor_from(oracle.fill_det(64 * 64, 2), shape=[64, 64], f16=True), kex.tensor([64, 64])
    kex.run_ops([ta.MatmulOp(a, b, c)])
    kex.run_matmuls_split_k2(kex.tensor([64, 2048]), kex.tensor([2048, 64]), kex.tensor([64, 64]), 4)
    assert hip.hipGetLastError() == 0


@pytest.mark.parametrize("name", ["f16w_sk_m128n128", "f16w_sk_m128n64", "f16w_sk_m64n128"])
@pytest.mark.parametrize("splits", ["1", "3", "5"])
def test_f16_split_k_kernels(ta, ctx, oracle, monkeypatch, name, splits):
    """ta_gemm_h16sk_*: f32 A rounded to f16 (RNE) by the pre-pass, K split
    over `splits` workgroups per tile and summed in split order inside the
    launch.  Ragged M/N tiles, a batched [B, N] bias with SiLU, a broadcast
    B, D (ADD_SCALED); f32 tolerance against the dual-rounded oracle, 2e-3
    against f32 A; bit-identical over repeated runs (fixed split order),
    and the tile counters left at zero (a second, different launch reusing
    them is still right)."""
    monkeypatch.setenv("TA_H16_SPLITS", splits)
    kex = ta.Executor(ctx, kernel_selection=name, tune=False)
    bt, m, n, k = 2, 300, 264, 640
    ha = oracle.fill_det(bt * m * k, 7200)
    hb = oracle.fill_normal(k * n, 7201, 0.05)
    hbias, hd = oracle.fill_det(bt * n, 7202), oracle.fill_det(bt * m * n, 7203)
    a, b = kex.tensor_from(ha, shape=[bt, m, k]), kex.tensor_from(hb, shape=[k, n], f16=True)
    bias, d, c = kex.tensor_from(hbias, shape=[bt, n]), kex.tensor_from(hd, shape=[bt, m, n]), kex.tensor([bt, m, n])
    epi = ta.Epilogue(bias=bias, activation=ta.ACTIVATION_SILU, binary=ta.BINARY_ADD_SCALED, d=d, beta=0.5)
    print(f"{name} splits={splits} B={bt} {m}x{n}x{k}", flush=True)
    kex.run_ops([ta.MatmulOp(a, b, c, alpha=0.75, epilogue=epi)])
    got = kex.download(c)
    refs = f16_mfma_refs(ha, hb, bt, m, n, k, oracle, alpha=0.75, bias=hbias, bias_batch_stride=n, act=2,
                         binary=1, d=hd, beta=0.5)
    check_f16_mfma(got, refs, k, oracle)
    for _ in range(3):
        kex.run_ops([ta.MatmulOp(a, b, c, alpha=0.75, epilogue=epi)])
        np.testing.assert_array_equal(kex.download(c), got)
    # a smaller plain launch after: counters must be back at zero
    m2, n2, k2 = 130, 72, 384
    ha2, hb2 = oracle.fill_det(m2 * k2, 7204), oracle.fill_normal(k2 * n2, 7205, 0.05)
    a2, b2, c2 = kex.tensor_from(ha2, shape=[m2, k2]), kex.tensor_from(hb2, shape=[k2, n2], f16=True), kex.tensor([m2, n2])
    kex.run_ops([ta.MatmulOp(a2, b2, c2)])
    check_f16_mfma(kex.download(c2), f16_mfma_refs(ha2, hb2, 1, m2, n2, k2, oracle), k2, oracle)


@pytest.mark.parametrize("shape", [(512, 2560, 2048), (512, 2048, 5632)])
def test_f16_split_k_prefill_shapes(ta, ctx, oracle, shape):
    """The split-K f16w kernels at config-5 shapes with their default split
    counts, against the oracle (the down projection 512x2048x5632 routes to
    f16w_sk_m128n128 by default)."""
    m, n, k = shape
    ha, hb = oracle.fill_det(m * k, 7210), oracle.fill_normal(k * n, 7211, 0.02)
    refs = f16_mfma_refs(ha, hb, 1, m, n, k, oracle)
    for name in ("f16w_sk_m128n128", "f16w_sk_m128n64"):
        kex = ta.Executor(ctx, kernel_selection=name, tune=False)
        a, b, c = kex.tensor_from(ha, shape=[m, k]), kex.tensor_from(hb, shape=[k, n], f16=True), kex.tensor([m, n])
        print(f"{name} {m}x{n}x{k}", flush=True)
        kex.run_ops([ta.MatmulOp(a, b, c)])
        check_f16_mfma(kex.download(c), refs, k, oracle)


def test_f16w_a_conversion_reused_only_while_valid(ta, ex, oracle):
    """Within one submission, f16w GEMMs with the same f32 A share one f16
    pre-pass copy; an op that writes A in between, or split-K planes that
    reuse the scratch, force a fresh conversion.  Results equal separate
    launches bit for bit."""
    m, k, n = 256, 512, 320
    hx, hw1, hw2 = oracle.fill_det(m * k, 7300), oracle.fill_normal(k * n, 7301, 0.05), oracle.fill_normal(k * n, 7302, 0.05)
    hwx = oracle.fill_normal(k * k, 7303, 0.05)
    x, w1, w2 = ex.tensor_from(hx, shape=[m, k]), ex.tensor_from(hw1, shape=[k, n], f16=True), ex.tensor_from(hw2, shape=[k, n], f16=True)
    wx = ex.tensor_from(hwx, shape=[k, k], f16=True)
    y0 = ex.tensor_from(oracle.fill_det(m * k, 7304), shape=[m, k])
    c1, c2, c3 = ex.tensor([m, n]), ex.tensor([m, n]), ex.tensor([m, n])
    # separate launches: the reference bits
    ex.run_ops([ta.MatmulOp(x, w1, c1)])
    ref1 = ex.download(c1)
    ex.run_ops([ta.MatmulOp(x, w2, c2)])
    ref2 = ex.download(c2)
    ex.run_ops([ta.MatmulOp(x, w1, c1), ta.MatmulOp(x, w2, c2)])  # shared conversion
    np.testing.assert_array_equal(ex.download(c1), ref1)
    np.testing.assert_array_equal(ex.download(c2), ref2)
    # A rewritten in the middle of a graph: x <- y0 @ wx, then x @ w1 again
    ex.upload(x, hx)
    ex.run_op_graph([ta.MatmulOp(x, w1, c1), ta.MatmulOp(y0, wx, x), ta.MatmulOp(x, w1, c3)])
    np.testing.assert_array_equal(ex.download(c1), ref1)
    new_x = ex.download(x)
    x2 = ex.tensor_from(new_x, shape=[m, k])
    ex.run_ops([ta.MatmulOp(x2, w1, c2)])
    np.testing.assert_array_equal(ex.download(c3), ex.download(c2))
    # split-K planes between two uses of the same A
    ex.upload(x, hx)
    a32, b32, cs = ex.tensor_from(oracle.fill_det(64 * 8192, 7305), shape=[64, 8192]), \
        ex.tensor_from(oracle.fill_det(8192 * 64, 7306), shape=[8192, 64]), ex.tensor([64, 64])
    assert ex.dispatch_info_for(1, 64, 64, 8192)["split_k2"], "expected a split-K route"
    ex.run_op_graph([ta.MatmulOp(x, w1, c1), ta.MatmulOp(a32, b32, cs), ta.MatmulOp(x, w2, c3)])
    np.testing.assert_array_equal(ex.download(c1), ref1)
    np.testing.assert_array_equal(ex.download(c3), ref2)


@pytest.mark.parametrize("lanes", ["4", "2", None])
def test_run_ops_independent_ops_run_concurrently_with_serial_bits(ta, ex, oracle, monkeypatch, lanes):
    """ta_run_ops takes independent ops with no barriers between them
    (src/executor/dispatch.rs:55-60): they are spread over several streams,
    each with its own scratch.  Every output equals its own single-op
    launch bit for bit, over two submissions (lane scratch reused).  The
    lane count is forced (TA_RUN_OPS_LANES) or left to the heuristic."""
    if lanes:
        monkeypatch.setenv("TA_RUN_OPS_LANES", lanes)
    ops, outs = [], []

    def f32(shape, seed):
        return ex.tensor_from(oracle.fill_det(int(np.prod(shape)), seed), shape=list(shape))

    def f16w(k, n, seed, packed=False):
        w = oracle.fill_normal(k * n, seed, 0.05)
        if packed:
            w = ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n))
        return ex.tensor_from(w, shape=[k, n], f16=True)

    cases = [  # (A shape, B, out shape, epilogue kwargs, packed)
        ((256, 512), f32((512, 384), 7401), (256, 384), dict(bias=f32((384,), 7402), activation=ta.ACTIVATION_GELU), False),
        ((512, 1024), f16w(1024, 640, 7403), (512, 640), dict(activation=ta.ACTIVATION_SILU), False),
        ((1, 2048), f16w(2048, 1024, 7404, packed=True), (1, 1024), {}, True),
        ((4, 2048), f16w(2048, 512, 7405, packed=True), (4, 512), {}, True),
        ((128, 4096), f32((4096, 128), 7406), (128, 128), {}, False),  # split-K route
        ((96, 320), f32((320, 200), 7407), (96, 200), dict(binary=ta.BINARY_ADD_SCALED, d=f32((96, 200), 7408), beta=0.5), False),
    ]
    for i, (ashape, b, oshape, epi, packed) in enumerate(cases):
        a = f32(ashape, 7410 + i)
        c = ex.tensor(list(oshape))
        ops.append(ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(**epi), packed_b=packed))
        outs.append(c)
    refs = []
    for op, c in zip(ops, outs):
        ex.run_ops([op])
        refs.append(ex.download(c).copy())
    if lanes is None:
        # long underfilled GEMMs with an epilogue (no split-K): the heuristic spreads these
        bias = f32((256,), 7440)
        big = [ta.MatmulOp(f32((256, 16384), 7420 + i), f32((16384, 256), 7430 + i), ex.tensor([256, 256]),
                           epilogue=ta.Epilogue(bias=bias, activation=ta.ACTIVATION_RELU)) for i in range(4)]
        monkeypatch.setenv("TA_RUN_OPS_LANES", "1")  # serial reference, same (non-split-K) routes
        ex.run_ops(big)
        big_refs = [ex.download(op.c).copy() for op in big]
        monkeypatch.delenv("TA_RUN_OPS_LANES")
        for op in big:
            ex.upload(op.c, np.zeros(256 * 256, np.float32))
        ex.run_ops(big)
        for op, r in zip(big, big_refs):
            np.testing.assert_array_equal(ex.download(op.c), r)
    for rep in range(2):
        for c in outs:
            ex.upload(c, np.full(int(np.prod(c.shape)), np.nan, np.float32))
        print(f"concurrent run_ops of {len(ops)} ops, round {rep}", flush=True)
        st = ex.run_ops(ops)
        assert st.n_calls == len(ops)
        for i, c in enumerate(outs):
            np.testing.assert_array_equal(ex.download(c), refs[i], err_msg=f"op {i}")
