"""GPU parity of the decode GEMV (packed / row-major, f16 / f32 weights, fused
SwiGLU pair) and of the deterministic two-stage split-K.

f16-weight tolerance: normwise rel err <= 2e-3 against the oracle run on the
same f16-rounded weights (f32 activations are not rounded), plus the abs
bound 2*tolerance(K) + 1e-4 scaled by max|W| (weights are N(0, 0.02)).
Split-K: f32 tolerances of test_gemm_gpu plus bit-identical output over 10
runs (tests/correctness/splitk2.rs:116-122).
"""

import math

import numpy as np
import pytest

from conftest import rel_err
from test_gemm_gpu import check_f32

pytestmark = pytest.mark.gpu


def f16_weights(oracle, k, n, seed):
    w = oracle.fill_normal(k * n, seed, 0.02)
    return w, oracle.round_via_f16(w)


def check_f16(got, ref, k, oracle):
    got = np.asarray(got, np.float32).reshape(-1)
    ref = np.asarray(ref, np.float32).reshape(-1)
    r = rel_err(got, ref)
    assert r <= 2e-3, f"rel err {r} > 2e-3"
    err, idx = oracle.max_abs_err(got, ref)
    assert err <= 2 * oracle.tolerance(k) + 1e-4, f"abs err {err} at {idx}"


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("k,n", [(2048, 5632), (5632, 2048), (300, 96), (64, 64), (2048, 32000)])
def test_packed_gemv(ta, ex, oracle, m, k, n):
    w, wr = f16_weights(oracle, k, n, 40 + m)
    x = oracle.fill_det(m * k, 41)
    tile = ta.f16w_row_tile_n(k, n)
    packed = ta.pack_f16w_row_tiles(w, k, n, tile)
    np.testing.assert_array_equal(packed, oracle.pack_row_tiles(w, k, n, tile))
    tw = ex.tensor_from(packed, shape=[k, n], f16=True)
    tx, ty = ex.tensor_from(x, shape=[m, k]), ex.tensor([m, n])
    ex.run_ops([ta.MatmulOp(tx, tw, ty, packed_b=True)])
    check_f16(ex.download(ty), oracle.cpu_bmm(x, wr, None, 1, m, n, k), k, oracle)


@pytest.mark.parametrize("m", [4, 5, 8])
def test_packed_gemv_matrix_core_row_scales(ta, ex, oracle, m):
    """4-8 rows on 64-column tiles run on f16 MFMA with each X row scaled
    by a power of two and split into three f16 pieces.  Rows of very
    different magnitude (1e-20, 1, 1e20, 0) in one launch, with K ragged
    against the 256-row load groups, must each stay f32-accurate: per-row
    normwise rel err <= 1e-5 against the oracle on the same f16 weights
    (f16 would give ~5e-4; f32 accumulation over K = 1000 ~1e-6)."""
    k, n = 1000, 2048
    tile = ta.f16w_row_tile_n(k, n)
    assert tile == 64, f"expected 64-column tiles for {k}x{n}, got {tile}"
    w, wr = f16_weights(oracle, k, n, 70 + m)
    scales = np.array([1e-20, 1.0, 1e20, 0.0, 3.0, 1e-3, 7e5, 1.0][:m], np.float64)
    x = (oracle.fill_det(m * k, 71).reshape(m, k) * scales[:, None]).astype(np.float32).reshape(-1)
    tw = ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, tile), shape=[k, n], f16=True)
    tx, ty = ex.tensor_from(x, shape=[m, k]), ex.tensor([m, n])
    ex.run_ops([ta.MatmulOp(tx, tw, ty, packed_b=True)])
    got = np.asarray(ex.download(ty), np.float64).reshape(m, n)
    ref = np.asarray(oracle.cpu_bmm(x, wr, None, 1, m, n, k), np.float64).reshape(m, n)
    for r in range(m):
        if scales[r] == 0.0:
            assert not got[r].any(), f"row {r}: zero input gave nonzero output"
            continue
        e = np.linalg.norm(got[r] - ref[r]) / np.linalg.norm(ref[r])
        assert e <= 1e-5, f"row {r} (scale {scales[r]:g}): rel err {e}"
    # an infinite X element gives +-inf (not NaN) where every weight of its
    # column is nonzero, as with f32 FMAs -- also in a row whose finite
    # values reach 7e5 (the row scale comes from the finite values only, so
    # they do not overflow the f16 pieces)
    xi = x.reshape(m, k).copy()
    inf_rows = [1] + ([6] if m > 6 else [])
    for r in inf_rows:
        xi[r, 5] = np.inf
    ex.upload(tx, xi.reshape(-1))
    ex.run_ops([ta.MatmulOp(tx, tw, ty, packed_b=True)])
    got = np.asarray(ex.download(ty), np.float32).reshape(m, n)
    want = np.where(wr.reshape(k, n)[5] > 0, np.inf, -np.inf)
    nz = wr.reshape(k, n)[5] != 0
    for r in inf_rows:
        np.testing.assert_array_equal(got[r][nz], want[nz])
    for r in range(m):
        if r not in inf_rows and scales[r] != 0.0:
            assert np.all(np.isfinite(got[r])), f"row {r} without inf went non-finite"


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("epi", [dict(bias=True, act=2), dict(act=3, binary=1, beta=1.0),
                                 dict(binary=2), dict(alpha=0.5, accumulate=True)])
def test_packed_gemv_epilogues(ta, ex, oracle, m, epi):
    k, n = 1024, 768
    w, wr = f16_weights(oracle, k, n, 7)
    x = oracle.fill_det(m * k, 8)
    tw = ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n)), shape=[k, n], f16=True)
    tx, ty = ex.tensor_from(x, shape=[m, k]), ex.tensor([m, n])
    epi = dict(epi)
    alpha, acc = epi.pop("alpha", 1.0), epi.pop("accumulate", False)
    e = ta.Epilogue(activation=epi.get("act", 0), binary=epi.get("binary", 0), beta=epi.get("beta", 0.0))
    hbias = hd = hc0 = None
    if epi.get("bias"):
        hbias = oracle.fill_det(n, 9)
        e.bias = ex.tensor_from(hbias, shape=[n])
    if e.binary:
        hd = oracle.fill_det(m * n, 10)
        e.d = ex.tensor_from(hd, shape=[m, n])
    if acc:
        hc0 = oracle.fill_det(m * n, 11)
        ex.upload(ty, hc0)
    ex.run_ops([ta.MatmulOp(tx, tw, ty, alpha, acc, e, packed_b=True)])
    ref = oracle.reference_gemm(x, wr, 1, m, n, k, alpha, hc0, acc, hbias, 0, e.activation,
                                e.binary, hd, e.beta)
    check_f16(ex.download(ty), ref, k, oracle)


@pytest.mark.parametrize("m", [1, 3, 4, 8])
def test_swiglu_mlp_graph(ta, ex, oracle, m, monkeypatch):
    """up; gate with SiLU*Mul{up}; down with +residual, as
    one dependent op graph (tools/llama-ash forward/mod.rs:186-210).  The
    three ops run as one persistent decode-MLP launch.  The gate/up outputs
    are bit-identical to the unfused launches (same K windows); the
    down-proj sums K in 256-row windows inside the MLP launch and in the
    planner's windows standalone, so both are checked against the oracle,
    and repeated MLP launches must repeat their bits."""
    monkeypatch.setenv("TA_MLP_MAX_ROWS", "8")  # the MLP launch at every M (the default)
    hdim, ffn = 2048, 5632
    wg, wgr = f16_weights(oracle, hdim, ffn, 101)
    wu, wur = f16_weights(oracle, hdim, ffn, 102)
    wd, wdr = f16_weights(oracle, ffn, hdim, 103)
    x = oracle.fill_det(m * hdim, 41)
    res = oracle.fill_det(m * hdim, 42)
    pk = lambda w, k, n: ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n)),
                                        shape=[k, n], f16=True)
    tg, tu, td = pk(wg, hdim, ffn), pk(wu, hdim, ffn), pk(wd, ffn, hdim)
    tx, tres = ex.tensor_from(x, shape=[m, hdim]), ex.tensor_from(res, shape=[m, hdim])
    up, h, y = ex.tensor([m, ffn]), ex.tensor([m, ffn]), ex.tensor([m, hdim])
    ops = [
        ta.MatmulOp(tx, tu, up, packed_b=True),
        ta.MatmulOp(tx, tg, h, epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up),
                    packed_b=True),
        ta.MatmulOp(h, td, y, epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=tres, beta=1.0), packed_b=True),
    ]
    ex.run_op_graph(ops)
    ref_up = oracle.cpu_bmm(x, wur, None, 1, m, ffn, hdim)
    ref_h = oracle.reference_gemm(x, wgr, 1, m, ffn, hdim, act=2, binary=2, d=ref_up)
    check_f16(ex.download(up), ref_up, hdim, oracle)
    check_f16(ex.download(h), ref_h, hdim, oracle)
    got_h = ex.download(h).reshape(-1)
    # down-proj checked against the oracle on the GPU's own h (isolates this GEMV)
    ref_y = oracle.reference_gemm(got_h, wdr, 1, m, hdim, ffn, binary=1, d=res, beta=1.0)
    check_f16(ex.download(y), ref_y, ffn, oracle)
    # end to end: the oracle's own h through the oracle's down projection
    ref_y_e2e = oracle.reference_gemm(ref_h, wdr, 1, m, hdim, ffn, binary=1, d=res, beta=1.0)
    check_f16(ex.download(y), ref_y_e2e, ffn, oracle)
    # same graph unfused (run_ops on independent pieces) gives identical bits
    up2, h2 = ex.tensor([m, ffn]), ex.tensor([m, ffn])
    ex.run_ops([ta.MatmulOp(tx, tu, up2, packed_b=True)])
    ex.run_ops([ta.MatmulOp(tx, tg, h2, epilogue=ta.Epilogue(activation=2, binary=2, d=up2), packed_b=True)])
    np.testing.assert_array_equal(ex.download(up2), ex.download(up))
    np.testing.assert_array_equal(ex.download(h2), ex.download(h))
    y_mlp = ex.download(y).copy()
    monkeypatch.setenv("TA_NO_MLP", "1")
    y2 = ex.tensor([m, hdim])
    ex.run_op_graph(ops[:2] + [ta.MatmulOp(h, td, y2, epilogue=ops[2].epilogue, packed_b=True)])
    check_f16(ex.download(y2), ref_y, ffn, oracle)
    monkeypatch.delenv("TA_NO_MLP")
    # repeated launches reuse the self-resetting tickets and flags
    for _ in range(3):
        ex.run_op_graph(ops)
        np.testing.assert_array_equal(ex.download(y), y_mlp)


def _mlp_layer_ops(ta, x, wts, up, h, y, res):
    wg, wu, wd = wts
    return [
        ta.MatmulOp(x, wu, up, packed_b=True),
        ta.MatmulOp(x, wg, h, epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up),
                    packed_b=True),
        ta.MatmulOp(h, wd, y, epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=res, beta=1.0), packed_b=True),
    ]


@pytest.mark.parametrize("m", [1, 4, 6, 8])
def test_decode_mlp_chain(ta, ex, oracle, m, monkeypatch):
    """Three config-3 decode layers in one op graph (layer l+1 reads layer
    l's y as x and as residual) run as one persistent MLP-chain launch.
    Every layer is checked against the oracle on the GPU's own layer input,
    and the chain must give the bits of separate per-layer MLP launches,
    eagerly and through a prepared graph, over repeated runs."""
    monkeypatch.setenv("TA_MLP_MAX_ROWS", "8")
    hdim, ffn, layers = 2048, 5632, 3
    pk = lambda w, k, n: ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n)),
                                        shape=[k, n], f16=True)
    wts, refs = [], []
    for l in range(layers):
        wg, wgr = f16_weights(oracle, hdim, ffn, 301 + 3 * l)
        wu, wur = f16_weights(oracle, hdim, ffn, 302 + 3 * l)
        wd, wdr = f16_weights(oracle, ffn, hdim, 303 + 3 * l)
        wts.append((pk(wg, hdim, ffn), pk(wu, hdim, ffn), pk(wd, ffn, hdim)))
        refs.append((wgr, wur, wdr))
    x0 = oracle.fill_det(m * hdim, 51)
    xs = [ex.tensor_from(x0, shape=[m, hdim])] + [ex.tensor([m, hdim]) for _ in range(layers)]
    ups = [ex.tensor([m, ffn]) for _ in range(layers)]
    hs = [ex.tensor([m, ffn]) for _ in range(layers)]
    ops = []
    for l in range(layers):
        ops += _mlp_layer_ops(ta, xs[l], wts[l], ups[l], hs[l], xs[l + 1], xs[l])
    ex.run_op_graph(ops)
    got = [ex.download(t).copy() for t in xs + ups + hs]
    for l in range(layers):
        wgr, wur, wdr = refs[l]
        xin = got[l]
        ref_up = oracle.cpu_bmm(xin, wur, None, 1, m, ffn, hdim)
        ref_h = oracle.reference_gemm(xin, wgr, 1, m, ffn, hdim, act=2, binary=2, d=ref_up)
        check_f16(got[layers + 1 + l], ref_up, hdim, oracle)
        check_f16(got[2 * layers + 1 + l], ref_h, hdim, oracle)
        ref_y = oracle.reference_gemm(got[2 * layers + 1 + l], wdr, 1, m, hdim, ffn, binary=1, d=xin,
                                      beta=1.0)
        check_f16(got[l + 1], ref_y, ffn, oracle)
    for t in xs[1:] + ups + hs:
        ex.upload(t, np.zeros(int(np.prod(t.shape)), np.float32))
    monkeypatch.setenv("TA_NO_MLP_CHAIN", "1")
    ex.run_op_graph(ops)
    monkeypatch.delenv("TA_NO_MLP_CHAIN")
    for a, b in zip([ex.download(t) for t in xs + ups + hs], got):
        np.testing.assert_array_equal(a, b)
    for _ in range(3):
        ex.run_op_graph(ops)
        np.testing.assert_array_equal(ex.download(xs[-1]), got[layers])
    prep = ex.prepare_op_graph(ops)
    for _ in range(3):
        ex.upload(xs[-1], np.zeros(m * hdim, np.float32))
        prep.run()
        np.testing.assert_array_equal(ex.download(xs[-1]), got[layers])
    prep.close()


@pytest.mark.parametrize("m", [1, 4])
def test_decode_mlp_chain_256_row_windows(ta, ex, oracle, m, monkeypatch):
    """Hidden 768 and FFN 1280: K windows of 256 rows in both phases, and
    an FFN width that is not a multiple of 512 (5 down windows).  Two
    chained layers, each checked against the oracle on the GPU's own layer
    input; the chain gives the bits of per-layer MLP launches."""
    monkeypatch.setenv("TA_MLP_MAX_ROWS", "8")
    hdim, ffn, layers = 768, 1280, 2
    pk = lambda w, k, n: ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n)),
                                        shape=[k, n], f16=True)
    wts, refs = [], []
    for l in range(layers):
        wg, wgr = f16_weights(oracle, hdim, ffn, 501 + 3 * l)
        wu, wur = f16_weights(oracle, hdim, ffn, 502 + 3 * l)
        wd, wdr = f16_weights(oracle, ffn, hdim, 503 + 3 * l)
        wts.append((pk(wg, hdim, ffn), pk(wu, hdim, ffn), pk(wd, ffn, hdim)))
        refs.append((wgr, wur, wdr))
    xs = [ex.tensor_from(oracle.fill_det(m * hdim, 53), shape=[m, hdim])]
    xs += [ex.tensor([m, hdim]) for _ in range(layers)]
    ups = [ex.tensor([m, ffn]) for _ in range(layers)]
    hs = [ex.tensor([m, ffn]) for _ in range(layers)]
    ops = []
    for l in range(layers):
        ops += _mlp_layer_ops(ta, xs[l], wts[l], ups[l], hs[l], xs[l + 1], xs[l])
    ex.run_op_graph(ops)
    got = [ex.download(t).copy() for t in xs + ups + hs]
    for l in range(layers):
        wgr, wur, wdr = refs[l]
        xin = got[l]
        ref_up = oracle.cpu_bmm(xin, wur, None, 1, m, ffn, hdim)
        ref_h = oracle.reference_gemm(xin, wgr, 1, m, ffn, hdim, act=2, binary=2, d=ref_up)
        check_f16(got[layers + 1 + l], ref_up, hdim, oracle)
        check_f16(got[2 * layers + 1 + l], ref_h, hdim, oracle)
        ref_y = oracle.reference_gemm(got[2 * layers + 1 + l], wdr, 1, m, hdim, ffn, binary=1, d=xin,
                                      beta=1.0)
        check_f16(got[l + 1], ref_y, ffn, oracle)
    for t in xs[1:] + ups + hs:
        ex.upload(t, np.zeros(int(np.prod(t.shape)), np.float32))
    monkeypatch.setenv("TA_NO_MLP_CHAIN", "1")
    ex.run_op_graph(ops)
    monkeypatch.delenv("TA_NO_MLP_CHAIN")
    for a, b in zip([ex.download(t) for t in xs + ups + hs], got):
        np.testing.assert_array_equal(a, b)


def test_decode_mlp_chain_long(ta, ex, oracle, monkeypatch):
    """18 layers over two ping-pong activation buffers and shared up/h
    buffers (the decode-forward form): the executor splits the chain into
    launches of at most 16 layers; bits equal separate per-layer launches."""
    m, hdim, ffn, layers = 2, 512, 1024, 18
    pk = lambda w, k, n: ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n)),
                                        shape=[k, n], f16=True)
    wts = [(pk(f16_weights(oracle, hdim, ffn, 400 + 3 * l)[0], hdim, ffn),
            pk(f16_weights(oracle, hdim, ffn, 401 + 3 * l)[0], hdim, ffn),
            pk(f16_weights(oracle, ffn, hdim, 402 + 3 * l)[0], ffn, hdim)) for l in range(3)]
    x0 = oracle.fill_det(m * hdim, 52)
    bufs = [ex.tensor([m, hdim]), ex.tensor([m, hdim])]
    up, h = ex.tensor([m, ffn]), ex.tensor([m, ffn])
    ops = []
    for l in range(layers):
        ops += _mlp_layer_ops(ta, bufs[l % 2], wts[l % 3], up, h, bufs[(l + 1) % 2], bufs[l % 2])
    outs = []
    for env in (None, "TA_NO_MLP_CHAIN"):
        if env:
            monkeypatch.setenv(env, "1")
        ex.upload(bufs[0], x0)
        ex.run_op_graph(ops)
        outs.append([ex.download(t).copy() for t in bufs + [up, h]])
        if env:
            monkeypatch.delenv(env)
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    assert np.all(np.isfinite(outs[0][0]))


@pytest.mark.parametrize("m", [1, 8])
def test_decode_mlp_down_epilogue(ta, ex, oracle, m, monkeypatch):
    """Persistent MLP with a general down-proj epilogue (bias + GELU) and a
    gate bias, on non-square dims (H=768, F=1536)."""
    monkeypatch.setenv("TA_MLP_MAX_ROWS", "8")
    hdim, ffn = 768, 1536
    wg, wgr = f16_weights(oracle, hdim, ffn, 201)
    wu, wur = f16_weights(oracle, hdim, ffn, 202)
    wd, wdr = f16_weights(oracle, ffn, hdim, 203)
    x = oracle.fill_det(m * hdim, 204)
    bg, bd = oracle.fill_det(ffn, 205), oracle.fill_det(hdim, 206)
    pk = lambda w, k, n: ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, 64), shape=[k, n], f16=True)
    tg, tu, td = pk(wg, hdim, ffn), pk(wu, hdim, ffn), pk(wd, ffn, hdim)
    tx = ex.tensor_from(x, shape=[m, hdim])
    tbg, tbd = ex.tensor_from(bg, shape=[ffn]), ex.tensor_from(bd, shape=[hdim])
    up, h, y = ex.tensor([m, ffn]), ex.tensor([m, ffn]), ex.tensor([m, hdim])
    ex.run_op_graph([
        ta.MatmulOp(tx, tu, up, alpha=0.5, packed_b=True),
        ta.MatmulOp(tx, tg, h, alpha=0.5, epilogue=ta.Epilogue(bias=tbg, activation=2, binary=2, d=up),
                    packed_b=True),
        ta.MatmulOp(h, td, y, epilogue=ta.Epilogue(bias=tbd, activation=3), packed_b=True),
    ])
    ref_up = oracle.cpu_bmm(x, wur, None, 1, m, ffn, hdim, 0.5)
    ref_h = oracle.reference_gemm(x, wgr, 1, m, ffn, hdim, 0.5, bias=bg, act=2, binary=2, d=ref_up)
    check_f16(ex.download(up), ref_up, hdim, oracle)
    check_f16(ex.download(h), ref_h, hdim, oracle)
    ref_y = oracle.reference_gemm(ex.download(h).reshape(-1), wdr, 1, m, hdim, ffn, bias=bd, act=3)
    check_f16(ex.download(y), ref_y, ffn, oracle)


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("m,k,n", [(1, 4096, 4096), (3, 1000, 998), (8, 512, 132), (2, 700, 130)])
def test_row_gemv(ta, ex, oracle, f16, m, k, n):
    """M <= 8 with row-major B routes to the decode GEMV when N allows its
    8-byte lane loads (N % 4 for f16, N % 2 for f32), else to the GEMM."""
    w = oracle.fill_det(k * n, 5)
    wr = oracle.round_via_f16(w) if f16 else w
    x = oracle.fill_det(m * k, 6)
    tw = ex.tensor_from(w, shape=[k, n], f16=f16)
    tx, ty = ex.tensor_from(x, shape=[m, k]), ex.tensor([m, n])
    routed = ex.dispatch_info_for(1, m, n, k, f16)["kernel"]
    assert ("gemv" in routed) == (n % (4 if f16 else 2) == 0), routed
    ex.matmul(tx, tw, ty)
    check_f32(ex.download(ty), oracle.cpu_bmm(x, wr, None, 1, m, n, k), k, oracle)


def test_gemv_deterministic(ta, ex, oracle):
    k, n = 5632, 2048
    w, _ = f16_weights(oracle, k, n, 3)
    x = oracle.fill_det(8 * k, 4)
    tw = ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, 64), shape=[k, n], f16=True)
    tx, ty = ex.tensor_from(x, shape=[8, k]), ex.tensor([8, n])
    outs = []
    for _ in range(5):
        ex.run_ops([ta.MatmulOp(tx, tw, ty, packed_b=True)])
        outs.append(ex.download(ty).copy())
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


# ---------------------------------------------------------------- split-K

@pytest.mark.parametrize("m,n,k", [(64, 256, 65536), (32, 128, 131072)])
@pytest.mark.parametrize("splits", [8, 16, 32])
def test_config4_splitk_deterministic(ta, ex, oracle, m, n, k, splits):
    """uniform A/B seeds 51, 52; within tolerance and
    bit-identical over 10 runs."""
    ha, hb = oracle.fill_det(m * k, 51), oracle.fill_det(k * n, 52)
    a, b, c = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n]), ex.tensor([m, n])
    st = ex.run_matmuls_split_k2(a, b, c, splits)
    assert st.total_flops == 2 * m * n * k
    first = ex.download(c).copy()
    check_f32(first, oracle.cpu_bmm(ha, hb, None, 1, m, n, k), k, oracle, epi=False)
    for _ in range(9):
        ex.run_matmuls_split_k2(a, b, c, splits)
        np.testing.assert_array_equal(ex.download(c), first)


@pytest.mark.parametrize("m,n,k,splits,alpha,batch", [
    (64, 64, 8192, 16, 1.0, 1), (256, 256, 4096, 4, 1.0, 1), (101, 103, 999, 7, 1.0, 1),
    (33, 65, 4000, 5, 0.25, 3),
    # windows of whole 64-deep stages: the pipelined stage-1 kernels
    (64, 512, 8192, 4, 0.5, 2), (32, 256, 16384, 8, 1.0, 1), (64, 256, 4160, 5, 1.0, 1),
    (32, 128, 8192, 2, 2.0, 3),
    # 64 x 64 stage-1 tiles, several per K window (dealt to the XCDs by window)
    (64, 256, 16384, 4, 1.0, 2), (64, 1024, 32768, 8, 0.5, 1),
])
def test_splitk_shapes(ta, ex, oracle, m, n, k, splits, alpha, batch):
    """tests/correctness/splitk2.rs:48-122 shapes (odd, batched, alpha)."""
    sa = [batch, m, k] if batch > 1 else [m, k]
    sc = [batch, m, n] if batch > 1 else [m, n]
    ha, hb = oracle.fill_det(batch * m * k, 61), oracle.fill_det(k * n, 62)
    a, b, c = ex.tensor_from(ha, shape=sa), ex.tensor_from(hb, shape=[k, n]), ex.tensor(sc)
    ex.run_matmuls_split_k2(a, b, c, splits, alpha)
    ref = oracle.cpu_bmm(ha, hb, None, batch, m, n, k, alpha)
    check_f32(ex.download(c), ref, k, oracle)


def test_splitk_errors(ta, ex):
    a, b, c = ex.tensor([4, 16]), ex.tensor([16, 8]), ex.tensor([4, 8])
    with pytest.raises(ta.TensorAshError, match="exceeds K=16"):
        ex.run_matmuls_split_k2(a, b, c, 17)


def test_auto_splitk_route(ta, ex, oracle):
    """Deep-K, few-tile plain op is routed through split-K automatically."""
    m, n, k = 64, 128, 16384
    info = ex.dispatch_info_for(1, m, n, k)
    assert info["split_k2"] is not None and info["split_k2"] >= 2
    ha, hb = oracle.fill_det(m * k, 1), oracle.fill_det(k * n, 2)
    a, b, c = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n]), ex.tensor([m, n])
    ex.matmul(a, b, c)
    check_f32(ex.download(c), oracle.cpu_bmm(ha, hb, None, 1, m, n, k), k, oracle, epi=False)


# ---------------------------------------------------------------- prepared

def test_prepared_replay(ta, ex, oracle):
    """tests/correctness/prepared.rs: record once, replay; graph with a chain."""
    m, n, k = 128, 96, 64
    ha, hb, hb2 = oracle.fill_det(m * k, 1), oracle.fill_det(k * n, 2), oracle.fill_det(n * n, 3)
    a, b, b2 = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n]), ex.tensor_from(hb2, shape=[n, n])
    c, c2 = ex.tensor([m, n]), ex.tensor([m, n])
    p = ex.prepare_op_graph([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(activation=1)),
                             ta.MatmulOp(c, b2, c2)])
    for _ in range(3):
        st = p.run()
        assert st.n_calls == 2
    ref1 = oracle.reference_gemm(ha, hb, 1, m, n, k, act=1)
    ref2 = oracle.cpu_bmm(ex.download(c), hb2, None, 1, m, n, n)
    check_f32(ex.download(c), ref1, k, oracle)
    check_f32(ex.download(c2), ref2, n, oracle)
    p.submit()
    with pytest.raises(ta.TensorAshError, match="already in flight"):
        p.submit()
    p.wait()
    with pytest.raises(ta.TensorAshError, match="nothing submitted"):
        p.wait()
    p.close()


def test_prepared_swiglu_graph_replays(ta, ex, oracle):
    """Decode MLP as one hipGraph (fused pair + down), replayed 5 times, each
    replay equal to the eager run."""
    hdim, ffn, m = 512, 1024, 1
    ws = [f16_weights(oracle, hdim, ffn, 11)[0], f16_weights(oracle, hdim, ffn, 12)[0],
          f16_weights(oracle, ffn, hdim, 13)[0]]
    pk = lambda w, k, n: ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, 64), shape=[k, n], f16=True)
    tg, tu, td = pk(ws[0], hdim, ffn), pk(ws[1], hdim, ffn), pk(ws[2], ffn, hdim)
    tx = ex.tensor_from(oracle.fill_det(hdim, 1), shape=[m, hdim])
    tres = ex.tensor_from(oracle.fill_det(hdim, 2), shape=[m, hdim])
    up, h, y = ex.tensor([m, ffn]), ex.tensor([m, ffn]), ex.tensor([m, hdim])
    ops = [ta.MatmulOp(tx, tu, up, packed_b=True),
           ta.MatmulOp(tx, tg, h, epilogue=ta.Epilogue(activation=2, binary=2, d=up), packed_b=True),
           ta.MatmulOp(h, td, y, epilogue=ta.Epilogue(binary=1, d=tres, beta=1.0), packed_b=True)]
    ex.run_op_graph(ops)
    eager = ex.download(y).copy()
    p = ex.prepare_op_graph(ops)
    for _ in range(5):
        ex.upload(y, np.zeros(m * hdim, np.float32))
        p.run()
        np.testing.assert_array_equal(ex.download(y), eager)
    p.close()
