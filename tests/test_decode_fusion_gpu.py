"""GPU parity of the decode fusions of MatmulOp: the normed-A GEMV
(RMSNorm of A folded into the product) and the store-time RoPE / KV-cache
scatter (tests/correctness/fusion.rs and store.rs of the reference).

Normed-A is checked against the oracle's f64 RMSNorm followed by cpu_bmm on
the f16-rounded weights, with the GEMV tolerances of test_gemv_splitk_gpu.
The store epilogue is checked against the same GEMV without the fusion,
followed by the oracle's rotation / scatter of that GPU output (the
reference compares fused against composed the same way): the rotation is
an f32 fma on identical inputs, so at most 1 ulp (the oracle's
double-rounded fma) may differ; scatters are exact.
"""

import numpy as np
import pytest

from test_gemv_splitk_gpu import check_f16, f16_weights

pytestmark = pytest.mark.gpu

EPS = 1e-5


def ulp_diff(a, b) -> int:
    a = np.asarray(a, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    return int(np.max(np.abs(a - b))) if a.size else 0


def weights_tensor(ta, ex, w, k, n, packed):
    if packed:
        return ex.tensor_from(ta.pack_f16w_row_tiles(w, k, n, ta.f16w_row_tile_n(k, n)), shape=[k, n], f16=True)
    return ex.tensor_from(w, shape=[k, n], f16=True)


def pos_cell(ex, value):
    """A device u32 position cell (a one-element tensor holding its bits)."""
    return ex.tensor_from(np.array([value], np.uint32).view(np.float32), shape=[1])


# ---------------------------------------------------------------- normed-A

@pytest.mark.parametrize("m,k,n,kind", [(1, 2048, 256, "f16"), (1, 256, 1024, "f16"), (1, 204, 36, "f16"),
                                        (1, 512, 300, "f32"), (1, 2048, 5632, "packed"), (3, 2048, 256, "f16"),
                                        (8, 1024, 512, "packed")])
def test_normed_a_gemv_matches_rms_reference(ta, ex, oracle, m, k, n, kind):
    """fusion.rs:62-107: C = rms_norm(A, w, eps) @ B on the decode GEMV
    (f16 row-major, f16 packed and f32 weights; 2-8 rows are this build's
    extension of the reference's M = 1)."""
    x, w_norm = oracle.fill_det(m * k, 11000 + k), oracle.fill_det(k, 11001 + k)
    if kind == "f32":
        wb = oracle.fill_det(k * n, 11002 + k)
        b, wr = ex.tensor_from(wb, shape=[k, n]), wb
    else:
        wb, wr = f16_weights(oracle, k, n, 11002 + k)
        b = weights_tensor(ta, ex, wb, k, n, kind == "packed")
    a, tw, c = ex.tensor_from(x, shape=[m, k]), ex.tensor_from(w_norm, shape=[k]), ex.tensor([m, n])
    assert "gemv" in ex.dispatch_info_for(1, m, n, k, kind != "f32")["kernel"]
    ex.run_ops([ta.MatmulOp(a, b, c, packed_b=kind == "packed", normed_a=(tw, EPS))])
    ref = oracle.cpu_bmm(oracle.rms_norm_rows(x, w_norm, m, k, EPS), wr, None, 1, m, n, k)
    check_f16(ex.download(c), ref, k, oracle)


def test_normed_a_composes_with_silu_mul_epilogue_in_graph(ta, ex, oracle):
    """fusion.rs:109-170: up = norm(x) @ Wu, h = silu(norm(x) @ Wg) * up in
    one dependent op graph (the pair with one norm runs as one dual GEMV
    launch)."""
    k, n = 1024, 768
    x, w_norm = oracle.fill_det(k, 12000), oracle.fill_det(k, 12001)
    wg, wgr = f16_weights(oracle, k, n, 12002)
    wu, wur = f16_weights(oracle, k, n, 12003)
    a, tw = ex.tensor_from(x, shape=[1, k]), ex.tensor_from(w_norm, shape=[k])
    tg, tu = weights_tensor(ta, ex, wg, k, n, True), weights_tensor(ta, ex, wu, k, n, True)
    up, h = ex.tensor([1, n]), ex.tensor([1, n])
    ex.run_op_graph([
        ta.MatmulOp(a, tu, up, packed_b=True, normed_a=(tw, EPS)),
        ta.MatmulOp(a, tg, h, packed_b=True, normed_a=(tw, EPS),
                    epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up)),
    ])
    xn = oracle.rms_norm_rows(x, w_norm, 1, k, EPS)
    up_ref = oracle.cpu_bmm(xn, wur, None, 1, 1, n, k)
    h_ref = oracle.epilogue(oracle.cpu_bmm(xn, wgr, None, 1, 1, n, k), n, n, act=2, binary=2, d=up_ref)
    check_f16(ex.download(up), up_ref, k, oracle)
    check_f16(ex.download(h), h_ref, k, oracle)


def test_normed_a_rejects_conflicting_forms(ta, ctx, ex, oracle):
    """fusion.rs:172-245 and recording.rs:204-220 error contracts."""
    k, n = 256, 128
    a, c = ex.tensor_from(oracle.fill_det(k, 1), shape=[1, k]), ex.tensor([1, n])
    b = ex.tensor_from(oracle.fill_det(k * n, 2), shape=[k, n], f16=True)
    w = ex.tensor_from(oracle.fill_det(k, 3), shape=[k])
    bad_len = ex.tensor_from(oracle.fill_det(k - 1, 3), shape=[k - 1])
    w16 = ex.tensor_from(oracle.fill_det(k, 3), shape=[k], f16=True)
    bias, d = ex.tensor([n]), ex.tensor([1, n])
    cases = [
        (ta.MatmulOp(a, b, c, normed_a=(bad_len, EPS)), "must equal K"),
        (ta.MatmulOp(a, b, c, normed_a=(w16, EPS)), "must be f32 storage"),
        (ta.MatmulOp(a, b, c, normed_a=(w, EPS), epilogue=ta.Epilogue(bias=bias)), "epilogue bias"),
        (ta.MatmulOp(a, b, c, normed_a=(w, EPS),
                     epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=d, beta=1.0)), "AddScaled"),
    ]
    for op, msg in cases:
        with pytest.raises(ta.TensorAshError, match=msg):
            ex.run_ops([op])
    # No decode GEMV route: M = 16 (auto) and an explicit GEMM selection.
    a16 = ex.tensor_from(oracle.fill_det(16 * k, 1), shape=[16, k])
    with pytest.raises(ta.TensorAshError, match="does not implement the fused normed-A GEMV"):
        ex.run_ops([ta.MatmulOp(a16, b, ex.tensor([16, n]), normed_a=(w, EPS))])
    gemm = ta.Executor(ctx, kernel_selection="f16w_m64n64", tune=False)
    a1, b1 = gemm.tensor_from(oracle.fill_det(k, 1), shape=[1, k]), gemm.tensor_from(oracle.fill_det(k * n, 2), shape=[k, n], f16=True)
    with pytest.raises(ta.TensorAshError, match="does not implement the fused normed-A GEMV"):
        gemm.run_ops([ta.MatmulOp(a1, b1, gemm.tensor([1, n]), normed_a=(gemm.tensor_from(oracle.fill_det(k, 3)), EPS))])


# ---------------------------------------------------------------- store epilogue

def store_case(ta, ex, oracle, k, n, hd, t_max, packed, seed):
    x = oracle.fill_det(k, seed)
    wb, _ = f16_weights(oracle, k, n, seed + 1)
    table = oracle.fill_det(t_max * hd, seed + 2)
    return (ex.tensor_from(x, shape=[1, k]), weights_tensor(ta, ex, wb, k, n, packed),
            ex.tensor_from(table, shape=[t_max, hd // 2, 2]), table)


@pytest.mark.parametrize("k,n,hd,packed", [(96, 128, 32, False), (96, 48, 16, False), (256, 160, 32, False),
                                           (2048, 2048, 64, True), (2048, 256, 64, True)])
@pytest.mark.parametrize("normed", [False, True])
def test_store_rope_matches_gemv_then_rope(ta, ex, oracle, k, n, hd, packed, normed):
    """store.rs:90-160: rope-at-store equals the same GEMV followed by the
    rotation of its output row."""
    t_max, pos = 16, 5
    a, b, table, host_table = store_case(ta, ex, oracle, k, n, hd, t_max, packed, 61000 + n)
    extra = dict(normed_a=(ex.tensor_from(oracle.fill_det(k, 61900 + n)), EPS)) if normed else {}
    plain, fused = ex.tensor([1, n]), ex.tensor([1, n])
    ex.run_ops([ta.MatmulOp(a, b, plain, packed_b=packed, **extra)])
    desc = ta.MatmulStoreDesc(head_dim=hd, pos_base=pos)
    ex.run_ops([ta.MatmulOp(a, b, fused, packed_b=packed, store=ta.MatmulStore(ta.STORE_ROPE, desc, table=table),
                            **extra)])
    want = oracle.rope_pairs(ex.download(plain), host_table, pos, hd)
    assert ulp_diff(ex.download(fused), want) <= 1


@pytest.mark.parametrize("f16_dst", [False, True])
def test_store_scatter_v_cache(ta, ex, oracle, f16_dst):
    """store.rs:240-300: scatter into a [H, T_max, dh] V cache; C and every
    other cache element stay untouched."""
    k, n, hd, t_max, pos = 512, 256, 64, 12, 9
    a, b, _, _ = store_case(ta, ex, oracle, k, n, hd, t_max, True, 62000)
    plain = ex.tensor([1, n])
    ex.run_ops([ta.MatmulOp(a, b, plain, packed_b=True)])
    h = n // hd
    init = oracle.fill_det(h * t_max * hd, 62100)
    if f16_dst:
        init = oracle.round_via_f16(init)
    dst = ex.tensor_from(init, shape=[h, t_max, hd], f16=f16_dst)
    sentinel = np.full(n, 7.25, np.float32)
    c = ex.tensor_from(sentinel, shape=[1, n])
    desc = ta.MatmulStoreDesc(head_dim=hd, pos_base=pos, pos_scale=hd, stride_head=t_max * hd, stride_dim=1)
    ex.run_ops([ta.MatmulOp(a, b, c, packed_b=True, store=ta.MatmulStore(ta.STORE_SCATTER, desc, dst=dst))])
    want = oracle.store_scatter(init, ex.download(plain), pos, hd, hd, t_max * hd, 1, f16=f16_dst)
    np.testing.assert_array_equal(ex.download(dst).reshape(-1), want)
    np.testing.assert_array_equal(ex.download(c).reshape(-1), sentinel)


def test_store_rope_scatter_kt_cache_with_position_cell(ta, ex, oracle):
    """store.rs:300-380: rotate then scatter into a [H, dh, T_max] Kt cache;
    the position read from a device cell (pos_base + *cell) gives the same
    bits as the same position given directly."""
    k, n, hd, t_max = 1024, 512, 64, 16
    a, b, table, host_table = store_case(ta, ex, oracle, k, n, hd, t_max, True, 63000)
    plain = ex.tensor([1, n])
    ex.run_ops([ta.MatmulOp(a, b, plain, packed_b=True)])
    h = n // hd
    shape = [h, hd, t_max]
    d_direct, d_cell = ex.tensor(shape), ex.tensor(shape)
    zero = np.zeros(h * hd * t_max, np.float32)
    ex.upload(d_direct, zero)
    ex.upload(d_cell, zero)
    cell = pos_cell(ex, 5)
    kt = dict(head_dim=hd, pos_scale=1, stride_head=hd * t_max, stride_dim=t_max)
    ex.run_ops([ta.MatmulOp(a, b, ex.tensor([1, n]), packed_b=True, store=ta.MatmulStore(
        ta.STORE_ROPE_SCATTER, ta.MatmulStoreDesc(pos_base=7, **kt), table=table, dst=d_direct))])
    ex.run_ops([ta.MatmulOp(a, b, ex.tensor([1, n]), packed_b=True, store=ta.MatmulStore(
        ta.STORE_ROPE_SCATTER, ta.MatmulStoreDesc(pos_base=2, pos_addr=cell.device_address, **kt),
        table=table, dst=d_cell))])
    got = ex.download(d_cell).reshape(-1)
    np.testing.assert_array_equal(got, ex.download(d_direct).reshape(-1))
    rot = oracle.rope_pairs(ex.download(plain), host_table, 7, hd)
    want = oracle.store_scatter(zero, rot, 7, hd, 1, hd * t_max, t_max)
    assert ulp_diff(got, want) <= 1


def test_store_prepared_replay_follows_position_cell(ta, ex, oracle):
    """A prepared graph replays per token: the position cell is read at
    execution time (src/matmul/api.rs:127-131), so updating it between
    replays appends at the new position."""
    k, n, hd, t_max = 512, 128, 32, 8
    a, b, _, _ = store_case(ta, ex, oracle, k, n, hd, t_max, True, 64000)
    plain = ex.tensor([1, n])
    ex.run_ops([ta.MatmulOp(a, b, plain, packed_b=True)])
    row = ex.download(plain).reshape(-1)
    h = n // hd
    dst = ex.tensor([h, t_max, hd])
    ex.upload(dst, np.zeros(h * t_max * hd, np.float32))
    cell = pos_cell(ex, 0)
    desc = ta.MatmulStoreDesc(head_dim=hd, pos_base=0, pos_scale=hd, stride_head=t_max * hd, stride_dim=1,
                              pos_addr=cell.device_address)
    prep = ex.prepare_op_graph([ta.MatmulOp(a, b, ex.tensor([1, n]), packed_b=True,
                                            store=ta.MatmulStore(ta.STORE_SCATTER, desc, dst=dst))])
    want = np.zeros(h * t_max * hd, np.float32)
    for p in (3, 6, 1):
        ex.upload(cell, np.array([p], np.uint32).view(np.float32))
        prep.run()
        want = oracle.store_scatter(want, row, p, hd, hd, t_max * hd, 1)
        np.testing.assert_array_equal(ex.download(dst).reshape(-1), want)
    prep.close()


def test_store_rejects_invalid_forms(ta, ex, oracle):
    """resolution.rs:243-316 error contracts."""
    k, n, hd = 256, 128, 32
    a1 = ex.tensor_from(oracle.fill_det(k, 1), shape=[1, k])
    a2 = ex.tensor_from(oracle.fill_det(2 * k, 1), shape=[2, k])
    b16 = ex.tensor_from(oracle.fill_det(k * n, 2), shape=[k, n], f16=True)
    b32 = ex.tensor_from(oracle.fill_det(k * n, 2), shape=[k, n])
    table = ex.tensor_from(oracle.fill_det(4 * hd, 3), shape=[4, hd // 2, 2])
    dst = ex.tensor([n // hd, 4, hd])
    rope = lambda **kw: ta.MatmulStore(ta.STORE_ROPE, ta.MatmulStoreDesc(**kw), table=table)
    cases = [
        (ta.MatmulOp(a2, b16, ex.tensor([2, n]), store=rope(head_dim=hd)), "requires M == 1"),
        (ta.MatmulOp(a1, b32, ex.tensor([1, n]), store=rope(head_dim=hd)), "requires f16 weights"),
        (ta.MatmulOp(a1, b16, ex.tensor([1, n]), accumulate=True, store=rope(head_dim=hd)), "accumulate"),
        (ta.MatmulOp(a1, b16, ex.tensor([1, n]), epilogue=ta.Epilogue(activation=ta.ACTIVATION_RELU),
                     store=rope(head_dim=hd)), "fused epilogue"),
        (ta.MatmulOp(a1, b16, ex.tensor([1, n]), store=rope(head_dim=3)), "must be even and divide N"),
        (ta.MatmulOp(a1, b16, ex.tensor([1, n]), store=rope(head_dim=48)), "must be even and divide N"),
        (ta.MatmulOp(a1, b16, ex.tensor([1, n]), store=rope(head_dim=hd, pos_base=4)), "does not cover pos_base"),
        (ta.MatmulOp(a1, b16, ex.tensor([1, n]), store=ta.MatmulStore(
            ta.STORE_SCATTER, ta.MatmulStoreDesc(head_dim=hd, pos_base=4, pos_scale=hd, stride_head=4 * hd,
                                                 stride_dim=1), dst=dst)), "out of bounds"),
    ]
    for op, msg in cases:
        with pytest.raises(ta.TensorAshError, match=msg):
            ex.run_ops([op])


# ------------------------------------------------- grouped decode GEMV launches

@pytest.mark.parametrize("form", ["graph", "prepared", "run_ops"])
def test_gemv_groups_match_separate_launches(ta, ex, oracle, monkeypatch, form):
    """A decode layer's one-row GEMVs: q (packed, normed A, RoPE at store),
    k (packed, normed A, RoPE + scatter into a Kt cache at a device position
    cell), v (row-major, normed A, scatter into a V cache), then o (residual)
    beside an independent biased job (ragged N = 1000), the normed SwiGLU
    pair (one dual launch) and down (residual).  Independent neighbours run
    as one grouped launch; every output and cache equals, bit for bit, the
    same ops run one launch per job with no fusion."""
    k, hd, t_max, kvn, ffn = 2048, 64, 16, 256, 1024
    x = ex.tensor_from(oracle.fill_det(k, 64000), shape=[1, k])
    x2 = ex.tensor_from(oracle.fill_det(k, 64001), shape=[1, k])
    norm = ex.tensor_from(oracle.fill_det(k, 64002) * 0.5 + 1.0, shape=[k])
    table = ex.tensor_from(oracle.fill_det(t_max * hd, 64003), shape=[t_max, hd // 2, 2])
    bias = ex.tensor_from(oracle.fill_det(1000, 64004), shape=[1000])
    cell = pos_cell(ex, 3)

    def w(kk, n, seed, packed=False):
        wb, _ = f16_weights(oracle, kk, n, seed)
        return weights_tensor(ta, ex, wb, kk, n, packed)

    wq, wk, wv = w(k, k, 64010, True), w(k, kvn, 64011, True), w(k, kvn, 64012)
    wo, wb, wu, wg, wd = w(k, k, 64013), w(k, 1000, 64014), w(k, ffn, 64015), w(k, ffn, 64016), w(ffn, k, 64017)
    h = kvn // hd
    kt_init = oracle.fill_det(h * hd * t_max, 64020)
    v_init = oracle.fill_det(h * t_max * hd, 64021)

    def run(group):
        if group:
            monkeypatch.delenv("TA_NO_GEMV_GROUP", raising=False)
            monkeypatch.delenv("TA_NO_FUSE", raising=False)
        else:
            monkeypatch.setenv("TA_NO_GEMV_GROUP", "1")
            monkeypatch.setenv("TA_NO_FUSE", "1")
        kt = ex.tensor_from(kt_init, shape=[h, hd, t_max])
        vc = ex.tensor_from(v_init, shape=[h, t_max, hd])
        q, kk_, v, o, bo, up, g, y = (ex.tensor([1, n]) for n in (k, kvn, kvn, k, 1000, ffn, ffn, k))
        nm = dict(normed_a=(norm, EPS))
        E = ta.Epilogue
        ops = [
            ta.MatmulOp(x, wq, q, packed_b=True, store=ta.MatmulStore(
                ta.STORE_ROPE, ta.MatmulStoreDesc(head_dim=hd, pos_base=2, pos_addr=cell.device_address),
                table=table), **nm),
            ta.MatmulOp(x, wk, kk_, packed_b=True, store=ta.MatmulStore(
                ta.STORE_ROPE_SCATTER, ta.MatmulStoreDesc(head_dim=hd, pos_base=2, pos_addr=cell.device_address,
                                                          pos_scale=1, stride_head=hd * t_max, stride_dim=t_max),
                table=table, dst=kt), **nm),
            ta.MatmulOp(x, wv, v, store=ta.MatmulStore(
                ta.STORE_SCATTER, ta.MatmulStoreDesc(head_dim=hd, pos_base=5, pos_scale=hd,
                                                     stride_head=t_max * hd, stride_dim=1), dst=vc), **nm),
            ta.MatmulOp(q, wo, o, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0)),
            ta.MatmulOp(x2, wb, bo, epilogue=E(bias=bias)),
            ta.MatmulOp(o, wu, up, **nm),
            ta.MatmulOp(o, wg, g, epilogue=E(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up), **nm),
            ta.MatmulOp(g, wd, y, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=o, beta=1.0)),
        ]
        outs = (q, kt, vc, o, bo, up, g, y)
        if form == "graph":
            ex.run_op_graph(ops)
        elif form == "prepared":
            p = ex.prepare_op_graph(ops)
            for _ in range(2):
                p.run()
            p.close()
        else:
            # independent ops only (the first three, then the two of the o group)
            ex.run_ops(ops[:3])
            ex.run_ops(ops[3:5])
            outs = outs[:5]
        return [ex.download(t).reshape(-1).copy() for t in outs]

    got, want = run(True), run(False)
    for i, (a, b) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(a, b, err_msg=f"output {i}")
    for a in want:
        assert np.isfinite(a).all() and np.abs(a).max() > 0


@pytest.mark.parametrize("m", [1, 2, 4, 8])
@pytest.mark.parametrize("packed", [True, False])
def test_normed_swiglu_mlp_matches_separate_launches(ta, ex, oracle, monkeypatch, m, packed):
    """The decode layer's MLP with its RMSNorm folded in: up = norm(o) @ Wu,
    h = silu(norm(o) @ Wg) * up, y = h @ Wd + o as one dependent graph (packed
    weights: one decode-MLP launch whose gate/up units normalise o;
    row-major: one dual GEMV launch, then down) gives the bits of the three
    ops run one launch each, and matches the f64 composition on
    the f16-rounded weights within the GEMV tolerance; two MLPs in a row
    where the second is normed again stay two launches.  The decode-MLP
    launch sums the down projection's K in its own 512-row windows, so with
    packed weights the down outputs (and the second MLP, which reads them)
    are held to the GEMV tolerance, as in the un-normed MLP's test."""
    hid, ffn = 2048, 5632
    o_h = oracle.fill_det(m * hid, 65000 + m)
    w_norm = oracle.fill_det(hid, 65001) * 0.5 + 1.0
    (wu, wur), (wg, wgr), (wd, wdr) = (f16_weights(oracle, kk, n, 65010 + i)
                                       for i, (kk, n) in enumerate(((hid, ffn), (hid, ffn), (ffn, hid))))
    o, tw = ex.tensor_from(o_h, shape=[m, hid]), ex.tensor_from(w_norm, shape=[hid])
    tu, tg, td = (weights_tensor(ta, ex, w, kk, n, packed) for w, (kk, n) in
                  ((wu, (hid, ffn)), (wg, (hid, ffn)), (wd, (ffn, hid))))
    E = ta.Epilogue

    def mlp(x, up, h, y):
        nm = dict(normed_a=(tw, EPS), packed_b=packed)
        return [ta.MatmulOp(x, tu, up, **nm),
                ta.MatmulOp(x, tg, h, epilogue=E(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up), **nm),
                ta.MatmulOp(h, td, y, packed_b=packed, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0))]

    def run(fused):
        if fused:
            monkeypatch.delenv("TA_NO_FUSE", raising=False)
        else:
            monkeypatch.setenv("TA_NO_FUSE", "1")
        t = [ex.tensor([m, n]) for n in (ffn, ffn, hid, ffn, ffn, hid)]
        ex.run_op_graph(mlp(o, *t[:3]) + mlp(t[2], *t[3:]))
        return [ex.download(x).reshape(-1).copy() for x in t]

    got, want = run(True), run(False)
    for i, (a, b) in enumerate(zip(got, want)):
        if packed and i >= 2:
            check_f16(a, b, (ffn, hid, hid, ffn)[i - 2], oracle)
        else:
            np.testing.assert_array_equal(a, b, err_msg=f"output {i}")
    xn = oracle.rms_norm_rows(o_h, w_norm, m, hid, EPS)
    up_ref = oracle.cpu_bmm(xn, wur, None, 1, m, ffn, hid)
    h_ref = oracle.epilogue(oracle.cpu_bmm(xn, wgr, None, 1, m, ffn, hid), ffn, m * ffn, act=2, binary=2, d=up_ref)
    y_ref = oracle.epilogue(oracle.cpu_bmm(h_ref, wdr, None, 1, m, hid, ffn), hid, m * hid, binary=1, d=o_h,
                            beta=1.0)
    check_f16(got[1], h_ref, hid, oracle)
    check_f16(got[2], y_ref, ffn, oracle)
