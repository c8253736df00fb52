"""The remaining model ops of the reference's mixed-op graphs: the binary
combine, RoPE scattered into a KV cache, and the f16 prefill QKV pack
(tests/correctness/elementwise.rs:526-558, 668-697 and fusion.rs:250-345,
346-535, 537-620), through the C ABI against the CPU oracle.

Bars: rope-scatter and the QKV pack are bit-exact (same rotation and
rounding as the oracle and as the composed rope + copy path); the binary
combine is within 1e-6 (add) / 1e-5 (SiLU) of the f64 oracle, and its f16
form equals the f32 form rounded to f16.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_binary_add_scaled_and_silu_mul(ta, ex, oracle):
    n = 4099  # not a multiple of 4: the tail
    ha, hb = oracle.fill_det(n, 7100), oracle.fill_det(n, 7101)
    a, b, out = ex.tensor_from(ha, shape=[n]), ex.tensor_from(hb, shape=[n]), ex.tensor([n])
    ex.binary(a, b, out, ta.BINARY_OP_ADD_SCALED, 0.5)
    assert np.abs(ex.download(out) - oracle.binary_combine(ha, hb, 0, 0.5)).max() <= 1e-6
    ex.binary(a, b, a, ta.BINARY_OP_SILU_MUL)  # in place
    assert np.abs(ex.download(a) - oracle.binary_combine(ha, hb, 1)).max() <= 1e-5


def test_binary_f16_matches_narrowed_f32(ta, ex, oracle):
    n = 4099
    ha = oracle.round_via_f16(oracle.fill_det(n, 6300))
    hb = oracle.round_via_f16(oracle.fill_det(n, 6301))
    a16, b16 = ex.tensor_from(ha, shape=[n], f16=True), ex.tensor_from(hb, shape=[n], f16=True)
    a32, b32 = ex.tensor_from(ha, shape=[n]), ex.tensor_from(hb, shape=[n])
    for op, beta in ((ta.BINARY_OP_ADD_SCALED, 0.5), (ta.BINARY_OP_SILU_MUL, 0.0)):
        o16, o32 = ex.tensor([n], f16=True), ex.tensor([n])
        ex.binary(a16, b16, o16, op, beta)
        ex.binary(a32, b32, o32, op, beta)
        assert np.array_equal(ex.download(o16), oracle.round_via_f16(ex.download(o32)))
    with pytest.raises(ta.TensorAshError, match="must match a"):
        ex.binary(a16, b32, ex.tensor([n], f16=True), ta.BINARY_OP_SILU_MUL)
    with pytest.raises(ta.TensorAshError, match="element counts differ"):
        ex.binary(a32, ex.tensor([n - 1]), ex.tensor([n]), ta.BINARY_OP_ADD_SCALED, 1.0)


@pytest.mark.parametrize("kv_f16", [False, True])
def test_rope_scatter_matches_rope_plus_copy(ta, ex, oracle, kv_f16):
    """fusion.rs:250-329: partial rotary, a warm pos_base; the fused op equals
    rope + strided copy bit for bit, and the oracle."""
    tokens, heads, dh, rot, t_max, pos = 3, 2, 8, 6, 16, 5
    hx = oracle.fill_det(tokens * heads * dh, 41000)
    htab = oracle.fill_det(t_max * rot, 41001)
    x, table = ex.tensor_from(hx, shape=[tokens, heads * dh]), ex.tensor_from(htab, shape=[t_max, rot // 2, 2])
    poison = np.full(heads * dh * t_max, 7.0, np.float32)
    ref = ex.tensor_from(poison, shape=[heads, dh, t_max], f16=kv_f16)
    fused = ex.tensor_from(poison, shape=[heads, dh, t_max], f16=kv_f16)
    desc = ta.RopeDesc(heads, dh, rot, pos)
    roped = ex.tensor([tokens, heads * dh])
    ex.rope(x, table, roped, heads, dh, rot, pos)
    ex.copy_strided(roped, ref, (dh, heads, tokens), (1, dh, heads * dh), (t_max, dh * t_max, 1), dst_offset=pos)
    ex.rope_scatter(x, table, fused, desc, ta.RopeScatterDesc(pos, (1, dh * t_max, t_max)))
    got = ex.download(fused).reshape(-1)
    assert np.array_equal(got, ex.download(ref).reshape(-1))
    want = oracle.rope_scatter(hx, htab, tokens, heads, dh, rot, pos, poison, pos, (1, dh * t_max, t_max), kv_f16)
    assert np.array_equal(got, want)


def test_rope_scatter_graph_with_position_cell_and_bounds(ta, ex, oracle):
    """fusion.rs:537-620: the decode k-rope + Kt append as one graph op,
    replayed at new positions through a position cell; a destination past
    the cache is rejected."""
    heads, dh, rot, t_max = 4, 16, 16, 32
    htab = oracle.fill_det(t_max * rot, 43001)
    table = ex.tensor_from(htab, shape=[t_max, rot // 2, 2])
    x = ex.tensor([1, heads * dh])
    cache = ex.tensor_from(np.zeros(heads * dh * t_max, np.float32), shape=[heads, dh, t_max])
    pos = ex.create_pos_buffer()
    op = ta.ExecOp.rope_scatter(x, table, cache, ta.RopeDesc(heads, dh, rot, 0, pos.device_address),
                                ta.RopeScatterDesc(0, (1, dh * t_max, t_max), pos_scale=1))
    prep = ex.prepare_exec_ops([op])
    want = np.zeros(heads * dh * t_max, np.float32)
    for p in (0, 7, 31):
        hx = oracle.fill_det(heads * dh, 43100 + p)
        ex.upload(x, hx)
        pos.set(p)
        prep.run()
        want = oracle.rope_scatter(hx, htab, 1, heads, dh, rot, p, want, p, (1, dh * t_max, t_max))
        assert np.array_equal(ex.download(cache).reshape(-1), want), f"pos {p}"
    prep.close()
    with pytest.raises(ta.TensorAshError, match="destination access reaches element"):
        ex.rope_scatter(x, table, cache, ta.RopeDesc(heads, dh, rot, 0),
                        ta.RopeScatterDesc(t_max, (1, dh * t_max, t_max)))
    with pytest.raises(ta.TensorAshError, match="must be different tensors"):
        ex.rope_scatter(x, table, x, ta.RopeDesc(heads, dh, rot, 0), ta.RopeScatterDesc(0, (1, 1, 1)))


@pytest.mark.parametrize("graph", [False, True])
def test_prefill_qkv_pack(ta, ex, oracle, graph):
    """fusion.rs:346-535: GQA, a warm pos_base and partial rotary; Q, the Kt
    columns and the V rows equal the oracle bit for bit and the rest of the
    caches is untouched."""
    tokens, heads, kvh, dh, rot, pos, t_max = 37, 8, 2, 64, 48, 9, 64
    n = heads * dh + 2 * kvh * dh
    hqkv = oracle.round_via_f16(oracle.fill_det(tokens * n, 44000))
    htab = oracle.fill_det(t_max * rot, 44001)
    kt0 = oracle.round_via_f16(oracle.fill_det(kvh * dh * t_max, 44002)).reshape(kvh, dh, t_max)
    v0 = oracle.round_via_f16(oracle.fill_det(kvh * t_max * dh, 44003)).reshape(kvh, t_max, dh)
    qkv = ex.tensor_from(hqkv, shape=[tokens, n], f16=True)
    table = ex.tensor_from(htab, shape=[t_max, rot // 2, 2])
    q = ex.tensor([heads, tokens, dh], f16=True)
    kt = ex.tensor_from(kt0, shape=[kvh, dh, t_max], f16=True)
    v = ex.tensor_from(v0, shape=[kvh, t_max, dh], f16=True)
    desc = ta.PrefillQkvPackDesc(heads, kvh, dh, rot, pos)
    if graph:
        ex.run_exec_ops([ta.ExecOp.prefill_qkv_pack(qkv, table, q, kt, v, desc)])
    else:
        ex.prefill_qkv_pack(qkv, table, q, kt, v, desc)
    wq, wkt, wv = oracle.prefill_qkv_pack(hqkv, htab, tokens, heads, kvh, dh, rot, pos, kt0, v0)
    assert np.array_equal(ex.download(q).reshape(wq.shape), wq)
    assert np.array_equal(ex.download(kt).reshape(wkt.shape), wkt)
    assert np.array_equal(ex.download(v).reshape(wv.shape), wv)


def test_prefill_qkv_pack_rejects_bad_geometry(ta, ex):
    desc = ta.PrefillQkvPackDesc(2, 1, 8, 8, 0)
    qkv, table = ex.tensor([4, 32], f16=True), ex.tensor([16, 4, 2])
    q, kt, v = ex.tensor([2, 4, 8], f16=True), ex.tensor([1, 8, 16], f16=True), ex.tensor([1, 16, 8], f16=True)
    with pytest.raises(ta.TensorAshError, match="qkv must be f16 storage"):
        ex.prefill_qkv_pack(ex.tensor([4, 32]), table, q, kt, v, desc)
    with pytest.raises(ta.TensorAshError, match="qkv N 32 != H\\*dh \\+ 2\\*H_kv\\*dh \\(32\\)|qkv N"):
        ex.prefill_qkv_pack(ex.tensor([4, 30], f16=True), table, q, kt, v, desc)
    with pytest.raises(ta.TensorAshError, match="exceeds T_max"):
        ex.prefill_qkv_pack(qkv, table, q, kt, v, ta.PrefillQkvPackDesc(2, 1, 8, 8, 13))
    with pytest.raises(ta.TensorAshError, match="invalid heads/kv_heads/dh/rot_dim"):
        ex.prefill_qkv_pack(qkv, table, q, kt, v, ta.PrefillQkvPackDesc(2, 1, 8, 3, 0))


# ---------------------------------------------------------------- GEMV chain

def _chain_ops(ta, x, attn, wo, w_up, w_gate, w_down, norm, o, up, gate, out):
    E = ta.Epilogue
    return [
        ta.MatmulOp(attn, wo, o, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0)),
        ta.MatmulOp(o, w_up, up, normed_a=(norm, 1e-5)),
        ta.MatmulOp(o, w_gate, gate, epilogue=E(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=up),
                    normed_a=(norm, 1e-5)),
        ta.MatmulOp(gate, w_down, out, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=o, beta=1.0)),
    ]


@pytest.mark.parametrize("persistent", [True, False])
def test_gemv_chain_mlp_matches_composed_graph(ta, ex, oracle, monkeypatch, persistent):
    """gemv_chain.rs:41-143: o-proj + normed SwiGLU MLP as one GEMV chain (and as
    a graph op) gives the composed graph's bits, as one persistent launch
    (ML_DEVICE_SCOPE=1) and as list-order launches."""
    if persistent:
        monkeypatch.setenv("ML_DEVICE_SCOPE", "1")
    else:
        monkeypatch.delenv("ML_DEVICE_SCOPE", raising=False)
    k, n_o, n_ff = 256, 256, 384
    f16w = lambda r, c, seed: ex.tensor_from(oracle.fill_det(r * c, seed), shape=[r, c], f16=True)
    x = ex.tensor_from(oracle.fill_det(k, 1), shape=[1, k])
    attn = ex.tensor_from(oracle.fill_det(k, 2), shape=[1, k])
    wo, w_up, w_gate, w_down = f16w(k, n_o, 3), f16w(n_o, n_ff, 4), f16w(n_o, n_ff, 5), f16w(n_ff, n_o, 6)
    norm = ex.tensor_from(oracle.fill_det(n_o, 7), shape=[n_o])
    bufs = lambda: (ex.tensor([1, n_o]), ex.tensor([1, n_ff]), ex.tensor([1, n_ff]), ex.tensor([1, n_o]))
    composed, chained, graphed = bufs(), bufs(), bufs()
    ex.run_exec_ops([ta.ExecOp.matmul(op) for op in
                     _chain_ops(ta, x, attn, wo, w_up, w_gate, w_down, norm, *composed)])
    st = ex.run_gemv_chain(_chain_ops(ta, x, attn, wo, w_up, w_gate, w_down, norm, *chained))
    assert st.n_calls == 4
    ex.run_exec_ops([ta.ExecOp.gemv_chain(_chain_ops(ta, x, attn, wo, w_up, w_gate, w_down, norm, *graphed))])
    want = ex.download(composed[3])
    assert np.array_equal(ex.download(chained[3]), want)
    assert np.array_equal(ex.download(graphed[3]), want)


@pytest.mark.parametrize("persistent", [True, False])
def test_gemv_chain_persistent_groups_and_windows(ta, ex, oracle, monkeypatch, persistent):
    """A chain with independent neighbours (one group: q, k, v reading the
    same x), dependent jobs (grid barriers), ragged N (1000 = 15 full
    64-column tiles + 40), deep K (several K windows per tile, reduced in
    window order) and normed-A, as one persistent launch (ML_DEVICE_SCOPE=1)
    and as list-order launches: every output equals the same ops run as
    separate launches, and repeated launches (self-resetting barrier) and a
    prepared graph's replays repeat the bits."""
    if persistent:
        monkeypatch.setenv("ML_DEVICE_SCOPE", "1")
    else:
        monkeypatch.delenv("ML_DEVICE_SCOPE", raising=False)
    k, kd = 2048, 4096
    f16w = lambda r, c, seed: ex.tensor_from(oracle.fill_normal(r * c, seed, 0.05), shape=[r, c], f16=True)
    x = ex.tensor_from(oracle.fill_det(k, 11), shape=[1, k])
    norm = ex.tensor_from(oracle.fill_det(k, 12), shape=[k])
    wq, wk, wv = f16w(k, 2048, 13), f16w(k, 1000, 14), f16w(k, 256, 15)
    w2 = f16w(2048, kd, 16)
    w3 = f16w(kd, 512, 17)
    res = ex.tensor_from(oracle.fill_det(512, 18), shape=[1, 512])
    E = ta.Epilogue

    def ops(q, kk, v, h, out):
        return [ta.MatmulOp(x, wq, q, normed_a=(norm, 1e-5)),
                ta.MatmulOp(x, wk, kk, alpha=0.5),
                ta.MatmulOp(x, wv, v, epilogue=E(activation=ta.ACTIVATION_SILU)),
                ta.MatmulOp(q, w2, h, epilogue=E(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL,
                                                 d=ex.tensor_from(oracle.fill_det(kd, 19), shape=[1, kd]))),
                ta.MatmulOp(h, w3, out, epilogue=E(binary=ta.BINARY_ADD_SCALED, d=res, beta=0.75))]

    shapes = [[1, 2048], [1, 1000], [1, 256], [1, kd], [1, 512]]
    chained = [ex.tensor(s_) for s_ in shapes]
    composed = [ex.tensor(s_) for s_ in shapes]
    st = ex.run_gemv_chain(ops(*chained))
    assert st.n_calls == 5
    ex.run_exec_ops([ta.ExecOp.matmul(op) for op in ops(*composed)])
    first = [ex.download(t).copy() for t in chained]
    for got, want in zip(first, composed):
        np.testing.assert_array_equal(got, ex.download(want))
    for _ in range(5):
        for t in chained:
            ex.upload(t, np.zeros(ex.download(t).size, np.float32))
        ex.run_gemv_chain(ops(*chained))
        for t, want in zip(chained, first):
            np.testing.assert_array_equal(ex.download(t), want)
    # as a graph op inside a prepared exec graph, replayed
    graphed = [ex.tensor(s_) for s_ in shapes]
    p = ex.prepare_exec_ops([ta.ExecOp.gemv_chain(ops(*graphed))])
    for _ in range(3):
        for t in graphed:
            ex.upload(t, np.zeros(ex.download(t).size, np.float32))
        p.run()
        for t, want in zip(graphed, first):
            np.testing.assert_array_equal(ex.download(t), want)
    p.close()


def test_gemv_chain_single_job_and_rejections(ta, ex, oracle):
    """gemv_chain.rs:145-175 (one job against the f64 CPU product) and the
    job rules of pack_gemv_job (gemv_chain.rs:106-179)."""
    k, n = 128, 96
    ha, hb = oracle.fill_det(k, 11), oracle.fill_det(k * n, 12)
    a, b, c = ex.tensor_from(ha, shape=[1, k]), ex.tensor_from(hb, shape=[k, n], f16=True), ex.tensor([1, n])
    ex.run_gemv_chain([ta.MatmulOp(a, b, c)])
    ref = oracle.cpu_bmm(ha, oracle.round_via_f16(hb), None, 1, 1, n, k)
    assert np.abs(ex.download(c).reshape(-1) - ref).max() <= oracle.tolerance(k)
    with pytest.raises(ta.TensorAshError, match="9 jobs exceeds max 8"):
        ex.run_gemv_chain([ta.MatmulOp(a, b, c)] * 9)
    with pytest.raises(ta.TensorAshError, match="B must be f16 storage"):
        ex.run_gemv_chain([ta.MatmulOp(a, ex.tensor([k, n]), c)])
    with pytest.raises(ta.TensorAshError, match="requires batch=1 M=1"):
        ex.run_gemv_chain([ta.MatmulOp(ex.tensor([2, k]), b, ex.tensor([2, n]))])
    with pytest.raises(ta.TensorAshError, match="bias epilogue is not supported"):
        ex.run_gemv_chain([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(bias=ex.tensor([n])))])
    with pytest.raises(ta.TensorAshError, match="unsupported activation"):
        ex.run_gemv_chain([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(activation=ta.ACTIVATION_GELU))])
    with pytest.raises(ta.TensorAshError, match="cannot combine with (the )?AddScaled"):
        ex.run_gemv_chain([ta.MatmulOp(a, b, c, normed_a=(ex.tensor([k]), 1e-5),
                                       epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=c, beta=1.0))])
    with pytest.raises(ta.TensorAshError, match="empty job list"):
        ex.run_gemv_chain([])
