"""A llama-style decoder layer's decode step composed purely from library
ops (tests/correctness/decoder.rs:1-417 of the reference): RMSNorm ->
Q/K/V GEMVs on f16 weights -> RoPE -> KV-cache append (strided copies) ->
masked attention (batched GEMM, prefix softmax, batched GEMM) -> output
projection with fused residual -> RMSNorm -> SwiGLU MLP with fused gating
and residual.  Checked against an f64 composition of the oracle's
functions on the same f16-rounded weights, with the reference's bound of
8x the single-matmul tolerance.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HIDDEN, HEADS, FFN, T_MAX, KV_LEN = 256, 4, 512, 32, 11
DH = HIDDEN // HEADS


def f16_weights(oracle, seed, rows, cols):
    return oracle.round_via_f16(oracle.fill_det(rows * cols, seed) * np.float32(0.125))


def rope_table():
    half = DH // 2
    theta = np.array([[p / 10000.0 ** (2.0 * i / DH) for i in range(half)] for p in range(T_MAX)])
    return np.stack([np.cos(theta), np.sin(theta)], axis=-1).astype(np.float32).reshape(-1)


def matvec(oracle, x, w, k, n):
    return oracle.cpu_bmm(x, w, None, 1, 1, n, k)


@pytest.mark.parametrize("graph", [False, True])
def test_decoder_layer_decode_step(ta, ex, oracle, graph):
    w = {name: f16_weights(oracle, seed, r, c) for name, seed, r, c in [
        ("wq", 3101, HIDDEN, HIDDEN), ("wk", 3102, HIDDEN, HIDDEN), ("wv", 3103, HIDDEN, HIDDEN),
        ("wo", 3104, HIDDEN, HIDDEN), ("w_gate", 3105, HIDDEN, FFN), ("w_up", 3106, HIDDEN, FFN),
        ("w_down", 3107, FFN, HIDDEN)]}
    norm_attn = (1.0 + 0.1 * oracle.fill_det(HIDDEN, 3108)).astype(np.float32)
    norm_mlp = (1.0 + 0.1 * oracle.fill_det(HIDDEN, 3109)).astype(np.float32)
    table = rope_table()
    fill = oracle.fill_det(HEADS * T_MAX * DH, 3200).reshape(HEADS, T_MAX, DH)
    kt0 = np.zeros((HEADS, DH, T_MAX), np.float32)
    v0 = np.zeros((HEADS, T_MAX, DH), np.float32)
    for step in range(KV_LEN):
        kt0[:, :, step] = fill[:, step, :] * np.float32(0.25)
        v0[:, step, :] = fill[:, T_MAX - 1 - step, :] * np.float32(0.25)
    host_x = oracle.fill_det(HIDDEN, 3201)

    dev = {name: ex.tensor_from(val, shape=[r, c], f16=True) for (name, val), (r, c) in zip(
        w.items(), [(HIDDEN, HIDDEN)] * 4 + [(HIDDEN, FFN), (HIDDEN, FFN), (FFN, HIDDEN)])}
    t_norm_attn, t_norm_mlp = ex.tensor_from(norm_attn, shape=[HIDDEN]), ex.tensor_from(norm_mlp, shape=[HIDDEN])
    t_table = ex.tensor_from(table, shape=[T_MAX, DH // 2, 2])
    kt_cache = ex.tensor_from(kt0, shape=[HEADS, DH, T_MAX])
    v_cache = ex.tensor_from(v0, shape=[HEADS, T_MAX, DH])
    x = ex.tensor_from(host_x, shape=[1, HIDDEN])
    t = {name: ex.tensor(shape) for name, shape in [
        ("xn", [1, HIDDEN]), ("q", [1, HIDDEN]), ("k", [1, HIDDEN]), ("v", [1, HIDDEN]),
        ("scores", [HEADS, 1, T_MAX]), ("attn", [HEADS, 1, DH]), ("q_heads", [HEADS, 1, DH]),
        ("attn_flat", [1, HIDDEN]), ("o", [1, HIDDEN]), ("on", [1, HIDDEN]), ("up", [1, FFN]),
        ("gated", [1, FFN]), ("out", [1, HIDDEN])]}

    def step():
        ex.rms_norm(x, t_norm_attn, t["xn"], 1e-5)
        for wt, out in (("wq", "q"), ("wk", "k"), ("wv", "v")):
            ex.matmul(t["xn"], dev[wt], t[out])
        ex.rope(t["q"], t_table, t["q"], HEADS, DH, DH, KV_LEN)
        ex.rope(t["k"], t_table, t["k"], HEADS, DH, DH, KV_LEN)
        ex.copy_strided(t["k"], kt_cache, (DH, HEADS, 1), (1, DH, 0), (T_MAX, DH * T_MAX, 0), dst_offset=KV_LEN)
        ex.copy_strided(t["v"], v_cache, (DH, HEADS, 1), (1, DH, 0), (1, T_MAX * DH, 0), dst_offset=KV_LEN * DH)
        ex.copy_strided(t["q"], t["q_heads"], (HIDDEN, 1, 1), (1, 0, 0), (1, 0, 0))
        ex.matmul(t["q_heads"], kt_cache, t["scores"])
        ex.softmax_rows(t["scores"], t["scores"], 1.0 / np.sqrt(DH), mask_kind=1, valid_or_prefix=KV_LEN + 1)
        ex.matmul(t["scores"], v_cache, t["attn"])
        ex.copy_strided(t["attn"], t["attn_flat"], (HIDDEN, 1, 1), (1, 0, 0), (1, 0, 0))
        ex.run_ops([ta.MatmulOp(t["attn_flat"], dev["wo"], t["o"],
                                epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0))])
        ex.rms_norm(t["o"], t_norm_mlp, t["on"], 1e-5)
        ex.matmul(t["on"], dev["w_up"], t["up"])
        ex.run_ops([ta.MatmulOp(t["on"], dev["w_gate"], t["gated"],
                                epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL,
                                                     d=t["up"]))])
        ex.run_ops([ta.MatmulOp(t["gated"], dev["w_down"], t["out"],
                                epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=t["o"], beta=1.0))])

    if graph:
        # The same layer as one recorded graph of mixed ops.
        ops = mixed_ops(ta, ex, x, t, dev, t_norm_attn, t_norm_mlp, t_table, kt_cache, v_cache)
        ex.run_exec_ops(ops)
    else:
        step()
    gpu = ex.download(t["out"]).reshape(-1)

    # f64 composition of the oracle's functions (decoder.rs:337-405).
    xn = oracle.rms_norm_rows(host_x, norm_attn, 1, HIDDEN, 1e-5)
    q, k, v = (matvec(oracle, xn, w[n], HIDDEN, HIDDEN) for n in ("wq", "wk", "wv"))
    q = oracle.rope_tokens(q, table, 1, HEADS, DH, DH, KV_LEN)
    k = oracle.rope_tokens(k, table, 1, HEADS, DH, DH, KV_LEN)
    kt, vc = kt0.copy(), v0.copy()
    kt[:, :, KV_LEN] = k.reshape(HEADS, DH)
    vc[:, KV_LEN, :] = v.reshape(HEADS, DH)
    valid = KV_LEN + 1
    attn = np.zeros((HEADS, DH))
    for h in range(HEADS):
        s = q.reshape(HEADS, DH)[h].astype(np.float64) @ kt[h, :, :valid].astype(np.float64) / np.sqrt(DH)
        p = np.exp(s - s.max())
        attn[h] = (p / p.sum()) @ vc[h, :valid, :].astype(np.float64)
    o = matvec(oracle, attn.astype(np.float32).reshape(-1), w["wo"], HIDDEN, HIDDEN) + host_x
    on = oracle.rms_norm_rows(o, norm_mlp, 1, HIDDEN, 1e-5)
    up = matvec(oracle, on, w["w_up"], HIDDEN, FFN)
    gate = matvec(oracle, on, w["w_gate"], HIDDEN, FFN).astype(np.float64)
    gated = (gate / (1.0 + np.exp(-gate)) * up).astype(np.float32)
    ref = matvec(oracle, gated, w["w_down"], FFN, HIDDEN) + o
    err, idx = oracle.max_abs_err(gpu, ref)
    assert err <= 8 * oracle.tolerance(HIDDEN), f"decoder layer error {err} at {idx}"
    # the caches now hold the appended step
    assert np.array_equal(ex.download(kt_cache).reshape(HEADS, DH, T_MAX)[:, :, :KV_LEN], kt0[:, :, :KV_LEN])


def mixed_ops(ta, ex, x, t, dev, norm_attn, norm_mlp, table, kt_cache, v_cache):
    E = ta.ExecOp
    copy = ta.CopyDesc
    return [
        E.rms_norm(x, norm_attn, t["xn"], 1e-5),
        E.matmul(ta.MatmulOp(t["xn"], dev["wq"], t["q"])),
        E.matmul(ta.MatmulOp(t["xn"], dev["wk"], t["k"])),
        E.matmul(ta.MatmulOp(t["xn"], dev["wv"], t["v"])),
        E.rope(t["q"], table, t["q"], ta.RopeDesc(HEADS, DH, DH, KV_LEN)),
        E.rope(t["k"], table, t["k"], ta.RopeDesc(HEADS, DH, DH, KV_LEN)),
        E.copy_strided(t["k"], kt_cache, copy((DH, HEADS, 1), (1, DH, 0), (T_MAX, DH * T_MAX, 0), 0, KV_LEN)),
        E.copy_strided(t["v"], v_cache, copy((DH, HEADS, 1), (1, DH, 0), (1, T_MAX * DH, 0), 0, KV_LEN * DH)),
        E.copy_strided(t["q"], t["q_heads"], copy((HIDDEN, 1, 1), (1, 0, 0), (1, 0, 0))),
        E.matmul(ta.MatmulOp(t["q_heads"], kt_cache, t["scores"])),
        E.softmax_rows(t["scores"], t["scores"], 1.0 / np.sqrt(DH), ta.SOFTMAX_MASK_PREFIX, KV_LEN + 1),
        E.matmul(ta.MatmulOp(t["scores"], v_cache, t["attn"])),
        E.copy_strided(t["attn"], t["attn_flat"], copy((HIDDEN, 1, 1), (1, 0, 0), (1, 0, 0))),
        E.matmul(ta.MatmulOp(t["attn_flat"], dev["wo"], t["o"],
                             epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=x, beta=1.0))),
        E.rms_norm(t["o"], norm_mlp, t["on"], 1e-5),
        E.matmul(ta.MatmulOp(t["on"], dev["w_up"], t["up"])),
        E.matmul(ta.MatmulOp(t["on"], dev["w_gate"], t["gated"],
                             epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=t["up"]))),
        E.matmul(ta.MatmulOp(t["gated"], dev["w_down"], t["out"],
                             epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=t["o"], beta=1.0))),
    ]
