"""a TinyLlama-1.1B-shaped decoder layer prefill (hidden
2048, 32 query heads / 4 KV heads, head_dim 64, FFN 5632, 512 tokens, f16
weights N(0, 0.02), f32 activations).

* The two config-5 GEMMs not covered elsewhere, at full size on the default
  route: O-proj 512x2048x2048 with the +residual epilogue, and the gate
  512x5632x2048 with SiLU * up.  Checked like every f16-MFMA GEMM: to f32
  tolerance against the oracle on f16-rounded A and W (the route rounds A at
  staging), and within 2e-3 normwise against the oracle on the f32 A.
* The whole layer as ONE mixed-op graph (the composition pattern of
  tests/correctness/decoder.rs in the reference): RMSNorm -> QKV GEMM ->
  Q/K/V pack with RoPE -> causal flash attention -> O-proj + residual ->
  RMSNorm -> up, gate*SiLU*up -> down + residual.  Checked against an f64
  composition of the oracle's pinned functions (rms_norm_rows, cpu_bmm,
  rope_tokens / prefill_qkv_pack, flash_attention, the f64 epilogue) on the
  same f16-rounded weights, normwise within 2e-3 (the north star's
  f16-weight bound).  Attention mixes every token, so Q/K/V are checked in
  full, and so is the rest of the layer (its GEMMs on the oracle's
  row-parallel cpu_bmm_rows, bit-identical to cpu_bmm).
"""

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

T, HID, H, HKV, DH, FFN = 512, 2048, 32, 4, 64, 5632
QKV_N = (H + 2 * HKV) * DH  # 2560
EPS = 1e-5


def _f16_mfma_check(got, ha, hb, m, n, k, oracle, **epi):
    """f32 tolerance against the dual-rounded oracle, 2e-3 against f32 A."""
    har, hbr = oracle.round_via_f16(ha), oracle.round_via_f16(hb)
    ref_dual = oracle.reference_gemm(har, hbr, 1, m, n, k, **epi)
    ref = oracle.reference_gemm(ha, hbr, 1, m, n, k, **epi)
    err, idx = oracle.max_abs_err(got.reshape(-1), ref_dual)
    tol = 2 * oracle.tolerance(k) + 1e-4
    assert err <= tol, f"abs err {err} at {idx} > {tol}"
    assert rel_err(got, ref) <= 2e-3


def test_config5_o_proj_residual(ta, ex, oracle):
    m, n, k = T, HID, HID
    ha, hb, hd = oracle.fill_det(m * k, 6101), oracle.fill_normal(k * n, 6102, 0.02), oracle.fill_det(m * n, 6103)
    assert "mfma" in ex.dispatch_info_for(1, m, n, k, True)["kernel"]
    a, b = ex.tensor_from(ha, shape=[m, k]), ex.tensor_from(hb, shape=[k, n], f16=True)
    d, c = ex.tensor_from(hd, shape=[m, n]), ex.tensor([m, n])
    print(f"o-proj {m}x{n}x{k} +residual", flush=True)
    ex.run_ops([ta.MatmulOp(a, b, c, epilogue=ta.Epilogue(binary=ta.BINARY_ADD_SCALED, d=d, beta=1.0))])
    _f16_mfma_check(ex.download(c), ha, hb, m, n, k, oracle, binary=1, d=hd, beta=1.0)


def test_config5_gate_silu_mul_up(ta, ex, oracle):
    m, n, k = T, FFN, HID
    ha = oracle.fill_det(m * k, 6111)
    wg, wu = oracle.fill_normal(k * n, 6112, 0.02), oracle.fill_normal(k * n, 6113, 0.02)
    a = ex.tensor_from(ha, shape=[m, k])
    tg, tu = ex.tensor_from(wg, shape=[k, n], f16=True), ex.tensor_from(wu, shape=[k, n], f16=True)
    up, gate = ex.tensor([m, n]), ex.tensor([m, n])
    print(f"gate {m}x{n}x{k} silu*up", flush=True)
    ex.run_op_graph([ta.MatmulOp(a, tu, up),
                     ta.MatmulOp(a, tg, gate, epilogue=ta.Epilogue(activation=ta.ACTIVATION_SILU,
                                                                   binary=ta.BINARY_MUL, d=up))])
    hup = ex.download(up)
    _f16_mfma_check(hup, ha, wu, m, n, k, oracle)
    # the gate's D is the GPU's own `up`, so both sides multiply the same values
    _f16_mfma_check(ex.download(gate), ha, wg, m, n, k, oracle, act=2, binary=2, d=hup)


def _rope_table():
    half = DH // 2
    inv = 10000.0 ** (-2.0 * np.arange(half) / DH)
    theta = np.arange(T)[:, None] * inv[None, :]
    return np.stack([np.cos(theta), np.sin(theta)], axis=-1).astype(np.float32).reshape(-1)


def _layer_inputs(oracle):
    x = oracle.fill_det(T * HID, 61)
    w = {name: oracle.round_via_f16(oracle.fill_normal(r * c, seed, 0.02)) for name, seed, r, c in [
        ("qkv", 62, HID, QKV_N), ("o", 63, HID, HID), ("gate", 64, HID, FFN), ("up", 65, HID, FFN),
        ("down", 66, FFN, HID)]}
    g1 = (1.0 + 0.1 * oracle.fill_det(HID, 67)).astype(np.float32)
    g2 = (1.0 + 0.1 * oracle.fill_det(HID, 68)).astype(np.float32)
    return x, w, g1, g2, _rope_table()


def _layer_graph(ta, ex, io16, x, w, g1, g2, table):
    """The layer as one list of ExecOps, plus the tensors the check reads."""
    E, MO, Ep = ta.ExecOp, ta.MatmulOp, ta.Epilogue
    dev = {n: ex.tensor_from(v, shape=[HID if n != "down" else FFN, v.size // (HID if n != "down" else FFN)],
                             f16=True) for n, v in w.items()}
    tx = ex.tensor_from(x, shape=[T, HID])
    tg1, tg2 = ex.tensor_from(g1, shape=[HID]), ex.tensor_from(g2, shape=[HID])
    ttab = ex.tensor_from(table, shape=[T, DH // 2, 2])
    t = {n: ex.tensor(s, f16=f16) for n, s, f16 in [
        ("xn", [T, HID], False), ("qkv", [T, QKV_N], False), ("attn", [T, HID], False), ("o", [T, HID], False),
        ("on", [T, HID], False), ("up", [T, FFN], False), ("gate", [T, FFN], False), ("out", [T, HID], False),
        ("kt", [HKV, DH, T], io16), ("v", [HKV, T, DH], io16)]}
    ops = [E.rms_norm(tx, tg1, t["xn"], EPS), E.matmul(MO(t["xn"], dev["qkv"], t["qkv"]))]
    flash = ta.FlashAttentionDesc(T, 0, 1.0 / np.sqrt(DH), out_token_major_heads=H)
    if io16:
        # f16 activations between the QKV GEMM and attention: the reference's
        # prefill pack (flash.rs:255-402) reads f16 QKV rows.
        t["qkv16"], t["q16"], t["attn16"] = (ex.tensor([T, QKV_N], f16=True), ex.tensor([H, T, DH], f16=True),
                                            ex.tensor([T, HID], f16=True))
        ops += [E.copy_strided(t["qkv"], t["qkv16"], ta.CopyDesc((QKV_N, T, 1), (1, QKV_N, 0), (1, QKV_N, 0))),
                E.prefill_qkv_pack(t["qkv16"], ttab, t["q16"], t["kt"], t["v"],
                                   ta.PrefillQkvPackDesc(H, HKV, DH, DH, 0)),
                E.flash_attn(t["q16"], t["kt"], t["v"], t["attn16"], flash),
                E.copy_strided(t["attn16"], t["attn"], ta.CopyDesc((HID, T, 1), (1, HID, 0), (1, HID, 0)))]
    else:
        # f32 throughout: Q and K cut out of the QKV rows and rotated, K
        # rotated straight into the [H_kv, dh, T] cache, V copied into
        # [H_kv, T, dh]; attention reads token-major Q.
        t["q"], t["k"] = ex.tensor([T, HID]), ex.tensor([T, HKV * DH])
        ops += [E.copy_strided(t["qkv"], t["q"], ta.CopyDesc((HID, T, 1), (1, QKV_N, 0), (1, HID, 0))),
                E.copy_strided(t["qkv"], t["k"], ta.CopyDesc((HKV * DH, T, 1), (1, QKV_N, 0), (1, HKV * DH, 0),
                                                             src_offset=HID)),
                E.rope(t["q"], ttab, t["q"], ta.RopeDesc(H, DH, DH, 0)),
                E.rope_scatter(t["k"], ttab, t["kt"], ta.RopeDesc(HKV, DH, DH, 0),
                               ta.RopeScatterDesc(0, (1, DH * T, T))),
                E.copy_strided(t["qkv"], t["v"], ta.CopyDesc((DH, HKV, T), (1, DH, QKV_N), (1, T * DH, DH),
                                                             src_offset=HID + HKV * DH)),
                E.flash_attn(t["q"], t["kt"], t["v"], t["attn"],
                             ta.FlashAttentionDesc(T, 0, 1.0 / np.sqrt(DH), token_major_heads=H,
                                                   out_token_major_heads=H))]
    ops += [
        E.matmul(MO(t["attn"], dev["o"], t["o"], epilogue=Ep(binary=ta.BINARY_ADD_SCALED, d=tx, beta=1.0))),
        E.rms_norm(t["o"], tg2, t["on"], EPS),
        E.matmul(MO(t["on"], dev["up"], t["up"])),
        E.matmul(MO(t["on"], dev["gate"], t["gate"],
                    epilogue=Ep(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=t["up"]))),
        E.matmul(MO(t["gate"], dev["down"], t["out"], epilogue=Ep(binary=ta.BINARY_ADD_SCALED, d=t["o"], beta=1.0))),
    ]
    return ops, t


def _oracle_attention(oracle, qkv, table, io16):
    """Q/K/V formation and causal attention in the oracle; returns the
    token-major attention output [T, HID] and the caches."""
    if io16:
        q, kt, v = oracle.prefill_qkv_pack(oracle.round_via_f16(qkv), table, T, H, HKV, DH, DH, 0,
                                           np.zeros((HKV, DH, T), np.float32), np.zeros((HKV, T, DH), np.float32))
        attn = oracle.flash_attention(q, kt, v, H, HKV, T, T, DH, T, 0, np.float32(1.0 / np.sqrt(DH)))
        attn = oracle.round_via_f16(attn)
    else:
        x = qkv.reshape(T, QKV_N)
        q = oracle.rope_tokens(np.ascontiguousarray(x[:, :HID]).reshape(-1), table, T, H, DH, DH, 0)
        k = oracle.rope_tokens(np.ascontiguousarray(x[:, HID:HID + HKV * DH]).reshape(-1), table, T, HKV, DH, DH, 0)
        q = q.reshape(T, H, DH).transpose(1, 0, 2).copy()
        kt = k.reshape(T, HKV, DH).transpose(1, 2, 0).copy()
        v = x[:, HID + HKV * DH:].reshape(T, HKV, DH).transpose(1, 0, 2).copy()
        attn = oracle.flash_attention(q, kt, v, H, HKV, T, T, DH, T, 0, np.float32(1.0 / np.sqrt(DH)))
    attn = attn.reshape(H, T, DH).transpose(1, 0, 2).reshape(T, HID)
    return attn, kt, v


@pytest.mark.parametrize("io16", [False, True], ids=["f32_activations", "f16_qkv_pack"])
def test_config5_prefill_layer_one_graph(ta, ex, oracle, io16):
    x, w, g1, g2, table = _layer_inputs(oracle)
    ops, t = _layer_graph(ta, ex, io16, x, w, g1, g2, table)
    print(f"config-5 prefill layer graph io16={io16}: {len(ops)} ops", flush=True)
    ex.run_exec_ops(ops)
    got = {n: ex.download(t[n]).reshape(-1) for n in ("qkv", "attn", "o", "out")}

    xn = oracle.rms_norm_rows(x, g1, T, HID, EPS)
    qkv = oracle.cpu_bmm(xn, w["qkv"], None, 1, T, QKV_N, HID)
    assert rel_err(got["qkv"], qkv) <= 2e-3
    # attention from the GPU's own QKV (isolates the attention step) ...
    attn_own, _, _ = _oracle_attention(oracle, got["qkv"], table, io16)
    assert rel_err(got["attn"], attn_own) <= 2e-3
    # ... and the whole layer from the oracle's QKV
    attn, kt, v = _oracle_attention(oracle, qkv, table, io16)
    assert rel_err(got["attn"], attn) <= 2e-3
    np.testing.assert_allclose(ex.download(t["kt"]).reshape(kt.shape), kt, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(ex.download(t["v"]).reshape(v.shape), v, rtol=2e-3, atol=2e-3)

    # The rest of the layer on every row (the oracle's GEMMs row-parallel).
    def gemm(a, b, m, n, k, **epi):
        raw = np.empty(m * n, np.float32)
        oracle.cpu_bmm_rows(a, b, 1, m, n, k, 1.0, raw, 0, m, min(16, oracle.max_threads()))
        return oracle.epilogue(raw, n, m * n, **epi) if epi else raw

    o = gemm(attn.reshape(-1), w["o"], T, HID, HID, binary=1, d=x, beta=1.0)
    on = oracle.rms_norm_rows(o, g2, T, HID, EPS)
    up = gemm(on, w["up"], T, FFN, HID)
    gate = gemm(on, w["gate"], T, FFN, HID, act=2, binary=2, d=up)
    out = gemm(gate, w["down"], T, HID, FFN, binary=1, d=o, beta=1.0)
    assert rel_err(got["o"], o) <= 2e-3
    e = rel_err(got["out"], out)
    assert e <= 2e-3, f"layer output normwise error {e}"
    assert np.all(np.isfinite(got["out"]))


def test_f16_copy_cache_reuse_and_invalidation(ta, ex, oracle):
    """The f16 copies of A a submission's conversion pre-passes leave
    behind: x converted for the first GEMM is reused by a later one after
    another A was converted in between, and an op that overwrites x forces
    a fresh conversion.  Every result equals the same GEMM run alone, bit
    for bit (the copy is the same RNE rounding either way)."""
    m, k, n = 256, 512, 384
    hx, ha2 = oracle.fill_det(m * k, 6201), oracle.fill_det(m * k, 6202)
    w1, w2, w3, w4 = (oracle.fill_normal(k * n, s, 0.02) for s in (6203, 6204, 6205, 6206))
    wx = oracle.fill_normal(k * k, 6207, 0.02)
    x, a2 = ex.tensor_from(hx, shape=[m, k]), ex.tensor_from(ha2, shape=[m, k])
    tw = [ex.tensor_from(w, shape=[k, n], f16=True) for w in (w1, w2, w3, w4)]
    twx = ex.tensor_from(wx, shape=[k, k], f16=True)
    assert "mfma" in ex.dispatch_info_for(1, m, n, k, True)["kernel"]
    c = [ex.tensor([m, n]) for _ in range(4)]

    def alone(a_t, w_t):
        out = ex.tensor([m, n])
        ex.run_ops([ta.MatmulOp(a_t, w_t, out)])
        return ex.download(out)

    print("f16 copy cache: x, a2, x (reuse)", flush=True)
    ex.run_op_graph([ta.MatmulOp(x, tw[0], c[0]), ta.MatmulOp(a2, tw[1], c[1]),
                     ta.MatmulOp(x, tw[2], c[2])])
    want_x2 = alone(x, tw[2])
    np.testing.assert_array_equal(ex.download(c[0]), alone(x, tw[0]))
    np.testing.assert_array_equal(ex.download(c[1]), alone(a2, tw[1]))
    np.testing.assert_array_equal(ex.download(c[2]), want_x2)

    # x overwritten in between (x = a2 @ Wx): the last GEMM must see new x.
    print("f16 copy cache: x, overwrite x, x", flush=True)
    x_b = ex.tensor_from(hx, shape=[m, k])
    ex.run_op_graph([ta.MatmulOp(x_b, tw[0], c[0]), ta.MatmulOp(a2, twx, x_b),
                     ta.MatmulOp(x_b, tw[3], c[3])])
    new_x = ex.download(x_b)
    assert not np.array_equal(new_x.reshape(-1), hx)
    np.testing.assert_array_equal(ex.download(c[3]), alone(x_b, tw[3]))
    ref = oracle.reference_gemm(oracle.round_via_f16(new_x.reshape(-1)), oracle.round_via_f16(w4), 1, m, n, k)
    err, idx = oracle.max_abs_err(ex.download(c[3]).reshape(-1), ref)
    assert err <= 2 * oracle.tolerance(k) + 1e-4, f"abs err {err} at {idx}"


def test_f16_copy_cache_two_swiglu_outputs(ta, ex, oracle):
    """Two SwiGLU triples in one submission, each dual launch leaving the
    f16 copy of its output h for its down projection in the same scratch.
    A later GEMM that reads the first h as A must not be served the second
    h's copy: it equals the same GEMM run alone, bit for bit."""
    m, hid, ffn = 256, 512, 768
    hx = oracle.fill_det(m * hid, 6301)
    x = ex.tensor_from(hx, shape=[m, hid])
    wt = lambda k, n, s: ex.tensor_from(oracle.fill_normal(k * n, s, 0.02), shape=[k, n], f16=True)
    wu1, wg1, wu2, wg2 = (wt(hid, ffn, s) for s in (6302, 6303, 6304, 6305))
    wd1, wd2, wd3 = (wt(ffn, hid, s) for s in (6306, 6307, 6308))
    u1, h1, u2, h2 = (ex.tensor([m, ffn]) for _ in range(4))
    y1, y2, z = (ex.tensor([m, hid]) for _ in range(3))
    E = ta.Epilogue
    ops = [ta.MatmulOp(x, wu1, u1),
           ta.MatmulOp(x, wg1, h1, epilogue=E(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=u1)),
           ta.MatmulOp(h1, wd1, y1),
           ta.MatmulOp(x, wu2, u2),
           ta.MatmulOp(x, wg2, h2, epilogue=E(activation=ta.ACTIVATION_SILU, binary=ta.BINARY_MUL, d=u2)),
           ta.MatmulOp(h2, wd2, y2),
           ta.MatmulOp(h1, wd3, z)]
    print("f16 copy cache: two SwiGLU outputs, first h re-read", flush=True)
    ex.run_op_graph(ops)
    got = {name: ex.download(t).copy() for name, t in (("h1", h1), ("h2", h2), ("y1", y1), ("y2", y2), ("z", z))}
    assert not np.array_equal(got["h1"], got["h2"])

    def alone(a_t, w_t):
        out = ex.tensor([m, hid])
        ex.run_ops([ta.MatmulOp(a_t, w_t, out)])
        return ex.download(out)

    np.testing.assert_array_equal(got["y1"], alone(h1, wd1))
    np.testing.assert_array_equal(got["y2"], alone(h2, wd2))
    np.testing.assert_array_equal(got["z"], alone(h1, wd3))


def test_f16_paired_conversion_skips_produced_inputs(ta, ex, oracle):
    """The two input A's a submission converts up front in one launch are
    the first two that no earlier op writes.  Here the second distinct A
    (y) is produced by the first op, so the pair is x and a2, and y is
    converted when its op runs.  Every result equals the same GEMM run
    alone, bit for bit."""
    m, k, n = 256, 512, 512
    hx, ha2 = oracle.fill_det(m * k, 6401), oracle.fill_det(m * k, 6402)
    w = [ex.tensor_from(oracle.fill_normal(k * n, s, 0.02), shape=[k, n], f16=True)
         for s in (6403, 6404, 6405, 6406)]
    x, a2 = ex.tensor_from(hx, shape=[m, k]), ex.tensor_from(ha2, shape=[m, k])
    y = ex.tensor([m, n])
    c = [ex.tensor([m, n]) for _ in range(3)]
    assert "mfma" in ex.dispatch_info_for(1, m, n, k, True)["kernel"]
    print("paired conversion: x -> y, y, a2, x", flush=True)
    ex.run_op_graph([ta.MatmulOp(x, w[0], y), ta.MatmulOp(y, w[1], c[0]),
                     ta.MatmulOp(a2, w[2], c[1]), ta.MatmulOp(x, w[3], c[2])])

    def alone(a_t, w_t):
        out = ex.tensor([m, n])
        ex.run_ops([ta.MatmulOp(a_t, w_t, out)])
        return ex.download(out)

    want_y = alone(x, w[0])
    np.testing.assert_array_equal(ex.download(y), want_y)
    np.testing.assert_array_equal(ex.download(c[0]), alone(y, w[1]))
    np.testing.assert_array_equal(ex.download(c[1]), alone(a2, w[2]))
    np.testing.assert_array_equal(ex.download(c[2]), alone(x, w[3]))


def test_f16_paired_conversion_batched_inputs(ta, ex, oracle):
    """Paired up-front conversion with batched A (each copy holds
    batch * m * k values): two batched inputs, the first read again by a
    third op, each result equal to the same GEMM run alone, bit for bit."""
    batch, m, k, n = 3, 128, 256, 256
    ha, hb = oracle.fill_det(batch * m * k, 6501), oracle.fill_det(batch * m * k, 6502)
    w = [ex.tensor_from(oracle.fill_normal(k * n, s, 0.02), shape=[k, n], f16=True)
         for s in (6503, 6504, 6505)]
    a, b = ex.tensor_from(ha, shape=[batch, m, k]), ex.tensor_from(hb, shape=[batch, m, k])
    c = [ex.tensor([batch, m, n]) for _ in range(3)]
    assert "mfma" in ex.dispatch_info_for(batch, m, n, k, True)["kernel"]
    print("paired conversion: batched a, b, a", flush=True)
    ex.run_op_graph([ta.MatmulOp(a, w[0], c[0]), ta.MatmulOp(b, w[1], c[1]), ta.MatmulOp(a, w[2], c[2])])

    def alone(a_t, w_t):
        out = ex.tensor([batch, m, n])
        ex.run_ops([ta.MatmulOp(a_t, w_t, out)])
        return ex.download(out)

    np.testing.assert_array_equal(ex.download(c[0]), alone(a, w[0]))
    np.testing.assert_array_equal(ex.download(c[1]), alone(b, w[1]))
    np.testing.assert_array_equal(ex.download(c[2]), alone(a, w[2]))
    # and the copy is the right one: against the oracle on f16-rounded inputs
    wb = oracle.round_via_f16(oracle.fill_normal(k * n, 6504, 0.02))
    ref = np.concatenate([oracle.cpu_bmm(oracle.round_via_f16(hb[i * m * k:(i + 1) * m * k]), wb, None, 1, m, n, k)
                          for i in range(batch)])
    err, idx = oracle.max_abs_err(ex.download(c[1]).reshape(-1), ref)
    assert err <= 2 * oracle.tolerance(k) + 1e-4, f"abs err {err} at {idx}"
