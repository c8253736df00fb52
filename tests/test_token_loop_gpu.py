"""The GPU token loop: greedy argmax, embedding gather and split-K decode
attention (tests/correctness/token_loop.rs and attn_decode.rs of the
reference), through the C ABI, against the CPU oracle.

Bars: argmax and gather are exact (index / copied bits); decode attention
is within 1e-4 of the f64 oracle (attn_decode.rs:166-170, the same bound
for f16 caches, whose rounded values the oracle sees) and within 1e-5 of
the composed scores / softmax / PV path.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

KV_HEADS, GROUP, T_MAX = 4, 8, 2048


# ---------------------------------------------------------------- argmax

@pytest.mark.parametrize("n,seed", [(1, 7101), (255, 7102), (257, 7103), (32000, 7104), (131075, 7105)])
def test_argmax_matches_oracle_across_sizes(ta, ex, oracle, n, seed):
    host = oracle.fill_det(n, seed)
    t = ex.tensor_from(host, shape=[1, n])
    cell = ex.create_host_u32_buffer()
    ex.argmax(t, cell)
    assert cell.read() == oracle.argmax_last(host)


def test_argmax_tie_break(ta, ex, oracle):
    """token_loop.rs:45-95: the last maximum wins."""
    n = 32000
    t = ex.tensor([1, n])
    cell = ex.create_host_u32_buffer()
    cases = [np.full(n, 1.5, np.float32)]
    x = oracle.fill_det(n, 7201)
    x[5] = x[20000] = 1.0e6
    cases.append(x)
    x = np.full(n, -2.0, np.float32)
    x[0] = 3.0
    cases.append(x)
    cases.append(np.full(n, -np.inf, np.float32))
    for host, want in zip(cases, [n - 1, 20000, 0, n - 1]):
        ex.upload(t, host)
        ex.argmax(t, cell)
        assert cell.read() == want == oracle.argmax_last(host)


def test_argmax_rejects_bad_inputs(ta, ex):
    cell = ex.create_host_u32_buffer()
    with pytest.raises(ta.TensorAshError, match="must be f32"):
        ex.argmax(ex.tensor([1, 16], f16=True), cell)


# ---------------------------------------------------------------- gather

def test_embed_gather_f32_and_f16_tables(ta, ex, oracle):
    """token_loop.rs:97-142: exact rows; f16 tables widen exactly; ids past
    the vocabulary clamp to the last row."""
    vocab, embd = 301, 320
    host = oracle.fill_det(vocab * embd, 7301)
    t32 = ex.tensor_from(host, shape=[vocab, embd])
    t16 = ex.tensor_from(host, shape=[vocab, embd], f16=True)
    out = ex.tensor([1, embd])
    token = ex.create_host_u32_buffer()
    for tok in (0, 7, vocab - 1, vocab + 100):
        token.set(tok)
        ex.embed_gather(token, t32, out)
        assert np.array_equal(ex.download(out).reshape(-1), oracle.embed_gather(host, vocab, embd, [tok]))
        ex.embed_gather(token, t16, out)
        assert np.array_equal(ex.download(out).reshape(-1),
                              oracle.embed_gather(oracle.round_via_f16(host), vocab, embd, [tok]))


@pytest.mark.parametrize("embd", [128, 130])
def test_embed_gather_rows(ta, ex, oracle, embd):
    """token_loop.rs:144-187: a prefill's t rows from a token-id list, f32
    and f16 destinations (and a row width that is not a multiple of 4)."""
    vocab, t = 64, 8
    host = oracle.fill_det(vocab * embd, 7601)
    ids = [(i * 7 + 3) % vocab for i in range(t)]
    tokens = ex.create_token_id_buffer(t)
    tokens.write(ids)
    t32 = ex.tensor_from(host, shape=[vocab, embd])
    out32, out16 = ex.tensor([t, embd]), ex.tensor([t, embd], f16=True)
    ex.embed_gather_rows(tokens, t32, out32)
    assert np.array_equal(ex.download(out32).reshape(-1), oracle.embed_gather(host, vocab, embd, ids))
    t16 = ex.tensor_from(host, shape=[vocab, embd], f16=True)
    ex.embed_gather_rows(tokens, t16, out16)
    assert np.array_equal(ex.download(out16).reshape(-1),
                          oracle.embed_gather(oracle.round_via_f16(host), vocab, embd, ids, out_f16=True))


def test_embed_gather_rejects_bad_geometry(ta, ex):
    table = ex.tensor([10, 16])
    token = ex.create_host_u32_buffer()
    with pytest.raises(ta.TensorAshError, match="must be \\[embd\\] or \\[t, embd\\]"):
        ex.embed_gather(token, table, ex.tensor([1, 8]))
    with pytest.raises(ta.TensorAshError, match="token buffer 4 B < 12 B for 3 ids"):
        ex.embed_gather(token, table, ex.tensor([3, 16]))
    with pytest.raises(ta.TensorAshError, match="exceeds cap"):
        token.write([1, 2])


# ---------------------------------------------------------------- decode tail as a graph

def test_exec_chain_matmul_argmax_gather(ta, ex, oracle):
    """token_loop.rs:189-241: lm-head matmul -> argmax -> gather as one
    graph matches the stepwise ops and the CPU sampler + gather."""
    embd, vocab = 256, 1000
    hx, hw, htab = (oracle.fill_det(embd, 7401), oracle.fill_det(embd * vocab, 7402),
                    oracle.fill_det(vocab * embd, 7403))
    x, w, table = ex.tensor_from(hx, shape=[1, embd]), ex.tensor_from(hw, shape=[embd, vocab]), \
        ex.tensor_from(htab, shape=[vocab, embd])
    logits, next_x = ex.tensor([1, vocab]), ex.tensor([1, embd])
    token = ex.create_host_u32_buffer()
    E = ta.ExecOp
    ex.run_exec_ops([E.matmul(ta.MatmulOp(x, w, logits)), E.argmax(logits, token),
                     E.embed_gather(token, table, next_x)])
    chained = token.read()
    ex.matmul(x, w, logits)
    want = oracle.argmax_last(ex.download(logits).reshape(-1))
    assert chained == want
    assert np.array_equal(ex.download(next_x).reshape(-1), oracle.embed_gather(htab, vocab, embd, [want]))


def test_prepared_argmax_gather_replays(ta, ex, oracle):
    """token_loop.rs:243-266: one recording, new logits between replays."""
    vocab, embd = 500, 64
    htab = oracle.fill_det(vocab * embd, 7501)
    table = ex.tensor_from(htab, shape=[vocab, embd])
    logits, out = ex.tensor([1, vocab]), ex.tensor([1, embd])
    token = ex.create_host_u32_buffer()
    prep = ex.prepare_exec_ops([ta.ExecOp.argmax(logits, token), ta.ExecOp.embed_gather(token, table, out)])
    for seed in (7502, 7503, 7504):
        hl = oracle.fill_det(vocab, seed)
        ex.upload(logits, hl)
        prep.run()
        want = oracle.argmax_last(hl)
        assert token.read() == want
        assert np.array_equal(ex.download(out).reshape(-1), oracle.embed_gather(htab, vocab, embd, [want]))
    prep.close()


# ---------------------------------------------------------------- decode attention

def make_caches(oracle, kv_len, f16, dh, poison=True):
    """attn_decode.rs:59-93: the kv_len prefix holds data (f16-rounded for f16
    caches), the tail 1e30 (+inf once stored as f16) unless poison is off."""
    fill = oracle.fill_det(KV_HEADS * dh * T_MAX, 7301)
    kt = np.full((KV_HEADS, dh, T_MAX), 1.0e30 if poison else 0.0, np.float32)
    v = np.full((KV_HEADS, T_MAX, dh), 1.0e30 if poison else 0.0, np.float32)
    h, d, p = np.meshgrid(np.arange(KV_HEADS), np.arange(dh), np.arange(kv_len), indexing="ij")
    kt_idx = (h * dh + d) * T_MAX + p
    v_idx = (h * T_MAX + p) * dh + d
    kt[h, d, p] = fill[kt_idx % fill.size]
    v[h, p, d] = fill[(v_idx * 7 + 3) % fill.size]
    if f16:
        kt[:, :, :kv_len] = oracle.round_via_f16(kt[:, :, :kv_len]).reshape(KV_HEADS, dh, kv_len)
        v[:, :kv_len] = oracle.round_via_f16(v[:, :kv_len]).reshape(KV_HEADS, kv_len, dh)
    return kt, v


def run_decode(ta, ex, oracle, kv_len, f16, dh, graph=False):
    hq = oracle.fill_det(KV_HEADS * GROUP * dh, 7300)
    hkt, hv = make_caches(oracle, kv_len, f16, dh)
    q = ex.tensor_from(hq, shape=[KV_HEADS, GROUP, dh])
    kt = ex.tensor_from(hkt, shape=[KV_HEADS, dh, T_MAX], f16=f16)
    v = ex.tensor_from(hv, shape=[KV_HEADS, T_MAX, dh], f16=f16)
    scratch = ex.tensor([KV_HEADS * ta.ATTN_DECODE_MAX_CHUNKS * GROUP * (dh + 2)])
    out = ex.tensor([KV_HEADS, GROUP, dh])
    desc = ta.AttnDecodeDesc(kv_len, scale=float(1.0 / np.sqrt(dh)))
    if graph:
        ex.run_exec_ops([ta.ExecOp.attn_decode(q, kt, v, scratch, out, desc)])
    else:
        ex.attn_decode(q, kt, v, scratch, out, desc)
    ref = oracle.attn_decode(hq, hkt, hv, KV_HEADS, GROUP, T_MAX, dh, kv_len, float(np.float32(desc.scale)))
    err = np.abs(ex.download(out).reshape(-1) - ref)
    assert err.max() <= 1e-4, f"kv_len {kv_len} f16 {f16} dh {dh}: max err {err.max()}"


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("kv_len", [1, 33, 640, 2048])
def test_attn_decode_matches_oracle(ta, ex, oracle, kv_len, f16):
    """attn_decode.rs:172-188, with poison past kv_len."""
    run_decode(ta, ex, oracle, kv_len, f16, 64)


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("kv_len", [5, 700, 2048])
def test_attn_decode_dh128(ta, ex, oracle, kv_len, f16):
    """dh 128 (compiled here; the reference compiles 64 only)."""
    run_decode(ta, ex, oracle, kv_len, f16, 128)


def test_attn_decode_graph_op(ta, ex, oracle):
    """attn_decode.rs:190-195."""
    run_decode(ta, ex, oracle, 640, False, 64, graph=True)
    run_decode(ta, ex, oracle, 640, True, 64, graph=True)


def test_attn_decode_matches_composed_path(ta, ex, oracle):
    """attn_decode.rs:197-283: fused vs scores matmul + prefix softmax + PV."""
    kv_len, dh = 517, 64
    hq = oracle.fill_det(KV_HEADS * GROUP * dh, 7400)
    hkt, hv = make_caches(oracle, kv_len, False, dh, poison=False)
    q = ex.tensor_from(hq, shape=[KV_HEADS, GROUP, dh])
    kt = ex.tensor_from(hkt, shape=[KV_HEADS, dh, T_MAX])
    v = ex.tensor_from(hv, shape=[KV_HEADS, T_MAX, dh])
    scale = float(1.0 / np.sqrt(dh))
    scratch = ex.tensor([KV_HEADS * ta.ATTN_DECODE_MAX_CHUNKS * GROUP * (dh + 2)])
    fused = ex.tensor([KV_HEADS, GROUP, dh])
    ex.attn_decode(q, kt, v, scratch, fused, ta.AttnDecodeDesc(kv_len, scale))
    scores, composed = ex.tensor([KV_HEADS, GROUP, T_MAX]), ex.tensor([KV_HEADS, GROUP, dh])
    ex.matmul(q, kt, scores)
    ex.softmax_rows(scores, scores, scale, mask_kind=ta.SOFTMAX_MASK_PREFIX, valid_or_prefix=kv_len)
    ex.matmul(scores, v, composed)
    assert np.abs(ex.download(fused) - ex.download(composed)).max() <= 1e-5


def test_attn_decode_position_cell_replay(ta, ex, oracle):
    """AttnDecodeDesc.pos_addr: recorded once with kv_len = 1, the effective
    length is 1 + the cell's value at each replay (fixed chunk grid)."""
    dh = 64
    hq = oracle.fill_det(KV_HEADS * GROUP * dh, 7700)
    hkt, hv = make_caches(oracle, T_MAX, False, dh)
    q = ex.tensor_from(hq, shape=[KV_HEADS, GROUP, dh])
    kt = ex.tensor_from(hkt, shape=[KV_HEADS, dh, T_MAX])
    v = ex.tensor_from(hv, shape=[KV_HEADS, T_MAX, dh])
    scratch = ex.tensor([KV_HEADS * ta.ATTN_DECODE_MAX_CHUNKS * GROUP * (dh + 2)])
    out = ex.tensor([KV_HEADS, GROUP, dh])
    pos = ex.create_pos_buffer()
    scale = float(1.0 / np.sqrt(dh))
    prep = ex.prepare_exec_ops([ta.ExecOp.attn_decode(q, kt, v, scratch, out,
                                                      ta.AttnDecodeDesc(1, scale, pos.device_address))])
    for p in (0, 31, 500, 2047):
        pos.set(p)
        prep.run()
        ref = oracle.attn_decode(hq, hkt, hv, KV_HEADS, GROUP, T_MAX, dh, p + 1, float(np.float32(scale)))
        assert np.abs(ex.download(out).reshape(-1) - ref).max() <= 1e-4, f"pos {p}"
    prep.close()


def test_attn_decode_rejects_bad_geometry(ta, ex):
    """attn_decode.rs:285-334 (dh 96 stands in for the reference's dh 128,
    which is compiled here)."""
    scratch = ex.tensor([4 * 32 * 8 * 130])
    desc = ta.AttnDecodeDesc(16, 1.0)
    with pytest.raises(ta.TensorAshError, match="head dimension 96"):
        ex.attn_decode(ex.tensor([4, 8, 96]), ex.tensor([4, 96, 64]), ex.tensor([4, 64, 96]), scratch,
                       ex.tensor([4, 8, 96]), desc)
    q, kt, v, out = ex.tensor([4, 8, 64]), ex.tensor([4, 64, 64]), ex.tensor([4, 64, 64]), ex.tensor([4, 8, 64])
    with pytest.raises(ta.TensorAshError, match="out of range"):
        ex.attn_decode(q, kt, v, scratch, out, ta.AttnDecodeDesc(65, 1.0))
    with pytest.raises(ta.TensorAshError, match="scratch length"):
        ex.attn_decode(q, kt, v, ex.tensor([16]), out, desc)
    with pytest.raises(ta.TensorAshError, match="GQA group 9"):
        ex.attn_decode(ex.tensor([4, 9, 64]), kt, v, scratch, ex.tensor([4, 9, 64]), desc)
    with pytest.raises(ta.TensorAshError, match="must share a storage type"):
        ex.attn_decode(q, kt, ex.tensor([4, 64, 64], f16=True), scratch, out, desc)
