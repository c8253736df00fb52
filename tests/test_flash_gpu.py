"""GPU parity of the causal prefill attention (run_flash_attention) and of
mixed-op graphs around it (the reference's tests/correctness/flash.rs).

Tolerances are the reference's: 1e-4 absolute against the f64 oracle
(softmax weights sum to 1, so the error stays absolute-bounded), 1e-5
against the composed scores/softmax/PV path and between layouts, and
bit-identical between a standalone call and the same op in a graph.
Cache positions past kv_len are poisoned with 1e30 (flash.rs:75-105), so
a masked key or value that leaked into the sums would show.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

POISON = np.float32(1.0e30)


def fill_kv(oracle, kv_heads, dh, t_max, kv_len, poison=True):
    """flash.rs:77-105: fill_det values in the valid prefix, the poison
    value (or zero) past it."""
    n = kv_heads * dh * t_max
    fill = oracle.fill_det(n, 5101)
    kt = np.zeros((kv_heads, dh, t_max), np.float32)
    v = np.zeros((kv_heads, t_max, dh), np.float32)
    kt_idx = np.arange(n).reshape(kv_heads, dh, t_max)
    v_idx = np.arange(n).reshape(kv_heads, t_max, dh)
    kt[:] = fill[kt_idx % n]
    v[:] = fill[(v_idx * 7 + 3) % n]
    kt[:, :, kv_len:] = POISON if poison else 0.0
    v[:, kv_len:, :] = POISON if poison else 0.0
    return kt, v


CASES = [  # label, H, H_kv, T_q, T_max, dh, kv_len, pos_base (flash.rs:173-240)
    ("fresh prefill dh64", 4, 4, 197, 256, 64, 197, 0),
    ("fresh prefill dh128 ragged", 3, 3, 129, 161, 128, 129, 0),
    ("warm cache offset", 4, 4, 64, 512, 64, 364, 300),
    ("gqa group of 4", 8, 2, 100, 128, 64, 100, 0),
    ("single-row decode style", 4, 4, 1, 96, 128, 77, 76),
    ("prefill 512 dh128 gqa", 32, 8, 512, 512, 128, 512, 0),
    ("kv_len cuts the causal frontier", 2, 1, 130, 200, 64, 90, 20),
]


@pytest.mark.parametrize("label,heads,kv_heads,t_q,t_max,dh,kv_len,pos_base", CASES, ids=[c[0] for c in CASES])
def test_flash_matches_oracle(ta, ex, oracle, label, heads, kv_heads, t_q, t_max, dh, kv_len, pos_base):
    q = oracle.fill_det(heads * t_q * dh, 5100)
    kt, v = fill_kv(oracle, kv_heads, dh, t_max, kv_len)
    tq = ex.tensor_from(q, shape=[heads, t_q, dh])
    tk, tv = ex.tensor_from(kt, shape=[kv_heads, dh, t_max]), ex.tensor_from(v, shape=[kv_heads, t_max, dh])
    out = ex.tensor([heads, t_q, dh])
    scale = float(1.0 / np.sqrt(np.float32(dh)))
    ex.flash_attention(tq, tk, tv, out, ta.FlashAttentionDesc(kv_len, pos_base, scale))
    got = ex.download(out).reshape(-1)
    ref = oracle.flash_attention(q, kt, v, heads, kv_heads, t_q, t_max, dh, kv_len, pos_base, scale)
    err, idx = oracle.max_abs_err(got, ref)
    assert err <= 1e-4, f"{label}: err {err} at {idx}"


@pytest.mark.parametrize("dh", [64, 128])
def test_flash_f16_caches(ta, ex, oracle, dh):
    """f16 Kt/V caches (op_flash_attention_kv16_*): widened exactly, so the
    f32 tolerance holds against the oracle on the f16-rounded caches."""
    heads, kv_heads, t_q, t_max, kv_len, pos_base = 8, 2, 150, 256, 190, 40
    q = oracle.fill_det(heads * t_q * dh, 5300)
    kt, v = fill_kv(oracle, kv_heads, dh, t_max, kv_len, poison=False)
    kt16, v16 = oracle.round_via_f16(kt), oracle.round_via_f16(v)
    tq = ex.tensor_from(q, shape=[heads, t_q, dh])
    tk = ex.tensor_from(kt, shape=[kv_heads, dh, t_max], f16=True)
    tv = ex.tensor_from(v, shape=[kv_heads, t_max, dh], f16=True)
    out = ex.tensor([heads, t_q, dh])
    ex.flash_attention(tq, tk, tv, out, ta.FlashAttentionDesc(kv_len, pos_base, 0.125))
    ref = oracle.flash_attention(q, kt16, v16, heads, kv_heads, t_q, t_max, dh, kv_len, pos_base, 0.125)
    err, idx = oracle.max_abs_err(ex.download(out).reshape(-1), ref)
    assert err <= 1e-4, f"err {err} at {idx}"


@pytest.mark.parametrize("dh", [64, 128])
def test_flash_io16_matches_f32_io_route(ta, ex, oracle, dh):
    """flash.rs:569-649: f16 q/out with f16 caches against the f32-io route
    on the same f16 inputs, 4e-3 (one f16 ulp of |out| <= max |V|); GQA,
    warm cache and ragged T_q."""
    heads, kv_heads, t_q, t_max, kv_len, pos_base = 8, 2, 333, 1024, 533, 200
    q = oracle.round_via_f16(oracle.fill_det(heads * t_q * dh, 5600))
    kt, v = fill_kv(oracle, kv_heads, dh, t_max, kv_len, poison=False)
    tk = ex.tensor_from(kt, shape=[kv_heads, dh, t_max], f16=True)
    tv = ex.tensor_from(v, shape=[kv_heads, t_max, dh], f16=True)
    q16, q32 = ex.tensor_from(q, shape=[heads, t_q, dh], f16=True), ex.tensor_from(q, shape=[heads, t_q, dh])
    out16, out32 = ex.tensor([heads, t_q, dh], f16=True), ex.tensor([heads, t_q, dh])
    desc = ta.FlashAttentionDesc(kv_len, pos_base, float(1.0 / np.sqrt(np.float32(dh))))
    ex.flash_attention(q16, tk, tv, out16, desc)
    ex.flash_attention(q32, tk, tv, out32, desc)
    g16, g32 = ex.download(out16).reshape(-1), ex.download(out32).reshape(-1)
    assert np.max(np.abs(g16 - g32)) <= 4e-3
    assert np.array_equal(g16, oracle.round_via_f16(g32))


def test_flash_matches_composed_path(ta, ex, oracle):
    """flash.rs:244-308: fused vs scores GEMM -> causal softmax -> PV GEMM
    on the same tensors, 1e-5."""
    heads, t, dh = 8, 256, 64
    q, kt, v = (oracle.fill_det(heads * t * dh, s) for s in (5200, 5201, 5202))
    tq = ex.tensor_from(q, shape=[heads, t, dh])
    tk, tv = ex.tensor_from(kt, shape=[heads, dh, t]), ex.tensor_from(v, shape=[heads, t, dh])
    scale = 0.125
    fused = ex.tensor([heads, t, dh])
    ex.flash_attention(tq, tk, tv, fused, ta.FlashAttentionDesc(t, 0, scale))
    scores, composed = ex.tensor([heads, t, t]), ex.tensor([heads, t, dh])
    ex.matmul(tq, tk, scores)
    ex.softmax_rows(scores, scores, scale, mask_kind=ta.SOFTMAX_MASK_CAUSAL, valid_or_prefix=0, rows_per_group=t)
    ex.matmul(scores, tv, composed)
    a, b = ex.download(fused).reshape(-1), ex.download(composed).reshape(-1)
    assert np.max(np.abs(a - b)) <= 1e-5


def test_flash_token_major_matches_head_major(ta, ex, oracle):
    """flash.rs:715-863: token-major q ([T, H*dh]) and token-major out give
    the head-major result permuted, 1e-5."""
    heads, kv_heads, t_q, t_max, dh = 8, 2, 128, 256, 64
    q = oracle.fill_det(heads * t_q * dh, 5500)
    kt, v = fill_kv(oracle, kv_heads, dh, t_max, t_q)
    tk, tv = ex.tensor_from(kt, shape=[kv_heads, dh, t_max]), ex.tensor_from(v, shape=[kv_heads, t_max, dh])
    hm = q.reshape(heads, t_q, dh)
    tm = np.ascontiguousarray(hm.transpose(1, 0, 2))
    q_hm, q_tm = ex.tensor_from(hm, shape=[heads, t_q, dh]), ex.tensor_from(tm, shape=[t_q, heads * dh])
    out_hm, out_tm, out_mixed = ex.tensor([heads, t_q, dh]), ex.tensor([t_q, heads * dh]), ex.tensor([t_q, heads * dh])
    ex.flash_attention(q_hm, tk, tv, out_hm, ta.FlashAttentionDesc(t_q, 0, 0.125))
    ex.flash_attention(q_tm, tk, tv, out_tm, ta.FlashAttentionDesc(t_q, 0, 0.125, token_major_heads=heads))
    ex.flash_attention(q_hm, tk, tv, out_mixed, ta.FlashAttentionDesc(t_q, 0, 0.125, out_token_major_heads=heads))
    ref = ex.download(out_hm).reshape(heads, t_q, dh)
    for o in (out_tm, out_mixed):
        got = ex.download(o).reshape(t_q, heads, dh).transpose(1, 0, 2)
        assert np.max(np.abs(got - ref)) <= 1e-5


def test_flash_in_graph_matches_standalone_bitwise(ta, ex, oracle):
    """flash.rs:364-419: the same op in a mixed graph (run and prepared)
    gives the standalone bits."""
    heads, kv_heads, t_q, t_max, dh, kv_len, pos_base = 8, 2, 100, 256, 64, 160, 60
    q = oracle.fill_det(heads * t_q * dh, 5400)
    kt, v = fill_kv(oracle, kv_heads, dh, t_max, kv_len)
    tq = ex.tensor_from(q, shape=[heads, t_q, dh])
    tk, tv = ex.tensor_from(kt, shape=[kv_heads, dh, t_max]), ex.tensor_from(v, shape=[kv_heads, t_max, dh])
    desc = ta.FlashAttentionDesc(kv_len, pos_base, 0.125)
    a, b, c = (ex.tensor([heads, t_q, dh]) for _ in range(3))
    ex.flash_attention(tq, tk, tv, a, desc)
    ex.run_exec_ops([ta.ExecOp.flash_attn(tq, tk, tv, b, desc)])
    prep = ex.prepare_exec_ops([ta.ExecOp.flash_attn(tq, tk, tv, c, desc)])
    for _ in range(3):
        prep.run()
        assert np.array_equal(ex.download(c), ex.download(a))
    prep.close()
    assert np.array_equal(ex.download(b), ex.download(a))


def test_flash_rejects_bad_geometry(ta, ex):
    """flash.rs:310-360 and 651-686: unsupported head dimension, kv_len
    past the cache, f16 q with f32 caches, mixed q/out storage, GQA and
    shape mismatches."""
    q = ex.tensor([2, 32, 96])
    with pytest.raises(ta.TensorAshError, match="head dimension 96"):
        ex.flash_attention(q, ex.tensor([2, 96, 64]), ex.tensor([2, 64, 96]), ex.tensor([2, 32, 96]),
                           ta.FlashAttentionDesc(32, 0, 1.0))
    q, kt, v, out = ex.tensor([2, 64, 64]), ex.tensor([2, 64, 64]), ex.tensor([2, 64, 64]), ex.tensor([2, 64, 64])
    with pytest.raises(ta.TensorAshError, match="exceeds cache T_max"):
        ex.flash_attention(q, kt, v, out, ta.FlashAttentionDesc(65, 0, 1.0))
    q16, out16 = ex.tensor([2, 64, 64], f16=True), ex.tensor([2, 64, 64], f16=True)
    with pytest.raises(ta.TensorAshError, match="f16 KV caches"):
        ex.flash_attention(q16, kt, v, out16, ta.FlashAttentionDesc(64, 0, 0.125))
    kt16, v16 = ex.tensor([2, 64, 64], f16=True), ex.tensor([2, 64, 64], f16=True)
    with pytest.raises(ta.TensorAshError, match="share a storage type"):
        ex.flash_attention(q16, kt16, v16, out, ta.FlashAttentionDesc(64, 0, 0.125))
    with pytest.raises(ta.TensorAshError, match="multiple of H_kv"):
        ex.flash_attention(ex.tensor([3, 64, 64]), kt, v, ex.tensor([3, 64, 64]), ta.FlashAttentionDesc(64, 0, 1.0))
    with pytest.raises(ta.TensorAshError, match="inconsistent cache shapes"):
        ex.flash_attention(q, kt, ex.tensor([2, 32, 64]), out, ta.FlashAttentionDesc(32, 0, 1.0))
    with pytest.raises(ta.TensorAshError, match="must equal q shape"):
        ex.flash_attention(q, kt, v, ex.tensor([2, 32, 64]), ta.FlashAttentionDesc(32, 0, 1.0))
    with pytest.raises(ta.TensorAshError, match="out_token_major_heads 3 != q heads 2"):
        ex.flash_attention(q, kt, v, out, ta.FlashAttentionDesc(32, 0, 1.0, out_token_major_heads=3))


def test_exec_graph_replays_with_position_cell(ta, ex, oracle):
    """prepare_exec_ops with a position cell (graph_ops.rs:271-336): RoPE
    and the KV append read the position when the graph runs, so one
    recording serves successive decode steps; each replay matches the
    standalone ops at that position."""
    heads, dh, t_max = 4, 64, 32
    half = dh // 2
    theta = np.array([[p / 10000.0 ** (2.0 * i / dh) for i in range(half)] for p in range(t_max)])
    table = np.stack([np.cos(theta), np.sin(theta)], axis=-1).astype(np.float32).reshape(-1)
    t_table = ex.tensor_from(table, shape=[t_max, half, 2])
    k = ex.tensor([1, heads * dh])
    k_rot = ex.tensor([1, heads * dh])
    cache = ex.tensor_from(np.zeros(heads * dh * t_max, np.float32), shape=[heads, dh, t_max])
    pos = ex.tensor_from(np.array([0], np.uint32).view(np.float32), shape=[1])
    addr = pos.device_address
    ops = [
        ta.ExecOp.copy_strided(k, k_rot, ta.CopyDesc((heads * dh, 1, 1), (1, 0, 0), (1, 0, 0))),
        ta.ExecOp.rope(k_rot, t_table, k_rot, ta.RopeDesc(heads, dh, dh, 0, pos_addr=addr)),
        ta.ExecOp.copy_strided(k_rot, cache, ta.CopyDesc((dh, heads, 1), (1, dh, 0), (t_max, dh * t_max, 0),
                                                         pos_addr=addr, pos_scale=1)),
    ]
    prep = ex.prepare_exec_ops(ops)
    want = np.zeros((heads, dh, t_max), np.float32)
    for step in (0, 1, 2, 7, 31):
        kv = oracle.fill_det(heads * dh, 5700 + step)
        ex.upload(k, kv)
        ex.upload(pos, np.array([step], np.uint32).view(np.float32))
        prep.run()
        rot = oracle.rope_tokens(kv, table, 1, heads, dh, dh, step)
        assert oracle.max_abs_err(ex.download(k_rot).reshape(-1), rot)[0] <= 1e-6
        want[:, :, step] = ex.download(k_rot).reshape(heads, dh)
        assert np.array_equal(ex.download(cache), want)
    prep.close()


def test_exec_ops_reject_before_launch(ta, ex):
    """graph_ops.rs:249-258: an invalid op anywhere fails the whole list
    before anything runs (the first op's output stays untouched)."""
    a = ex.tensor_from(np.ones(64, np.float32), shape=[4, 16])
    b = ex.tensor_from(np.full(64, 3.0, np.float32), shape=[4, 16])
    with pytest.raises(ta.TensorAshError, match="weight length"):
        ex.run_exec_ops([
            ta.ExecOp.softmax_rows(a, b, 1.0),
            ta.ExecOp.rms_norm(a, ex.tensor([15]), b, 1e-5),
        ])
    assert np.all(ex.download(b) == 3.0)
    with pytest.raises(ta.TensorAshError, match="empty"):
        ex.run_exec_ops([])
