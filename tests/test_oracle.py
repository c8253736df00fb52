"""Pinning the CPU oracle (oracle/oracle.c) before it is trusted.

Each oracle function is checked against the reference's own known-answer
tests (file:line cited) and against what mathematics or an independent
library fixes, chosen so a plausible slip (dropped term, wrong sign or
index, transposed operand) fails:

  function            pinned by
  ------------------  -------------------------------------------------------
  fill_det / LcgRng   reference property tests (tools/test-support/src/lib.rs
                      :168-200) + uniform moments + committed first values
                      (tests/golden/fill_det.json).  The reference holds no
                      golden values for the exact stream: exact-stream parity
                      with the reference is UNPINNED (inputs only; no GPU
                      parity result depends on it).
  cpu_bmm             reference KATs (lib.rs:221-277) + numpy float64 matmul
                      on random shapes (library routine), batch broadcasting
  max_abs_err         reference KATs (lib.rs:205-218, 280-284)
  tolerance           reference KAT (lib.rs:286-291) + closed form 8*K*eps
  f16 encode/decode   reference KATs (src/dtype.rs:118-163) + numpy.float16
                      (IEEE binary16, RNE) bit-exact: all 65536 halves and
                      2^20 f32 values across the whole exponent range
  pack_row_tiles      reference KAT (src/matmul/api.rs:355-380) + inverse
  epilogue            closed forms: ReLU, x*expit(x) (scipy), torch GELU
                      (approximate="tanh"); order bias->act->binary checked
                      on a case where any other order differs; c_smoke KAT
  split_window        invariants: windows tile [0, K) exactly, sizes differ
                      by at most one, larger windows first
  fill_normal         own definition (no reference counterpart): moments and
                      a Kolmogorov-Smirnov test against N(0, sigma)
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- fill_det

def test_fill_det_deterministic_range_seed(oracle):
    """lib.rs:168-193."""
    assert np.array_equal(oracle.fill_det(8, 42), oracle.fill_det(8, 42))
    v = oracle.fill_det(1024, 7)
    assert np.all(v >= -1.0) and np.all(v < 1.0)
    assert not np.array_equal(oracle.fill_det(16, 1), oracle.fill_det(16, 2))


def test_fill_det_moments(oracle):
    v = oracle.fill_det(1 << 20, 3).astype(np.float64)
    assert abs(v.mean()) < 3e-3
    assert abs(v.var() - 1.0 / 3.0) < 3e-3
    # 24-bit grid: every value is k / 2^23 - 1
    assert np.all(np.round((v + 1.0) * 2 ** 23) == (v + 1.0) * 2 ** 23)


def test_fill_det_golden(oracle):
    g = json.loads((GOLDEN / "fill_det.json").read_text())
    for seed, vals in g["values"].items():
        np.testing.assert_array_equal(oracle.fill_det(len(vals), int(seed)), np.array(vals, np.float32))


def test_lcg_range(oracle):
    """lib.rs:194-208."""
    r = oracle.lcg_range(0xCAFE, 7, 13, 1000)
    assert r.min() >= 7 and r.max() <= 13 and len(set(r.tolist())) == 7
    assert np.all(oracle.lcg_range(1, 42, 42, 16) == 42)
    with pytest.raises(ValueError):
        oracle.lcg_range(1, 5, 4, 1)


# ---------------------------------------------------------------- cpu_bmm

A2 = [1.0, 2.0, 3.0, 4.0]
B2 = [5.0, 6.0, 7.0, 8.0]


def test_cpu_bmm_reference_kats(oracle):
    """lib.rs:221-277."""
    assert oracle.cpu_bmm(A2, B2, None, 1, 2, 2, 2).tolist() == [19, 22, 43, 50]
    assert oracle.cpu_bmm(A2, B2, [100] * 4, 1, 2, 2, 2, 1.0, True).tolist() == [119, 122, 143, 150]
    assert oracle.cpu_bmm(A2, B2, None, 1, 2, 2, 2, 0.5).tolist() == [9.5, 11, 21.5, 25]
    eye = [1.0, 0.0, 0.0, 1.0]
    bb = [1, 2, 3, 4, 10, 20, 30, 40]
    assert oracle.cpu_bmm(eye, bb, None, 2, 2, 2, 2).tolist() == bb
    assert oracle.cpu_bmm(bb, eye, None, 2, 2, 2, 2).tolist() == bb


def test_cpu_bmm_rejects_bad_lengths(oracle):
    with pytest.raises(ValueError):
        oracle.cpu_bmm([1.0] * 3, B2, None, 1, 2, 2, 2)


@pytest.mark.parametrize("batch,ba,bb,m,n,k", [(1, 1, 1, 7, 5, 3), (3, 3, 1, 17, 9, 33),
                                              (4, 1, 4, 5, 31, 64), (2, 2, 2, 40, 41, 129)])
def test_cpu_bmm_matches_numpy_f64(oracle, batch, ba, bb, m, n, k):
    rng = np.random.default_rng(m * n + k)
    a = rng.uniform(-1, 1, (ba, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (bb, k, n)).astype(np.float32)
    got = oracle.cpu_bmm(a, b, None, batch, m, n, k, 0.75).reshape(batch, m, n)
    ref = (np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32) * np.float32(0.75))
    ref = np.broadcast_to(ref, (batch, m, n))
    # f64 sums differ only in summation order: both round to the same or an adjacent f32
    np.testing.assert_allclose(got, ref, rtol=2e-7, atol=1e-7)


def test_cpu_bmm_rows_bit_identical(oracle):
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, 3 * 20 * 30).astype(np.float32)
    b = rng.uniform(-1, 1, 30 * 11).astype(np.float32)
    full = oracle.cpu_bmm(a, b, None, 3, 20, 11, 30, 1.0)
    out = np.zeros(3 * 20 * 11, np.float32)
    oracle.cpu_bmm_rows(a, b, 3, 20, 11, 30, 1.0, out, 0, 60, 4)
    assert np.array_equal(out, full)
    out2 = np.zeros_like(out)
    oracle.cpu_bmm_rows(a, b, 3, 20, 11, 30, 1.0, out2, 0, 60, 3, reference_order=True)
    assert np.array_equal(out2, full)


# ---------------------------------------------------------------- errors

def test_max_abs_err_kats(oracle):
    """lib.rs:205-218, 280-284."""
    assert oracle.max_abs_err([1.0, float("nan")], [1.0, 2.0]) == (math.inf, 1)
    assert oracle.max_abs_err([1.0, 3.0, -5.0], [1.5, 1.0, -4.0]) == (2.0, 1)
    with pytest.raises(ValueError):
        oracle.max_abs_err([1.0], [1.0, 2.0])


def test_tolerance(oracle):
    """lib.rs:160-162, 286-291."""
    assert oracle.tolerance(0) == 0.0
    assert oracle.tolerance(200) > oracle.tolerance(100)
    assert oracle.tolerance(512) == np.float32(8 * 512 * np.finfo(np.float32).eps)


# ---------------------------------------------------------------- f16

def test_f16_reference_kats(oracle):
    """src/dtype.rs:118-163."""
    enc = lambda v: int(oracle.f32_to_f16_bits([v])[0])
    for v in [0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 65504.0, -65504.0, 0.25, 1024.0]:
        r = oracle.round_via_f16([v])[0]
        assert r == v and np.float32(r).tobytes() == np.float32(v).tobytes()
    assert enc(1.0) == 0x3C00 and enc(-2.0) == 0xC000 and enc(65504.0) == 0x7BFF
    assert enc(math.inf) == 0x7C00 and enc(65520.0) == 0x7C00
    assert enc(6.104e-5) == 0x0400 and enc(5.96e-8) == 0x0001 and enc(1e-10) == 0
    assert math.isnan(oracle.f16_bits_to_f32([enc(math.nan)])[0])
    assert oracle.round_via_f16([1.0 + 2 ** -11])[0] == 1.0
    assert oracle.round_via_f16([1.0 + 3 * 2 ** -11])[0] == np.float32(1.0 + 2 ** -9)
    v = 0.001
    while v < 60000.0:
        r = oracle.round_via_f16([v])[0]
        assert abs((r - np.float32(v)) / np.float32(v)) <= 2 ** -11
        v *= 1.37


def test_f16_decode_all_halves_vs_numpy(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_vs_numpy(oracle):
    rng = np.random.default_rng(11)
    exps = rng.uniform(-30, 17, 1 << 20)
    x = (rng.choice([-1.0, 1.0], 1 << 20) * np.exp2(exps)).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, 65519.99, 65520.0, 2 ** -25,
                                     3 * 2 ** -26, 2 ** -24 * 1.5], np.float32)])
    got = oracle.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r} got {got[bad[0]]:#x} ref {ref[bad[0]]:#x}"


# ---------------------------------------------------------------- packing

def test_pack_reference_kat(oracle):
    """src/matmul/api.rs:355-380."""
    got = oracle.pack_row_tiles(np.arange(16, dtype=np.float32), 4, 4, 2)
    assert got.tolist() == [0, 1, 4, 5, 8, 9, 12, 13, 2, 3, 6, 7, 10, 11, 14, 15]


def test_pack_inverse(oracle):
    k, n, t = 37, 192, 64
    w = np.arange(k * n, dtype=np.float32)
    p = oracle.pack_row_tiles(w, k, n, t).reshape(n // t, k, t)
    assert np.array_equal(p.transpose(1, 0, 2).reshape(k, n), w.reshape(k, n))
    with pytest.raises(ValueError):
        oracle.pack_row_tiles(w, k, n, 50)


# ---------------------------------------------------------------- epilogue

def test_epilogue_closed_forms(oracle):
    import scipy.special
    import torch
    x = np.linspace(-9, 9, 2001, dtype=np.float32)
    n = x.size
    relu = oracle.epilogue(x, n, n, act=1)
    assert np.array_equal(relu, np.maximum(x, 0))
    silu = oracle.epilogue(x, n, n, act=2)
    np.testing.assert_allclose(silu, x.astype(np.float64) * scipy.special.expit(x.astype(np.float64)),
                               rtol=1e-6, atol=1e-7)
    gelu = oracle.epilogue(x, n, n, act=3)
    tg = torch.nn.functional.gelu(torch.from_numpy(x.astype(np.float64)), approximate="tanh").numpy()
    np.testing.assert_allclose(gelu, tg, rtol=1e-6, atol=1e-7)


def test_epilogue_order_and_binary(oracle):
    """bias -> act -> binary (shaders/matmul_epilogue_common.glsl:14-21)."""
    c = np.array([-1.0, 2.0, 0.5, -3.0], np.float32)
    bias = np.array([2.0, -3.0], np.float32)  # flips the sign of both columns of row 0
    d = np.array([10.0, 20.0, 30.0, 40.0], np.float32)
    got = oracle.epilogue(c, 2, 4, bias, 0, 1, 1, d, 0.5)
    ref = np.maximum(c + np.tile(bias, 2), 0) + 0.5 * d
    assert np.array_equal(got, ref.astype(np.float32))
    got = oracle.epilogue(c, 2, 4, None, 0, 0, 2, d)
    assert np.array_equal(got, c * d)
    # batched bias [B, N]: plane b uses row b
    c2 = np.zeros(2 * 2 * 2, np.float32)
    bb = np.array([1, 2, 3, 4], np.float32)
    got = oracle.epilogue(c2, 2, 4, bb, 2)
    assert got.tolist() == [1, 2, 1, 2, 3, 4, 3, 4]


def test_epilogue_c_smoke_kat(oracle):
    """examples/c_smoke.c:80-104: 58 + (-58.5) then SiLU -> silu(-0.5)."""
    out = oracle.reference_gemm([1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12], 1, 2, 2, 3,
                                bias=[-58.5, 0.0], act=2)
    assert abs(out[0] - (-0.5 / (1 + math.exp(0.5)))) < 1e-6
    assert abs(out[3] - 154.0) < 1e-4


# ---------------------------------------------------------------- split-K

@pytest.mark.parametrize("k,s", [(1, 1), (7, 7), (999, 7), (65536, 32), (131072, 16), (100, 3), (33, 32)])
def test_split_window_invariants(oracle, k, s):
    wins = [oracle.split_window(k, s, i) for i in range(s)]
    assert wins[0][0] == 0 and wins[-1][1] == k
    for (lo, hi), (lo2, _) in zip(wins, wins[1:]):
        assert hi == lo2
    sizes = [hi - lo for lo, hi in wins]
    assert max(sizes) - min(sizes) <= 1 and sizes == sorted(sizes, reverse=True)


# ---------------------------------------------------------------- normal

def test_fill_normal_distribution(oracle):
    import scipy.stats
    v = oracle.fill_normal(200001, 21, 0.02).astype(np.float64)
    assert abs(v.mean()) < 2e-4 and abs(v.std() - 0.02) < 2e-4
    assert scipy.stats.kstest(v / 0.02, "norm").pvalue > 1e-3
    assert np.array_equal(oracle.fill_normal(9, 5, 1.0), oracle.fill_normal(9, 5, 1.0))


# ---------------------------------------------------------------- decode fusions

def test_rms_norm_matches_torch_and_closed_form(oracle):
    """rms_norm_rows pinned against torch's rms_norm in float64 (same
    formula, independent implementation) and against the closed form of a
    constant row: x = c gives w * c / sqrt(c^2 + eps)."""
    import torch
    m, k, eps = 3, 203, 1e-5
    x = oracle.fill_det(m * k, 70)
    w = oracle.fill_det(k, 71)
    got = oracle.rms_norm_rows(x, w, m, k, eps).reshape(m, k)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x.reshape(m, k)).double(), (k,),
                                       torch.from_numpy(w).double(), eps=float(np.float32(eps)))
    assert np.allclose(got, ref.numpy(), rtol=2e-7, atol=1e-7)
    c = np.float32(0.75)
    got = oracle.rms_norm_rows(np.full(k, c, np.float32), w, 1, k, eps)
    want = (w.astype(np.float64) * c / math.sqrt(float(c) ** 2 + float(np.float32(eps)))).astype(np.float32)
    assert np.array_equal(got, want)
    # A scaled row normalizes to the same values (up to eps).
    big = oracle.rms_norm_rows(x[:k] * 1000.0, w, 1, k, 0.0)
    assert np.allclose(big, oracle.rms_norm_rows(x[:k], w, 1, k, 0.0), rtol=1e-6, atol=1e-7)


def test_rope_pairs_is_a_rotation(oracle):
    """rope_pairs pinned against complex multiplication: each (even, odd)
    pair of head h at position p is multiplied by cos + i sin of its own
    angle; the identity angle leaves the row bit-exact and a quarter turn
    maps (a, b) to (-b, a) exactly."""
    hd, t_max, pos, n = 8, 6, 4, 32
    y = oracle.fill_det(n, 72)
    theta = np.linspace(0.1, 2.9, t_max * hd // 2).reshape(t_max, hd // 2)
    table = np.stack([np.cos(theta), np.sin(theta)], axis=-1).astype(np.float32)
    got = oracle.rope_pairs(y, table, pos, hd)
    z = y[0::2].astype(np.float64) + 1j * y[1::2].astype(np.float64)
    ang = table[pos, (np.arange(n // 2) % (hd // 2))].astype(np.float64)
    rot = z * (ang[:, 0] + 1j * ang[:, 1])
    assert np.allclose(got[0::2], rot.real, atol=1e-6) and np.allclose(got[1::2], rot.imag, atol=1e-6)
    ident = np.tile(np.array([1.0, 0.0], np.float32), t_max * hd // 2)
    assert np.array_equal(oracle.rope_pairs(y, ident, pos, hd), y)
    quarter = np.tile(np.array([0.0, 1.0], np.float32), t_max * hd // 2)
    q = oracle.rope_pairs(y, quarter, pos, hd)
    assert np.array_equal(q[0::2], -y[1::2]) and np.array_equal(q[1::2], y[0::2])


def test_scatter_index_matches_cache_layouts(oracle):
    """scatter_index pinned by the two KV layouts the reference scatters
    into (src/matmul/api.rs:160-168): V cache [H, T_max, dh] (pos_scale dh,
    stride_head T_max*dh, stride_dim 1) and Kt cache [H, dh, T_max]
    (pos_scale 1, stride_head dh*T_max, stride_dim T_max); placing the row
    and reading the cache back through numpy indexing recovers it."""
    h, dh, t_max, pos = 4, 8, 10, 7
    y = oracle.fill_det(h * dh, 73)
    v_cache = oracle.store_scatter(np.zeros(h * t_max * dh), y, pos, dh, dh, t_max * dh, 1)
    assert np.array_equal(v_cache.reshape(h, t_max, dh)[:, pos, :].reshape(-1), y)
    assert np.count_nonzero(v_cache) == np.count_nonzero(y)
    kt_cache = oracle.store_scatter(np.zeros(h * dh * t_max), y, pos, dh, 1, dh * t_max, t_max)
    assert np.array_equal(kt_cache.reshape(h, dh, t_max)[:, :, pos].reshape(-1), y)
    f16 = oracle.store_scatter(np.zeros(h * t_max * dh), y, pos, dh, dh, t_max * dh, 1, f16=True)
    assert np.array_equal(f16.reshape(h, t_max, dh)[:, pos, :].reshape(-1),
                          y.astype(np.float16).astype(np.float32))


# ---------------------------------------------------------------- model ops

def test_softmax_rows_pinned(oracle):
    """softmax_rows pinned against scipy's softmax (f64) on every valid
    prefix; masked tails are exactly 0, rows sum to 1, an all-masked row
    is all zeros."""
    import scipy.special
    rows, cols, scale = 6, 517, 0.125
    x = oracle.fill_det(rows * cols, 2100)
    full = oracle.softmax_rows(x, rows, cols, scale, cols).reshape(rows, cols)
    want = scipy.special.softmax(x.reshape(rows, cols).astype(np.float64) * np.float32(scale), axis=1)
    assert np.allclose(full, want, rtol=1e-6, atol=1e-9)
    causal = oracle.softmax_rows(x, rows, cols, scale, lambda r: 100 + r % 3 + 1).reshape(rows, cols)
    for r in range(rows):
        v = 100 + r % 3 + 1
        assert np.all(causal[r, v:] == 0) and abs(causal[r].sum() - 1) < 1e-6
        ref = scipy.special.softmax(x.reshape(rows, cols)[r, :v].astype(np.float64) * np.float32(scale))
        assert np.allclose(causal[r, :v], ref, rtol=1e-6, atol=1e-9)
    assert np.all(oracle.softmax_rows(x, rows, cols, scale, 0) == 0)


def test_layer_norm_pinned(oracle):
    """layer_norm_rows pinned against torch's layer_norm in f64 and the
    invariant that a normalized row (w = 1, b = 0) has mean 0 and
    variance var / (var + eps)."""
    import torch
    rows, cols, eps = 5, 771, 1e-5
    x, w, b = oracle.fill_det(rows * cols, 2200), oracle.fill_det(cols, 2201), oracle.fill_det(cols, 2202)
    got = oracle.layer_norm_rows(x, w, b, rows, cols, eps).reshape(rows, cols)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x.reshape(rows, cols)).double(), (cols,),
                                         torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                                         eps=float(np.float32(eps)))
    assert np.allclose(got, ref.numpy(), rtol=1e-6, atol=1e-6)
    y = oracle.layer_norm_rows(x, np.ones(cols), np.zeros(cols), rows, cols, 0.0).reshape(rows, cols)
    assert np.allclose(y.mean(axis=1), 0, atol=1e-6) and np.allclose((y.astype(np.float64) ** 2).mean(axis=1), 1, atol=1e-5)


def test_rope_tokens_pinned(oracle):
    """rope_tokens pinned against complex multiplication with the Llama
    table theta = pos / 10000^(2i/rot_dim) (tests/correctness/
    elementwise.rs:146-222), and lanes past rot_dim passing through."""
    tokens, heads, hd, rot, t_max, pos_base = 3, 4, 16, 12, 32, 7
    x = oracle.fill_det(tokens * heads * hd, 2300)
    half = rot // 2
    theta = np.array([[p / 10000.0 ** (2.0 * i / rot) for i in range(half)] for p in range(t_max)])
    table = np.stack([np.cos(theta), np.sin(theta)], axis=-1).astype(np.float32)
    got = oracle.rope_tokens(x, table, tokens, heads, hd, rot, pos_base).reshape(tokens, heads, hd)
    xv = x.reshape(tokens, heads, hd).astype(np.float64)
    z = xv[:, :, 0:rot:2] + 1j * xv[:, :, 1:rot:2]
    ang = table[pos_base:pos_base + tokens].astype(np.float64)
    rot_z = z * (ang[:, None, :, 0] + 1j * ang[:, None, :, 1])
    assert np.allclose(got[:, :, 0:rot:2], rot_z.real, atol=1e-6)
    assert np.allclose(got[:, :, 1:rot:2], rot_z.imag, atol=1e-6)
    assert np.array_equal(got[:, :, rot:], x.reshape(tokens, heads, hd)[:, :, rot:])


def test_copy_strided_pinned(oracle):
    """copy_strided pinned by numpy transposes: a stride swap transposes a
    37x53 matrix, and the Kt-cache append of elementwise.rs:275-300
    lands the vector in column t of [heads, dh, t_max]."""
    r, c = 37, 53
    src = oracle.fill_det(r * c, 2400)
    t = oracle.copy_strided(src, np.zeros(r * c), (c, r, 1), 0, (1, c, 0), 0, (r, 1, 0))
    assert np.array_equal(t.reshape(c, r), src.reshape(r, c).T)
    heads, dh, t_max, step = 4, 8, 16, 5
    k = oracle.fill_det(heads * dh, 2401)
    cache = oracle.copy_strided(k, np.zeros(heads * dh * t_max), (dh, heads, 1), 0, (1, dh, 0), step,
                                (t_max, dh * t_max, 0)).reshape(heads, dh, t_max)
    assert np.array_equal(cache[:, :, step], k.reshape(heads, dh))
    assert np.count_nonzero(cache) == np.count_nonzero(k)


def test_flash_attention_pinned(oracle):
    """flash_attention pinned three ways: a scalar triple loop restating
    cpu_flash (flash.rs:10-61) on a tiny GQA case with an offset; torch's
    scaled_dot_product_attention in f64 with an explicit boolean mask on a
    larger case; and closed forms (kv_len 1 returns V[0]; scale 0 returns
    the mean of the valid V rows)."""
    import math
    import torch
    heads, kv_heads, t_q, t_max, dh, kv_len, pos_base = 4, 2, 5, 12, 8, 9, 4
    q = oracle.fill_det(heads * t_q * dh, 2500)
    kt = oracle.fill_det(kv_heads * dh * t_max, 2501)
    v = oracle.fill_det(kv_heads * t_max * dh, 2502)
    got = oracle.flash_attention(q, kt, v, heads, kv_heads, t_q, t_max, dh, kv_len, pos_base, 0.35)
    want = np.zeros(heads * t_q * dh)
    for h in range(heads):
        kh = h // (heads // kv_heads)
        for i in range(t_q):
            valid = min(kv_len, pos_base + i + 1)
            sc = [sum(float(q[(h * t_q + i) * dh + d]) * float(kt[(kh * dh + d) * t_max + p]) for d in range(dh))
                  * float(np.float32(0.35)) for p in range(valid)]
            mx = max(sc)
            e = [math.exp(x - mx) for x in sc]
            tot = sum(e)
            for d in range(dh):
                want[(h * t_q + i) * dh + d] = sum(e[p] / tot * float(v[(kh * t_max + p) * dh + d])
                                                   for p in range(valid))
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)

    heads, kv_heads, t_q, t_max, dh, kv_len, pos_base = 8, 2, 70, 128, 64, 100, 30
    q = oracle.fill_det(heads * t_q * dh, 2510)
    kt = oracle.fill_det(kv_heads * dh * t_max, 2511)
    v = oracle.fill_det(kv_heads * t_max * dh, 2512)
    got = oracle.flash_attention(q, kt, v, heads, kv_heads, t_q, t_max, dh, kv_len, pos_base, 0.125)
    tq = torch.from_numpy(q.reshape(heads, t_q, dh)).double()
    tk = torch.from_numpy(kt.reshape(kv_heads, dh, t_max)).double().transpose(1, 2).repeat_interleave(4, 0)
    tv = torch.from_numpy(v.reshape(kv_heads, t_max, dh)).double().repeat_interleave(4, 0)
    mask = torch.arange(t_max)[None, :] < torch.clamp(torch.arange(t_q) + pos_base + 1, max=kv_len)[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask,
                                                           scale=float(np.float32(0.125)))
    assert np.allclose(got, ref.numpy().reshape(-1), rtol=1e-6, atol=1e-7)

    one = oracle.flash_attention(q, kt, v, heads, kv_heads, t_q, t_max, dh, 1, 0, 0.125).reshape(heads, t_q, dh)
    vv = v.reshape(kv_heads, t_max, dh)
    assert np.array_equal(one[5, 17], vv[1, 0])
    flat = oracle.flash_attention(q, kt, v, heads, kv_heads, t_q, t_max, dh, kv_len, pos_base, 0.0)
    flat = flat.reshape(heads, t_q, dh)
    assert np.allclose(flat[3, 10], vv[0, :41].astype(np.float64).mean(axis=0), atol=1e-7)
    assert not np.any(oracle.flash_attention(q, kt, v, heads, kv_heads, t_q, t_max, dh, 0, 0, 0.125))


def _scan_argmax(v):
    """The greedy sampler as a scan: keep the last element >= the running best."""
    best, idx = float("-inf"), 0
    for i, x in enumerate(v):
        if x >= best:
            best, idx = x, i
    return idx


def test_argmax_last_pinned(oracle):
    """tests/correctness/token_loop.rs:55-95 known answers (last maximum wins),
    a brute-force scan on tie-heavy vectors, and numpy on reversed input."""
    n = 32000
    assert oracle.argmax_last(np.full(n, 1.5, np.float32)) == n - 1
    x = oracle.fill_det(n, 7201)
    x[5] = 1.0e6
    x[20000] = 1.0e6
    assert oracle.argmax_last(x) == 20000
    x = np.full(n, -2.0, np.float32)
    x[0] = 3.0
    assert oracle.argmax_last(x) == 0
    assert oracle.argmax_last(np.full(n, -np.inf, np.float32)) == n - 1
    rng = np.random.default_rng(7)
    for size in (1, 2, 7, 64, 1000):
        v = rng.integers(-3, 4, size).astype(np.float32)
        assert oracle.argmax_last(v) == _scan_argmax(v.tolist())
        assert oracle.argmax_last(v) == size - 1 - int(np.argmax(v[::-1]))
    v = np.array([1.0, np.nan, 3.0, np.nan, 3.0, 2.0], np.float32)
    assert oracle.argmax_last(v) == 4
    assert oracle.argmax_last(np.full(4, np.nan, np.float32)) == 0


def test_embed_gather_pinned(oracle):
    """tests/correctness/token_loop.rs:97-142: rows by id, ids past the
    vocabulary clamp to the last row, f16 outputs round each value."""
    vocab, embd = 301, 320
    table = oracle.fill_det(vocab * embd, 7301)
    rows = oracle.embed_gather(table, vocab, embd, [0, 7, vocab - 1, vocab + 100])
    t = table.reshape(vocab, embd)
    assert np.array_equal(rows.reshape(4, embd), np.stack([t[0], t[7], t[vocab - 1], t[vocab - 1]]))
    r16 = oracle.embed_gather(table, vocab, embd, [7], out_f16=True)
    assert np.array_equal(r16, t[7].astype(np.float16).astype(np.float32))


def test_attn_decode_pinned(oracle):
    """Decode attention equals the (separately pinned) causal prefill oracle
    for one query row per head at position kv_len - 1; uniform scores (q = 0)
    give the mean of the valid V rows; a single position returns its V row."""
    kv_heads, group, t_max, dh, kv_len = 3, 4, 96, 64, 70
    q = oracle.fill_det(kv_heads * group * dh, 7300)
    kt = oracle.fill_det(kv_heads * dh * t_max, 7301)
    v = oracle.fill_det(kv_heads * t_max * dh, 7302)
    got = oracle.attn_decode(q, kt, v, kv_heads, group, t_max, dh, kv_len, 0.125)
    ref = oracle.flash_attention(q, kt, v, kv_heads * group, kv_heads, 1, t_max, dh, kv_len, kv_len - 1, 0.125)
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-7)
    vv = v.reshape(kv_heads, t_max, dh)
    flat = oracle.attn_decode(np.zeros_like(q), kt, v, kv_heads, group, t_max, dh, kv_len, 0.125)
    flat = flat.reshape(kv_heads, group, dh)
    assert np.allclose(flat[2, 3], vv[2, :kv_len].astype(np.float64).mean(axis=0), atol=1e-7)
    one = oracle.attn_decode(q, kt, v, kv_heads, group, t_max, dh, 1, 0.125).reshape(kv_heads, group, dh)
    assert np.array_equal(one[1, 2], vv[1, 0])


def test_binary_combine_pinned(oracle):
    """op_binary_body.glsl: a + beta*b, and silu(a)*b against torch's silu."""
    import torch
    a, b = oracle.fill_det(4099, 7100), oracle.fill_det(4099, 7101)
    assert np.allclose(oracle.binary_combine(a, b, 0, 0.5), a.astype(np.float64) + 0.5 * b, rtol=1e-7, atol=0)
    ref = (torch.nn.functional.silu(torch.from_numpy(a).double()) * torch.from_numpy(b).double()).numpy()
    assert np.allclose(oracle.binary_combine(a, b, 1), ref, rtol=1e-6, atol=1e-7)
    assert oracle.binary_combine(np.zeros(3, np.float32), np.ones(3, np.float32), 1).tolist() == [0.0] * 3


def test_rope_scatter_pinned(oracle):
    """rope_scatter equals the (pinned) rope_tokens followed by the (pinned)
    strided copy into the Kt cache layout, for f32 and f16 destinations
    (tests/correctness/fusion.rs:250-329)."""
    tokens, heads, dh, rot, t_max, pos = 3, 2, 8, 6, 16, 5
    x = oracle.fill_det(tokens * heads * dh, 41000)
    table = oracle.fill_det(t_max * rot // 2 * 2, 41001)
    cache = np.full(heads * dh * t_max, 7.0, np.float32)
    got = oracle.rope_scatter(x, table, tokens, heads, dh, rot, pos, cache, pos, (1, dh * t_max, t_max))
    roped = oracle.rope_tokens(x, table, tokens, heads, dh, rot, pos)
    want = oracle.copy_strided(roped, cache, (dh, heads, tokens), 0, (1, dh, heads * dh), pos,
                               (t_max, dh * t_max, 1))
    assert np.array_equal(got, want)
    got16 = oracle.rope_scatter(x, table, tokens, heads, dh, rot, pos, cache, pos, (1, dh * t_max, t_max), True)
    assert np.array_equal(got16, np.where(got == 7.0, 7.0, oracle.round_via_f16(got)))


def test_prefill_qkv_pack_pinned(oracle):
    """prefill_qkv_pack against a per-element restatement of the three jobs
    (Q head-major, K into Kt columns, V into V rows) on a GQA case with a
    warm pos_base and partial rotary."""
    tokens, heads, kvh, dh, rot, pos, t_max = 5, 4, 2, 8, 6, 3, 12
    n = heads * dh + 2 * kvh * dh
    qkv = oracle.round_via_f16(oracle.fill_det(tokens * n, 42000))
    table = oracle.fill_det(t_max * rot, 42001)
    kt0, v0 = np.zeros((kvh, dh, t_max), np.float32), np.zeros((kvh, t_max, dh), np.float32)
    q, kt, v = oracle.prefill_qkv_pack(qkv, table, tokens, heads, kvh, dh, rot, pos, kt0, v0)
    x = qkv.reshape(tokens, n)
    tab = table.reshape(t_max, rot // 2, 2)
    def rot_vec(vec, p):
        out = vec.astype(np.float64).copy()
        for i in range(rot // 2):
            c, s = float(tab[p, i, 0]), float(tab[p, i, 1])
            x0, x1 = float(vec[2 * i]), float(vec[2 * i + 1])
            out[2 * i], out[2 * i + 1] = x0 * c - x1 * s, x0 * s + x1 * c
        return out
    for t in range(tokens):
        for h in range(heads):
            assert np.allclose(q[h, t], rot_vec(x[t, h * dh:(h + 1) * dh], pos + t), atol=2e-3)
        for h in range(kvh):
            k = x[t, heads * dh + h * dh: heads * dh + (h + 1) * dh]
            assert np.allclose(kt[h, :, pos + t], rot_vec(k, pos + t), atol=2e-3)
            assert np.array_equal(v[h, pos + t], x[t, heads * dh + kvh * dh + h * dh:][:dh])
            assert np.array_equal(q[0, t, rot:], x[t, rot:dh])  # pass-through lanes
    assert not kt[:, :, :pos].any() and not v[:, pos + tokens:].any()
    assert np.array_equal(q, oracle.round_via_f16(q).reshape(q.shape))
