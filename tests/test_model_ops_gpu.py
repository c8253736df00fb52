"""GPU parity of the model ops around the GEMM path: row softmax, RMSNorm,
LayerNorm, RoPE and strided copy (include/tensor_ash.h ta_softmax_rows ...
ta_copy_strided; the reference's tests/correctness/elementwise.rs).

Cases and tolerances follow the reference's tests: softmax 1e-6 absolute
against an f64 reference with row sums within 1e-5 and masked columns
exactly 0; norms 1e-4 against f64 references; RoPE 1e-5 (here: at most one
f32 ulp against the oracle's fma restatement) and in-place equal to
out-of-place bit for bit; copies exact (f16 destinations hold the
round-to-nearest-even value).
"""

import numpy as np
import pytest


pytestmark = pytest.mark.gpu

EPS = 1e-5


def ulp_diff(a, b) -> int:
    a = np.asarray(a, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).reshape(-1).view(np.int32).astype(np.int64)
    return int(np.max(np.abs(a - b))) if a.size else 0


def llama_table(t_max, rot):
    half = rot // 2
    theta = np.array([[p / 10000.0 ** (2.0 * i / rot) for i in range(half)] for p in range(t_max)])
    return np.stack([np.cos(theta), np.sin(theta)], axis=-1).astype(np.float32).reshape(-1)


# ---------------------------------------------------------------- softmax

@pytest.mark.parametrize("rows,cols", [(6, 517), (512, 4096), (3, 8), (2, 1)])
def test_softmax_full(ex, oracle, rows, cols):
    """elementwise.rs:17-95 (full case): every column valid, scale 0.125."""
    x = oracle.fill_det(rows * cols, 3000 + cols)
    a, out = ex.tensor_from(x, shape=[rows, cols]), ex.tensor([rows, cols])
    ex.softmax_rows(a, out, 0.125)
    got = ex.download(out).reshape(rows, cols)
    ref = oracle.softmax_rows(x, rows, cols, 0.125, cols).reshape(rows, cols)
    assert np.max(np.abs(got - ref)) <= 1e-6
    assert np.max(np.abs(got.astype(np.float64).sum(axis=1) - 1.0)) <= 1e-5


@pytest.mark.parametrize("valid", [300, 1, 0, 517, 9999])
def test_softmax_prefix_mask(ex, oracle, valid):
    """elementwise.rs:17-95 (prefix case): columns past `valid` store exactly 0; valid 0
    gives an all-zero row; valid past the row clamps to the row."""
    rows, cols = 6, 517
    x = oracle.fill_det(rows * cols, 3100)
    a, out = ex.tensor_from(x, shape=[rows, cols]), ex.tensor([rows, cols])
    ex.upload(out, np.full(rows * cols, 7.0, np.float32))
    ex.softmax_rows(a, out, 0.125, mask_kind=1, valid_or_prefix=valid)
    got = ex.download(out).reshape(rows, cols)
    ref = oracle.softmax_rows(x, rows, cols, 0.125, valid).reshape(rows, cols)
    v = min(valid, cols)
    assert np.all(got[:, v:] == 0.0)
    assert np.max(np.abs(got - ref)) <= 1e-6


def test_softmax_causal_mask(ex, oracle):
    """elementwise.rs:17-95 (causal case): row r of a group of 3 attends to
    prefix + (r % 3) + 1 columns."""
    rows, cols, prefix, rpg = 6, 517, 100, 3
    x = oracle.fill_det(rows * cols, 3200)
    a, out = ex.tensor_from(x, shape=[rows, cols]), ex.tensor([rows, cols])
    ex.softmax_rows(a, out, 0.125, mask_kind=2, valid_or_prefix=prefix, rows_per_group=rpg)
    got = ex.download(out).reshape(rows, cols)
    ref = oracle.softmax_rows(x, rows, cols, 0.125, lambda r: prefix + r % rpg + 1).reshape(rows, cols)
    for r in range(rows):
        assert np.all(got[r, prefix + r % rpg + 1:] == 0.0)
    assert np.max(np.abs(got - ref)) <= 1e-6


def test_softmax_in_place(ex, oracle):
    rows, cols = 4, 777
    x = oracle.fill_det(rows * cols, 3300)
    a = ex.tensor_from(x, shape=[rows, cols])
    ex.softmax_rows(a, a, 0.5)
    ref = oracle.softmax_rows(x, rows, cols, 0.5, cols)
    assert np.max(np.abs(ex.download(a).reshape(-1) - ref)) <= 1e-6


def test_softmax_rejects_bad_arguments(ta, ex):
    a, out = ex.tensor([6, 8]), ex.tensor([6, 8])
    with pytest.raises(ta.TensorAshError, match="rows_per_group"):
        ex.softmax_rows(a, out, 1.0, mask_kind=2, valid_or_prefix=0, rows_per_group=4)
    with pytest.raises(ta.TensorAshError, match="shape"):
        ex.softmax_rows(a, ex.tensor([6, 9]), 1.0)
    with pytest.raises(ta.TensorAshError, match="f32"):
        ex.softmax_rows(ex.tensor([6, 8], f16=True), out, 1.0)
    with pytest.raises(ta.TensorAshError):
        ex.softmax_rows(a, out, 1.0, mask_kind=3)


# ---------------------------------------------------------------- norms

@pytest.mark.parametrize("rows,cols", [(5, 771), (4, 768), (1, 4096), (300, 2048), (2, 3)])
def test_rms_norm(ex, oracle, rows, cols):
    """elementwise.rs:99-142: f64 reference, 1e-4 tolerance (the widths
    cover the scalar and the 128-bit paths)."""
    x, w = oracle.fill_det(rows * cols, 3400 + cols), oracle.fill_det(cols, 3401 + cols)
    a, tw, out = ex.tensor_from(x, shape=[rows, cols]), ex.tensor_from(w, shape=[cols]), ex.tensor([rows, cols])
    ex.rms_norm(a, tw, out, EPS)
    ref = oracle.rms_norm_rows(x, w, rows, cols, EPS)
    assert np.max(np.abs(ex.download(out).reshape(-1) - ref)) <= 1e-4


@pytest.mark.parametrize("rows,cols", [(5, 771), (4, 768), (300, 2048)])
def test_layer_norm(ex, oracle, rows, cols):
    """elementwise.rs:99-142: mean / population variance in f64, 1e-4."""
    x, w, b = (oracle.fill_det(rows * cols, 3500 + cols), oracle.fill_det(cols, 3501 + cols),
               oracle.fill_det(cols, 3502 + cols))
    a, out = ex.tensor_from(x, shape=[rows, cols]), ex.tensor([rows, cols])
    tw, tb = ex.tensor_from(w, shape=[cols]), ex.tensor_from(b, shape=[cols])
    ex.layer_norm(a, tw, tb, out, EPS)
    ref = oracle.layer_norm_rows(x, w, b, rows, cols, EPS)
    assert np.max(np.abs(ex.download(out).reshape(-1) - ref)) <= 1e-4


def test_norms_in_place(ex, oracle):
    rows, cols = 3, 1000
    x, w, b = oracle.fill_det(rows * cols, 3600), oracle.fill_det(cols, 3601), oracle.fill_det(cols, 3602)
    tw, tb = ex.tensor_from(w, shape=[cols]), ex.tensor_from(b, shape=[cols])
    a = ex.tensor_from(x, shape=[rows, cols])
    ex.rms_norm(a, tw, a, EPS)
    assert np.max(np.abs(ex.download(a).reshape(-1) - oracle.rms_norm_rows(x, w, rows, cols, EPS))) <= 1e-4
    a = ex.tensor_from(x, shape=[rows, cols])
    ex.layer_norm(a, tw, tb, a, EPS)
    assert np.max(np.abs(ex.download(a).reshape(-1) - oracle.layer_norm_rows(x, w, b, rows, cols, EPS))) <= 1e-4


@pytest.mark.parametrize("rows,cols", [(4, 768), (3, 771)])
def test_rms_norm_f16_io(ex, oracle, rows, cols):
    """f16 activations in and out (f32 weight, f32 arithmetic): the result
    is the f32 result rounded to f16, so it may differ from the rounded
    reference by one f16 ulp (2^-10 relative)."""
    x, w = oracle.fill_det(rows * cols, 3700 + cols), oracle.fill_det(cols, 3701 + cols)
    xr = oracle.round_via_f16(x)
    a, out = ex.tensor_from(x, shape=[rows, cols], f16=True), ex.tensor([rows, cols], f16=True)
    ex.rms_norm(a, ex.tensor_from(w, shape=[cols]), out, EPS)
    ref = oracle.rms_norm_rows(xr, w, rows, cols, EPS)
    got = ex.download(out).reshape(-1)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 1e-4)


def test_norms_reject_bad_arguments(ta, ex):
    a, out = ex.tensor([4, 8]), ex.tensor([4, 8])
    w, b = ex.tensor([8]), ex.tensor([8])
    with pytest.raises(ta.TensorAshError, match="weight length"):
        ex.rms_norm(a, ex.tensor([7]), out, EPS)
    with pytest.raises(ta.TensorAshError, match="bias length"):
        ex.layer_norm(a, w, ex.tensor([9]), out, EPS)
    with pytest.raises(ta.TensorAshError, match="RMSNorm only"):
        ex.layer_norm(ex.tensor([4, 8], f16=True), w, b, ex.tensor([4, 8], f16=True), EPS)
    with pytest.raises(ta.TensorAshError, match="storage type"):
        ex.rms_norm(a, w, ex.tensor([4, 8], f16=True), EPS)
    with pytest.raises(ta.TensorAshError, match="shape"):
        ex.rms_norm(a, w, ex.tensor([8, 4]), EPS)


# ---------------------------------------------------------------- RoPE

@pytest.mark.parametrize("tokens,heads,hd,rot,pos_base", [(3, 4, 16, 12, 7), (1, 32, 128, 128, 0),
                                                           (17, 8, 64, 32, 100), (5, 2, 96, 64, 3)])
def test_rope(ex, oracle, tokens, heads, hd, rot, pos_base):
    """elementwise.rs:146-222: Llama table, partial rotary, pos_base; the
    rotation is the reference's fma order, so at most 1 ulp from the
    oracle's double-rounded fma; pass-through lanes are exact."""
    t_max = pos_base + tokens + 4
    x, table = oracle.fill_det(tokens * heads * hd, 3800 + hd), llama_table(t_max, rot)
    a, out, tt = ex.tensor_from(x, shape=[tokens, heads * hd]), ex.tensor([tokens, heads * hd]), \
        ex.tensor_from(table, shape=[t_max, rot // 2, 2])
    ex.rope(a, tt, out, heads, hd, rot, pos_base)
    got = ex.download(out).reshape(-1)
    ref = oracle.rope_tokens(x, table, tokens, heads, hd, rot, pos_base)
    assert ulp_diff(got, ref) <= 1
    # in place equals out of place bit for bit
    ex.rope(a, tt, a, heads, hd, rot, pos_base)
    assert np.array_equal(ex.download(a).reshape(-1), got)


def test_rope_f16_io(ex, oracle):
    tokens, heads, hd, rot = 4, 8, 64, 64
    x, table = oracle.fill_det(tokens * heads * hd, 3900), llama_table(16, rot)
    a, out = ex.tensor_from(x, shape=[tokens, heads * hd], f16=True), ex.tensor([tokens, heads * hd], f16=True)
    ex.rope(a, ex.tensor_from(table, shape=[16, rot // 2, 2]), out, heads, hd, rot, 2)
    ref = oracle.round_via_f16(oracle.rope_tokens(oracle.round_via_f16(x), table, tokens, heads, hd, rot, 2))
    got = ex.download(out).reshape(-1)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 1e-7)


def test_rope_rejects_bad_arguments(ta, ex):
    a, out = ex.tensor([2, 64]), ex.tensor([2, 64])
    table = ex.tensor([8, 8, 2])
    with pytest.raises(ta.TensorAshError, match="rot_dim"):
        ex.rope(a, table, out, 4, 16, 11)
    with pytest.raises(ta.TensorAshError, match="rot_dim"):
        ex.rope(a, table, out, 4, 16, 18)
    with pytest.raises(ta.TensorAshError, match="multiple"):
        ex.rope(a, table, out, 3, 16, 16)
    with pytest.raises(ta.TensorAshError, match="table length"):
        ex.rope(a, table, out, 4, 16, 16, pos_base=7)


# ---------------------------------------------------------------- strided copy

def test_copy_transpose(ex, oracle):
    """elementwise.rs:226-318: a 37x53 transpose through the strides."""
    r, c = 37, 53
    x = oracle.fill_det(r * c, 4000)
    src, dst = ex.tensor_from(x, shape=[r, c]), ex.tensor([c, r])
    ex.copy_strided(src, dst, (c, r, 1), (1, c, 0), (r, 1, 0))
    assert np.array_equal(ex.download(dst).reshape(c, r), x.reshape(r, c).T)


def test_copy_kv_append(ex, oracle):
    """elementwise.rs:226-318: append K of one step into column t of a
    transposed cache [heads, dh, t_max]; the rest of the cache is kept."""
    heads, dh, t_max = 4, 8, 16
    cache0 = oracle.fill_det(heads * dh * t_max, 4100)
    cache = ex.tensor_from(cache0, shape=[heads, dh, t_max])
    want = cache0.copy()
    for t in (0, 5, 15):
        k = oracle.fill_det(heads * dh, 4101 + t)
        ex.copy_strided(ex.tensor_from(k, shape=[heads * dh]), cache, (dh, heads, 1), (1, dh, 0),
                        (t_max, dh * t_max, 0), dst_offset=t)
        want = oracle.copy_strided(k, want, (dh, heads, 1), 0, (1, dh, 0), t, (t_max, dh * t_max, 0))
    assert np.array_equal(ex.download(cache).reshape(-1), want)


@pytest.mark.parametrize("src_f16,dst_f16", [(False, True), (True, False), (True, True)])
def test_copy_f16_pairings(ex, oracle, src_f16, dst_f16):
    """The f16 shader variants (op_copy_strided_{f16,f16_to_f32,f32_to_f16}; elementwise.rs:701):
    f16 sources hold f16 values; an f16 destination rounds to nearest even."""
    a, b, cdim = 5, 7, 3
    x = oracle.fill_det(a * b * cdim, 4200) * 1000.0
    src = ex.tensor_from(x, shape=[a * b * cdim], f16=src_f16)
    dst = ex.tensor([a * b * cdim], f16=dst_f16)
    # permute [a, b, c] -> [c, a, b]
    ex.copy_strided(src, dst, (cdim, b, a), (1, cdim, b * cdim), (a * b, 1, b))
    xs = oracle.round_via_f16(x) if src_f16 else x
    want = oracle.copy_strided(xs, np.zeros(a * b * cdim), (cdim, b, a), 0, (1, cdim, b * cdim), 0,
                               (a * b, 1, b), dst_f16=dst_f16)
    assert np.array_equal(ex.download(dst).reshape(-1), want)


def test_copy_large_bandwidth_shape(ex, oracle):
    """A [2048, 4096] transpose: more elements than one grid pass covers."""
    r, c = 2048, 4096
    x = oracle.fill_det(r * c, 4300)
    src, dst = ex.tensor_from(x, shape=[r, c]), ex.tensor([c, r])
    ex.copy_strided(src, dst, (c, r, 1), (1, c, 0), (r, 1, 0))
    assert np.array_equal(ex.download(dst).reshape(c, r), x.reshape(r, c).T)


def test_copy_rejects_bad_descriptors(ta, ex):
    """ops.rs:387-437: out-of-bounds reach, zero extents and aliasing."""
    src, dst = ex.tensor([37, 53]), ex.tensor([53, 37])
    with pytest.raises(ta.TensorAshError, match="source access"):
        ex.copy_strided(src, dst, (53, 37, 1), (1, 53, 0), (37, 1, 0), src_offset=1)
    with pytest.raises(ta.TensorAshError, match="destination access"):
        ex.copy_strided(src, dst, (53, 37, 1), (1, 53, 0), (38, 1, 0))
    with pytest.raises(ta.TensorAshError, match="zero axis"):
        ex.copy_strided(src, dst, (53, 0, 1), (1, 53, 0), (37, 1, 0))
    with pytest.raises(ta.TensorAshError, match="different tensors"):
        ex.copy_strided(src, src, (1, 1, 1), (1, 1, 1), (1, 1, 1))
