"""ctypes binding of the CPU oracle (oracle/oracle.c -> oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() (as the
checker) and bench.py's cpu_baseline leg (as the timed CPU baseline).  The
shipped library never loads it.  See oracle.c for what each function restates
and how it is pinned.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_SO = Path(__file__).resolve().parent / "liboracle.so"
if not _SO.exists():
    raise ImportError(f"{_SO} is missing: build it with `python tensor-ash_amd/build.py`")
_lib = C.CDLL(str(_SO))

_F = C.POINTER(C.c_float)
_U16 = C.POINTER(C.c_uint16)
_U32 = C.POINTER(C.c_uint32)


def _sig(name, res, *args):
    f = getattr(_lib, name)
    f.restype = res
    f.argtypes = list(args)


_sig("ta_oracle_fill_det", None, _F, C.c_size_t, C.c_uint64)
_sig("ta_oracle_fill_normal", None, _F, C.c_size_t, C.c_uint64, C.c_float)
_sig("ta_oracle_lcg_range", C.c_int, C.c_uint64, C.c_uint32, C.c_uint32, _U32, C.c_size_t)
_sig("ta_oracle_cpu_bmm", C.c_int, _F, C.c_size_t, _F, C.c_size_t, _F, C.c_uint32, C.c_uint32,
     C.c_uint32, C.c_uint32, C.c_float, C.c_int, _F)
_sig("ta_oracle_cpu_bmm_rows", C.c_int, _F, C.c_size_t, _F, C.c_size_t, C.c_uint32, C.c_uint32,
     C.c_uint32, C.c_uint32, C.c_float, _F, C.c_uint64, C.c_uint64, C.c_int, C.c_int)
_sig("ta_oracle_max_threads", C.c_int)
_sig("ta_oracle_max_abs_err", C.c_float, _F, _F, C.c_size_t, C.POINTER(C.c_size_t))
_sig("ta_oracle_tolerance", C.c_float, C.c_uint32)
_sig("ta_oracle_f32_to_f16", C.c_uint16, C.c_float)
_sig("ta_oracle_f16_to_f32", C.c_float, C.c_uint16)
_sig("ta_oracle_f32_to_f16_array", None, _F, _U16, C.c_size_t)
_sig("ta_oracle_f16_to_f32_array", None, _U16, _F, C.c_size_t)
_sig("ta_oracle_round_via_f16", None, _F, C.c_size_t)
_sig("ta_oracle_pack_row_tiles", C.c_int, _F, C.c_size_t, C.c_size_t, C.c_size_t, _F)
_sig("ta_oracle_epilogue", None, _F, C.c_size_t, C.c_uint32, C.c_size_t, _F, C.c_uint32,
     C.c_uint32, C.c_uint32, _F, C.c_float)
_sig("ta_oracle_split_window", None, C.c_uint32, C.c_uint32, C.c_uint32, _U32, _U32)


def _f(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


def fill_det(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _lib.ta_oracle_fill_det(_f(out), n, seed)
    return out


def fill_normal(n: int, seed: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _lib.ta_oracle_fill_normal(_f(out), n, seed, std)
    return out


def lcg_range(seed: int, lo: int, hi: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint32)
    if _lib.ta_oracle_lcg_range(seed, lo, hi, out.ctypes.data_as(_U32), count) != 0:
        raise ValueError(f"LcgRng::range_u32 lo {lo} > hi {hi}")
    return out


def cpu_bmm(a, b, c_init, batch: int, m: int, n: int, k: int, alpha: float = 1.0,
            accumulate: bool = False) -> np.ndarray:
    a = _c32(a)
    b = _c32(b)
    out = np.empty(batch * m * n, dtype=np.float32)
    cp = None
    if c_init is not None:
        c_init = _c32(c_init)
        if c_init.size != out.size:
            raise ValueError("cpu_bmm: C init has wrong length")
        cp = _f(c_init)
    rc = _lib.ta_oracle_cpu_bmm(_f(a), a.size, _f(b), b.size, cp, batch, m, n, k, alpha,
                                int(accumulate), _f(out))
    if rc != 0:
        raise ValueError("cpu_bmm: A/B length matches neither broadcast nor batched")
    return out


def cpu_bmm_rows(a, b, batch, m, n, k, alpha, out, row_begin, row_end, threads=0,
                 reference_order=False) -> None:
    """Rows [row_begin, row_end) of cpu_bmm (parallel, bit-identical to it).
    reference_order=True uses the reference's j-outer/k-inner loop (slow;
    for timing the CPU baseline)."""
    rc = _lib.ta_oracle_cpu_bmm_rows(_f(a), a.size, _f(b), b.size, batch, m, n, k, alpha, _f(out),
                                     row_begin, row_end, threads, int(reference_order))
    if rc != 0:
        raise ValueError("cpu_bmm_rows: bad shapes")


def max_threads() -> int:
    return int(_lib.ta_oracle_max_threads())


def max_abs_err(a, b):
    a = _c32(a)
    b = _c32(b)
    if a.size != b.size:
        raise ValueError("max_abs_err: slice lengths differ")
    idx = C.c_size_t(0)
    e = _lib.ta_oracle_max_abs_err(_f(a), _f(b), a.size, C.byref(idx))
    return float(e), int(idx.value)


def tolerance(k: int) -> float:
    return float(_lib.ta_oracle_tolerance(k))


def f32_to_f16_bits(x) -> np.ndarray:
    x = _c32(x)
    out = np.empty(x.size, dtype=np.uint16)
    _lib.ta_oracle_f32_to_f16_array(_f(x), out.ctypes.data_as(_U16), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.empty(h.size, dtype=np.float32)
    _lib.ta_oracle_f16_to_f32_array(h.ctypes.data_as(_U16), _f(out), h.size)
    return out


def round_via_f16(x) -> np.ndarray:
    out = _c32(x).copy()
    _lib.ta_oracle_round_via_f16(_f(out), out.size)
    return out


def pack_row_tiles(src, k: int, n: int, tile: int) -> np.ndarray:
    src = _c32(src)
    out = np.empty_like(src)
    if _lib.ta_oracle_pack_row_tiles(_f(src), k, n, tile, _f(out)) != 0:
        raise ValueError(f"N={n} is not a multiple of tile_n={tile}")
    return out


def epilogue(c, n: int, mn: int, bias=None, bias_batch_stride: int = 0, act: int = 0,
             binary: int = 0, d=None, beta: float = 0.0) -> np.ndarray:
    out = _c32(c).copy()
    bias_p = _f(_c32(bias)) if bias is not None else None
    bias_keep = _c32(bias) if bias is not None else None
    if bias_keep is not None:
        bias_p = _f(bias_keep)
    d_keep = _c32(d) if d is not None else None
    _lib.ta_oracle_epilogue(_f(out), out.size, n, mn, bias_p, bias_batch_stride, act, binary,
                            _f(d_keep) if d_keep is not None else None, beta)
    return out


def split_window(k: int, splits: int, s: int):
    lo, hi = C.c_uint32(0), C.c_uint32(0)
    _lib.ta_oracle_split_window(k, splits, s, C.byref(lo), C.byref(hi))
    return lo.value, hi.value


def reference_gemm(a, b, batch, m, n, k, alpha=1.0, c_init=None, accumulate=False, bias=None,
                   bias_batch_stride=0, act=0, binary=0, d=None, beta=0.0) -> np.ndarray:
    """cpu_bmm followed by the f64 epilogue: the full fused-op reference."""
    c = cpu_bmm(a, b, c_init, batch, m, n, k, alpha, accumulate)
    return epilogue(c, n, m * n, bias, bias_batch_stride, act, binary, d, beta)


# ---- decode fusions (numpy restatements; pinned in tests/test_oracle.py) ----

def rms_norm_rows(x, w, m: int, k: int, eps: float) -> np.ndarray:
    """Normed-A reference of tests/correctness/fusion.rs:15-24
    (cpu_rms_norm_f64): per row, x * w / sqrt(mean(x^2) + eps) in f64,
    rounded to f32."""
    x64 = np.asarray(x, dtype=np.float32).reshape(m, k).astype(np.float64)
    w64 = np.asarray(w, dtype=np.float32).reshape(k).astype(np.float64)
    inv = 1.0 / np.sqrt((x64 * x64).sum(axis=1, keepdims=True) / k + float(np.float32(eps)))
    return (x64 * inv * w64).astype(np.float32).reshape(-1)


def _fma32(a, b, c):
    """f32 fused multiply-add: the product of two f32 is exact in f64; the
    sum is then rounded to f64 and to f32 (a double rounding that can
    differ from a single one only on exact f32 midpoints)."""
    return (np.asarray(a, np.float32).astype(np.float64) * np.asarray(b, np.float32).astype(np.float64)
            + np.asarray(c, np.float32).astype(np.float64)).astype(np.float32)


def rope_pairs(y, table, pos: int, head_dim: int) -> np.ndarray:
    """Store-time RoPE of one output row (shaders/matmul_row_bda_kernel.glsl:
    163-176): column c with partner c ^ 1 and dim = c % head_dim takes the
    (cos, sin) at table[(pos * head_dim/2 + dim/2) * 2 + {0, 1}];
    even dim: fma(v, cos, -partner*sin); odd dim: fma(partner, sin, v*cos)."""
    y = np.asarray(y, dtype=np.float32).reshape(-1)
    t = np.asarray(table, dtype=np.float32).reshape(-1)
    c = np.arange(y.size)
    dim = c % head_dim
    angle = (pos * (head_dim // 2) + dim // 2) * 2
    cos_t, sin_t = t[angle], t[angle + 1]
    partner = y[c ^ 1]
    even = _fma32(y, cos_t, (-partner * sin_t).astype(np.float32))
    odd = _fma32(partner, sin_t, (y * cos_t).astype(np.float32))
    return np.where(dim % 2 == 0, even, odd).astype(np.float32)


def scatter_index(pos: int, n: int, head_dim: int, pos_scale: int, stride_head: int,
                  stride_dim: int) -> np.ndarray:
    """Store-scatter element index of each output column c
    (src/matmul/api.rs:107-116): pos * pos_scale + (c / head_dim) *
    stride_head + (c % head_dim) * stride_dim."""
    c = np.arange(n, dtype=np.int64)
    return pos * pos_scale + (c // head_dim) * stride_head + (c % head_dim) * stride_dim


def store_scatter(dst, y, pos: int, head_dim: int, pos_scale: int, stride_head: int,
                  stride_dim: int, f16: bool = False) -> np.ndarray:
    """dst with the row y scattered in; an f16 destination holds the
    RNE-rounded values (returned widened to f32)."""
    out = np.array(dst, dtype=np.float32).reshape(-1).copy()
    v = np.asarray(y, dtype=np.float32).reshape(-1)
    if f16:
        v = round_via_f16(v)
    out[scatter_index(pos, v.size, head_dim, pos_scale, stride_head, stride_dim)] = v
    return out


# ---- model ops (numpy restatements; pinned in tests/test_oracle.py) ----

def softmax_rows(x, rows: int, cols: int, scale: float, valid) -> np.ndarray:
    """Row softmax of shaders/op_softmax_f32_row.comp semantics in f64:
    row r uses its first valid(r) columns of x * scale; masked columns and
    all-masked rows are 0.  `valid` is an int or a per-row callable."""
    x = np.asarray(x, dtype=np.float32).reshape(rows, cols)
    out = np.zeros((rows, cols), dtype=np.float64)
    for r in range(rows):
        v = min(cols, valid(r) if callable(valid) else valid)
        if v == 0:
            continue
        z = (x[r, :v] * np.float32(scale)).astype(np.float64)
        e = np.exp(z - z.max())
        out[r, :v] = e / e.sum()
    return out.astype(np.float32).reshape(-1)


def layer_norm_rows(x, w, b, rows: int, cols: int, eps: float) -> np.ndarray:
    """LayerNorm of tests/correctness/elementwise.rs:99-142: (x - mean) /
    sqrt(var + eps) in f64 (population variance), rounded to f32, then
    * w + b in f32."""
    x64 = np.asarray(x, dtype=np.float32).reshape(rows, cols).astype(np.float64)
    mean = x64.mean(axis=1, keepdims=True)
    var = ((x64 - mean) ** 2).mean(axis=1, keepdims=True)
    y = ((x64 - mean) / np.sqrt(var + float(np.float32(eps)))).astype(np.float32)
    return (y * np.asarray(w, np.float32) + np.asarray(b, np.float32)).reshape(-1)


def rope_tokens(x, table, tokens: int, heads: int, head_dim: int, rot_dim: int, pos_base: int) -> np.ndarray:
    """RoPE of shaders/op_rope_body.glsl: pair i < rot_dim/2 of (token, head)
    rotates by table[(pos_base + token) * rot_dim/2 + i] = (c, s):
    r0 = fma(x0, c, -x1*s), r1 = fma(x0, s, x1*c); lanes >= rot_dim pass."""
    x = np.asarray(x, dtype=np.float32).reshape(tokens, heads, head_dim)
    t = np.asarray(table, dtype=np.float32).reshape(-1, rot_dim // 2, 2)
    out = x.copy()
    cs = t[pos_base:pos_base + tokens]           # [tokens, half, 2]
    c, s = cs[:, None, :, 0], cs[:, None, :, 1]  # broadcast over heads
    x0, x1 = x[:, :, 0:rot_dim:2], x[:, :, 1:rot_dim:2]
    out[:, :, 0:rot_dim:2] = _fma32(x0, c, (-x1 * s).astype(np.float32))
    out[:, :, 1:rot_dim:2] = _fma32(x0, s, (x1 * c).astype(np.float32))
    return out.reshape(-1)


def copy_strided(src, dst, extent, src_offset, src_strides, dst_offset, dst_strides,
                 dst_f16: bool = False) -> np.ndarray:
    """Strided 3-D copy of shaders/op_copy_strided_body.glsl: element
    (x, y, z) < extent moves src[src_offset + x*ss0 + y*ss1 + z*ss2] to
    dst[dst_offset + x*ds0 + y*ds1 + z*ds2]; an f16 destination holds the
    RNE-rounded value (returned widened)."""
    out = np.array(dst, dtype=np.float32).reshape(-1).copy()
    s = np.asarray(src, dtype=np.float32).reshape(-1)
    xs, ys, zs = np.meshgrid(np.arange(extent[0]), np.arange(extent[1]), np.arange(extent[2]), indexing="ij")
    si = src_offset + xs * src_strides[0] + ys * src_strides[1] + zs * src_strides[2]
    di = dst_offset + xs * dst_strides[0] + ys * dst_strides[1] + zs * dst_strides[2]
    v = s[si.reshape(-1)]
    out[di.reshape(-1)] = round_via_f16(v) if dst_f16 else v
    return out


def flash_attention(q, kt, v, heads: int, kv_heads: int, t_q: int, t_max: int, dh: int, kv_len: int,
                    pos_base: int, scale: float) -> np.ndarray:
    """Causal prefill attention of tests/correctness/flash.rs:10-61
    (cpu_flash) in f64: head h reads kv head h / (heads / kv_heads); query
    row i attends to cache positions < min(kv_len, pos_base + i + 1) with
    softmax(q . k * scale); q/out are head-major [H, T_q, dh], kt is
    [H_kv, dh, T_max], v is [H_kv, T_max, dh].  A row with no valid
    position is all zeros."""
    q64 = np.asarray(q, np.float32).reshape(heads, t_q, dh).astype(np.float64)
    kt64 = np.asarray(kt, np.float32).reshape(kv_heads, dh, t_max).astype(np.float64)
    v64 = np.asarray(v, np.float32).reshape(kv_heads, t_max, dh).astype(np.float64)
    out = np.zeros((heads, t_q, dh))
    group = heads // kv_heads
    valid = np.minimum(kv_len, pos_base + np.arange(t_q) + 1)
    span = int(valid.max()) if t_q else 0
    if span == 0:
        return out.astype(np.float32).reshape(-1)
    mask = np.arange(span)[None, :] < valid[:, None]
    for h in range(heads):
        kh = h // group
        s = (q64[h] @ kt64[kh, :, :span]) * float(np.float32(scale))
        s = np.where(mask, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        p = np.where(mask, np.exp(s - m), 0.0)
        out[h] = (p / p.sum(axis=1, keepdims=True)) @ v64[kh, :span]
    return out.astype(np.float32).reshape(-1)


def argmax_last(x) -> int:
    """Greedy-sampling argmax of shaders/op_argmax_f32.comp and
    tests/correctness/token_loop.rs:14-22 (cpu_argmax, Rust
    `max_by(total_cmp)`): the index of the largest value, the LARGEST index
    among equal maxima; NaNs never win (an all-NaN vector gives 0)."""
    v = np.asarray(x, np.float32).reshape(-1)
    if v.size == 0:
        raise ValueError("argmax of an empty vector")
    finite = ~np.isnan(v)
    if not finite.any():
        return 0
    return int(np.nonzero(v == v[finite].max())[0][-1])


def embed_gather(table, vocab: int, embd: int, tokens, out_f16: bool = False) -> np.ndarray:
    """Embedding rows of shaders/op_embed_gather.comp: row t of the output is
    row min(tokens[t], vocab - 1) of the [vocab, embd] table (already holding
    the stored, e.g. f16-rounded, values); an f16 output holds the values
    rounded to f16 (RNE)."""
    t = np.asarray(table, np.float32).reshape(vocab, embd)
    ids = np.minimum(np.asarray(tokens, np.int64).reshape(-1), vocab - 1)
    rows = t[ids].reshape(-1)
    return round_via_f16(rows) if out_f16 else rows.copy()


def attn_decode(q, kt, v, kv_heads: int, group: int, t_max: int, dh: int, kv_len: int,
                scale: float) -> np.ndarray:
    """Decode attention of tests/correctness/attn_decode.rs:14-54
    (cpu_attn_decode) in f64: each of the `group` query rows of kv head h
    (q [kv_heads, group, dh]) attends to cache positions < kv_len with
    softmax(q . k * scale); kt [kv_heads, dh, t_max], v [kv_heads, t_max, dh];
    out [kv_heads, group, dh]."""
    q64 = np.asarray(q, np.float32).reshape(kv_heads, group, dh).astype(np.float64)
    kt64 = np.asarray(kt, np.float32).reshape(kv_heads, dh, t_max)[:, :, :kv_len].astype(np.float64)
    v64 = np.asarray(v, np.float32).reshape(kv_heads, t_max, dh)[:, :kv_len].astype(np.float64)
    out = np.zeros((kv_heads, group, dh))
    for h in range(kv_heads):
        s = (q64[h] @ kt64[h]) * float(scale)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[h] = (p / p.sum(axis=1, keepdims=True)) @ v64[h]
    return out.astype(np.float32).reshape(-1)


def binary_combine(a, b, mode: int, beta: float = 0.0) -> np.ndarray:
    """Binary combine of shaders/op_binary_body.glsl in f64: mode 0 a + beta * b
    (residual add), mode 1 silu(a) * b = a / (1 + exp(-a)) * b (SwiGLU gating)."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    if mode == 0:
        return (a64 + float(np.float32(beta)) * b64).astype(np.float32)
    return (a64 / (1.0 + np.exp(-a64)) * b64).astype(np.float32)


def rope_scatter(x, table, tokens: int, heads: int, head_dim: int, rot_dim: int, pos_base: int,
                 dst, dst_offset: int, dst_strides, dst_f16: bool = False) -> np.ndarray:
    """Fused RoPE + scatter of src/executor/elementwise/ops.rs:243-316: the rotation
    of rope_tokens, element (t, h, d) stored at dst_offset + t*s0 + h*s1 + d*s2 of
    a copy of dst (f16 destinations hold the RNE-rounded value)."""
    y = rope_tokens(x, table, tokens, heads, head_dim, rot_dim, pos_base).reshape(tokens, heads, head_dim)
    out = np.asarray(dst, np.float32).reshape(-1).copy()
    t, h, d = np.meshgrid(np.arange(tokens), np.arange(heads), np.arange(head_dim), indexing="ij")
    idx = dst_offset + t * dst_strides[0] + h * dst_strides[1] + d * dst_strides[2]
    out[idx.reshape(-1)] = round_via_f16(y.reshape(-1)) if dst_f16 else y.reshape(-1)
    return out


def prefill_qkv_pack(qkv, table, tokens: int, heads: int, kv_heads: int, head_dim: int, rot_dim: int,
                     pos_base: int, kt, v):
    """Prefill QKV pack of src/executor/elementwise/flash.rs:255-402 on f16 data
    (inputs hold f16 values): Q of each token (rope_tokens rotation, rounded to
    f16) in head-major [H, T, dh]; K rotated and rounded into kt [H_kv, dh, T_max]
    at column pos_base + t; V copied into v [H_kv, T_max, dh] at row pos_base + t.
    Returns (q, kt, v) as new arrays."""
    x = np.asarray(qkv, np.float32).reshape(tokens, -1)
    embd, kv_dim = heads * head_dim, kv_heads * head_dim
    q = rope_tokens(np.ascontiguousarray(x[:, :embd]).reshape(-1), table, tokens, heads, head_dim, rot_dim,
                    pos_base)
    q = round_via_f16(q).reshape(tokens, heads, head_dim).transpose(1, 0, 2).copy()
    k = rope_tokens(np.ascontiguousarray(x[:, embd:embd + kv_dim]).reshape(-1), table, tokens, kv_heads,
                    head_dim, rot_dim, pos_base)
    k = round_via_f16(k).reshape(tokens, kv_heads, head_dim)
    kt_out = np.asarray(kt, np.float32).copy()
    v_out = np.asarray(v, np.float32).copy()
    for t in range(tokens):
        kt_out[:, :, pos_base + t] = k[t]
        v_out[:, pos_base + t, :] = x[t, embd + kv_dim:].reshape(kv_heads, head_dim)
    return q, kt_out, v_out
